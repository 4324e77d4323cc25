// Kernel launchers shared between the kernel translation units and the C-ABI layer (jamhip.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace jamhip {

// F1: q [n][k] int8, d [n][k/32], asum [n][k/32] (float Σq), s16 [n][k/16] (int Σq).
hipError_t launch_quant_f1(const float* a, int lda, int n, int k, int8_t* q, float* d, float* asum, int* s16,
                           hipStream_t st);
// F2: q [n][k] int8, d [n][k/32], xs [n][k/16] (raw f32 Σx).
hipError_t launch_quant_f2(const float* a, int lda, int n, int k, int8_t* q, float* d, float* xs, hipStream_t st);

// raw GGUF rows (rb blocks each, stride raw_stride bytes) -> the device layout with G groups per row
hipError_t launch_repack(int dt, const uint8_t* raw, int64_t raw_stride, int64_t rows, int64_t rb, int64_t G,
                         uint8_t* qs, uint8_t* sc, hipStream_t st);

// flavour 1: n in [1, 7], F1 activations; with `a` non-null the kernel quantizes A itself (requires
// gemv_fusable(n, k)), else it reads A's quantized copy from `A`. flavour 2: any n >= 1, F2
// activations from `A`, 8 tokens per grid row.
bool gemv_fusable(int n, int k, const float* a, int lda);   // a, lda: the f32 activations (16-byte aligned rows)
hipError_t launch_gemv(int dt, int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m,
                       int n, float* c, int ldc, hipStream_t st);

// Rows [r0, r0 + rows) of an n >= 8 call as jam's bands compute their <16-row tail: an f32 dot of the
// dequantized weight row with the f32 activations a [n][lda].
hipError_t launch_rows_float(int dt, const WeightView& w, const float* a, int lda, int k, int r0, int rows, int n,
                             float* c, int ldc, hipStream_t st);

// int8-MFMA prefill GEMM (F2 activations), n >= 1; returns hipErrorNotSupported for dtypes it lacks.
hipError_t launch_gemm(int dt, const WeightView& w, const ActQ& A, int k, int m, int n, float* c, int ldc,
                       hipStream_t st);

}  // namespace jamhip
