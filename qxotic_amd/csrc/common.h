// Shared device/host definitions for the jamhip kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jamhip {

// ggml / jam dtype tags (jam/jam-native/include/jam.h:59-77).
enum Dtype : int { F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14, BF16 = 30, MXFP4 = 39 };

// GGUF block geometry (jam/jam-core/src/main/java/com/qxotic/jam/GGMLType.java:15-26).
__host__ __device__ constexpr int block_elems(int dt) {
    return dt == Q4_K || dt == Q5_K || dt == Q6_K ? 256 : (dt == Q8_0 || dt == Q4_0 || dt == MXFP4) ? 32 : 1;
}
__host__ __device__ constexpr int block_bytes(int dt) {
    return dt == Q8_0 ? 34 : dt == Q4_0 ? 18 : dt == MXFP4 ? 17 : dt == Q4_K ? 144 : dt == Q5_K ? 176
         : dt == Q6_K ? 210 : dt == F32 ? 4 : 2;
}

// Device layout of a pinned weight tensor of `rows` rows and `rb` blocks per row.
//   plane 0 ("qs")   : rows × rb × qs_bytes  — the 16-byte-aligned part of every block
//   plane 1 ("sc")   : rows × rb × sc_bytes  — the scalar scale (fp16 d, or the E8M0 byte)
// Q4_K's 144-byte blocks are already 16-byte multiples and stay whole in plane 0 (sc_bytes 0).
//   Q8_0 : qs 32 (int8 q)                 | d fp16
//   Q4_0 : qs 16 (nibbles)                | d fp16
//   MXFP4: qs 16 (nibbles)                | e8m0
//   Q6_K : ql 128 | qh 64 | scales 16 = 208 | d fp16
//   Q4_K : whole block 144                | —
// Bytes are exactly the GGUF bytes; only their order changes.
__host__ __device__ constexpr int qs_bytes(int dt) {
    return dt == Q8_0 ? 32 : dt == Q4_0 ? 16 : dt == MXFP4 ? 16 : dt == Q6_K ? 208 : dt == Q4_K ? 144 : 0;
}
__host__ __device__ constexpr int sc_bytes(int dt) {
    return dt == Q8_0 ? 2 : dt == Q4_0 ? 2 : dt == MXFP4 ? 1 : dt == Q6_K ? 2 : 0;
}

struct WeightView {
    const uint8_t* qs;   // plane 0 at row 0 of the view
    const uint8_t* sc;   // plane 1 at row 0 of the view (nullptr for Q4_K)
    int64_t rb;          // blocks per row in the device layout
};

// Activation quantization outputs (per token row j of k elements, nb = k/32 blocks).
struct ActQ {
    const int8_t* q;    // [n][k]
    const float* d;     // [n][nb]   per-32 scale
    const float* s;     // F1: [n][nb] (float)Σq per 32;  F2: [n][k/16] raw f32 Σx per 16
    const int* s16;     // F1 only: [n][k/16] Σq per 16 (exact ints; Q6_K's -32 fold)
};

#define JAMHIP_DEV __device__ __forceinline__

JAMHIP_DEV float h2f(uint32_t bits16) { return (float) __builtin_bit_cast(_Float16, (uint16_t) bits16); }

JAMHIP_DEV int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

JAMHIP_DEV float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// E8M0 -> 2^(e-128) (jam/jam-native/src/kernels/jam_mxfp4.h:17-24): e=0 -> 2^-128, e=255 -> +Inf.
JAMHIP_DEV float e8m0_half(uint32_t e) {
    uint32_t bits = e == 0 ? 0x00400000u : (e << 23);
    return 0.5f * __builtin_bit_cast(float, bits);
}

}  // namespace jamhip
