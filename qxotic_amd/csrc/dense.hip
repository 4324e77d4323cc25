// Dense weights (F32, F16, BF16) @ F32 activations -> F32: jam's dense paths (jam/jam-native/src/jam.c:596-660).
//
// Semantics. F32 and F16 weights multiply the f32 activations as they are (f16 -> f32 is exact); BF16 weights
// multiply activations rounded to bf16 (round to nearest even) wherever jam's bf16 kernels take the call on an
// AVX-512-BF16 host (n >= 8 with k even: the packed-panel kernel; k % 32 == 0: the convert-once kernel) and the
// f32 activations otherwise (the convert-and-FMA floor). Every product is exact in f32 (bf16 x bf16, f16 x f32
// and f32 x f32 products are formed exactly by the FMA / the matrix cores); only the f32 summation order
// differs from jam's.
//
// Layout. A device copy keeps the rows row-major, each padded with zeros to a 256-byte pitch (WeightView::G),
// so every row starts 16-byte aligned and a 16-byte load never crosses into the next row.
//
// Kernels.
//  * dense_gemv_kernel (n <= 8; HBM-bound): a wave streams 8 rows with 16-byte loads and keeps NT tokens'
//    dot products in registers; the activations come from L2 and are reused by the wave's 8 rows.
//  * dense_mfma_kernel (n > 8): each wave owns 32 rows x 64 tokens on the matrix cores, its A and B fragments
//    loaded straight from global memory: v_mfma_f32_32x32x16_bf16 on bf16-rounded activations, else
//    v_mfma_f32_32x32x2_f32 on exact f32 operands.
#include "common.h"
#include "launch.h"

namespace jamhip {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// jam's bf16 activation rounding (vcvtne2ps2bf16): round to nearest even on the dropped 16 bits; NaN stays NaN.
JAMHIP_DEV uint32_t bf16_bits(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
JAMHIP_DEV float bf16_round(float x) { return __builtin_bit_cast(float, bf16_bits(x) << 16); }

// 16 weight bytes -> V = 16 / element size f32 values
template <int DT> JAMHIP_DEV void wvals(const uint4 v, float* f) {
    if constexpr (DT == F32) {
        f[0] = __builtin_bit_cast(float, v.x);
        f[1] = __builtin_bit_cast(float, v.y);
        f[2] = __builtin_bit_cast(float, v.z);
        f[3] = __builtin_bit_cast(float, v.w);
    } else {
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if constexpr (DT == F16) {
                f[2 * i] = h2f(u[i] & 0xffffu);
                f[2 * i + 1] = h2f(u[i] >> 16);
            } else {
                f[2 * i] = __builtin_bit_cast(float, u[i] << 16);
                f[2 * i + 1] = __builtin_bit_cast(float, u[i] & 0xffff0000u);
            }
        }
    }
}

JAMHIP_DEV uint4 ld16_nt(const void* p) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

constexpr int DG_WAVES = 4, DG_RPW = 8;   // GEMV: waves per workgroup, rows per wave

// ------------------------------------------------------------------------------------------ GEMV
template <int DT, int NT>
__global__ void __launch_bounds__(64 * DG_WAVES) dense_gemv_kernel(WeightView w, const float* __restrict__ a, int lda,
                                                                   int k, int m, int n, float* __restrict__ c, int ldc,
                                                                   int rnd, Epi ep) {
    constexpr int ES = block_bytes(DT), V = 16 / ES;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row0 = ((int64_t) blockIdx.x * DG_WAVES + wave) * DG_RPW;
    if (row0 >= m) return;   // wave-uniform; the kernel has no barrier
    const int t0 = blockIdx.y * NT, ntv = n - t0 < NT ? n - t0 : NT;
    const uint8_t* wr[DG_RPW];
#pragma unroll
    for (int r = 0; r < DG_RPW; r++) {
        const int64_t row = row0 + r < m ? row0 + r : m - 1;
        wr[r] = w.qs + (w.r0 + row) * w.G;
    }
    float acc[DG_RPW][NT];
#pragma unroll
    for (int r = 0; r < DG_RPW; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[r][t] = 0.0f;
    for (int e0 = lane * V; e0 < k; e0 += 64 * V) {   // e0·ES + 16 <= the pitch: pieces never cross rows
        uint4 raw[DG_RPW];
#pragma unroll
        for (int r = 0; r < DG_RPW; r++) raw[r] = ld16_nt(wr[r] + (int64_t) e0 * ES);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (t >= ntv) break;
            const float* ar = a + (int64_t) (t0 + t) * lda;
            float x[V];
#pragma unroll
            for (int i = 0; i < V; i++) {
                const float v = e0 + i < k ? ar[e0 + i] : 0.0f;
                x[i] = rnd ? bf16_round(v) : v;
            }
#pragma unroll
            for (int r = 0; r < DG_RPW; r++) {
                float f[V];
                wvals<DT>(raw[r], f);
#pragma unroll
                for (int i = 0; i < V; i++) {
                    const float wv = e0 + i < k ? f[i] : 0.0f;   // a pinned row's columns past k may hold anything
                    acc[r][t] = fmaf(wv, x[i], acc[r][t]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < DG_RPW; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float v = wave_sum(acc[r][t]);
            const int64_t row = row0 + r;
            if (lane == 0 && t < ntv && row < m) {
                float* dst = c + (int64_t) (t0 + t) * ldc + row;
                *dst = epilogue(ep, v, row, dst);
            }
        }
}

// ------------------------------------------------------------------------------------------ GEMM
// Wave tile: 32 rows x 64 tokens (two 32x32 accumulators sharing the A fragment). Lane (r, q) = (lane % 32,
// lane / 32) loads row r's and token r's operands for the K positions the instruction assigns to q; the
// accumulator holds token r, rows 8·(e / 4) + 4q + e % 4.
constexpr int DM_WAVES = 4;

template <int DT, bool BF16MMA>
__global__ void __launch_bounds__(64 * DM_WAVES) dense_mfma_kernel(WeightView w, const float* __restrict__ a, int lda,
                                                                   int k, int m, int n, float* __restrict__ c, int ldc,
                                                                   Epi ep) {
    constexpr int ES = block_bytes(DT);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane & 31, q = lane >> 5;
    const int64_t row0 = ((int64_t) blockIdx.x * DM_WAVES + wave) * 32;
    if (row0 >= m) return;   // wave-uniform; no barrier
    const int t0 = blockIdx.y * 64;
    const int64_t wrow = row0 + r < m ? row0 + r : m - 1;
    const uint8_t* wp = w.qs + (w.r0 + wrow) * w.G;
    const int tA = t0 + r, tB = t0 + 32 + r;
    const float* aA = a + (int64_t) (tA < n ? tA : n - 1) * lda;
    const float* aB = a + (int64_t) (tB < n ? tB : n - 1) * lda;
    const bool vA = tA < n, vB = tB < n;
    floatx16 accA = floatx16{}, accB = floatx16{};
    if constexpr (BF16MMA) {
        // one 32x32x16 step: lane (r, q) holds K positions 8q .. 8q + 7 of the step
        for (int k0 = 0; k0 < k; k0 += 16) {
            const int kb = k0 + 8 * q;
            uint4 wv = kb < k ? *reinterpret_cast<const uint4*>(wp + (int64_t) kb * ES) : make_uint4(0, 0, 0, 0);
            if (kb + 8 > k) {   // the row's last piece: columns past k (a pinned row's may hold anything) -> 0
                uint32_t u[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (kb + i >= k) u[i >> 1] &= (i & 1) ? 0x0000ffffu : 0xffff0000u;
                wv = make_uint4(u[0], u[1], u[2], u[3]);
            }
            const bf16x8 A = __builtin_bit_cast(bf16x8, wv);
            uint32_t ba[4], bb[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int kk = kb + 2 * i;
                const uint32_t a0 = bf16_bits(kk < k && vA ? aA[kk] : 0.0f), a1 = bf16_bits(kk + 1 < k && vA ? aA[kk + 1] : 0.0f);
                const uint32_t b0 = bf16_bits(kk < k && vB ? aB[kk] : 0.0f), b1 = bf16_bits(kk + 1 < k && vB ? aB[kk + 1] : 0.0f);
                ba[i] = a0 | (a1 << 16);
                bb[i] = b0 | (b1 << 16);
            }
            const bf16x8 BA = __builtin_bit_cast(bf16x8, make_uint4(ba[0], ba[1], ba[2], ba[3]));
            const bf16x8 BB = __builtin_bit_cast(bf16x8, make_uint4(bb[0], bb[1], bb[2], bb[3]));
            accA = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, BA, accA, 0, 0, 0);
            accB = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, BB, accB, 0, 0, 0);
        }
    } else {
        // four 32x32x2 steps per 8 K positions: lane (r, q) loads positions 4q .. 4q + 3, step j takes the j-th
        for (int k0 = 0; k0 < k; k0 += 8) {
            const int kb = k0 + 4 * q;
            float wf[4];
            if constexpr (DT == F32) {
                const uint4 v = kb < k ? *reinterpret_cast<const uint4*>(wp + (int64_t) kb * 4) : make_uint4(0, 0, 0, 0);
                wvals<F32>(v, wf);
            } else {
                const uint2 v = kb < k ? *reinterpret_cast<const uint2*>(wp + (int64_t) kb * 2) : make_uint2(0, 0);
                float f8[8];
                wvals<DT>(make_uint4(v.x, v.y, 0u, 0u), f8);
#pragma unroll
                for (int i = 0; i < 4; i++) wf[i] = f8[i];
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int kk = kb + j;
                wf[j] = kk < k ? wf[j] : 0.0f;   // columns past k (a pinned row's may hold anything) -> 0
                const float xa = kk < k && vA ? aA[kk] : 0.0f, xb = kk < k && vB ? aB[kk] : 0.0f;
                accA = __builtin_amdgcn_mfma_f32_32x32x2f32(wf[j], xa, accA, 0, 0, 0);
                accB = __builtin_amdgcn_mfma_f32_32x32x2f32(wf[j], xb, accB, 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const int64_t row = row0 + 8 * (e >> 2) + 4 * q + (e & 3);
        if (row >= m) continue;
        if (vA) {
            float* dst = c + (int64_t) tA * ldc + row;
            *dst = epilogue(ep, accA[e], row, dst);
        }
        if (vB) {
            float* dst = c + (int64_t) tB * ldc + row;
            *dst = epilogue(ep, accB[e], row, dst);
        }
    }
}

// ----------------------------------------------------------------------------------------- launchers
// jam rounds BF16's activations to bf16 where its bf16 kernels take the call (jam.c:622-652).
static bool bf16_rounds(int n, int k) { return (n >= 8 && k % 2 == 0) || k % 32 == 0; }

template <int DT, int NT>
static void gemv_go(const WeightView& w, const float* a, int lda, int k, int m, int n, float* c, int ldc, int rnd,
                    hipStream_t st, const Epi& ep) {
    const int rows_per_wg = DG_WAVES * DG_RPW;
    const dim3 grid((unsigned) ((m + rows_per_wg - 1) / rows_per_wg), (unsigned) ((n + NT - 1) / NT));
    dense_gemv_kernel<DT, NT><<<grid, 64 * DG_WAVES, 0, st>>>(w, a, lda, k, m, n, c, ldc, rnd, ep);
}

template <int DT>
static hipError_t dense_go(const WeightView& w, const float* a, int lda, int k, int m, int n, float* c, int ldc,
                           hipStream_t st, const Epi& ep) {
    const bool rnd = DT == BF16 && bf16_rounds(n, k);
    if (n <= 8) {
        if (n == 1) gemv_go<DT, 1>(w, a, lda, k, m, n, c, ldc, rnd, st, ep);
        else if (n == 2) gemv_go<DT, 2>(w, a, lda, k, m, n, c, ldc, rnd, st, ep);
        else if (n <= 4) gemv_go<DT, 4>(w, a, lda, k, m, n, c, ldc, rnd, st, ep);
        else gemv_go<DT, 8>(w, a, lda, k, m, n, c, ldc, rnd, st, ep);
        return hipGetLastError();
    }
    const dim3 grid((unsigned) ((m + 32 * DM_WAVES - 1) / (32 * DM_WAVES)), (unsigned) ((n + 63) / 64));
    if constexpr (DT == BF16) {
        if (rnd) {
            dense_mfma_kernel<DT, true><<<grid, 64 * DM_WAVES, 0, st>>>(w, a, lda, k, m, n, c, ldc, ep);
            return hipGetLastError();
        }
    }
    dense_mfma_kernel<DT, false><<<grid, 64 * DM_WAVES, 0, st>>>(w, a, lda, k, m, n, c, ldc, ep);
    return hipGetLastError();
}

hipError_t launch_dense(int dt, const WeightView& w, const float* a, int lda, int k, int m, int n, float* c, int ldc,
                        hipStream_t st, const Epi& ep) {
    switch (dt) {
    case F32: return dense_go<F32>(w, a, lda, k, m, n, c, ldc, st, ep);
    case F16: return dense_go<F16>(w, a, lda, k, m, n, c, ldc, st, ep);
    case BF16: return dense_go<BF16>(w, a, lda, k, m, n, c, ldc, st, ep);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace jamhip
