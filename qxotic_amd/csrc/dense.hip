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
//  * dense_gemv2_kernel (n <= 8 while the token tile's activations fit 64 KB of LDS; HBM-bound): activations
//    staged in LDS, each wave streaming 1..4 rows two 16-byte pieces per lane deep; dense_gemv_kernel
//    otherwise: a wave streams 8 rows with 16-byte loads, the activations from L2.
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

// GEMV with the activations in LDS and the weight stream two steps deep in registers (n <= 8 where the NT-token
// tile's activations fit 64 KB of LDS). A workgroup of 4 waves stages its tile's activations (bf16-rounded
// where jam rounds them; zero past k), each wave streams RPW rows: per step a lane loads one 16-byte piece of
// every row (the wave reads RPW contiguous 1 KB runs), and step j + 1's pieces are in flight while step j
// is multiplied. The loads are unconditional (a step past the row's end re-reads the last piece and adds
// nothing), so the compiler waits for exactly the step it computes. Columns past k inside a row's last
// piece are zeroed before use (a pinned row's may hold anything, NaN included).
constexpr int DG2_LDS_MAX = 64 * 1024;

template <int DT, int NT, int RPW>
__global__ void __launch_bounds__(64 * DG_WAVES) dense_gemv2_kernel(WeightView w, const float* __restrict__ a, int lda,
                                                                    int k, int m, int n, float* __restrict__ c,
                                                                    int ldc, int rnd, int kp, Epi ep) {
    constexpr int ES = block_bytes(DT), V = 16 / ES;
    extern __shared__ __align__(16) float xs[];   // [NT][kp], kp a multiple of 64·V
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t0 = blockIdx.y * NT, ntv = n - t0 < NT ? n - t0 : NT;
    const int64_t row0 = ((int64_t) blockIdx.x * DG_WAVES + wave) * RPW;
    const int S = kp / (64 * V);                  // steps per row
    const uint8_t* wr[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const int64_t row = row0 + r < m ? row0 + r : m - 1;
        wr[r] = w.qs + (w.r0 + row) * w.G;
    }
    // the last piece holding a column of the row: later steps re-read it (in bounds of the row's pitch)
    const int elast = (k - 1) / V * V;
    auto load = [&](uint4 (&raw)[RPW], int j) {
        const int e0 = min((j * 64 + lane) * V, elast);
#pragma unroll
        for (int r = 0; r < RPW; r++) raw[r] = ld16_nt(wr[r] + (int64_t) e0 * ES);
    };
    uint4 raw[2][RPW];
    load(raw[0], 0);
    load(raw[1], 1);
    // stage the tile's activations: float4 slots of [NT][kp]
    const int q4 = kp / 4;
    for (int i = threadIdx.x; i < NT * q4; i += 64 * DG_WAVES) {
        const int t = i / q4, e = 4 * (i - t * q4);
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float x = t < ntv && e + u < k ? a[(int64_t) (t0 + t) * lda + e + u] : 0.0f;
            v[u] = rnd ? bf16_round(x) : x;
        }
        *reinterpret_cast<float4*>(xs + (int64_t) t * kp + e) = make_float4(v[0], v[1], v[2], v[3]);
    }
    __syncthreads();
    if (row0 >= m) return;   // wave-uniform; after the workgroup's only barrier
    float acc[RPW][NT];
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[r][t] = 0.0f;
    auto step = [&](const uint4 (&rv)[RPW], int j) {
        const int e0 = (j * 64 + lane) * V;
        const bool tail = e0 + V > k;   // the row's last piece (or past it): columns >= k -> 0
        float f[RPW][V];
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            wvals<DT>(rv[r], f[r]);
            if (tail)
#pragma unroll
                for (int i = 0; i < V; i++) f[r][i] = e0 + i < k ? f[r][i] : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (t >= ntv) break;
            float x[V];
#pragma unroll
            for (int i = 0; i < V; i += 4) {
                const float4 v = *reinterpret_cast<const float4*>(xs + (int64_t) t * kp + e0 + i);
                x[i] = v.x, x[i + 1] = v.y, x[i + 2] = v.z, x[i + 3] = v.w;
            }
#pragma unroll
            for (int r = 0; r < RPW; r++)
#pragma unroll
                for (int i = 0; i < V; i++) acc[r][t] = fmaf(f[r][i], x[i], acc[r][t]);
        }
    };
    for (int j = 0; j < S; j += 2) {
        step(raw[0], j);
        load(raw[0], j + 2);
        if (j + 1 < S) step(raw[1], j + 1);
        load(raw[1], j + 3);
    }
#pragma unroll
    for (int r = 0; r < RPW; r++)
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
    if (vA) store_column(c + (int64_t) tA * ldc, row0 + 4 * q, m, accA, 1.0f, ep, false);
    if (vB) store_column(c + (int64_t) tB * ldc, row0 + 4 * q, m, accB, 1.0f, ep, false);
}

// ------------------------------------------------------------------------- staged matrix-core GEMM (n >= 9)
// F16 weights and BF16 weights with bf16-rounded activations (k even or k % 32 == 0: jam's bf16 kernels) run
// on the f16 / bf16 matrix cores with LDS-staged operands, the structure of the quantized prefill GEMM
// (mma.hip) without its per-block scales:
//  * dense_prep_kernel (one workgroup per token) writes the activations in the MFMA operand order, planes
//    [Kp/16 K-steps][2 halves][NP slots][8] (half h = elements 8h..8h+7 of the K-step, zero past k): for F16
//    weights the f16 high part and f16 remainder of x·2^-e_t, e_t putting the token's largest |x| in
//    [2^14, 2^15) (hi + lo hold x to about 22 bits), and es[t] = 2^e_t; for BF16 weights jam's bf16(x), es = 1.
//  * dense_mma_kernel: a workgroup of 4 waves owns 128 rows x 64 tokens and walks k in stages of 64 elements.
//    Each stage's operands are copied global -> LDS by the waves (global_load_lds, double-buffered): a wave's
//    own 32 rows as 8 pieces of 32 rows x 16 bytes (lane r of a piece reads row r: the LDS tile is the
//    fragment layout, conflict-free to read), and 1 KB pieces of the activation planes. Per 16-element K-step
//    and 32-token tile one MFMA per plane: f16 weights x hi, then x lo; bf16 x bf16. Products are exact in f32;
//    only the summation order differs from jam's f32 FMA chain, plus for F16 the ~2^-22 relative remainder
//    of x that hi + lo drop. Weight columns past k in the last stage are zeroed in the fragment (a pinned
//    row's may hold anything). Small grids split k like the quantized GEMM (partials summed in slice order).
constexpr int DMM_STAGE = 64;

int dense_mma_planes(int dt, int n, int k);   // below
static int dense_np(int n) { return (n + 63) / 64 * 64; }
static int dense_kp(int k) { return (k + DMM_STAGE - 1) / DMM_STAGE * DMM_STAGE; }

size_t dense_act_bytes(int dt, int n, int k) {
    const int pl = dense_mma_planes(dt, n, k);
    const size_t plane = ((size_t) dense_kp(k) * dense_np(n) * 2 + 255) / 256 * 256;
    return pl * plane + ((size_t) dense_np(n) * 4 + 255) / 256 * 256;
}

__global__ void __launch_bounds__(256) dense_prep_kernel(const float* __restrict__ a, int lda, int n, int k, int Kp,
                                                         int NP, int hl, uint16_t* __restrict__ hi,
                                                         uint16_t* __restrict__ lo, float* __restrict__ es) {
    __shared__ float wmax[4];
    const int t = blockIdx.x;
    const float* x = a + (int64_t) t * lda;
    float down = 1.0f;
    if (hl) {   // the token's largest |x|; a non-finite one leaves the scale at 1 (the outputs go non-finite)
        float mx = 0.0f;
        for (int e = threadIdx.x; e < k; e += 256) mx = fmaxf(mx, fabsf(x[e]));
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = mx;
        __syncthreads();
        mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
        int ex;
        if (mx > 0.0f && mx <= 3.40282347e38f) {
            int e2;
            frexpf(mx, &e2);   // mx in [2^(e2-1), 2^e2)
            ex = 15 - e2;
            ex = ex > 126 ? 126 : ex;
        } else {
            ex = 0;
        }
        down = ldexpf(1.0f, ex);
        if (threadIdx.x == 0) es[t] = ldexpf(1.0f, -ex);
    } else if (threadIdx.x == 0) {
        es[t] = 1.0f;
    }
    // 8-element runs: run g = elements 8g..8g+7 = K-step g / 2, half g % 2
    for (int g = threadIdx.x; g < Kp / 8; g += 256) {
        float v[8];
        const int e0 = 8 * g;
        if (e0 + 8 <= k && ((reinterpret_cast<uintptr_t>(x + e0) & 15) == 0)) {
            const float4 f0 = *reinterpret_cast<const float4*>(x + e0), f1 = *reinterpret_cast<const float4*>(x + e0 + 4);
            v[0] = f0.x, v[1] = f0.y, v[2] = f0.z, v[3] = f0.w, v[4] = f1.x, v[5] = f1.y, v[6] = f1.z, v[7] = f1.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = e0 + i < k ? x[e0 + i] : 0.0f;
        }
        uint32_t h[4], l[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (hl) {
                const F16Pair p0 = split_f16(v[2 * i] * down), p1 = split_f16(v[2 * i + 1] * down);
                h[i] = (uint32_t) __builtin_bit_cast(uint16_t, p0.hi) | ((uint32_t) __builtin_bit_cast(uint16_t, p1.hi) << 16);
                l[i] = (uint32_t) __builtin_bit_cast(uint16_t, p0.lo) | ((uint32_t) __builtin_bit_cast(uint16_t, p1.lo) << 16);
            } else {
                h[i] = bf16_bits(v[2 * i]) | (bf16_bits(v[2 * i + 1]) << 16);
            }
        }
        const int64_t o = ((int64_t) g * NP + t) * 8;   // (K-step g/2, half g%2) = plane row g
        *reinterpret_cast<uint4*>(hi + o) = make_uint4(h[0], h[1], h[2], h[3]);
        if (hl) *reinterpret_cast<uint4*>(lo + o) = make_uint4(l[0], l[1], l[2], l[3]);
    }
}

typedef _Float16 half8d __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void_d;

template <bool HL>
__global__ void __launch_bounds__(256, 2) dense_mma_kernel(WeightView w, const uint16_t* __restrict__ xh,
                                                           const uint16_t* __restrict__ xl, const float* __restrict__ es,
                                                           int NP, int Kp, int k, int m, int n, float* __restrict__ c,
                                                           int ldc, int nrb, int ncb, int st_per, int64_t c_slice,
                                                           Epi ep) {
    constexpr int PL = HL ? 2 : 1, A_BYTES = 4 * 4096, BYTES = A_BYTES + PL * 8192;
    extern __shared__ __align__(1024) unsigned char dsm[];
    const int total = nrb * ncb, lin = tile_of_block(false, total);
    if (lin >= total) return;
    const int rb = lin / ncb, cb = lin % ncb;
    const int lane = threadIdx.x & 63, r = lane & 31, q = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t row0 = (int64_t) rb * 128 + 32 * wave;
    const int n0 = cb * 64;
    const int nstk = Kp / DMM_STAGE;
    const int st0 = st_per > 0 ? st_per * (int) blockIdx.y : 0;
    const int nst = st_per > 0 ? min(nstk, st0 + st_per) : nstk;
    const int64_t crow = row0 + r < m ? row0 + r : m - 1;   // the row this lane copies (clamped to the view)
    const uint8_t* wrow = w.qs + (w.r0 + crow) * w.G + 16 * q;
    const uint16_t* bsrc = xh + ((int64_t) (2 * wave) * NP + n0) * 8 + 8 * lane;
    const int64_t plane_off = xl - xh;
    auto issue = [&](int st, unsigned char* buf) {
        // weights: pieces 2i + q (elements 64·st + 8(2i + q)..) of row r, 4 instructions of 1 KB
#pragma unroll
        for (int i = 0; i < 4; i++)
            __builtin_amdgcn_global_load_lds(wrow + ((int64_t) DMM_STAGE * st + 16 * i) * 2,
                                             (lds_void_d*) (buf + wave * 4096 + i * 1024), 16, 0, 0);
        // activations: plane rows 8·st + 2·wave and + 1 (K-step 4st + wave, halves 0 and 1), 1 KB each
#pragma unroll
        for (int pl = 0; pl < PL; pl++)
#pragma unroll
            for (int h = 0; h < 2; h++)
                __builtin_amdgcn_global_load_lds(bsrc + pl * plane_off + ((int64_t) (8 * st + h)) * NP * 8,
                                                 (lds_void_d*) (buf + A_BYTES + pl * 8192 + (2 * wave + h) * 1024), 16, 0,
                                                 0);
    };
    floatx16 acc[2] = {floatx16{}, floatx16{}};
    issue(st0, dsm + (st0 & 1) * BYTES);   // a K slice may start on an odd stage
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int st = st0; st < nst; st++) {
        unsigned char* buf = dsm + (st & 1) * BYTES;
        uint4 af[4];
        uint4 bf[PL][4][2];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            af[ks] = *reinterpret_cast<const uint4*>(buf + wave * 4096 + (2 * ks + q) * 512 + 16 * r);
#pragma unroll
            for (int pl = 0; pl < PL; pl++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    bf[pl][ks][j] = *reinterpret_cast<const uint4*>(buf + A_BYTES + pl * 8192 + (2 * ks + q) * 1024 +
                                                                   (32 * j + r) * 16);
        }
        if (DMM_STAGE * (st + 1) > k) {   // the stage holding column k - 1: columns >= k -> 0
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const int e0 = DMM_STAGE * st + 16 * ks + 8 * q;
                uint32_t u[4] = {af[ks].x, af[ks].y, af[ks].z, af[ks].w};
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (e0 + i >= k) u[i >> 1] &= (i & 1) ? 0x0000ffffu : 0xffff0000u;
                af[ks] = make_uint4(u[0], u[1], u[2], u[3]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (st + 1 < nst) issue(st + 1, dsm + ((st + 1) & 1) * BYTES);
#pragma unroll
        for (int ks = 0; ks < 4; ks++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int pl = 0; pl < PL; pl++) {
                    if constexpr (HL)
                        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8d, af[ks]),
                                                                        __builtin_bit_cast(half8d, bf[pl][ks][j]), acc[j], 0, 0, 0);
                    else
                        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[ks]),
                                                                         __builtin_bit_cast(bf16x8, bf[pl][ks][j]), acc[j], 0, 0, 0);
                }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    // lane holds token n0 + 32j + r, rows 8·(e/4) + 4q + e%4 of the wave's 32; a K slice writes its partial
    // result at c + y·c_slice
    if (st_per > 0) c += (int64_t) blockIdx.y * c_slice;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int t = n0 + 32 * j + r;
        if (t >= n) continue;
        const float sc = es[t];
        store_column(c + (int64_t) t * ldc, row0 + 4 * q, m, acc[j], sc, ep, st_per > 0);
    }
}

// ----------------------------------------------------------------------------------------- launchers
// jam rounds BF16's activations to bf16 where its bf16 kernels take the call (jam.c:622-652).
static bool bf16_rounds(int n, int k) { return (n >= 8 && k % 2 == 0) || k % 32 == 0; }

template <int DT, int NT, int RPW>
static void gemv2_go(const WeightView& w, const float* a, int lda, int k, int kp, int m, int n, float* c, int ldc,
                     int rnd, hipStream_t st, const Epi& ep) {
    const int rows_per_wg = DG_WAVES * RPW;
    const dim3 grid((unsigned) ((m + rows_per_wg - 1) / rows_per_wg), (unsigned) ((n + NT - 1) / NT));
    dense_gemv2_kernel<DT, NT, RPW><<<grid, 64 * DG_WAVES, (size_t) NT * kp * 4, st>>>(w, a, lda, k, m, n, c, ldc, rnd,
                                                                                       kp, ep);
}

template <int DT, int NT>
static void gemv_go(const WeightView& w, const float* a, int lda, int k, int m, int n, float* c, int ldc, int rnd,
                    hipStream_t st, const Epi& ep) {
    constexpr int V = 16 / block_bytes(DT);
    const int kp = (k + 64 * V - 1) / (64 * V) * (64 * V);
    if ((size_t) NT * kp * 4 <= (size_t) DG2_LDS_MAX) {
        // rows per wave: about 2048 waves or more over the device, 4 rows a wave at most
        if (m >= 4 * 2048) return gemv2_go<DT, NT, 4>(w, a, lda, k, kp, m, n, c, ldc, rnd, st, ep);
        if (m >= 2 * 2048) return gemv2_go<DT, NT, 2>(w, a, lda, k, kp, m, n, c, ldc, rnd, st, ep);
        return gemv2_go<DT, NT, 1>(w, a, lda, k, kp, m, n, c, ldc, rnd, st, ep);
    }
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

// 2 planes (F16: hi, lo), 1 (BF16 with jam's bf16 rounding), 0: the staged GEMM does not take the call. It
// takes n >= DENSE_MMA_MIN_N, and from 2 tokens the calls whose token tile's activations would not fit the
// LDS-staged GEMV (k = 14336 at n = 2: 63 against 95 us for BF16 4096x14336; k = 4096 at n = 8: 63 against
// 128 us for F16 14336x4096). The staged GEMV stays ahead where it fits (F16 14336x4096 n = 4: 46 against 63).
int dense_mma_planes(int dt, int n, int k) {
    if (dt != F16 && !(dt == BF16 && bf16_rounds(n, k))) return 0;
    if (n < DENSE_MMA_MIN_N) {
        if (n < 2) return 0;
        const int nt = n == 2 ? 2 : n <= 4 ? 4 : 8, kp = (k + 64 * 8 - 1) / (64 * 8) * (64 * 8);
        if ((size_t) nt * kp * 4 <= (size_t) DG2_LDS_MAX) return 0;
    }
    return dt == F16 ? 2 : 1;
}

// K slices for a grid of `total` workgroups: about two workgroups per CU (the quantized GEMM's rule).
static void dense_split(int total, int nstk, int* ns, int* st_per) {
    int want = total >= 384 ? 1 : (512 + total - 1) / total;
    want = want < nstk ? want : nstk;
    *st_per = want > 1 ? (nstk + want - 1) / want : 0;
    *ns = want > 1 ? (nstk + *st_per - 1) / *st_per : 1;
}

size_t dense_mma_split_floats(int dt, int k, int m, int n) {
    if (!dense_mma_planes(dt, n, k)) return 0;
    int ns, st_per;
    dense_split(((m + 127) / 128) * (dense_np(n) / 64), dense_kp(k) / DMM_STAGE, &ns, &st_per);
    return ns > 1 ? (size_t) ns * n * m : 0;
}

hipError_t launch_dense_mma(int dt, const WeightView& w, const float* a, int lda, int k, int m, int n, float* c,
                            int ldc, void* scratch, float* part, hipStream_t st, const Epi& ep) {
    const int pl = dense_mma_planes(dt, n, k);
    if (!pl) return hipErrorNotSupported;
    const int NP = dense_np(n), Kp = dense_kp(k);
    const size_t plane = ((size_t) Kp * NP * 2 + 255) / 256 * 256;
    uint16_t* xh = (uint16_t*) scratch;
    uint16_t* xl = (uint16_t*) ((uint8_t*) scratch + plane);
    float* es = (float*) ((uint8_t*) scratch + pl * plane);
    dense_prep_kernel<<<n, 256, 0, st>>>(a, lda, n, k, Kp, NP, pl == 2, xh, pl == 2 ? xl : xh, es);
    const int nrb = (m + 127) / 128, ncb = NP / 64, total = nrb * ncb;
    int ns, st_per;
    dense_split(total, Kp / DMM_STAGE, &ns, &st_per);
    if (ns > 1 && part == nullptr) return hipErrorInvalidValue;
    const int grid = tile_grid(false, total);
    float* out = ns > 1 ? part : c;
    const int ldo = ns > 1 ? m : ldc;
    const int64_t slice = (int64_t) n * m;
    const size_t lds = 2 * (size_t) (4 * 4096 + pl * 8192);
    if (pl == 2)
        dense_mma_kernel<true><<<dim3(grid, ns), 256, lds, st>>>(w, xh, xl, es, NP, Kp, k, m, n, out, ldo, nrb, ncb,
                                                                 st_per, slice, ns > 1 ? Epi{} : ep);
    else
        dense_mma_kernel<false><<<dim3(grid, ns), 256, lds, st>>>(w, xh, xh, es, NP, Kp, k, m, n, out, ldo, nrb, ncb,
                                                                  st_per, slice, ns > 1 ? Epi{} : ep);
    if (ns > 1) return launch_split_reduce(part, ns, slice, m, n, c, ldc, st, ep);
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
