// Prefill GEMM for n >= 32 tokens: C[n][m] = W[m][k] · A[n][k]^T with jam's F2 semantics (the n >= 8
// bands of jam_kernels_q4k_avx512.c): activations quantized per 32 to int8 (quant_f2_kernel), every
// 32-element block's integer dot combined in f32 with the block's weight and activation scales.
//
// Matrix-core mapping. The integer block dots run on v_mfma_f32_16x16x32_f16 with integer-valued
// operands that f16 holds exactly: the activation codes (int8) and, per weight type, the weight codes
// with the block's integer sub-scale folded in — Q4_K sc·nib (<= 945), Q6_K sc·q6 split as
// 64·(v >> 6) + (v & 63), Q8_0 q, Q4_0 nib, MXFP4 e2m1 code·2. Every product is an integer of at most
// 20 bits and every block sum stays below 2^24, so the MFMA's f32 result is the exact integer dot
// (Q6_K's two-plane sum may round in its last bit above 2^24). With the sub-scale inside the
// operand, each 32-block costs one f32 FMA per output (its activation scale) instead of the convert,
// scale product and FMA that an int32 result would need, and K-quant row scales apply once per
// super-block.
//
// Per-type combine (jam's F2 decompositions, summed in a different order):
//   Q4_K  d·Σ_s dx_s·(Σ sc_s·nib·xq)  −  Σ_s fl(dmin·mn_s)·fl(xs0+xs1)          (q4k_avx512.c:76-95)
//   Q6_K  d·Σ_s dx_s·(Σ sc·q6·xq)     −  Σ_t fl(d·sc_t)·fl(32·xs16_t)           (q4k_avx512.c:222-236)
//   Q8_0  Σ_s fl(d_s·dx_s)·Σ q·xq                                               (q4k_avx512.c:347-362)
//   Q4_0  Σ_s fl(d_s·dx_s)·Σ nib·xq  −  fl(8·d_s)·fl(xs0+xs1)                   (q4k_avx512.c:463-480)
//   MXFP4 Σ_s fl(dhalf_s·dx_s)·Σ code·xq                                        (q4k_avx512.c:692-711)
//
// Tiling. A 256-thread workgroup (2x2 waves) owns BM weight rows x BN tokens and walks K in chunks of
// 256 elements (one super-block, or 8 blocks of 32): it dequantizes the chunk's weight codes to f16 in
// LDS (rows padded by 16 bytes so fragment reads are conflict-free), converts the chunk's int8
// activations to f16 in LDS, stages the per-block scales, then each wave runs its (BM/2)x(BN/2) tile
// of 16x16 MFMA blocks.
#include "common.h"
#include "launch.h"

namespace jamhip {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int KC = 256;           // K elements per chunk
constexpr int LROW = KC + 8;      // f16 per LDS row

template <int DT> constexpr int planes() { return DT == Q6_K ? 2 : 1; }
template <int DT> constexpr bool kquant() { return DT == Q4_K || DT == Q6_K; }

template <int DT, int BM, int BN> struct GemmSmem {
    _Float16 a[planes<DT>()][BM][LROW];
    _Float16 b[BN][LROW];
    float dx[8][BN];      // activation scale of each block of the chunk
    float xs[16][BN];     // Q4_K / Q4_0: xs0 + xs1 per block; Q6_K: 32·xs16 per 16-group
    float ws[16][BM];     // Q4_K: dmin·mn per block; Q6_K: d·sc per 16-group; Q8_0/Q4_0/MXFP4: block scale
    float ws2[8][BM];     // Q4_0: 8·d per block
    float d[BM];          // K-quants: super-block scale d
};

JAMHIP_DEV uint4 gld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
JAMHIP_DEV uint32_t gld_u16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

// 16 consecutive f16 values into LDS (two 16-byte stores).
JAMHIP_DEV void st16h(_Float16* dst, const float (&v)[16]) {
    half8 lo, hi;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        lo[i] = (_Float16) v[i];
        hi[i] = (_Float16) v[8 + i];
    }
    *reinterpret_cast<half8*>(dst) = lo;
    *reinterpret_cast<half8*>(dst + 8) = hi;
}

JAMHIP_DEV int bytei(const uint4& v, int j) {   // unsigned byte j of a 16-byte vector
    const uint32_t w = j < 4 ? v.x : j < 8 ? v.y : j < 12 ? v.z : v.w;
    return (int) ((w >> (8 * (j & 3))) & 0xff);
}

JAMHIP_DEV void q4k_scale_min(const uint4 h, int s, int& sc, int& mn) {   // jam_kquant.h:26-33
    const uint8_t* b = reinterpret_cast<const uint8_t*>(&h) + 4;
    if (s < 4) {
        sc = b[s] & 63;
        mn = b[s + 4] & 63;
    } else {
        sc = (b[s + 4] & 15) | ((b[s - 4] >> 6) << 4);
        mn = (b[s + 4] >> 4) | ((b[s] >> 6) << 4);
    }
}

JAMHIP_DEV int mx_code(int nib) {   // e2m1 value x2 (jam_mxfp4.h:14-15)
    const int mag = (nib & 7) < 4 ? (nib & 7) : (nib & 7) == 4 ? 4 : (nib & 7) == 5 ? 6 : (nib & 7) == 6 ? 8 : 12;
    return nib & 8 ? -mag : mag;
}

// Stage the weight codes (and per-row scales) of rows [m0, m0+BM), chunk kc (= layout group kc/256), into
// LDS. Unit u of a row is 32 elements: Q4_K chunk u, Q6_K ql chunk u (+ its qh chunk), or block u.
template <int DT, int BM, int BN>
JAMHIP_DEV void stage_w(GemmSmem<DT, BM, BN>& S, const WeightView& w, int64_t m0, int m, int kc, int nblk) {
    const int64_t g = kc / 256;
    for (int ui = threadIdx.x; ui < BM * 8; ui += 256) {
        const int row = ui >> 3, u = ui & 7;
        const int64_t grow = m0 + row < m ? m0 + row : m - 1;   // clamp: in bounds, never stored
        const uint8_t* rq = group_q<DT>(w, grow, g);
        const uint8_t* rs = group_s<DT>(w, grow, g);
        auto chunk = [&](int c) { return gld16(rq + c * CHUNK_STRIDE); };
        float v[16], v2[16];
        if constexpr (DT == Q4_K) {
            const uint4 q = chunk(u);
            const uint4 h = gld16(rs);
            const int gp = u >> 1, e0 = 16 * (u & 1);
            int sc0, mn0, sc1, mn1;
            q4k_scale_min(h, 2 * gp, sc0, mn0);
            q4k_scale_min(h, 2 * gp + 1, sc1, mn1);
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int b = bytei(q, j);
                v[j] = (float) (sc0 * (b & 15));
                v2[j] = (float) (sc1 * (b >> 4));
            }
            st16h(&S.a[0][row][64 * gp + e0], v);
            st16h(&S.a[0][row][64 * gp + 32 + e0], v2);
            if (u == 0) {
                const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
                S.d[row] = d;
#pragma unroll
                for (int sb = 0; sb < 8; sb++) {
                    int sc, mn;
                    q4k_scale_min(h, sb, sc, mn);
                    S.ws[sb][row] = dmin * (float) mn;
                }
            }
        } else if constexpr (DT == Q6_K) {
            const int h = u >> 2, jj = (u >> 1) & 1, lh = u & 1;
            const uint4 ql = chunk(u);
            const uint4 qh = chunk(8 + 2 * h + lh);
            const uint4 scv = chunk(12);
            const int8_t* scs = reinterpret_cast<const int8_t*>(&scv);
            const int sca = scs[8 * h + 2 * jj + lh], scb = scs[8 * h + 2 * (jj + 2) + lh];
            float p0[16], p1[16], r0[16], r1[16];
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int bl = bytei(ql, j), bh = bytei(qh, j);
                const int qa = (bl & 15) | (((bh >> (2 * jj)) & 3) << 4);
                const int qb = (bl >> 4) | (((bh >> (2 * jj + 4)) & 3) << 4);
                const int va = sca * qa, vb = scb * qb;
                p0[j] = (float) (64 * (va >> 6));
                p1[j] = (float) (va & 63);
                r0[j] = (float) (64 * (vb >> 6));
                r1[j] = (float) (vb & 63);
            }
            const int ea = 128 * h + 32 * jj + 16 * lh, eb = ea + 64;
            st16h(&S.a[0][row][ea], p0);
            st16h(&S.a[planes<DT>() - 1][row][ea], p1);
            st16h(&S.a[0][row][eb], r0);
            st16h(&S.a[planes<DT>() - 1][row][eb], r1);
            if (u == 0) {
                const float d = h2f(gld_u16(rs));
                S.d[row] = d;
#pragma unroll
                for (int t = 0; t < 16; t++) S.ws[t][row] = d * (float) scs[t];
            }
        } else {
            if (u >= nblk) continue;
            if constexpr (DT == Q8_0) {
                const uint4 q0 = chunk(2 * u), q1 = chunk(2 * u + 1);
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    v[j] = (float) (int8_t) bytei(q0, j);
                    v2[j] = (float) (int8_t) bytei(q1, j);
                }
                S.ws[u][row] = h2f(gld_u16(rs + 2 * u));
            } else if constexpr (DT == Q4_0) {
                const uint4 q = chunk(u);
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    v[j] = (float) (bytei(q, j) & 15);
                    v2[j] = (float) (bytei(q, j) >> 4);
                }
                const float d = h2f(gld_u16(rs + 2 * u));
                S.ws[u][row] = d;
                S.ws2[u][row] = 8.0f * d;
            } else {
                const uint4 q = chunk(u);
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    v[j] = (float) mx_code(bytei(q, j) & 15);
                    v2[j] = (float) mx_code(bytei(q, j) >> 4);
                }
                S.ws[u][row] = e8m0_half(rs[u]);
            }
            st16h(&S.a[0][row][32 * u], v);
            st16h(&S.a[0][row][32 * u + 16], v2);
        }
    }
}

// Stage the activation codes (f16) and per-block scales of tokens [n0, n0+BN), chunk kc, into LDS.
template <int DT, int BM, int BN>
JAMHIP_DEV void stage_x(GemmSmem<DT, BM, BN>& S, const ActQ& A, int n0, int n, int k, int kc, int nblk) {
    const int nb = k >> 5, n16 = k >> 4;
    for (int ci = threadIdx.x; ci < BN * 16; ci += 256) {
        const int tok = ci >> 4, c16 = ci & 15;
        if ((c16 >> 1) >= nblk) continue;
        const int gt = n0 + tok < n ? n0 + tok : n - 1;
        const uint4 q = gld16(A.q + (int64_t) gt * k + kc + 16 * c16);
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; j++) v[j] = (float) (int8_t) bytei(q, j);
        st16h(&S.b[tok][16 * c16], v);
    }
    for (int e = threadIdx.x; e < BN * 8; e += 256) {
        const int tok = e >> 3, s = e & 7;
        if (s >= nblk) continue;
        const int gt = n0 + tok < n ? n0 + tok : n - 1;
        const int b = kc / 32 + s;
        S.dx[s][tok] = A.d[(int64_t) gt * nb + b];
        if constexpr (DT == Q4_K || DT == Q4_0)
            S.xs[s][tok] = A.s[(int64_t) gt * n16 + 2 * b] + A.s[(int64_t) gt * n16 + 2 * b + 1];
    }
    if constexpr (DT == Q6_K) {
        for (int e = threadIdx.x; e < BN * 16; e += 256) {
            const int tok = e >> 4, t = e & 15;
            const int gt = n0 + tok < n ? n0 + tok : n - 1;
            S.xs[t][tok] = 32.0f * A.s[(int64_t) gt * n16 + kc / 16 + t];
        }
    }
}

template <int DT, int BM, int BN>
__global__ void __launch_bounds__(256) gemm_kernel(WeightView w, ActQ A, int k, int m, int n, float* __restrict__ c,
                                                   int ldc, Epi ep) {
    __shared__ GemmSmem<DT, BM, BN> S;
    constexpr int RT = BM / 32, CT = BN / 32;   // 16x16 tiles per wave
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t m0 = (int64_t) blockIdx.x * BM;
    const int n0 = blockIdx.y * BN;
    const int lr = lane & 15, lk = 8 * (lane >> 4), l4 = 4 * (lane >> 4);

    floatx4 acc[RT][CT], tmp[RT][CT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int ct = 0; ct < CT; ct++) acc[rt][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};

    for (int kc = 0; kc < k; kc += KC) {
        const int nblk = (k - kc) >> 5 < 8 ? (k - kc) >> 5 : 8;
        __syncthreads();   // the previous chunk's LDS reads are done
        stage_w<DT, BM, BN>(S, w, m0, m, kc, nblk);
        stage_x<DT, BM, BN>(S, A, n0, n, k, kc, nblk);
        __syncthreads();
        for (int s = 0; s < nblk; s++) {
            half8 af[planes<DT>()][RT], bf[CT];
#pragma unroll
            for (int p = 0; p < planes<DT>(); p++)
#pragma unroll
                for (int rt = 0; rt < RT; rt++)
                    af[p][rt] = *reinterpret_cast<const half8*>(&S.a[p][wm * (BM / 2) + rt * 16 + lr][32 * s + lk]);
#pragma unroll
            for (int ct = 0; ct < CT; ct++)
                bf[ct] = *reinterpret_cast<const half8*>(&S.b[wn * (BN / 2) + ct * 16 + lr][32 * s + lk]);
#pragma unroll
            for (int ct = 0; ct < CT; ct++) {
                const int tok = wn * (BN / 2) + ct * 16 + lr;
                const float dxv = S.dx[s][tok];
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    floatx4 J = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[0][rt], bf[ct], zero, 0, 0, 0);
                    if constexpr (planes<DT>() == 2)
                        J = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[1][rt], bf[ct], J, 0, 0, 0);
                    const int row = wm * (BM / 2) + rt * 16 + l4;
                    if constexpr (kquant<DT>()) {
                        if (s == 0) tmp[rt][ct] = J * dxv;
                        else
#pragma unroll
                            for (int i = 0; i < 4; i++) tmp[rt][ct][i] = fmaf(J[i], dxv, tmp[rt][ct][i]);
                        if constexpr (DT == Q4_K) {
                            const float xv = S.xs[s][tok];
#pragma unroll
                            for (int i = 0; i < 4; i++) acc[rt][ct][i] = fmaf(-S.ws[s][row + i], xv, acc[rt][ct][i]);
                        } else {
                            const float xa = S.xs[2 * s][tok], xb = S.xs[2 * s + 1][tok];
#pragma unroll
                            for (int i = 0; i < 4; i++) {
                                acc[rt][ct][i] = fmaf(-S.ws[2 * s][row + i], xa, acc[rt][ct][i]);
                                acc[rt][ct][i] = fmaf(-S.ws[2 * s + 1][row + i], xb, acc[rt][ct][i]);
                            }
                        }
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[rt][ct][i] = fmaf(J[i], S.ws[s][row + i] * dxv, acc[rt][ct][i]);
                        if constexpr (DT == Q4_0) {
                            const float xv = S.xs[s][tok];
#pragma unroll
                            for (int i = 0; i < 4; i++) acc[rt][ct][i] = fmaf(-S.ws2[s][row + i], xv, acc[rt][ct][i]);
                        }
                    }
                }
            }
        }
        if constexpr (kquant<DT>()) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int ct = 0; ct < CT; ct++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[rt][ct][i] = fmaf(tmp[rt][ct][i], S.d[wm * (BM / 2) + rt * 16 + l4 + i], acc[rt][ct][i]);
        }
    }

#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int ct = 0; ct < CT; ct++) {
            const int tok = n0 + wn * (BN / 2) + ct * 16 + lr;
            const int64_t row = m0 + wm * (BM / 2) + rt * 16 + l4;
            if (tok < n) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (row + i < m) {
                        float* dst = c + (int64_t) tok * ldc + row + i;
                        *dst = epilogue(ep, acc[rt][ct][i], row + i, dst);
                    }
            }
        }
}

template <int DT, int BM, int BN>
static hipError_t gemm_go(const WeightView& w, const ActQ& A, int k, int m, int n, float* c, int ldc, hipStream_t st,
                          const Epi& ep) {
    const dim3 grid((unsigned) ((m + BM - 1) / BM), (unsigned) ((n + BN - 1) / BN));
    gemm_kernel<DT, BM, BN><<<grid, 256, 0, st>>>(w, A, k, m, n, c, ldc, ep);
    return hipGetLastError();
}

bool gemm_covers(int dt) { return dt == Q4_K || dt == Q6_K || dt == Q8_0 || dt == Q4_0 || dt == MXFP4; }

hipError_t launch_gemm(int dt, const WeightView& w, const ActQ& A, int k, int m, int n, float* c, int ldc,
                       hipStream_t st, const Epi& ep) {
    switch (dt) {
    case Q4_K: return gemm_go<Q4_K, 128, 64>(w, A, k, m, n, c, ldc, st, ep);
    case Q6_K: return gemm_go<Q6_K, 64, 64>(w, A, k, m, n, c, ldc, st, ep);
    case Q8_0: return gemm_go<Q8_0, 128, 64>(w, A, k, m, n, c, ldc, st, ep);
    case Q4_0: return gemm_go<Q4_0, 128, 64>(w, A, k, m, n, c, ldc, st, ep);
    case MXFP4: return gemm_go<MXFP4, 128, 64>(w, A, k, m, n, c, ldc, st, ep);
    default: return hipErrorNotSupported;
    }
}

}  // namespace jamhip
