// Weight-streaming matmul for few tokens: decode GEMV (n < 8, jam's F1 decomposition) and the skinny
// n >= 8 fallback (F2 decomposition, 8 tokens per launch row). HBM-bound: every weight byte is read once
// per launch with 128-bit loads; int8 dots run on v_dot4_i32_i8; the per-block f32 combine follows the
// jam kernel named at each dot below.
//
// Work split: a 256-thread workgroup = 4 waves; a wave owns ROWS consecutive weight rows; lane l owns the
// "unit" u = pass*64 + l of every one of those rows, where a unit is 64 elements (Q4_K: one scale pair
// of a super-block) or 32 elements (Q8_0/Q4_0/MXFP4: one block; Q6_K: one 16-byte ql slice). A wave reads
// contiguous row bytes, then folds its 64 lane partials with xor-shuffles.
#include "common.h"
#include "launch.h"
#include "quant.h"

namespace jamhip {

template <int DT> constexpr int unit_elems() { return DT == Q4_K ? 64 : 32; }

// -------------------------------------------------------------------------------------------- weights
struct WQ4K { uint4 h, q0, q1; };
struct WQ8 { uint4 q0, q1; uint32_t d; };
struct WQ4 { uint4 q; uint32_t d; };        // Q4_0 and MXFP4 (d = fp16 bits or the e8m0 byte)
struct WQ6 { uint4 ql, qh, sc; uint32_t d; };

template <int DT> struct WRegs;
template <> struct WRegs<Q4_K> { using T = WQ4K; };
template <> struct WRegs<Q8_0> { using T = WQ8; };
template <> struct WRegs<Q4_0> { using T = WQ4; };
template <> struct WRegs<MXFP4> { using T = WQ4; };
template <> struct WRegs<Q6_K> { using T = WQ6; };

JAMHIP_DEV uint4 ld16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }

template <int DT> JAMHIP_DEV typename WRegs<DT>::T load_w(const WeightView& w, int64_t row, int u) {
    typename WRegs<DT>::T r;
    if constexpr (DT == Q4_K) {
        const uint8_t* p = w.qs + (row * w.rb + (u >> 2)) * 144;
        const int g = u & 3;
        r.h = ld16(p);
        r.q0 = ld16(p + 16 + 32 * g);
        r.q1 = ld16(p + 32 + 32 * g);
    } else if constexpr (DT == Q8_0) {
        const int64_t i = row * w.rb + u;
        r.q0 = ld16(w.qs + i * 32);
        r.q1 = ld16(w.qs + i * 32 + 16);
        r.d = *reinterpret_cast<const uint16_t*>(w.sc + i * 2);
    } else if constexpr (DT == Q4_0) {
        const int64_t i = row * w.rb + u;
        r.q = ld16(w.qs + i * 16);
        r.d = *reinterpret_cast<const uint16_t*>(w.sc + i * 2);
    } else if constexpr (DT == MXFP4) {
        const int64_t i = row * w.rb + u;
        r.q = ld16(w.qs + i * 16);
        r.d = w.sc[i];
    } else {   // Q6_K: unit t = u & 7 of super-block u >> 3
        const int64_t i = row * w.rb + (u >> 3);
        const int t = u & 7, h = t >> 2, jj = (t >> 1) & 1, lh = t & 1;
        const uint8_t* body = w.qs + i * 208;
        r.ql = ld16(body + 64 * h + 32 * jj + 16 * lh);
        r.qh = ld16(body + 128 + 32 * h + 16 * lh);
        r.sc = ld16(body + 192);
        r.d = *reinterpret_cast<const uint16_t*>(w.sc + i * 2);
    }
    return r;
}

// ------------------------------------------------------------------------------------- int8 helpers
JAMHIP_DEV int dot16(const uint4 w, const uint4 a, int c) {
    c = dot4((int) w.x, (int) a.x, c);
    c = dot4((int) w.y, (int) a.y, c);
    c = dot4((int) w.z, (int) a.z, c);
    return dot4((int) w.w, (int) a.w, c);
}
JAMHIP_DEV uint4 and4(uint4 v, uint32_t m) { return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m); }
JAMHIP_DEV uint4 shr4(uint4 v, int s) { return make_uint4(v.x >> s, v.y >> s, v.z >> s, v.w >> s); }

// MXFP4 nibble -> signed int8 code (value x2: 0,1,2,3,4,6,8,12 and negatives; jam_mxfp4.h:14-15),
// four at a time: v_perm picks the magnitude and its negation from 8-entry tables, bit 3 selects.
JAMHIP_DEV uint32_t mxfp4_codes(uint32_t nib4) {
    const uint32_t idx = nib4 & 0x07070707u;
    const uint32_t pos = __builtin_amdgcn_perm(0x0C080604u, 0x03020100u, idx);
    const uint32_t neg = __builtin_amdgcn_perm(0xF4F8FAFCu, 0xFDFEFF00u, idx);
    const uint32_t msk = ((nib4 >> 3) & 0x01010101u) * 0xFFu;
    return (neg & msk) | (pos & ~msk);
}
JAMHIP_DEV uint4 mxfp4_codes4(uint4 n) {
    return make_uint4(mxfp4_codes(n.x), mxfp4_codes(n.y), mxfp4_codes(n.z), mxfp4_codes(n.w));
}

// Q4_K 6-bit (scale, min) of sub-blocks 2g and 2g+1 (jam/jam-native/src/jam_kquant.h:26-33), from the
// three scale words (bytes 4..15 of the block).
JAMHIP_DEV void q4k_pair_scales(const uint4 h, int g, int& sc0, int& sc1, int& mn0, int& mn1) {
    const uint32_t u0 = h.y, u1 = h.z, u2 = h.w;
    const uint32_t scA = u0 & 0x3f3f3f3fu, mnA = u1 & 0x3f3f3f3fu;
    const uint32_t scB = (u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4);
    const uint32_t mnB = ((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4);
    const uint32_t scw = g < 2 ? scA : scB, mnw = g < 2 ? mnA : mnB;
    const int sh = (g & 1) * 16;
    sc0 = (scw >> sh) & 0xff;
    sc1 = (scw >> (sh + 8)) & 0xff;
    mn0 = (mnw >> sh) & 0xff;
    mn1 = (mnw >> (sh + 8)) & 0xff;
}

JAMHIP_DEV int sbyte(uint32_t w, int b) { return (int) (int8_t) (w >> (8 * b)); }

// -------------------------------------------------------------------------------- per-unit partials
// F1: activations from jam_q8_0_requant — q, d per 32, asum per 32 (float), s16 per 16 (int).
template <int DT>
JAMHIP_DEV float unit_f1(const typename WRegs<DT>::T& w, int u, const ActQ& A, int t, int k) {
    const int nb = k >> 5;
    const int8_t* aq = A.q + (int64_t) t * k;
    const float* ad = A.d + (int64_t) t * nb;
    if constexpr (DT == Q4_K) {
        // jam_mm_q4k_avx512vnni (jam_kernels_q4k_avx512.c:956-1054):
        //   Σ_s I_s·fl(fl(ad·sc)·d)  −  dmin·Σ_s mn·fl(asum·ad)
        const int sb = u >> 2, g = u & 3, base = sb * 256 + 64 * g, bl = sb * 8 + 2 * g;
        const uint4 a0 = ld16((const uint8_t*) aq + base), a1 = ld16((const uint8_t*) aq + base + 16);
        const uint4 a2 = ld16((const uint8_t*) aq + base + 32), a3 = ld16((const uint8_t*) aq + base + 48);
        int ilo = dot16(and4(w.q0, 0x0f0f0f0fu), a0, 0);
        ilo = dot16(and4(w.q1, 0x0f0f0f0fu), a1, ilo);
        int ihi = dot16(and4(shr4(w.q0, 4), 0x0f0f0f0fu), a2, 0);
        ihi = dot16(and4(shr4(w.q1, 4), 0x0f0f0f0fu), a3, ihi);
        int sc0, sc1, mn0, mn1;
        q4k_pair_scales(w.h, g, sc0, sc1, mn0, mn1);
        const float d = h2f(w.h.x & 0xffffu), dmin = h2f(w.h.x >> 16);
        const float ad0 = ad[bl], ad1 = ad[bl + 1];
        const float as0 = A.s[(int64_t) t * nb + bl], as1 = A.s[(int64_t) t * nb + bl + 1];
        const float f0 = (ad0 * (float) sc0) * d, f1 = (ad1 * (float) sc1) * d;
        return (float) ilo * f0 + (float) ihi * f1 - dmin * ((float) mn0 * (as0 * ad0) + (float) mn1 * (as1 * ad1));
    } else if constexpr (DT == Q8_0) {
        // jam_mm_q8_0_gemv_avx512 / q256 engine (avx512.c:374-390, jam_gemm_q256.inc:28-36): fl(d·ad)·Σq·aq
        const uint4 a0 = ld16((const uint8_t*) aq + 32 * u), a1 = ld16((const uint8_t*) aq + 32 * u + 16);
        const int I = dot16(w.q1, a1, dot16(w.q0, a0, 0));
        return (float) I * (h2f(w.d) * ad[u]);
    } else if constexpr (DT == Q4_0) {
        // jam_decode_q4_0_256 + q256 engine: fl(d·ad)·Σ(nib-8)·aq, with Σ(nib-8)·aq = Σnib·aq - 8·Σaq
        const uint4 a0 = ld16((const uint8_t*) aq + 32 * u), a1 = ld16((const uint8_t*) aq + 32 * u + 16);
        int I = dot16(and4(w.q, 0x0f0f0f0fu), a0, 0);
        I = dot16(and4(shr4(w.q, 4), 0x0f0f0f0fu), a1, I);
        I -= 8 * (int) A.s[(int64_t) t * nb + u];
        return (float) I * (h2f(w.d) * ad[u]);
    } else if constexpr (DT == MXFP4) {
        // jam_decode_mxfp4_256 + q256 engine: fl(dhalf·ad)·Σcode·aq
        const uint4 a0 = ld16((const uint8_t*) aq + 32 * u), a1 = ld16((const uint8_t*) aq + 32 * u + 16);
        int I = dot16(mxfp4_codes4(and4(w.q, 0x0f0f0f0fu)), a0, 0);
        I = dot16(mxfp4_codes4(and4(shr4(w.q, 4), 0x0f0f0f0fu)), a1, I);
        return (float) I * (e8m0_half(w.d) * ad[u]);
    } else {
        // jam_mm_q6k_sse3 (jam_kernels_kquant_sse3.c:125-169): ad·(fl(d·sc)·Σ(q6-32)·aq) per 16-half,
        // with Σ(q6-32)·aq = Σq6·aq - 32·Σaq (exact ints).
        const int sb = u >> 3, tt = u & 7, h = tt >> 2, jj = (tt >> 1) & 1, lh = tt & 1;
        const int blka = sb * 8 + 4 * h + jj, blkb = blka + 2;
        const uint4 aa = ld16((const uint8_t*) aq + 32 * blka + 16 * lh);
        const uint4 ab = ld16((const uint8_t*) aq + 32 * blkb + 16 * lh);
        const uint4 hia = and4(shr4(w.qh, 2 * jj), 0x03030303u), hib = and4(shr4(w.qh, 2 * jj + 4), 0x03030303u);
        const uint4 lo = and4(w.ql, 0x0f0f0f0fu), hi = and4(shr4(w.ql, 4), 0x0f0f0f0fu);
        const uint4 qa = make_uint4(lo.x | (hia.x << 4), lo.y | (hia.y << 4), lo.z | (hia.z << 4), lo.w | (hia.w << 4));
        const uint4 qb = make_uint4(hi.x | (hib.x << 4), hi.y | (hib.y << 4), hi.z | (hib.z << 4), hi.w | (hib.w << 4));
        const int* s16 = A.s16 + (int64_t) t * (k >> 4);
        const int ia = dot16(qa, aa, 0) - 32 * s16[2 * blka + lh];
        const int ib = dot16(qb, ab, 0) - 32 * s16[2 * blkb + lh];
        const int byte = 2 * jj + lh;
        const int sca = sbyte(h ? w.sc.z : w.sc.x, byte), scb = sbyte(h ? w.sc.w : w.sc.y, byte);
        const float d = h2f(w.d);
        return ad[blka] * ((d * (float) sca) * (float) ia) + ad[blkb] * ((d * (float) scb) * (float) ib);
    }
}

// F2: activations from quantize_row_q8s — q, d per 32, raw f32 Σx per 16 (A.s).
template <int DT>
JAMHIP_DEV float unit_f2(const typename WRegs<DT>::T& w, int u, const ActQ& A, int t, int k) {
    const int nb = k >> 5;
    const int8_t* aq = A.q + (int64_t) t * k;
    const float* dx = A.d + (int64_t) t * nb;
    const float* xs = A.s + (int64_t) t * (k >> 4);
    if constexpr (DT == Q4_K) {
        // q4k_block16 (jam_kernels_q4k_avx512.c:76-95): fl(fl(d·sc)·dx)·I − fl(dmin·mn)·fl(xs0+xs1)
        const int sb = u >> 2, g = u & 3, base = sb * 256 + 64 * g, bl = sb * 8 + 2 * g;
        const uint4 a0 = ld16((const uint8_t*) aq + base), a1 = ld16((const uint8_t*) aq + base + 16);
        const uint4 a2 = ld16((const uint8_t*) aq + base + 32), a3 = ld16((const uint8_t*) aq + base + 48);
        int ilo = dot16(and4(w.q0, 0x0f0f0f0fu), a0, 0);
        ilo = dot16(and4(w.q1, 0x0f0f0f0fu), a1, ilo);
        int ihi = dot16(and4(shr4(w.q0, 4), 0x0f0f0f0fu), a2, 0);
        ihi = dot16(and4(shr4(w.q1, 4), 0x0f0f0f0fu), a3, ihi);
        int sc0, sc1, mn0, mn1;
        q4k_pair_scales(w.h, g, sc0, sc1, mn0, mn1);
        const float d = h2f(w.h.x & 0xffffu), dmin = h2f(w.h.x >> 16);
        const float dw0 = d * (float) sc0, dw1 = d * (float) sc1, mw0 = dmin * (float) mn0, mw1 = dmin * (float) mn1;
        return (float) ilo * (dw0 * dx[bl]) - mw0 * (xs[2 * bl] + xs[2 * bl + 1])
             + (float) ihi * (dw1 * dx[bl + 1]) - mw1 * (xs[2 * bl + 2] + xs[2 * bl + 3]);
    } else if constexpr (DT == Q8_0) {
        // q8_block16 (jam_kernels_q4k_avx512.c:347-362): fl(d·dx)·Σq·xq
        const uint4 a0 = ld16((const uint8_t*) aq + 32 * u), a1 = ld16((const uint8_t*) aq + 32 * u + 16);
        const int I = dot16(w.q1, a1, dot16(w.q0, a0, 0));
        return (float) I * (h2f(w.d) * dx[u]);
    } else if constexpr (DT == Q4_0) {
        // q4_0_block16 (jam_kernels_q4k_avx512.c:463-480): fl(d·dx)·Σnib·xq − fl(8d)·fl(xs0+xs1)
        const uint4 a0 = ld16((const uint8_t*) aq + 32 * u), a1 = ld16((const uint8_t*) aq + 32 * u + 16);
        int I = dot16(and4(w.q, 0x0f0f0f0fu), a0, 0);
        I = dot16(and4(shr4(w.q, 4), 0x0f0f0f0fu), a1, I);
        const float d = h2f(w.d);
        return (float) I * (d * dx[u]) - (8.0f * d) * (xs[2 * u] + xs[2 * u + 1]);
    } else if constexpr (DT == MXFP4) {
        // mxfp4_block16 (jam_kernels_q4k_avx512.c:692-711): fl(dhalf·dx)·Σcode·xq
        const uint4 a0 = ld16((const uint8_t*) aq + 32 * u), a1 = ld16((const uint8_t*) aq + 32 * u + 16);
        int I = dot16(mxfp4_codes4(and4(w.q, 0x0f0f0f0fu)), a0, 0);
        I = dot16(mxfp4_codes4(and4(shr4(w.q, 4), 0x0f0f0f0fu)), a1, I);
        return (float) I * (e8m0_half(w.d) * dx[u]);
    } else {
        // q6k_block16 (jam_kernels_q4k_avx512.c:222-236): fl(fl(d·sc)·dx)·Σq6·xq − fl(d·sc)·fl(32·xs16)
        const int sb = u >> 3, tt = u & 7, h = tt >> 2, jj = (tt >> 1) & 1, lh = tt & 1;
        const int blka = sb * 8 + 4 * h + jj, blkb = blka + 2;
        const uint4 aa = ld16((const uint8_t*) aq + 32 * blka + 16 * lh);
        const uint4 ab = ld16((const uint8_t*) aq + 32 * blkb + 16 * lh);
        const uint4 hia = and4(shr4(w.qh, 2 * jj), 0x03030303u), hib = and4(shr4(w.qh, 2 * jj + 4), 0x03030303u);
        const uint4 lo = and4(w.ql, 0x0f0f0f0fu), hi = and4(shr4(w.ql, 4), 0x0f0f0f0fu);
        const uint4 qa = make_uint4(lo.x | (hia.x << 4), lo.y | (hia.y << 4), lo.z | (hia.z << 4), lo.w | (hia.w << 4));
        const uint4 qb = make_uint4(hi.x | (hib.x << 4), hi.y | (hib.y << 4), hi.z | (hib.z << 4), hi.w | (hib.w << 4));
        const int ia = dot16(qa, aa, 0), ib = dot16(qb, ab, 0);
        const int byte = 2 * jj + lh;
        const int sca = sbyte(h ? w.sc.z : w.sc.x, byte), scb = sbyte(h ? w.sc.w : w.sc.y, byte);
        const float d = h2f(w.d);
        const float dwa = d * (float) sca, dwb = d * (float) scb;
        return (float) ia * (dwa * dx[blka]) - dwa * (32.0f * xs[2 * blka + lh])
             + (float) ib * (dwb * dx[blkb]) - dwb * (32.0f * xs[2 * blkb + lh]);
    }
}

// ------------------------------------------------------------------------------------------ kernel
// FL = 1 (n < 8): NT is the exact token count. FL = 2 (skinny n >= 8): blockIdx.y picks 8 tokens,
// the last group may hold fewer (ntv). FUSE (FL = 1 only): the workgroup quantizes A into LDS itself
// (F1, bit-exact) while its first weight loads are in flight, so a decode matmul is a single launch.
template <int DT, int FL, int NT, int ROWS, bool FUSE>
__global__ void __launch_bounds__(256) gemv_kernel(WeightView w, ActQ A, const float* __restrict__ a, int lda,
                                                   int k, int m, int n, float* __restrict__ c, int ldc) {
    const int lane = threadIdx.x & 63;
    const int64_t row0 = ((int64_t) blockIdx.x * 4 + (threadIdx.x >> 6)) * ROWS;
    const int t0 = blockIdx.y * NT;
    const int ntv = n - t0 < NT ? n - t0 : NT;
    constexpr int UE = unit_elems<DT>();
    const int units = k / UE;

    typename WRegs<DT>::T wr[ROWS];
    if constexpr (FUSE) {
        extern __shared__ __align__(16) unsigned char smem[];
        const int nb = k >> 5;
        int8_t* lq = reinterpret_cast<int8_t*>(smem);
        float* ld = reinterpret_cast<float*>(smem + NT * k);
        float* las = ld + NT * nb;
        int* ls16 = reinterpret_cast<int*>(las + NT * nb);
        if (lane < units && row0 < m) {   // first weight loads go out before the quantization
#pragma unroll
            for (int r = 0; r < ROWS; r++) wr[r] = load_w<DT>(w, row0 + r < m ? row0 + r : m - 1, lane);
        }
        for (int e = threadIdx.x; e < NT * k; e += 256) {   // 32-lane groups are whole blocks
            const int j = e / k, ee = e - j * k;
            float db;
            int h16, h32;
            lq[e] = (int8_t) f1_lane(a[(int64_t) j * lda + ee], db, h16, h32);
            if ((ee & 15) == 0) ls16[j * (k >> 4) + (ee >> 4)] = h16;
            if ((ee & 31) == 0) {
                ld[j * nb + (ee >> 5)] = db;
                las[j * nb + (ee >> 5)] = (float) h32;
            }
        }
        __syncthreads();
        A = ActQ{lq, ld, las, ls16};
    }
    if (row0 >= m) return;

    float acc[ROWS][NT];
#pragma unroll
    for (int r = 0; r < ROWS; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[r][t] = 0.0f;

    bool loaded = FUSE;
    for (int u = lane; u < units; u += 64) {
        if (!loaded) {
#pragma unroll
            for (int r = 0; r < ROWS; r++) wr[r] = load_w<DT>(w, row0 + r < m ? row0 + r : m - 1, u);  // clamp: in bounds
        }
        loaded = false;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (FL == 2 && t >= ntv) break;
            const int tt = FUSE ? t : t0 + t;
#pragma unroll
            for (int r = 0; r < ROWS; r++)
                acc[r][t] += FL == 1 ? unit_f1<DT>(wr[r], u, A, tt, k) : unit_f2<DT>(wr[r], u, A, tt, k);
        }
    }
#pragma unroll
    for (int r = 0; r < ROWS; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (FL == 2 && t >= ntv) break;
            const float v = wave_sum(acc[r][t]);
            if (lane == 0 && row0 + r < m) c[(int64_t) (t0 + t) * ldc + row0 + r] = v;
        }
}

// Fused F1 quantization keeps A's int8 copy in LDS: 1.5 bytes per element (q, d, asum, Σ16).
constexpr int kFuseMaxElems = 32768;

template <int DT, int FL, int NT, int ROWS>
static hipError_t go(const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m, int n, float* c,
                     int ldc, hipStream_t st) {
    const int waves = (m + ROWS - 1) / ROWS;
    dim3 grid((waves + 3) / 4, FL == 1 ? 1 : (n + NT - 1) / NT);
    if (FL == 1 && a != nullptr) {
        const size_t lds = (size_t) NT * k + (size_t) NT * (k / 32) * 8 + (size_t) NT * (k / 16) * 4;
        gemv_kernel<DT, FL, NT, ROWS, true><<<grid, 256, lds, st>>>(w, A, a, lda, k, m, n, c, ldc);
    } else {
        gemv_kernel<DT, FL, NT, ROWS, false><<<grid, 256, 0, st>>>(w, A, a, lda, k, m, n, c, ldc);
    }
    return hipGetLastError();
}

template <int DT>
static hipError_t gemv_dt(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m,
                          int n, float* c, int ldc, hipStream_t st) {
    if (flavour == 2) return go<DT, 2, 8, 1>(w, A, nullptr, 0, k, m, n, c, ldc, st);
    const bool big = m >= 8192;
    switch (n) {
    case 1:
        return big ? go<DT, 1, 1, 4>(w, A, a, lda, k, m, n, c, ldc, st) : go<DT, 1, 1, 1>(w, A, a, lda, k, m, n, c, ldc, st);
    case 2:
        return big ? go<DT, 1, 2, 2>(w, A, a, lda, k, m, n, c, ldc, st) : go<DT, 1, 2, 1>(w, A, a, lda, k, m, n, c, ldc, st);
    case 3: return go<DT, 1, 3, 1>(w, A, a, lda, k, m, n, c, ldc, st);
    case 4: return go<DT, 1, 4, 1>(w, A, a, lda, k, m, n, c, ldc, st);
    case 5: return go<DT, 1, 5, 1>(w, A, a, lda, k, m, n, c, ldc, st);
    case 6: return go<DT, 1, 6, 1>(w, A, a, lda, k, m, n, c, ldc, st);
    case 7: return go<DT, 1, 7, 1>(w, A, a, lda, k, m, n, c, ldc, st);
    default: return hipErrorInvalidValue;
    }
}

bool gemv_fusable(int n, int k) { return n < 8 && (int64_t) n * k <= kFuseMaxElems; }

hipError_t launch_gemv(int dt, int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m,
                       int n, float* c, int ldc, hipStream_t st) {
    switch (dt) {
    case Q4_K: return gemv_dt<Q4_K>(flavour, w, A, a, lda, k, m, n, c, ldc, st);
    case Q6_K: return gemv_dt<Q6_K>(flavour, w, A, a, lda, k, m, n, c, ldc, st);
    case Q8_0: return gemv_dt<Q8_0>(flavour, w, A, a, lda, k, m, n, c, ldc, st);
    case Q4_0: return gemv_dt<Q4_0>(flavour, w, A, a, lda, k, m, n, c, ldc, st);
    case MXFP4: return gemv_dt<MXFP4>(flavour, w, A, a, lda, k, m, n, c, ldc, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace jamhip
