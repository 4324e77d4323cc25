#pragma once
// Weight-streaming matmul for few tokens (device code and launch templates; one translation unit per weight
// type instantiates them, gemv.hip dispatches): the decode GEMV (n < 8, jam's F1 decomposition) and the skinny
// n >= 8 path (F2 decomposition). HBM-bound: every weight byte is read once per launch with aligned
// 128-bit loads; int8 dots run on v_dot4_i32_i8; the per-block f32 combine follows the jam kernel named
// at each dot below.
//
// Work split. A lane owns whole 256-element groups of the row-tiled device layout (common.h): the 64 lanes
// of a wave take 8 consecutive rows (a "band") x 8 groups, so for each chunk index c they read 8 groups x 8
// rows of 16 bytes, i.e. eight full 128-byte lines, and one group's scales come in one more load. Eight
// waves share a workgroup, the activation prologue and the LDS in which every lane's per-group partial is
// parked and each row's partials are summed (see mv_kernel). In the fused F1 variant the workgroup quantizes A into LDS (bit-exact F1) once
// for all of its rows; its activation loads go out first and its weight stream right behind them.
#include "common.h"
#include "launch.h"
#include "quant.h"

#include <mutex>
#include <utility>
#include <vector>

namespace jamhip {

// -------------------------------------------------------------------------------------------- weights
template <int DT> struct Group {
    uint4 q[group_chunks(DT)];
    uint4 s;   // the group's scale bytes (Q4_K header; Q8_0/Q4_0 8 x fp16; MXFP4 8 x e8m0; Q6_K d in s.x)
};

JAMHIP_DEV uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
// The weight stream is read once per call: non-temporal loads keep it from displacing the lines that are
// reused (the activations, the partials) in L2 and the MALL (measured 2-4% faster on every decode shape).
JAMHIP_DEV uint4 ld16_stream(const void* p) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Group g of view row `row` (row-tiled layout of common.h: chunk c at +c·512 from chunk 0).
// Issue order: the chunks in the order the dot products use them (loads retire in issue order) and the
// scales first, except for Q4_K, whose scales go last (measured faster on the Llama shapes).
template <int DT> JAMHIP_DEV constexpr int chunk_order(int i) {
    // Q6_K: the scale chunk, the qh chunks of half 0, ql 0-3, the qh chunks of half 1, ql 4-7
    return DT != Q6_K ? i : i == 0 ? 12 : i < 3 ? 7 + i : i < 7 ? i - 3 : i < 9 ? i + 3 : i - 5;
}
template <int DT>
JAMHIP_DEV void load_scales(Group<DT>& r, const uint8_t* s) {
    if constexpr (DT == Q6_K) {
        r.s.x = *reinterpret_cast<const uint16_t*>(s);
    } else if constexpr (DT == Q1_0) {
        r.s.x = *reinterpret_cast<const uint32_t*>(s);
    } else if constexpr (DT == MXFP4) {
        const uint2 v = *reinterpret_cast<const uint2*>(s);
        r.s = make_uint4(v.x, v.y, 0u, 0u);
    } else {
        r.s = ld16_stream(s);
    }
}
template <int DT>
JAMHIP_DEV void load_group(Group<DT>& r, const WeightView& w, int64_t row, int g) {
    const uint8_t* q = group_q<DT>(w, row, g);
    const uint8_t* s = group_s<DT>(w, row, g);
    if constexpr (DT != Q4_K) load_scales<DT>(r, s);
#pragma unroll
    for (int i = 0; i < group_chunks(DT); i++) {
        const int c = chunk_order<DT>(i);
        r.q[c] = ld16_stream(q + c * CHUNK_STRIDE);
    }
    if constexpr (DT == Q4_K) load_scales<DT>(r, s);
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
JAMHIP_DEV uint4 lo_nib(uint4 v) { return and4(v, 0x0f0f0f0fu); }
JAMHIP_DEV uint4 hi_nib(uint4 v) { return and4(shr4(v, 4), 0x0f0f0f0fu); }
JAMHIP_DEV uint32_t word(const uint4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

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

// Q4_K 6-bit scale and min of sub-block s (jam/jam-native/src/jam_kquant.h:26-33) from the header words.
JAMHIP_DEV void q4k_sm(const uint4 h, int s, int& sc, int& mn) {
    const uint32_t u0 = h.y, u1 = h.z, u2 = h.w;   // scale bytes 0-3, 4-7, 8-11
    const int sh = 8 * (s & 3);
    if (s < 4) {
        sc = (u0 >> sh) & 63;
        mn = (u1 >> sh) & 63;
    } else {
        sc = ((u2 >> sh) & 15) | ((((u0 >> sh) >> 6) & 3) << 4);
        mn = (((u2 >> sh) >> 4) & 15) | ((((u1 >> sh) >> 6) & 3) << 4);
    }
}

JAMHIP_DEV int sbyte(uint32_t w, int b) { return (int) (int8_t) (w >> (8 * b)); }


// Q1_0: sign bits b0..b3 of a nibble -> the bytes (b0, b1, b2, b3) as 0 / 1 (the products b·2^(7j) land on
// distinct bits, so the multiply carries nothing into the kept ones).
JAMHIP_DEV uint32_t bits4_to_bytes(uint32_t b) { return ((b & 15u) * 0x00204081u) & 0x01010101u; }

// Σ bit·q over one 32-element block: its 32 sign bits against its 32 int8 activation codes.
JAMHIP_DEV int q1_dot01(uint32_t bits, const int8_t* aq) {
    const uint4 a0 = ld16(aq), a1 = ld16(aq + 16);
    int I = dot4((int) bits4_to_bytes(bits), (int) a0.x, 0);
    I = dot4((int) bits4_to_bytes(bits >> 4), (int) a0.y, I);
    I = dot4((int) bits4_to_bytes(bits >> 8), (int) a0.z, I);
    I = dot4((int) bits4_to_bytes(bits >> 12), (int) a0.w, I);
    I = dot4((int) bits4_to_bytes(bits >> 16), (int) a1.x, I);
    I = dot4((int) bits4_to_bytes(bits >> 20), (int) a1.y, I);
    I = dot4((int) bits4_to_bytes(bits >> 24), (int) a1.z, I);
    return dot4((int) bits4_to_bytes(bits >> 28), (int) a1.w, I);
}

// Q6_K 6-bit codes of ql chunk c with the matching qh chunk: the low-nibble group and the high one.
JAMHIP_DEV void q6k_codes(const uint4 ql, const uint4 qh, int jj, uint4& qa, uint4& qb) {
    const uint4 hia = and4(shr4(qh, 2 * jj), 0x03030303u), hib = and4(shr4(qh, 2 * jj + 4), 0x03030303u);
    const uint4 lo = lo_nib(ql), hi = hi_nib(ql);
    qa = make_uint4(lo.x | (hia.x << 4), lo.y | (hia.y << 4), lo.z | (hia.z << 4), lo.w | (hia.w << 4));
    qb = make_uint4(hi.x | (hib.x << 4), hi.y | (hib.y << 4), hi.z | (hib.z << 4), hi.w | (hib.w << 4));
}

// -------------------------------------------------------------------------------- per-group partials
// Activations of one token for one group: aq -> the group's 256 int8 codes, ad -> its 8 block scales,
// as -> F1: 8 block sums (float Σq) / F2: 16 raw f32 sums Σx per 16, s16 -> F1: 16 int Σq per 16.
// nbv = blocks of the group inside the call's k (8 but for a row's last group of a 32-element type);
// blocks past it contribute nothing and read the last valid block's activations.
template <int DT, int FL>
JAMHIP_DEV float group_dot(const Group<DT>& w, const int8_t* aq, const float* ad, const float* as, const int* s16,
                           int nbv) {
    if constexpr (DT == Q4_K) {
        const uint4 h = w.s;
        const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
        float acc = 0.0f, msum = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; s++) {   // sub-block s: chunks 2(s>>1), 2(s>>1)+1, low nibbles if s even
            const int c0 = 2 * (s >> 1);
            const uint4 w0 = (s & 1) ? hi_nib(w.q[c0]) : lo_nib(w.q[c0]);
            const uint4 w1 = (s & 1) ? hi_nib(w.q[c0 + 1]) : lo_nib(w.q[c0 + 1]);
            const int I = dot16(w1, ld16(aq + 32 * s + 16), dot16(w0, ld16(aq + 32 * s), 0));
            int sc, mn;
            q4k_sm(h, s, sc, mn);
            if constexpr (FL == 1) {
                // jam_mm_q4k_avx512vnni (jam_kernels_q4k_avx512.c:956-1054):
                //   Σ_s I_s·fl(fl(ad·sc)·d)  −  dmin·Σ_s mn·fl(asum·ad)
                acc += (float) I * ((ad[s] * (float) sc) * d);
                msum += (float) mn * (as[s] * ad[s]);
            } else {
                // q4k_block16 (jam_kernels_q4k_avx512.c:76-95): fl(fl(d·sc)·dx)·I − fl(dmin·mn)·fl(xs0+xs1)
                acc += (float) I * ((d * (float) sc) * ad[s]);
                msum += (dmin * (float) mn) * (as[2 * s] + as[2 * s + 1]);
            }
        }
        return FL == 1 ? acc - dmin * msum : acc - msum;
    } else if constexpr (DT == Q5_K) {
        const uint4 h = w.s;
        const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
        float acc = 0.0f, msum = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; s++) {   // sub-block s: Q4_K's nibbles plus bit s of qh[l] as bit 4
            const int c0 = 2 * (s >> 1);
            const uint4 b0 = make_uint4((w.q[8].x >> s) & 0x01010101u, (w.q[8].y >> s) & 0x01010101u,
                                        (w.q[8].z >> s) & 0x01010101u, (w.q[8].w >> s) & 0x01010101u);
            const uint4 b1 = make_uint4((w.q[9].x >> s) & 0x01010101u, (w.q[9].y >> s) & 0x01010101u,
                                        (w.q[9].z >> s) & 0x01010101u, (w.q[9].w >> s) & 0x01010101u);
            const uint4 n0 = (s & 1) ? hi_nib(w.q[c0]) : lo_nib(w.q[c0]);
            const uint4 n1 = (s & 1) ? hi_nib(w.q[c0 + 1]) : lo_nib(w.q[c0 + 1]);
            const uint4 w0 = make_uint4(n0.x | (b0.x << 4), n0.y | (b0.y << 4), n0.z | (b0.z << 4), n0.w | (b0.w << 4));
            const uint4 w1 = make_uint4(n1.x | (b1.x << 4), n1.y | (b1.y << 4), n1.z | (b1.z << 4), n1.w | (b1.w << 4));
            const int I = dot16(w1, ld16(aq + 32 * s + 16), dot16(w0, ld16(aq + 32 * s), 0));
            int sc, mn;
            q4k_sm(h, s, sc, mn);
            const float dl = d * (float) sc, ml = dmin * (float) mn;
            if constexpr (FL == 1) {
                // jam_mm_q5k_sse3 (jam_kernels_kquant_sse3.c:70-121): ad·(fl(dl·I) − fl(ml·asum)) per 32
                acc += ad[s] * (dl * (float) I - ml * as[s]);
            } else {
                // q5k_block16 (jam_kernels_q4k_avx512.c:798-811): fl(dl·dx)·I − ml·fl(xs0+xs1)
                acc += (float) I * (dl * ad[s]);
                msum += ml * (as[2 * s] + as[2 * s + 1]);
            }
        }
        return acc - msum;
    } else if constexpr (DT == NVFP4) {
        // jam_mm_nvfp4_avx512 (jam_kernels_avx512bw.c:111-142; jam's only NVFP4 kernel shape: F1 at every n):
        // per 16-element sub-block s of 64-block j, Σ code·q times fl(ue4m3(d_s)·ad of its 32-block)
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const bool live = 2 * j < nbv;
            const int jj = live ? j : nbv / 2 - 1;   // stay inside the token's activations
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const uint4 ch = w.q[2 * j + (s >> 1)];
                const uint32_t w0 = word(ch, 2 * (s & 1)), w1 = word(ch, 2 * (s & 1) + 1);
                const uint4 A = ld16(aq + 64 * jj + 16 * s);
                int I = dot4((int) mxfp4_codes(w0 & 0x0f0f0f0fu), (int) A.x, 0);
                I = dot4((int) mxfp4_codes(w1 & 0x0f0f0f0fu), (int) A.y, I);
                I = dot4((int) mxfp4_codes((w0 >> 4) & 0x0f0f0f0fu), (int) A.z, I);
                I = dot4((int) mxfp4_codes((w1 >> 4) & 0x0f0f0f0fu), (int) A.w, I);
                const float sc = ue4m3((word(w.s, j) >> (8 * s)) & 0xffu) * ad[2 * jj + (s >> 1)];
                acc += live ? (float) I * sc : 0.0f;
            }
        }
        return acc;
    } else if constexpr (DT == Q1_0) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const bool live = 4 * j < nbv;
            const int jj = live ? j : nbv / 4 - 1;   // stay inside the token's activations
            const float d = h2f((w.s.x >> (16 * j)) & 0xffffu);
            if constexpr (FL == 1) {
                // jam_mm_q1_0_avx2 (jam_kernels_q1_0_avx2.c:45-86): d · Σ_K fma(ad_K, Σ±q) per 128-block,
                // Σ±q = 2·Σbit·q − Σq (exact ints)
                float fb = 0.0f;
#pragma unroll
                for (int K = 0; K < 4; K++) {
                    const int b = 4 * jj + K;
                    const int I = 2 * q1_dot01(word(w.q[j], K), aq + 32 * b) - (s16[2 * b] + s16[2 * b + 1]);
                    fb = fmaf(ad[b], (float) I, fb);
                }
                acc += live ? d * fb : 0.0f;
            } else {
                // q1_0_block16 (jam_kernels_q4k_avx512.c:580-598): fl(d·fl(2·dx))·Σbit·xq − d·fl(xs0+xs1)
#pragma unroll
                for (int K = 0; K < 4; K++) {
                    const int b = 4 * jj + K;
                    const int I = q1_dot01(word(w.q[j], K), aq + 32 * b);
                    const float v = (float) I * (d * (2.0f * ad[b])) - d * (as[2 * b] + as[2 * b + 1]);
                    acc += live ? v : 0.0f;
                }
            }
        }
        return acc;
    } else if constexpr (DT == Q6_K) {
        const float d = h2f(w.s.x & 0xffffu);
        const uint4 scv = w.q[12];
        float blk[8];
#pragma unroll
        for (int b = 0; b < 8; b++) blk[b] = 0.0f;
        float off = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) {   // ql chunk c: half h, j = jj (low nibbles) and jj+2, l = 16lh..
            const int h = c >> 2, jj = (c >> 1) & 1, lh = c & 1;
            uint4 qa, qb;
            q6k_codes(w.q[c], w.q[8 + 2 * h + lh], jj, qa, qb);
            const int ta = 8 * h + 2 * jj + lh, tb = ta + 4;   // 16-element groups (= scale index)
            const int ia = dot16(qa, ld16(aq + 16 * ta), 0), ib = dot16(qb, ld16(aq + 16 * tb), 0);
            const float sa = d * (float) sbyte(word(scv, ta >> 2), ta & 3);
            const float sb = d * (float) sbyte(word(scv, tb >> 2), tb & 3);
            if constexpr (FL == 1) {
                // jam_mm_q6k_sse3 (jam_kernels_kquant_sse3.c:125-169): ad·(fl(d·sc)·Σ(q6-32)·aq) per 16
                blk[ta >> 1] += sa * (float) (ia - 32 * s16[ta]);
                blk[tb >> 1] += sb * (float) (ib - 32 * s16[tb]);
            } else {
                // q6k_block16 (jam_kernels_q4k_avx512.c:222-236): fl(fl(d·sc)·dx)·Σq6·xq − fl(d·sc)·fl(32·xs16)
                blk[ta >> 1] += (float) ia * (sa * ad[ta >> 1]);
                blk[tb >> 1] += (float) ib * (sb * ad[tb >> 1]);
                off += sa * (32.0f * as[ta]) + sb * (32.0f * as[tb]);
            }
        }
        float acc = 0.0f;
#pragma unroll
        for (int b = 0; b < 8; b++) acc += FL == 1 ? ad[b] * blk[b] : blk[b];
        return acc - off;
    } else {
        float acc = 0.0f;
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const int bb = b < nbv ? b : nbv - 1;   // stay inside the token's activations
            int I;
            float sw;
            if constexpr (DT == Q8_0) {
                I = dot16(w.q[2 * b + 1], ld16(aq + 32 * bb + 16), dot16(w.q[2 * b], ld16(aq + 32 * bb), 0));
                sw = h2f((word(w.s, b >> 1) >> (16 * (b & 1))) & 0xffffu);
            } else if constexpr (DT == Q4_0) {
                I = dot16(hi_nib(w.q[b]), ld16(aq + 32 * bb + 16), dot16(lo_nib(w.q[b]), ld16(aq + 32 * bb), 0));
                sw = h2f((word(w.s, b >> 1) >> (16 * (b & 1))) & 0xffffu);
                if constexpr (FL == 1) I -= 8 * (s16[2 * bb] + s16[2 * bb + 1]);
            } else {
                I = dot16(mxfp4_codes4(hi_nib(w.q[b])), ld16(aq + 32 * bb + 16),
                          dot16(mxfp4_codes4(lo_nib(w.q[b])), ld16(aq + 32 * bb), 0));
                sw = e8m0_half((word(w.s, b >> 2) >> (8 * (b & 3))) & 0xffu);
            }
            // F1 (q256 engine, jam_gemm_q256.inc:28-36) and F2 (q8/q4_0/mxfp4_block16): fl(sw·da)·I;
            // Q4_0 under F2 also takes − fl(8·d)·fl(xs0+xs1) (jam_kernels_q4k_avx512.c:463-480)
            float v = (float) I * (sw * ad[bb]);
            if constexpr (DT == Q4_0 && FL == 2) v -= (8.0f * sw) * (as[2 * bb] + as[2 * bb + 1]);
            acc += b < nbv ? v : 0.0f;
        }
        return acc;
    }
}

// MXFP4 F1 dot of one group against f16 activation pairs (QS_F16 layout of the fused prologue): byte u of a
// block's 16 code bytes converts, by the hardware e2m1 conversion scaled by 2 (jam's doubled codes,
// jam_mxfp4.h:14-15), to the codes of elements u and u + 16, which v_dot2 multiplies with the pair
// (q_u, q_{u+16}). Products and partial sums are integers below 2^16, exact in f32, so a block's sum is jam's
// integer I exactly; then fl(sw·da)·I as in group_dot. Half the VALU work of the int8 form (a byte's two
// codes in two instructions instead of a table lookup per four nibbles and a v_dot4).
JAMHIP_DEV float mx_dot_f16(const Group<MXFP4>& w, const int8_t* a2, const float* ad, int nbv) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < 8; b++) {
        const int bb = b < nbv ? b : nbv - 1;   // stay inside the token's activations
        float I = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint4 A = ld16(a2 + 64 * bb + 16 * j);   // pairs 4j .. 4j + 3
            const uint32_t wj = word(w.q[b], j);          // code bytes 4j .. 4j + 3
            I = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wj, 2.0f, 0),
                                       __builtin_bit_cast(h2, A.x), I, false);
            I = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wj, 2.0f, 1),
                                       __builtin_bit_cast(h2, A.y), I, false);
            I = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wj, 2.0f, 2),
                                       __builtin_bit_cast(h2, A.z), I, false);
            I = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wj, 2.0f, 3),
                                       __builtin_bit_cast(h2, A.w), I, false);
        }
        const float sw = e8m0_half((word(w.s, b >> 2) >> (8 * (b & 3))) & 0xffu);
        const float v = I * (sw * ad[bb]);
        acc += b < nbv ? v : 0.0f;
    }
    return acc;
}

// NVFP4 F1 dot (jam_mm_nvfp4_avx512, jam_kernels_avx512bw.c:111-142) against f16 activation pairs: byte u of a
// 16-element sub-block's 8 code bytes holds elements u (low nibble) and u + 8, which the e2m1 conversion
// (scaled by 2) returns as one pair for v_dot2 with (q_u, q_{u+8}); the sub-block sums are jam's integer I
// exactly (integers below 2^15), then fl(ue4m3(d_s)·ad)·I as in group_dot.
JAMHIP_DEV float nv_dot_f16(const Group<NVFP4>& w, const int8_t* a2, const float* ad, int nbv) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const bool live = 2 * j < nbv;
        const int jj = live ? j : nbv / 2 - 1;   // stay inside the token's activations
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const uint4 ch = w.q[2 * j + (s >> 1)];
            const uint32_t w0 = word(ch, 2 * (s & 1)), w1 = word(ch, 2 * (s & 1) + 1);
            const uint4 P0 = ld16(a2 + 32 * (4 * jj + s)), P1 = ld16(a2 + 32 * (4 * jj + s) + 16);
            float I = 0.0f;
            I = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w0, 2.0f, 0), __builtin_bit_cast(h2, P0.x), I, false);
            I = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w0, 2.0f, 1), __builtin_bit_cast(h2, P0.y), I, false);
            I = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w0, 2.0f, 2), __builtin_bit_cast(h2, P0.z), I, false);
            I = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w0, 2.0f, 3), __builtin_bit_cast(h2, P0.w), I, false);
            I = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w1, 2.0f, 0), __builtin_bit_cast(h2, P1.x), I, false);
            I = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w1, 2.0f, 1), __builtin_bit_cast(h2, P1.y), I, false);
            I = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w1, 2.0f, 2), __builtin_bit_cast(h2, P1.z), I, false);
            I = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w1, 2.0f, 3), __builtin_bit_cast(h2, P1.w), I, false);
            const float sc = ue4m3((word(w.s, j) >> (8 * s)) & 0xffu) * ad[2 * jj + (s >> 1)];
            acc += live ? I * sc : 0.0f;
        }
    }
    return acc;
}

// Q4_0 F1 decode with 3..7 tokens: the group's nibbles and block scales unpacked once for all the tokens
// (measured faster for Q4_0 only; the other types unpack per token in group_dot), then per token
// group_dot's Q4_0 arithmetic.
struct Q40Codes {
    uint4 c[16];   // block b: low nibbles c[2b], high nibbles c[2b + 1]
    float f[8];    // block scales
};

JAMHIP_DEV void q40_unpack(const Group<Q4_0>& w, Q40Codes& u) {
#pragma unroll
    for (int b = 0; b < 8; b++) {
        u.c[2 * b] = lo_nib(w.q[b]);
        u.c[2 * b + 1] = hi_nib(w.q[b]);
        u.f[b] = h2f((word(w.s, b >> 1) >> (16 * (b & 1))) & 0xffffu);
    }
}

// F2 (q4_0 block16, jam_kernels_q4k_avx512.c:463-480): fl(sw·dx)·I − fl(8·sw)·fl(xs0+xs1) per block, with
// I over the raw nibbles (0..15).
JAMHIP_DEV float q40_dot_f2(const Q40Codes& u, const int8_t* aq, const float* ad, const float* as, int nbv) {
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < 8; b++) {
        const int bq = b < nbv ? b : nbv - 1;   // stay inside the token's activations
        const int I = dot16(u.c[2 * b + 1], ld16(aq + 32 * bq + 16), dot16(u.c[2 * b], ld16(aq + 32 * bq), 0));
        float v = (float) I * (u.f[b] * ad[bq]);
        v -= (8.0f * u.f[b]) * (as[2 * bq] + as[2 * bq + 1]);
        acc += b < nbv ? v : 0.0f;
    }
    return acc;
}

JAMHIP_DEV float q40_dot_f1(const Q40Codes& u, const int8_t* aq, const float* ad, const int* s16, int nbv) {
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < 8; b++) {
        const int bq = b < nbv ? b : nbv - 1;   // stay inside the token's activations
        int I = dot16(u.c[2 * b + 1], ld16(aq + 32 * bq + 16), dot16(u.c[2 * b], ld16(aq + 32 * bq), 0));
        I -= 8 * (s16[2 * bq] + s16[2 * bq + 1]);
        const float v = (float) I * (u.f[b] * ad[bq]);   // q256 engine (jam_gemm_q256.inc:28-36): fl(sw·da)·I
        acc += b < nbv ? v : 0.0f;
    }
    return acc;
}

// ------------------------------------------------------------------------------ fused F1 prologue
// Quantizes NT activation rows into LDS with jam's F1 (quant.h) in the group layout: per token and group
// 256 int8 codes padded to QS_LDS bytes (conflict-free reads), 8 block scales, 8 block sums, 16 Σq per 16.
// One thread per 16-element half-block; the halves of a 32-block sit in adjacent lanes, which exchange
// their |x| maxima and Σq. Elements past k (a partial last group) quantize as zeros.
constexpr int QS_LDS = 272;
// The e2m1 types with one token (fused prologue): the codes go to LDS as f16 pairs in the order in which the
// e2m1 conversion returns a weight byte's two codes: (q_i, q_{i+16}) of each 32-block for MXFP4 (mode 1,
// mx_dot_f16), (q_i, q_{i+8}) of each 16-element sub-block for NVFP4 (mode 2, nv_dot_f16); 512 bytes per
// group, padded to QS_F16. Mode 0: int8 codes.
constexpr int QS_F16 = 528;
template <int DT, int FL, int NT, int HP> constexpr int f16_pairs() {
    return FL == 1 && NT == 1 && HP > 0 ? (DT == MXFP4 ? 1 : DT == NVFP4 ? 2 : 0) : 0;
}
constexpr int MV_WAVES = 8;   // waves per GEMV workgroup (512 threads)

// The prologue runs in two steps so that its activation loads go out before the weight stream: a_load
// issues HP unconditional half-block loads per thread (indices clamped; halves past k read as zero),
// f1_store quantizes them and writes LDS. HP = ceil(NT·16·Gk / 512) half-blocks per thread.
template <int HP> struct APre { float x[HP][16]; };

// Half-block i of this thread in the fused F1 prologue: wave w takes the contiguous half-blocks
// [64·HP·w, 64·HP·(w + 1)), lane l every 64th of them (pairs of a block on adjacent lanes). When a band
// fills the workgroup (one token, one item per wave, J = NWV, HP = 2) these are exactly the 8 groups the
// wave's own dot products read, so the prologue needs no workgroup barrier.
template <int HP> JAMHIP_DEV int pro_half(int i) { return 64 * HP * (int) (threadIdx.x >> 6) + 64 * i + (int) (threadIdx.x & 63); }

template <int NT, int HP, int NWV, bool GATHER = false>
JAMHIP_DEV void a_load(APre<HP>& pre, const float* __restrict__ a, int lda, int k, int Gk, int ntv,
                       const int* __restrict__ rows = nullptr, int rdiv = 1) {
    // GATHER: token j's row is a[rows[j] / rdiv] (a grouped call with the gather folded in)
    // four 16-byte loads per half-block (the launcher checks a and lda for 16-byte alignment); a half past
    // the token's last element (a partial last group) re-reads the token's last half, zeroed by f1_store
    // (zeroing here would make the wave wait for these loads before issuing the weight loads). Only the
    // ntv tokens present are quantized (a grouped call's expert may hold fewer rows than NT).
    const int halves = 16 * Gk, total = (NT == 1 ? 1 : ntv) * halves, kh = k >> 4;
#pragma unroll
    for (int i = 0; i < HP; i++) {
        const int h0 = pro_half<HP>(i), h = h0 < total ? h0 : total - 1;
        const int j = NT == 1 ? 0 : h / halves, hh = h - j * halves, jr = j < ntv ? j : ntv - 1;   // rows past ntv: clamp
        const bool in = hh < kh;   // clamp only; the zeroing happens in f1_store
        const int64_t rj = GATHER ? (int64_t) (rows[jr] / rdiv) : (int64_t) jr;
        const float4* src = reinterpret_cast<const float4*>(a + rj * lda + 16 * (in ? hh : kh - 1));
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float4 f = src[v];
            pre.x[i][4 * v + 0] = f.x;
            pre.x[i][4 * v + 1] = f.y;
            pre.x[i][4 * v + 2] = f.z;
            pre.x[i][4 * v + 3] = f.w;
        }
    }
}

template <int NT, int HP, int NWV, int F16P = 0>
JAMHIP_DEV void f1_store(const APre<HP>& pre, int k, int Gk, int ntv, int8_t* lq, float* ld, float* las, int* ls16,
                         char* dummy) {
    // branch-free: a thread past the last half-block (its loads were clamped) quantizes anyway and writes to
    // a dummy LDS slot; pairs stay aligned because the half-block count is even
    const int halves = 16 * Gk, total = (NT == 1 ? 1 : ntv) * halves;
#pragma unroll
    for (int i = 0; i < HP; i++) {
        const int h0 = pro_half<HP>(i);
        const bool valid = h0 < total;
        const int h = valid ? h0 : 0;
        const int j = NT == 1 ? 0 : h / halves, hh = h - j * halves;
        const bool in = hh < (k >> 4);
        float x[16];
#pragma unroll
        for (int e = 0; e < 16; e++) x[e] = in ? pre.x[i][e] : 0.0f;
        float am = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; e++) am = fmaxf(am, fabsf(x[e]));
        am = fmaxf(am, xor1_f(am));
        const float db = am / 127.0f;
        const float id = db > 0.0f ? 1.0f / db : 0.0f;
        if constexpr (F16P == 2) {
            // pair slot u of this half (an NVFP4 sub-block) is (q_u, q_{u+8}), both this thread's; exact in f16
            if (valid) {
                uint32_t sp[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const float q0 = fminf(fmaxf(rintf(x[u] * id), -128.0f), 127.0f);
                    const float q1 = fminf(fmaxf(rintf(x[u + 8] * id), -128.0f), 127.0f);
                    sp[u] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(q0, q1));
                }
                uint4* p4 = reinterpret_cast<uint4*>(lq + (int64_t) (hh >> 4) * QS_F16 + 32 * (hh & 15));
                p4[0] = make_uint4(sp[0], sp[1], sp[2], sp[3]);
                p4[1] = make_uint4(sp[4], sp[5], sp[6], sp[7]);
                if ((hh & 1) == 0) ld[hh >> 1] = db;
            }
            continue;
        }
        if constexpr (F16P == 1) {
            // element e of this half is f16 number (hh & 1) of pair slot e of its block (the codes are
            // integers in [-128, 127], exact in f16 whatever the rounding); MXFP4 reads no sums
            if (valid) {
                uint16_t* p2 = reinterpret_cast<uint16_t*>(lq + (int64_t) (hh >> 4) * QS_F16 + 64 * ((hh >> 1) & 7) +
                                                           2 * (hh & 1));
#pragma unroll
                for (int e = 0; e < 16; e += 2) {
                    const float q0 = fminf(fmaxf(rintf(x[e] * id), -128.0f), 127.0f);
                    const float q1 = fminf(fmaxf(rintf(x[e + 1] * id), -128.0f), 127.0f);
                    const uint32_t v = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(q0, q1));
                    p2[2 * e] = (uint16_t) (v & 0xffffu);
                    p2[2 * e + 2] = (uint16_t) (v >> 16);
                }
                if ((hh & 1) == 0) ld[hh >> 1] = db;
            }
            continue;
        }
        uint32_t pk[4];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint32_t v = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                // lrintf then clamp; a NaN product (non-finite input) lands on -128 like LONG_MIN does
                const int q = (int) fminf(fmaxf(rintf(x[4 * g + e] * id), -128.0f), 127.0f);
                v |= (uint32_t) (q & 0xff) << (8 * e);
            }
            pk[g] = v;
        }
        int s = dot4((int) pk[0], 0x01010101, 0);
        s = dot4((int) pk[1], 0x01010101, s);
        s = dot4((int) pk[2], 0x01010101, s);
        s = dot4((int) pk[3], 0x01010101, s);
        const int s32 = s + xor1_i(s);
        int8_t* pq = valid ? lq + (int64_t) (j * Gk + (hh >> 4)) * QS_LDS + 16 * (hh & 15) : (int8_t*) dummy;
        int* p16 = valid ? ls16 + j * halves + hh : (int*) (dummy + 16);
        const bool first = (hh & 1) == 0;
        float* pd = valid && first ? ld + j * 8 * Gk + (hh >> 1) : (float*) (dummy + 20);
        float* ps = valid && first ? las + j * 8 * Gk + (hh >> 1) : (float*) (dummy + 24);
        *reinterpret_cast<uint4*>(pq) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        *p16 = s;
        *pd = db;
        *ps = (float) s32;
    }
}

// F2 activations staged in LDS (8-token tiles, already quantized by quant_f2_kernel into A): the tile's
// codes in the fused layout (group g of token t at lq + (t·Gk + g)·QS_LDS), block scales (ld, 8 per group)
// and per-16 sums (lx, 16 per group), copied once per workgroup so that the dot products read LDS instead
// of each lane fetching its tokens' activations from L2 (measured slower for F1 at large k, which keeps
// the L2 reads). As for the fused F1 quantizer, stage_load's loads go out before the weight stream and
// stage_store writes LDS after it. Tokens past ntv repeat token ntv - 1; 16-byte pieces past k (a partial
// last group) re-read the row's last piece and are never read back (group_dot clamps to the group's last
// valid block). SP = ceil(NT·Gk·16 / 512) code pieces per thread, 2·SP floats.
template <int SP> struct FPre {
    uint4 q[SP];
    float f[2 * SP];
};

// k: the row length of A (its stride); elements [k0, k0 + kl) of each token are staged (k0 % 256 == 0).
template <int NT, int SP, int NWV>
JAMHIP_DEV void stage_load(FPre<SP>& pre, const ActQ& A, int k, int k0, int kl, int Gk, int t0, int ntv) {
    const int nbf = k >> 5, nb = kl >> 5, units = NT * Gk * 16, nf = NT * 3 * nb;
#pragma unroll
    for (int i = 0; i < SP; i++) {
        const int u0 = threadIdx.x + 64 * NWV * i, u = u0 < units ? u0 : units - 1;
        const int t = u / (Gk * 16), r = u - t * Gk * 16, tc = t < ntv ? t : ntv - 1;
        const int off = 256 * (r >> 4) + 16 * (r & 15);
        pre.q[i] = ld16(A.q + (int64_t) (t0 + tc) * k + k0 + (off < kl ? off : kl - 16));
    }
#pragma unroll
    for (int i = 0; i < 2 * SP; i++) {
        const int v0 = threadIdx.x + 64 * NWV * i, v = v0 < nf ? v0 : nf - 1;
        const int t = v / (3 * nb), r = v - t * 3 * nb, tc = t < ntv ? t : ntv - 1;
        pre.f[i] = r < nb ? A.d[(int64_t) (t0 + tc) * nbf + (k0 >> 5) + r]
                          : A.s[(int64_t) (t0 + tc) * 2 * nbf + (k0 >> 4) + (r - nb)];
    }
}

template <int NT, int SP, int NWV>
JAMHIP_DEV void stage_store(const FPre<SP>& pre, int k, int Gk, int8_t* lq, float* ld, float* lx) {
    const int nb = k >> 5, units = NT * Gk * 16, nf = NT * 3 * nb;
#pragma unroll
    for (int i = 0; i < SP; i++) {
        const int u = threadIdx.x + 64 * NWV * i;
        if (u < units) {
            const int t = u / (Gk * 16), r = u - t * Gk * 16;
            *reinterpret_cast<uint4*>(lq + (t * Gk + (r >> 4)) * QS_LDS + 16 * (r & 15)) = pre.q[i];
        }
    }
#pragma unroll
    for (int i = 0; i < 2 * SP; i++) {
        const int v = threadIdx.x + 64 * NWV * i;
        if (v < nf) {
            const int t = v / (3 * nb), r = v - t * 3 * nb;
            if (r < nb) ld[t * 8 * Gk + r] = pre.f[i];
            else lx[t * 16 * Gk + (r - nb)] = pre.f[i];
        }
    }
}

// ------------------------------------------------------------------------------------------ kernel
// One workgroup (8 waves) computes one block of rows with straight-line code: the compiler can then count
// every outstanding load exactly (a branch between a load and its use makes it drain the whole queue).
// Lanes: RB consecutive rows (lane % RB) x GS = 64 / RB group slots (lane / RB), so chunk c of an item is
// GS runs of 16·RB contiguous bytes in the row-tiled layout. An item is a band of RB rows x GS groups; a
// row band needs J = ceil(Gk / GS) items and a block is QB bands x J items = at most 8·ITEMS items, wave w
// taking items w·ITEMS .. w·ITEMS+ITEMS-1 (an item past the block re-reads a real group and adds nothing).
// Order: the activation loads, then every weight load of the wave, then the F1 quantization into LDS
// (waiting for the activations only), a barrier, the items in order, each lane parking its per-group
// partial in LDS, and finally each row's J·GS partials summed in a fixed order (deterministic, no
// atomics, no cross-lane shuffles).
// FL = 1: F1 activations, NT = n (1..7). HP > 0: quantized into LDS by this workgroup (HP half-blocks
// per thread); HP = 0: read from A. FL = 2: F2 activations from A; blockIdx.y picks NT tokens, the last
// group may hold fewer (ntv).
// GR (grouped matmul): FL = 1 takes expert blockIdx.y if it has 1..7 rows (ntv of them, CSR rows from
// off[e]); FL = 2 takes the 8-token tile blockIdx.y of map8. The expert's weight rows start at e·gm.
// The kernel body; by is the workgroup's column (a column of one flavour's range in mv_pair_kernel).
template <int DT, int FL, int NT, int HP, int RB, int ITEMS, bool GR, bool SK, int NWV>
__device__ __attribute__((always_inline)) inline void mv_body(WeightView w, ActQ A, const float* __restrict__ a,
                                                              int lda, int k, int m, int n, float* __restrict__ c,
                                                              int ldc, Groups gp, int ks, int64_t cz, Epi ep,
                                                              unsigned by) {
#define MV_COL by
#include "gemv_body.inc"
#undef MV_COL
}

template <int DT, int FL, int NT, int HP, int RB, int ITEMS, bool GR, bool SK, int NWV>
__global__ void __launch_bounds__(64 * NWV) mv_kernel(WeightView w, ActQ A, const float* __restrict__ a,
                                                          int lda, int k, int m, int n, float* __restrict__ c,
                                                          int ldc, Groups gp, int ks, int64_t cz, Epi ep) {
#define MV_COL blockIdx.y
#include "gemv_body.inc"
#undef MV_COL
}

// Both F1 grouped flavours in one launch (decode-sized calls whose experts come from the counts): columns
// [0, n1) run the one-token body over the experts with one row, the rest the seven-token body over those
// with 2..7 rows.
template <int DT, int HP1, int HP7, int RB, int ITEMS>
__global__ void __launch_bounds__(64 * MV_WAVES) mv_pair_kernel(WeightView w, ActQ A, const float* __restrict__ a,
                                                                 int lda, int k, float* __restrict__ c, int ldc,
                                                                 Groups gp, int n1) {
    const int y = (int) blockIdx.y;
    if (y < n1)
        mv_body<DT, 1, 1, HP1, RB, ITEMS, true, false, MV_WAVES>(w, A, a, lda, k, gp.gm, 0, c, ldc, gp, k, 0, Epi{}, (unsigned) y);
    else
        mv_body<DT, 1, 7, HP7, RB, ITEMS, true, false, MV_WAVES>(w, A, a, lda, k, gp.gm, 0, c, ldc, gp, k, 0, Epi{},
                                                                 (unsigned) (y - n1));
}

// ----------------------------------------------------------------------------- float-dot tail rows
// The last m % 16 rows of an n >= 8 call: jam's bands compute them with an exact float dot of the
// dequantized weight against the f32 activations ("<16-row tail: scalar exact dot",
// jam_kernels_q4k_avx512.c:185-188 and its siblings). One wave per (row, 8-token group); lane l takes
// the 32-element chunks l, l+64, ...; products accumulate in f32.
template <int DT>
JAMHIP_DEV float deq(const WeightView& w, int64_t row, int elem) {
    const int64_t g = elem >> 8;
    const int e = elem & 255;
    const uint8_t* q = group_q<DT>(w, row, g);
    const uint8_t* s = group_s<DT>(w, row, g);
    auto qb = [&](int byte) { return q[(byte >> 4) * CHUNK_STRIDE + (byte & 15)]; };   // group byte
    auto f16 = [&](const uint8_t* p) { return h2f((uint32_t) p[0] | ((uint32_t) p[1] << 8)); };
    if constexpr (DT == Q8_0) {
        return f16(s + 2 * (e >> 5)) * (float) (int8_t) qb(e);
    } else if constexpr (DT == Q4_0) {
        const uint8_t b = qb(16 * (e >> 5) + (e & 15));
        return f16(s + 2 * (e >> 5)) * (float) (((e & 31) < 16 ? b & 15 : b >> 4) - 8);
    } else if constexpr (DT == MXFP4) {
        const uint8_t b = qb(16 * (e >> 5) + (e & 15));
        const uint32_t code = mxfp4_codes((e & 31) < 16 ? b & 15 : b >> 4);
        return e8m0_half(s[e >> 5]) * (float) (int8_t) (code & 0xff);
    } else if constexpr (DT == NVFP4) {   // 64-block j, sub-block s: byte 8s + (i & 7), high nibble from i = 8
        const int j = e >> 6, sb = (e >> 4) & 3, i = e & 15;
        const uint8_t b = qb(32 * j + 8 * sb + (i & 7));
        const uint32_t code = mxfp4_codes(i < 8 ? b & 15 : b >> 4);
        return ue4m3(s[4 * j + sb]) * (float) (int8_t) (code & 0xff);
    } else if constexpr (DT == Q1_0) {
        const int j = e >> 7, i = e & 127;
        const float d = f16(s + 2 * j);
        return (qb(16 * j + (i >> 3)) >> (i & 7)) & 1 ? d : -d;
    } else if constexpr (DT == Q4_K || DT == Q5_K) {
        const int gp = e >> 6, half = (e >> 5) & 1, l = e & 31, sb = 2 * gp + half;
        const uint8_t b = qb(32 * gp + l);
        const int hb = DT == Q5_K ? ((qb(128 + l) >> sb) & 1) << 4 : 0;
        const uint4 h = make_uint4(s[0] | s[1] << 8 | s[2] << 16 | (uint32_t) s[3] << 24,
                                   s[4] | s[5] << 8 | s[6] << 16 | (uint32_t) s[7] << 24,
                                   s[8] | s[9] << 8 | s[10] << 16 | (uint32_t) s[11] << 24,
                                   s[12] | s[13] << 8 | s[14] << 16 | (uint32_t) s[15] << 24);
        int sc, mn;
        q4k_sm(h, sb, sc, mn);
        return f16(s) * (float) sc * (float) ((half ? b >> 4 : b & 15) | hb) - f16(s + 2) * (float) mn;
    } else {
        const int hh = e >> 7, j = (e & 127) >> 5, l = e & 31;
        const uint8_t qlb = qb(64 * hh + (j & 1) * 32 + l);
        const int q6 = (j < 2 ? qlb & 15 : qlb >> 4) | (((qb(128 + 32 * hh + l) >> (2 * j)) & 3) << 4);
        const int sc = (int) (int8_t) qb(192 + 8 * hh + 2 * j + l / 16);
        return f16(s) * (float) sc * (float) (q6 - 32);
    }
}

template <int DT>
__global__ void __launch_bounds__(64) rows_float_kernel(WeightView w, const float* __restrict__ a, int lda, int k,
                                                        int r0, int n, float* __restrict__ c, int ldc, Epi ep) {
    const int64_t row = r0 + blockIdx.x;
    const int t0 = blockIdx.y * 8, nt = n - t0 < 8 ? n - t0 : 8;
    const int lane = threadIdx.x;
    float acc[8];
#pragma unroll
    for (int t = 0; t < 8; t++) acc[t] = 0.0f;
    for (int chunk = lane; chunk < k / 32; chunk += 64) {   // 32 consecutive elements per lane and step
        for (int e = 32 * chunk; e < 32 * chunk + 32; e++) {
            const float v = deq<DT>(w, row, e);
#pragma unroll
            for (int t = 0; t < 8; t++)
                if (t < nt) acc[t] += v * a[(int64_t) (t0 + t) * lda + e];
        }
    }
#pragma unroll
    for (int t = 0; t < 8; t++) {
        const float v = wave_sum(acc[t]);
        if (lane == 0 && t < nt) {
            float* dst = c + (int64_t) (t0 + t) * ldc + row;
            *dst = epilogue(ep, v, row, dst);
        }
    }
}

// ---------------------------------------------------------------------------------------- launchers
// Fused F1 quantization keeps A's codes, scales and sums in LDS: 400 bytes per token and group; its
// prologue holds up to 4 half-blocks of A per thread in registers.
constexpr int kFuseMaxBytes = 96 * 1024;
// Dynamic LDS above 64 KB needs the kernel's limit raised (once per kernel, to the largest size asked).
static void lds_allow(const void* fn, size_t bytes) {
    static std::mutex mu;
    static std::vector<std::pair<const void*, size_t>> done;
    if (bytes <= 65536) return;
    std::lock_guard<std::mutex> lock(mu);
    for (auto& d : done)
        if (d.first == fn) {
            if (d.second >= bytes) return;
            (void) hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int) bytes);
            d.second = bytes;
            return;
        }
    (void) hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int) bytes);
    done.emplace_back(fn, bytes);
}
static size_t fuse_lds(int n, int k, bool f16p = false) {
    return (size_t) n * ((k / 32 + 7) / 8) * ((f16p ? QS_F16 : QS_LDS) + 32 + 32 + 64);
}
static int fuse_hp(int n, int k) { return (n * 16 * ((k / 32 + 7) / 8) + 64 * MV_WAVES - 1) / (64 * MV_WAVES); }

// Work split: bands of RB = 8 rows (x 8 group slots: chunk loads are 128-byte lines; 16-row bands measured
// slower at every BASELINE shape, 4-row bands 1.5-1.75x slower at k = 14336) and the fewest items per wave that fit a band in one block, 1, 2 or 4
// for k up to 16384, 32768, 65536. More items per wave only add registers. JAM_HIP_MV_ITEMS overrides
// (tuning sweeps). Returns false past k = 65536.
constexpr int MV_RB = 8;
static bool mv_items(int k, int* items) {
    const int Gk = (k / 32 + 7) / 8, J = (Gk + 64 / MV_RB - 1) / (64 / MV_RB);
    const char* vi = getenv("JAM_HIP_MV_ITEMS");
    int it = vi ? atoi(vi) : 1;
    const int lo = (J + MV_WAVES - 1) / MV_WAVES;
    it = it < lo ? lo : it;
    it = it <= 1 ? 1 : it <= 2 ? 2 : 4;
    *items = it;
    return J <= MV_WAVES * it;
}

// Split K: from k = 2·GEMV_SLICE on and for 2 or more tokens, the workgroups of a band take GEMV_SLICE-element
// slices of k (grid z) so that a block keeps 32-row bands and its slice of every token's activations fits
// LDS; partials are summed after. One token's activations fit unsplit (measured faster unsplit) up to
// k = 65536, the most a row band holds (mv_items); past that one token takes slices of GEMV_SLICE1.
constexpr int GEMV_SLICE = 4096, GEMV_SLICE1 = 32768, GEMV_K1_MAX = 65536;
inline int gemv_slice(int k, int n) {
    return n >= 2 && k >= 2 * GEMV_SLICE ? GEMV_SLICE : n == 1 && k > GEMV_K1_MAX ? GEMV_SLICE1 : k;
}

// ks: elements per K slice (= k unsplit); cz: floats between the slices' partial outputs; NWV: waves per
// workgroup.
template <int DT, int FL, int NT, int HP, int RB, int ITEMS, int NWV = MV_WAVES>
static void launch_shape(int k, int ks, int64_t cz, int m, int n, const WeightView& w, const ActQ& A, const float* a,
                         int lda, float* c, int ldc, hipStream_t st, const Epi& ep) {
    constexpr int GS = 64 / RB;
    const int Gk = (ks / 32 + 7) / 8, J = (Gk + GS - 1) / GS;
    const int QB = NWV * ITEMS / J;
    const int64_t bands = ((int64_t) m + RB - 1) / RB;
    const dim3 grid((unsigned) ((bands + QB - 1) / QB), (n + NT - 1) / NT, (unsigned) ((k + ks - 1) / ks));
    const size_t lds = (size_t) NWV * ITEMS * 64 * NT * sizeof(float) +
                       (HP > 0 ? 32 + fuse_lds(NT, ks, f16_pairs<DT, FL, NT, HP>()) : 0);
    {   // split K (2 or more tokens from k = 8192, one token past k = 65536)
        if (ks < k) {
            lds_allow((const void*) mv_kernel<DT, FL, NT, HP, RB, ITEMS, false, true, NWV>, lds);
            mv_kernel<DT, FL, NT, HP, RB, ITEMS, false, true, NWV><<<grid, 64 * NWV, lds, st>>>(
                w, A, a, lda, k, m, n, c, ldc, Groups{}, ks, cz, Epi{});
            return;
        }
    }
    lds_allow((const void*) mv_kernel<DT, FL, NT, HP, RB, ITEMS, false, false, NWV>, lds);
    mv_kernel<DT, FL, NT, HP, RB, ITEMS, false, false, NWV><<<grid, 64 * NWV, lds, st>>>(w, A, a, lda, k, m, n, c, ldc,
                                                                                        Groups{}, k, 0, ep);
}

template <int DT, int FL, int NT, int HP, int RB, int ITEMS>
static void launch_shape_grouped(int k, const Groups& g, int ny, const WeightView& w, const ActQ& A, const float* a,
                                 int lda, float* c, int ldc, hipStream_t st) {
    constexpr int GS = 64 / RB;
    const int Gk = (k / 32 + 7) / 8, J = (Gk + GS - 1) / GS;
    const int QB = MV_WAVES * ITEMS / J;
    const int64_t bands = ((int64_t) g.gm + RB - 1) / RB;
    const dim3 grid((unsigned) ((bands + QB - 1) / QB), (unsigned) ny);
    const size_t lds = (size_t) MV_WAVES * ITEMS * 64 * NT * sizeof(float) +
                       (HP > 0 ? 32 + fuse_lds(NT, k, f16_pairs<DT, FL, NT, HP>()) : 0);
    lds_allow((const void*) mv_kernel<DT, FL, NT, HP, RB, ITEMS, true, false, MV_WAVES>, lds);
    mv_kernel<DT, FL, NT, HP, RB, ITEMS, true, false, MV_WAVES><<<grid, 64 * MV_WAVES, lds, st>>>(w, A, a, lda, k, g.gm,
                                                                                                 0, c, ldc, g, k, 0, Epi{});
}

template <int DT, int FL, int NT, int HP>
static hipError_t go_grouped(int k, const Groups& g, int ny, const WeightView& w, const ActQ& A, const float* a,
                             int lda, float* c, int ldc, hipStream_t st) {
    int items;
    if (!mv_items(k, &items)) return hipErrorNotSupported;
    if (items == 1) launch_shape_grouped<DT, FL, NT, HP, MV_RB, 1>(k, g, ny, w, A, a, lda, c, ldc, st);
    else if (items == 2) launch_shape_grouped<DT, FL, NT, HP, MV_RB, 2>(k, g, ny, w, A, a, lda, c, ldc, st);
    else launch_shape_grouped<DT, FL, NT, HP, MV_RB, 4>(k, g, ny, w, A, a, lda, c, ldc, st);
    return hipGetLastError();
}

template <int DT, int HP1, int HP7, int RB, int ITEMS>
static void launch_pair(int k, const Groups& g, int n1, int n2, const WeightView& w, const ActQ& A, const float* a,
                        int lda, float* c, int ldc, hipStream_t st) {
    constexpr int GS = 64 / RB;
    const int Gk = (k / 32 + 7) / 8, J = (Gk + GS - 1) / GS;
    const int QB = MV_WAVES * ITEMS / J;
    const int64_t bands = ((int64_t) g.gm + RB - 1) / RB;
    const dim3 grid((unsigned) ((bands + QB - 1) / QB), (unsigned) (n1 + n2));
    const size_t l1 = (size_t) MV_WAVES * ITEMS * 64 * sizeof(float) +
                      (HP1 > 0 ? 32 + fuse_lds(1, k, f16_pairs<DT, 1, 1, HP1>()) : 0);
    const size_t l7 = (size_t) MV_WAVES * ITEMS * 64 * 7 * sizeof(float) +
                      (HP7 > 0 ? 32 + fuse_lds(7, k, f16_pairs<DT, 1, 7, HP7>()) : 0);
    const size_t lds = l1 > l7 ? l1 : l7;
    lds_allow((const void*) mv_pair_kernel<DT, HP1, HP7, RB, ITEMS>, lds);
    mv_pair_kernel<DT, HP1, HP7, RB, ITEMS><<<grid, 64 * MV_WAVES, lds, st>>>(w, A, a, lda, k, c, ldc, g, n1);
}

template <int DT, int HP1, int HP7>
static hipError_t go_pair(int k, const Groups& g, int n1, int n2, const WeightView& w, const ActQ& A, const float* a,
                          int lda, float* c, int ldc, hipStream_t st) {
    int items;
    if (!mv_items(k, &items)) return hipErrorNotSupported;
    if (items == 1) launch_pair<DT, HP1, HP7, MV_RB, 1>(k, g, n1, n2, w, A, a, lda, c, ldc, st);
    else if (items == 2) launch_pair<DT, HP1, HP7, MV_RB, 2>(k, g, n1, n2, w, A, a, lda, c, ldc, st);
    else launch_pair<DT, HP1, HP7, MV_RB, 4>(k, g, n1, n2, w, A, a, lda, c, ldc, st);
    return hipGetLastError();
}

template <int DT>
hipError_t gemv_grouped_dt(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k,
                                  const Groups& g, int E, int cap8, float* c, int ldc, hipStream_t st) {
    if (flavour == 2) return go_grouped<DT, 2, 8, 0>(k, g, cap8, w, A, nullptr, 0, c, ldc, st);
    if (flavour == 3) {   // both F1 flavours in one launch, experts from g.counts: E = n1 columns, cap8 = n2
        if (a == nullptr) return go_pair<DT, 0, 0>(k, g, E, cap8, w, A, nullptr, 0, c, ldc, st);
        const int h1 = fuse_hp(1, k), h7 = fuse_hp(7, k);
        if (h7 <= 1) return go_pair<DT, 1, 1>(k, g, E, cap8, w, A, a, lda, c, ldc, st);
        if (h7 == 2) return h1 <= 1 ? go_pair<DT, 1, 2>(k, g, E, cap8, w, A, a, lda, c, ldc, st)
                                    : go_pair<DT, 2, 2>(k, g, E, cap8, w, A, a, lda, c, ldc, st);
        return h1 <= 1 ? go_pair<DT, 1, 4>(k, g, E, cap8, w, A, a, lda, c, ldc, st)
                       : h1 == 2 ? go_pair<DT, 2, 4>(k, g, E, cap8, w, A, a, lda, c, ldc, st)
                                 : go_pair<DT, 4, 4>(k, g, E, cap8, w, A, a, lda, c, ldc, st);
    }
    if (flavour == 0) {   // one-row experts: one token's registers, LDS and prologue
        if (a == nullptr) return go_grouped<DT, 1, 1, 0>(k, g, E, w, A, nullptr, 0, c, ldc, st);
        const int hp = fuse_hp(1, k);
        if (hp <= 1) return go_grouped<DT, 1, 1, 1>(k, g, E, w, A, a, lda, c, ldc, st);
        if (hp == 2) return go_grouped<DT, 1, 1, 2>(k, g, E, w, A, a, lda, c, ldc, st);
        return go_grouped<DT, 1, 1, 4>(k, g, E, w, A, a, lda, c, ldc, st);
    }
    if (a == nullptr) return go_grouped<DT, 1, 7, 0>(k, g, E, w, A, nullptr, 0, c, ldc, st);
    const int hp = fuse_hp(7, k);
    if (hp <= 1) return go_grouped<DT, 1, 7, 1>(k, g, E, w, A, a, lda, c, ldc, st);
    if (hp == 2) return go_grouped<DT, 1, 7, 2>(k, g, E, w, A, a, lda, c, ldc, st);
    return go_grouped<DT, 1, 7, 4>(k, g, E, w, A, a, lda, c, ldc, st);
}


template <int DT, int FL, int NT, int HP>
static hipError_t go_hp(int k, int ks, int64_t cz, int m, int n, const WeightView& w, const ActQ& A, const float* a,
                        int lda, float* c, int ldc, hipStream_t st, const Epi& ep) {
    int items;
    if (!mv_items(ks, &items)) return hipErrorNotSupported;
    if constexpr (FL == 2 && HP > 0) {   // staged activations: one item per wave (slices <= 16384)
        if (items != 1) return go_hp<DT, FL, NT, 0>(k, ks, cz, m, n, w, A, a, lda, c, ldc, st, ep);
        launch_shape<DT, FL, NT, HP, MV_RB, 1>(k, ks, cz, m, n, w, A, a, lda, c, ldc, st, ep);
        return hipGetLastError();
    }
    if (items == 1) launch_shape<DT, FL, NT, HP, MV_RB, 1>(k, ks, cz, m, n, w, A, a, lda, c, ldc, st, ep);
    else if (items == 2) launch_shape<DT, FL, NT, HP, MV_RB, 2>(k, ks, cz, m, n, w, A, a, lda, c, ldc, st, ep);
    else launch_shape<DT, FL, NT, HP, MV_RB, 4>(k, ks, cz, m, n, w, A, a, lda, c, ldc, st, ep);
    return hipGetLastError();
}

// Waves per workgroup for one token. A row band of J items that does not divide 8 (J = 3, 5, 6, 7: k up to
// 6144, 10240, 12288, 14336, e.g. Llama's FFN down projection at 14336) takes workgroups of J·floor(8 / J)
// waves: with 8, the spare waves only re-read the next band's weights (measured at k = 14336: Q6_K 4096x14336
// 12.9 -> 12.1 us). With one or two items per band (k <= 4096) a workgroup of 4 or 8 waves holds 4 / J or
// 8 / J bands; the one whose last partial round of workgroups over the CUs is fuller (workgroups / CUs over
// its ceiling) wins, and on a tie 8 waves, unless both fill every round (then 4). Q4_K at k = 4096, graph-timed
// (4 / 8 waves, us): 4096 rows 4.04 / 4.37, 6144 5.30 / 4.88, 10240 6.53 / 6.85, 14336 7.99 / 7.46, 20480
// 9.94 / 10.32, 28672 12.59 / 13.25, 57344 22.2 / 23.7; MXFP4 5760x2880 5.66 / 5.48; 12, 14 and 16 waves
// and 2 items per wave were slower everywhere. JAM_HIP_MV_WAVES overrides (tuning sweeps).
static int one_token_waves(int k, int m) {
    int items;
    if (!mv_items(k, &items) || items != 1) return MV_WAVES;
    const int Gk = (k / 32 + 7) / 8, J = (Gk + 64 / MV_RB - 1) / (64 / MV_RB);
    const int64_t bands = ((int64_t) m + MV_RB - 1) / MV_RB;
    if (const char* v = getenv("JAM_HIP_MV_WAVES")) {
        const int x = atoi(v);
        if (x >= 4 && x <= 8 && x % J == 0) return x;
    }
    if (J == 3 || J == 5 || J == 6 || J == 7) return J * (MV_WAVES / J);
    if (J > 2) return MV_WAVES;
    const int64_t cus = device_cus() >= 8 ? device_cus() : 256;
    const int64_t w4 = (bands + 4 / J - 1) / (4 / J), w8 = (bands + 8 / J - 1) / (8 / J);
    const int64_t r4 = (w4 + cus - 1) / cus, r8 = (w8 + cus - 1) / cus;   // rounds
    // fullness w / (r·cus), compared without division
    if (w4 * r8 != w8 * r4) return w4 * r8 > w8 * r4 ? 4 : 8;
    return w4 == r4 * cus && w8 == r8 * cus ? 4 : 8;
}

template <int DT, int NWV>
static hipError_t go_one(const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m, float* c, int ldc,
                         hipStream_t st, const Epi& ep) {
    // at most 2 half-blocks per thread in the fused prologue (J <= NWV items of 8 groups, 16 half-blocks each)
    const int Gk = (k / 32 + 7) / 8, hp = a != nullptr ? (16 * Gk + 64 * NWV - 1) / (64 * NWV) : 0;
    if (hp == 0) launch_shape<DT, 1, 1, 0, MV_RB, 1, NWV>(k, k, 0, m, 1, w, A, a, lda, c, ldc, st, ep);
    else if (hp == 1) launch_shape<DT, 1, 1, 1, MV_RB, 1, NWV>(k, k, 0, m, 1, w, A, a, lda, c, ldc, st, ep);
    else launch_shape<DT, 1, 1, 2, MV_RB, 1, NWV>(k, k, 0, m, 1, w, A, a, lda, c, ldc, st, ep);
    return hipGetLastError();
}

template <int DT, int FL, int NT>
static hipError_t go(const WeightView& w, const ActQ& A, const float* a, int lda, int k, int ks, int64_t cz, int m,
                     int n, float* c, int ldc, hipStream_t st, const Epi& ep) {
    if constexpr (FL == 1 && NT == 1) {
        if (ks == k) {
            const int nw = one_token_waves(k, m);
            if (nw == 4) return go_one<DT, 4>(w, A, a, lda, k, m, c, ldc, st, ep);
            if (nw == 5) return go_one<DT, 5>(w, A, a, lda, k, m, c, ldc, st, ep);
            if (nw == 6) return go_one<DT, 6>(w, A, a, lda, k, m, c, ldc, st, ep);
            if (nw == 7) return go_one<DT, 7>(w, A, a, lda, k, m, c, ldc, st, ep);
        }
    }
    if constexpr (FL == 2) {   // stage the tile's activations in LDS when they fit
        const int hp = (NT * ((ks / 32 + 7) / 8) * 16 + 64 * MV_WAVES - 1) / (64 * MV_WAVES);
        if (fuse_lds(NT, ks) <= (size_t) kFuseMaxBytes && hp <= 8) {
            if (hp <= 2) return go_hp<DT, FL, NT, 2>(k, ks, cz, m, n, w, A, a, lda, c, ldc, st, ep);
            if (hp <= 4) return go_hp<DT, FL, NT, 4>(k, ks, cz, m, n, w, A, a, lda, c, ldc, st, ep);
            return go_hp<DT, FL, NT, 8>(k, ks, cz, m, n, w, A, a, lda, c, ldc, st, ep);
        }
    }
    if constexpr (FL == 1) {
        if (a != nullptr) {
            const int hp = fuse_hp(NT, ks);
            if (hp <= 1) return go_hp<DT, FL, NT, 1>(k, ks, cz, m, n, w, A, a, lda, c, ldc, st, ep);
            if (hp == 2) return go_hp<DT, FL, NT, 2>(k, ks, cz, m, n, w, A, a, lda, c, ldc, st, ep);
            return go_hp<DT, FL, NT, 4>(k, ks, cz, m, n, w, A, a, lda, c, ldc, st, ep);
        }
    }
    return go_hp<DT, FL, NT, 0>(k, ks, cz, m, n, w, A, a, lda, c, ldc, st, ep);
}

// Split calls (gemv_slice(k, n) < k) write each slice's partial result to part ([slices][n][m]) and sum them
// into c in slice order.
template <int DT>
hipError_t gemv_dt(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m,
                          int n, float* c, int ldc, hipStream_t st, float* part, const Epi& ep) {
    const int ks = gemv_slice(k, n), ns = (k + ks - 1) / ks;
    if (ns > 1 && part == nullptr) return hipErrorInvalidValue;
    const int64_t cz = ns > 1 ? (int64_t) n * m : 0;
    float* out = ns > 1 ? part : c;
    const int ldo = ns > 1 ? m : ldc;
    const Epi eo = ns > 1 ? Epi{} : ep;   // split: the reduce applies the epilogue
    hipError_t e;
    if (flavour == 2) {
        e = go<DT, 2, 8>(w, A, nullptr, 0, k, ks, cz, m, n, out, ldo, st, eo);
    } else if (flavour == 3) {   // F1 codes from A, 8-token tiles (any n)
        e = go<DT, 1, 8>(w, A, nullptr, 0, k, ks, cz, m, n, out, ldo, st, eo);
    } else {
        switch (n) {
        case 1: e = go<DT, 1, 1>(w, A, a, lda, k, ks, cz, m, n, out, ldo, st, eo); break;
        case 2: e = go<DT, 1, 2>(w, A, a, lda, k, ks, cz, m, n, out, ldo, st, eo); break;
        case 3: e = go<DT, 1, 3>(w, A, a, lda, k, ks, cz, m, n, out, ldo, st, eo); break;
        case 4: e = go<DT, 1, 4>(w, A, a, lda, k, ks, cz, m, n, out, ldo, st, eo); break;
        case 5: e = go<DT, 1, 5>(w, A, a, lda, k, ks, cz, m, n, out, ldo, st, eo); break;
        case 6: e = go<DT, 1, 6>(w, A, a, lda, k, ks, cz, m, n, out, ldo, st, eo); break;
        case 7: e = go<DT, 1, 7>(w, A, a, lda, k, ks, cz, m, n, out, ldo, st, eo); break;
        default: return hipErrorInvalidValue;
        }
    }
    if (e != hipSuccess || ns == 1) return e;
    return launch_split_reduce(part, ns, cz, m, n, c, ldc, st, ep);
}

template <int DT>
hipError_t rows_float_dt(const WeightView& w, const float* a, int lda, int k, int r0, int rows, int n, float* c, int ldc,
                         hipStream_t st, const Epi& ep) {
    const dim3 grid((unsigned) rows, (unsigned) ((n + 7) / 8));
    rows_float_kernel<DT><<<grid, 64, 0, st>>>(w, a, lda, k, r0, n, c, ldc, ep);
    return hipGetLastError();
}

}  // namespace jamhip
