// Matrix-core prefill GEMM for Q4_K, Q5_K, Q6_K, MXFP4, Q4_0 and Q8_0 weights: C[n][m] = W[m][k] · A[n][k]^T with jam's
// F2 semantics (the n >= 8 bands of jam_kernels_q4k_avx512.c), activations from launch_gemm_prep.
//
// Arithmetic. Each 32-element block's integer dot runs on v_mfma_f32_32x32x16_f16 with integer operands
// that f16 holds exactly: the activation codes (int8) and the weight codes with their integer sub-scale
// folded in (Q4_K sc·nib <= 945, Q5_K sc·q5 <= 1953; Q6_K sc·q6 / 4 in two planes, sc·(q6 & 15) / 4 and
// sc·(q6 & 48) / 4).
// Every product and every 32-term sum is an exact f32 integer (a quarter-integer for Q6_K), so the MFMA
// returns the block's exact dot; one f32 FMA per output then applies the block's activation scale, and
// the super-block scale d is applied once per 256 elements. The super-block's other term runs on the
// matrix cores too, with the activation sums split into an f16 high part and an f16 remainder (about 22
// significant bits):
//   Q4_K  −Σ_s fl(dmin·mn_s)·fl(xs0+xs1)_s   v_mfma_f32_32x32x8_f16 per super-block, −dmin·mn split the
//                                             same way (hi·hi + hi·lo + lo·hi)   (q4k_avx512.c:76-95)
//   Q6_K  −Σ_t fl(d·sc_t)·fl(32·xs_t)         one 32x32x16 step with A' = −8·sc_t (exact), summed into
//                                             the super-block accumulator before d   (q4k_avx512.c:222-236)
// The result equals jam's up to f32 summation order (the oracle tests bound it).
//
// Operands. With the 32-row tiles of the device layout, the A fragment of lane (r, q) (row r = lane % 32,
// q = lane / 32) for K-step ks of a block is the low or high nibbles of bytes 8ks..8ks+7 of one 16-byte
// chunk, turned into f16 pairs from bytes (0,2), (1,3), (4,6), (5,7) by mask-and-or with 0x6400 (1024 + v)
// and one packed FMA with the scale (which removes the 1024). MXFP4 instead converts each byte's two nibbles
// (elements e, e + 16) with the hardware e2m1 conversion. The activation codes are stored in the matching
// order (GemmAct::b), so no shuffle is needed on either side.
//
// Tiling. A workgroup of 4 waves owns 4·RT row tiles (32 rows each, wave w the RT tiles w·RT..) x CT token
// tiles (32 tokens each) and walks k in stages of 128 elements (half a super-block). Each stage's weight
// chunks, scales, activation codes, block scales and sums are copied global -> LDS by the waves
// themselves with global_load_lds_dwordx4 (16 bytes per lane, no registers), double-buffered: stage s+1
// is in flight while stage s is computed. Workgroups that share a row block are placed on one XCD so the
// weight tile is read from HBM into that XCD's L2 once.
#include "common.h"
#include "launch.h"

#include <atomic>
#include <type_traits>

namespace jamhip {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int MMA_WAVES = 4, MMA_THREADS = 64 * MMA_WAVES;

JAMHIP_DEV void dma16(const void* g, void* lds_base) {
    // lane l's 16 bytes at g land at lds_base + 16·l (lds_base is wave-uniform)
    __builtin_amdgcn_global_load_lds(g, (lds_void*) lds_base, 16, 0, 0);
}

JAMHIP_DEV uint32_t hbits(_Float16 h) { return (uint32_t) __builtin_bit_cast(uint16_t, h); }
JAMHIP_DEV uint32_t pack2(_Float16 lo, _Float16 hi) { return hbits(lo) | (hbits(hi) << 16); }

// f16 pair (1024 + v_a, 1024 + v_b) -> mul·pair + add (one v_pk_fma_f16, exact for these operands)
JAMHIP_DEV uint32_t pkfma(uint32_t x, uint32_t mul, uint32_t add) {
    const half2v r = __builtin_elementwise_fma(__builtin_bit_cast(half2v, x), __builtin_bit_cast(half2v, mul),
                                               __builtin_bit_cast(half2v, add));
    return __builtin_bit_cast(uint32_t, r);
}

// 8 f16 of one K-step from two words: nibble/bit field `mask` of bytes (0,2), (1,3) of w0 then of w1; the
// field sits at bits 0-3 or 4-7 of each byte (sh selects which byte pair holds it after shifting).
JAMHIP_DEV half8 frag8(uint32_t w0, uint32_t w1, uint32_t mask, uint32_t mul, uint32_t add) {
    const uint32_t m = 0x64006400u;
    const uint32_t p0 = pkfma((w0 & mask) | m, mul, add), p1 = pkfma(((w0 >> 8) & mask) | m, mul, add);
    const uint32_t p2 = pkfma((w1 & mask) | m, mul, add), p3 = pkfma(((w1 >> 8) & mask) | m, mul, add);
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(half8, u32x4{p0, p1, p2, p3});
}

// Q5_K: frag8 of a nibble word pair with the 5th bit of each element merged in. Bit b (the stage's block) of
// each qh byte (h0 / h1: the qh bytes of the nibble bytes of w0 / w1) goes to bit 4 of the lo-nibble field
// (value nib + 16·bit, b even) or to bit 8 for the hi-nibble field (16·(nib + 16·bit), b odd), so
// 0x6400 | field is the f16 1024 + v5 or 1024 + 16·v5 that mul / add turn into sc·v5 (<= 1953, exact).
JAMHIP_DEV half8 frag8q5(uint32_t w0, uint32_t w1, uint32_t h0, uint32_t h1, int b, uint32_t mask, uint32_t mul,
                         uint32_t add) {
    const uint32_t m = 0x64006400u;
    const bool hi = b & 1;
    const uint32_t hm = hi ? 0x01000100u : 0x00100010u;
    // bytes (0, 2): bit b -> bit 4 (lo) / 8 (hi); bytes (1, 3) (the word shifted down by 8): bit 8 + b -> the same
    const int up = hi ? 8 - b : 4 - b, dn = hi ? b : b + 4;
    const uint32_t e0 = ((h0 << up) & hm) | m, e1 = ((h0 >> dn) & hm) | m;
    const uint32_t e2 = ((h1 << up) & hm) | m, e3 = ((h1 >> dn) & hm) | m;
    const uint32_t p0 = pkfma((w0 & mask) | e0, mul, add), p1 = pkfma(((w0 >> 8) & mask) | e1, mul, add);
    const uint32_t p2 = pkfma((w1 & mask) | e2, mul, add), p3 = pkfma(((w1 >> 8) & mask) | e3, mul, add);
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(half8, u32x4{p0, p1, p2, p3});
}

// Q4_K 6-bit scale and min of sub-block s (jam/jam-native/src/jam_kquant.h:26-33); h = the 16-byte header.
JAMHIP_DEV void q4k_scmn(const uint4 h, int s, int& sc, int& mn) {
    const uint32_t u0 = h.y, u1 = h.z, u2 = h.w;
    const int sh = 8 * (s & 3);
    if (s < 4) {
        sc = (u0 >> sh) & 63;
        mn = (u1 >> sh) & 63;
    } else {
        sc = ((u2 >> sh) & 15) | ((((u0 >> sh) >> 6) & 3) << 4);
        mn = (((u2 >> sh) >> 4) & 15) | ((((u1 >> sh) >> 6) & 3) << 4);
    }
}

JAMHIP_DEV uint32_t word(const uint4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

JAMHIP_DEV float h2f_bits(uint32_t b) { return (float) __builtin_bit_cast(_Float16, (uint16_t) (b & 0xffffu)); }

// MXFP4: 8 f16 of one K-step from one word (4 bytes) of a block's nibble bytes, by the hardware e2m1
// conversion: byte u gives the pair (e2m1(low nibble), e2m1(high nibble))·scale, elements e and e + 16 of the
// block (the activation codes are stored in the same order, GemmAct). scale = 2^(e_block − e_ref + 1) turns
// e2m1 into jam's doubled value x2 (jam_mxfp4.h:14-15: 0,1,2,3,4,6,8,12) times 2^(e_block − e_ref).
JAMHIP_DEV half8 mx_frag(uint32_t w, float scale) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 0);
    const h2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 1);
    const h2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 2);
    const h2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 3);
    return half8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// Q1_0: 8 f16 of one K-step from one byte of sign bits, bit j = element j of the run, each as 2^-14 (the
// smallest normal f16, bit 10) or 0, in the frag8 pair order (bits 0,2), (1,3), (4,6), (5,7): with x = B | B << 14
// bit j sits at j and j + 14, so x << (10 - j0) puts bits j0 and j0 + 2 at bits 10 and 26.
JAMHIP_DEV half8 q1_frag(uint32_t b) {
    const uint32_t x = b | (b << 14), m = 0x04000400u;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(half8, u32x4{(x << 10) & m, (x << 9) & m, (x << 6) & m, (x << 5) & m});
}

// NVFP4: 8 f16 of one K-step from one word (bytes 4q..4q+3 of a 16-element sub-block): byte u's two codes are
// elements u and u + 8 (jam_kernels_generic.c:128-131), converted with scale 2 (jam's integer codes kv, 0..12)
// and multiplied by the sub-block's scale d: slots 2j, 2j + 1 = elements 4q + j, 4q + j + 8 (GemmAct order 2).
JAMHIP_DEV half8 nv_frag(uint32_t w, _Float16 d) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 dd = {d, d};
    const h2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 2.0f, 0) * dd;
    const h2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 2.0f, 1) * dd;
    const h2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 2.0f, 2) * dd;
    const h2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 2.0f, 3) * dd;
    return half8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// ------------------------------------------------------------------------------------ stage layout
// Per stage buffer (bytes): A chunks [TW][NCS][32][16], header [TW][32][HB], codes [8][BN][32],
// block scales [4][BN] f32, sums hi/lo [BN][SW] f16 each.
template <int DT, int RT, int CT> struct Stage {
    static constexpr int TW = MMA_WAVES * RT, BN = 32 * CT;
    // chunks per stage (Q6_K: 4 ql, 2 qh, scales; Q5_K: 4 nibble chunks, then the super-block's 2 qh chunks;
    // Q1_0: the 128-block's 16 sign bytes)
    static constexpr int NCS = DT == Q6_K ? 7 : DT == Q8_0 ? 8 : DT == Q5_K ? 6 : DT == Q1_0 ? 1 : 4;
    static constexpr int HB = DT == Q6_K ? 2 : DT == Q1_0 ? 4 : 16;   // header bytes per row (Q6_K: d; Q1_0: 2 d)
    static constexpr int SW = DT == Q4_K || DT == Q5_K || DT == Q4_0 || DT == Q1_0 ? 8 : DT == Q6_K ? 16 : 0;   // sums per token per group
    static constexpr int A_OFF = 0;
    static constexpr int H_OFF = A_OFF + TW * NCS * 512;
    static constexpr int B_OFF = (H_OFF + TW * 32 * HB + 1023) / 1024 * 1024;
    static constexpr int DX_OFF = B_OFF + 8 * BN * 32;
    static constexpr int S_OFF = DX_OFF + 4 * BN * 4;
    static constexpr int BYTES = S_OFF + 2 * BN * SW * 2;
};

// ------------------------------------------------------------------------------------------ kernel
template <int DT, int RT, int CT>
__global__ void __launch_bounds__(MMA_THREADS, 2) kq_gemm_kernel(WeightView w, GemmAct A, int m, int n,
                                                                 float* __restrict__ c, int ldc, int nrb, int ncb,
                                                                 int64_t tiles, Groups gp, int sb_per,
                                                                 int64_t c_slice, Epi ep, int xsplit) {
    using S = Stage<DT, RT, CT>;
    constexpr int TW = S::TW, BN = S::BN, NCS = S::NCS;
    extern __shared__ __align__(1024) unsigned char smem[];
    __shared__ float q40_srow[DT == Q4_0 || DT == Q8_0 ? MMA_WAVES * RT * 32 : 1];   // 2^-s of each row

    // XCD-aware placement (tile_of_block); grouped calls take their tiles in expert-major order
    // xsplit > 0 (ungrouped): the last xsplit tiles of each XCD's run are split into two workgroups of 32
    // tokens each (sub 0 and 1), dispatched after the run's whole tiles, so that a last partial round of whole
    // tiles becomes one of half tiles
    const int total = nrb * ncb;
    int lin, sub = -1;
    if (xsplit > 0) {
        const int T8 = (total + 7) / 8, x = (int) blockIdx.x % 8, i = (int) blockIdx.x / 8, nf = T8 - xsplit;
        lin = x * T8 + (i < nf ? i : nf + (i - nf) / 2);
        if (i >= nf) sub = (i - nf) & 1;
    } else {
        lin = tile_of_block(gp.map64 != nullptr, total);
    }
    if (lin >= total) return;
    int rb = lin / ncb, cb = lin % ncb;
    if (gp.map64 != nullptr && grouped_tile(gp, lin, nrb, &rb, &cb) < 0) return;   // before any barrier
    const int64_t T0 = (int64_t) rb * TW;        // first row tile of the workgroup
    const int n0 = cb * BN + (sub > 0 ? 32 : 0); // first token slot of GemmAct

    const int lane = threadIdx.x & 63, r = lane & 31, q = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = (int) w.G, nsb = A.Kp / 256;
    // split K (sb_per > 0): slice blockIdx.y takes super-blocks [sb_per·y, sb_per·(y + 1)) and writes its
    // partial result to c + y·c_slice (summed by split_reduce_kernel); stages are half super-blocks
    const int st0 = sb_per > 0 ? 2 * sb_per * (int) blockIdx.y : 0;
    // stages that hold at least one block of k (MXFP4 pads k to whole groups: k = 2880 needs 23 of 24)
    const int nstk = min(2 * nsb, (A.K / 32 + 3) / 4);
    const int nst = sb_per > 0 ? min(nstk, st0 + 2 * sb_per) : nstk;
    int64_t r0t = w.r0 >> 5;                     // the view's first row is tile-aligned (launcher checks)
    int slot0 = 0, crow0 = 0, nvalid = n;        // token slot -> C row: crow0 + (slot - slot0), < nvalid
    if (gp.map64 != nullptr) {                   // grouped: this slot block's expert
        const int e = __builtin_amdgcn_readfirstlane(gp.map64[cb]);
        if (e < 0) return;                       // whole workgroup, before any barrier
        r0t = (w.r0 + (int64_t) e * gp.gm) >> 5;
        tiles = gp.gm / 32;
        m = gp.gm;
        slot0 = __builtin_amdgcn_readfirstlane(gp.poff64[e]);
        crow0 = __builtin_amdgcn_readfirstlane(gp.off[e]);
        nvalid = __builtin_amdgcn_readfirstlane(gp.off[e + 1]) - crow0;
        if (gp.bias != nullptr) ep.bias = gp.bias + (int64_t) e * gp.gm;
    }
    // valid tokens of this slot block all in its first 32 slots, or one half of a split tile: the second token
    // tile is neither copied nor computed nor stored
    const bool half = CT == 2 && (sub >= 0 || nvalid - (n0 - slot0) <= 32);

    // ---- global -> LDS copy of one stage. Every wave issues a fixed set of 1 KB pieces: the weight chunks
    // of its own row tile, the activation codes of K-steps 2·wave and 2·wave + 1, and one of the small
    // pieces (headers, block scales, sums). Base addresses are computed once; a stage only adds offsets.
    static_assert(TW == MMA_WAVES, "one row tile per wave");
    static_assert(BN == 64, "one 1 KB piece per K-step half");
    constexpr int NC = group_chunks(DT);
    const int64_t Tw = T0 + wave < tiles ? T0 + wave : tiles - 1;             // this wave's row tile
    const uint8_t* a_src = w.qs + (r0t + Tw) * G * (NC * CHUNK_STRIDE) + 16 * lane;
    const int a_dst = S::A_OFF + wave * NCS * 512;
    // headers: Q4_K / MXFP4 16 B per row, tiles 2·wave + q (waves 0, 1); Q6_K d, 8 rows per lane (wave 0)
    const uint8_t* h_src;
    if constexpr (DT == Q1_0) {   // 4 B per row: lanes 0..31 of wave 0 copy 16 B each, tile lane / 8
        const int64_t T = T0 + (lane >> 3) < tiles ? T0 + (lane >> 3) : tiles - 1;
        h_src = w.sc + (r0t + T) * G * 128 + (lane & 7) * 16;
    } else if constexpr (DT != Q6_K) {
        const int64_t T = T0 + 2 * (wave & 1) + q < tiles ? T0 + 2 * (wave & 1) + q : tiles - 1;
        h_src = w.sc + ((r0t + T) * G * 32 + r) * 16;
    } else {
        const int64_t T = T0 + (lane >> 2) < tiles ? T0 + (lane >> 2) : tiles - 1;
        h_src = w.sc + ((r0t + T) * G * 32 + 8 * (lane & 3)) * 2;
    }
    // GemmAct::b holds 8 f16 (16 bytes) per (K-step, half, token slot), the two halves of a K-step in planes
    const uint8_t* b_src = reinterpret_cast<const uint8_t*>(A.b) + (int64_t) (2 * wave) * A.NP * 32 + n0 * 16 + 16 * lane;
    const int64_t b_kstep = (int64_t) A.NP * 32;                                  // bytes per K-step
    const float* dx_src = A.dx + (int64_t) (lane >> 4) * A.NP + n0 + 4 * (lane & 15);
    constexpr int SWB = S::SW * 2;                                                // sum bytes per token per plane
    constexpr int SPC = S::SW > 0 ? BN * SWB / 1024 : 0;                          // 1 KB pieces per plane
    const int s_pl = SPC == 1 ? (wave >> 1) & 1 : wave >> 1, s_p = SPC == 1 ? 0 : wave & 1;
    const uint8_t* s_src = S::SW > 0 ? reinterpret_cast<const uint8_t*>(s_pl ? A.slo : A.shi) + (int64_t) n0 * SWB + s_p * 1024 + 16 * lane
                                     : nullptr;
    auto issue = [&](int st, unsigned char* buf) {
        const int g = st >> 1, h2 = st & 1;
        const uint8_t* ag = a_src + (int64_t) g * (NC * CHUNK_STRIDE);
        if constexpr (DT == Q1_0) {   // chunk h2 (512 B: lanes 0..31)
            if (lane < 32) dma16(ag + h2 * CHUNK_STRIDE, buf + a_dst);
        } else if constexpr (DT == Q5_K) {   // nibble chunks 4h2..4h2+3 as Q4_K, then the qh chunks 8, 9
#pragma unroll
            for (int p = 0; p < 2; p++) dma16(ag + (4 * h2 + 2 * p) * CHUNK_STRIDE, buf + a_dst + 2 * p * 512);
            dma16(ag + 8 * CHUNK_STRIDE, buf + a_dst + 4 * 512);
        } else if constexpr (DT != Q6_K) {   // Q4_K chunks 4h2..4h2+3 (sub-block pairs), MXFP4 / Q4_0 blocks
                                             // 4h2..4h2+3, Q8_0 chunks 8h2..8h2+7 (two per block)
#pragma unroll
            for (int p = 0; p < NCS / 2; p++)
                dma16(ag + (NCS * h2 + 2 * p) * CHUNK_STRIDE, buf + a_dst + 2 * p * 512);
        } else {   // ql chunks 4h2..4h2+3, qh chunks 8+2h2, 9+2h2, the scales chunk 12 (512 B)
#pragma unroll
            for (int p = 0; p < 2; p++) dma16(ag + (4 * h2 + 2 * p) * CHUNK_STRIDE, buf + a_dst + 2 * p * 512);
            dma16(ag + (8 + 2 * h2) * CHUNK_STRIDE, buf + a_dst + 4 * 512);
            if (lane < 32) dma16(ag + 12 * CHUNK_STRIDE, buf + a_dst + 6 * 512);
        }
        // activation codes: K-steps 8·st + 2·wave, +1; in LDS, as in GemmAct, each K-step's two 8-element halves
        // are planes [kk][half][BN tokens][16 B] so a fragment read is 512 contiguous bytes per half-wave
        // (conflict-free) and each piece copied is 1 KB contiguous
        const uint8_t* bs = b_src + (int64_t) (8 * st) * b_kstep;
        if (!half || lane < 32) {   // lane l copies token slot n0 + l
#pragma unroll
            for (int kl = 0; kl < 2; kl++)
#pragma unroll
                for (int p = 0; p < 2; p++)
                    dma16(bs + kl * b_kstep + p * (b_kstep / 2), buf + S::B_OFF + (2 * (2 * wave + kl) + p) * 1024);
        }
        if constexpr (DT == Q1_0) {
            if (wave == 0 && lane < 32) dma16(h_src + (int64_t) g * 128, buf + S::H_OFF);
        } else if constexpr (DT != Q6_K) {
            if (wave < 2) dma16(h_src + (int64_t) g * 32 * 16, buf + S::H_OFF + wave * 1024);
        } else {
            if (wave == 0 && h2 == 1 && lane < 4 * TW) dma16(h_src + (int64_t) g * 32 * 2, buf + S::H_OFF);
        }
        // block scales: 4 blocks x BN tokens (f32; lane l: block l / 16, tokens 4·(l % 16)..); a half tile
        // copies its 32 tokens only (the second half of the call's last slot block has no slots past it)
        if (wave == 2 && (!half || (lane & 15) < 8)) dma16(dx_src + (int64_t) (4 * st) * A.NP, buf + S::DX_OFF);
        // sums: Q4_K needs them at the super-block's end (odd stage), Q6_K at its start (even stage); a plane's
        // piece p holds tokens 32p.. (two pieces) or a token per lane (one piece)
        if constexpr (S::SW > 0) {
            if ((DT == Q4_0 || DT == Q1_0 || (DT == Q4_K || DT == Q5_K) == (h2 == 1)) && (SPC == 2 || wave == 1 || wave == 3) &&
                (!half || (SPC == 2 ? s_p == 0 : lane < 32)))
                dma16(s_src + (int64_t) g * A.NP * SWB, buf + S::S_OFF + s_pl * BN * SWB + s_p * 1024);
        }
    };

    // nibble masks in VGPRs: with one operand in a VGPR the mask-and-or is a single v_and_or_b32
    uint32_t vmask_lo, vmask_hi;
    asm volatile("v_mov_b32 %0, 0x000F000F" : "=v"(vmask_lo));
    asm volatile("v_mov_b32 %0, 0x00F000F0" : "=v"(vmask_hi));
    uint32_t vmask_qh, vmask_b;
    asm volatile("v_mov_b32 %0, 0x00300030" : "=v"(vmask_qh));
    asm volatile("v_mov_b32 %0, 0x00FF00FF" : "=v"(vmask_b));
    (void) vmask_qh;
    (void) vmask_b;

    floatx16 acc[RT][CT], accs[RT][CT];
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int j = 0; j < CT; j++) acc[i][j] = accs[i][j] = floatx16{};

    issue(st0, smem);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    // the stage loop for CA active token tiles: a slot block whose valid tokens all fall in its first
    // 32 (an expert's or the call's last block) runs only the first tile's fragments and products
    auto run = [&](auto ca) {
        constexpr int CA = decltype(ca)::value;
        for (int st = st0; st < nst; st++) {
            unsigned char* buf = smem + (st & 1) * S::BYTES;
            // each type issues the next stage's copy itself, after its last LDS read of this stage: the compiler
            // makes any LDS read that follows a global -> LDS copy wait for that copy
            const int h2 = st & 1;
            const unsigned char* LA = buf + S::A_OFF;
            const unsigned char* LB = buf + S::B_OFF;
            const float* LDX = reinterpret_cast<const float*>(buf + S::DX_OFF);

            if constexpr (DT == Q4_K || DT == Q5_K) {   // accs starts at zero and is cleared where it is consumed
                uint4 hdr[RT];
                uint32_t scs[RT];   // the stage's 4 sub-block scales (6-bit), one per byte
    #pragma unroll
                for (int i = 0; i < RT; i++) {
                    hdr[i] = *reinterpret_cast<const uint4*>(buf + S::H_OFF + ((wave * RT + i) * 32 + r) * 16);
                    // jam_kquant.h:26-33: sub-blocks 0-3 scale = byte & 63; 4-7 = low nibble of bytes 8-11 with
                    // the top 2 bits of bytes 0-3
                    scs[i] = h2 == 0 ? hdr[i].y & 0x3F3F3F3Fu
                                     : (hdr[i].w & 0x0F0F0F0Fu) | ((hdr[i].y >> 2) & 0x30303030u);
                }
                // every LDS read of the stage up front (the wave then works down an in-order queue)
                uint4 chs[2][RT];
                uint4 qhs[RT];   // Q5_K: the qh bytes of this lane's 16 elements (bit s = sub-block s), shifted so
                                 // that bit bl is the stage's block bl
                half8 bfs[4][CT][2];
                float dxs[4][CT];
    #pragma unroll
                for (int gpl = 0; gpl < 2; gpl++)
    #pragma unroll
                    for (int i = 0; i < RT; i++)
                        chs[gpl][i] = *reinterpret_cast<const uint4*>(LA + ((wave * RT + i) * NCS + 2 * gpl + q) * 512 + 16 * r);
                if constexpr (DT == Q5_K) {
    #pragma unroll
                    for (int i = 0; i < RT; i++) {
                        const uint4 h = *reinterpret_cast<const uint4*>(LA + ((wave * RT + i) * NCS + 4 + q) * 512 + 16 * r);
                        const int sh = 4 * h2;
                        qhs[i] = make_uint4(h.x >> sh, h.y >> sh, h.z >> sh, h.w >> sh);
                    }
                }
    #pragma unroll
                for (int bl = 0; bl < 4; bl++)
    #pragma unroll
                    for (int j = 0; j < CA; j++) {
    #pragma unroll
                        for (int ks = 0; ks < 2; ks++)
                            bfs[bl][j][ks] = *reinterpret_cast<const half8*>(LB + ((2 * bl + ks) * 2 + q) * BN * 16 + (32 * j + r) * 16);
                        dxs[bl][j] = LDX[bl * BN + 32 * j + r];
                    }
                // super-block end (odd stage): d of the 16 output rows this lane holds, and the sums' fragments
                float dds[RT][16];
                half4 shi[CT], slo[CT];
                if (h2 == 1) {
    #pragma unroll
                    for (int i = 0; i < RT; i++) {
                        const unsigned char* H = buf + S::H_OFF + (wave * RT + i) * 32 * 16;
    #pragma unroll
                        for (int e = 0; e < 16; e++)
                            dds[i][e] = h2f_bits(*reinterpret_cast<const uint16_t*>(H + (8 * (e >> 2) + 4 * q + (e & 3)) * 16));
                    }
    #pragma unroll
                    for (int j = 0; j < CA; j++) {
                        const unsigned char* SP = buf + S::S_OFF + (32 * j + r) * 16 + 8 * q;
                        shi[j] = *reinterpret_cast<const half4*>(SP);
                        slo[j] = *reinterpret_cast<const half4*>(SP + BN * 16);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead of the compute
                // this stage's LDS reads are all issued: start copying the next stage into the other buffer
                if (st + 1 < nst) issue(st + 1, smem + ((st + 1) & 1) * S::BYTES);
                // Software pipeline over the stage's 4 blocks: block bl's products go out on the matrix cores into
                // D[bl & 1] before block bl-1's scale FMAs, which then run while the matrix cores work.
                floatx16 Dp[2][RT][CT];
    #pragma unroll
                for (int bl = 0; bl < 5; bl++) {
                    if (bl < 4) {
                        const uint4* ch = chs[bl >> 1];
                        const int sub = bl & 1;
                        half8 af[RT][2];
    #pragma unroll
                        for (int i = 0; i < RT; i++) {
                            // lo nibble: (1024 + v)·sc − 1024·sc; hi nibble (bits 4-7): (1024 + 16v)·sc/16 − 64·sc
                            const uint32_t sc = (scs[i] >> (8 * bl)) & 0xffu;
                            const uint32_t dup = sc | (sc << 16) | 0x64006400u;   // f16 pair (1024 + sc, 1024 + sc)
                            const half2v one = __builtin_bit_cast(half2v, dup) - __builtin_bit_cast(half2v, 0x64006400u);
                            const half2v mulv = sub ? one * (_Float16) 0.0625f : one;
                            const half2v addv = one * (sub ? (_Float16) -64.0f : (_Float16) -1024.0f);
                            const uint32_t mul = __builtin_bit_cast(uint32_t, mulv), add = __builtin_bit_cast(uint32_t, addv);
                            const uint32_t mask = sub ? vmask_hi : vmask_lo;
                            if constexpr (DT == Q5_K) {   // the 5th bit (qh bit bl of each byte) at bit 4 (lo) or 8 (hi)
                                af[i][0] = frag8q5(ch[i].x, ch[i].y, qhs[i].x, qhs[i].y, bl, mask, mul, add);
                                af[i][1] = frag8q5(ch[i].z, ch[i].w, qhs[i].z, qhs[i].w, bl, mask, mul, add);
                            } else {
                                af[i][0] = frag8(ch[i].x, ch[i].y, mask, mul, add);
                                af[i][1] = frag8(ch[i].z, ch[i].w, mask, mul, add);
                            }
                        }
    #pragma unroll
                        for (int i = 0; i < RT; i++)
    #pragma unroll
                            for (int j = 0; j < CA; j++) {
                                floatx16 D = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i][0], bfs[bl][j][0], floatx16{}, 0, 0, 0);
                                Dp[bl & 1][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i][1], bfs[bl][j][1], D, 0, 0, 0);
                            }
                    }
                    if (bl > 0) {
                        const int pb = bl - 1;
    #pragma unroll
                        for (int i = 0; i < RT; i++)
    #pragma unroll
                            for (int j = 0; j < CA; j++)
    #pragma unroll
                                for (int e = 0; e < 16; e++)
                                    accs[i][j][e] = fmaf(Dp[pb & 1][i][j][e], dxs[pb][j], accs[i][j][e]);
                    }
                }
                if (h2 == 1) {   // super-block end: d, then the mins on the matrix cores
    #pragma unroll
                    for (int i = 0; i < RT; i++) {
    #pragma unroll
                        for (int j = 0; j < CA; j++) {
    #pragma unroll
                            for (int e = 0; e < 16; e++) acc[i][j][e] = fmaf(dds[i][e], accs[i][j][e], acc[i][j][e]);
                            accs[i][j] = floatx16{};
                        }
                        // A' = −dmin·mn_s for sub-blocks 4q..4q+3 of row r, split hi + lo
                        const float dmin = h2f_bits(hdr[i].x >> 16);
                        half4 ahi, alo;
    #pragma unroll
                        for (int e = 0; e < 4; e++) {
                            int sc, mn;
                            q4k_scmn(hdr[i], 4 * q + e, sc, mn);
                            const F16Pair p = split_f16(-(dmin * (float) mn));
                            ahi[e] = p.hi;
                            alo[e] = p.lo;
                        }
    #pragma unroll
                        for (int j = 0; j < CA; j++) {
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x8f16(ahi, shi[j], acc[i][j], 0, 0, 0);
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x8f16(ahi, slo[j], acc[i][j], 0, 0, 0);
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x8f16(alo, shi[j], acc[i][j], 0, 0, 0);
                        }
                    }
                }
            } else if constexpr (DT == Q4_0 || DT == Q8_0) {   // group of 8 blocks; stage h2 = blocks 4h2..4h2+3
                // The weight operand is d'·code with d' = d·2^s_r (s_r per row and group: the row's largest block
                // scale lands in [2^10, 2^11) for Q4_0's nibbles, [2^7, 2^8) for Q8_0's int8, so |d'·code| < 2^15),
                // split exactly into f16 hi + lo (d'·code has at most 15 significant bits for Q4_0, 19 for Q8_0). Each block's dot then runs as two MFMAs per K-step,
                // one FMA per output applies dx, and at the group end (Q4_0) −8·Σ_b d'_b·xs_b joins on the matrix
                // cores before the 2^-s_r of each row.
                const bool gend = h2 == 1 || st == nstk - 1;   // the last group may end after its first half
                uint4 hdr[RT], chs[RT][4];
                half8 bfs[4][CT][2];
                float dxs[4][CT];
                half4 shi[CT], slo[CT];
    #pragma unroll
                for (int i = 0; i < RT; i++) {
                    hdr[i] = *reinterpret_cast<const uint4*>(buf + S::H_OFF + ((wave * RT + i) * 32 + r) * 16);
    #pragma unroll
                    for (int bl = 0; bl < 4; bl++) {   // Q4_0: block bl's chunk; Q8_0: its half q (elements 16q..)
                        const int cl = DT == Q8_0 ? 2 * bl + q : bl;
                        chs[i][bl] = *reinterpret_cast<const uint4*>(LA + ((wave * RT + i) * NCS + cl) * 512 + 16 * r);
                    }
                }
    #pragma unroll
                for (int bl = 0; bl < 4; bl++)
    #pragma unroll
                    for (int j = 0; j < CA; j++) {
    #pragma unroll
                        for (int ks = 0; ks < 2; ks++)
                            bfs[bl][j][ks] = *reinterpret_cast<const half8*>(LB + ((2 * bl + ks) * 2 + q) * BN * 16 + (32 * j + r) * 16);
                        dxs[bl][j] = LDX[bl * BN + 32 * j + r];
                    }
                if (DT == Q4_0 && gend) {
    #pragma unroll
                    for (int j = 0; j < CA; j++) {
                        const unsigned char* SP = buf + S::S_OFF + (32 * j + r) * 16 + 8 * q;
                        shi[j] = *reinterpret_cast<const half4*>(SP);
                        slo[j] = *reinterpret_cast<const half4*>(SP + BN * 16);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                if (st + 1 < nst) issue(st + 1, smem + ((st + 1) & 1) * S::BYTES);
                // s_r of row r from its 8 block scales (f16 exponent fields); 2^-s_r goes to LDS at the group's
                // first stage for the lanes that hold row r's outputs
                int sr[RT];
                // d'_b = d_b·2^s_r of block b of the group, exact in f32 and (above 2^-14) in f16
                auto dq = [&](int i, int b) { return ldexpf(h2f_bits(word(hdr[i], b >> 1) >> (16 * (b & 1))), sr[i]); };
    #pragma unroll
                for (int i = 0; i < RT; i++) {
                    const uint32_t e01 = max(hdr[i].x & 0x7C00u, (hdr[i].x >> 16) & 0x7C00u);
                    const uint32_t e23 = max(hdr[i].y & 0x7C00u, (hdr[i].y >> 16) & 0x7C00u);
                    const uint32_t e45 = max(hdr[i].z & 0x7C00u, (hdr[i].z >> 16) & 0x7C00u);
                    const uint32_t e67 = max(hdr[i].w & 0x7C00u, (hdr[i].w >> 16) & 0x7C00u);
                    const int emax = (int) (max(max(e01, e23), max(e45, e67)) >> 10);   // biased exponent, 0..31
                    sr[i] = (DT == Q8_0 ? 22 : 25) - emax;   // |d'·code| < 2^15 (f16 range)
                    if (h2 == 0 && q == 0) q40_srow[(wave * RT + i) * 32 + r] = ldexpf(1.0f, -sr[i]);
                }
                floatx16 Dp[2][RT][CT];
    #pragma unroll
                for (int bl = 0; bl < 5; bl++) {
                    if (bl < 4) {
                        half8 ah[RT][2], al[RT][2];
    #pragma unroll
                        for (int i = 0; i < RT; i++) {
                            const uint4 ch = chs[i][bl];
                            const float df = dq(i, 4 * h2 + bl);
                            const _Float16 dh = (_Float16) df;
                            const half2v d2 = {dh, dh};
                            half8 v0, v1;   // the codes as exact f16
                            if constexpr (DT == Q4_0) {   // lane half q takes the low (elements 0-15) or high nibbles
                                const uint32_t mask = q ? vmask_hi : vmask_lo;
                                const uint32_t mul = q ? 0x2C002C00u : 0x3C003C00u;   // f16 pairs (1/16, 1/16) or (1, 1)
                                const uint32_t add = q ? 0xD400D400u : 0xE400E400u;   // (-64, -64) or (-1024, -1024)
                                v0 = frag8(ch.x, ch.y, mask, mul, add);
                                v1 = frag8(ch.z, ch.w, mask, mul, add);
                            } else {   // int8 ^ 0x80 = q + 128, as the f16 1024 + q + 128, minus 1152
                                v0 = frag8(ch.x ^ 0x80808080u, ch.y ^ 0x80808080u, vmask_b, 0x3C003C00u, 0xE480E480u);
                                v1 = frag8(ch.z ^ 0x80808080u, ch.w ^ 0x80808080u, vmask_b, 0x3C003C00u, 0xE480E480u);
                            }
    #pragma unroll
                            for (int e = 0; e < 8; e += 2) {
                                const half2v a0 = {v0[e], v0[e + 1]}, a1 = {v1[e], v1[e + 1]};
                                const half2v h0 = a0 * d2, h1 = a1 * d2;
                                const half2v l0 = __builtin_elementwise_fma(a0, d2, -h0), l1 = __builtin_elementwise_fma(a1, d2, -h1);
                                ah[i][0][e] = h0[0], ah[i][0][e + 1] = h0[1], ah[i][1][e] = h1[0], ah[i][1][e + 1] = h1[1];
                                al[i][0][e] = l0[0], al[i][0][e + 1] = l0[1], al[i][1][e] = l1[0], al[i][1][e + 1] = l1[1];
                            }
                        }
    #pragma unroll
                        for (int i = 0; i < RT; i++)
    #pragma unroll
                            for (int j = 0; j < CA; j++) {
                                floatx16 D = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][0], bfs[bl][j][0], floatx16{}, 0, 0, 0);
                                D = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][0], bfs[bl][j][0], D, 0, 0, 0);
                                D = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][1], bfs[bl][j][1], D, 0, 0, 0);
                                Dp[bl & 1][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][1], bfs[bl][j][1], D, 0, 0, 0);
                            }
                    }
                    if (bl > 0) {
                        const int pb = bl - 1;
    #pragma unroll
                        for (int i = 0; i < RT; i++)
    #pragma unroll
                            for (int j = 0; j < CA; j++)
    #pragma unroll
                                for (int e = 0; e < 16; e++)
                                    accs[i][j][e] = fmaf(Dp[pb & 1][i][j][e], dxs[pb][j], accs[i][j][e]);
                    }
                }
                if (gend) {   // group end: (Q4_0) accs −= 8·Σ_b d'_b·xs_b (hi + lo of the sums), then acc += 2^-s · accs
                    if (h2 == 0) __syncthreads();   // 2^-s of this stage's group was written above
    #pragma unroll
                    for (int i = 0; i < RT; i++) {
                        if constexpr (DT == Q4_0) {
                            half4 a8;   // −8·d'_b for blocks 4q..4q+3 of row r (exact: d'_b < 2^11)
    #pragma unroll
                            for (int e = 0; e < 4; e++) a8[e] = (_Float16) (-8.0f * dq(i, 4 * q + e));
    #pragma unroll
                            for (int j = 0; j < CA; j++) {
                                accs[i][j] = __builtin_amdgcn_mfma_f32_32x32x8f16(a8, shi[j], accs[i][j], 0, 0, 0);
                                accs[i][j] = __builtin_amdgcn_mfma_f32_32x32x8f16(a8, slo[j], accs[i][j], 0, 0, 0);
                            }
                        }
                        const float* SR = q40_srow + (wave * RT + i) * 32;
    #pragma unroll
                        for (int j = 0; j < CA; j++) {
    #pragma unroll
                            for (int e = 0; e < 16; e++)
                                acc[i][j][e] = fmaf(SR[8 * (e >> 2) + 4 * q + (e & 3)], accs[i][j][e], acc[i][j][e]);
                            accs[i][j] = floatx16{};
                        }
                    }
                }
            } else if constexpr (DT == MXFP4) {   // group of 8 blocks; stage h2 = blocks 4h2..4h2+3
                // every LDS read of the stage up front, then the next stage's copy, then the compute
                uint4 hdr[RT];
                uint2 chs[RT][4];   // lane half q: bytes 8q..8q+7 of each block (K-step 0 word 2q, K-step 1 word 2q + 1)
                half8 bfs[4][CT][2];
                float dxs[4][CT];
                float sg[RT][16];
    #pragma unroll
                for (int i = 0; i < RT; i++) {
                    hdr[i] = *reinterpret_cast<const uint4*>(buf + S::H_OFF + ((wave * RT + i) * 32 + r) * 16);
    #pragma unroll
                    for (int bl = 0; bl < 4; bl++)
                        chs[i][bl] = *reinterpret_cast<const uint2*>(LA + ((wave * RT + i) * NCS + bl) * 512 + 16 * r + 8 * q);
                }
    #pragma unroll
                for (int bl = 0; bl < 4; bl++)
    #pragma unroll
                    for (int j = 0; j < CA; j++) {
    #pragma unroll
                        for (int ks = 0; ks < 2; ks++)
                            bfs[bl][j][ks] = *reinterpret_cast<const half8*>(LB + ((2 * bl + ks) * 2 + q) * BN * 16 + (32 * j + r) * 16);
                        dxs[bl][j] = LDX[bl * BN + 32 * j + r];
                    }
                const bool gend = h2 == 1 || st == nstk - 1;   // the last group may end after its first half
                if (gend) {   // group end: 2^(e_ref - 128) of the 16 output rows this lane holds (header bytes 12..15)
    #pragma unroll
                    for (int i = 0; i < RT; i++) {
                        const unsigned char* H = buf + S::H_OFF + (wave * RT + i) * 32 * 16 + 12;
    #pragma unroll
                        for (int e = 0; e < 16; e++)
                            sg[i][e] = *reinterpret_cast<const float*>(H + (8 * (e >> 2) + 4 * q + (e & 3)) * 16);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                if (st + 1 < nst) issue(st + 1, smem + ((st + 1) & 1) * S::BYTES);
                // software pipeline: block bl's products go out before block bl-1's scale FMAs
                floatx16 Dp[2][RT][CT];
    #pragma unroll
                for (int bl = 0; bl < 5; bl++) {
                    if (bl < 4) {
                        half8 af[RT][2];
    #pragma unroll
                        for (int i = 0; i < RT; i++) {
                            const uint2 ch = chs[i][bl];
                            const int eb = (int) (((h2 ? hdr[i].y : hdr[i].x) >> (8 * bl)) & 0xffu);
                            const int er = (int) (hdr[i].z & 0xffu);
                            // f32 bits of 2^(eb - er + 1): (eb - er)·2^23 + bits(2.0); a scale below 2^-126 (only a
                            // zero-code block stored as e = 0 under a reference >= 128) comes out <= 0 and becomes 0
                            const int sb = (eb - er) * (1 << 23) + 0x40000000;
                            const float scale = __builtin_bit_cast(float, max(sb, 0));
                            af[i][0] = mx_frag(ch.x, scale);
                            af[i][1] = mx_frag(ch.y, scale);
                        }
    #pragma unroll
                        for (int i = 0; i < RT; i++)
    #pragma unroll
                            for (int j = 0; j < CA; j++) {
                                floatx16 D = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i][0], bfs[bl][j][0], floatx16{}, 0, 0, 0);
                                Dp[bl & 1][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i][1], bfs[bl][j][1], D, 0, 0, 0);
                            }
                    }
                    if (bl > 0) {
                        const int pb = bl - 1;
    #pragma unroll
                        for (int i = 0; i < RT; i++)
    #pragma unroll
                            for (int j = 0; j < CA; j++)
    #pragma unroll
                                for (int e = 0; e < 16; e++)
                                    accs[i][j][e] = fmaf(Dp[pb & 1][i][j][e], dxs[pb][j], accs[i][j][e]);
                    }
                }
                if (gend) {   // group end: acc += 2^(e_ref - 128) · accs
    #pragma unroll
                    for (int i = 0; i < RT; i++)
    #pragma unroll
                        for (int j = 0; j < CA; j++) {
    #pragma unroll
                            for (int e = 0; e < 16; e++) acc[i][j][e] = fmaf(sg[i][e], accs[i][j][e], acc[i][j][e]);
                            accs[i][j] = floatx16{};
                        }
                }
            } else if constexpr (DT == Q1_0) {
                // stage h2 = 128-block h2 of the group (one chunk of sign bits, d = the row's fp16 d[h2]). jam's F2
                // decomposition per 32-block (q1_0_block16, jam_kernels_q4k_avx512.c:580-598): fl(d·fl(2·dx))·
                // Σbit·xq − d·fl(xs0 + xs1). The bits go to the matrix cores as the f16 2^-14 (normal) or 0, so a
                // block's MFMA result is 2^-14·Σbit·xq exactly; one FMA per output applies 2·dx into accs,
                // 2^14·d comes in once per stage, and the −d·sums term runs on the matrix cores at the
                // group's end (A' = −d of each block's 128-block against the sums' hi and lo parts).
                const bool gend = h2 == 1 || st == nstk - 1;
                uint32_t dh[RT];   // row r's two fp16 d
                uint4 chs[RT];
                half8 bfs[4][CT][2];
                float dxs[4][CT];
                half4 shi[CT], slo[CT];
    #pragma unroll
                for (int i = 0; i < RT; i++) {
                    dh[i] = *reinterpret_cast<const uint32_t*>(buf + S::H_OFF + (wave * RT + i) * 128 + r * 4);
                    chs[i] = *reinterpret_cast<const uint4*>(LA + (wave * RT + i) * NCS * 512 + 16 * r);
                }
    #pragma unroll
                for (int bl = 0; bl < 4; bl++)
    #pragma unroll
                    for (int j = 0; j < CA; j++) {
    #pragma unroll
                        for (int ks = 0; ks < 2; ks++)
                            bfs[bl][j][ks] = *reinterpret_cast<const half8*>(LB + ((2 * bl + ks) * 2 + q) * BN * 16 + (32 * j + r) * 16);
                        dxs[bl][j] = LDX[bl * BN + 32 * j + r] * 2.0f;   // 2·dx, exact
                    }
                float dds[RT][16];   // 2^14·d[h2] of the 16 output rows this lane holds (exact, finite)
    #pragma unroll
                for (int i = 0; i < RT; i++) {
                    const unsigned char* H = buf + S::H_OFF + (wave * RT + i) * 128 + 2 * h2;
    #pragma unroll
                    for (int e = 0; e < 16; e++)
                        dds[i][e] = 16384.0f * h2f_bits(*reinterpret_cast<const uint16_t*>(H + (8 * (e >> 2) + 4 * q + (e & 3)) * 4));
                }
                if (gend) {
    #pragma unroll
                    for (int j = 0; j < CA; j++) {
                        const unsigned char* SP = buf + S::S_OFF + (32 * j + r) * 16 + 8 * q;
                        shi[j] = *reinterpret_cast<const half4*>(SP);
                        slo[j] = *reinterpret_cast<const half4*>(SP + BN * 16);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                if (st + 1 < nst) issue(st + 1, smem + ((st + 1) & 1) * S::BYTES);
                floatx16 Dp[2][RT][CT];
    #pragma unroll
                for (int bl = 0; bl < 5; bl++) {
                    if (bl < 4) {
                        half8 af[RT][2];
    #pragma unroll
                        for (int i = 0; i < RT; i++)
    #pragma unroll
                            for (int ks = 0; ks < 2; ks++)   // elements 16q + 8ks + j: byte 4bl + 2q + ks, bit j
                                af[i][ks] = q1_frag((word(chs[i], bl) >> (8 * (2 * q + ks))) & 0xffu);
    #pragma unroll
                        for (int i = 0; i < RT; i++)
    #pragma unroll
                            for (int j = 0; j < CA; j++) {
                                floatx16 D = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i][0], bfs[bl][j][0], floatx16{}, 0, 0, 0);
                                Dp[bl & 1][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i][1], bfs[bl][j][1], D, 0, 0, 0);
                            }
                    }
                    if (bl > 0) {
                        const int pb = bl - 1;
    #pragma unroll
                        for (int i = 0; i < RT; i++)
    #pragma unroll
                            for (int j = 0; j < CA; j++)
    #pragma unroll
                                for (int e = 0; e < 16; e++)
                                    accs[i][j][e] = fmaf(Dp[pb & 1][i][j][e], dxs[pb][j], accs[i][j][e]);
                    }
                }
    #pragma unroll
                for (int i = 0; i < RT; i++) {   // stage end: acc += d·accs; group end: acc −= Σ_b d_b·sums_b
    #pragma unroll
                    for (int j = 0; j < CA; j++) {
    #pragma unroll
                        for (int e = 0; e < 16; e++) acc[i][j][e] = fmaf(dds[i][e], accs[i][j][e], acc[i][j][e]);
                        accs[i][j] = floatx16{};
                    }
                    if (gend) {
                        const _Float16 nd = -__builtin_bit_cast(_Float16, (uint16_t) (dh[i] >> (16 * q)));
                        const half4 a8 = {nd, nd, nd, nd};   // blocks 4q..4q+3 of the group: 128-block q
    #pragma unroll
                        for (int j = 0; j < CA; j++) {
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x8f16(a8, shi[j], acc[i][j], 0, 0, 0);
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x8f16(a8, slo[j], acc[i][j], 0, 0, 0);
                        }
                    }
                }
            } else if constexpr (DT == NVFP4) {
                // stage h2 = 64-blocks 2h2, 2h2 + 1; its chunk bl holds 16-element sub-blocks S = 8h2 + 2bl + ks
                // (ks = 0, 1: the 32-block bl's two K-steps), 8 bytes each, byte u = elements u and u + 8. Lane half q
                // takes bytes 4q..4q+3 of a sub-block: the hardware e2m1 conversion (scale 2: jam's codes kv) gives
                // the pairs (u, u + 8), and one packed multiply applies the sub-block's UE4M3 scale d (kv·d has at
                // most 6 significant bits and lies in [2^-10, 5760]: exact in f16). jam's F1 activation scale of the
                // 32-block then comes in with one FMA per output, straight into acc (no group scale).
                uint4 hdr[RT], chs[RT][4];
                half8 bfs[4][CT][2];
                float dxs[4][CT];
    #pragma unroll
                for (int i = 0; i < RT; i++) {
                    hdr[i] = *reinterpret_cast<const uint4*>(buf + S::H_OFF + ((wave * RT + i) * 32 + r) * 16);
    #pragma unroll
                    for (int bl = 0; bl < 4; bl++)
                        chs[i][bl] = *reinterpret_cast<const uint4*>(LA + ((wave * RT + i) * NCS + bl) * 512 + 16 * r);
                }
    #pragma unroll
                for (int bl = 0; bl < 4; bl++)
    #pragma unroll
                    for (int j = 0; j < CA; j++) {
    #pragma unroll
                        for (int ks = 0; ks < 2; ks++)
                            bfs[bl][j][ks] = *reinterpret_cast<const half8*>(LB + ((2 * bl + ks) * 2 + q) * BN * 16 + (32 * j + r) * 16);
                        dxs[bl][j] = LDX[bl * BN + 32 * j + r];
                    }
                __builtin_amdgcn_sched_barrier(0);
                if (st + 1 < nst) issue(st + 1, smem + ((st + 1) & 1) * S::BYTES);
                floatx16 Dp[2][RT][CT];
    #pragma unroll
                for (int bl = 0; bl < 5; bl++) {
                    if (bl < 4) {
                        half8 af[RT][2];
    #pragma unroll
                        for (int i = 0; i < RT; i++) {
                            const uint4 ch = chs[i][bl];
    #pragma unroll
                            for (int ks = 0; ks < 2; ks++) {
                                const int sb = 8 * h2 + 2 * bl + ks;   // the sub-block's scale byte in the header
                                const uint32_t sbyte = (word(hdr[i], sb >> 2) >> (8 * (sb & 3))) & 0xffu;
                                const _Float16 d = (_Float16) ue4m3(sbyte);
                                af[i][ks] = nv_frag(ks ? (q ? ch.w : ch.z) : (q ? ch.y : ch.x), d);
                            }
                        }
    #pragma unroll
                        for (int i = 0; i < RT; i++)
    #pragma unroll
                            for (int j = 0; j < CA; j++) {
                                floatx16 D = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i][0], bfs[bl][j][0], floatx16{}, 0, 0, 0);
                                Dp[bl & 1][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i][1], bfs[bl][j][1], D, 0, 0, 0);
                            }
                    }
                    if (bl > 0) {
                        const int pb = bl - 1;
    #pragma unroll
                        for (int i = 0; i < RT; i++)
    #pragma unroll
                            for (int j = 0; j < CA; j++)
    #pragma unroll
                                for (int e = 0; e < 16; e++)
                                    acc[i][j][e] = fmaf(Dp[pb & 1][i][j][e], dxs[pb][j], acc[i][j][e]);
                    }
                }
            } else {   // Q6_K: stage h2 = half h of the super-block, blocks j = 0..3 (elements 128h + 32j + l)
                // every LDS read of the stage up front, then the next stage's copy, then the compute
                uint4 ql[RT][2], qh[RT];
                int scl[RT][4];
                uint2 sco[RT];             // h2 = 0: the 8 scales of row r's 16-groups 8q..8q+7 (offset term)
                half8 bhi[CT], blo[CT];    // h2 = 0: the sums' fragments
                half8 bfs[4][CT][2];
                float dxs[4][CT];
    #pragma unroll
                for (int i = 0; i < RT; i++) {
                    const unsigned char* T = LA + (wave * RT + i) * NCS * 512 + 16 * r;
                    ql[i][0] = *reinterpret_cast<const uint4*>(T + (0 + q) * 512);
                    ql[i][1] = *reinterpret_cast<const uint4*>(T + (2 + q) * 512);
                    qh[i] = *reinterpret_cast<const uint4*>(T + (4 + q) * 512);
                    // the row's 16 int8 scales in one 16-byte read (the 32 rows' reads are 512 contiguous bytes;
                    // byte reads at a 16-byte stride would conflict 4 ways), then the bytes this stage needs:
                    // scale 8h2 + 2jb + q (word 2h2 + jb/2, byte 2(jb % 2) + q) and, at h2 = 0, words 2q, 2q + 1
                    const uint4 sv = *reinterpret_cast<const uint4*>(T + 6 * 512);
    #pragma unroll
                    for (int jb = 0; jb < 4; jb++) {
                        const uint32_t wv = jb < 2 ? (h2 ? sv.z : sv.x) : (h2 ? sv.w : sv.y);
                        scl[i][jb] = __builtin_amdgcn_sbfe(wv, 8 * (2 * (jb & 1) + q), 8);
                    }
                    sco[i] = q ? make_uint2(sv.z, sv.w) : make_uint2(sv.x, sv.y);
                }
                if (h2 == 0) {
    #pragma unroll
                    for (int j = 0; j < CA; j++) {
                        const unsigned char* SP = buf + S::S_OFF + (32 * j + r) * 32 + 16 * q;
                        bhi[j] = *reinterpret_cast<const half8*>(SP);
                        blo[j] = *reinterpret_cast<const half8*>(SP + BN * 32);
                    }
                }
    #pragma unroll
                for (int jb = 0; jb < 4; jb++)
    #pragma unroll
                    for (int j = 0; j < CA; j++) {
    #pragma unroll
                        for (int ks = 0; ks < 2; ks++)
                            bfs[jb][j][ks] = *reinterpret_cast<const half8*>(LB + ((2 * jb + ks) * 2 + q) * BN * 16 + (32 * j + r) * 16);
                        dxs[jb][j] = LDX[jb * BN + 32 * j + r];
                    }
                if (h2 == 0) {
                    // accs = −8·Σ_t sc_t·xs_t (the −32 offset, in units of 1/4), one 32x32x16 step hi + lo
    #pragma unroll
                    for (int i = 0; i < RT; i++) {
                        half8 ao;
    #pragma unroll
                        for (int e = 0; e < 8; e++)
                            ao[e] = (_Float16) (-8.0f * (float) (int8_t) (((e < 4 ? sco[i].x : sco[i].y) >> (8 * (e & 3))) & 0xffu));
    #pragma unroll
                        for (int j = 0; j < CA; j++) {
                            accs[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ao, bhi[j], floatx16{}, 0, 0, 0);
                            accs[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ao, blo[j], accs[i][j], 0, 0, 0);
                        }
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                if (st + 1 < nst) issue(st + 1, smem + ((st + 1) & 1) * S::BYTES);
    #pragma unroll
                for (int jb = 0; jb < 4; jb++) {
                    half8 a1[RT][2], a2[RT][2];
    #pragma unroll
                    for (int i = 0; i < RT; i++) {
                        const float sc = (float) scl[i][jb];
                        // ql nibble: lo (1024 + v)·sc/4 − 256·sc; hi (1024 + 16v)·sc/64 − 16·sc
                        const bool hi = jb >= 2;
                        const float fm = hi ? sc * 0.015625f : sc * 0.25f, fa = hi ? -16.0f * sc : -256.0f * sc;
                        const uint32_t mul1 = pack2((_Float16) fm, (_Float16) fm), add1 = pack2((_Float16) fa, (_Float16) fa);
                        const uint4 L = ql[i][jb & 1];
                        const uint32_t m1 = hi ? vmask_hi : vmask_lo;
                        a1[i][0] = frag8(L.x, L.y, m1, mul1, add1);
                        a1[i][1] = frag8(L.z, L.w, m1, mul1, add1);
                        // qh bits 2jb..2jb+1 moved to bits 4-5: (1024 + 16v)·sc/4 − 256·sc = 4·sc·v = sc·(16v)/4
                        const float fm2 = sc * 0.25f, fa2 = -256.0f * sc;
                        const uint32_t mul2 = pack2((_Float16) fm2, (_Float16) fm2), add2 = pack2((_Float16) fa2, (_Float16) fa2);
                        const uint4 Q = qh[i];
                        const int sh = 2 * jb;   // bits 2jb..2jb+1 -> 4..5
                        auto mv = [&](uint32_t x) { return sh <= 4 ? x << (4 - sh) : x >> (sh - 4); };
                        a2[i][0] = frag8(mv(Q.x), mv(Q.y), vmask_qh, mul2, add2);
                        a2[i][1] = frag8(mv(Q.z), mv(Q.w), vmask_qh, mul2, add2);
                    }
    #pragma unroll
                    for (int i = 0; i < RT; i++)
    #pragma unroll
                        for (int j = 0; j < CA; j++) {
                            floatx16 D = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1[i][0], bfs[jb][j][0], floatx16{}, 0, 0, 0);
                            D = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1[i][1], bfs[jb][j][1], D, 0, 0, 0);
                            D = __builtin_amdgcn_mfma_f32_32x32x16_f16(a2[i][0], bfs[jb][j][0], D, 0, 0, 0);
                            D = __builtin_amdgcn_mfma_f32_32x32x16_f16(a2[i][1], bfs[jb][j][1], D, 0, 0, 0);
    #pragma unroll
                            for (int e = 0; e < 16; e++) accs[i][j][e] = fmaf(D[e], dxs[jb][j], accs[i][j][e]);
                        }
                }
                if (h2 == 1) {   // super-block end: acc += 4d · accs (d read here: the next copy has had the stage)
    #pragma unroll
                    for (int i = 0; i < RT; i++) {
                        const unsigned char* H = buf + S::H_OFF + (wave * RT + i) * 32 * 2;
                        float dd[16];
    #pragma unroll
                        for (int e = 0; e < 16; e++) {
                            const int row = 8 * (e >> 2) + 4 * q + (e & 3);
                            dd[e] = 4.0f * h2f_bits(*reinterpret_cast<const uint16_t*>(H + row * 2));
                        }
    #pragma unroll
                        for (int j = 0; j < CA; j++)
    #pragma unroll
                            for (int e = 0; e < 16; e++) acc[i][j][e] = fmaf(dd[e], accs[i][j][e], acc[i][j][e]);
                    }
                }
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        }
    };
    if (CT == 2 && half)
        run(std::integral_constant<int, 1>{});
    else
        run(std::integral_constant<int, CT>{});

    // epilogue: lane holds token n0 + 32j + r, rows 8·(e/4) + 4q + e%4 of each tile; scale back by 2^e_t
#pragma unroll
    for (int j = 0; j < CT; j++) {
        const int t = n0 + 32 * j + r, tl = t - slot0;
        if (tl >= nvalid || (half && j > 0)) continue;
        const float sc = A.es[t];
        float* ct = c + (int64_t) blockIdx.y * c_slice + (int64_t) (crow0 + tl) * ldc;
#pragma unroll
        for (int i = 0; i < RT; i++)   // split K: the reduce applies the epilogue
            store_column(ct, (T0 + wave * RT + i) * 32 + 4 * q, m, acc[i][j], sc, ep, sb_per > 0);
    }
}

// Deterministic sum of the split-K partials: c[t][row] = Σ_s part[s][t][row] in slice order.
__global__ void __launch_bounds__(256) split_reduce_kernel(const float* __restrict__ part, int ns, int64_t slice,
                                                          int m, float* __restrict__ c, int ldc, Epi ep) {
    const int row = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
    if (row >= m) return;
    const float* p = part + (int64_t) t * m + row;
    float v = p[0];
    for (int s = 1; s < ns; s++) v += p[(int64_t) s * slice];
    float* dst = c + (int64_t) t * ldc + row;
    *dst = epilogue(ep, v, row, dst);
}

hipError_t launch_split_reduce(const float* part, int ns, int64_t slice, int m, int n, float* c, int ldc,
                               hipStream_t st, const Epi& ep) {
    split_reduce_kernel<<<dim3((m + 255) / 256, n), 256, 0, st>>>(part, ns, slice, m, c, ldc, ep);
    return hipGetLastError();
}

// K slices for a grid of `total` workgroups: enough for about two workgroups per CU, whole super-blocks each.
static void split_plan(int total, int nsb, int* ns, int* sb_per) {
    int want = total >= 384 ? 1 : (512 + total - 1) / total;
    want = want < nsb ? want : nsb;
    *sb_per = want > 1 ? (nsb + want - 1) / want : 0;
    *ns = want > 1 ? (nsb + *sb_per - 1) / *sb_per : 1;
}

// Workgroups of two resident per CU take about the same CU time whether a CU holds one or two, so a call
// takes ceil(tiles per CU) tile times: Q4_K 14336x4096 at n = 448, 512 and 576 (784, 896 and 1008 tiles)
// all ran 128 us. Each XCD takes a contiguous run of T8 = ceil(tiles / 8) tiles over its CUs; when that
// leaves r <= CUs / 2 tiles for a last partial round, those r tiles run as 2r half tiles (32 tokens) instead,
// one per CU. Returns r, or 0 for no split.
// CUs per device, filled by gemm_tail_prime at context creation (before any caller can be capturing a graph)
static std::atomic<int> g_cus[64];
void gemm_tail_prime(int dev) {
    int n = 0;
    if (dev >= 0 && dev < 64 && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
        g_cus[dev].store(n, std::memory_order_relaxed);
}
int device_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    return g_cus[dev].load(std::memory_order_relaxed);
}
static int tail_split(int total) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    const int n = g_cus[dev].load(std::memory_order_relaxed);
    if (n < 8) return 0;   // not primed: no split
    const int cu8 = n / 8, T8 = (total + 7) / 8, r = T8 % cu8;
    return r > 0 && 2 * r <= cu8 ? r : 0;
}

template <int DT, int RT, int CT>
static hipError_t kq_go(const WeightView& w, const GemmAct& A, int m, int n, float* c, int ldc, hipStream_t st,
                        const Groups& gp = Groups{}, float* part = nullptr, const Epi& ep = Epi{}) {
    using S = Stage<DT, RT, CT>;
    const int nrb = (m + 32 * S::TW - 1) / (32 * S::TW), ncb = A.NP / S::BN;
    const int64_t tiles = (w.r0 + tiled_rows(m)) / 32 - w.r0 / 32;   // tiles of the view that exist
    const int total = nrb * ncb, grid = tile_grid(gp.map64 != nullptr, total);
    const size_t lds = 2 * (size_t) S::BYTES;
    static std::atomic<bool> attr{false};   // threads racing here both set the same value
    if (!attr.load(std::memory_order_acquire)) {
        hipError_t e = hipFuncSetAttribute((const void*) kq_gemm_kernel<DT, RT, CT>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
        if (e != hipSuccess) return e;
        attr.store(true, std::memory_order_release);
    }
    int ns = 1, sb_per = 0;
    if (part != nullptr) split_plan(total, A.Kp / 256, &ns, &sb_per);
    if (ns == 1) {
        const int xs = gp.map64 == nullptr ? tail_split(total) : 0;
        kq_gemm_kernel<DT, RT, CT><<<grid + 8 * xs, MMA_THREADS, lds, st>>>(w, A, m, n, c, ldc, nrb, ncb, tiles, gp, 0,
                                                                            0, ep, xs);
        return hipGetLastError();
    }
    const int64_t slice = (int64_t) n * m;
    kq_gemm_kernel<DT, RT, CT><<<dim3(grid, ns), MMA_THREADS, lds, st>>>(w, A, m, n, part, m, nrb, ncb, tiles, gp,
                                                                         sb_per, slice, Epi{}, 0);
    split_reduce_kernel<<<dim3((m + 255) / 256, n), 256, 0, st>>>(part, ns, slice, m, c, ldc, ep);
    return hipGetLastError();
}

size_t gemm_mma_split_floats(int dt, int k, int m, int n) {
    if (dt != Q4_K && dt != Q5_K && dt != Q6_K && dt != MXFP4 && dt != Q4_0 && dt != Q8_0 && dt != NVFP4 && dt != Q1_0)
        return 0;
    const int nrb = (m + 32 * MMA_WAVES - 1) / (32 * MMA_WAVES), ncb = (n + 63) / 64, nsb = (k + 255) / 256;
    int ns, sb_per;
    split_plan(nrb * ncb, nsb, &ns, &sb_per);
    return ns > 1 ? (size_t) ns * n * m : 0;
}

hipError_t launch_gemm_mma(int dt, const WeightView& w, const GemmAct& A, int k, int m, int n, float* c, int ldc,
                           hipStream_t st, float* part, const Epi& ep) {
    if (((dt == Q4_K || dt == Q5_K || dt == Q6_K) && k % 256) || (w.r0 & 31) || A.NP % 64) return hipErrorNotSupported;
    switch (dt) {
    case Q4_K: return kq_go<Q4_K, 1, 2>(w, A, m, n, c, ldc, st, Groups{}, part, ep);
    case Q5_K: return kq_go<Q5_K, 1, 2>(w, A, m, n, c, ldc, st, Groups{}, part, ep);
    case NVFP4: return kq_go<NVFP4, 1, 2>(w, A, m, n, c, ldc, st, Groups{}, part, ep);
    case Q1_0: return kq_go<Q1_0, 1, 2>(w, A, m, n, c, ldc, st, Groups{}, part, ep);
    case Q4_0: return kq_go<Q4_0, 1, 2>(w, A, m, n, c, ldc, st, Groups{}, part, ep);
    case Q8_0: return kq_go<Q8_0, 1, 2>(w, A, m, n, c, ldc, st, Groups{}, part, ep);
    case Q6_K: return kq_go<Q6_K, 1, 2>(w, A, m, n, c, ldc, st, Groups{}, part, ep);
    case MXFP4: return kq_go<MXFP4, 1, 2>(w, A, m, n, c, ldc, st, Groups{}, part, ep);
    default: return hipErrorNotSupported;
    }
}

hipError_t launch_gemm_mma_grouped(int dt, const WeightView& w, const GemmAct& A, int k, const Groups& g, int cap64,
                                   float* c, int ldc, hipStream_t st) {
    if (((dt == Q4_K || dt == Q6_K) && k % 256) || (w.r0 & 31) || (g.gm & 31) || A.NP != cap64 * 64)
        return hipErrorNotSupported;
    if (cap64 <= 0) return hipSuccess;
    switch (dt) {
    case Q4_K: return kq_go<Q4_K, 1, 2>(w, A, g.gm, A.NP, c, ldc, st, g);
    case Q4_0: return kq_go<Q4_0, 1, 2>(w, A, g.gm, A.NP, c, ldc, st, g);
    case Q8_0: return kq_go<Q8_0, 1, 2>(w, A, g.gm, A.NP, c, ldc, st, g);
    case Q6_K: return kq_go<Q6_K, 1, 2>(w, A, g.gm, A.NP, c, ldc, st, g);
    case MXFP4: return kq_go<MXFP4, 1, 2>(w, A, g.gm, A.NP, c, ldc, st, g);
    default: return hipErrorNotSupported;
    }
}

}  // namespace jamhip
