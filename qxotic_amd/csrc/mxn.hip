// Opt-in native-MX path for MXFP4 weights (jamhip_ctx_set_mx_native): the weights go to the matrix cores as
// the fp4 (e2m1) codes they are stored in, the activations as MX-FP8 (OCP e4m3 codes with one e8m0 scale
// per 32-element block) split into a high and a low part, and v_mfma_scale_f32_32x32x64_f8f6f4 applies both
// operands' block scales in hardware. No per-block VALU work is left: the f32 accumulators run over all of K.
//
// This is NOT jam's activation semantics (jam quantizes activations to int8 with an f32 scale per block,
// jam_kernels_q4k_avx512.c:25-37, and multiplies MXFP4's doubled e2m1 codes by them, jam_mxfp4.h:14-24):
// it is a separate mode with its own tolerance. The weight values are exactly jam's (e2m1 · 2^(e - 127) =
// kv · 2^(e - 128)); the activation x is represented as hi + lo with
//   E   = the smallest exponent with max|x_block| · 2^-E <= 448 (e4m3's largest finite),
//   hi  = e4m3(x · 2^-E)            (round to nearest even), block scale 2^E,
//   lo  = e4m3((x · 2^-E - hi) · 16), block scale 2^(E - 4),
// about 8 significant bits per element (jam's int8 codes carry the block maximum / 127 steps); mode 2 drops
// lo (one MFMA per step, about 4 bits). The hardware's scaled block dot is not exact: its results move in
// steps of about 2^-16 at unit magnitude (measured), far below either mode's activation error.
//
// Operand layout (gfx950, 32x32x64, verified on the device): A lane (r, q) holds row r's K elements 32q..32q+31
// as 32 nibbles, nibble n at byte n / 2 (low nibble first), with A's scale for that 32-block; B lane (c, q)
// holds 32 bytes: bytes 0-15 are K 16q..16q+15 (first 32-block), bytes 16-31 are K 32+16q..32+16q+15 (second
// 32-block), and B's scale operand of lane (c, q) is that of K-block q. An MXFP4 block's byte b holds elements
// b (low nibble) and b + 16 (high), so MFMA nibble n of a block is element n/2 + 16·(n % 2): the weight bytes
// are used as stored, and the activation codes are written in that element order.
#include "common.h"
#include "launch.h"

#include <atomic>

namespace jamhip {

namespace mxn {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

// OCP e4m3 (E4M3FN) code of v, |v| <= 448, round to nearest even (no NaN or saturation arises in range).
JAMHIP_DEV uint32_t e4m3(float v) {
    const uint32_t sgn = v < 0.0f ? 0x80u : 0u;
    const float a = fabsf(v);
    if (a < 0.015625f) {                          // below 2^-6: subnormal codes, step 2^-9 (8 -> 0x08, normal)
        const uint32_t q = (uint32_t) rintf(a * 512.0f);
        return sgn | q;
    }
    int e;
    (void) frexpf(a, &e);                         // a = f · 2^e, f in [0.5, 1): exponent of a is e - 1
    const int ex = e - 1;
    uint32_t mt = (uint32_t) rintf(ldexpf(a, 3 - ex));   // in [8, 16]
    int be = ex + 7;
    if (mt == 16) {
        mt = 8;
        be += 1;
    }
    return sgn | ((uint32_t) be << 3) | (mt - 8);
}
JAMHIP_DEV float e4m3_value(uint32_t c) {
    const uint32_t be = (c >> 3) & 15, mt = c & 7;
    const float mag = be == 0 ? (float) mt * 0.001953125f : ldexpf((float) (8 + mt), (int) be - 10);
    return (c & 0x80u) ? -mag : mag;
}

JAMHIP_DEV int slot_source(int t, int n, const int* gmap, const int* goff, const int* gpoff) {
    if (gmap == nullptr) return t < n ? t : -1;
    const int ex = gmap[t >> 6];
    if (ex < 0) return -1;
    const int l = t - gpoff[ex];
    return l < goff[ex + 1] - goff[ex] ? goff[ex] + l : -1;
}

}  // namespace mxn

// One workgroup of 256 threads per token slot; a half-wave (32 lanes) per 32-element block, one element per
// lane: the block maximum by shuffles, E, the hi / lo codes in the MFMA B order, the two scale bytes. The
// codes of 8 blocks (4 K-steps x 2 halves x 32 bytes per plane) are assembled in LDS and written as 16-byte
// pieces. A padding slot (past n, or past its expert's rows) is left unwritten: its token column is computed
// but never stored. Mode 2 writes no lo plane (the GEMM reads none).
__global__ void __launch_bounds__(256) mxn_prep_kernel(const float* __restrict__ a, int lda, int n, int k, int Kp,
                                                       int NP, int mode, uint8_t* __restrict__ hi,
                                                       uint8_t* __restrict__ lo, uint8_t* __restrict__ shi,
                                                       uint8_t* __restrict__ slo, const int* __restrict__ gmap,
                                                       const int* __restrict__ goff, const int* __restrict__ gpoff) {
    using namespace mxn;
    __shared__ __align__(16) uint8_t lh[256], ll[256];  // 8 blocks' codes: [4 steps][2 halves][32 bytes]
    const int t = blockIdx.x;
    const int src = slot_source(t, n, gmap, goff, gpoff);
    if (src < 0) return;
    const int e = threadIdx.x & 31;                     // element within the block
    for (int b = threadIdx.x >> 5; b < Kp / 32; b += 8) {
        const int col = 32 * b + e;
        const float x = src >= 0 && col < k ? a[(int64_t) src * lda + col] : 0.0f;
        float amax = fabsf(x);
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 32));
        int E = -127;
        if (amax > 0.0f) {
            int ee;
            const float f = frexpf(amax / 448.0f, &ee);   // amax / 448 = f · 2^ee
            E = f == 0.5f ? ee - 1 : ee;
            if (ldexpf(amax, -E) > 448.0f) E += 1;        // rounding in amax / 448
            E = max(-127, min(127, E));
        }
        const float v = ldexpf(x, -E);
        const uint32_t ch = e4m3(v);
        const bool lo_ok = mode == 1 && E - 4 >= -127;
        const uint32_t cl = lo_ok ? e4m3((v - e4m3_value(ch)) * 16.0f) : 0u;
        // B order: K-step s = b / 2, bytes 16·(b % 2) + j of lane half q, element 8q + j/2 + 16·(j % 2)
        const int q = (e & 15) >> 3, j = 2 * ((e & 15) - 8 * q) + (e >> 4);
        const int bl = b & 7;                            // block within the 8 of this pass
        const int li = ((bl >> 1) * 2 + q) * 32 + 16 * (bl & 1) + j;
        lh[li] = (uint8_t) ch;
        ll[li] = (uint8_t) cl;
        if (e == 0) {
            shi[(int64_t) b * NP + t] = (uint8_t) (E + 127);
            if (mode == 1) slo[(int64_t) b * NP + t] = lo_ok ? (uint8_t) (E - 4 + 127) : (uint8_t) 0;
        }
        __syncthreads();
        // 16 pieces of 16 bytes per plane: piece p = (step s, half q, 16-byte half h) of this pass's 4 steps
        if (threadIdx.x < (mode == 1 ? 32 : 16)) {
            const int pl = threadIdx.x >> 4, p = threadIdx.x & 15, s = p >> 2, qq = (p >> 1) & 1, h = p & 1;
            const int step = (b - bl) / 2 + s;
            uint8_t* dst = (pl ? lo : hi) + (((int64_t) step * 2 + qq) * NP + t) * 32 + 16 * h;
            *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>((pl ? ll : lh) + (s * 2 + qq) * 32 + 16 * h);
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------- GEMM
// Workgroup: 4 waves x 32 rows (wave w: row tile w) x 64 tokens (2 token tiles per wave); stages of 128 K (two
// 64-K MFMA steps) copied global -> LDS, double-buffered. Stage buffer: weight chunks [4 tiles][4 blocks][32 rows]
// [16 B], header [4 tiles][32 rows][16 B], B hi / lo [2 steps][2 halves][64 tokens][32 B] each, scales hi / lo
// [4 blocks][64 tokens] bytes each.
namespace mxn {
constexpr int A_OFF = 0, H_OFF = 8192, BH_OFF = 10240, BL_OFF = 18432, SH_OFF = 26624, SL_OFF = 26880;
constexpr int STAGE = 27648;
JAMHIP_DEV void dma16(const void* g, void* lds_base) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*) lds_base, 16, 0, 0);
}
}  // namespace mxn

template <int MODE>
__global__ void __launch_bounds__(256, 2) mxn_gemm_kernel(WeightView w, MxAct A, int m, int n, float* __restrict__ c,
                                                          int ldc, int nrb, int ncb, int64_t tiles, Groups gp, Epi ep) {
    using namespace mxn;
    __shared__ __align__(1024) unsigned char smem[2 * STAGE];
    const int total = nrb * ncb;
    const int lin = tile_of_block(gp.map64 != nullptr, total);
    if (lin >= total) return;
    int rb = lin / ncb, cb = lin % ncb;
    if (gp.map64 != nullptr && grouped_tile(gp, lin, nrb, &rb, &cb) < 0) return;
    const int64_t T0 = (int64_t) rb * 4;
    const int n0 = cb * 64;
    const int lane = threadIdx.x & 63, r = lane & 31, q = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = (int) w.G;
    const int nst = (A.K / 32 + 3) / 4;                 // stages holding at least one block of k
    int64_t r0t = w.r0 >> 5;
    int slot0 = 0, crow0 = 0, nvalid = n;
    if (gp.map64 != nullptr) {                          // grouped: this slot block's expert
        const int e = __builtin_amdgcn_readfirstlane(gp.map64[cb]);
        if (e < 0) return;
        r0t = (w.r0 + (int64_t) e * gp.gm) >> 5;
        tiles = gp.gm / 32;
        m = gp.gm;
        slot0 = __builtin_amdgcn_readfirstlane(gp.poff64[e]);
        crow0 = __builtin_amdgcn_readfirstlane(gp.off[e]);
        nvalid = __builtin_amdgcn_readfirstlane(gp.off[e + 1]) - crow0;
        if (gp.bias != nullptr) ep.bias = gp.bias + (int64_t) e * gp.gm;
    }
    constexpr int NC = group_chunks(MXFP4);
    const int64_t Tw = T0 + wave < tiles ? T0 + wave : tiles - 1;
    const uint8_t* a_src = w.qs + (r0t + Tw) * G * (NC * CHUNK_STRIDE) + 16 * lane;
    const int64_t Th = T0 + 2 * (wave & 1) + q < tiles ? T0 + 2 * (wave & 1) + q : tiles - 1;
    const uint8_t* h_src = w.sc + ((r0t + Th) * G * 32 + r) * 16;
    const int64_t bstep = (int64_t) 2 * A.NP * 32;      // bytes per 64-K step (both halves)
    // B pieces (1 KB = 32 tokens x 32 B): wave w takes plane w >> 1 (hi, lo) and (step, half) pairs 2(w&1), +1
    const uint8_t* bplane = (wave >> 1) ? A.lo : A.hi;
    const int boff = (wave >> 1) ? BL_OFF : BH_OFF;
    auto issue = [&](int st, unsigned char* buf) {
        const int g = st >> 1, h2 = st & 1;
        const uint8_t* ag = a_src + (int64_t) g * (NC * CHUNK_STRIDE) + (4 * h2) * CHUNK_STRIDE;
        dma16(ag, buf + A_OFF + wave * 2048);
        dma16(ag + 2 * CHUNK_STRIDE, buf + A_OFF + wave * 2048 + 1024);
        if (MODE == 1 || wave < 2) {   // mode 2 has no lo plane
#pragma unroll
            for (int p = 0; p < 2; p++) {
                const int sq = 2 * (wave & 1) + p;     // (step, half) = (sq >> 1, sq & 1)
#pragma unroll
                for (int th = 0; th < 2; th++)
                    dma16(bplane + (int64_t) (2 * st + (sq >> 1)) * bstep + ((int64_t) (sq & 1) * A.NP + n0 + 32 * th) * 32 + 16 * lane,
                          buf + boff + (sq * 64 + 32 * th) * 32);
            }
        }
        if (wave < 2) dma16(h_src + (int64_t) g * 32 * 16, buf + H_OFF + wave * 1024);
        if ((wave == 2 || (wave == 3 && MODE == 1)) && lane < 16) {   // scales: 4 blocks x 64 tokens, a byte each
            const uint8_t* s = (wave == 2 ? A.shi : A.slo) + (int64_t) (4 * st + (lane >> 2)) * A.NP + n0 + 16 * (lane & 3);
            dma16(s, buf + (wave == 2 ? SH_OFF : SL_OFF));
        }
    };
    floatx16 acc[2] = {floatx16{}, floatx16{}};
    issue(0, smem);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int st = 0; st < nst; st++) {
        unsigned char* buf = smem + (st & 1) * STAGE;
        const int h2 = st & 1;
        v8i av[2], bh[2][2], bl[2][2];
        int sa[2], sbh[2][2], sbl[2][2];
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            const uint4 x = *reinterpret_cast<const uint4*>(buf + A_OFF + (wave * 4 + 2 * kk + q) * 512 + 16 * r);
            av[kk] = v8i{(int) x.x, (int) x.y, (int) x.z, (int) x.w, 0, 0, 0, 0};
            sa[kk] = buf[H_OFF + (wave * 32 + r) * 16 + 4 * h2 + 2 * kk + q];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int bo = ((2 * kk + q) * 64 + 32 * j + r) * 32;
                bh[kk][j] = *reinterpret_cast<const v8i*>(buf + BH_OFF + bo);
                sbh[kk][j] = buf[SH_OFF + (2 * kk + q) * 64 + 32 * j + r];
                if (MODE == 1) {
                    bl[kk][j] = *reinterpret_cast<const v8i*>(buf + BL_OFF + bo);
                    sbl[kk][j] = buf[SL_OFF + (2 * kk + q) * 64 + 32 * j + r];
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (st + 1 < nst) issue(st + 1, smem + ((st + 1) & 1) * STAGE);
#pragma unroll
        for (int kk = 0; kk < 2; kk++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av[kk], bh[kk][j], acc[j], 4, 0, 0, sa[kk], 0,
                                                                         sbh[kk][j]);
                if (MODE == 1)
                    acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av[kk], bl[kk][j], acc[j], 4, 0, 0, sa[kk],
                                                                             0, sbl[kk][j]);
            }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    // epilogue: lane holds token n0 + 32j + r, rows 8·(e/4) + 4q + e%4 of the wave's tile
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int t = n0 + 32 * j + r, tl = t - slot0;
        if (tl >= nvalid) continue;
        float* ct = c + (int64_t) (crow0 + tl) * ldc;
        const int64_t rowb = (T0 + wave) * 32 + 4 * q;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int64_t row = rowb + 8 * (e >> 2) + (e & 3);
            if (row < m) ct[row] = epilogue(ep, acc[j][e], row, ct + row);
        }
    }
}

static int64_t a256(int64_t v) { return (v + 255) & ~(int64_t) 255; }

size_t mx_act_bytes_np(int NP, int k) {
    const int64_t Kp = (k + 255) / 256 * 256;
    return (size_t) (2 * a256(Kp * NP) + 2 * a256((Kp / 32) * NP));
}

static hipError_t mx_prep_np(const float* a, int lda, int n, int NP, int k, int mode, void* scratch, MxAct* out,
                             const int* gmap, const int* goff, const int* gpoff, hipStream_t st) {
    const int Kp = (k + 255) / 256 * 256;
    uint8_t* p = (uint8_t*) scratch;
    uint8_t* hi = p;
    uint8_t* lo = hi + a256((int64_t) Kp * NP);
    uint8_t* shi = lo + a256((int64_t) Kp * NP);
    uint8_t* slo = shi + a256((int64_t) (Kp / 32) * NP);
    *out = MxAct{hi, lo, shi, slo, NP, Kp, k};
    if (NP <= 0) return hipSuccess;
    mxn_prep_kernel<<<NP, 256, 0, st>>>(a, lda, n, k, Kp, NP, mode, hi, lo, shi, slo, gmap, goff, gpoff);
    return hipGetLastError();
}

hipError_t launch_mx_prep(const float* a, int lda, int n, int k, int mode, void* scratch, MxAct* out, hipStream_t st) {
    return mx_prep_np(a, lda, n, (n + 63) / 64 * 64, k, mode, scratch, out, nullptr, nullptr, nullptr, st);
}
hipError_t launch_mx_prep_grouped(const float* a, int lda, int k, int mode, const Groups& g, int cap64, void* scratch,
                                  MxAct* out, hipStream_t st) {
    return mx_prep_np(a, lda, 0, cap64 * 64, k, mode, scratch, out, g.map64, g.off, g.poff64, st);
}

static hipError_t mx_go(int mode, const WeightView& w, const MxAct& A, int m, int n, float* c, int ldc, const Groups& gp,
                        const Epi& ep, hipStream_t st) {
    if ((w.r0 & 31) || A.NP % 64) return hipErrorNotSupported;
    const int nrb = (m + 127) / 128, ncb = A.NP / 64;
    const int64_t tiles = (w.r0 + tiled_rows(m)) / 32 - w.r0 / 32;
    const int grid = tile_grid(gp.map64 != nullptr, nrb * ncb);
    if (mode == 1) mxn_gemm_kernel<1><<<grid, 256, 0, st>>>(w, A, m, n, c, ldc, nrb, ncb, tiles, gp, ep);
    else mxn_gemm_kernel<2><<<grid, 256, 0, st>>>(w, A, m, n, c, ldc, nrb, ncb, tiles, gp, ep);
    return hipGetLastError();
}

hipError_t launch_mx_gemm(int mode, const WeightView& w, const MxAct& A, int m, int n, float* c, int ldc, hipStream_t st,
                          const Epi& ep) {
    return mx_go(mode, w, A, m, n, c, ldc, Groups{}, ep, st);
}
hipError_t launch_mx_gemm_grouped(int mode, const WeightView& w, const MxAct& A, const Groups& g, int cap64, float* c,
                                  int ldc, hipStream_t st) {
    if ((g.gm & 31) || A.NP != cap64 * 64) return hipErrorNotSupported;
    if (cap64 <= 0) return hipSuccess;
    return mx_go(mode, w, A, g.gm, A.NP, c, ldc, g, Epi{}, st);
}

}  // namespace jamhip
