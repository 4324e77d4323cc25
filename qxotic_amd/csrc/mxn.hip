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
#include "groups.h"

#include <atomic>
#include <type_traits>

namespace jamhip {

namespace mxn {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

JAMHIP_DEV int slot_source(int t, int n, const int* gmap, const int* goff, const int* gpoff) {
    if (gmap == nullptr) return t < n ? t : -1;
    const int ex = gmap[t >> 6];
    if (ex < 0) return -1;
    const int l = t - gpoff[ex];
    return l < goff[ex + 1] - goff[ex] ? goff[ex] + l : -1;
}

}  // namespace mxn

// A workgroup of 256 threads per token slot, eight lanes per 32-element block (lane s of a group: elements
// 4s..4s+3), 32 blocks per round; the row's loads for up to four rounds are issued before any is used, and no
// step waits on another lane group, so a slot costs about one load latency. Per block: the maximum by shuffles
// within the group, E, the hi / lo codes. The MFMA B order puts elements 8q..8q+7 and 8q+16..8q+23 of a block,
// interleaved, in the 16 bytes of lane half q: lane s < 4 interleaves its four codes with those of lane s + 4
// and stores the 8 bytes. A padding slot (past n, or past its expert's rows) is left unwritten: its token column
// is computed but never stored. Mode 2 writes no lo plane (the GEMM reads none).
// Fused grouped mode (pg.counts set): every workgroup derives the expert table from the device counts
// (fused_scan; workgroup 0 also publishes the offsets and the slot map the GEMM reads), then takes its XCD's
// share of the slots [0, P) in turn, as gemm_prep does; otherwise workgroup t takes slot t.
__global__ void __launch_bounds__(256) mxn_prep_kernel(const float* __restrict__ a, int lda, int n, int k, int Kp,
                                                       int NP, int mode, uint8_t* __restrict__ hi,
                                                       uint8_t* __restrict__ lo, uint8_t* __restrict__ shi,
                                                       uint8_t* __restrict__ slo, const int* __restrict__ gmap,
                                                       const int* __restrict__ goff, const int* __restrict__ gpoff,
                                                       int vec, PrepGroups pg) {
    using namespace mxn;
    __shared__ int own;
    SlotOwner so;
    const bool fused = pg.counts != nullptr;
    const int P = fused ? fused_scan(pg, blockIdx.x == 0, &so) : NP;
    const int x8 = (int) (blockIdx.x % 8), nw = (int) (gridDim.x >> 3), P8 = ((P + 7) / 8 + 7) & ~7;
    const int t_first = fused ? x8 * P8 + (int) (blockIdx.x >> 3) : (int) blockIdx.x;
    const int t_end = fused ? min((x8 + 1) * P8, P) : (int) blockIdx.x + 1;
    const int sub = threadIdx.x & 7, nb = Kp / 32;
    constexpr int RQ = 4;   // rounds in flight
    // slot t's source row (-1: padding); in fused mode the owner thread passes it through LDS (every thread calls)
    auto resolve = [&](int t) -> int {
        if (!fused) return slot_source(t, n, gmap, goff, gpoff);
        slot_owner_store(pg, so, t, &own, nullptr);
        __syncthreads();
        const int r = own;
        __syncthreads();   // own is the next slot's
        return r;
    };
    // the loads of pass r0 of row src (blocks r0 .. r0 + 32·RQ - 1, eight lanes per block; zeros past k)
    auto load = [&](int src, int r0, float (&x)[RQ][4]) {
        const float* row = a + (int64_t) (src >= 0 ? src : 0) * lda;
#pragma unroll
        for (int u = 0; u < RQ; u++) {
            const int b = r0 + 32 * u + (threadIdx.x >> 3), col = 32 * b + 4 * sub;
            if (src >= 0 && b < nb && vec && col + 3 < k) {   // a and lda 16-byte aligned (the launcher checks)
                const float4 f = *reinterpret_cast<const float4*>(row + col);
                x[u][0] = f.x, x[u][1] = f.y, x[u][2] = f.z, x[u][3] = f.w;
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) x[u][i] = src >= 0 && b < nb && col + i < k ? row[col + i] : 0.0f;
            }
        }
    };
    // the codes, scales and stores of pass r0 of slot t
    auto code = [&](int t, int r0, float (&x)[RQ][4]) {
#pragma unroll
        for (int u = 0; u < RQ; u++) {
            const int b = r0 + 32 * u + (threadIdx.x >> 3);
            if (r0 + 32 * u >= nb) break;   // uniform: no block of this load step exists
            float amax = fmaxf(fmaxf(fabsf(x[u][0]), fabsf(x[u][1])), fmaxf(fabsf(x[u][2]), fabsf(x[u][3])));
#pragma unroll
            for (int o = 4; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 8));
            int E = -127;
            if (amax > 0.0f) {
                int ee;
                const float f = frexpf(amax / 448.0f, &ee);   // amax / 448 = f · 2^ee
                E = f == 0.5f ? ee - 1 : ee;
                if (ldexpf(amax, -E) > 448.0f) E += 1;        // rounding in amax / 448
                E = max(-127, min(127, E));
            }
            const bool lo_ok = mode == 1 && E - 4 >= -127;
            // x·2^-E is exact (|v| <= 448); the hardware conversion gives the nearest OCP e4m3 code, ties to the
            // even code; + 0.0f turns a -0 into +0 (code 0x00, not 0x80)
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = ldexpf(x[u][i], -E) + 0.0f;
            uint32_t ch = (uint32_t) __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
            ch = (uint32_t) __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], (int) ch, true);
            uint32_t cl = 0;
            if (lo_ok) {
                const float hv[4] = {__builtin_amdgcn_cvt_f32_fp8((int) ch, 0), __builtin_amdgcn_cvt_f32_fp8((int) ch, 1),
                                     __builtin_amdgcn_cvt_f32_fp8((int) ch, 2), __builtin_amdgcn_cvt_f32_fp8((int) ch, 3)};
                float rr[4];
#pragma unroll
                for (int i = 0; i < 4; i++) rr[i] = (v[i] - hv[i]) * 16.0f + 0.0f;
                cl = (uint32_t) __builtin_amdgcn_cvt_pk_fp8_f32(rr[0], rr[1], 0, false);
                cl = (uint32_t) __builtin_amdgcn_cvt_pk_fp8_f32(rr[2], rr[3], (int) cl, true);
            }
            const uint32_t ph = __shfl_xor(ch, 4, 8), pl = __shfl_xor(cl, 4, 8);
            if (b < nb && sub < 4) {
                // bytes: own0, partner0, own1, partner1, ... (elements e, e + 16 of the block)
                auto mix = [](uint32_t o, uint32_t p) {
                    const uint32_t lo16 = (o & 0xffu) | ((p & 0xffu) << 8) | ((o & 0xff00u) << 8) | ((p & 0xff00u) << 16);
                    const uint32_t hi16 = ((o >> 16) & 0xffu) | (((p >> 16) & 0xffu) << 8) | ((o >> 24) << 16) | ((p >> 24) << 24);
                    return make_uint2(lo16, hi16);
                };
                const int64_t off = ((int64_t) ((b >> 1) * 2 + (sub >> 1)) * NP + t) * 32 + 16 * (b & 1) + 8 * (sub & 1);
                *reinterpret_cast<uint2*>(hi + off) = mix(ch, ph);
                if (mode == 1) *reinterpret_cast<uint2*>(lo + off) = mix(cl, pl);
                if (sub == 0) {
                    shi[(int64_t) b * NP + t] = (uint8_t) (E + 127);
                    if (mode == 1) slo[(int64_t) b * NP + t] = lo_ok ? (uint8_t) (E - 4 + 127) : (uint8_t) 0;
                }
            }
        }
    };
    const int step = fused ? nw : 1;
    if (nb <= 32 * RQ) {
        // one pass per slot: the next slot's loads are issued before this slot's codes are computed
        float xa[RQ][4], xb[RQ][4];
        int t = t_first, src = t < t_end ? resolve(t) : -1;
        if (t < t_end && src >= 0) load(src, 0, xa);
        while (t < t_end) {
            const int tn = t + step;
            const int srcn = tn < t_end ? resolve(tn) : -1;   // uniform: every thread resolves
            if (srcn >= 0) load(srcn, 0, xb);
            if (src >= 0) code(t, 0, xa);
#pragma unroll
            for (int u = 0; u < RQ; u++)
#pragma unroll
                for (int i = 0; i < 4; i++) xa[u][i] = xb[u][i];
            t = tn;
            src = srcn;
        }
        return;
    }
    for (int t = t_first; t < t_end; t += step) {
        const int src = resolve(t);
        if (src < 0) continue;   // uniform over the workgroup
        for (int r0 = 0; r0 < nb; r0 += 32 * RQ) {
            float x[RQ][4];
            load(src, r0, x);
            code(t, r0, x);
        }
    }
}

// ------------------------------------------------------------------------------------------- GEMM
// Workgroup: MW waves x 32 rows (wave w: row tile w) x 64 tokens (2 token tiles per wave), 8 / MW per CU; K in
// stages of KS 64-K MFMA steps. The kernel does no per-block VALU work, so the matrix cores wait only on memory,
// and every operand goes global -> LDS (global_load_lds) RB - 1 stages ahead into a ring of RB stage buffers.
// Each buffer is its own LDS object, and every copy in flight is such a copy, so the compiler's wait before a
// buffer's reads covers only the copies into that buffer. Stage buffer:
//   weights  [MW waves][KS steps][64 lanes][16 B]     (lane (r, q) of step kk: block 2kk + q of row r)
//   headers  [MW waves][256 B]                        (the rows' exponents of the stage's 2·KS blocks)
//   codes    [KS steps][2 halves][2 planes][64 tokens][16 B] (plane p = bytes 16p..16p+15 of a token's 32, so a
//                                                      fragment read is 1 KB contiguous over the wave: no bank
//                                                      conflicts; piece i = (step, half, plane) is copied by
//                                                      wave i / (4·KS / MW))
//   scales   [MW waves][256 B]                        (piece i: blocks 4i..4i+3 x 64 tokens, copied by the
//                                                      waves w with w % (KS / 2) == i into their own slot)
// Every wave issues the same copies each stage (KS + 4·KS / MW + 2), so the wait for a stage's own copies is one
// fixed count of later copies; the stage barrier is then a plain s_barrier (a workgroup fence would wait for
// every copy in flight). Past the end of K the copies re-read the last stage. PLANE selects the hi (0) or lo (1)
// codes and scales: mode 2 is one launch over hi, mode 1 a second launch over lo that adds its products into C
// (the first launch applied the call's epilogue).
namespace mxn {
// 4 waves, 256-K stages, two buffers: two workgroups per CU, each a stage ahead (measured against 8 waves with 3
// buffers, 128-K stages with 3-5 buffers and 2-wave workgroups: fastest at n = 512 and 2048)
#ifndef JAMHIP_MXN_KS
#define JAMHIP_MXN_MW 4
#define JAMHIP_MXN_KS 4
#define JAMHIP_MXN_RB 2
#endif
constexpr int MW = JAMHIP_MXN_MW, KS = JAMHIP_MXN_KS, RB = JAMHIP_MXN_RB;   // waves, steps per stage, buffers
constexpr int WPC = 8 / MW;                             // workgroups per CU
constexpr int PPW = 4 * KS / MW;                        // code pieces per wave and stage
constexpr int NPW = KS + PPW + 2;                       // copies per wave and stage
constexpr int OA = 0, OH = OA + MW * KS * 1024, OB = OH + MW * 256, OS = OB + 4 * KS * 1024, BSTAGE = OS + MW * 256;
static_assert(WPC * RB * BSTAGE <= 160 * 1024 && (KS == 2 || KS == 4) && PPW >= 1 && RB >= 2 && RB <= 6, "ring");
// s_waitcnt with only vmcnt set (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
template <int N> JAMHIP_DEV void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
}  // namespace mxn

template <int PLANE>
__global__ void __launch_bounds__(64 * mxn::MW, mxn::WPC) mxn_gemm_kernel(WeightView w, MxAct A, int m, int n,
                                                                   float* __restrict__ c, int ldc, int nrb, int ncb,
                                                                   int64_t tiles, Groups gp, Epi ep) {
    using namespace mxn;
    __shared__ __align__(1024) unsigned char sb0[BSTAGE], sb1[BSTAGE], sb2[RB > 2 ? BSTAGE : 1], sb3[RB > 3 ? BSTAGE : 1],
        sb4[RB > 4 ? BSTAGE : 1], sb5[RB > 5 ? BSTAGE : 1];
    const int total = nrb * ncb;
    const int lin = tile_of_block(gp.map64 != nullptr, total);
    if (lin >= total) return;
    int rb = lin / ncb, cb = lin % ncb;
    if (gp.map64 != nullptr && grouped_tile(gp, lin, nrb, &rb, &cb) < 0) return;
    const int64_t T0 = (int64_t) rb * MW;
    const int n0 = cb * 64;
    const int lane = threadIdx.x & 63, r = lane & 31, q = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = (int) w.G;
    const int nsg = A.Kp / (64 * KS);                   // stages
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
    // valid tokens of this slot block all in its first 32 slots: the second token tile is neither copied nor
    // computed (its epilogue stores nothing either)
    const bool half = nvalid - (n0 - slot0) <= 32;
    constexpr int NC = group_chunks(MXFP4);
    const int64_t Tw = T0 + wave < tiles ? T0 + wave : tiles - 1;
    const uint8_t* a_src = w.qs + (r0t + Tw) * G * (NC * CHUNK_STRIDE) + 16 * lane;   // + group · 4096
    // headers: KS == 4, lane l copies word l % 2 of row l / 2's exponents; KS == 2, lane l word h of row l % 32
    const uint8_t* h_src = KS == 4 ? w.sc + ((r0t + Tw) * G * 32 + (lane >> 1)) * 16 + 4 * (lane & 1)
                                   : w.sc + ((r0t + Tw) * G * 32 + r) * 16;
    const int64_t sstep = (int64_t) A.NP * 32;          // bytes per (64-K step, half) plane
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    floatx16 acc[2] = {floatx16{}, floatx16{}};
    auto ring = [&](int i) -> unsigned char* {
        return i == 0 ? sb0 : i == 1 ? sb1 : i == 2 ? sb2 : i == 3 ? sb3 : i == 4 ? sb4 : sb5;
    };
    const uint8_t* codes = PLANE ? A.lo : A.hi;
    const uint8_t* scales = PLANE ? A.slo : A.shi;
    auto issue = [&](int s, unsigned char* buf) {
        const int64_t gs = (int64_t) min(s, nsg - 1) * KS;   // the stage's first 64-K step
        const int64_t g = gs / 4, k4 = gs % 4;                // its group, and step within the group
        const uint8_t* ag = a_src + g * (NC * CHUNK_STRIDE) + k4 * 2 * CHUNK_STRIDE;
#pragma unroll
        for (int kk = 0; kk < KS; kk++)   // chunks 2kk, 2kk + 1 of the stage: 1 KB contiguous
            __builtin_amdgcn_global_load_lds(ag + kk * 2 * CHUNK_STRIDE, (lds_void*) (buf + OA + (wave * KS + kk) * 1024),
                                             16, 0, 0);
        __builtin_amdgcn_global_load_lds(h_src + g * 512 + (KS == 2 ? 4 * (k4 >> 1) : 0), (lds_void*) (buf + OH + wave * 256),
                                         4, 0, 0);
#pragma unroll
        for (int i = 0; i < PPW; i++) {
            const int pc = wave * PPW + i, st = pc >> 2, hf = (pc >> 1) & 1, pl = pc & 1;
            if (!half || lane < 32)
                __builtin_amdgcn_global_load_lds(codes + (2 * (gs + st) + hf) * sstep + (int64_t) (n0 + lane) * 32 + 16 * pl,
                                                 (lds_void*) (buf + OB + pc * 1024), 16, 0, 0);
        }
        const int sp = wave % (KS / 2);
        __builtin_amdgcn_global_load_lds(scales + (2 * gs + 4 * sp + (lane >> 4)) * A.NP + n0 + 4 * (lane & 15),
                                         (lds_void*) (buf + OS + wave * 256), 4, 0, 0);
    };
#pragma unroll
    for (int s = 0; s < RB - 1; s++) issue(s, ring(s));
    auto stage = [&](auto U, int s) {
        constexpr int u = decltype(U)::value;
        const unsigned char* buf = ring(u);
        // stage s's copies were issued RB - 1 stages ago and RB - 2 stages' copies follow them; then every wave's
        // copies are in, and every wave is done reading the buffer that the next issue overwrites
        wait_vm<(RB - 2) * NPW>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        issue(s + RB - 1, ring((u + RB - 1) % RB));
        // the stage's operands, read up front as 16-byte loads (a 32-byte LDS load is split without the alias
        // information that keeps the compiler from waiting for every copy in flight)
        u32x4 av[KS];
        v8i bq[KS][2];
        int sq[KS][2];
        const uint2 hx = KS == 4 ? *reinterpret_cast<const uint2*>(buf + OH + wave * 256 + 8 * r)
                                 : make_uint2(*reinterpret_cast<const uint32_t*>(buf + OH + wave * 256 + 4 * r), 0u);
#pragma unroll
        for (int kk = 0; kk < KS; kk++) {
            av[kk] = *reinterpret_cast<const u32x4*>(buf + OA + (wave * KS + kk) * 1024 + 16 * lane);
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const u32x4 b0 = *reinterpret_cast<const u32x4*>(buf + OB + ((2 * kk + q) * 128 + 32 * j + r) * 16);
                const u32x4 b1 = *reinterpret_cast<const u32x4*>(buf + OB + ((2 * kk + q) * 128 + 64 + 32 * j + r) * 16);
                bq[kk][j] = v8i{(int) b0.x, (int) b0.y, (int) b0.z, (int) b0.w, (int) b1.x, (int) b1.y, (int) b1.z,
                                (int) b1.w};
                // block 2kk + q of the stage: scale piece (2kk + q) / 4, row (2kk + q) % 4 of 64 tokens
                sq[kk][j] = buf[OS + ((2 * kk + q) >> 2) * 256 + ((2 * kk + q) & 3) * 64 + 32 * j + r];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < KS; kk++) {
            const u32x4 x = av[kk];
            const v8i a8 = v8i{(int) x.x, (int) x.y, (int) x.z, (int) x.w, 0, 0, 0, 0};
            const int sa = (int) (((kk < 2 ? hx.x : hx.y) >> (8 * (2 * (kk & 1) + q))) & 0xffu);
            acc[0] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, bq[kk][0], acc[0], 4, 0, 0, sa, 0, sq[kk][0]);
            if (!half)
                acc[1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, bq[kk][1], acc[1], 4, 0, 0, sa, 0,
                                                                         sq[kk][1]);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // one turn of the ring per loop trip; a stage past the end of K is skipped (uniform over the workgroup)
    for (int s = 0; s < nsg; s += RB) {
        stage(std::integral_constant<int, 0>{}, s);
        if (s + 1 < nsg) {
            stage(std::integral_constant<int, 1 % RB>{}, s + 1);
            if (RB > 2 && s + 2 < nsg) {
                stage(std::integral_constant<int, 2 % RB>{}, s + 2);
                if constexpr (RB > 3) {
                    if (s + 3 < nsg) {
                        stage(std::integral_constant<int, 3 % RB>{}, s + 3);
                        if constexpr (RB > 4) {
                            if (s + 4 < nsg) {
                                stage(std::integral_constant<int, 4 % RB>{}, s + 4);
                                if constexpr (RB > 5)
                                    if (s + 5 < nsg) stage(std::integral_constant<int, 5 % RB>{}, s + 5);
                            }
                        }
                    }
                }
            }
        }
    }
    wait_vm<0>();   // no copy may still be writing this workgroup's LDS when it exits
    // epilogue: lane holds token n0 + 32j + r, rows 8·(e/4) + 4q + e%4 of the wave's tile
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int t = n0 + 32 * j + r, tl = t - slot0;
        if (tl >= nvalid) continue;
        store_column(c + (int64_t) (crow0 + tl) * ldc, (T0 + wave) * 32 + 4 * q, m, acc[j], 1.0f, ep, false);
    }
}

static int64_t a256(int64_t v) { return (v + 255) & ~(int64_t) 255; }

size_t mx_act_bytes_np(int NP, int k) {
    const int64_t Kp = (k + 255) / 256 * 256;
    return (size_t) (2 * a256(Kp * NP) + 2 * a256((Kp / 32) * NP));
}

static hipError_t mx_prep_np(const float* a, int lda, int n, int NP, int k, int mode, void* scratch, MxAct* out,
                             const int* gmap, const int* goff, const int* gpoff, hipStream_t st,
                             const PrepGroups& pg = PrepGroups{}) {
    const int Kp = (k + 255) / 256 * 256;
    uint8_t* p = (uint8_t*) scratch;
    uint8_t* hi = p;
    uint8_t* lo = hi + a256((int64_t) Kp * NP);
    uint8_t* shi = lo + a256((int64_t) Kp * NP);
    uint8_t* slo = shi + a256((int64_t) (Kp / 32) * NP);
    *out = MxAct{hi, lo, shi, slo, NP, Kp, k};
    if (NP <= 0) return hipSuccess;
    const int vec = (reinterpret_cast<uintptr_t>(a) & 15) == 0 && (lda & 3) == 0;
    // fused grouped mode: at most 1024 workgroups (all resident), each looping over its XCD's slots
    const int grid = pg.counts != nullptr ? (NP < 1024 ? (NP + 7) / 8 * 8 : 1024) : NP;
    mxn_prep_kernel<<<grid, 256, 0, st>>>(a, lda, n, k, Kp, NP, mode, hi, lo, shi, slo, gmap, goff, gpoff, vec, pg);
    return hipGetLastError();
}

hipError_t launch_mx_prep(const float* a, int lda, int n, int k, int mode, void* scratch, MxAct* out, hipStream_t st) {
    return mx_prep_np(a, lda, n, (n + 63) / 64 * 64, k, mode, scratch, out, nullptr, nullptr, nullptr, st);
}
hipError_t launch_mx_prep_grouped(const float* a, int lda, int k, int mode, const Groups& g, int cap64, void* scratch,
                                  MxAct* out, hipStream_t st) {
    return mx_prep_np(a, lda, 0, cap64 * 64, k, mode, scratch, out, g.map64, g.off, g.poff64, st);
}
hipError_t launch_mx_prep_grouped_fused(const float* a, int lda, int k, int mode, const PrepGroups& pg, void* scratch,
                                        MxAct* out, hipStream_t st) {
    if (pg.counts == nullptr || pg.E < 1 || pg.E > PREP_FUSED_MAX_E || pg.rows_cap < 0 || pg.cap64 < 1)
        return hipErrorInvalidValue;
    return mx_prep_np(a, lda, 0, pg.cap64 * 64, k, mode, scratch, out, nullptr, nullptr, nullptr, st, pg);
}

static hipError_t mx_go(int mode, const WeightView& w, const MxAct& A, int m, int n, float* c, int ldc, const Groups& gp,
                        const Epi& ep, hipStream_t st) {
    if ((w.r0 & 31) || A.NP % 64) return hipErrorNotSupported;
    const int nrb = (m + 32 * mxn::MW - 1) / (32 * mxn::MW), ncb = A.NP / 64;
    const int64_t tiles = (w.r0 + tiled_rows(m)) / 32 - w.r0 / 32;
    const int grid = tile_grid(gp.map64 != nullptr, nrb * ncb);
    mxn_gemm_kernel<0><<<grid, 64 * mxn::MW, 0, st>>>(w, A, m, n, c, ldc, nrb, ncb, tiles, gp, ep);
    if (mode == 1) {   // the lo codes' products, added into C behind the first launch
        Epi add;
        add.accumulate = 1;
        mxn_gemm_kernel<1><<<grid, 64 * mxn::MW, 0, st>>>(w, A, m, n, c, ldc, nrb, ncb, tiles, gp, add);
    }
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
