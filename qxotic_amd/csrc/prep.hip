// Activation quantizer kernels (jam's F1 and F2, bit-exact; lane math in quant.h) and the one-time
// weight repack into the device layout.
#include "common.h"
#include "launch.h"
#include "quant.h"
#include "groups.h"

#include <atomic>

namespace jamhip {

// One lane per activation element; a 32-lane half-wave owns one 32-element block (quant.h).
// k % 32 == 0 is checked by the caller, so whole blocks retire together at the row end.
__global__ void __launch_bounds__(256) quant_f1_kernel(const float* __restrict__ a, int lda, int k,
                                                       int8_t* __restrict__ q, float* __restrict__ d,
                                                       float* __restrict__ asum, int* __restrict__ s16) {
    const int j = blockIdx.y;
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= k) return;
    float db;
    int h16, h32;
    const int v = f1_lane(a[(int64_t) j * lda + e], db, h16, h32);
    q[(int64_t) j * k + e] = (int8_t) v;
    if ((e & 15) == 0) s16[(int64_t) j * (k >> 4) + (e >> 4)] = h16;
    if ((e & 31) == 0) {
        d[(int64_t) j * (k >> 5) + (e >> 5)] = db;
        asum[(int64_t) j * (k >> 5) + (e >> 5)] = (float) h32;
    }
}

__global__ void __launch_bounds__(256) quant_f2_kernel(const float* __restrict__ a, int lda, int k,
                                                       int8_t* __restrict__ q, float* __restrict__ d,
                                                       float* __restrict__ xs) {
    const int j = blockIdx.y;
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= k) return;
    float db, s;
    const int v = f2_lane(a[(int64_t) j * lda + e], db, s);
    q[(int64_t) j * k + e] = (int8_t) v;
    if ((e & 15) == 0) xs[(int64_t) j * (k >> 4) + (e >> 4)] = s;
    if ((e & 31) == 0) d[(int64_t) j * (k >> 5) + (e >> 5)] = db;
}

// Weight repack: raw GGUF rows (stride raw_stride bytes, rb blocks) -> the row-tiled group layout of
// common.h. One thread per (tile, group, row of the tile), consecutive threads on consecutive rows so each
// chunk store of 32 threads fills 512 contiguous bytes; a group past the row's last block, and every row
// past `rows` in the last tile, is zero-filled. Runs once per pinned tensor.
//
// Q8_0, Q4_0 and MXFP4 groups are also checked for the matrix-core GEMM (mma.hip), which folds each block's
// scale into an f16 weight operand relative to a per-row, per-group reference: MXFP4 codes times
// 2^(e_b - e_ref + 1), Q4_0 / Q8_0 codes times d_b·2^s_r with s_r set by the group's largest fp16 exponent.
// That is exact while every folded operand is a normal f16 (>= 2^-14). A block whose products are zero
// whatever its scale (MXFP4: every code 0 or -0; Q8_0: every q 0) must not set the reference, or a large
// scale on it would push its neighbours below f16's range: such a block's scale is stored as 0 (MXFP4 e=0,
// Q8_0 d=0; its terms are zero on every path either way) and the reference comes from the other blocks. A
// Q4_0 block always counts (jam's n >= 8 term -fl(8d)·fl(xs0+xs1) does not vanish with the codes). A group
// whose blocks still span more than the f16 range below its reference (MXFP4 e_b < e_ref - 14; Q8_0
// |d_b| < 2^(F - 36), Q4_0 |d_b| < 2^(F - 39), F the largest fp16 exponent field), or that holds a non-finite
// scale (MXFP4 e = 255, which jam decodes as +Inf; an fp16 Inf/NaN), sets *flag: the host then keeps the
// tensor off the matrix cores, on kernels that apply every block scale in f32 as jam does.
template <int DT>
__global__ void __launch_bounds__(256) repack_kernel(const uint8_t* __restrict__ raw, int64_t raw_stride,
                                                     int64_t rows, int64_t rb, int64_t G, uint8_t* __restrict__ qs,
                                                     uint8_t* __restrict__ sc, int* __restrict__ flag) {
    constexpr int NC = group_chunks(DT), SB = group_scale_bytes(DT), BPG = blocks_per_group(DT);
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= tiled_rows(rows) * G) return;
    const int64_t rr = i & 31, tg = i >> 5, T = tg / G, g = tg - T * G, r = 32 * T + rr;
    const bool live = r < rows;
    const uint8_t* row = raw + (live ? r : 0) * raw_stride;
    uint8_t* dq = qs + (T * G + g) * (NC * CHUNK_STRIDE) + rr * 16;   // chunk c at dq + c·512
    uint8_t* ds = sc + (T * G + g) * (SB * ROW_TILE) + rr * SB;
    auto chunk = [&](int c) { return dq + (int64_t) c * CHUNK_STRIDE; };
    if constexpr (DT == Q4_K) {                        // d, dmin, scales @0..15, nibbles @16..143
        const uint8_t* b = row + g * 144;
        for (int t = 0; t < 16; t++) ds[t] = live ? b[t] : 0;
        for (int c = 0; c < 8; c++)
            for (int t = 0; t < 16; t++) chunk(c)[t] = live ? b[16 + 16 * c + t] : 0;
    } else if constexpr (DT == Q5_K) {                 // d, dmin, scales @0..15, qh @16..47, qs @48..175
        const uint8_t* b = row + g * 176;
        for (int t = 0; t < 16; t++) ds[t] = live ? b[t] : 0;
        for (int c = 0; c < 8; c++)
            for (int t = 0; t < 16; t++) chunk(c)[t] = live ? b[48 + 16 * c + t] : 0;
        for (int c = 0; c < 2; c++)
            for (int t = 0; t < 16; t++) chunk(8 + c)[t] = live ? b[16 + 16 * c + t] : 0;
    } else if constexpr (DT == NVFP4) {                // per 64-block: d[4] UE4M3 @0..3, qs @4..35
        for (int j = 0; j < 4; j++) {
            const int64_t blk = g * 4 + j;
            const bool in = live && blk < rb;
            const uint8_t* b = row + (in ? blk : 0) * 36;
            for (int t = 0; t < 4; t++) ds[4 * j + t] = in ? b[t] : 0;
            for (int h = 0; h < 2; h++)
                for (int t = 0; t < 16; t++) chunk(2 * j + h)[t] = in ? b[4 + 16 * h + t] : 0;
        }
    } else if constexpr (DT == Q1_0) {                 // per 128-block: fp16 d @0..1, sign bytes @2..17
        for (int j = 0; j < 2; j++) {
            const int64_t blk = g * 2 + j;
            const bool in = live && blk < rb;
            const uint8_t* b = row + (in ? blk : 0) * 18;
            ds[2 * j] = in ? b[0] : 0;
            ds[2 * j + 1] = in ? b[1] : 0;
            for (int t = 0; t < 16; t++) chunk(j)[t] = in ? b[2 + t] : 0;
            // a non-finite d keeps the tensor off the matrix cores, whose per-stage order of d's products
            // would turn jam's per-block Inf/NaN pattern into a different one
            if (flag != nullptr && (ds[2 * j + 1] & 0x7C) == 0x7C) atomicOr(flag, 1);
        }
    } else if constexpr (DT == Q6_K) {                 // ql @0..127, qh @128..191, scales @192..207, d @208
        const uint8_t* b = row + g * 210;
        for (int c = 0; c < 13; c++)
            for (int t = 0; t < 16; t++) chunk(c)[t] = live ? b[16 * c + t] : 0;
        ds[0] = live ? b[208] : 0;
        ds[1] = live ? b[209] : 0;
    } else {
        bool nz[BPG];   // the block has a code whose product is not zero
        for (int j = 0; j < BPG; j++) {
            const int64_t blk = g * BPG + j;
            uint8_t q[32] = {0}, s[2] = {0, 0};   // a block past the row end, or a padding row, stays zero
            if (live && blk < rb) {
                const uint8_t* b = row + blk * block_bytes(DT);
                const int sbytes = DT == MXFP4 ? 1 : 2, qbytes = DT == Q8_0 ? 32 : 16;
                for (int t = 0; t < sbytes; t++) s[t] = b[t];
                for (int t = 0; t < qbytes; t++) q[t] = b[sbytes + t];
            }
            uint8_t any = 0;   // Q8_0: any q != 0; MXFP4: any nibble other than +-0 (codes 0 and 8)
            for (int t = 0; t < 32; t++) any |= DT == MXFP4 ? (uint8_t) (q[t] & 0x77) : q[t];
            nz[j] = any != 0;
            if constexpr (DT == Q8_0) {                // d fp16 @0, q @2..33
                ds[2 * j] = s[0];
                ds[2 * j + 1] = s[1];
                for (int t = 0; t < 16; t++) {
                    chunk(2 * j)[t] = q[t];
                    chunk(2 * j + 1)[t] = q[16 + t];
                }
            } else if constexpr (DT == Q4_0) {         // d fp16 @0, nibbles @2..17
                ds[2 * j] = s[0];
                ds[2 * j + 1] = s[1];
                for (int t = 0; t < 16; t++) chunk(j)[t] = q[t];
            } else {                                   // MXFP4: e8m0 @0, nibbles @1..16
                ds[j] = s[0];
                for (int t = 0; t < 16; t++) chunk(j)[t] = q[t];
            }
        }
        bool bad = false;   // the matrix cores' folding would not be exact for this row's group
        if constexpr (DT == MXFP4) {   // byte 8: the reference exponent (largest of the counted blocks); 9..11
                                       // zero; 12..15: the f32 2^(e_ref - 128) that the matrix cores apply per group
            uint8_t er = 0;
            for (int j = 0; j < BPG; j++) {
                if (!nz[j] && ds[j] != 255) ds[j] = 0;
                er = ds[j] > er ? ds[j] : er;
                bad |= ds[j] == 255;
            }
            for (int j = 0; j < BPG; j++) bad |= nz[j] && (int) ds[j] + 14 < (int) er;
            ds[8] = er;
            for (int t = 9; t < 12; t++) ds[t] = 0;
            const uint32_t f = __builtin_bit_cast(uint32_t, e8m0_half(er));
            for (int t = 0; t < 4; t++) ds[12 + t] = (uint8_t) (f >> (8 * t));
        } else {
            uint32_t hs[BPG];
            int F = 0;   // largest fp16 exponent field of the group
            for (int j = 0; j < BPG; j++) {
                hs[j] = (uint32_t) ds[2 * j] | ((uint32_t) ds[2 * j + 1] << 8);
                if (DT == Q8_0 && !nz[j] && (hs[j] & 0x7C00u) != 0x7C00u) {
                    ds[2 * j] = ds[2 * j + 1] = 0;
                    hs[j] = 0;
                }
                const int f = (int) ((hs[j] >> 10) & 31);
                F = f > F ? f : F;
            }
            if (F == 31) {
                bad = true;
            } else {
                const float lim = ldexpf(1.0f, F - (DT == Q8_0 ? 36 : 39));
                for (int j = 0; j < BPG; j++) {
                    const float v = h2f(hs[j] & 0x7FFFu);
                    bad |= v != 0.0f && v < lim;
                }
            }
        }
        if (bad && flag != nullptr) atomicOr(flag, 1);
    }
}

__global__ void flag_clear_kernel(int* flag) { *flag = 0; }

// ------------------------------------------------------------------------- matrix-core GEMM activations
// Position of element j of an 8-element run inside an A-operand fragment (its own inverse): the weight
// dequantization builds f16 pairs from bytes (0,2), (1,3), (4,6), (5,7) of two 32-bit words.
JAMHIP_DEV int perm8(int j) { return j == 1 ? 2 : j == 2 ? 1 : j == 5 ? 6 : j == 6 ? 5 : j; }

int gemm_sums_kind(int dt) { return dt == Q4_K || dt == Q5_K || dt == Q4_0 || dt == Q1_0 ? 1 : dt == Q6_K ? 2 : 0; }

// A workgroup takes a group of SG token slots at a time (256 threads, a thread per 16-element half of a block
// of one slot, 128 / SG blocks per round; at most PREP_GRID workgroups, each looping over its XCD's share of
// the groups): jam's F2 quantization of the slots' activation rows (f2_lane's arithmetic, bit-exact; a block's
// two halves sit SG lanes apart and exchange their maxima), each half's codes stored as two 16-byte pieces of
// GemmAct::b's fragment order (with SG = 8 the eight slots of a group fill whole 128-byte lines), the block
// scales and per-16 sums parked in LDS together with each row's largest |sum| (SK 1: per-32 xs0 + xs1, jam's
// fl(xs0 + xs1); SK 2: per-16; SK 0: none); then each slot's power of two from that maximum and the scaled
// block scales and sums.
// Grouped form (gmap non-null): slot t belongs to expert gmap[t / 64] (-1: padding) and holds that
// expert's row t - gpoff[e] (CSR row goff[e] + t - gpoff[e]) while that is below its row count.
JAMHIP_DEV int prep_src(int t, int n, const int* gmap, const int* goff, const int* gpoff) {
    if (gmap == nullptr) return t < n ? t : -1;
    const int ex = gmap[t >> 6];
    if (ex < 0) return -1;
    const int l = t - gpoff[ex];
    return l < goff[ex + 1] - goff[ex] ? goff[ex] + l : -1;
}

template <int CTRL> JAMHIP_DEV float dppf(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// lane ^ SG's value (the other half of the thread's block in gemm_prep)
template <int SG> JAMHIP_DEV float pair_other(float v) {
    if constexpr (SG == 1) return dppf<0xB1>(v);         // quad_perm [1, 0, 3, 2]
    else if constexpr (SG == 8) return dppf<0x128>(v);   // row_ror:8 inside 16-lane rows
    else return __shfl_xor(v, SG);
}
constexpr int PREP_MAX_KP = 65536;   // LDS: Kp/32 + Kp/16 floats per slot
constexpr int PREP_SG_KP = 16384;    // groups of 8 slots up to this Kp (48 KB of LDS)
constexpr int PREP_GRID = 1024;      // a multiple of 8 (XCDs)

// F2 exactly as f2_lane: the block max over both halves, d = max/127, inv = 127/max, q = sat8(rne(x·inv))
// with NaN/overflow -> -128, and the per-16 sums in _mm512_reduce_add_ps's pairing (distance 8, 4, 2, 1),
// all inside the lane. A lane holds elements 16h..16h+15 of its block (half h), or for MXO elements
// 8h..8h+7 and 16+8h..16+8h+7: exactly the two (K-step, half) planes it stores.
// MXO: the MXFP4 element order (the GEMM converts a weight byte's two nibbles, elements e and e + 16 of the
// block, into one f16 pair): K-step 2·block + ks, half q, slot i holds element 8q + 4ks + i/2 + 16·(i % 2).
// ORD: the element order of the codes inside a K-step, matching the weight operand the GEMM builds:
//   0  elements 16q + 8ks + perm8(i)            (nibble / byte fields, Q4_K, Q5_K, Q6_K, Q4_0, Q8_0, Q1_0)
//   1  pairs (e, e + 16) of the 32-block         (MXFP4: a weight byte's two e2m1 codes)
//   2  pairs (u, u + 8) of each 16-element sub-block, K-step ks = sub-block ks of the block (NVFP4)
// f1all: jam's F1 quantization for every slot (NVFP4, whose only jam path is F1 at every n, jam.c:662-668).
template <int SK, int ORD, int SG>
__global__ void __launch_bounds__(256) gemm_prep(const float* __restrict__ a, int lda, int n, int k, int Kp, int NP,
                                                 _Float16* __restrict__ bq, float* __restrict__ dx,
                                                 _Float16* __restrict__ shi, _Float16* __restrict__ slo,
                                                 float* __restrict__ es, const int* __restrict__ gmap,
                                                 const int* __restrict__ goff, const int* __restrict__ gpoff, int vec,
                                                 PrepGroups pg, int f1all) {
    // LDS: per slot of the group [Kp/32] block scales and [Kp/16] per-16 sums, then [4][SG] wave maxima
    extern __shared__ float lsm[];
    __shared__ int own[2 * SG];      // fused grouped mode: each slot's source row and its expert's row count
    const int nbp = Kp >> 5;
    float* lmx = lsm + SG * 3 * nbp;
    const int nbk = k >> 5, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int s = lane % SG;          // the thread's slot in the group
    float* ldb = lsm + s * 3 * nbp;   // its block scales and sums
    float* lxs = ldb + nbp;
    // the slots that can hold rows: [0, n) dense, [0, P) fused grouped (P from the counts), all NP otherwise
    SlotOwner so;
    const int P = pg.counts != nullptr ? fused_scan(pg, blockIdx.x == 0, &so) : gmap != nullptr ? NP : n;
    // workgroup i runs on XCD i % 8: each XCD takes a contiguous run of the groups of SG slots (a multiple of
    // 8 slots), its workgroups the run's groups in turn, so that slots sharing an output line (the codes, block
    // scales and sums are token-interleaved) are written through one L2
    const int G = (P + SG - 1) / SG, rnd = 8 / SG;
    const int x = (int) (blockIdx.x % 8), nw = (int) (gridDim.x >> 3), PG8 = ((G + 7) / 8 + rnd - 1) / rnd * rnd;
    const int g_end = min((x + 1) * PG8, G);
    for (int g = x * PG8 + (int) (blockIdx.x >> 3); g < g_end; g += nw) {
        const int t0 = g * SG, t = t0 + s;
        // fused grouped mode (counts on the device): F1 codes for an expert of 1..7 rows, else F2
        int src, cnt = 8;
        if (pg.counts != nullptr) {
#pragma unroll
            for (int i = 0; i < SG; i++) slot_owner_store(pg, so, t0 + i, &own[2 * i], &own[2 * i + 1]);
            __syncthreads();
            src = t < P ? own[2 * s] : -1;
            cnt = own[2 * s + 1];
        } else {
            src = prep_src(t, n, gmap, goff, gpoff);
        }
        const bool f1 = f1all != 0 || (pg.counts != nullptr && cnt < 8);
        // one slot: its padding leaves it unwritten (the GEMM's token column for it is computed but never stored,
        // and no other column reads it); in a group of 8 every slot is written, a padding slot as a zero row, so
        // that each store covers whole 128-byte lines, and a group of padding slots only is skipped
        bool any = src >= 0;
        if (SG > 1) any = __syncthreads_or(any);
        if (any) {
            const int hh = (lane / SG) & 1;   // which half of its block the thread holds
            float m2 = 0.0f;
            typedef _Float16 half8 __attribute__((ext_vector_type(8)));
            // one 16-element half of one block per thread (the threads of slot s, 256 / SG of them, hold
            // consecutive halves; a block's two halves sit SG lanes apart): 128 / SG blocks per round of the
            // workgroup, two rounds' loads in flight (more measured no faster); blocks past k (up to Kp)
            // quantize zeros
            constexpr int BPR = 128 / SG, NU = 2;
            const float* row = a + (int64_t) (src >= 0 ? src : 0) * lda;
            for (int r0 = threadIdx.x / (2 * SG); r0 < nbp; r0 += NU * BPR) {
                float xr[NU][16];
#pragma unroll
                for (int u = 0; u < NU; u++) {
                    const int b = r0 + BPR * u;
#pragma unroll
                    for (int i = 0; i < 16; i++) xr[u][i] = 0.0f;
                    if (b < nbk && src >= 0 && ORD == 2) {   // elements 4hh.., 8+4hh.., 16+4hh.., 24+4hh.. (4 each)
                        const float* p0 = row + 32 * b + 4 * hh;
#pragma unroll
                        for (int v = 0; v < 4; v++) {
                            if (vec) {
                                const float4 f = *reinterpret_cast<const float4*>(p0 + 8 * v);
                                xr[u][4 * v + 0] = f.x, xr[u][4 * v + 1] = f.y, xr[u][4 * v + 2] = f.z, xr[u][4 * v + 3] = f.w;
                            } else {
#pragma unroll
                                for (int i = 0; i < 4; i++) xr[u][4 * v + i] = p0[8 * v + i];
                            }
                        }
                    } else if (b < nbk && src >= 0) {
                        // ORD 1: elements 8hh..8hh+7 and 16+8hh..16+8hh+7 (the order the GEMM pairs them in); else
                        // 16hh..16hh+15
                        constexpr bool MXO = ORD == 1;
                        const float* p0 = row + 32 * b + (MXO ? 8 * hh : 16 * hh);
                        const float* p1 = p0 + (MXO ? 16 : 8);
                        if (vec) {   // a and lda 16-byte aligned (the launcher checks)
#pragma unroll
                            for (int v = 0; v < 2; v++) {
                                const float4 f0 = *reinterpret_cast<const float4*>(p0 + 4 * v);
                                const float4 f1 = *reinterpret_cast<const float4*>(p1 + 4 * v);
                                xr[u][4 * v + 0] = f0.x, xr[u][4 * v + 1] = f0.y;
                                xr[u][4 * v + 2] = f0.z, xr[u][4 * v + 3] = f0.w;
                                xr[u][8 + 4 * v + 0] = f1.x, xr[u][8 + 4 * v + 1] = f1.y;
                                xr[u][8 + 4 * v + 2] = f1.z, xr[u][8 + 4 * v + 3] = f1.w;
                            }
                        } else {
#pragma unroll
                            for (int i = 0; i < 8; i++) xr[u][i] = p0[i], xr[u][8 + i] = p1[i];
                        }
                    }
                }
#pragma unroll
                for (int u = 0; u < NU; u++) {
                    const int b = r0 + BPR * u;
                    if (b >= nbp) break;   // the two halves of a block stay together: b is the same for both
                    const float* x = xr[u];
                    float mx = 0.0f;
#pragma unroll
                    for (int i = 0; i < 16; i++) mx = fmaxf(mx, fabsf(x[i]));
                    mx = fmaxf(mx, pair_other<SG>(mx));   // the block's other half
                    const float db = mx / 127.0f;
                    float qf[16];
                    if (f1) {
                        // F1 (jam_q8_0_requant, jam_kernels_generic.c:71-94): id = 1/d, q = clamp(rint(x·id));
                        // a NaN product lands on -128 like LONG_MIN does
                        const float id = db > 0.0f ? 1.0f / db : 0.0f;
#pragma unroll
                        for (int i = 0; i < 16; i++) qf[i] = fminf(fmaxf(rintf(x[i] * id), -128.0f), 127.0f);
                    } else {
                        const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
#pragma unroll
                        for (int i = 0; i < 16; i++) {
                            const float p = x[i] * inv;
                            const bool ok = p > -2147483648.0f && p < 2147483648.0f;
                            qf[i] = ok ? fminf(fmaxf(rintf(p), -128.0f), 127.0f) : -128.0f;
                        }
                    }
                    // the thread's two (K-step, half) planes: 8 f16 (16 bytes) each at the slot
#pragma unroll
                    for (int ks = 0; ks < 2; ks++) {
                        half8 hv;
#pragma unroll
                        for (int i = 0; i < 8; i++) {
                            if constexpr (ORD == 0) hv[perm8(i)] = (_Float16) qf[8 * ks + i];   // elements 16hh + 8ks + i
                            else if constexpr (ORD == 1) hv[2 * (i & 3) + (i >> 2)] = (_Float16) qf[8 * (i >> 2) + 4 * ks + (i & 3)];
                            // ORD 2: slot 2j = element 16ks + 4hh + j, slot 2j + 1 = element 16ks + 4hh + 8 + j
                            else hv[2 * (i & 3) + (i >> 2)] = (_Float16) qf[8 * ks + 4 * (i >> 2) + (i & 3)];
                        }
                        *reinterpret_cast<half8*>(bq + ((int64_t) (2 * (2 * b + ks) + hh) * NP + t) * 8) = hv;
                    }
                    if (hh == 0) ldb[b] = db;
                    if (SK != 0 && f1) {
                        // F1's offset terms take the integer code sums times d (Q4_K and Q4_0 fl(asum·ad) per
                        // 32, Q6_K's −32 per 16): the sums slot holds Σq·d, the 32-sum in the block's first half
                        float s16 = 0.0f;
#pragma unroll
                        for (int i = 0; i < 16; i++) s16 += qf[i];   // exact: |Σ| <= 2048
                        const float s32 = s16 + pair_other<SG>(s16);
                        const float xs = SK == 1 ? s32 * db : s16 * db;
                        lxs[2 * b + hh] = SK == 1 && hh == 1 ? 0.0f : xs;
                        m2 = fmaxf(m2, fabsf(xs));
                    } else if constexpr (SK != 0) {
                        // per-16 sum in _mm512_reduce_add_ps's pairing: distance 8, 4, 2, 1
                        float s8[8];
#pragma unroll
                        for (int i = 0; i < 8; i++) s8[i] = x[i] + x[i + 8];
#pragma unroll
                        for (int i = 0; i < 4; i++) s8[i] = s8[i] + s8[i + 4];
                        s8[0] = s8[0] + s8[2];
                        s8[1] = s8[1] + s8[3];
                        const float xs16 = s8[0] + s8[1];
                        lxs[2 * b + hh] = xs16;
                        const float other = pair_other<SG>(xs16);   // the block's other half
                        m2 = fmaxf(m2, SK == 1 ? fabsf(hh == 0 ? xs16 + other : other + xs16) : fabsf(xs16));
                    }
                }
            }
            if constexpr (SK != 0) {   // each slot's largest |sum| over its threads (lanes s, s + SG, ...)
#pragma unroll
                for (int o = 32; o >= SG; o >>= 1) m2 = fmaxf(m2, __shfl_xor(m2, o));
                if (lane < SG) lmx[wave * SG + lane] = m2;
            }
            __syncthreads();
            // a slot's power of two: the largest |sum| lands in [2^13, 2^14); zero or non-finite sums keep 2^0
            auto slot_exp = [&](int sl) {
                int ex = 0;
                if constexpr (SK != 0) {
                    const float mx = fmaxf(fmaxf(lmx[sl], lmx[SG + sl]), fmaxf(lmx[2 * SG + sl], lmx[3 * SG + sl]));
                    if (mx > 0.0f && mx <= 3.0e38f) {
                        frexpf(mx, &ex);
                        ex -= 14;
                    }
                }
                return ex;
            };
            if (threadIdx.x < SG && (SG > 1 || src >= 0)) es[t0 + threadIdx.x] = ldexpf(1.0f, slot_exp(threadIdx.x));
            auto put = [&](int64_t o, float v) {
                const F16Pair p = split_f16(v);
                shi[o] = p.hi;
                slo[o] = p.lo;
            };
            // block scales and sums of the group's slots, consecutive threads on consecutive slots (dx) or on
            // consecutive entries of a slot's 8 / 16 sums (shi, slo)
            for (int i = threadIdx.x; i < nbp * SG; i += 256) {
                const int sl = i % SG, b = i / SG;
                dx[(int64_t) b * NP + t0 + sl] = lsm[sl * 3 * nbp + b] * ldexpf(1.0f, -slot_exp(sl));
            }
            if constexpr (SK != 0) {
                constexpr int NS = SK == 1 ? 8 : 16;   // sums per slot and group of 8 blocks
                for (int i = threadIdx.x; i < (nbp / 8) * SG * NS; i += 256) {
                    const int c = i % NS, sl = (i / NS) % SG, gb = i / (NS * SG);
                    const float* xs = lsm + sl * 3 * nbp + nbp;
                    const float down = ldexpf(1.0f, -slot_exp(sl));
                    const int64_t o = ((int64_t) gb * NP + t0 + sl) * NS + c;
                    if constexpr (SK == 1) put(o, (xs[2 * (8 * gb + c)] + xs[2 * (8 * gb + c) + 1]) * down);
                    else put(o, xs[2 * (8 * gb) + c] * down);
                }
            }
        }
        __syncthreads();   // the LDS (and own) is the next group's
    }
}

static int64_t a256(int64_t v) { return (v + 255) & ~(int64_t) 255; }

// GemmAct buffers: codes, block scales, sums hi/lo, slot powers of two.
size_t gemm_act_bytes_np(int dt, int NP, int k) {
    const int64_t Kp = (k + 255) / 256 * 256, sk = gemm_sums_kind(dt);
    const int64_t sb = sk == 0 ? 0 : a256((Kp / 256) * NP * (sk == 1 ? 8 : 16) * 2);
    return (size_t) (a256(Kp * NP * 2) + a256((Kp / 32) * NP * 4) + 2 * sb + a256((int64_t) NP * 4));
}
size_t gemm_act_bytes(int dt, int n, int k) { return gemm_act_bytes_np(dt, (n + 63) / 64 * 64, k); }
bool gemm_prep_fits(int k) { return (k + 255) / 256 * 256 <= PREP_MAX_KP; }

static hipError_t prep_np(int dt, const float* a, int lda, int n, int NP, int k, void* scratch, GemmAct* out,
                          const int* gmap, const int* goff, const int* gpoff, hipStream_t st,
                          const PrepGroups& pg = PrepGroups{}) {
    const int Kp = (k + 255) / 256 * 256, sk = gemm_sums_kind(dt);
    if (Kp > PREP_MAX_KP) return hipErrorNotSupported;
    uint8_t* p = (uint8_t*) scratch;
    _Float16* bq = (_Float16*) p;
    p += a256((int64_t) Kp * NP * 2);
    float* dx = (float*) p;
    p += a256((int64_t) (Kp / 32) * NP * 4);
    const int64_t sb = sk == 0 ? 0 : a256((int64_t) (Kp / 256) * NP * (sk == 1 ? 8 : 16) * 2);
    _Float16* shi = (_Float16*) p;
    _Float16* slo = (_Float16*) (p + sb);
    p += 2 * sb;
    float* es = (float*) p;
    *out = GemmAct{bq, dx, shi, slo, es, NP, Kp, k};
    if (NP <= 0) return hipSuccess;
    const int vec = ((reinterpret_cast<uintptr_t>(a) & 15) == 0 && (lda & 3) == 0) ? 1 : 0;
    const int kind = dt == MXFP4 ? 3 : dt == NVFP4 ? 4 : sk;
    const int f1all = dt == NVFP4;
    // groups of 8 slots (every code store a whole 128-byte line) when that still gives a workgroup per CU
    const int sg = NP >= 8 * 256 && Kp <= PREP_SG_KP ? 8 : 1;
    const size_t lds = ((size_t) sg * 3 * (Kp / 32) + 4 * sg) * sizeof(float);
    // at most PREP_GRID workgroups (all resident), each looping over its XCD's groups
    const int ng = NP / sg;
    const unsigned grid = (unsigned) (ng < PREP_GRID ? ng : PREP_GRID);
    const void* fn;
#define JAMHIP_PREP_FN(SG) \
    fn = kind == 1 ? (const void*) gemm_prep<1, 0, SG> : kind == 2 ? (const void*) gemm_prep<2, 0, SG> \
       : kind == 3 ? (const void*) gemm_prep<0, 1, SG> : kind == 4 ? (const void*) gemm_prep<0, 2, SG> \
       : (const void*) gemm_prep<0, 0, SG>
    if (sg == 8) JAMHIP_PREP_FN(8);
    else JAMHIP_PREP_FN(1);
#undef JAMHIP_PREP_FN
    // the LDS limit is raised once per kernel; threads racing here both set the same value
    static std::atomic<bool> attr[2][5];
    if (!attr[sg == 8][kind].load(std::memory_order_acquire)) {
        const size_t mx = sg == 8 ? (size_t) 8 * 3 * (PREP_SG_KP / 32) + 32 : (size_t) 3 * (PREP_MAX_KP / 32) + 4;
        const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int) (mx * sizeof(float)));
        if (e != hipSuccess) return e;
        attr[sg == 8][kind].store(true, std::memory_order_release);
    }
#define JAMHIP_PREP(SK, ORD, SG) gemm_prep<SK, ORD, SG><<<grid, 256, lds, st>>>(a, lda, n, k, Kp, NP, bq, dx, shi, slo, es, \
                                                                           gmap, goff, gpoff, vec, pg, f1all)
#define JAMHIP_PREP_SG(SG)                      \
    if (kind == 1) JAMHIP_PREP(1, 0, SG);       \
    else if (kind == 2) JAMHIP_PREP(2, 0, SG);  \
    else if (kind == 3) JAMHIP_PREP(0, 1, SG);  \
    else if (kind == 4) JAMHIP_PREP(0, 2, SG);  \
    else JAMHIP_PREP(0, 0, SG)
    if (sg == 8) { JAMHIP_PREP_SG(8); }
    else { JAMHIP_PREP_SG(1); }
#undef JAMHIP_PREP_SG
#undef JAMHIP_PREP
    return hipGetLastError();
}

hipError_t launch_gemm_prep(int dt, const float* a, int lda, int n, int k, void* scratch, GemmAct* out,
                            hipStream_t st) {
    return prep_np(dt, a, lda, n, (n + 63) / 64 * 64, k, scratch, out, nullptr, nullptr, nullptr, st);
}

hipError_t launch_gemm_prep_grouped(int dt, const float* a, int lda, int k, const Groups& g, int cap64,
                                    void* scratch, GemmAct* out, hipStream_t st) {
    return prep_np(dt, a, lda, 0, cap64 * 64, k, scratch, out, g.map64, g.off, g.poff64, st);
}

hipError_t launch_gemm_prep_grouped_fused(int dt, const float* a, int lda, int k, const PrepGroups& pg,
                                          void* scratch, GemmAct* out, hipStream_t st) {
    if (pg.counts == nullptr || pg.E < 1 || pg.E > PREP_FUSED_MAX_E || pg.rows_cap < 0 || pg.cap64 < 1)
        return hipErrorInvalidValue;
    return prep_np(dt, a, lda, 0, pg.cap64 * 64, k, scratch, out, nullptr, nullptr, nullptr, st, pg);
}

// Host-to-device staging of jamhip_mm's activations by the shader cores: the pinned host buffer is read over
// the bus 16 bytes per thread (a handful of workgroups for a decode vector) and written to device memory.
__global__ void __launch_bounds__(256) stage_copy_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                         int64_t n16) {
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t) gridDim.x * 256) dst[i] = src[i];
}

hipError_t launch_stage_copy(const void* src, void* dst, size_t bytes, hipStream_t st) {
    const int64_t n16 = (int64_t) (bytes / 16);
    if (bytes % 16 || (reinterpret_cast<uintptr_t>(src) & 15) || (reinterpret_cast<uintptr_t>(dst) & 15))
        return hipErrorInvalidValue;
    if (n16 == 0) return hipSuccess;
    const int64_t blocks = (n16 + 255) / 256;
    stage_copy_kernel<<<(unsigned) (blocks < 64 ? blocks : 64), 256, 0, st>>>((const uint4*) src, (uint4*) dst, n16);
    return hipGetLastError();
}

hipError_t launch_quant_f1(const float* a, int lda, int n, int k, int8_t* q, float* d, float* asum, int* s16,
                           hipStream_t st) {
    dim3 grid((k + 255) / 256, n);
    quant_f1_kernel<<<grid, 256, 0, st>>>(a, lda, k, q, d, asum, s16);
    return hipGetLastError();
}

hipError_t launch_quant_f2(const float* a, int lda, int n, int k, int8_t* q, float* d, float* xs,
                           hipStream_t st) {
    dim3 grid((k + 255) / 256, n);
    quant_f2_kernel<<<grid, 256, 0, st>>>(a, lda, k, q, d, xs);
    return hipGetLastError();
}

// Dense weights: row r (rb elements of the raw row) to the device copy at pitch G bytes, the rest of the pitch
// zero. One thread per 16-byte piece of the pitch.
__global__ void __launch_bounds__(256) repack_dense_kernel(const uint8_t* __restrict__ raw, int64_t raw_stride,
                                                           int64_t rows, int64_t row_bytes, int64_t G,
                                                           uint8_t* __restrict__ dst) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x, per = G / 16;
    if (i >= rows * per) return;
    const int64_t r = i / per, o = (i - r * per) * 16;
    uint8_t v[16];
    const uint8_t* src = raw + r * raw_stride + o;
    for (int t = 0; t < 16; t++) v[t] = o + t < row_bytes ? src[t] : 0;
    uint8_t* d = dst + r * G + o;
    for (int t = 0; t < 16; t++) d[t] = v[t];
}

hipError_t launch_repack(int dt, const uint8_t* raw, int64_t raw_stride, int64_t rows, int64_t rb, int64_t G,
                         uint8_t* qs, uint8_t* sc, hipStream_t st, int* flag) {
    if (is_dense(dt)) {   // G: the pitch; rb: elements per row
        const int64_t n = rows * (G / 16);
        repack_dense_kernel<<<(unsigned) ((n + 255) / 256), 256, 0, st>>>(raw, raw_stride, rows, rb * block_bytes(dt), G,
                                                                          qs);
        return hipGetLastError();
    }
    if (flag != nullptr && (dt == Q8_0 || dt == Q4_0 || dt == MXFP4 || dt == Q1_0)) flag_clear_kernel<<<1, 1, 0, st>>>(flag);
    const int64_t n = tiled_rows(rows) * G;
    const dim3 grid((unsigned) ((n + 255) / 256));
    switch (dt) {
    case Q5_K: repack_kernel<Q5_K><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, G, qs, sc, nullptr); break;
    case NVFP4: repack_kernel<NVFP4><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, G, qs, sc, nullptr); break;
    case Q1_0: repack_kernel<Q1_0><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, G, qs, sc, flag); break;
    case Q8_0: repack_kernel<Q8_0><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, G, qs, sc, flag); break;
    case Q4_0: repack_kernel<Q4_0><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, G, qs, sc, flag); break;
    case MXFP4: repack_kernel<MXFP4><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, G, qs, sc, flag); break;
    case Q6_K: repack_kernel<Q6_K><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, G, qs, sc, nullptr); break;
    case Q4_K: repack_kernel<Q4_K><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, G, qs, sc, nullptr); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace jamhip
