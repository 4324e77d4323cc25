// Activation quantizer kernels (jam's F1 and F2, bit-exact; lane math in quant.h) and the one-time
// weight repack into the device layout.
#include "common.h"
#include "launch.h"
#include "quant.h"

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
template <int DT>
__global__ void __launch_bounds__(256) repack_kernel(const uint8_t* __restrict__ raw, int64_t raw_stride,
                                                     int64_t rows, int64_t rb, int64_t G, uint8_t* __restrict__ qs,
                                                     uint8_t* __restrict__ sc) {
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
    } else if constexpr (DT == Q6_K) {                 // ql @0..127, qh @128..191, scales @192..207, d @208
        const uint8_t* b = row + g * 210;
        for (int c = 0; c < 13; c++)
            for (int t = 0; t < 16; t++) chunk(c)[t] = live ? b[16 * c + t] : 0;
        ds[0] = live ? b[208] : 0;
        ds[1] = live ? b[209] : 0;
    } else {
        for (int j = 0; j < BPG; j++) {
            const int64_t blk = g * BPG + j;
            uint8_t q[32] = {0}, s[2] = {0, 0};   // a block past the row end, or a padding row, stays zero
            if (live && blk < rb) {
                const uint8_t* b = row + blk * block_bytes(DT);
                const int sbytes = DT == MXFP4 ? 1 : 2, qbytes = DT == Q8_0 ? 32 : 16;
                for (int t = 0; t < sbytes; t++) s[t] = b[t];
                for (int t = 0; t < qbytes; t++) q[t] = b[sbytes + t];
            }
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
        if constexpr (DT == MXFP4) {                   // byte 8: the group's largest exponent; 9..15 zero
            uint8_t mx = 0;
            for (int j = 0; j < BPG; j++) mx = ds[j] > mx ? ds[j] : mx;
            ds[8] = mx;
            for (int t = 9; t < 16; t++) ds[t] = 0;
        }
    }
}

// ------------------------------------------------------------------------- matrix-core GEMM activations
// Position of element j of an 8-element run inside an A-operand fragment (its own inverse): the weight
// dequantization builds f16 pairs from bytes (0,2), (1,3), (4,6), (5,7) of two 32-bit words.
JAMHIP_DEV int perm8(int j) { return j == 1 ? 2 : j == 2 ? 1 : j == 5 ? 6 : j == 6 ? 5 : j; }

int gemm_sums_kind(int dt) { return dt == Q4_K || dt == Q4_0 ? 1 : dt == Q6_K ? 2 : 0; }

// One workgroup per (padded) token: jam's F2 quantization of every 32-element block (f2_lane, bit-exact),
// the codes scattered into the fragment order of GemmAct::b, then the token's power-of-two scale and the
// scaled block scales and sums. SK: 0 no sums, 1 per-32 sums xs0 + xs1 (jam's fl(xs0 + xs1)), 2 per-16.
// Grouped form (gmap non-null): slot t belongs to expert gmap[t / 64] (-1: padding) and holds that
// expert's row t - gpoff[e] (CSR row goff[e] + t - gpoff[e]) while that is below its row count.
template <int SK>
__global__ void __launch_bounds__(256) gemm_prep_kernel(const float* __restrict__ a, int lda, int n, int k, int Kp,
                                                        int NP, _Float16* __restrict__ bq, float* __restrict__ dx,
                                                        _Float16* __restrict__ shi, _Float16* __restrict__ slo,
                                                        float* __restrict__ es, const int* __restrict__ gmap,
                                                        const int* __restrict__ goff, const int* __restrict__ gpoff) {
    extern __shared__ float psm[];   // block scales [Kp/32], per-16 sums [Kp/16]
    __shared__ float red[4];
    const int t = blockIdx.x, nbp = Kp >> 5, nbk = k >> 5, e = threadIdx.x & 31;
    float* sdb = psm;
    float* sxs = psm + nbp;
    int src = t;
    bool live = t < n;
    if (gmap != nullptr) {
        const int ex = gmap[t >> 6];
        live = false;
        if (ex >= 0) {
            const int l = t - gpoff[ex];
            live = l < goff[ex + 1] - goff[ex];
            src = goff[ex] + l;
        }
    }
    for (int b = threadIdx.x >> 5; b < nbp; b += 8) {   // b is uniform in each 32-lane group
        const float x = live && b < nbk ? a[(int64_t) src * lda + 32 * b + e] : 0.0f;
        float db, xs16;
        const int v = f2_lane(x, db, xs16);
        const int q = e >> 4, ks = (e >> 3) & 1;
        bq[((int64_t) (2 * b + ks) * NP + t) * 16 + 8 * q + perm8(e & 7)] = (_Float16) v;
        if (e == 0) sdb[b] = db;
        if ((e & 15) == 0) sxs[2 * b + q] = xs16;
    }
    __syncthreads();
    float mx = 0.0f;
    if constexpr (SK == 1)
        for (int b = threadIdx.x; b < nbp; b += 256) mx = fmaxf(mx, fabsf(sxs[2 * b] + sxs[2 * b + 1]));
    if constexpr (SK == 2)
        for (int i = threadIdx.x; i < 2 * nbp; i += 256) mx = fmaxf(mx, fabsf(sxs[i]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int ex = 0;
    if (SK != 0 && mx > 0.0f && mx <= 3.0e38f) {   // zero or non-finite sums keep 2^0
        frexpf(mx, &ex);                         // mx < 2^ex
        ex -= 14;
    }
    const float down = ldexpf(1.0f, -ex);
    if (threadIdx.x == 0) es[t] = ldexpf(1.0f, ex);
    for (int b = threadIdx.x; b < nbp; b += 256) dx[(int64_t) b * NP + t] = sdb[b] * down;
    if constexpr (SK == 1) {
        for (int b = threadIdx.x; b < nbp; b += 256) {
            const float v = (sxs[2 * b] + sxs[2 * b + 1]) * down;
            const _Float16 h = (_Float16) v;
            const int64_t o = ((int64_t) (b >> 3) * NP + t) * 8 + (b & 7);
            shi[o] = h;
            slo[o] = (_Float16) (v - (float) h);
        }
    }
    if constexpr (SK == 2) {
        for (int i = threadIdx.x; i < 2 * nbp; i += 256) {
            const float v = sxs[i] * down;
            const _Float16 h = (_Float16) v;
            const int64_t o = ((int64_t) (i >> 4) * NP + t) * 16 + (i & 15);
            shi[o] = h;
            slo[o] = (_Float16) (v - (float) h);
        }
    }
}

static int64_t a256(int64_t v) { return (v + 255) & ~(int64_t) 255; }

size_t gemm_act_bytes_np(int dt, int NP, int k) {
    const int64_t Kp = (k + 255) / 256 * 256, sk = gemm_sums_kind(dt);
    const int64_t sb = sk == 0 ? 0 : a256((Kp / 256) * NP * (sk == 1 ? 8 : 16) * 2);
    return (size_t) (a256(Kp * NP * 2) + a256((Kp / 32) * NP * 4) + 2 * sb + a256((int64_t) NP * 4));
}
size_t gemm_act_bytes(int dt, int n, int k) { return gemm_act_bytes_np(dt, (n + 63) / 64 * 64, k); }

static hipError_t prep_np(int dt, const float* a, int lda, int n, int NP, int k, void* scratch, GemmAct* out,
                          const int* gmap, const int* goff, const int* gpoff, hipStream_t st) {
    const int Kp = (k + 255) / 256 * 256, sk = gemm_sums_kind(dt);
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
    *out = GemmAct{bq, dx, shi, slo, es, NP, Kp};
    const size_t lds = (size_t) (Kp / 32) * 12;
    if (lds > 64 * 1024) return hipErrorNotSupported;
    if (NP <= 0) return hipSuccess;
    if (sk == 1)
        gemm_prep_kernel<1><<<NP, 256, lds, st>>>(a, lda, n, k, Kp, NP, bq, dx, shi, slo, es, gmap, goff, gpoff);
    else if (sk == 2)
        gemm_prep_kernel<2><<<NP, 256, lds, st>>>(a, lda, n, k, Kp, NP, bq, dx, shi, slo, es, gmap, goff, gpoff);
    else
        gemm_prep_kernel<0><<<NP, 256, lds, st>>>(a, lda, n, k, Kp, NP, bq, dx, shi, slo, es, gmap, goff, gpoff);
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

hipError_t launch_repack(int dt, const uint8_t* raw, int64_t raw_stride, int64_t rows, int64_t rb, int64_t G,
                         uint8_t* qs, uint8_t* sc, hipStream_t st) {
    const int64_t n = tiled_rows(rows) * G;
    const dim3 grid((unsigned) ((n + 255) / 256));
    switch (dt) {
    case Q8_0: repack_kernel<Q8_0><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, G, qs, sc); break;
    case Q4_0: repack_kernel<Q4_0><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, G, qs, sc); break;
    case MXFP4: repack_kernel<MXFP4><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, G, qs, sc); break;
    case Q6_K: repack_kernel<Q6_K><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, G, qs, sc); break;
    case Q4_K: repack_kernel<Q4_K><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, G, qs, sc); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace jamhip
