// Device side of jinfer's CSR-grouped MoE dispatch (jinfer/jinfer-kernels/.../Moe.java:178-232) and the
// bookkeeping of the grouped matmul: per-expert counts -> CSR offsets (device prefix sum), the route ->
// slot assignment in dispatch's order, the row gather, and the prob-weighted combine in dispatch's
// expert order; and Moe.selectTopK's router top-k. Everything is deterministic: every sum in a fixed order, the
// only atomics integer counts.
#include "common.h"
#include "launch.h"

#include <type_traits>

#include <atomic>

namespace jamhip {

constexpr int MOE_THREADS = 1024;

// Exclusive scan of v over the workgroup's threads (v of thread i at position i), Hillis-Steele in LDS.
JAMHIP_DEV int block_exclusive_scan(int v, int* tmp) {
    const int t = threadIdx.x;
    tmp[t] = v;
    __syncthreads();
    for (int o = 1; o < MOE_THREADS; o <<= 1) {
        const int x = t >= o ? tmp[t - o] : 0;
        __syncthreads();
        tmp[t] += x;
        __syncthreads();
    }
    const int incl = tmp[t];
    __syncthreads();
    return incl - v;
}

// counts[E] (device, clamped to >= 0 and so that the total stays within rows_cap) -> off[E+1] (CSR row
// offsets), and for the experts with at least 8 rows (jam's band threshold, jam_kquant.h:23) the token
// slots of the matrix-core activation layout (poff64: each expert padded to 64 slots) and of the 8-token
// decode tiles (poff8), with the tile -> expert maps map64[cap64] / map8[cap8] (-1 = no expert), and the F1
// decode kernels' expert lists: small[0..n1) the experts with exactly one row, small[n1..n1 + n2) those with
// 2..7 rows, each in expert order and -1 past its last.
__global__ void __launch_bounds__(MOE_THREADS) moe_offsets_kernel(const int* __restrict__ counts, int E, int rows_cap,
                                                                 int* __restrict__ off, int* __restrict__ poff64,
                                                                 int* __restrict__ poff8, int* __restrict__ map64,
                                                                 int cap64, int* __restrict__ map8, int cap8,
                                                                 int* __restrict__ small, int n1, int n2) {
    __shared__ int tmp[MOE_THREADS];
    const int e = threadIdx.x;
    const int c0 = e < E ? min(max(counts[e], 0), rows_cap) : 0;   // changes no clamped count; no overflow
    const int o = block_exclusive_scan(c0, tmp);
    const int c = e < E ? max(0, min(c0, rows_cap - o)) : 0;   // rows past rows_cap are dropped
    const int oc = block_exclusive_scan(c, tmp);
    const int big = c >= 8;
    const int p64 = block_exclusive_scan(big ? (c + 63) / 64 * 64 : 0, tmp);
    const int p8 = block_exclusive_scan(big ? (c + 7) / 8 * 8 : 0, tmp);
    const int s1 = c == 1, r1 = block_exclusive_scan(s1, tmp);               // the F1 lists
    const int s2 = c >= 2 && c <= 7, r2 = block_exclusive_scan(s2, tmp);
    for (int i = e; i < cap64; i += MOE_THREADS) map64[i] = -1;
    for (int i = e; i < cap8; i += MOE_THREADS) map8[i] = -1;
    for (int i = e; i < n1 + n2; i += MOE_THREADS) small[i] = -1;
    __syncthreads();
    if (s1) small[r1] = e;        // r1 < n1: each listed expert holds a row
    if (s2) small[n1 + r2] = e;   // r2 < n2: each listed expert holds two or more
    if (e < E) {
        off[e] = oc;
        poff64[e] = p64;
        poff8[e] = p8;
        if (big) {
            for (int t = p64 / 64; t < (p64 + (c + 63) / 64 * 64) / 64 && t < cap64; t++) map64[t] = e;
            for (int t = p8 / 8; t < (p8 + (c + 7) / 8 * 8) / 8 && t < cap8; t++) map8[t] = e;
        }
        if (e == E - 1) {
            off[E] = oc + c;
            poff64[E] = p64 + (big ? (c + 63) / 64 * 64 : 0);
            poff8[E] = p8 + (big ? (c + 7) / 8 * 8 : 0);
        }
    }
}

// The same for E <= 64 in a single wave: the four exclusive scans are wave scans (shuffles, no barriers).
__global__ void __launch_bounds__(64) moe_offsets_wave_kernel(const int* __restrict__ counts, int E, int rows_cap,
                                                             int* __restrict__ off, int* __restrict__ poff64,
                                                             int* __restrict__ poff8, int* __restrict__ map64,
                                                             int cap64, int* __restrict__ map8, int cap8,
                                                             int* __restrict__ small, int n1, int n2) {
    const int e = threadIdx.x;
    const int c0 = e < E ? min(max(counts[e], 0), rows_cap) : 0;   // changes no clamped count; no overflow
    const int o = wave_exclusive_scan(c0);
    const int c = e < E ? max(0, min(c0, rows_cap - o)) : 0;   // rows past rows_cap are dropped
    const int oc = wave_exclusive_scan(c);
    const int big = c >= 8;
    const int a64 = big ? (c + 63) / 64 * 64 : 0, a8 = big ? (c + 7) / 8 * 8 : 0;
    const int p64 = wave_exclusive_scan(a64);
    const int p8 = wave_exclusive_scan(a8);
    const int s1 = c == 1, r1 = wave_exclusive_scan(s1);               // the F1 lists
    const int s2 = c >= 2 && c <= 7, r2 = wave_exclusive_scan(s2);
    for (int i = e; i < cap64; i += 64) map64[i] = -1;
    for (int i = e; i < cap8; i += 64) map8[i] = -1;
    for (int i = e; i < n1 + n2; i += 64) small[i] = -1;
    __syncthreads();
    if (s1) small[r1] = e;        // r1 < n1: each listed expert holds a row
    if (s2) small[n1 + r2] = e;   // r2 < n2: each listed expert holds two or more
    if (e < E) {
        off[e] = oc;
        poff64[e] = p64;
        poff8[e] = p8;
        if (big) {
            for (int t = p64 / 64; t < (p64 + a64) / 64 && t < cap64; t++) map64[t] = e;
            for (int t = p8 / 8; t < (p8 + a8) / 8 && t < cap8; t++) map8[t] = e;
        }
        if (e == E - 1) {
            off[E] = oc + c;
            poff64[E] = p64 + a64;
            poff8[E] = p8 + a8;
        }
    }
}

// Moe.dispatch's CSR build (Moe.java:188-206): counts per expert, off = exclusive prefix sum, then the
// routes in (s, k) order each take the next slot of their expert: slot_route[slot] = route index s·topk+k,
// route_slot[route] = slot. One workgroup of 16 waves over chunks of 1024 routes. Per chunk and wave, one
// ballot per expert gives every route its rank among the wave's earlier routes of the same expert
// (popcount below its lane) and the wave's count; a per-expert prefix over the waves plus the expert's
// running cursor then give the slot — the reference's cursor order, with no atomics. Two passes: counts,
// then slots. Routes naming an expert outside [0, E) take no slot (route_slot = -1).
constexpr int ROUTE_WAVES = MOE_THREADS / 64;
__global__ void __launch_bounds__(MOE_THREADS) moe_route_kernel(const int* __restrict__ route_expert, int R, int E,
                                                               int* __restrict__ counts, int* __restrict__ off,
                                                               int* __restrict__ slot_route, int* __restrict__ route_slot) {
    __shared__ int tmp[MOE_THREADS];
    extern __shared__ int wsm[];   // per-wave counts of the chunk [ROUTE_WAVES][E], then the cursors [E]
    int* wcnt = wsm;
    int* curs = wsm + ROUTE_WAVES * E;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint64_t below = (1ull << lane) - 1ull;
    int total = 0;
    for (int base = 0; base < R; base += MOE_THREADS) {   // pass 1: counts
        const int r = base + t;
        const int e = r < R ? route_expert[r] : -1;
        for (int x = 0; x < E; x++) {
            const uint64_t m = __ballot(e == x);
            if (lane == 0) wcnt[wave * E + x] = __popcll(m);
        }
        __syncthreads();
        if (t < E)
            for (int w = 0; w < ROUTE_WAVES; w++) total += wcnt[w * E + t];
        __syncthreads();
    }
    const int o = block_exclusive_scan(t < E ? total : 0, tmp);
    if (t < E) {
        counts[t] = total;
        off[t] = o;
        curs[t] = o;
        if (t == E - 1) off[E] = o + total;
    }
    __syncthreads();
    for (int base = 0; base < R; base += MOE_THREADS) {   // pass 2: slots
        const int r = base + t;
        const int e = r < R ? route_expert[r] : -1;
        int rank = 0;
        for (int x = 0; x < E; x++) {
            const uint64_t m = __ballot(e == x);
            if (e == x) rank = __popcll(m & below);
            if (lane == 0) wcnt[wave * E + x] = __popcll(m);
        }
        __syncthreads();
        if (r < R) {
            if (e >= 0 && e < E) {
                int pre = 0;
                for (int w = 0; w < wave; w++) pre += wcnt[w * E + e];
                const int slot = curs[e] + pre + rank;
                slot_route[slot] = r;
                route_slot[r] = slot;
            } else {
                route_slot[r] = -1;
            }
        }
        __syncthreads();
        if (t < E) {
            int cnt = 0;
            for (int w = 0; w < ROUTE_WAVES; w++) cnt += wcnt[w * E + t];
            curs[t] += cnt;
        }
        __syncthreads();
    }
}

// The same CSR build spread over chunks of 256 routes, for E <= 256 (two launches, still no atomics):
// moe_route_count_kernel writes each chunk's per-expert counts; moe_route_slot_kernel gives every chunk the
// totals, the experts' offsets (exclusive scan of the totals) and the counts of the chunks before it, so each
// route's slot is off[e] + (earlier chunks' routes of e) + (earlier waves' of the chunk) + (its rank in the
// wave): the same slots as the single-workgroup kernel.
constexpr int RCH = 256, RCH_WAVES = RCH / 64;
JAMHIP_DEV void chunk_wave_counts(int e, int E, int* wcnt, int* rank) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t below = (1ull << lane) - 1ull;
    for (int x = 0; x < E; x++) {
        const uint64_t m = __ballot(e == x);
        if (e == x) *rank = __popcll(m & below);
        if (lane == 0) wcnt[wave * E + x] = __popcll(m);
    }
}
__global__ void __launch_bounds__(RCH) moe_route_count_kernel(const int* __restrict__ route_expert, int R, int E,
                                                             int* __restrict__ ccnt) {
    __shared__ int wcnt[RCH_WAVES * 256];
    const int r = blockIdx.x * RCH + threadIdx.x;
    const int e = r < R ? route_expert[r] : -1;
    int rank = 0;
    chunk_wave_counts(e, E, wcnt, &rank);
    __syncthreads();
    if (threadIdx.x < E) {
        int s = 0;
        for (int w = 0; w < RCH_WAVES; w++) s += wcnt[w * E + threadIdx.x];
        ccnt[(int64_t) blockIdx.x * E + threadIdx.x] = s;
    }
}
// Chunk blockIdx.x's slots from expert e's total (thread e) and its routes in the chunks before this one.
JAMHIP_DEV void chunk_slots(const int* __restrict__ route_expert, int R, int E, int total, int before,
                            int* __restrict__ counts, int* __restrict__ off, int* __restrict__ slot_route,
                            int* __restrict__ route_slot) {
    __shared__ int wcnt[RCH_WAVES * 256], base[256], scan[RCH];
    const int t = threadIdx.x, wave = t >> 6;
    // exclusive scan of the totals over the experts: one wave's shuffles for up to 64 experts (no barrier),
    // else Hillis-Steele in LDS
    int oe = 0;
    if (E <= 64) {
        if (t < 64) oe = wave_exclusive_scan(t < E ? total : 0);
    } else {
        scan[t] = t < E ? total : 0;
        __syncthreads();
        for (int o = 1; o < RCH; o <<= 1) {
            const int x = t >= o ? scan[t - o] : 0;
            __syncthreads();
            scan[t] += x;
            __syncthreads();
        }
        oe = scan[t] - (t < E ? total : 0);
    }
    if (t < E) {
        base[t] = oe + before;
        if (blockIdx.x == 0) {
            counts[t] = total;
            off[t] = oe;
            if (t == E - 1) off[E] = oe + total;
        }
    }
    const int r = blockIdx.x * RCH + t;
    const int e = r < R ? route_expert[r] : -1;
    int rank = 0;
    chunk_wave_counts(e, E, wcnt, &rank);
    __syncthreads();
    if (r < R) {
        if (e >= 0 && e < E) {
            int pre = 0;
            for (int w = 0; w < wave; w++) pre += wcnt[w * E + e];
            const int slot = base[e] + pre + rank;
            slot_route[slot] = r;
            route_slot[r] = slot;
        } else {
            route_slot[r] = -1;
        }
    }
}
__global__ void __launch_bounds__(RCH) moe_route_slot_kernel(const int* __restrict__ route_expert, int R, int E,
                                                            const int* __restrict__ ccnt, int nch,
                                                            int* __restrict__ counts, int* __restrict__ off,
                                                            int* __restrict__ slot_route, int* __restrict__ route_slot) {
    int total = 0, before = 0;
    if (threadIdx.x < E)
        for (int c = 0; c < nch; c++) {
            const int v = ccnt[(int64_t) c * E + threadIdx.x];
            total += v;
            before += c < (int) blockIdx.x ? v : 0;
        }
    chunk_slots(route_expert, R, E, total, before, counts, off, slot_route, route_slot);
}
// One launch for up to ROUTE_FUSED_MAX routes: every chunk's workgroup counts all routes itself (integer LDS
// atomics: the totals, and the routes before its chunk), then takes its chunk's slots as above.
constexpr int ROUTE_FUSED_MAX = 16384;
__global__ void __launch_bounds__(RCH) moe_route_fused_kernel(const int* __restrict__ route_expert, int R, int E,
                                                             int* __restrict__ counts, int* __restrict__ off,
                                                             int* __restrict__ slot_route, int* __restrict__ route_slot) {
    __shared__ int tot[256], bef[256];
    const int t = threadIdx.x, lim = (int) blockIdx.x * RCH;
    tot[t] = 0;
    bef[t] = 0;
    __syncthreads();
    for (int r = t; r < R; r += RCH) {
        const int e = route_expert[r];
        if (e >= 0 && e < E) {
            atomicAdd(&tot[e], 1);
            if (r < lim) atomicAdd(&bef[e], 1);
        }
    }
    __syncthreads();
    chunk_slots(route_expert, R, E, t < E ? tot[t] : 0, t < E ? bef[t] : 0, counts, off, slot_route, route_slot);
}

// The same CSR build for at most 64 routes and 64 experts (decode-time MoE) in one wave, with no barrier:
// lane l holds route l (expert e_l) and expert l's count. One ballot per expert gives the count (popcount)
// and each route its rank among the earlier routes of its expert (popcount below its lane); a wave scan of
// the counts gives off, so route l's slot is off[e_l] + rank: Moe.dispatch's cursor order.
__global__ void __launch_bounds__(64) moe_route_wave_kernel(const int* __restrict__ route_expert, int R, int E,
                                                           int* __restrict__ counts, int* __restrict__ off,
                                                           int* __restrict__ slot_route, int* __restrict__ route_slot) {
    const int lane = threadIdx.x;
    const uint64_t below = (1ull << lane) - 1ull;
    const int e = lane < R ? route_expert[lane] : -1;
    int cnt = 0, rank = 0;
    for (int x = 0; x < E; x++) {
        const uint64_t m = __ballot(e == x);
        if (lane == x) cnt = __popcll(m);
        if (e == x) rank = __popcll(m & below);
    }
    const int o = wave_exclusive_scan(cnt);   // lanes past E hold count 0
    if (lane < E) {
        counts[lane] = cnt;
        off[lane] = o;
        if (lane == E - 1) off[E] = o + cnt;
    }
    const int oe = __shfl(o, e >= 0 && e < E ? e : 0);
    if (lane < R) {
        if (e >= 0 && e < E) {
            slot_route[oe + rank] = lane;
            route_slot[lane] = oe + rank;
        } else {
            route_slot[lane] = -1;
        }
    }
}

// Moe.dispatch's gather (Moe.java:214-222): g[slot] = x[slot_route[slot] / topk] (dim floats per row).
// Slots past off[E] (routes with an expert id outside [0, E) leave them unassigned) are not written. V4:
// rows copied as float4 (the launcher checks 16-byte alignment of both rows and dim % 4 == 0).
template <bool V4>
__global__ void __launch_bounds__(256) moe_gather_kernel(const float* __restrict__ x, int ldx,
                                                        const int* __restrict__ slot_route,
                                                        const int* __restrict__ off, int E, int topk, int dim,
                                                        float* __restrict__ g, int ldg) {
    const int slot = blockIdx.x;
    if (slot >= off[E]) return;
    const int s = slot_route[slot] / topk;
    const float* src = x + (int64_t) s * ldx;
    float* dst = g + (int64_t) slot * ldg;
    if constexpr (V4) {
        for (int i = threadIdx.x; i < dim / 4; i += 256)
            reinterpret_cast<float4*>(dst)[i] = reinterpret_cast<const float4*>(src)[i];
    } else {
        for (int i = threadIdx.x; i < dim; i += 256) dst[i] = src[i];
    }
}

// Moe.dispatch's weighted scatter-add (Moe.java:208, 223-231): out is zero-filled, then every expert in
// ascending order adds prob·y to its rows with one fused multiply-add (Ops.saxpyInPlace's fma,
// Ops.java:688-725). Here each output row sums its own routes, sorted by (expert, k) — the order in
// which the expert loop reaches them — so the result is bit-identical and needs no atomics. The row's
// routes are loaded once into LDS; one thread drops the ones without a slot and sorts the rest (stable
// insertion sort on the expert id) into (slot, prob) lists; then every thread runs the fma chain for its
// columns (four at a time when V4: rows 16-byte aligned, dim % 4 == 0). Workgroup column blockIdx.y takes
// every gridDim.y-th 256-column piece (few tokens: several workgroups per token, one piece each).
template <bool V4>
__global__ void __launch_bounds__(256) moe_combine_kernel(const float* __restrict__ y, int ldy,
                                                         const int* __restrict__ route_expert,
                                                         const float* __restrict__ route_prob,
                                                         const int* __restrict__ route_slot, int seq, int topk,
                                                         int E, int dim, float* __restrict__ out, int ldo) {
    __shared__ int r_ex[16], r_slot[16], l_ex[16], l_slot[16];
    __shared__ float r_prob[16], l_prob[16];
    __shared__ int l_n;
    const int s = blockIdx.x;
    if (s >= seq) return;
    const int kk = topk < 16 ? topk : 16;
    if (threadIdx.x < kk) {
        r_ex[threadIdx.x] = route_expert[s * topk + threadIdx.x];
        r_slot[threadIdx.x] = route_slot[s * topk + threadIdx.x];
        r_prob[threadIdx.x] = route_prob[s * topk + threadIdx.x];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int nv = 0;
        for (int k = 0; k < kk; k++) {
            const int e = r_ex[k], sl = r_slot[k];
            if (e < 0 || e >= E || sl < 0) continue;
            int b = nv - 1;   // insert after every kept route with a smaller or equal expert id (stable)
            while (b >= 0 && l_ex[b] > e) {
                l_ex[b + 1] = l_ex[b];
                l_slot[b + 1] = l_slot[b];
                l_prob[b + 1] = l_prob[b];
                b--;
            }
            l_ex[b + 1] = e;
            l_slot[b + 1] = sl;
            l_prob[b + 1] = r_prob[k];
            nv++;
        }
        l_n = nv;
    }
    __syncthreads();
    const int nv = l_n;
    float* o = out + (int64_t) s * ldo;
    if constexpr (V4) {
        for (int i = threadIdx.x + 256 * blockIdx.y; i < dim / 4; i += 256 * gridDim.y) {
            float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            for (int j = 0; j < nv; j++) {
                const float p = l_prob[j];
                const float4 v = reinterpret_cast<const float4*>(y + (int64_t) l_slot[j] * ldy)[i];
                acc.x = fmaf(p, v.x, acc.x);
                acc.y = fmaf(p, v.y, acc.y);
                acc.z = fmaf(p, v.z, acc.z);
                acc.w = fmaf(p, v.w, acc.w);
            }
            reinterpret_cast<float4*>(o)[i] = acc;
        }
    } else {
        for (int i = threadIdx.x + 256 * blockIdx.y; i < dim; i += 256 * gridDim.y) {
            float acc = 0.0f;
            for (int j = 0; j < nv; j++) acc = fmaf(l_prob[j], y[(int64_t) l_slot[j] * ldy + i], acc);
            o[i] = acc;
        }
    }
}

hipError_t launch_moe_offsets(const int* counts, int E, int rows_cap, int* off, int* poff64, int* poff8, int* map64,
                              int cap64, int* map8, int cap8, int* small, int n1, int n2, hipStream_t st) {
    if (E < 1 || E > MOE_THREADS) return hipErrorNotSupported;
    if (rows_cap < 0 || n1 < (E < rows_cap ? E : rows_cap) || n2 < (E < rows_cap / 2 ? E : rows_cap / 2))
        return hipErrorInvalidValue;
    if (E <= 64)
        moe_offsets_wave_kernel<<<1, 64, 0, st>>>(counts, E, rows_cap, off, poff64, poff8, map64, cap64, map8, cap8,
                                                  small, n1, n2);
    else
        moe_offsets_kernel<<<1, MOE_THREADS, 0, st>>>(counts, E, rows_cap, off, poff64, poff8, map64, cap64, map8, cap8,
                                                      small, n1, n2);
    return hipGetLastError();
}

size_t moe_route_scratch_ints(int R, int E) { return E <= 256 && R > RCH ? (size_t) ((R + RCH - 1) / RCH) * E : 0; }

hipError_t launch_moe_route(const int* route_expert, int R, int E, int* counts, int* off, int* slot_route,
                            int* route_slot, hipStream_t st, int* scratch) {
    if (E < 1 || E > MOE_THREADS) return hipErrorNotSupported;
    if (R <= 64 && E <= 64) {   // one wave
        moe_route_wave_kernel<<<1, 64, 0, st>>>(route_expert, R, E, counts, off, slot_route, route_slot);
        return hipGetLastError();
    }
    if (R > RCH && R <= ROUTE_FUSED_MAX && E <= 256) {   // chunked, one launch
        moe_route_fused_kernel<<<(R + RCH - 1) / RCH, RCH, 0, st>>>(route_expert, R, E, counts, off, slot_route,
                                                                    route_slot);
        return hipGetLastError();
    }
    if (scratch != nullptr && moe_route_scratch_ints(R, E) > 0) {   // chunked: R > 256 routes, E <= 256
        const int nch = (R + RCH - 1) / RCH;
        moe_route_count_kernel<<<nch, RCH, 0, st>>>(route_expert, R, E, scratch);
        moe_route_slot_kernel<<<nch, RCH, 0, st>>>(route_expert, R, E, scratch, nch, counts, off, slot_route, route_slot);
        return hipGetLastError();
    }
    const size_t lds = (size_t) (ROUTE_WAVES + 1) * E * sizeof(int);
    static std::atomic<bool> attr{false};   // threads racing here both set the same value
    if (!attr.load(std::memory_order_acquire)) {
        const hipError_t e = hipFuncSetAttribute((const void*) moe_route_kernel,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (ROUTE_WAVES + 1) * MOE_THREADS * (int) sizeof(int));
        if (e != hipSuccess) return e;
        attr.store(true, std::memory_order_release);
    }
    moe_route_kernel<<<1, MOE_THREADS, lds, st>>>(route_expert, R, E, counts, off, slot_route, route_slot);
    return hipGetLastError();
}

static bool rows16(const float* p, int ld, int dim) {
    return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && (ld & 3) == 0 && (dim & 3) == 0;
}

hipError_t launch_moe_gather(const float* x, int ldx, const int* slot_route, const int* off, int E, int R, int topk,
                             int dim, float* g, int ldg, hipStream_t st) {
    if (R <= 0) return hipSuccess;
    if (rows16(x, ldx, dim) && rows16(g, ldg, dim))
        moe_gather_kernel<true><<<R, 256, 0, st>>>(x, ldx, slot_route, off, E, topk, dim, g, ldg);
    else
        moe_gather_kernel<false><<<R, 256, 0, st>>>(x, ldx, slot_route, off, E, topk, dim, g, ldg);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------ top-k
// jinfer's Moe.selectTopK (Moe.java:76-127), one wave per router row, the row's scores in registers (EPL per
// lane, expert e in lane e % 64, slot e / 64). Each of the k passes takes the lane's first strict maximum in
// ascending expert order, then the wave's largest value with the lowest expert on ties: the first maximum, as
// the Java loop's strict `>` keeps it; NaN never wins, and a row with nothing above -Inf picks expert 0 (the
// loop's initial best). The winner's owner lane reads its combine weight (from the registers in the
// one-source form, so a masked entry reads as -Inf exactly as in the Java array; from `wts` in the two-source
// form) and masks the score to -Inf in registers and in `sel`, which the call consumes like jinfer does.
// Lane 0 then runs the row's weight step sequentially in jinfer's f32 order: gpt-oss's softmax over the k
// selected logits times expertWeightsScale (GptOss.java:320-345: Math.max with NaN propagation, the exp in
// double rounded to f32, a sequential f32 sum, 1/sum or 0), or Moe.normalizeTopP (Moe.java:146-152), then
// Moe.dispatch's expertScale fold (Moe.java:187-203), and writes the row's routes in (token, k) order. counts
// (zeroed by the launcher) take one atomic add per route.
template <int EPL>
__global__ void __launch_bounds__(256) moe_topk_kernel(float* __restrict__ sel, const float* wts, int rows, int E,
                                                       int ld, int topk, int mode, float wscale,
                                                       const float* __restrict__ escale, int* __restrict__ route_expert,
                                                       float* __restrict__ route_prob, int* __restrict__ counts) {
    __shared__ float sp[4][MOE_TOPK_MAX];
    __shared__ int se[4][MOE_TOPK_MAX];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int row = blockIdx.x * 4 + wv;
    if (row >= rows) return;   // the whole wave
    float* srow = sel + (int64_t) row * ld;
    const bool one = wts == sel;
    float v[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + 64 * j;
        v[j] = e < E ? srow[e] : -INFINITY;
    }
    for (int ki = 0; ki < topk; ki++) {
        float bv = -INFINITY;
        int bi = INT_MAX;
#pragma unroll
        for (int j = 0; j < EPL; j++)
            if (v[j] > bv) {
                bv = v[j];
                bi = lane + 64 * j;
            }
        // the wave's largest value, lowest expert on ties, by DPP steps (quad swaps, then rotations by 4 and 8
        // inside each 16-lane row, then each row's result passed on by row_bcast:15 / :31): lane 63 holds it
        auto take = [&](float ov, int oi) {
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        };
        auto dpp_step = [&](auto C, auto RM) {
            constexpr int ctrl = decltype(C)::value, row_mask = decltype(RM)::value;
            const int vb = __builtin_bit_cast(int, bv);
            const float ov = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(vb, vb, ctrl, row_mask, 0xF, false));
            const int oi = __builtin_amdgcn_update_dpp(bi, bi, ctrl, row_mask, 0xF, false);
            take(ov, oi);
        };
        using I = std::integral_constant<int, 0xF>;
        dpp_step(std::integral_constant<int, 0xB1>{}, I{});               // quad_perm [1, 0, 3, 2]
        dpp_step(std::integral_constant<int, 0x4E>{}, I{});               // quad_perm [2, 3, 0, 1]
        dpp_step(std::integral_constant<int, 0x124>{}, I{});              // row_ror:4
        dpp_step(std::integral_constant<int, 0x128>{}, I{});              // row_ror:8
        dpp_step(std::integral_constant<int, 0x142>{}, std::integral_constant<int, 0xA>{});   // row_bcast:15
        dpp_step(std::integral_constant<int, 0x143>{}, std::integral_constant<int, 0xC>{});   // row_bcast:31
        bi = __builtin_amdgcn_readlane(bi, 63);
        const int best = bi == INT_MAX || bi < 0 || bi >= E ? 0 : bi;
        float pw = 0.0f;
        if (lane == (best & 63)) {
#pragma unroll
            for (int j = 0; j < EPL; j++)
                if (j == (best >> 6)) {
                    pw = one ? v[j] : wts[(int64_t) row * ld + best];
                    v[j] = -INFINITY;
                }
            srow[best] = -INFINITY;
            sp[wv][ki] = pw;
            se[wv][ki] = best;
            if (counts != nullptr) atomicAdd(&counts[best], 1);
        }
        __builtin_amdgcn_wave_barrier();
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // softmax: lane i < topk takes the exp of the i-th logit (the double exp is the long part), then lane 0 runs
    // the rest in order
    if (mode == MOE_TOPK_SOFTMAX && lane < topk) {
        float mx = -INFINITY;
        for (int i = 0; i < topk; i++) {
            const float q = sp[wv][i];
            mx = (isnan(mx) || isnan(q)) ? __builtin_nanf("") : fmaxf(mx, q);
        }
        const float ex = (float) exp((double) __fsub_rn(sp[wv][lane], mx));
        __builtin_amdgcn_wave_barrier();   // every lane has read sp before lane i overwrites entry i
        sp[wv][lane] = ex;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane != 0) return;
    // loops unrolled over the maximum with a guard, so p stays in registers; each runs i = 0, 1, ... in order
    float p[MOE_TOPK_MAX];
#pragma unroll
    for (int i = 0; i < MOE_TOPK_MAX; i++) p[i] = i < topk ? sp[wv][i] : 0.0f;
    if (mode == MOE_TOPK_SOFTMAX) {
        float total = 0.0f;
#pragma unroll
        for (int i = 0; i < MOE_TOPK_MAX; i++)
            if (i < topk) total = __fadd_rn(total, p[i]);   // p[i] = exp(logit_i - max), from lane i
        const float inv = total == 0.0f ? 0.0f : __fdiv_rn(1.0f, total);
#pragma unroll
        for (int i = 0; i < MOE_TOPK_MAX; i++) p[i] = __fmul_rn(__fmul_rn(p[i], inv), wscale);
    } else if (mode == MOE_TOPK_NORMALIZE) {
        float total = 0.0f;
#pragma unroll
        for (int i = 0; i < MOE_TOPK_MAX; i++)
            if (i < topk) total = __fadd_rn(total, p[i]);
#pragma unroll
        for (int i = 0; i < MOE_TOPK_MAX; i++) p[i] = __fdiv_rn(p[i], total);
    }
#pragma unroll
    for (int i = 0; i < MOE_TOPK_MAX; i++)
        if (i < topk) {
            const int e = se[wv][i];
            route_expert[(int64_t) row * topk + i] = e;
            route_prob[(int64_t) row * topk + i] = escale != nullptr ? __fmul_rn(p[i], escale[e]) : p[i];
        }
}

__global__ void moe_fill_int_kernel(int* __restrict__ p, int n, int v) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = v;
}

hipError_t launch_moe_topk(float* sel, const float* wts, int rows, int E, int ld, int topk, int mode, float wscale,
                           const float* escale, int* route_expert, float* route_prob, int* counts, hipStream_t st) {
    if (E < 1 || E > 1024 || topk < 1 || topk > MOE_TOPK_MAX || rows < 0 || ld < E) return hipErrorInvalidValue;
    if (counts != nullptr) moe_fill_int_kernel<<<(E + 255) / 256, 256, 0, st>>>(counts, E, 0);
    if (rows == 0) return hipGetLastError();
    const dim3 grid((unsigned) ((rows + 3) / 4));
#define JAMHIP_TOPK(EPL) moe_topk_kernel<EPL><<<grid, 256, 0, st>>>(sel, wts ? wts : sel, rows, E, ld, topk, mode, \
                                                                     wscale, escale, route_expert, route_prob, counts)
    if (E <= 64) JAMHIP_TOPK(1);
    else if (E <= 128) JAMHIP_TOPK(2);
    else if (E <= 256) JAMHIP_TOPK(4);
    else if (E <= 512) JAMHIP_TOPK(8);
    else JAMHIP_TOPK(16);
#undef JAMHIP_TOPK
    return hipGetLastError();
}

hipError_t launch_moe_combine(const float* y, int ldy, const int* route_expert, const float* route_prob,
                              const int* route_slot, int seq, int topk, int E, int dim, float* out, int ldo,
                              hipStream_t st) {
    if (topk > 16) return hipErrorNotSupported;
    if (seq <= 0) return hipSuccess;
    const bool v4 = rows16(y, ldy, dim) && rows16(out, ldo, dim);
    // below 256 tokens a token's columns are split over up to 64 workgroups of 256 threads (one piece each)
    const int pieces = ((v4 ? dim / 4 : dim) + 255) / 256;
    const dim3 grid((unsigned) seq, (unsigned) (seq >= 256 ? 1 : pieces < 64 ? (pieces > 0 ? pieces : 1) : 64));
    if (v4)
        moe_combine_kernel<true><<<grid, 256, 0, st>>>(y, ldy, route_expert, route_prob, route_slot, seq, topk, E, dim,
                                                       out, ldo);
    else
        moe_combine_kernel<false><<<grid, 256, 0, st>>>(y, ldy, route_expert, route_prob, route_slot, seq, topk, E, dim,
                                                        out, ldo);
    return hipGetLastError();
}

}  // namespace jamhip
