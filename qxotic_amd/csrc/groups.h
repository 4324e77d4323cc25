// Device-side expert tables of the grouped matmul's fused preps (prep.hip, mxn.hip): every workgroup derives
// the CSR offsets and the 64-slot layout from the expert counts itself, so no separate offsets launch runs.
#pragma once
#include "common.h"
#include "launch.h"

namespace jamhip {

// Exclusive scans of (x, y) over the lanes of the first wave (wide false) or of the 256 lanes of the
// workgroup (wide true: every thread must call it; two barriers); lane e holds expert e; *tot = the sums.
JAMHIP_DEV int2 block_scan2(int x, int y, int2* tot, int2* sm, bool wide) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int sx = x, sy = y;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int ux = __shfl_up(sx, o), uy = __shfl_up(sy, o);
        if (lane >= o) sx += ux, sy += uy;
    }
    if (!wide) {
        *tot = make_int2(__shfl(sx, 63), __shfl(sy, 63));
        return make_int2(sx - x, sy - y);
    }
    if (lane == 63) sm[wave] = make_int2(sx, sy);
    __syncthreads();
    int bx = 0, by = 0, tx = 0, ty = 0;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const int2 v = sm[w];
        if (w < wave) bx += v.x, by += v.y;
        tx += v.x, ty += v.y;
    }
    __syncthreads();   // sm is reused by the next scan
    *tot = make_int2(tx, ty);
    return make_int2(bx + sx - x, by + sy - y);
}

// The fused grouped prep's expert table, from the expert counts on the device (one expert per thread: the
// first wave for up to 64 experts, else the workgroup). Expert e keeps c_e rows: its count, clamped so that
// the experts' rows fit rows_cap in expert order (rows past rows_cap are dropped, as by launch_moe_offsets);
// its C rows start at oc_e (exclusive scan of c), and an expert with rows owns roundup(c_e, 64) token slots
// from p_e (exclusive scan), so the slots [0, P) are all owned. Returns P. With pub set, also writes
// off[0..E] (and off_out), poff64[0..E] and map64[0..cap64) (the owner of each 64-slot block, -1 past the
// last). Every thread of the workgroup must call it.
struct SlotOwner {
    int oc = 0, c = 0, p64 = 0, a64 = 0;
};
JAMHIP_DEV int fused_scan(const PrepGroups& pg, bool pub, SlotOwner* so) {
    __shared__ int2 sm[4];
    __shared__ int ptot;
    const bool wide = pg.E > 64;   // up to 64 experts: the first wave alone
    if (wide || threadIdx.x < 64) {
        const int e = threadIdx.x, nt = wide ? 256 : 64;
        const bool in = e < pg.E;
        // min(count, rows_cap) changes no clamped count and keeps the scan within E·rows_cap
        const int c0 = in ? min(max(pg.counts[e], 0), pg.rows_cap) : 0;
        int2 tot;
        const int o = block_scan2(c0, 0, &tot, sm, wide).x;
        const int c = in ? max(0, min(c0, pg.rows_cap - o)) : 0;
        const int a64 = (c + 63) / 64 * 64;
        const int2 s = block_scan2(c, a64, &tot, sm, wide);
        const int oc = s.x, p64 = s.y;
        so->oc = oc, so->c = c, so->p64 = p64, so->a64 = a64;
        if (threadIdx.x == 0) ptot = tot.y;
        if (pub) {
            if (in) {
                pg.off[e] = oc;
                pg.poff64[e] = p64;
                if (pg.off_out != nullptr) pg.off_out[e] = oc;
                for (int i = p64 / 64; i < (p64 + a64) / 64 && i < pg.cap64; i++) pg.map64[i] = e;
            }
            if (e == 0) {
                pg.off[pg.E] = tot.x;
                pg.poff64[pg.E] = tot.y;
                if (pg.off_out != nullptr) pg.off_out[pg.E] = tot.x;
            }
            for (int i = tot.y / 64 + e; i < pg.cap64; i += nt) pg.map64[i] = -1;
        }
    }
    __syncthreads();
    return ptot;
}

// The CSR row of slot t (-1 for a padding slot) from this thread's expert (the thread whose expert owns t
// writes *own; every thread reads it after the barrier; a second barrier before *own is written again is the
// caller's). With pg.rows set, the row is the gathered source row pg.rows[r] / pg.rdiv instead.
JAMHIP_DEV void slot_owner_store(const PrepGroups& pg, const SlotOwner& so, int t, int* own, int* own_count) {
    if (so.a64 > 0 && t >= so.p64 && t < so.p64 + so.a64) {   // exactly one owner for t < P
        const int r = so.oc + (t - so.p64);
        *own = t - so.p64 < so.c ? (pg.rows != nullptr ? pg.rows[r] / pg.rdiv : r) : -1;
        if (own_count != nullptr) *own_count = so.c;
    }
}

}  // namespace jamhip
