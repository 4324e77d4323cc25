// jam's activation quantizers as per-lane device functions: lane e of a 32-lane group holds element e
// of one 32-element block (groups never straddle a 32-lane half of the wave, so every reduction below is
// an xor-shuffle inside the group). Used by the standalone quantizer kernels and by the fused decode
// GEMV. Only multiplies, divisions and adds of loaded values appear: nothing here can contract to FMA.
#pragma once

#include "common.h"

namespace jamhip {

// F1 (jam_q8_0_requant, jam/jam-native/src/kernels/jam_kernels_generic.c:71-94):
//   amax = max|x|; d = amax/127f; id = d > 0 ? 1f/d : 0; q = clamp(rint(x*id), -128, 127).
// Returns q; d, Σq over the lane's 16-half (s16) and over the block (s32) come back by reference.
JAMHIP_DEV int f1_lane(float x, float& db, int& s16, int& s32) {
    float amax = fabsf(x);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    db = amax / 127.0f;
    const float id = db > 0.0f ? 1.0f / db : 0.0f;
    // lrintf then clamp; a NaN product (only from non-finite input) lands on -128 like LONG_MIN does.
    const int v = (int) fminf(fmaxf(rintf(x * id), -128.0f), 127.0f);
    int s = v;
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o);
    s16 = s;
    s32 = s + __shfl_xor(s, 16);
    return v;
}

// F2 (quantize_row_q8s, jam/jam-native/src/kernels/jam_kernels_q4k_avx512.c:25-37):
//   d = max/127f; inv = max > 0 ? 127f/max : 0; q = sat8(rne(x*inv)), cvtps_epi32's NaN/overflow ->
//   INT_MIN -> -128; raw f32 Σx per 16 folded 8, 4, 2, 1 — _mm512_reduce_add_ps's pairing, so the
//   sums are bit-identical to jam's.
JAMHIP_DEV int f2_lane(float x, float& db, float& xs16) {
    float mx = fabsf(x);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    db = mx / 127.0f;
    const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
    const float p = x * inv;
    int v;
    if (!(p > -2147483648.0f && p < 2147483648.0f)) v = -128;
    else v = (int) fminf(fmaxf(rintf(p), -128.0f), 127.0f);
    float s = x;
    s = __shfl_xor(s, 8) + s;
    s = __shfl_xor(s, 4) + s;
    s = __shfl_xor(s, 2) + s;
    s = __shfl_xor(s, 1) + s;
    xs16 = s;
    return v;
}

}  // namespace jamhip
