// Shared device/host definitions for the jamhip kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jamhip {

// ggml / jam dtype tags (jam/jam-native/include/jam.h:59-77).
enum Dtype : int {
    F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14, BF16 = 30, MXFP4 = 39, NVFP4 = 40, Q1_0 = 41
};

// GGUF block geometry (jam/jam-core/src/main/java/com/qxotic/jam/GGMLType.java:15-26).
__host__ __device__ constexpr int block_elems(int dt) {
    return dt == Q4_K || dt == Q5_K || dt == Q6_K ? 256 : (dt == Q8_0 || dt == Q4_0 || dt == MXFP4) ? 32
         : dt == NVFP4 ? 64 : dt == Q1_0 ? 128 : 1;
}
__host__ __device__ constexpr int block_bytes(int dt) {
    return dt == Q8_0 ? 34 : dt == Q4_0 ? 18 : dt == MXFP4 ? 17 : dt == Q4_K ? 144 : dt == Q5_K ? 176
         : dt == Q6_K ? 210 : dt == NVFP4 ? 36 : dt == Q1_0 ? 18 : dt == F32 ? 4 : 2;
}
// Dense (one element per block) weight types: F32, F16, BF16.
__host__ __device__ constexpr bool is_dense(int dt) { return dt == F32 || dt == F16 || dt == BF16; }

// Device layout of a pinned weight tensor ("row-tiled groups"). A row of k elements is cut into groups
// of 256 elements (one super-block, or 8 blocks of 32; a row whose block count is not a multiple of 8
// ends in a zero-padded group). A group's packed quants are NC 16-byte chunks and its scales SB bytes:
//   Q4_K : NC 8  chunk c = nibble bytes 16c..16c+15            | SB 16: d, dmin fp16, 12 scale bytes
//   Q6_K : NC 13 chunks 0-7 ql, 8-11 qh, 12 the 16 int8 scales | SB 2 : d fp16
//   Q8_0 : NC 16 chunk c = half c&1 of block c>>1 (int8 q)     | SB 16: the 8 blocks' fp16 d
//   Q4_0 : NC 8  chunk c = block c's 16 nibble bytes           | SB 16: the 8 blocks' fp16 d
//   MXFP4: NC 8  chunk c = block c's 16 nibble bytes           | SB 16: the 8 blocks' e8m0, then their
//                                                                maximum (the group's reference exponent)
//   Q5_K : NC 10 chunks 0-7 qs nibble bytes, 8-9 the qh bytes   | SB 16: d, dmin, 12 scale bytes
//   NVFP4: NC 8  chunk 2j + h = half h of 64-block j's qs       | SB 16: the 4 blocks' 4 UE4M3 scales
//   Q1_0 : NC 2  chunk j = 128-block j's 16 sign bytes          | SB 4 : the 2 blocks' fp16 d
// Rows are taken in tiles of 32 (the row count is padded up to a multiple of 32 with zero rows). Plane 0
// ("qs") holds chunk c of group g of row r at byte ((T·G + g)·NC + c)·512 + (r mod 32)·16 with T = r / 32
// and G = groups per row: for a fixed (tile, group, chunk) the 32 rows' chunks are 512 contiguous bytes,
// which is both the A-operand fragment of a 32-row matrix-core tile and, for 4..32 consecutive rows, a
// fully used 64..512-byte segment for the decode kernels. Plane 1 ("sc") holds group g's scales of row r
// at byte ((T·G + g)·32 + r mod 32)·SB. Every GGUF byte is kept; only the order changes.
constexpr int ROW_TILE = 32;   // the shifts below assume 32
__host__ __device__ constexpr int group_chunks(int dt) {
    return dt == Q4_K ? 8 : dt == Q6_K ? 13 : dt == Q8_0 ? 16 : dt == Q4_0 ? 8 : dt == MXFP4 ? 8 : dt == Q5_K ? 10
         : dt == NVFP4 ? 8 : dt == Q1_0 ? 2 : 0;
}
__host__ __device__ constexpr int group_scale_bytes(int dt) {
    return dt == Q4_K ? 16 : dt == Q6_K ? 2 : dt == Q8_0 ? 16 : dt == Q4_0 ? 16 : dt == MXFP4 ? 16 : dt == Q5_K ? 16
         : dt == NVFP4 ? 16 : dt == Q1_0 ? 4 : 0;
}
__host__ __device__ constexpr int blocks_per_group(int dt) { return 256 / block_elems(dt); }
// groups per row for a row of `blocks` blocks
__host__ __device__ constexpr int64_t groups_of(int dt, int64_t blocks) {
    return (blocks + blocks_per_group(dt) - 1) / blocks_per_group(dt);
}
// rows held by a device copy of m rows (whole 32-row tiles)
__host__ __device__ constexpr int64_t tiled_rows(int64_t m) { return (m + ROW_TILE - 1) / ROW_TILE * ROW_TILE; }

// Dense weights are kept row-major on the device, each row padded with zeros to a 256-byte pitch (so every
// row starts 16-byte aligned for vector loads and the padding reads as zeros); WeightView::G then holds the
// pitch in bytes. The sizes of a device copy of `rows` rows of `ldw` elements, for any weight type:
__host__ __device__ constexpr int64_t dense_pitch(int dt, int64_t ldw) { return (ldw * block_bytes(dt) + 255) / 256 * 256; }
// WeightView::G of such a copy: groups per row (quantized) or the pitch (dense)
__host__ __device__ constexpr int64_t view_G(int dt, int64_t ldw) {
    return is_dense(dt) ? dense_pitch(dt, ldw) : groups_of(dt, ldw / block_elems(dt));
}
// plane-0 and plane-1 bytes of the copy (plane 0 rounded to 256 bytes; dense types have no plane 1)
__host__ __device__ constexpr int64_t plane0_bytes(int dt, int64_t rows, int64_t ldw) {
    return is_dense(dt) ? rows * dense_pitch(dt, ldw)
                        : (tiled_rows(rows) * view_G(dt, ldw) * group_chunks(dt) * 16 + 255) / 256 * 256;
}
__host__ __device__ constexpr int64_t plane1_bytes(int dt, int64_t rows, int64_t ldw) {
    return is_dense(dt) ? 0 : tiled_rows(rows) * view_G(dt, ldw) * group_scale_bytes(dt);
}

// Fused epilogue of a matmul's final store: C = [C_old +] (W·A [+ bias[row]]), the bias add first and the
// residual add second, the f32 operations jinfer runs after MatMul.gemm (Ops.addRowBiasInPlace, then
// Ops.addInPlace; jinfer/jinfer-kernels/src/main/java/com/qxotic/jinfer/kernels/Ops.java:326-400).
// Empty (bias null, accumulate 0) = the plain store.
struct Epi {
    const float* bias = nullptr;   // [m], indexed by the output row of the call
    int accumulate = 0;            // 1: add the value already in C (residual add in place)
};

__device__ inline float epilogue(const Epi& e, float v, int64_t row, const float* dst) {
    if (e.bias != nullptr) v += e.bias[row];
    if (e.accumulate) v = *dst + v;
    return v;
}

// One lane's column of a 32x32 MFMA accumulator tile (16 values v[e]): C row `ct`, rows rowb + 8·(e/4) + e%4
// (rowb = the tile's first row + 4·(lane / 32)), each times `scale` and through the epilogue unless `raw`
// (split-K partials). Four consecutive rows go out as one 16-byte store where all four are below m and
// ct + rowb is 16-byte aligned; the values and their order of operations are the scalar path's.
template <typename V>
__device__ inline void store_column(float* ct, int64_t rowb, int64_t m, const V& v, float scale, const Epi& ep,
                                    bool raw) {
    const bool al = (reinterpret_cast<uintptr_t>(ct + rowb) & 15) == 0;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const int64_t r0 = rowb + 8 * g;
        if (al && r0 + 3 < m) {
            float x[4];
#pragma unroll
            for (int i = 0; i < 4; i++) x[i] = v[4 * g + i] * scale;
            if (!raw) {
                if (ep.bias != nullptr)
#pragma unroll
                    for (int i = 0; i < 4; i++) x[i] += ep.bias[r0 + i];
                if (ep.accumulate) {
                    const float4 o = *reinterpret_cast<const float4*>(ct + r0);
                    x[0] = o.x + x[0], x[1] = o.y + x[1], x[2] = o.z + x[2], x[3] = o.w + x[3];
                }
            }
            *reinterpret_cast<float4*>(ct + r0) = make_float4(x[0], x[1], x[2], x[3]);
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t row = r0 + i;
                if (row < m) {
                    const float val = v[4 * g + i] * scale;
                    ct[row] = raw ? val : epilogue(ep, val, row, ct + row);
                }
            }
        }
    }
}

struct WeightView {
    const uint8_t* qs;   // plane 0 of the device copy
    const uint8_t* sc;   // plane 1 of the device copy
    int64_t G;           // groups per row of the device layout
    int64_t r0;          // device-copy row of the view's row 0
    // Host-side routing facts, unused by the kernels: whether every group's block scales fold exactly into
    // the matrix-core GEMM's f16 operands (repack_kernel), and for a copy staged by the current call the
    // device flag the repack left, read only when a call would take the matrix cores.
    int fold_ok = 1;
    const int* fold_flag = nullptr;
};

// Plane-0 address of chunk 0 of group g of view row `row` (chunk c at +c·512), and its plane-1 address.
template <int DT> __host__ __device__ inline const uint8_t* group_q(const WeightView& w, int64_t row, int64_t g) {
    const int64_t r = w.r0 + row;
    return w.qs + ((r >> 5) * w.G + g) * (group_chunks(DT) * 16 * ROW_TILE) + (r & 31) * 16;   // r >= 0
}
template <int DT> __host__ __device__ inline const uint8_t* group_s(const WeightView& w, int64_t row, int64_t g) {
    const int64_t r = w.r0 + row;
    return w.sc + ((r >> 5) * w.G + g) * (group_scale_bytes(DT) * ROW_TILE) + (r & 31) * group_scale_bytes(DT);
}
constexpr int CHUNK_STRIDE = 16 * ROW_TILE;   // bytes between chunks c and c+1 of one row's group

// Activation quantization outputs (per token row j of k elements, nb = k/32 blocks).
struct ActQ {
    const int8_t* q;    // [n][k]
    const float* d;     // [n][nb]   per-32 scale
    const float* s;     // F1: [n][nb] (float)Σq per 32;  F2: [n][k/16] raw f32 Σx per 16
    const int* s16;     // F1 only: [n][k/16] Σq per 16 (exact ints; Q6_K's -32 fold)
};

#define JAMHIP_DEV __device__ __forceinline__

JAMHIP_DEV float h2f(uint32_t bits16) { return (float) __builtin_bit_cast(_Float16, (uint16_t) bits16); }

// v as f16 hi + lo: hi = f16(v), lo = f16(v - hi), about 22 significant bits together. The empty asm makes v
// an opaque f32 register first: left visible, a product v = x·y has its f16 conversion rewritten into one
// v_fma_mixlo_f16 (the exact product rounded once), and the compiler may do that for the hi it subtracts but
// not for the hi it stores; on an f16 tie the two differ by one ulp and hi + lo misses v by that ulp.
struct F16Pair {
    _Float16 hi, lo;
};
JAMHIP_DEV F16Pair split_f16(float v) {
    asm volatile("" : "+v"(v));
    const _Float16 hi = (_Float16) v;
    return {hi, (_Float16) (v - (float) hi)};
}

JAMHIP_DEV int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }
// The value of lane ^ 1 through DPP (quad_perm [1, 0, 3, 2]): no LDS round trip; both lanes of the pair active.
JAMHIP_DEV int xor1_i(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, true); }
JAMHIP_DEV float xor1_f(float v) { return __builtin_bit_cast(float, xor1_i(__builtin_bit_cast(int, v))); }

template <int CTRL> JAMHIP_DEV float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
JAMHIP_DEV float lane_f(float v, int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l)); }

// Sum over the 64 lanes of a wave, the same value in every lane, in a fixed order (reruns are bit-identical).
// Within each row of 16 lanes a DPP butterfly (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror) leaves the row sum in all 16 lanes; the four row sums are then read back with v_readlane.
JAMHIP_DEV float wave_sum(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

// Exclusive prefix sum over the 64 lanes of a wave (lane l gets the sum of lanes below it).
JAMHIP_DEV int wave_exclusive_scan(int v) {
    const int lane = threadIdx.x & 63;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    return x - v;
}

// E8M0 -> 2^(e-128) (jam/jam-native/src/kernels/jam_mxfp4.h:17-24): e=0 -> 2^-128, e=255 -> +Inf.
JAMHIP_DEV float e8m0_half(uint32_t e) {
    uint32_t bits = e == 0 ? 0x00400000u : (e << 23);
    return 0.5f * __builtin_bit_cast(float, bits);
}

// UE4M3 byte -> float as jam_ue4m3_to_float (jam/jam-native/src/kernels/jam_nvfp4.h:19-25): 0x00 and 0x7F give
// 0, otherwise bit 7 is ignored; normal (1 + m/8)·2^(e-7) built from its bits, subnormal m·2^-9 (exact).
JAMHIP_DEV float ue4m3(uint32_t x) {
    const uint32_t e = (x >> 3) & 15u, m = x & 7u;
    const float normal = __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
    const float sub = (float) m * 0.001953125f;
    return (x & 0xffu) == 0u || (x & 0xffu) == 0x7fu ? 0.0f : e ? normal : sub;
}

}  // namespace jamhip
