// Kernel launchers shared between the kernel translation units and the C-ABI layer (jamhip.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace jamhip {

// F1: q [n][k] int8, d [n][k/32], asum [n][k/32] (float Σq), s16 [n][k/16] (int Σq).
hipError_t launch_quant_f1(const float* a, int lda, int n, int k, int8_t* q, float* d, float* asum, int* s16,
                           hipStream_t st);
// F2: q [n][k] int8, d [n][k/32], xs [n][k/16] (raw f32 Σx).
hipError_t launch_quant_f2(const float* a, int lda, int n, int k, int8_t* q, float* d, float* xs, hipStream_t st);

// raw GGUF rows (rb blocks each, stride raw_stride bytes) -> the device layout with G groups per row. For
// Q8_0, Q4_0 and MXFP4 with a non-null flag (device int), *flag ends 1 if some group's block scales cannot
// be folded exactly into the matrix-core GEMM's f16 operands (prep.hip, repack_kernel), else 0.
hipError_t launch_repack(int dt, const uint8_t* raw, int64_t raw_stride, int64_t rows, int64_t rb, int64_t G,
                         uint8_t* qs, uint8_t* sc, hipStream_t st, int* flag = nullptr);

// Expert grouping of a grouped matmul (moe.hip): CSR row offsets off[E+1] of the experts' rows in A and
// C, the 8-token tile map (poff8, map8) and the 64-token slot map (poff64, map64) of the experts with at
// least 8 rows, and the weight rows per expert (expert e = view rows [e·gm, (e+1)·gm)). Device pointers.
struct Groups {
    const int* off;
    const int* poff8;
    const int* map8;
    const int* poff64;
    const int* map64;
    int gm;
    const float* bias = nullptr;   // per-expert bias [E][gm] added in the store (expert e at bias + e·gm)
    // an expert list in expert order, -1 past its last (launch_moe_offsets): the F1 grouped kernel's workgroup
    // column y takes expert small[y] (null: expert y)
    const int* small = nullptr;
    // or, when counts is set (at most 64 experts, fewer than 8 rows in all): the F1 grouped kernel finds its
    // expert and rows from the device counts itself, with launch_moe_offsets' clamps to rows_cap
    const int* counts = nullptr;
    int n_experts = 0, rows_cap = 0;
    // the gather folded in (F1 grouped kernels with the fused prologue): slot t's row is a[rows[t] / rdiv]
    const int* rows = nullptr;
    int rdiv = 1;
};

// Matrix-core GEMM workgroup -> linear tile; workgroup b runs on XCD b % 8. Ungrouped: each XCD takes one
// contiguous run of tiles (a row block's token blocks share its L2). Grouped: runs of GCH consecutive
// expert-major tiles are dealt to the XCDs in turn, so each XCD gets a share of every expert (their tiles
// differ in cost: an expert's last slot block may be half empty) while a run keeps its weight rows and
// activation slots in one L2. tile_grid is the launch size that covers every tile.
constexpr int GCH = 16;
JAMHIP_DEV int tile_of_block(bool grouped, int total) {
    const int b = (int) blockIdx.x, x = b % 8, i = b / 8;
    if (grouped) return ((i / GCH) * 8 + x) * GCH + i % GCH;
    return x * ((total + 7) / 8) + i;
}
inline int tile_grid(bool grouped, int total) {
    return grouped ? (total + 8 * GCH - 1) / (8 * GCH) * (8 * GCH) : (total + 7) / 8 * 8;
}

// Grouped matrix-core GEMMs: linear workgroup `lin` of nrb row blocks x the 64-slot blocks -> (row block,
// slot block) in expert-major order. Expert e's slot blocks [cbs, cbs + ns) own the linear range
// [nrb·cbs, nrb·(cbs + ns)), row block-major inside it, so workgroups placed next to each other (one XCD
// takes a contiguous run) share the expert's weight rows and its activation slots stay in that XCD's L2.
// Returns the expert, or -1 for a slot block past the last expert's.
JAMHIP_DEV int grouped_tile(const Groups& gp, int lin, int nrb, int* rb, int* cb) {
    const int e = __builtin_amdgcn_readfirstlane(gp.map64[lin / nrb]);
    if (e < 0) return -1;
    const int p = __builtin_amdgcn_readfirstlane(gp.poff64[e]), cbs = p / 64;
    const int ns = (__builtin_amdgcn_readfirstlane(gp.poff64[e + 1]) - p) / 64;   // >= 1: e owns slot block lin / nrb
    const int l = lin - nrb * cbs;
    *rb = l / ns;
    *cb = cbs + l % ns;
    return e;
}

// flavour 3: any n, F1 activations read from A in 8-token tiles (NVFP4, whose only jam kernel is F1 at
// every n). flavour 1: n in [1, 7], F1 activations; with `a` non-null the kernel quantizes A itself (requires
// gemv_fusable(n, k)), else it reads A's quantized copy from `A`. flavour 2: any n >= 1, F2
// activations from `A`, 8 tokens per grid row. From k = 8192 on, for n >= 2, the kernel splits K into
// 4096-element slices, and past k = 65536 for n = 1 into 32768-element slices: `part` must then hold
// gemv_split_floats(k, m, n) floats (the slices' partial results, summed into c in slice order);
// gemv_split_floats is 0 otherwise and part may be null.
bool gemv_fusable(int n, int k, const float* a, int lda);   // a, lda: the f32 activations (16-byte aligned rows)
size_t gemv_split_floats(int k, int m, int n);
hipError_t launch_gemv(int dt, int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m,
                       int n, float* c, int ldc, hipStream_t st, float* part = nullptr, const Epi& ep = Epi{});
// c[t][row] = Σ_s part[s·slice + t·m + row] for s = 0..ns-1 in order (rows < m, tokens < n)
hipError_t launch_split_reduce(const float* part, int ns, int64_t slice, int m, int n, float* c, int ldc,
                               hipStream_t st, const Epi& ep = Epi{});

// Grouped forms (one launch for all experts). flavour 0 / 1: F1 over the experts of g.small (E workgroup
// columns) holding exactly one row / 2..7 rows (one-token / seven-token kernels; experts with other counts
// are skipped), the kernel quantizing its expert's rows itself when `a` is non-null (then
// gemv_grouped_fusable(k, a, lda) must hold), else reading them from A (CSR rows). flavour 2: the 8-token
// tiles of map8 (experts with >= 8 rows), F2 activations from A (CSR rows). flavour 3: flavours 0 and 1 in
// one launch with the experts taken from g.counts (E = the one-token columns, cap8 = the seven-token
// columns). m here is the rows per expert (g.gm).
bool gemv_grouped_fusable(int k, const float* a, int lda);
hipError_t launch_gemv_grouped(int dt, int flavour, const WeightView& w, const ActQ& A, const float* a, int lda,
                               int k, const Groups& g, int E, int cap8, float* c, int ldc, hipStream_t st);

// Rows [r0, r0 + rows) of an n >= 8 call as jam's bands compute their <16-row tail: an f32 dot of the
// dequantized weight row with the f32 activations a [n][lda].
hipError_t launch_rows_float(int dt, const WeightView& w, const float* a, int lda, int k, int r0, int rows, int n,
                             float* c, int ldc, hipStream_t st, const Epi& ep = Epi{});

// int8-MFMA prefill GEMM (F2 activations), n >= 1; returns hipErrorNotSupported for dtypes it lacks
// (gemm_covers is false for them).
bool gemm_covers(int dt);
hipError_t launch_gemm(int dt, const WeightView& w, const ActQ& A, int k, int m, int n, float* c, int ldc,
                       hipStream_t st, const Epi& ep = Epi{});

// Activations of the matrix-core GEMM, written by launch_gemm_prep: jam's F2 quantization of n tokens
// (bit-exact codes and scales) laid out for the MFMA operand loads. Tokens are padded to NP (a multiple
// of 64) and k to Kp (a multiple of 256) with zeros. Token t carries a power of two 2^e_t chosen so that
// its largest activation sum lies in [2^13, 2^14): the GEMM accumulates in units of 2^-e_t (the block
// scales and sums below are pre-multiplied by it, exactly) and multiplies by 2^e_t on the way out.
struct GemmAct {
    const _Float16* b;     // [Kp/16][2][NP][8] activation codes; kstep k16 = 2·block + ks, half q, slot i holds
                           // element 32·block + 16q + 8ks + perm8(i)
    const float* dx;       // [Kp/32][NP] block scale d · 2^-e_t
    const _Float16* shi;   // per-32 sums (Q4_K, Q4_0) [Kp/256][NP][8] or per-16 sums (Q6_K) [Kp/256][NP][16],
    const _Float16* slo;   //   · 2^-e_t, split as f16 high part + f16 remainder
    const float* es;       // [NP] 2^e_t
    int NP, Kp;
    int K;                 // the call's k (blocks past it are zero)
};
int gemm_sums_kind(int dt);   // 0 none, 1 per-32 sums, 2 per-16 sums
size_t gemm_act_bytes(int dt, int n, int k);
bool gemm_prep_fits(int k);
// jamhip_mm's activation upload by a copy kernel (bytes and both pointers 16-byte aligned; src device-visible
// pinned host memory); hipErrorInvalidValue otherwise
hipError_t launch_stage_copy(const void* src, void* dst, size_t bytes, hipStream_t st);
// Caches device dev's CU count for the matrix-core GEMM's last-round balancing (called at context creation).
void gemm_tail_prime(int dev);
int device_cus();   // CUs of the current device (gemm_tail_prime's record; 0 before it)
   // the activation prep holds a slot's block scales and sums in LDS
hipError_t launch_gemm_prep(int dt, const float* a, int lda, int n, int k, void* scratch, GemmAct* out,
                            hipStream_t st);
// Matrix-core GEMM over GemmAct (f16 MFMA on exact integer operands); hipErrorNotSupported for dtypes it
// does not cover. Grouped form: GemmAct laid out by the 64-token slots of g (launch_gemm_prep_grouped),
// cap64 slot blocks, m = g.gm rows per expert.
// Small grids split K over extra workgroups (partials in `part`, gemm_mma_split_floats(dt, k, m, n) floats,
// summed in a fixed order; part == nullptr: no split).
size_t gemm_mma_split_floats(int dt, int k, int m, int n);
hipError_t launch_gemm_mma(int dt, const WeightView& w, const GemmAct& A, int k, int m, int n, float* c, int ldc,
                           hipStream_t st, float* part = nullptr, const Epi& ep = Epi{});
hipError_t launch_gemm_mma_grouped(int dt, const WeightView& w, const GemmAct& A, int k, const Groups& g, int cap64,
                                   float* c, int ldc, hipStream_t st);
size_t gemm_act_bytes_np(int dt, int NP, int k);

// Opt-in native-MX path for MXFP4 (mxn.hip): activations as MX-FP8 hi + lo codes (mode 1) or hi only
// (mode 2) in the scaled MFMA's B operand order, one e8m0 scale per 32-block for each part.
struct MxAct {
    const uint8_t* hi;    // [Kp/64][2][NP][32] e4m3 codes (64-K step, lane half, token slot, byte)
    const uint8_t* lo;
    const uint8_t* shi;   // [Kp/32][NP] e8m0 scale of each block's hi codes
    const uint8_t* slo;
    int NP, Kp, K;
};
size_t mx_act_bytes_np(int NP, int k);
hipError_t launch_mx_prep(const float* a, int lda, int n, int k, int mode, void* scratch, MxAct* out, hipStream_t st);
hipError_t launch_mx_prep_grouped(const float* a, int lda, int k, int mode, const Groups& g, int cap64, void* scratch,
                                  MxAct* out, hipStream_t st);
hipError_t launch_mx_gemm(int mode, const WeightView& w, const MxAct& A, int m, int n, float* c, int ldc, hipStream_t st,
                          const Epi& ep = Epi{});
hipError_t launch_mx_gemm_grouped(int mode, const WeightView& w, const MxAct& A, const Groups& g, int cap64, float* c,
                                  int ldc, hipStream_t st);

// Dense weights (F32, F16, BF16; dense.hip): jam's dense paths, any n, any k (rows padded to a 256-byte pitch,
// WeightView::G = the pitch).
hipError_t launch_dense(int dt, const WeightView& w, const float* a, int lda, int k, int m, int n, float* c, int ldc,
                        hipStream_t st, const Epi& ep = Epi{});
// From DENSE_MMA_MIN_N tokens (from 2 where the staged GEMV's activation tile would not fit LDS) F16, and BF16
// where jam rounds the activations to bf16, take the staged matrix-core GEMM instead
// (dense_mma_planes(dt, n, k) > 0): scratch of dense_act_bytes(dt, n, k) bytes for
// the operand-ordered activations, and dense_mma_split_floats(dt, k, m, n) floats of split-K partials
// (nullptr when that is 0).
constexpr int DENSE_MMA_MIN_N = 9;
int dense_mma_planes(int dt, int n, int k);
size_t dense_act_bytes(int dt, int n, int k);
size_t dense_mma_split_floats(int dt, int k, int m, int n);
hipError_t launch_dense_mma(int dt, const WeightView& w, const float* a, int lda, int k, int m, int n, float* c,
                            int ldc, void* scratch, float* part, hipStream_t st, const Epi& ep = Epi{});

// In place on gate [rows][ldg]: act 1 SwiGLU silu(gate)·up, act 2 gpt-oss clamped SwiGLU (epilogue.hip); lanes 0
// the full-scalar arithmetic, lanes > 0 jinfer's Vector API arithmetic with a species of `lanes` floats.
hipError_t launch_glu(int act, float* gate, int ldg, const float* up, int ldu, int rows, int cols, hipStream_t st,
                      int lanes = 0);

// Streaming read of `bytes` (a multiple of 16; 16-byte aligned p) with the decode kernel's load shape, nothing
// written but a word at `sink` if the loads xor to a fixed value (readfloor.hip).
hipError_t launch_read_floor(const void* p, int64_t bytes, uint32_t* sink, hipStream_t st);
// The grouped prep that builds its own slot map (one launch instead of offsets + F1 decode + prep; E <= 256):
// every expert with rows gets 64-token slots (experts with 1..7 rows quantized with jam's F1, the rest with
// F2), and workgroup 0 writes the CSR offsets (off, and off_out if non-null), poff64 and map64 for the GEMM.
struct PrepGroups {
    const int* counts;
    int E, rows_cap;
    int *off, *poff64, *map64;
    int cap64;
    int* off_out;
    // gathered input: CSR row r of A is row rows[r] / rdiv of the activations (null: row r)
    const int* rows = nullptr;
    int rdiv = 1;
};
constexpr int PREP_FUSED_MAX_E = 256;
hipError_t launch_gemm_prep_grouped_fused(int dt, const float* a, int lda, int k, const PrepGroups& pg,
                                          void* scratch, GemmAct* out, hipStream_t st);
hipError_t launch_gemm_prep_grouped(int dt, const float* a, int lda, int k, const Groups& g, int cap64,
                                    void* scratch, GemmAct* out, hipStream_t st);
// The native-MX prep (mxn.hip) for a grouped call that derives its expert table from the device counts in
// the same way: also writes pg's offsets, 64-slot offsets and slot map.
hipError_t launch_mx_prep_grouped_fused(const float* a, int lda, int k, int mode, const PrepGroups& pg, void* scratch,
                                        MxAct* out, hipStream_t st);

// MoE bookkeeping (moe.hip)
// small[0..n1): the experts with exactly one row, small[n1..n1 + n2): those with 2..7 rows, each list in expert
// order and -1 past its last; n1 >= min(E, rows_cap), n2 >= min(E, rows_cap / 2) (at most that many experts can
// hold one row / two or more).
hipError_t launch_moe_offsets(const int* counts, int E, int rows_cap, int* off, int* poff64, int* poff8, int* map64,
                              int cap64, int* map8, int cap8, int* small, int n1, int n2, hipStream_t st);
// scratch: moe_route_scratch_ints(R, E) ints of device memory for the chunked form (R > 256 routes, E <= 256),
// or null for the single-workgroup kernel; both give the same slots.
size_t moe_route_scratch_ints(int R, int E);
hipError_t launch_moe_route(const int* route_expert, int R, int E, int* counts, int* off, int* slot_route,
                            int* route_slot, hipStream_t st, int* scratch = nullptr);
hipError_t launch_moe_gather(const float* x, int ldx, const int* slot_route, const int* off, int E, int R, int topk,
                             int dim, float* g, int ldg, hipStream_t st);
// Router top-k (Moe.selectTopK + the caller's weight step): sel [rows][ld] scores, consumed (winners masked to
// -Inf); wts the combine weights (null: sel itself); mode MOE_TOPK_RAW / _SOFTMAX / _NORMALIZE; escale [E] per
// expert (nullable); outputs route_expert / route_prob [rows][topk], counts [E] (nullable, zeroed then filled).
constexpr int MOE_TOPK_MAX = 16;
constexpr int MOE_TOPK_RAW = 0, MOE_TOPK_SOFTMAX = 1, MOE_TOPK_NORMALIZE = 2;
hipError_t launch_moe_topk(float* sel, const float* wts, int rows, int E, int ld, int topk, int mode, float wscale,
                           const float* escale, int* route_expert, float* route_prob, int* counts, hipStream_t st);
hipError_t launch_moe_combine(const float* y, int ldy, const int* route_expert, const float* route_prob,
                              const int* route_slot, int seq, int topk, int E, int dim, float* out, int ldo,
                              hipStream_t st);

}  // namespace jamhip
