#ifndef JAMHIP_H
#define JAMHIP_H

/* jamhip — jam's quantized matmul R = W @ Aᵀ on one AMD Instinct MI355X (gfx950).
 *
 * The drop-in boundary for jam's JAM SPI: a new jam backend ("hip") binds these entry points through
 * Panama FFM exactly as NativeJAM binds libjam's jam_mm (jam/jam-native/src/main/java/com/qxotic/jam/
 * NativeJAM.java:174-231). Plain C types only; every pointer is a raw address.
 *
 *   semantics : identical to jam_mm (jam/jam-native/include/jam.h:118-143). W [m×k] weights in a GGUF
 *               block layout selected by `wt`, row stride ldw ELEMENTS; A [n×k] f32, stride lda; C f32
 *               TOKEN-major: C[j*ldc + i] = dot(W[i,:], A[j,:]), ldc >= m, columns [m, ldc) untouched.
 *               Activations are quantized to int8 exactly as jam's CPU path does: per-32 "F1"
 *               (jam_q8_0_requant, jam_kernels_generic.c:71-94) for n < 8, per-32 "F2" with per-16 f32
 *               sums (quantize_row_q8s, jam_kernels_q4k_avx512.c:25-37) for n >= 8, and each dtype's
 *               per-block combine follows the matching jam kernel's decomposition.
 *   dtypes    : every weight type of jam's JAM contract (JAM.java:74-84): Q8_0, Q4_0, Q4_K, Q5_K, Q6_K,
 *               MXFP4, NVFP4, Q1_0 through jam's int8 pipeline, F32, F16, BF16 through jam's dense paths
 *               (BF16 activations rounded to bf16 where jam's bf16 kernels round them, jam.c:622-652); A and C
 *               F32. JAMHIP_EUNSUPPORTED exactly where jam_mm refuses: another A/C type, k off the block, ldw off
 *               the block for the 32-element types and Q1_0 (jam.c:662-685, 752).
 *   residency : weights live on the GPU once pinned (jamhip_weight_pin). jamhip_mm on an unpinned W
 *               stages it for that call only (correct, slow). Pinning uploads and repacks once into the
 *               device layout; it is keyed by host address range, so the caller evicts before freeing or
 *               rewriting a pinned range.
 *   streams   : a context owns one HIP stream and its scratch: a SERIAL stream, as a jam_ctx is
 *               (jam.h:16-20). A concurrent call on a busy context returns JAMHIP_EBUSY.
 *   ctx NULL  : every entry point that takes a context uses the process-global one when ctx == NULL, as
 *               jam_mm(NULL, ...) does (jam.h:128, jam.c:765-768): created on first use on the current
 *               device, released only by jamhip_global_destroy.
 *   scratch   : device scratch a context hands to kernels is never freed or moved while the context
 *               lives (a grown buffer's old allocation is kept until jamhip_ctx_destroy), so a HIP graph
 *               captured around a call stays valid after later, larger calls.
 */

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype tags: numerically jam_dtype / ggml_type (jam/jam-native/include/jam.h:59-77). */
enum {
    JAMHIP_F32 = 0, JAMHIP_F16 = 1, JAMHIP_Q4_0 = 2, JAMHIP_Q8_0 = 8, JAMHIP_Q4_K = 12,
    JAMHIP_Q5_K = 13, JAMHIP_Q6_K = 14, JAMHIP_BF16 = 30, JAMHIP_MXFP4 = 39, JAMHIP_NVFP4 = 40, JAMHIP_Q1_0 = 41
};

/* status: numerically jam_status (jam.h:81-86; JAM.java:87). */
typedef enum {
    JAMHIP_OK = 0,
    JAMHIP_EINVAL = 1,        /* null pointer, m/n/k <= 0, ldw < k, lda < k, ldc < m, HIP failure */
    JAMHIP_EUNSUPPORTED = 2,  /* dtype combination or block misalignment; caller falls back */
    JAMHIP_EBUSY = 3          /* another call is in flight on this context */
} jamhip_status;

typedef struct jamhip_ctx jamhip_ctx;

/* 1 if a gfx950 device is visible and usable, else 0. Replaces the JAM.Provider.isAvailable probe
 * (NativeJAMProvider.java:15-21 / JAM.java:65-71). Env JAM_HIP_DISABLE=1 forces 0. */
int jamhip_device_available(void);

/* Context on `device` (-1 = current). NULL on failure (see jamhip_last_error(NULL)).
 * Mirrors jam_ctx_create/jam_ctx_destroy (jam.h:110-111). */
jamhip_ctx* jamhip_ctx_create(int device);
void        jamhip_ctx_destroy(jamhip_ctx* ctx);

/* Destroy the process-global context (the one ctx == NULL selects) with its pins, scratch and stream.
 * A no-op if it was never created; a later NULL-context call creates it again. Not run automatically:
 * call it for a clean teardown before unloading the library or at process shutdown. Not safe concurrently
 * with calls on the global context. Mirrors jam_global_destroy (jam.h:149-155). */
void        jamhip_global_destroy(void);

/* The device architecture string ("gfx950"); stands in for jam_active_isa/jam_isa_name (jam.h:146,92). */
const char* jamhip_ctx_arch(const jamhip_ctx* ctx);

/* Last error message of `ctx`; for ctx == NULL, of this thread's last failed create or last failed call on
 * the global context. Never NULL; valid until this thread's next jamhip_last_error call. */
const char* jamhip_last_error(const jamhip_ctx* ctx);

/* The matmul, host pointers (jam_mm, jam.h:139-143; FFM descriptor NativeJAM.java:225-230).
 * Synchronous: C is written when it returns. */
jamhip_status jamhip_mm(jamhip_ctx* ctx,
                        const void* w, int wt, int ldw,
                        const void* a, int at, int lda,
                        void*       c, int ct, int ldc,
                        int m, int n, int k);

/* Weight residency (no counterpart in jam: jam_mm borrows host memory per call, jam.h:24-25).
 * pin: upload rows [0, m) of a host weight tensor (m rows of ldw elements, dtype wt) and repack it into
 * the device layout; later calls whose W lies inside [w, w + span) at a row boundary with the same
 * (wt, ldw) read the device copy. evict: drop the entry that starts at w. */
jamhip_status jamhip_weight_pin(jamhip_ctx* ctx, const void* w, int wt, int ldw, int m);
jamhip_status jamhip_weight_evict(jamhip_ctx* ctx, const void* w);
/* Bytes of device memory held by pinned weights. */
int64_t       jamhip_weight_bytes(const jamhip_ctx* ctx);

/* Autopin: residency for callers that never pin (no counterpart in jam; it stands in for the host-address
 * registry the SPI lacks, since JAM.mm carries no weight identity and jinfer passes the same mmap'd
 * address of a tensor on every call, MatMul.java:1783-1830, ModelLoader.java:70-104). Off by default.
 * With sightings = N >= 1, jamhip_mm pins a whole contiguous W (ldw == k, rows [0, m)) that no pin holds on
 * its N-th call with the same (address, dtype, ldw, m), taking a 64-bit hash of every 4 KiB page of the
 * host range; later calls read the device copy after hashing two of its pages again (one rotating, one
 * scattered, so repeated calls sweep the range). A mismatch means the caller rewrote the range in place
 * (an arena reused for another tensor): the pin is evicted and the call stages W. A rewrite that leaves
 * both checked pages unchanged is not seen on that call; callers that rewrite weights evict them
 * (jamhip_weight_evict) or keep autopin off. max_bytes caps the device bytes autopin holds (0: no cap; a
 * range over the cap stays staged). Applies to jamhip_mm only (the device-pointer entry points read pins
 * made explicitly, so a captured graph never refers to a copy that a check could evict). Env at context
 * creation: JAM_HIP_AUTOPIN=N, JAM_HIP_AUTOPIN_MAX_BYTES. */
jamhip_status jamhip_ctx_set_autopin(jamhip_ctx* ctx, int sightings, int64_t max_bytes);
/* out4 = {ranges autopinned, calls served from an autopin, calls staged while autopin was on, pins evicted
 * by a failed check}, since the context was created. */
jamhip_status jamhip_ctx_autopin_stats(const jamhip_ctx* ctx, int64_t* out4);

/* Native-MX mode for MXFP4 weights (no counterpart in jam; off by default). The MXFP4 calls this library
 * runs on the matrix cores (from the same size-dependent token count as the int8 path, 9 to 17 tokens; in
 * jamhip_mm_grouped every expert when rows_cap >= 8·n_experts, else the experts with 8 or more rows) then feed the weights to v_mfma_scale_f32_32x32x64_f8f6f4 as their own fp4 codes and the
 * activations as MX-FP8: per 32-element block E = the smallest exponent with max|x|·2^-E <= 448,
 * hi = e4m3(x·2^-E) (round to nearest even) with scale 2^E, lo = e4m3((x·2^-E - hi)·16) with scale 2^(E-4);
 * mode 1 multiplies hi and lo (about 8 significant bits per activation), mode 2 hi only (about 4). The
 * weights keep jam's exact values; the activations are NOT jam's int8 F2 codes, so results differ from
 * jam's by up to its own quantization error (tests bound mode 1 against the f64 product of the unquantized
 * activations at 5e-3·Σ|w·a|; measured 6e-5, jam's int8 path 2.3e-3). The hardware's scaled block dot
 * itself rounds (steps of about 2^-16 at unit magnitude, measured). Non-finite activations give unspecified (finite-bounded) results. Decode
 * calls (fewer tokens) keep jam's semantics. Env at context creation: JAM_HIP_MX_NATIVE=1|2. */
jamhip_status jamhip_ctx_set_mx_native(jamhip_ctx* ctx, int mode);

/* Device-resident variant of jamhip_mm: W is a pinned host address (the registry key); A and C are
 * device pointers; the work is queued on the context stream and NOT synchronized. Same validation and
 * status codes as jamhip_mm. For callers that keep activations on the GPU (graph capture, benches). */
jamhip_status jamhip_mm_device(jamhip_ctx* ctx,
                               const void* w, int wt, int ldw,
                               const void* a_dev, int at, int lda,
                               void*       c_dev, int ct, int ldc,
                               int m, int n, int k);

/* jamhip_mm_device that allocates nothing: no hipMalloc, hipFree or other allocating call on its path. No
 * counterpart in the reference; it is for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation). W must already be resident (jamhip_weight_pin or the
 * GGUF registry), else JAMHIP_EUNSUPPORTED. The kernels' scratch (activation codes, the matrix-core operand
 * layout, split-K partial sums) comes from one static device array of JAMHIP_NOALLOC_SCRATCH_BYTES per GPU,
 * held by the process until it ends; a call needing more returns JAMHIP_EUNSUPPORTED with the size in
 * jamhip_last_error and queues nothing (jamhip_mm_device covers it). Every call on one GPU, from any context,
 * shares that GPU's array: calls that overlap in time on one GPU (two streams, two threads, two contexts)
 * race on it, so callers serialize them. Same validation, results and status codes as jamhip_mm_device. */
#define JAMHIP_NOALLOC_SCRATCH_BYTES ((size_t) 64 << 20)   /* 64 MiB: config 4's M = 512 prefill fits */
jamhip_status jamhip_mm_device_noalloc(jamhip_ctx* ctx,
                                       const void* w, int wt, int ldw,
                                       const void* a_dev, int at, int lda,
                                       void*       c_dev, int ct, int ldc,
                                       int m, int n, int k);

/* jam's activation quantizers alone (device pointers, context stream, not synchronized); the matmul
 * entry points run the same kernels internally. flavour 1 = F1 (jam_kernels_generic.c:71-94):
 * q[n][k] int8, d[n][k/32], s[n][k/32] = (float)Σq. flavour 2 = F2 (jam_kernels_q4k_avx512.c:25-37):
 * q[n][k], d[n][k/32], s[n][k/16] = raw f32 Σx per 16. k % 32 == 0. */
jamhip_status jamhip_quantize_device(jamhip_ctx* ctx, int flavour, const void* a_dev, int lda, int n, int k,
                                     void* q_dev, void* d_dev, void* s_dev);

/* ---- Mixture-of-experts (device pointers, context stream, not synchronized) -------------------------
 * These replace jinfer's host-side CSR dispatch (jinfer/jinfer-kernels/src/main/java/com/qxotic/jinfer/
 * kernels/Moe.java:178-232) and its per-expert loop of jam calls (GptOss.java:290-314): the same
 * routing order, gather, per-expert jam_mm semantics and fused-multiply-add combine, with the counts
 * and offsets staying on the GPU. */

/* Grouped matmul. The n_experts weight matrices are one tensor of n_experts·m rows at w (dtype wt, row
 * stride ldw; expert e = rows [e·m, (e+1)·m)), pinned or staged like jamhip_mm's W. counts_dev[e]
 * (int32) is expert e's row count; off = their exclusive prefix sum, computed on the device (written to
 * offsets_dev[0..n_experts] when non-NULL). Expert e's rows are A/C rows [off[e], off[e] + counts[e])
 * (CSR order, as Moe.dispatch gathers them); for each expert the result is jam_mm(W_e, A_e, C_e, m,
 * counts[e], k) under jam's routing (F1 below 8 rows, 16-row F2 bands from 8). rows_cap is the number
 * of rows A and C hold: rows past it (a prefix sum beyond rows_cap) are not computed and never read.
 * W is Q8_0, Q4_0, Q4_K, Q6_K or MXFP4; m must be a multiple of 16, n_experts <= 1024 and
 * n_experts·rows_cap below 2^31 (else JAMHIP_EUNSUPPORTED). Replaces the per-expert
 * MatMul.gemm calls of Moe.dispatch's kernel closure (GptOss.java:295-314). */
jamhip_status jamhip_mm_grouped(jamhip_ctx* ctx,
                                const void* w, int wt, int ldw, int m, int n_experts,
                                const void* counts_dev,
                                const void* a_dev, int at, int lda,
                                void*       c_dev, int ct, int ldc,
                                int k, int rows_cap, void* offsets_dev);

/* jamhip_mm_grouped with the experts' biases added in the matmul's store: bias_dev is f32 [n_experts][m],
 * expert e's row i gets bias_dev[e·m + i] (NULL = none), the f32 add of Ops.addRowBiasInPlace on the
 * expert's rows (gpt-oss's gate / up / down expert biases, GptOss.java:301-315). No counterpart in jam. */
jamhip_status jamhip_mm_grouped_ex(jamhip_ctx* ctx,
                                   const void* w, int wt, int ldw, int m, int n_experts,
                                   const void* counts_dev,
                                   const void* a_dev, int at, int lda,
                                   void*       c_dev, int ct, int ldc,
                                   int k, int rows_cap, void* offsets_dev, const void* bias_dev);

/* jamhip_moe_gather and jamhip_mm_grouped_ex in one call: A is not materialised; CSR row r of A is row
 * slot_route_dev[r] / topk of x_dev [seq][ldx] (slot_route_dev as jamhip_moe_route writes it for the same
 * counts), read by the activation quantization itself where the call takes the matrix cores with at least
 * 8·n_experts rows of capacity (other paths gather into context scratch first). Results bit-identical to
 * the two calls. No counterpart in jam: it replaces Moe.dispatch's gather (Moe.java:214-222) followed by
 * the grouped matmul (GptOss.java:295-314), for the gate and up projections that read the gathered rows. */
jamhip_status jamhip_mm_grouped_gather(jamhip_ctx* ctx,
                                       const void* w, int wt, int ldw, int m, int n_experts,
                                       const void* counts_dev,
                                       const void* x_dev, int at, int ldx, const void* slot_route_dev, int topk,
                                       void*       c_dev, int ct, int ldc,
                                       int k, int rows_cap, void* offsets_dev, const void* bias_dev);

/* Moe.dispatch's CSR build (Moe.java:188-206) from route_expert_dev[seq·topk] (int32 expert of route
 * s·topk + j, Moe.selectTopK's rowTopE): counts_dev[n_experts], offsets_dev[n_experts + 1], and the
 * slot of every route in (s, j) order within its expert: slot_route_dev[slot] = route,
 * route_slot_dev[route] = slot (-1 for an expert id outside [0, n_experts)). n_experts <= 1024. */
jamhip_status jamhip_moe_route(jamhip_ctx* ctx, const void* route_expert_dev, int seq, int topk, int n_experts,
                               void* counts_dev, void* offsets_dev, void* slot_route_dev, void* route_slot_dev);

/* Moe.dispatch's gather (Moe.java:214-222): g[slot] = x[slot_route[slot] / topk] for the slots below
 * offsets[n_experts]; dim floats per row, row strides ldx / ldg (elements). */
jamhip_status jamhip_moe_gather(jamhip_ctx* ctx, const void* x_dev, int ldx, const void* slot_route_dev,
                                const void* offsets_dev, int n_experts, int seq, int topk, int dim,
                                void* g_dev, int ldg);

/* Moe.dispatch's weighted scatter-add (Moe.java:208, 223-231; Ops.saxpyInPlace's fma, Ops.java:688-725):
 * out[s] = 0, then for each route of s in ascending expert order (then route order),
 * out[s] = fma(route_prob[route], y[route_slot[route]], out[s]). Bit-identical to the host loop.
 * topk <= 16. */
jamhip_status jamhip_moe_combine(jamhip_ctx* ctx, const void* y_dev, int ldy, const void* route_expert_dev,
                                 const void* route_prob_dev, const void* route_slot_dev, int seq, int topk,
                                 int n_experts, int dim, void* out_dev, int ldo);

/* Router top-k on the device, replacing jinfer's host-side Moe.selectTopK (jinfer/jinfer-kernels/src/main/
 * java/com/qxotic/jinfer/kernels/Moe.java:76-127) and the weight step that follows it:
 *   for each row s, topk passes: best = the first expert with the row's largest selection score (strict >;
 *   NaN never wins; a row with nothing above -Inf picks expert 0), route_expert[s*topk + k] = best,
 *   p = weights[s][best] (the selection array itself when weights_dev is NULL, read before the mask),
 *   selection[s][best] = -Inf (the selection array is consumed in place, as in jinfer);
 *   counts_dev (int [n_experts], may be NULL) is zeroed, then counts[best]++ per route;
 * then per row, by mode:
 *   JAMHIP_TOPK_RAW        route_prob = p                                   (Moe.selectTopK)
 *   JAMHIP_TOPK_SOFTMAX    softmax over the topk selected values, times weights_scale   (gpt-oss:
 *                          GptOss.java:320-345; f32 order of the Java code, exp in double rounded to f32)
 *   JAMHIP_TOPK_NORMALIZE  p / sum of the row's topk p                      (Moe.normalizeTopP, :146-152)
 * and, with expert_scale_dev (f32 [n_experts]) non-NULL, route_prob *= expert_scale[best] (Moe.dispatch's
 * expertScale fold, Moe.java:187-203). selection and weights are f32 [rows][ld], ld >= n_experts;
 * 1 <= n_experts <= 1024, 1 <= topk <= 16. route_expert / route_prob feed jamhip_moe_route and
 * jamhip_moe_combine directly. */
#define JAMHIP_TOPK_RAW 0
#define JAMHIP_TOPK_SOFTMAX 1
#define JAMHIP_TOPK_NORMALIZE 2
jamhip_status jamhip_moe_select_topk(jamhip_ctx* ctx, void* selection_dev, const void* weights_dev, int rows,
                                     int n_experts, int ld, int topk, int mode, float weights_scale,
                                     const void* expert_scale_dev, void* route_expert_dev, void* route_prob_dev,
                                     void* counts_dev);

/* ---- Fused epilogues (no counterpart in jam: jinfer runs these as separate passes after MatMul.gemm).
 * mm_device_ex: jamhip_mm_device with the epilogue applied in the matmul's own final store,
 *   C[j][i] = [C[j][i] +] (dot(W[i,:], A[j,:]) [+ bias[i]])
 * bias_dev: f32 [m] or NULL (Ops.addRowBiasInPlace, jinfer/jinfer-kernels/src/main/java/com/qxotic/
 * jinfer/kernels/Ops.java:375-400, as gpt-oss's expert and attention biases, GptOss.java:301-315);
 * accumulate = 1 adds the result to C in place (Ops.addInPlace, Ops.java:326-360: the residual add after
 * attention's output projection and the FFN's down projection); 0 overwrites C. The f32 operations and
 * their order are those of the separate passes. Same validation and status codes as jamhip_mm_device. */
jamhip_status jamhip_mm_device_ex(jamhip_ctx* ctx,
                                  const void* w, int wt, int ldw,
                                  const void* a_dev, int at, int lda,
                                  void*       c_dev, int ct, int ldc,
                                  int m, int n, int k,
                                  const void* bias_dev, int accumulate);

/* Gated activation in place on gate [rows][ldg] (device f32), up [rows][ldu], `cols` per row:
 * JAMHIP_ACT_SWIGLU      gate = silu(gate)·up                   (Activations.siluMultiply; Ops.java:578-583)
 * JAMHIP_ACT_SWIGLU_OAI  gate = quickgelu(min(gate, 7))·(clamp(up, ±7) + 1)   (gpt-oss;
 *                        Activations.clampedSwiglu, Activations.java:183-187)
 * in the reference's full-scalar arithmetic. Context stream, not synchronized. */
enum { JAMHIP_ACT_SWIGLU = 1, JAMHIP_ACT_SWIGLU_OAI = 2 };
jamhip_status jamhip_glu_device(jamhip_ctx* ctx, int act, void* gate_dev, int ldg, const void* up_dev, int ldu,
                                int rows, int cols);

/* jamhip_glu_device in the arithmetic jinfer runs by default, its Vector API loops (jdk.incubator.vector on;
 * `lanes` = the float species length, 8 on AVX2 hosts, 16 on AVX-512): per row, elements [0, cols - cols %
 * lanes) take the vector body with njuffa's rational tanh (Ops.tanhApprox, Ops.java:620-663):
 *   JAMHIP_ACT_SWIGLU      g·(tanh(g/2)·0.5 + 0.5)·u                      (Ops.java:540-563)
 *   JAMHIP_ACT_SWIGLU_OAI  min(g,7)·0.5·(1 + tanh(0.851·min(g,7)))·(clamp(u,±7) + 1)   (Activations.java:209-224)
 * and the rest the loop's scalar tail (SwiGLU: the full-scalar double formula, Ops.java:566-575; gpt-oss:
 * clampedSwigluApprox, Activations.java:189-194). f32 operations rounded where the Java code rounds, fma fused.
 * lanes = 0 is jamhip_glu_device. */
jamhip_status jamhip_glu_device_vector(jamhip_ctx* ctx, int act, void* gate_dev, int ldg, const void* up_dev,
                                       int ldu, int rows, int cols, int lanes);

/* Use `stream` (a hipStream_t; NULL = the context's own) for subsequent work of this context. */
jamhip_status jamhip_ctx_set_stream(jamhip_ctx* ctx, void* stream);
void*         jamhip_ctx_stream(const jamhip_ctx* ctx);
jamhip_status jamhip_ctx_synchronize(jamhip_ctx* ctx);

/* Measurement aid with no counterpart in the reference: a streaming read of `bytes` of device memory at p_dev
 * (16-byte aligned, bytes a multiple of 16) in the decode kernel's load shape, on the context stream, not
 * synchronized. It computes nothing; sink_dev (one device word) is written only if the loads xor to a fixed
 * value. Its time over a weight-sized buffer is the read floor the matmul kernels are measured against. */
jamhip_status jamhip_read_floor(jamhip_ctx* ctx, const void* p_dev, int64_t bytes, void* sink_dev);

/* ---- GGUF device weight registry (model load).
 * Replaces the load step of jinfer's ModelLoader (jinfer/jinfer-kernels/src/main/java/com/qxotic/jinfer/
 * kernels/ModelLoader.java:35-104: GGUF.read of the header, then one READ_ONLY mapping of the tensor data
 * region and one view per tensor) for the weights that jam multiplies, and adds what that loader leaves to
 * the first jam_mm call: the device copy. open parses a GGUF v3 file with the checks of the qxotic reader
 * (gguf/src/main/java/com/qxotic/format/gguf/impl/ReaderImpl.java:31-380) and maps its data region;
 * pin uploads and repacks every tensor of a jam weight dtype once, keyed exactly as jamhip_weight_pin
 * keys it. A tensor of GGUF dims [d0, d1, d2] (d0 contiguous) is pinned as d1·d2 rows of ldw = d0, so an
 * expert slice of a stacked expert tensor (GptOss.java:673-684) resolves inside it at row e·d1, and
 * jamhip_mm_grouped takes the stacked tensor itself with m = d1. */
typedef struct jamhip_gguf jamhip_gguf;

typedef struct {
    const char* name;      /* valid while the handle is open */
    int         type;      /* ggml_type id (GGMLType.java:31-277) */
    int         n_dims;    /* 0..4 */
    int64_t     dims[4];   /* GGUF order, dims[0] contiguous; unused dims are 1 */
    int64_t     offset;    /* from the start of the tensor data region */
    int64_t     bytes;
    const void* data;      /* inside the handle's read-only mapping; NULL if the region is empty */
} jamhip_gguf_tensor;

/* NULL on failure, with the reason in err (err_cap bytes, NUL-terminated; err may be NULL). No GPU use. */
jamhip_gguf*  jamhip_gguf_open(const char* path, char* err, size_t err_cap);
void          jamhip_gguf_close(jamhip_gguf* g);
int64_t       jamhip_gguf_tensor_count(const jamhip_gguf* g);
jamhip_status jamhip_gguf_tensor_at(const jamhip_gguf* g, int64_t i, jamhip_gguf_tensor* out);
int64_t       jamhip_gguf_find(const jamhip_gguf* g, const char* name);   /* index or -1 */
int64_t       jamhip_gguf_data_offset(const jamhip_gguf* g);              /* file offset of the data region */
int           jamhip_gguf_alignment(const jamhip_gguf* g);

/* Pin every tensor of g of 2 or more dims and a jam weight type (quantized or F32 / F16 / BF16) at
 * data_base + offset: data_base is the caller's own mapping of the same file's data region (the addresses its
 * jam calls will pass), or NULL for the handle's mapping. 1-D tensors (norms, biases) and other types are
 * skipped. Tensors of one dtype and row length stored back to
 * back (a block's attn_q|attn_k|attn_v, ffn_gate|ffn_up), each starting on a 32-row boundary of the run,
 * share one device range: every tensor still resolves on its own, and one call with W = the first
 * tensor's address and m = the rows of several computes them together (their outputs concatenated in
 * C). Every tensor is checked first (JAMHIP_EUNSUPPORTED, nothing pinned, the tensor's name in
 * jamhip_last_error, for a row extent that is not whole blocks or exceeds 32-bit extents); a device
 * failure stops the pinning, and the ranges pinned before it stay pinned. n_pinned / bytes_pinned
 * (either may be NULL) receive the count and file bytes of the tensors now resident. evict drops the
 * file's ranges. Pins are keyed by address: evict them before the mapping they were taken from goes
 * away (jamhip_gguf_close for data_base = NULL, the caller's unmap otherwise), or a later mapping at the
 * same addresses would be served the old weights. */
jamhip_status jamhip_gguf_pin(jamhip_ctx* ctx, const jamhip_gguf* g, const void* data_base, int64_t* n_pinned,
                              int64_t* bytes_pinned);
jamhip_status jamhip_gguf_evict(jamhip_ctx* ctx, const jamhip_gguf* g, const void* data_base, int64_t* n_evicted);

#ifdef __cplusplus
}
#endif
#endif /* JAMHIP_H */
