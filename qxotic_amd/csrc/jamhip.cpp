// C-ABI of the MI355X jam backend (include/jamhip.h): context, device weight registry, argument
// validation in jam_mm's order, and dispatch to the HIP kernels. Host-side C++; compiled by hipcc.
#include "jamhip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"
#include "gguf.h"
#include "launch.h"

using namespace jamhip;

namespace {

// Device buffer of a context, grown on demand. For the scratch that kernels of jamhip_mm_device and the
// grouped / MoE entry points use (RETIRE = true), a grown buffer's old allocation is retired, not freed: a
// HIP graph captured around an earlier call keeps that address, so every scratch address a context ever
// handed to a kernel stays valid until jamhip_ctx_destroy (growth is geometric, so the retired total stays
// below four times the current size). Staging for host copies (RETIRE = false) is freed on growth.
template <bool RETIRE> struct DevBufT {
    void* p = nullptr;
    size_t cap = 0;
    std::vector<void*> retired;
    hipError_t ensure(size_t bytes) {
        if (bytes <= cap) return hipSuccess;
        size_t want = bytes + bytes / 4;
        void* q = nullptr;
        if (!RETIRE && p) {
            (void) hipFree(p);
            p = nullptr;
            cap = 0;
        }
        hipError_t e = hipMalloc(&q, want);
        if (e != hipSuccess) return e;
        if (p) retired.push_back(p);
        p = q;
        cap = want;
        return hipSuccess;
    }
    void release() {
        for (void* r : retired) (void) hipFree(r);
        retired.clear();
        if (p) (void) hipFree(p);
        p = nullptr;
        cap = 0;
    }
};
using DevBuf = DevBufT<true>;
using StageBuf = DevBufT<false>;

// Pinned host bounce buffer (hipHostMalloc): small copies from it are single DMA transfers, where a
// pageable source is first staged by the runtime.
struct HostBuf {
    void* p = nullptr;
    size_t cap = 0;
    hipError_t ensure(size_t bytes) {
        if (bytes <= cap) return hipSuccess;
        if (p) (void) hipHostFree(p);
        p = nullptr;
        cap = 0;
        const size_t want = bytes + bytes / 4;
        hipError_t e = hipHostMalloc(&p, want, hipHostMallocDefault);
        if (e == hipSuccess) cap = want;
        return e;
    }
    void release() {
        if (p) (void) hipHostFree(p);
        p = nullptr;
        cap = 0;
    }
};

struct Pin {
    uintptr_t host;     // registry key: [host, host + span)
    int64_t span;
    int dt, ldw;
    int64_t rows, G;    // rows and groups per row of the device copy
    uint8_t* dev;       // plane 0
    uint8_t* sc;        // plane 1
    int64_t bytes;      // device bytes held
    // autopin only (pinned by jamhip_mm on a repeat sighting): a hash of every 4 KiB page of the host range
    // taken at pin time, and the count of per-call spot checks made against it
    std::vector<uint64_t> pages;
    uint64_t checks = 0;
    int fold_ok = 1;    // the repack's check: block scales fold exactly into the matrix-core operands
};

// A host weight range seen by jamhip_mm while not resident (the autopin candidates).
struct Sight {
    uintptr_t host;
    int dt, ldw;
    int64_t rows;
    int count;
};

constexpr int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

// Every weight type of jam's JAM contract (JAM.java:74-84): the int8-pipeline types and the dense ones.
bool supported_w(int dt) {
    return dt == Q8_0 || dt == Q4_0 || dt == Q4_K || dt == Q6_K || dt == MXFP4 || dt == Q5_K || dt == NVFP4 ||
           dt == Q1_0 || dt == F32 || dt == F16 || dt == BF16;
}
// The grouped (MoE) matmul covers the types with a grouped kernel.
bool grouped_w(int dt) { return dt == Q8_0 || dt == Q4_0 || dt == Q4_K || dt == Q6_K || dt == MXFP4; }

// jam's block rule (jam.c:665-685, 752): k on the block for every quantized type; ldw on it too for the
// 32-element types and Q1_0, while the K-quants and NVFP4 stride rows by (ldw / block) blocks, and the dense
// types take any k and ldw.
bool block_aligned(int dt, int ldw, int k) {
    const int be = block_elems(dt);
    if (k % be) return false;
    if (dt == Q4_K || dt == Q5_K || dt == Q6_K || dt == NVFP4 || is_dense(dt)) return true;
    return ldw % be == 0;
}

// Device scratch of jamhip_mm_device_noalloc: one fixed array per GPU, in the code object (no allocation
// call ever sizes it), shared by every call on that GPU. In host code `scratch` is only a stand-in for the
// symbol: its device address comes from hipGetSymbolAddress, taken once per device when the first context
// on that device is created (noalloc_scratch_init) and used everywhere host code refers to the array.
constexpr size_t NOALLOC_SCRATCH_BYTES = JAMHIP_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[MAX_DEVICES] = {};          // device address of `scratch` on each device, once known
hipError_t g_scratch_err[MAX_DEVICES] = {};

// Takes the address of `scratch` on `device` (which must be current) the first time; later calls return
// the recorded outcome.
hipError_t noalloc_scratch_init(int device) {
    if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[device] || g_scratch_err[device] != hipSuccess) return g_scratch_err[device];
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
        g_scratch_err[device] = e != hipSuccess ? e : hipErrorInvalidSymbol;
        return g_scratch_err[device];
    }
    g_scratch_ptr[device] = static_cast<uint8_t*>(ptr);
    return hipSuccess;
}

uint8_t* noalloc_scratch(int device) {
    if (device < 0 || device >= MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return g_scratch_ptr[device];
}

// Error text of calls with no context of their own: a failed jamhip_ctx_create, or a failed call made with
// ctx == NULL (the process-global context). Per thread; jamhip_last_error(NULL) returns it.
thread_local char g_null_error[512] = "";

void set_null_error(const std::string& s) { snprintf(g_null_error, sizeof g_null_error, "%s", s.c_str()); }

}  // namespace

struct jamhip_gguf {
    GgufFile* f;
};

struct jamhip_ctx {
    int device = 0;
    hipStream_t own = nullptr;
    hipStream_t stream = nullptr;
    std::atomic<int> busy{0};
    std::mutex err_mu;   // err is written by a failing call while another thread may read or write it
    std::string err;
    char arch[64] = {0};
    mutable std::mutex pin_mu;
    std::vector<Pin> pins;
    int64_t pinned_bytes = 0;   // sum of pins[].bytes, under pin_mu
    DevBuf act, gact, part, moe, route, gath; // kernel scratch (addresses may be captured in graphs)
    DevBuf fold;                              // the repack's fold flag (one int)
    StageBuf a_stage, c_stage, w_raw, w_stage;   // staging of host copies
    HostBuf a_host, c_host;   // jamhip_mm's pinned bounce buffers for A and C
    // autopin (jamhip_ctx_set_autopin): pin a host weight range on its `autopin`-th sighting, 0 = off
    int autopin = 0;
    int64_t autopin_cap = 0;        // bytes autopin may hold on the device (0: no limit)
    int64_t autopin_bytes = 0;      // held by autopins now, under pin_mu
    std::vector<Sight> sights;      // under pin_mu, at most AUTOPIN_SIGHTS entries
    int64_t ap_stats[4] = {0, 0, 0, 0};   // pins made, calls served by an autopin, staged calls, invalidations
    int mx_native = 0;   // MXFP4 matrix-core calls: 0 jam's int8 semantics, 1 / 2 the native-MX path (mxn.hip)
};

namespace {

jamhip_status fail(jamhip_ctx* ctx, jamhip_status st, const std::string& msg) {
    if (ctx) {
        std::lock_guard<std::mutex> lk(ctx->err_mu);
        ctx->err = msg;
    }
    return st;
}

std::string error_of(jamhip_ctx* ctx) {
    std::lock_guard<std::mutex> lk(ctx->err_mu);
    return ctx->err;
}

jamhip_status hip_fail(jamhip_ctx* ctx, hipError_t e, const char* what) {
    // a shape no kernel here covers (hipErrorNotSupported from a launcher) is jam's EUNSUPPORTED: the
    // caller falls through to the next backend
    return fail(ctx, e == hipErrorNotSupported ? JAMHIP_EUNSUPPORTED : JAMHIP_EINVAL,
                std::string(what) + ": " + hipGetErrorString(e));
}

struct Busy {   // the serial-stream guard of jam_mm (jam/jam-native/src/jam.c:777-783)
    jamhip_ctx* c;
    bool ok;
    explicit Busy(jamhip_ctx* ctx) : c(ctx), ok(ctx->busy.exchange(1, std::memory_order_acquire) == 0) {}
    ~Busy() {
        if (ok) c->busy.store(0, std::memory_order_release);
    }
};

// jam_mm's EINVAL contract (jam.c:771-775), then the dtype/alignment EUNSUPPORTED classes (jam.c:759-762).
jamhip_status validate(jamhip_ctx* ctx, const void* w, int wt, int ldw, const void* a, int at, int lda, void* c,
                       int ct, int ldc, int m, int n, int k) {
    if (!ctx) return JAMHIP_EINVAL;
    if (!w || !a || !c) return fail(ctx, JAMHIP_EINVAL, "null operand");
    if (m <= 0 || n <= 0 || k <= 0) return fail(ctx, JAMHIP_EINVAL, "m, n, k must be positive");
    if (ldw < k || lda < k || ldc < m) return fail(ctx, JAMHIP_EINVAL, "stride below extent (ldw<k, lda<k or ldc<m)");
    if (at != F32 || ct != F32) return fail(ctx, JAMHIP_EUNSUPPORTED, "A and C must be F32");
    if (!supported_w(wt)) return fail(ctx, JAMHIP_EUNSUPPORTED, "weight dtype not supported on the GPU backend");
    if (!block_aligned(wt, ldw, k)) return fail(ctx, JAMHIP_EUNSUPPORTED, "k (and for this dtype ldw) must be a multiple of the block size");
    return JAMHIP_OK;
}

int64_t row_bytes(int dt, int64_t elems) { return elems / block_elems(dt) * block_bytes(dt); }

// Registry lookup: W inside a pinned range, on a row boundary, same (dtype, ldw), rows [r0, r0+m) held.
// Pins are kept sorted by host address and never overlap, so the only candidate is the last pin that
// starts at or below W: one binary search per call. An autopin (a pin with page hashes) serves only
// jamhip_mm calls that start at its first byte, after their spot check (autopin_lookup): every other
// lookup passes explicit_only and does not see it, so a device entry point (whose launches a graph may
// capture) never refers to a copy that a failed check could free, and a call at a row offset into an
// autopinned range is staged rather than served without a check.
bool lookup(jamhip_ctx* ctx, const void* w, int dt, int ldw, int m, WeightView* out, bool explicit_only = true) {
    std::lock_guard<std::mutex> lk(ctx->pin_mu);
    const uintptr_t p = reinterpret_cast<uintptr_t>(w);
    auto it = std::upper_bound(ctx->pins.begin(), ctx->pins.end(), p,
                               [](uintptr_t v, const Pin& pin) { return v < pin.host; });
    if (it == ctx->pins.begin()) return false;
    const Pin& pin = *(it - 1);
    if (explicit_only && !pin.pages.empty()) return false;
    if (pin.dt != dt || pin.ldw != ldw || p >= pin.host + (uintptr_t) pin.span) return false;
    const int64_t off = (int64_t) (p - pin.host), rbytes = row_bytes(dt, ldw);
    if (off % rbytes) return false;
    const int64_t r0 = off / rbytes;
    if (r0 + m > pin.rows) return false;
    out->qs = pin.dev;
    out->sc = pin.sc;
    out->G = pin.G;
    out->r0 = r0;
    out->fold_ok = pin.fold_ok;
    out->fold_flag = nullptr;
    return true;
}

// Upload `rows` raw host rows (stride raw_stride bytes, rb blocks used per row) into a device-layout
// buffer of G groups per row at dst (plane 0) / dst_sc (plane 1) via a staging copy and the repack kernel.
// The repack also leaves the fold flag (launch_repack) in ctx->fold for Q8_0 / Q4_0 / MXFP4 / Q1_0; *flag gets its
// device address then (null otherwise).
jamhip_status upload(jamhip_ctx* ctx, const uint8_t* host, int dt, int64_t raw_stride, int64_t rows, int64_t rb,
                     int64_t G, uint8_t* dst, uint8_t* dst_sc, const int** flag) {
    const int64_t span = (rows - 1) * raw_stride + rb * block_bytes(dt);
    hipError_t e;
    if ((e = ctx->w_raw.ensure((size_t) span)) != hipSuccess) return hip_fail(ctx, e, "weight staging alloc");
    int* fl = nullptr;
    if (dt == Q8_0 || dt == Q4_0 || dt == MXFP4 || dt == Q1_0) {
        if ((e = ctx->fold.ensure(sizeof(int))) != hipSuccess) return hip_fail(ctx, e, "fold flag alloc");
        fl = (int*) ctx->fold.p;
    }
    if ((e = hipMemcpyAsync(ctx->w_raw.p, host, (size_t) span, hipMemcpyHostToDevice, ctx->stream)) != hipSuccess)
        return hip_fail(ctx, e, "weight upload");
    if ((e = launch_repack(dt, (const uint8_t*) ctx->w_raw.p, raw_stride, rows, rb, G, dst, dst_sc, ctx->stream, fl)) !=
        hipSuccess)
        return hip_fail(ctx, e, "weight repack");
    *flag = fl;
    return JAMHIP_OK;
}

// Reads a fold flag the repack left (stream-ordered, then a synchronize): 1 when every group folds exactly.
jamhip_status read_fold(jamhip_ctx* ctx, const int* flag, int* fold_ok) {
    int v = 0;
    hipError_t e = hipMemcpyAsync(&v, flag, sizeof v, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "fold flag read");
    *fold_ok = v == 0;
    return JAMHIP_OK;
}

// Resolve W to a device view: the registry, else a per-call staged copy of rows [0, m), k elements each.
jamhip_status resolve_w(jamhip_ctx* ctx, const void* w, int dt, int ldw, int m, int k, WeightView* wv) {
    if (lookup(ctx, w, dt, ldw, m, wv, true)) return JAMHIP_OK;
    const int64_t rb = k / block_elems(dt), G = view_G(dt, k);
    const int64_t qsz = plane0_bytes(dt, m, k), ssz = plane1_bytes(dt, m, k);
    hipError_t e = ctx->w_stage.ensure((size_t) (qsz + ssz));
    if (e != hipSuccess) return hip_fail(ctx, e, "weight stage alloc");
    uint8_t* dst = (uint8_t*) ctx->w_stage.p;
    uint8_t* dsc = dst + qsz;
    const int* flag = nullptr;
    jamhip_status st = upload(ctx, (const uint8_t*) w, dt, row_bytes(dt, ldw), m, rb, G, dst, dsc, &flag);
    if (st != JAMHIP_OK) return st;
    wv->qs = dst;
    wv->sc = dsc;
    wv->G = G;
    wv->r0 = 0;
    wv->fold_ok = 1;
    wv->fold_flag = flag;
    return JAMHIP_OK;
}

bool env_true(const char* name) {
    const char* v = getenv(name);
    return v && (!strcmp(v, "1") || !strcasecmp(v, "true") || !strcasecmp(v, "yes"));
}

// The matrix-core GEMM covers Q4_K, Q5_K, Q6_K (k a multiple of 256), MXFP4, NVFP4, Q4_0, Q8_0 and Q1_0 on
// 32-row-aligned views (launch_gemm_mma), for k up to the activation prep's limit (gemm_prep_fits).
bool mma_path(int dt, int k, const WeightView& wv) {
    if (env_true("JAM_HIP_NO_MMA")) return false;
    return (((dt == Q4_K || dt == Q5_K || dt == Q6_K) && k % 256 == 0) || dt == MXFP4 || dt == NVFP4 || dt == Q4_0 ||
            dt == Q8_0 || dt == Q1_0) &&
           (wv.r0 & 31) == 0 && gemm_prep_fits(k);
}

// mma_path for jam's semantics: also every group of W must fold its block scales exactly (Q8_0, Q4_0, MXFP4,
// Q1_0; repack_kernel). A copy staged by this call has its flag read here, once (a synchronize), and only
// when the call would otherwise take the matrix cores.
bool mma_exact(jamhip_ctx* ctx, int dt, int k, WeightView& wv) {
    if (!mma_path(dt, k, wv)) return false;
    if (wv.fold_flag != nullptr) {
        int ok = 0;
        if (read_fold(ctx, wv.fold_flag, &ok) != JAMHIP_OK) ok = 0;   // unknown: the exact kernels
        wv.fold_ok = ok;
        wv.fold_flag = nullptr;
    }
    return wv.fold_ok != 0;
}

// Smallest n that takes the matrix cores (n >= 8 is F2 either way; small grids split K), from a sweep of
// both paths (graph-timed, rotating weights). The F2 decode kernel reads W once per 8-token tile and wins
// every shape at one tile (n = 8: Q4_K 14336x4096 21.9 us against 28.4). On weights of up to ~17.8M elements
// (4096x4096, 5760x2880, 2880x4096) its tiles run side by side on the idle CUs and it wins through n = 16
// for every dtype (Q8_0 4096x4096 n = 16: 15.2 against 22.9 us) and through n = 32 for Q4_0, Q4_K and
// Q6_K (Q4_K 4096x4096 n = 32: 21.2 against 26.1). On larger weights the matrix cores win from the second
// tile (14336x4096 n = 12: Q8_0 32.7 against 43.1 us), except at k > 8192 where they win from n = 16
// (Q4_0 4096x14336 n = 12: F2 36.3, matrix cores 40.6). JAM_HIP_MMA_MIN_N overrides (tuning).
static int mma_min_n(int dt, int m, int k) {
    const char* v = getenv("JAM_HIP_MMA_MIN_N");
    if (v) return atoi(v) < 8 ? 8 : atoi(v);
    if ((int64_t) m * k <= (int64_t) 17 << 20) return dt == Q4_0 || dt == Q4_K || dt == Q5_K || dt == Q6_K || dt == Q1_0 ? 33 : 17;
    return k > 8192 ? 16 : 9;
}

// Smallest n that takes gemm_kernel, the fallback when mma_path declines (a view not aligned to 32 rows, k
// past the prep's limit); below it the F2 decode kernel, whose time grows linearly in n. Measured
// crossovers: Q8_0 14336x4096 ~60 tokens; at k = 14336 gemm_kernel's small grid takes ~600 us at any n
// (~320 tokens).
// JAM_HIP_GEMM_MIN_N overrides (tuning).
static int gemm_min_n(int dt, int k) {
    const char* v = getenv("JAM_HIP_GEMM_MIN_N");
    const int x = v ? atoi(v) : k >= 8192 ? 320 : dt == Q8_0 ? 64 : 96;
    return x < 8 ? 8 : x;
}

// Where compute() takes its device scratch: the context's growable buffers, or (the allocation-free entry
// point) consecutive 256-byte-aligned pieces of one fixed region. Every branch of compute() takes all its
// pieces before its first launch, so a call that does not fit the fixed region queues nothing.
struct Scratch {
    jamhip_ctx* ctx;
    uint8_t* fixed = nullptr;   // null: the context's DevBufs
    size_t cap = 0, used = 0;
    size_t over = 0;            // fixed mode: the bytes a refused piece would have needed in total
    hipError_t get(DevBuf& b, size_t bytes, void** out) {
        if (!fixed) {
            const hipError_t e = b.ensure(bytes);
            *out = b.p;
            return e;
        }
        const size_t at = (used + 255) & ~(size_t) 255;
        if (at + bytes > cap) {
            over = at + bytes;
            return hipErrorOutOfMemory;
        }
        *out = fixed + at;
        used = at + bytes;
        return hipSuccess;
    }
};

jamhip_status scratch_fail(jamhip_ctx* ctx, const Scratch& sc, hipError_t e, const char* what) {
    if (sc.fixed && sc.over)
        return fail(ctx, JAMHIP_EUNSUPPORTED,
                    std::string(what) + ": the call needs " + std::to_string(sc.over) +
                        " bytes of scratch, above the static scratch maximum of " + std::to_string(sc.cap) +
                        " bytes (use jamhip_mm_device)");
    return hip_fail(ctx, e, what);
}

// Quantize A (device, f32 [n][lda]) and run the matmul into C (device, [n][ldc]). Decode-sized calls
// with k < 8192 are one fused launch and touch no scratch (safe under stream capture once W is pinned);
// from k = 8192 (one token: past k = 65536) the decode kernels split K and sum the slices from the context's
// split buffer.
jamhip_status compute(jamhip_ctx* ctx, Scratch& sc, int dt, WeightView wv, const float* a, int lda, float* c,
                      int ldc, int m, int n, int k, const Epi& ep = Epi{}) {
    hipError_t e;
    float* gpart = nullptr;   // the decode kernels' K-split partials
    auto decode_part = [&](int rows) -> hipError_t {
        const size_t pf = gemv_split_floats(k, rows, n);
        if (pf == 0) return hipSuccess;
        return sc.get(ctx->part, pf * sizeof(float), (void**) &gpart);
    };
    if (is_dense(dt)) {   // jam's dense paths: no activation quantization
        if (dense_mma_planes(dt, n, k) > 0) {   // the staged matrix-core GEMM: operand-ordered activations
            void* dact = nullptr;
            float* part = nullptr;
            if ((e = sc.get(ctx->gact, dense_act_bytes(dt, n, k), &dact)) != hipSuccess)
                return scratch_fail(ctx, sc, e, "dense activation scratch");
            if (const size_t pf = dense_mma_split_floats(dt, k, m, n))
                if ((e = sc.get(ctx->part, pf * sizeof(float), (void**) &part)) != hipSuccess)
                    return scratch_fail(ctx, sc, e, "dense split scratch");
            if ((e = launch_dense_mma(dt, wv, a, lda, k, m, n, c, ldc, dact, part, ctx->stream, ep)) != hipSuccess)
                return hip_fail(ctx, e, "dense gemm launch");
            return JAMHIP_OK;
        }
        if ((e = launch_dense(dt, wv, a, lda, k, m, n, c, ldc, ctx->stream, ep)) != hipSuccess)
            return hip_fail(ctx, e, "dense launch");
        return JAMHIP_OK;
    }
    if (gemv_fusable(n, k, a, lda)) {
        if ((e = decode_part(m)) != hipSuccess) return scratch_fail(ctx, sc, e, "gemv split scratch");
        if ((e = launch_gemv(dt, 1, wv, ActQ{}, a, lda, k, m, n, c, ldc, ctx->stream, gpart, ep)) != hipSuccess)
            return hip_fail(ctx, e, "gemv launch");
        return JAMHIP_OK;
    }
    // n >= 8: jam's 16-row F2 bands on rows [0, m16); the last m % 16 rows take the band's float-dot tail
    // (jam_kernels_q4k_avx512.c:185-188).
    const int m16 = m - m % 16;
    if (dt == MXFP4 && ctx->mx_native && n >= mma_min_n(dt, m, k) && mma_path(dt, k, wv)) {
        // opt-in native MX (not jam's activation semantics): every row on the scaled fp4 x fp8 MFMA
        MxAct X;
        void* gact = nullptr;
        if ((e = sc.get(ctx->gact, mx_act_bytes_np((n + 63) / 64 * 64, k), &gact)) != hipSuccess)
            return scratch_fail(ctx, sc, e, "mx activation scratch");
        if ((e = launch_mx_prep(a, lda, n, k, ctx->mx_native, gact, &X, ctx->stream)) != hipSuccess)
            return hip_fail(ctx, e, "mx prep launch");
        if ((e = launch_mx_gemm(ctx->mx_native, wv, X, m, n, c, ldc, ctx->stream, ep)) != hipSuccess)
            return hip_fail(ctx, e, "mx gemm launch");
        return JAMHIP_OK;
    }
    // NVFP4 has no 16-row band in jam (F1 on every row at every n, jam.c:662-668): all m rows on the matrix cores
    const int mm_rows = dt == NVFP4 ? m : m16;
    if (n >= mma_min_n(dt, m, k) && mm_rows > 0 && mma_exact(ctx, dt, k, wv)) {
        GemmAct G;
        void* gact = nullptr;
        float* part = nullptr;
        if ((e = sc.get(ctx->gact, gemm_act_bytes(dt, n, k), &gact)) != hipSuccess)
            return scratch_fail(ctx, sc, e, "gemm activation scratch");
        if (const size_t pf = gemm_mma_split_floats(dt, k, mm_rows, n))
            if ((e = sc.get(ctx->part, pf * sizeof(float), (void**) &part)) != hipSuccess)
                return scratch_fail(ctx, sc, e, "gemm split scratch");
        if ((e = launch_gemm_prep(dt, a, lda, n, k, gact, &G, ctx->stream)) != hipSuccess)
            return hip_fail(ctx, e, "gemm prep launch");
        if ((e = launch_gemm_mma(dt, wv, G, k, mm_rows, n, c, ldc, ctx->stream, part, ep)) != hipSuccess)
            return hip_fail(ctx, e, "gemm launch");
        if (mm_rows < m &&
            (e = launch_rows_float(dt, wv, a, lda, k, m16, m - m16, n, c, ldc, ctx->stream, ep)) != hipSuccess)
            return hip_fail(ctx, e, "tail rows launch");
        return JAMHIP_OK;
    }
    const int64_t nb = k / 32;
    const int64_t qb = align256((int64_t) n * k), db = align256(n * nb * 4), sb = align256((int64_t) n * (k / 16) * 4);
    uint8_t* base = nullptr;
    if ((e = sc.get(ctx->act, (size_t) (qb + db + 2 * sb), (void**) &base)) != hipSuccess)
        return scratch_fail(ctx, sc, e, "activation scratch");
    int8_t* q = (int8_t*) base;
    float* d = (float*) (base + qb);
    float* s = (float*) (base + qb + db);
    int* s16 = (int*) (base + qb + db + sb);
    const ActQ A{q, d, s, s16};
    if (n < 8 || dt == NVFP4) {   // F1 on every row: decode, and NVFP4 at any n (jam.c:662-668)
        if ((e = decode_part(m)) != hipSuccess) return scratch_fail(ctx, sc, e, "gemv split scratch");
        if ((e = launch_quant_f1(a, lda, n, k, q, d, s, s16, ctx->stream)) != hipSuccess)
            return hip_fail(ctx, e, "quant_f1 launch");
        if ((e = launch_gemv(dt, n < 8 ? 1 : 3, wv, A, nullptr, 0, k, m, n, c, ldc, ctx->stream, gpart, ep)) != hipSuccess)
            return hip_fail(ctx, e, "gemv launch");
        return JAMHIP_OK;
    }
    if (m16 > 0) {
        const bool gemm = n >= gemm_min_n(dt, k) && gemm_covers(dt);
        if (!gemm && (e = decode_part(m16)) != hipSuccess) return scratch_fail(ctx, sc, e, "gemv split scratch");
        if ((e = launch_quant_f2(a, lda, n, k, q, d, s, ctx->stream)) != hipSuccess)
            return hip_fail(ctx, e, "quant_f2 launch");
        e = gemm ? launch_gemm(dt, wv, A, k, m16, n, c, ldc, ctx->stream, ep)
                 : launch_gemv(dt, 2, wv, A, nullptr, 0, k, m16, n, c, ldc, ctx->stream, gpart, ep);
        if (e != hipSuccess) return hip_fail(ctx, e, "matmul launch");
    }
    if ((e = launch_rows_float(dt, wv, a, lda, k, m16, m - m16, n, c, ldc, ctx->stream, ep)) != hipSuccess)
        return hip_fail(ctx, e, "tail rows launch");
    return JAMHIP_OK;
}

jamhip_status compute(jamhip_ctx* ctx, int dt, const WeightView& wv, const float* a, int lda, float* c, int ldc,
                      int m, int n, int k, const Epi& ep = Epi{}) {
    Scratch sc{ctx};
    return compute(ctx, sc, dt, wv, a, lda, c, ldc, m, n, k, ep);
}

// Drop the pin that starts at host (caller holds the Busy guard, device current); false if none does.
bool evict_at(jamhip_ctx* ctx, uintptr_t host) {
    std::lock_guard<std::mutex> lk(ctx->pin_mu);
    auto it = std::lower_bound(ctx->pins.begin(), ctx->pins.end(), host,
                               [](const Pin& pin, uintptr_t v) { return pin.host < v; });
    if (it == ctx->pins.end() || it->host != host) return false;
    (void) hipStreamSynchronize(ctx->stream);
    (void) hipFree(it->dev);
    ctx->pinned_bytes -= it->bytes;
    if (!it->pages.empty()) ctx->autopin_bytes -= it->bytes;
    ctx->pins.erase(it);
    return true;
}

// Pin rows [0, m) of the host tensor at w (caller holds the Busy guard, device current). The staging
// buffer is kept when `keep_staging` (a registry load reuses it for every tensor). An explicit pin (the
// caller's jamhip_weight_pin or a registry load, not autopin) takes over autopins in its way: they are
// evicted and the range is copied afresh (an autopin's copy is only spot-checked, so it may predate the bytes
// the caller is pinning); an overlapping explicit pin is an error.
jamhip_status pin_range(jamhip_ctx* ctx, const void* w, int wt, int ldw, int64_t m, bool keep_staging,
                        bool explicit_pin) {
    const uintptr_t host = reinterpret_cast<uintptr_t>(w);
    const int64_t rb = ldw / block_elems(wt), G = view_G(wt, ldw), span = m * row_bytes(wt, ldw);
    std::vector<uintptr_t> drop;   // autopins overlapping [host, host + span)
    {
        std::lock_guard<std::mutex> lk(ctx->pin_mu);
        auto it = std::lower_bound(ctx->pins.begin(), ctx->pins.end(), host,
                                   [](const Pin& pin, uintptr_t v) { return pin.host < v; });
        if (it != ctx->pins.end() && it->host == host && it->dt == wt && it->ldw == ldw && it->rows == m &&
            it->pages.empty() == explicit_pin)
            return JAMHIP_OK;   // already pinned
        auto first = it;
        if (first != ctx->pins.begin() && host < (first - 1)->host + (uintptr_t) (first - 1)->span) --first;
        for (auto p = first; p != ctx->pins.end() && p->host < host + (uintptr_t) span; ++p) {
            if (!explicit_pin || p->pages.empty())
                return fail(ctx, JAMHIP_EINVAL, "pin: range overlaps a pinned tensor (evict it first)");
            drop.push_back(p->host);
        }
    }
    for (uintptr_t h : drop) evict_at(ctx, h);
    const int64_t qsz = plane0_bytes(wt, m, ldw), ssz = plane1_bytes(wt, m, ldw);
    uint8_t* dev = nullptr;
    hipError_t e = hipMalloc((void**) &dev, (size_t) (qsz + ssz));
    if (e != hipSuccess) return hip_fail(ctx, e, "pin: device alloc");
    uint8_t* sc = dev + qsz;
    const int* flag = nullptr;
    int fold_ok = 1;
    jamhip_status st = upload(ctx, (const uint8_t*) w, wt, row_bytes(wt, ldw), m, rb, G, dev, sc, &flag);
    if (st == JAMHIP_OK && (e = hipStreamSynchronize(ctx->stream)) != hipSuccess) st = hip_fail(ctx, e, "pin: sync");
    if (st == JAMHIP_OK && flag) st = read_fold(ctx, flag, &fold_ok);
    if (st != JAMHIP_OK) {
        (void) hipFree(dev);
        return st;
    }
    if (!keep_staging) ctx->w_raw.release();   // staging is sized to the tensor; do not hold it
    std::lock_guard<std::mutex> lk(ctx->pin_mu);
    auto it = std::lower_bound(ctx->pins.begin(), ctx->pins.end(), host,
                               [](const Pin& pin, uintptr_t v) { return pin.host < v; });
    Pin pin{host, span, wt, ldw, m, G, dev, sc, qsz + ssz};
    pin.fold_ok = fold_ok;
    ctx->pins.insert(it, std::move(pin));
    ctx->pinned_bytes += qsz + ssz;
    return JAMHIP_OK;
}

// ---- autopin: residency for callers that never pin (an unedited jinfer passes the same mmap'd address for
// a tensor on every call, MatMul.java:1783-1830). A range is pinned on its N-th sighting; from then on each
// call spot-checks two 4 KiB pages of the host range against the hashes taken at pin time (a rotating page
// and a scattered one, so repeated calls sweep the whole range), and a mismatch (the caller rewrote the
// range in place, e.g. an arena reused for another tensor) evicts the pin and stages the call.
constexpr int64_t AUTOPIN_PAGE = 4096;
constexpr size_t AUTOPIN_SIGHTS = 4096;

// 64-bit hash of `bytes` host bytes (a multiply-xorshift over 8-byte words, then the tail bytes).
uint64_t page_hash(const uint8_t* p, int64_t bytes) {
    uint64_t h = 0x243F6A8885A308D3ull ^ (uint64_t) bytes;
    int64_t i = 0;
    for (; i + 8 <= bytes; i += 8) {
        uint64_t w;
        std::memcpy(&w, p + i, 8);
        h = (h ^ w) * 0x9E3779B97F4A7C15ull;
        h ^= h >> 29;
    }
    for (; i < bytes; i++) h = (h ^ p[i]) * 0x100000001B3ull;
    return h;
}

std::vector<uint64_t> range_hashes(const uint8_t* p, int64_t span) {
    std::vector<uint64_t> v((size_t) ((span + AUTOPIN_PAGE - 1) / AUTOPIN_PAGE));
    for (size_t i = 0; i < v.size(); i++)
        v[i] = page_hash(p + (int64_t) i * AUTOPIN_PAGE, std::min(AUTOPIN_PAGE, span - (int64_t) i * AUTOPIN_PAGE));
    return v;
}

// The autopin (if any) that serves W: true with its device view after the spot check passes; a failed check
// evicts it (the call then stages).
bool autopin_lookup(jamhip_ctx* ctx, const void* w, int dt, int ldw, int m, WeightView* out) {
    uintptr_t host = 0;
    {
        std::lock_guard<std::mutex> lk(ctx->pin_mu);
        const uintptr_t p = reinterpret_cast<uintptr_t>(w);
        auto it = std::upper_bound(ctx->pins.begin(), ctx->pins.end(), p,
                                   [](uintptr_t v, const Pin& pin) { return v < pin.host; });
        if (it == ctx->pins.begin()) return false;
        Pin& pin = *(it - 1);
        if (pin.pages.empty() || pin.host != p || pin.dt != dt || pin.ldw != ldw || pin.rows < m) return false;
        const uint64_t np = pin.pages.size(), c = pin.checks++;
        const uint64_t pg[2] = {c % np, (c * 2654435761ull + 1) % np};
        bool same = true;
        for (uint64_t i : pg) {
            const int64_t at = (int64_t) i * AUTOPIN_PAGE;
            same = same && page_hash((const uint8_t*) pin.host + at, std::min(AUTOPIN_PAGE, pin.span - at)) == pin.pages[i];
        }
        if (same) {
            out->qs = pin.dev;
            out->sc = pin.sc;
            out->G = pin.G;
            out->r0 = 0;
            out->fold_ok = pin.fold_ok;
            out->fold_flag = nullptr;
            ctx->ap_stats[1]++;
            return true;
        }
        host = pin.host;
        ctx->ap_stats[3]++;
    }
    evict_at(ctx, host);
    return false;
}

// Count a sighting of a non-resident W; on the autopin-th, pin it (a failed pin, e.g. out of device memory or
// over the cap, leaves the call staged). Only whole contiguous matrices are taken (ldw == k), so the bytes
// pinned and hashed are exactly the bytes the call reads.
void autopin_sight(jamhip_ctx* ctx, const void* w, int dt, int ldw, int m, int k) {
    if (ctx->autopin <= 0 || ldw != k) return;
    const uintptr_t host = reinterpret_cast<uintptr_t>(w);
    const int64_t span = (int64_t) m * row_bytes(dt, ldw);
    bool pin_now = false;
    {
        std::lock_guard<std::mutex> lk(ctx->pin_mu);
        auto it = std::find_if(ctx->sights.begin(), ctx->sights.end(), [&](const Sight& s) {
            return s.host == host && s.dt == dt && s.ldw == ldw && s.rows == m;
        });
        if (it == ctx->sights.end()) {
            if (ctx->sights.size() >= AUTOPIN_SIGHTS) ctx->sights.erase(ctx->sights.begin(), ctx->sights.begin() + AUTOPIN_SIGHTS / 2);
            ctx->sights.push_back(Sight{host, dt, ldw, m, 0});
            it = ctx->sights.end() - 1;
        }
        if (++it->count >= ctx->autopin) {
            const int64_t dev_bytes = plane0_bytes(dt, m, ldw) + plane1_bytes(dt, m, ldw);
            pin_now = ctx->autopin_cap <= 0 || ctx->autopin_bytes + dev_bytes <= ctx->autopin_cap;
            ctx->sights.erase(it);
        }
    }
    if (!pin_now) return;
    std::vector<uint64_t> pages = range_hashes((const uint8_t*) w, span);
    if (pin_range(ctx, w, dt, ldw, m, true, false) != JAMHIP_OK) return;   // overlap, allocation: stay staged
    std::lock_guard<std::mutex> lk(ctx->pin_mu);
    auto it = std::lower_bound(ctx->pins.begin(), ctx->pins.end(), host,
                               [](const Pin& pin, uintptr_t v) { return pin.host < v; });
    if (it != ctx->pins.end() && it->host == host && it->pages.empty()) {
        it->pages = std::move(pages);
        ctx->autopin_bytes += it->bytes;
        ctx->ap_stats[0]++;
    }
}

}  // namespace

namespace {

// Synchronizes the stream when a call returns early after queueing a copy from a pinned bounce buffer, so
// the next call may reuse or free that buffer.
struct SyncOnError {
    jamhip_ctx* ctx;
    bool armed = false;
    ~SyncOnError() {
        if (armed) (void) hipStreamSynchronize(ctx->stream);
    }
};

// Largest A / C (bytes) that jamhip_mm moves by the shader cores: A uploaded by a copy kernel, C stored by the
// matmul kernels straight into the pinned bounce buffer.
constexpr size_t kDirectCBytes = 1 << 20;

jamhip_status mm_impl(jamhip_ctx* ctx, const void* w, int wt, int ldw, const void* a, int at, int lda, void* c,
                        int ct, int ldc, int m, int n, int k) {
    jamhip_status st = validate(ctx, w, wt, ldw, a, at, lda, c, ct, ldc, m, n, k);
    if (st != JAMHIP_OK) return st;
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    WeightView wv;
    bool served = false;   // by an autopin whose spot check passed
    if (ctx->autopin > 0 && !(served = autopin_lookup(ctx, w, wt, ldw, m, &wv))) {
        WeightView probe;
        if (!lookup(ctx, w, wt, ldw, m, &probe)) {   // not resident by an explicit pin: count the sighting
            autopin_sight(ctx, w, wt, ldw, m, k);
            if (!(served = autopin_lookup(ctx, w, wt, ldw, m, &wv))) {
                std::lock_guard<std::mutex> lk(ctx->pin_mu);
                ctx->ap_stats[2]++;
            }
        }
    }
    // an explicit pin, else a staged copy (an autopinned range is never served without its check)
    if (!served && (st = resolve_w(ctx, w, wt, ldw, m, k, &wv)) != JAMHIP_OK) return st;
    hipError_t e;
    const size_t abytes = (size_t) n * k * 4, cbytes = (size_t) n * m * 4;
    if ((e = ctx->a_stage.ensure(abytes)) != hipSuccess) return hip_fail(ctx, e, "A staging alloc");
    if ((e = ctx->c_stage.ensure(cbytes)) != hipSuccess) return hip_fail(ctx, e, "C staging alloc");
    if ((e = ctx->a_host.ensure(abytes)) != hipSuccess) return hip_fail(ctx, e, "A pinned alloc");
    if ((e = ctx->c_host.ensure(cbytes)) != hipSuccess) return hip_fail(ctx, e, "C pinned alloc");
    // A's rows packed into the pinned buffer (lda >= k), then one contiguous transfer
    const float* af = static_cast<const float*>(a);
    float* ah = static_cast<float*>(ctx->a_host.p);
    for (int j = 0; j < n; j++) std::memcpy(ah + (size_t) j * k, af + (size_t) j * lda, (size_t) k * 4);
    SyncOnError pending{ctx};
    // a small A goes up by a copy kernel reading the pinned buffer (lower latency than the runtime's copy)
    if (abytes <= kDirectCBytes && abytes % 16 == 0)
        e = launch_stage_copy(ah, ctx->a_stage.p, abytes, ctx->stream);
    else
        e = hipMemcpyAsync(ctx->a_stage.p, ah, abytes, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "A upload");
    pending.armed = true;
    // A small C (decode: m floats per token) is stored by the kernels straight into the pinned buffer, which
    // the device addresses directly: no separate device-to-host copy. A large one goes through device memory
    // and one copy.
    const bool direct_c = cbytes <= kDirectCBytes;
    float* cdst = static_cast<float*>(direct_c ? ctx->c_host.p : ctx->c_stage.p);
    if ((st = compute(ctx, wt, wv, (const float*) ctx->a_stage.p, k, cdst, m, m, n, k)) != JAMHIP_OK) return st;
    if (!direct_c &&
        (e = hipMemcpyAsync(ctx->c_host.p, ctx->c_stage.p, cbytes, hipMemcpyDeviceToHost, ctx->stream)) != hipSuccess)
        return hip_fail(ctx, e, "C download");
    pending.armed = false;
    if ((e = hipStreamSynchronize(ctx->stream)) != hipSuccess) return hip_fail(ctx, e, "stream sync");
    // C columns [m, ldc) stay untouched (jam.h:131-138): m floats per token row
    const float* ch = static_cast<const float*>(ctx->c_host.p);
    float* cf = static_cast<float*>(c);
    for (int j = 0; j < n; j++) std::memcpy(cf + (size_t) j * ldc, ch + (size_t) j * m, (size_t) m * 4);
    return JAMHIP_OK;
}

jamhip_status mm_device_impl(jamhip_ctx* ctx, const void* w, int wt, int ldw, const void* a_dev, int at, int lda,
                               void* c_dev, int ct, int ldc, int m, int n, int k) {
    jamhip_status st = validate(ctx, w, wt, ldw, a_dev, at, lda, c_dev, ct, ldc, m, n, k);
    if (st != JAMHIP_OK) return st;
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    WeightView wv;
    if ((st = resolve_w(ctx, w, wt, ldw, m, k, &wv)) != JAMHIP_OK) return st;
    return compute(ctx, wt, wv, (const float*) a_dev, lda, (float*) c_dev, ldc, m, n, k);
}

// jamhip_mm_device with W required resident and every piece of scratch taken from the device's static array:
// no allocation of any kind on the call's path.
jamhip_status mm_device_noalloc_impl(jamhip_ctx* ctx, const void* w, int wt, int ldw, const void* a_dev, int at,
                                     int lda, void* c_dev, int ct, int ldc, int m, int n, int k) {
    jamhip_status st = validate(ctx, w, wt, ldw, a_dev, at, lda, c_dev, ct, ldc, m, n, k);
    if (st != JAMHIP_OK) return st;
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    uint8_t* base = noalloc_scratch(ctx->device);
    if (!base) return fail(ctx, JAMHIP_EINVAL, "noalloc: the static scratch array has no device address on this device");
    WeightView wv;
    if (!lookup(ctx, w, wt, ldw, m, &wv))
        return fail(ctx, JAMHIP_EUNSUPPORTED, "noalloc: W is not resident (pin it first: staging it would allocate)");
    Scratch sc{ctx, base, NOALLOC_SCRATCH_BYTES};
    return compute(ctx, sc, wt, wv, (const float*) a_dev, lda, (float*) c_dev, ldc, m, n, k);
}

jamhip_status mm_device_ex_impl(jamhip_ctx* ctx, const void* w, int wt, int ldw, const void* a_dev, int at, int lda,
                                  void* c_dev, int ct, int ldc, int m, int n, int k, const void* bias_dev,
                                  int accumulate) {
    jamhip_status st = validate(ctx, w, wt, ldw, a_dev, at, lda, c_dev, ct, ldc, m, n, k);
    if (st != JAMHIP_OK) return st;
    if (accumulate != 0 && accumulate != 1) return fail(ctx, JAMHIP_EINVAL, "accumulate must be 0 or 1");
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    WeightView wv;
    if ((st = resolve_w(ctx, w, wt, ldw, m, k, &wv)) != JAMHIP_OK) return st;
    Epi ep;
    ep.bias = static_cast<const float*>(bias_dev);
    ep.accumulate = accumulate;
    return compute(ctx, wt, wv, (const float*) a_dev, lda, (float*) c_dev, ldc, m, n, k, ep);
}

jamhip_status glu_device_impl(jamhip_ctx* ctx, int act, void* gate_dev, int ldg, const void* up_dev, int ldu,
                                int rows, int cols, int lanes = 0) {
    if (!ctx) return JAMHIP_EINVAL;
    if (!gate_dev || !up_dev) return fail(ctx, JAMHIP_EINVAL, "glu: null operand");
    if (rows < 0 || cols < 0 || ldg < cols || ldu < cols) return fail(ctx, JAMHIP_EINVAL, "glu: bad extents");
    if (act != JAMHIP_ACT_SWIGLU && act != JAMHIP_ACT_SWIGLU_OAI)
        return fail(ctx, JAMHIP_EUNSUPPORTED, "glu: unknown activation");
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    if (lanes < 0) return fail(ctx, JAMHIP_EINVAL, "glu: lanes must be >= 0");
    const hipError_t e = launch_glu(act, (float*) gate_dev, ldg, (const float*) up_dev, ldu, rows, cols, ctx->stream,
                                    lanes);
    return e == hipSuccess ? JAMHIP_OK : hip_fail(ctx, e, "glu launch");
}

jamhip_status read_floor_impl(jamhip_ctx* ctx, const void* p, int64_t bytes, void* sink) {
    if (!ctx) return JAMHIP_EINVAL;
    if (!p || !sink || bytes < 0 || bytes % 16 || (reinterpret_cast<uintptr_t>(p) & 15))
        return fail(ctx, JAMHIP_EINVAL, "read_floor: null pointer, or bytes / address not 16-byte aligned");
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    const hipError_t e = launch_read_floor(p, bytes, (uint32_t*) sink, ctx->stream);
    return e == hipSuccess ? JAMHIP_OK : hip_fail(ctx, e, "read_floor launch");
}

jamhip_status weight_pin_impl(jamhip_ctx* ctx, const void* w, int wt, int ldw, int m) {
    if (!ctx) return JAMHIP_EINVAL;
    if (!w || m <= 0 || ldw <= 0) return fail(ctx, JAMHIP_EINVAL, "pin: null weight or empty shape");
    if (!supported_w(wt)) return fail(ctx, JAMHIP_EUNSUPPORTED, "pin: weight dtype not supported");
    const int be = block_elems(wt);   // whole rows of ldw elements: at least one block, on the block where jam needs it
    if (ldw < be || !block_aligned(wt, ldw, ldw / be * be))
        return fail(ctx, JAMHIP_EUNSUPPORTED, "pin: ldw not a block multiple");
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    return pin_range(ctx, w, wt, ldw, m, false, true);
}

jamhip_status set_autopin_impl(jamhip_ctx* ctx, int sightings, int64_t max_bytes) {
    if (!ctx) return JAMHIP_EINVAL;
    if (sightings < 0 || max_bytes < 0) return fail(ctx, JAMHIP_EINVAL, "autopin: sightings and max_bytes must be >= 0");
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    std::lock_guard<std::mutex> lk(ctx->pin_mu);
    ctx->autopin = sightings;
    ctx->autopin_cap = max_bytes;
    if (sightings == 0) ctx->sights.clear();
    return JAMHIP_OK;
}

jamhip_status set_mx_native_impl(jamhip_ctx* ctx, int mode) {
    if (!ctx) return JAMHIP_EINVAL;
    if (mode < 0 || mode > 2) return fail(ctx, JAMHIP_EINVAL, "mx_native: mode must be 0, 1 or 2");
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    ctx->mx_native = mode;
    return JAMHIP_OK;
}

jamhip_status weight_evict_impl(jamhip_ctx* ctx, const void* w) {
    if (!ctx || !w) return JAMHIP_EINVAL;
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    if (!evict_at(ctx, reinterpret_cast<uintptr_t>(w))) return fail(ctx, JAMHIP_EINVAL, "evict: no pinned tensor starts at this address");
    return JAMHIP_OK;
}


jamhip_status quantize_device_impl(jamhip_ctx* ctx, int flavour, const void* a_dev, int lda, int n, int k,
                                     void* q_dev, void* d_dev, void* s_dev) {
    if (!ctx) return JAMHIP_EINVAL;
    if (!a_dev || !q_dev || !d_dev || !s_dev) return fail(ctx, JAMHIP_EINVAL, "quantize: null pointer");
    if (n <= 0 || k <= 0 || lda < k) return fail(ctx, JAMHIP_EINVAL, "quantize: bad shape");
    if (k % 32) return fail(ctx, JAMHIP_EUNSUPPORTED, "quantize: k must be a multiple of 32");
    if (flavour != 1 && flavour != 2) return fail(ctx, JAMHIP_EINVAL, "quantize: flavour must be 1 or 2");
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    hipError_t e;
    if (flavour == 1) {
        if ((e = ctx->act.ensure((size_t) n * (k / 16) * 4)) != hipSuccess) return hip_fail(ctx, e, "scratch alloc");
        e = launch_quant_f1((const float*) a_dev, lda, n, k, (int8_t*) q_dev, (float*) d_dev, (float*) s_dev,
                            (int*) ctx->act.p, ctx->stream);
    } else {
        e = launch_quant_f2((const float*) a_dev, lda, n, k, (int8_t*) q_dev, (float*) d_dev, (float*) s_dev,
                            ctx->stream);
    }
    return e == hipSuccess ? JAMHIP_OK : hip_fail(ctx, e, "quantize launch");
}

// x_rows (gathered input): CSR row r of A is row x_rows[r] / rdiv of a_dev (jamhip_moe_gather folded in); the
// fused preps read it there, the other paths gather the rows into scratch first.
jamhip_status mm_grouped_ex_impl(jamhip_ctx* ctx, const void* w, int wt, int ldw, int m, int n_experts,
                                   const void* counts_dev, const void* a_dev, int at, int lda, void* c_dev, int ct,
                                   int ldc, int k, int rows_cap, void* offsets_dev, const void* bias_dev,
                                   const int* x_rows = nullptr, int rdiv = 1) {
    if (!ctx) return JAMHIP_EINVAL;
    if (!w || !counts_dev || !a_dev || !c_dev) return fail(ctx, JAMHIP_EINVAL, "grouped: null operand");
    if (rdiv < 1) return fail(ctx, JAMHIP_EINVAL, "grouped gather: topk must be positive");
    if (m <= 0 || k <= 0 || n_experts <= 0 || rows_cap < 0)
        return fail(ctx, JAMHIP_EINVAL, "grouped: m, k, n_experts must be positive and rows_cap >= 0");
    if (ldw < k || lda < k || ldc < m) return fail(ctx, JAMHIP_EINVAL, "grouped: stride below extent");
    if (at != F32 || ct != F32) return fail(ctx, JAMHIP_EUNSUPPORTED, "grouped: A and C must be F32");
    if (!grouped_w(wt)) return fail(ctx, JAMHIP_EUNSUPPORTED, "grouped: weight dtype not supported");
    if (k % block_elems(wt) || ldw % block_elems(wt))
        return fail(ctx, JAMHIP_EUNSUPPORTED, "grouped: k and ldw must be multiples of the block size");
    if (m % 16) return fail(ctx, JAMHIP_EUNSUPPORTED, "grouped: m must be a multiple of 16");
    if (n_experts > 1024) return fail(ctx, JAMHIP_EUNSUPPORTED, "grouped: at most 1024 experts");
    if ((int64_t) m * n_experts > INT32_MAX) return fail(ctx, JAMHIP_EUNSUPPORTED, "grouped: too many rows");
    // the device prefix sums of the (rows_cap-clamped) counts stay below n_experts·rows_cap
    if ((int64_t) rows_cap * n_experts >= INT32_MAX)
        return fail(ctx, JAMHIP_EUNSUPPORTED, "grouped: n_experts·rows_cap must be below 2^31");
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    jamhip_status st;
    WeightView wv;
    if ((st = resolve_w(ctx, w, wt, ldw, m * n_experts, k, &wv)) != JAMHIP_OK) return st;
    const int E = n_experts;
    const int cap64 = (int) (((int64_t) rows_cap + 63 * E + 63) / 64), cap8 = (int) (((int64_t) rows_cap + 7 * E + 7) / 8);
    hipError_t e;
    if ((e = ctx->moe.ensure((size_t) (3 * (E + 1) + cap64 + cap8 + 2 * E) * sizeof(int))) != hipSuccess)
        return hip_fail(ctx, e, "grouped: scratch alloc");
    int* off = (int*) ctx->moe.p;
    int* poff64 = off + (E + 1);
    int* poff8 = poff64 + (E + 1);
    int* map64 = poff8 + (E + 1);
    int* map8 = map64 + cap64;
    // the F1 decode kernels' workgroup columns: the experts with one row (at most rows_cap of them), then
    // those with 2..7 rows (at most rows_cap / 2)
    int* small = map8 + cap8;
    const int n1 = E < rows_cap ? E : rows_cap, n2 = E < rows_cap / 2 ? E : rows_cap / 2;
    const float* a = (const float*) a_dev;
    float* c = (float*) c_dev;
    // Matrix-core path with at least 8 rows per expert on average: one prep launch builds the offsets and the
    // slot map from the device counts and quantizes every expert's rows (F1 for experts of 1..7 rows, whose
    // 64-slot blocks then take the GEMM's single-token-tile form), so neither the offsets kernel nor the F1
    // decode launch runs. Sparser calls keep the F1 decode kernel for their small experts.
    // Native-MX mode, the same density: one prep launch (expert table from the counts, MX-FP8 codes of every
    // expert's rows) and the native GEMM over every expert, those with fewer than 8 rows included.
    if (rows_cap >= 8 * E && E <= PREP_FUSED_MAX_E && m % 32 == 0 && wt == MXFP4 && ctx->mx_native &&
        mma_path(wt, k, wv)) {
        const PrepGroups pg{(const int*) counts_dev, E, rows_cap, off, poff64, map64, cap64, (int*) offsets_dev,
                            x_rows, rdiv};
        const Groups g{off, poff8, map8, poff64, map64, m, static_cast<const float*>(bias_dev)};
        MxAct X;
        if ((e = ctx->gact.ensure(mx_act_bytes_np(cap64 * 64, k))) != hipSuccess)
            return hip_fail(ctx, e, "grouped: mx activation scratch alloc");
        if ((e = launch_mx_prep_grouped_fused(a, lda, k, ctx->mx_native, pg, ctx->gact.p, &X, ctx->stream)) !=
                hipSuccess ||
            (e = launch_mx_gemm_grouped(ctx->mx_native, wv, X, g, cap64, c, ldc, ctx->stream)) != hipSuccess)
            return hip_fail(ctx, e, "grouped: mx gemm launch");
        return JAMHIP_OK;
    }
    if (rows_cap >= 8 * E && E <= PREP_FUSED_MAX_E && m % 32 == 0 && !(wt == MXFP4 && ctx->mx_native) &&
        mma_exact(ctx, wt, k, wv)) {
        const PrepGroups pg{(const int*) counts_dev, E, rows_cap, off, poff64, map64, cap64, (int*) offsets_dev,
                            x_rows, rdiv};
        const Groups g{off, poff8, map8, poff64, map64, m, static_cast<const float*>(bias_dev)};
        GemmAct G;
        if ((e = ctx->gact.ensure(gemm_act_bytes_np(wt, cap64 * 64, k))) != hipSuccess)
            return hip_fail(ctx, e, "grouped: gemm activation scratch alloc");
        if ((e = launch_gemm_prep_grouped_fused(wt, a, lda, k, pg, ctx->gact.p, &G, ctx->stream)) != hipSuccess ||
            (e = launch_gemm_mma_grouped(wt, wv, G, k, g, cap64, c, ldc, ctx->stream)) != hipSuccess)
            return hip_fail(ctx, e, "grouped: gemm launch");
        return JAMHIP_OK;
    }
    // Decode-sized calls (fewer than 8 rows in all, at most 64 experts, no offsets asked for; a gather only where
    // the fused prologue reads the routed rows itself): the F1 kernels find their experts and rows from the
    // counts, so neither the offsets kernel nor the gather runs.
    const bool derive = rows_cap < 8 && E <= 64 && offsets_dev == nullptr &&
                        (x_rows == nullptr || gemv_grouped_fusable(k, a, lda));   // a gather folds into the prologue
    if (!derive && (e = launch_moe_offsets((const int*) counts_dev, E, rows_cap, off, poff64, poff8, map64, cap64,
                                           map8, cap8, small, n1, n2, ctx->stream)) != hipSuccess)
        return hip_fail(ctx, e, "grouped: offsets launch");
    if (offsets_dev &&
        (e = hipMemcpyAsync(offsets_dev, off, (size_t) (E + 1) * sizeof(int), hipMemcpyDeviceToDevice, ctx->stream)) !=
            hipSuccess)
        return hip_fail(ctx, e, "grouped: offsets copy");
    if (rows_cap == 0) return JAMHIP_OK;
    if (x_rows != nullptr && !derive) {   // the gathered rows, in CSR order, for the kernels below
        if ((e = ctx->gath.ensure((size_t) rows_cap * k * sizeof(float))) != hipSuccess)
            return hip_fail(ctx, e, "grouped gather: scratch alloc");
        if ((e = launch_moe_gather(a, lda, x_rows, off, E, rows_cap, rdiv, k, (float*) ctx->gath.p, k, ctx->stream)) !=
            hipSuccess)
            return hip_fail(ctx, e, "grouped gather: gather launch");
        a = (const float*) ctx->gath.p;
        lda = k;
    }
    const Groups g{off, poff8, map8, poff64, map64, m, static_cast<const float*>(bias_dev)};
    // activation scratch for the decode kernels (rows_cap rows; F1 then F2 reuse it in stream order)
    const int64_t nb = k / 32, n = rows_cap;
    const int64_t qb = align256(n * k), db = align256(n * nb * 4), sb = align256(n * (k / 16) * 4);
    auto actq = [&](ActQ* A) -> hipError_t {
        hipError_t r = ctx->act.ensure((size_t) (qb + db + 2 * sb));
        uint8_t* base = (uint8_t*) ctx->act.p;
        *A = ActQ{(int8_t*) base, (float*) (base + qb), (float*) (base + qb + db), (int*) (base + qb + db + sb)};
        return r;
    };
    // experts with 1..7 rows: jam's F1 decode path, a workgroup column per listed expert: one launch of the
    // one-token kernel over the experts with one row (decode: every expert), one of the seven-token kernel
    // over those with 2..7 (none can exist below rows_cap = 2)
    Groups g1 = g, g2 = g;
    if (derive) {
        g1.counts = g2.counts = (const int*) counts_dev;
        g1.n_experts = g2.n_experts = E;
        g1.rows_cap = g2.rows_cap = rows_cap;
        g1.rows = g2.rows = x_rows;   // null without a gather
        g1.rdiv = g2.rdiv = rdiv;
    } else {
        g1.small = small;
        g2.small = small + n1;
    }
    const bool fuse = gemv_grouped_fusable(k, a, lda);
    ActQ A{};
    if (!fuse) {
        if ((e = actq(&A)) != hipSuccess) return hip_fail(ctx, e, "grouped: activation scratch alloc");
        if ((e = launch_quant_f1(a, lda, rows_cap, k, (int8_t*) A.q, (float*) A.d, (float*) A.s, (int*) A.s16,
                                 ctx->stream)) != hipSuccess)
            return hip_fail(ctx, e, "grouped: quantize launch");
    }
    const float* af = fuse ? a : nullptr;
    const int laf = fuse ? lda : 0;
    if (derive) {   // both flavours in one launch (n1 one-token columns, then n2 seven-token columns)
        if ((e = launch_gemv_grouped(wt, 3, wv, A, af, laf, k, g1, n1, n2, c, ldc, ctx->stream)) != hipSuccess)
            return hip_fail(ctx, e, "grouped: gemv launch");
    } else if ((e = launch_gemv_grouped(wt, 0, wv, A, af, laf, k, g1, n1, cap8, c, ldc, ctx->stream)) != hipSuccess ||
               (n2 > 0 &&
                (e = launch_gemv_grouped(wt, 1, wv, A, af, laf, k, g2, n2, cap8, c, ldc, ctx->stream)) != hipSuccess))
        return hip_fail(ctx, e, "grouped: gemv launch");
    // fewer than 8 rows in all (decode-time MoE): no expert reaches the F2 bands, nothing more to launch
    if (rows_cap < 8) return JAMHIP_OK;
    // experts with >= 8 rows: jam's F2 bands (m % 16 == 0: no float-dot tail rows)
    if (wt == MXFP4 && ctx->mx_native && mma_path(wt, k, wv) && m % 32 == 0) {   // opt-in native MX
        MxAct X;
        if ((e = ctx->gact.ensure(mx_act_bytes_np(cap64 * 64, k))) != hipSuccess)
            return hip_fail(ctx, e, "grouped: mx activation scratch alloc");
        if ((e = launch_mx_prep_grouped(a, lda, k, ctx->mx_native, g, cap64, ctx->gact.p, &X, ctx->stream)) != hipSuccess ||
            (e = launch_mx_gemm_grouped(ctx->mx_native, wv, X, g, cap64, c, ldc, ctx->stream)) != hipSuccess)
            return hip_fail(ctx, e, "grouped: mx gemm launch");
    } else if (m % 32 == 0 && mma_exact(ctx, wt, k, wv)) {
        GemmAct G;
        if ((e = ctx->gact.ensure(gemm_act_bytes_np(wt, cap64 * 64, k))) != hipSuccess)
            return hip_fail(ctx, e, "grouped: gemm activation scratch alloc");
        if ((e = launch_gemm_prep_grouped(wt, a, lda, k, g, cap64, ctx->gact.p, &G, ctx->stream)) != hipSuccess ||
            (e = launch_gemm_mma_grouped(wt, wv, G, k, g, cap64, c, ldc, ctx->stream)) != hipSuccess)
            return hip_fail(ctx, e, "grouped: gemm launch");
    } else {
        ActQ A;
        if ((e = actq(&A)) != hipSuccess) return hip_fail(ctx, e, "grouped: activation scratch alloc");
        if ((e = launch_quant_f2(a, lda, rows_cap, k, (int8_t*) A.q, (float*) A.d, (float*) A.s, ctx->stream)) !=
                hipSuccess ||
            (e = launch_gemv_grouped(wt, 2, wv, A, nullptr, 0, k, g, E, cap8, c, ldc, ctx->stream)) != hipSuccess)
            return hip_fail(ctx, e, "grouped: band launch");
    }
    return JAMHIP_OK;
}

jamhip_status moe_route_impl(jamhip_ctx* ctx, const void* route_expert_dev, int seq, int topk, int n_experts,
                               void* counts_dev, void* offsets_dev, void* slot_route_dev, void* route_slot_dev) {
    if (!ctx) return JAMHIP_EINVAL;
    if (!route_expert_dev || !counts_dev || !offsets_dev || !slot_route_dev || !route_slot_dev)
        return fail(ctx, JAMHIP_EINVAL, "route: null pointer");
    if (seq <= 0 || topk <= 0 || n_experts <= 0) return fail(ctx, JAMHIP_EINVAL, "route: bad shape");
    if (n_experts > 1024) return fail(ctx, JAMHIP_EUNSUPPORTED, "route: at most 1024 experts");
    if ((int64_t) seq * topk > INT32_MAX) return fail(ctx, JAMHIP_EUNSUPPORTED, "route: too many routes");
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    int* scratch = nullptr;
    if (const size_t ni = moe_route_scratch_ints(seq * topk, n_experts)) {   // chunk counts of the spread kernel
        if (ctx->route.ensure(ni * sizeof(int)) == hipSuccess) scratch = (int*) ctx->route.p;
    }
    const hipError_t e = launch_moe_route((const int*) route_expert_dev, seq * topk, n_experts, (int*) counts_dev,
                                          (int*) offsets_dev, (int*) slot_route_dev, (int*) route_slot_dev, ctx->stream,
                                          scratch);
    return e == hipSuccess ? JAMHIP_OK : hip_fail(ctx, e, "route launch");
}

jamhip_status moe_gather_impl(jamhip_ctx* ctx, const void* x_dev, int ldx, const void* slot_route_dev,
                                const void* offsets_dev, int n_experts, int seq, int topk, int dim, void* g_dev,
                                int ldg) {
    if (!ctx) return JAMHIP_EINVAL;
    if (!x_dev || !slot_route_dev || !offsets_dev || !g_dev) return fail(ctx, JAMHIP_EINVAL, "gather: null pointer");
    if (seq <= 0 || topk <= 0 || dim <= 0 || n_experts <= 0 || ldx < dim || ldg < dim)
        return fail(ctx, JAMHIP_EINVAL, "gather: bad shape");
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    const hipError_t e = launch_moe_gather((const float*) x_dev, ldx, (const int*) slot_route_dev,
                                           (const int*) offsets_dev, n_experts, seq * topk, topk, dim, (float*) g_dev,
                                           ldg, ctx->stream);
    return e == hipSuccess ? JAMHIP_OK : hip_fail(ctx, e, "gather launch");
}

jamhip_status moe_combine_impl(jamhip_ctx* ctx, const void* y_dev, int ldy, const void* route_expert_dev,
                                 const void* route_prob_dev, const void* route_slot_dev, int seq, int topk,
                                 int n_experts, int dim, void* out_dev, int ldo) {
    if (!ctx) return JAMHIP_EINVAL;
    if (!y_dev || !route_expert_dev || !route_prob_dev || !route_slot_dev || !out_dev)
        return fail(ctx, JAMHIP_EINVAL, "combine: null pointer");
    if (seq <= 0 || topk <= 0 || dim <= 0 || n_experts <= 0 || ldy < dim || ldo < dim)
        return fail(ctx, JAMHIP_EINVAL, "combine: bad shape");
    if (topk > 16) return fail(ctx, JAMHIP_EUNSUPPORTED, "combine: topk above 16");
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    const hipError_t e = launch_moe_combine((const float*) y_dev, ldy, (const int*) route_expert_dev,
                                            (const float*) route_prob_dev, (const int*) route_slot_dev, seq, topk,
                                            n_experts, dim, (float*) out_dev, ldo, ctx->stream);
    return e == hipSuccess ? JAMHIP_OK : hip_fail(ctx, e, "combine launch");
}

jamhip_status moe_topk_impl(jamhip_ctx* ctx, void* sel, const void* wts, int rows, int E, int ld, int topk, int mode,
                            float wscale, const void* escale, void* route_expert, void* route_prob, void* counts) {
    if (!ctx) return JAMHIP_EINVAL;
    if (!sel || !route_expert || !route_prob) return fail(ctx, JAMHIP_EINVAL, "topk: null pointer");
    if (rows <= 0 || E <= 0 || topk <= 0 || ld < E) return fail(ctx, JAMHIP_EINVAL, "topk: bad shape");
    if (mode != JAMHIP_TOPK_RAW && mode != JAMHIP_TOPK_SOFTMAX && mode != JAMHIP_TOPK_NORMALIZE)
        return fail(ctx, JAMHIP_EINVAL, "topk: mode must be JAMHIP_TOPK_RAW, _SOFTMAX or _NORMALIZE");
    if (E > 1024) return fail(ctx, JAMHIP_EUNSUPPORTED, "topk: at most 1024 experts");
    if (topk > MOE_TOPK_MAX) return fail(ctx, JAMHIP_EUNSUPPORTED, "topk: topk above 16");
    if ((int64_t) rows * topk > INT32_MAX) return fail(ctx, JAMHIP_EUNSUPPORTED, "topk: too many routes");
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    const hipError_t e = launch_moe_topk((float*) sel, (const float*) wts, rows, E, ld, topk, mode, wscale,
                                         (const float*) escale, (int*) route_expert, (float*) route_prob, (int*) counts,
                                         ctx->stream);
    return e == hipSuccess ? JAMHIP_OK : hip_fail(ctx, e, "topk launch");
}

jamhip_status ctx_set_stream_impl(jamhip_ctx* ctx, void* stream) {
    if (!ctx) return JAMHIP_EINVAL;
    Busy guard(ctx);   // the stream is read by every call in flight on this context
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    ctx->stream = stream ? (hipStream_t) stream : ctx->own;
    return JAMHIP_OK;
}

jamhip_status ctx_synchronize_impl(jamhip_ctx* ctx) {
    if (!ctx) return JAMHIP_EINVAL;
    (void) hipSetDevice(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? JAMHIP_OK : hip_fail(ctx, e, "sync");
}

}  // namespace

namespace {

jamhip_ctx* create_ctx(int device, std::string* err) {
    if (env_true("JAM_HIP_DISABLE")) {
        *err = "disabled by JAM_HIP_DISABLE";
        return nullptr;
    }
    int dev = device;
    if (dev < 0 && hipGetDevice(&dev) != hipSuccess) {
        *err = "no HIP device";
        return nullptr;
    }
    hipDeviceProp_t prop;
    if (hipSetDevice(dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        *err = "hipSetDevice/hipGetDeviceProperties failed";
        return nullptr;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        *err = std::string("unsupported device architecture ") + prop.gcnArchName + " (need gfx950)";
        return nullptr;
    }
    (void) noalloc_scratch_init(dev);   // a failure is reported by jamhip_mm_device_noalloc itself
    gemm_tail_prime(dev);
    auto* ctx = new jamhip_ctx();
    ctx->device = dev;
    snprintf(ctx->arch, sizeof ctx->arch, "%s", prop.gcnArchName);
    if (hipStreamCreate(&ctx->own) != hipSuccess) {
        *err = "hipStreamCreate failed";
        delete ctx;
        return nullptr;
    }
    ctx->stream = ctx->own;
    if (const char* v = getenv("JAM_HIP_AUTOPIN")) ctx->autopin = atoi(v) > 0 ? atoi(v) : 0;
    if (const char* v = getenv("JAM_HIP_AUTOPIN_MAX_BYTES")) ctx->autopin_cap = atoll(v) > 0 ? atoll(v) : 0;
    if (const char* v = getenv("JAM_HIP_MX_NATIVE")) ctx->mx_native = atoi(v) == 1 || atoi(v) == 2 ? atoi(v) : 0;
    return ctx;
}

void destroy_ctx(jamhip_ctx* ctx) {
    (void) hipSetDevice(ctx->device);
    (void) hipStreamSynchronize(ctx->stream);
    for (Pin& p : ctx->pins) (void) hipFree(p.dev);
    ctx->pins.clear();
    ctx->act.release();
    ctx->a_host.release();
    ctx->c_host.release();
    ctx->gact.release();
    ctx->part.release();
    ctx->moe.release();
    ctx->route.release();
    ctx->gath.release();
    ctx->a_stage.release();
    ctx->c_stage.release();
    ctx->w_raw.release();
    ctx->w_stage.release();
    if (ctx->own) (void) hipStreamDestroy(ctx->own);
    delete ctx;
}

// The process-global context that ctx == NULL selects (jam.c:420-437, 765-768: created lazily on first use,
// on the current device; never destroyed implicitly, only by jamhip_global_destroy).
std::mutex g_global_mu;
jamhip_ctx* g_global = nullptr;

jamhip_ctx* global_ctx() {
    std::lock_guard<std::mutex> lk(g_global_mu);
    if (!g_global) {
        std::string err;
        g_global = create_ctx(-1, &err);
        if (!g_global) set_null_error("global context: " + err);
    }
    return g_global;
}

// Runs f on ctx, or on the process-global context when ctx is NULL; a failure there records its message for
// jamhip_last_error(NULL).
template <class F> jamhip_status on_ctx(jamhip_ctx* ctx, F&& f) {
    if (ctx) return f(ctx);
    jamhip_ctx* g = global_ctx();
    if (!g) return JAMHIP_EINVAL;
    const jamhip_status st = f(g);
    if (st != JAMHIP_OK) set_null_error(error_of(g));
    return st;
}

}  // namespace

extern "C" {

int jamhip_device_available(void) {
    if (env_true("JAM_HIP_DISABLE")) return 0;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    hipDeviceProp_t prop;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
    return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

jamhip_ctx* jamhip_ctx_create(int device) {
    std::string err;
    jamhip_ctx* ctx = create_ctx(device, &err);
    if (!ctx) set_null_error(err);
    return ctx;
}

void jamhip_ctx_destroy(jamhip_ctx* ctx) {
    if (ctx) destroy_ctx(ctx);
}

void jamhip_global_destroy(void) {
    std::lock_guard<std::mutex> lk(g_global_mu);
    if (g_global) destroy_ctx(g_global);
    g_global = nullptr;
}

const char* jamhip_ctx_arch(const jamhip_ctx* ctx) {
    if (!ctx) ctx = global_ctx();
    return ctx ? ctx->arch : "";
}

const char* jamhip_last_error(const jamhip_ctx* ctx) {
    if (!ctx) return g_null_error;
    thread_local std::string copy;   // a stable copy: another thread may overwrite the context's message
    copy = error_of(const_cast<jamhip_ctx*>(ctx));
    return copy.c_str();
}

jamhip_status jamhip_mm(jamhip_ctx* ctx, const void* w, int wt, int ldw, const void* a, int at, int lda, void* c,
                        int ct, int ldc, int m, int n, int k) {
    return on_ctx(ctx, [&](jamhip_ctx* x) { return mm_impl(x, w, wt, ldw, a, at, lda, c, ct, ldc, m, n, k); });
}

jamhip_status jamhip_mm_device(jamhip_ctx* ctx, const void* w, int wt, int ldw, const void* a_dev, int at, int lda,
                               void* c_dev, int ct, int ldc, int m, int n, int k) {
    return on_ctx(ctx, [&](jamhip_ctx* x) {
        return mm_device_impl(x, w, wt, ldw, a_dev, at, lda, c_dev, ct, ldc, m, n, k);
    });
}

jamhip_status jamhip_mm_device_noalloc(jamhip_ctx* ctx, const void* w, int wt, int ldw, const void* a_dev, int at,
                                       int lda, void* c_dev, int ct, int ldc, int m, int n, int k) {
    return on_ctx(ctx, [&](jamhip_ctx* x) {
        return mm_device_noalloc_impl(x, w, wt, ldw, a_dev, at, lda, c_dev, ct, ldc, m, n, k);
    });
}

jamhip_status jamhip_mm_device_ex(jamhip_ctx* ctx, const void* w, int wt, int ldw, const void* a_dev, int at, int lda,
                                  void* c_dev, int ct, int ldc, int m, int n, int k, const void* bias_dev,
                                  int accumulate) {
    return on_ctx(ctx, [&](jamhip_ctx* x) {
        return mm_device_ex_impl(x, w, wt, ldw, a_dev, at, lda, c_dev, ct, ldc, m, n, k, bias_dev, accumulate);
    });
}

jamhip_status jamhip_glu_device(jamhip_ctx* ctx, int act, void* gate_dev, int ldg, const void* up_dev, int ldu,
                                int rows, int cols) {
    return on_ctx(ctx, [&](jamhip_ctx* x) { return glu_device_impl(x, act, gate_dev, ldg, up_dev, ldu, rows, cols); });
}

jamhip_status jamhip_glu_device_vector(jamhip_ctx* ctx, int act, void* gate_dev, int ldg, const void* up_dev,
                                       int ldu, int rows, int cols, int lanes) {
    return on_ctx(ctx, [&](jamhip_ctx* x) {
        return glu_device_impl(x, act, gate_dev, ldg, up_dev, ldu, rows, cols, lanes);
    });
}

jamhip_status jamhip_read_floor(jamhip_ctx* ctx, const void* p_dev, int64_t bytes, void* sink_dev) {
    return on_ctx(ctx, [&](jamhip_ctx* x) { return read_floor_impl(x, p_dev, bytes, sink_dev); });
}

jamhip_status jamhip_ctx_set_autopin(jamhip_ctx* ctx, int sightings, int64_t max_bytes) {
    return on_ctx(ctx, [&](jamhip_ctx* x) { return set_autopin_impl(x, sightings, max_bytes); });
}

jamhip_status jamhip_ctx_set_mx_native(jamhip_ctx* ctx, int mode) {
    return on_ctx(ctx, [&](jamhip_ctx* x) { return set_mx_native_impl(x, mode); });
}

jamhip_status jamhip_ctx_autopin_stats(const jamhip_ctx* ctx, int64_t* out4) {
    jamhip_ctx* x = ctx ? const_cast<jamhip_ctx*>(ctx) : global_ctx();
    if (!x || !out4) return JAMHIP_EINVAL;
    std::lock_guard<std::mutex> lk(x->pin_mu);
    for (int i = 0; i < 4; i++) out4[i] = x->ap_stats[i];
    return JAMHIP_OK;
}

jamhip_status jamhip_weight_pin(jamhip_ctx* ctx, const void* w, int wt, int ldw, int m) {
    return on_ctx(ctx, [&](jamhip_ctx* x) { return weight_pin_impl(x, w, wt, ldw, m); });
}

jamhip_status jamhip_weight_evict(jamhip_ctx* ctx, const void* w) {
    return on_ctx(ctx, [&](jamhip_ctx* x) { return weight_evict_impl(x, w); });
}

int64_t jamhip_weight_bytes(const jamhip_ctx* ctx) {
    if (!ctx) {
        std::lock_guard<std::mutex> lk(g_global_mu);
        ctx = g_global;
        if (!ctx) return 0;
    }
    std::lock_guard<std::mutex> lk(ctx->pin_mu);
    return ctx->pinned_bytes;
}

jamhip_status jamhip_quantize_device(jamhip_ctx* ctx, int flavour, const void* a_dev, int lda, int n, int k,
                                     void* q_dev, void* d_dev, void* s_dev) {
    return on_ctx(ctx, [&](jamhip_ctx* x) {
        return quantize_device_impl(x, flavour, a_dev, lda, n, k, q_dev, d_dev, s_dev);
    });
}

jamhip_status jamhip_mm_grouped(jamhip_ctx* ctx, const void* w, int wt, int ldw, int m, int n_experts,
                                const void* counts_dev, const void* a_dev, int at, int lda, void* c_dev, int ct,
                                int ldc, int k, int rows_cap, void* offsets_dev) {
    return on_ctx(ctx, [&](jamhip_ctx* x) {
        return mm_grouped_ex_impl(x, w, wt, ldw, m, n_experts, counts_dev, a_dev, at, lda, c_dev, ct, ldc, k, rows_cap,
                                  offsets_dev, nullptr);
    });
}

jamhip_status jamhip_mm_grouped_ex(jamhip_ctx* ctx, const void* w, int wt, int ldw, int m, int n_experts,
                                   const void* counts_dev, const void* a_dev, int at, int lda, void* c_dev, int ct,
                                   int ldc, int k, int rows_cap, void* offsets_dev, const void* bias_dev) {
    return on_ctx(ctx, [&](jamhip_ctx* x) {
        return mm_grouped_ex_impl(x, w, wt, ldw, m, n_experts, counts_dev, a_dev, at, lda, c_dev, ct, ldc, k, rows_cap,
                                  offsets_dev, bias_dev);
    });
}

jamhip_status jamhip_mm_grouped_gather(jamhip_ctx* ctx, const void* w, int wt, int ldw, int m, int n_experts,
                                       const void* counts_dev, const void* x_dev, int at, int ldx,
                                       const void* slot_route_dev, int topk, void* c_dev, int ct, int ldc, int k,
                                       int rows_cap, void* offsets_dev, const void* bias_dev) {
    return on_ctx(ctx, [&](jamhip_ctx* x) {
        if (!slot_route_dev) return fail(x, JAMHIP_EINVAL, "grouped gather: null slot_route");
        return mm_grouped_ex_impl(x, w, wt, ldw, m, n_experts, counts_dev, x_dev, at, ldx, c_dev, ct, ldc, k, rows_cap,
                                  offsets_dev, bias_dev, static_cast<const int*>(slot_route_dev), topk);
    });
}

jamhip_status jamhip_moe_route(jamhip_ctx* ctx, const void* route_expert_dev, int seq, int topk, int n_experts,
                               void* counts_dev, void* offsets_dev, void* slot_route_dev, void* route_slot_dev) {
    return on_ctx(ctx, [&](jamhip_ctx* x) {
        return moe_route_impl(x, route_expert_dev, seq, topk, n_experts, counts_dev, offsets_dev, slot_route_dev,
                              route_slot_dev);
    });
}

jamhip_status jamhip_moe_gather(jamhip_ctx* ctx, const void* x_dev, int ldx, const void* slot_route_dev,
                                const void* offsets_dev, int n_experts, int seq, int topk, int dim, void* g_dev,
                                int ldg) {
    return on_ctx(ctx, [&](jamhip_ctx* x) {
        return moe_gather_impl(x, x_dev, ldx, slot_route_dev, offsets_dev, n_experts, seq, topk, dim, g_dev, ldg);
    });
}

jamhip_status jamhip_moe_combine(jamhip_ctx* ctx, const void* y_dev, int ldy, const void* route_expert_dev,
                                 const void* route_prob_dev, const void* route_slot_dev, int seq, int topk,
                                 int n_experts, int dim, void* out_dev, int ldo) {
    return on_ctx(ctx, [&](jamhip_ctx* x) {
        return moe_combine_impl(x, y_dev, ldy, route_expert_dev, route_prob_dev, route_slot_dev, seq, topk, n_experts,
                                dim, out_dev, ldo);
    });
}

jamhip_status jamhip_moe_select_topk(jamhip_ctx* ctx, void* selection_dev, const void* weights_dev, int rows,
                                     int n_experts, int ld, int topk, int mode, float weights_scale,
                                     const void* expert_scale_dev, void* route_expert_dev, void* route_prob_dev,
                                     void* counts_dev) {
    return on_ctx(ctx, [&](jamhip_ctx* x) {
        return moe_topk_impl(x, selection_dev, weights_dev, rows, n_experts, ld, topk, mode, weights_scale,
                             expert_scale_dev, route_expert_dev, route_prob_dev, counts_dev);
    });
}

jamhip_status jamhip_ctx_set_stream(jamhip_ctx* ctx, void* stream) {
    return on_ctx(ctx, [&](jamhip_ctx* x) { return ctx_set_stream_impl(x, stream); });
}

void* jamhip_ctx_stream(const jamhip_ctx* ctx) {
    if (!ctx) ctx = global_ctx();
    return ctx ? (void*) ctx->stream : nullptr;
}

jamhip_status jamhip_ctx_synchronize(jamhip_ctx* ctx) {
    return on_ctx(ctx, [&](jamhip_ctx* x) { return ctx_synchronize_impl(x); });
}

// ------------------------------------------------------------------ GGUF weight registry
jamhip_gguf* jamhip_gguf_open(const char* path, char* err, size_t err_cap) {
    std::string e;
    GgufFile* f = gguf_read(path, &e);
    if (err && err_cap) snprintf(err, err_cap, "%s", f ? "" : e.c_str());
    return f ? new jamhip_gguf{f} : nullptr;
}

void jamhip_gguf_close(jamhip_gguf* g) {
    if (!g) return;
    gguf_free(g->f);
    delete g;
}

int64_t jamhip_gguf_tensor_count(const jamhip_gguf* g) { return g ? (int64_t) g->f->tensors.size() : -1; }
int64_t jamhip_gguf_data_offset(const jamhip_gguf* g) { return g ? g->f->data_offset : -1; }
int     jamhip_gguf_alignment(const jamhip_gguf* g) { return g ? (int) g->f->alignment : -1; }

jamhip_status jamhip_gguf_tensor_at(const jamhip_gguf* g, int64_t i, jamhip_gguf_tensor* out) {
    if (!g || !out || i < 0 || i >= (int64_t) g->f->tensors.size()) return JAMHIP_EINVAL;
    const GgufTensor& t = g->f->tensors[(size_t) i];
    out->name = t.name.c_str();
    out->type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; d++) out->dims[d] = t.dims[d];
    out->offset = t.offset;
    out->bytes = t.bytes;
    out->data = g->f->data ? g->f->data + t.offset : nullptr;
    return JAMHIP_OK;
}

int64_t jamhip_gguf_find(const jamhip_gguf* g, const char* name) {
    if (!g || !name) return -1;
    for (size_t i = 0; i < g->f->tensors.size(); i++)
        if (g->f->tensors[i].name == name) return (int64_t) i;
    return -1;
}

namespace {
// A tensor the registry pins: a jam weight dtype with data; ldw = dims[0], rows = the other dims' product.
// A tensor whose row extent dims[0] is not a whole number of blocks (dims[0] below one block included) is
// taken here too, with rows = 0, so that registry_runs reports it instead of dividing by a zero row size.
bool registry_shape(const GgufTensor& t, int* ldw, int64_t* rows) {
    if (!supported_w(t.type) || t.bytes == 0 || t.n_dims < 2) return false;   // 1-D: norms, biases
    *ldw = (int) t.dims[0];
    *rows = t.dims[0] % block_elems(t.type) ? 0 : t.bytes / row_bytes(t.type, t.dims[0]);
    return true;
}

// The registry's device ranges for a file: its jam tensors in offset order, adjacent tensors of one dtype
// and row length (back to back in the file, every member starting on a 32-row tile) merged into one run,
// so a call may span them (q|k|v, gate|up) while each tensor still resolves inside the run.
struct Run {
    int64_t offset, bytes, rows, members;
    int type, ldw;
};

jamhip_status registry_runs(jamhip_ctx* ctx, const GgufFile& f, std::vector<Run>* runs) {
    std::vector<const GgufTensor*> ts;
    for (const GgufTensor& t : f.tensors) {
        int ldw;
        int64_t rows;
        if (!registry_shape(t, &ldw, &rows)) continue;
        if (t.dims[0] % block_elems(t.type))
            return fail(ctx, JAMHIP_EUNSUPPORTED, "gguf pin: tensor " + t.name + ": row extent is not a whole number of blocks");
        if (t.dims[0] > (1 << 30) || rows > INT32_MAX)
            return fail(ctx, JAMHIP_EUNSUPPORTED, "gguf pin: tensor " + t.name + " exceeds the kernels' 32-bit extents");
        ts.push_back(&t);
    }
    std::sort(ts.begin(), ts.end(), [](const GgufTensor* x, const GgufTensor* y) { return x->offset < y->offset; });
    runs->clear();
    for (const GgufTensor* t : ts) {
        const int64_t rows = t->bytes / row_bytes(t->type, t->dims[0]);   // dims[0] is a block multiple here
        Run* r = runs->empty() ? nullptr : &runs->back();
        if (r && r->type == t->type && r->ldw == (int) t->dims[0] && r->offset + r->bytes == t->offset &&
            r->rows % 32 == 0 && r->rows + rows <= INT32_MAX) {
            r->bytes += t->bytes;
            r->rows += rows;
            r->members++;
        } else {
            runs->push_back(Run{t->offset, t->bytes, rows, 1, t->type, (int) t->dims[0]});
        }
    }
    return JAMHIP_OK;
}
}  // namespace

}  // extern "C"

namespace {
jamhip_status gguf_pin_impl(jamhip_ctx* ctx, const jamhip_gguf* g, const void* data_base, int64_t* n_pinned,
                            int64_t* bytes_pinned);
jamhip_status gguf_evict_impl(jamhip_ctx* ctx, const jamhip_gguf* g, const void* data_base, int64_t* n_evicted);
}  // namespace

extern "C" {

jamhip_status jamhip_gguf_pin(jamhip_ctx* ctx, const jamhip_gguf* g, const void* data_base, int64_t* n_pinned,
                              int64_t* bytes_pinned) {
    if (n_pinned) *n_pinned = 0;
    if (bytes_pinned) *bytes_pinned = 0;
    return on_ctx(ctx, [&](jamhip_ctx* x) { return gguf_pin_impl(x, g, data_base, n_pinned, bytes_pinned); });
}

jamhip_status jamhip_gguf_evict(jamhip_ctx* ctx, const jamhip_gguf* g, const void* data_base, int64_t* n_evicted) {
    if (n_evicted) *n_evicted = 0;
    return on_ctx(ctx, [&](jamhip_ctx* x) { return gguf_evict_impl(x, g, data_base, n_evicted); });
}

}  // extern "C"

namespace {

jamhip_status gguf_pin_impl(jamhip_ctx* ctx, const jamhip_gguf* g, const void* data_base, int64_t* n_pinned,
                            int64_t* bytes_pinned) {
    if (!g) return fail(ctx, JAMHIP_EINVAL, "gguf pin: null handle");
    const uint8_t* base = data_base ? static_cast<const uint8_t*>(data_base) : g->f->data;
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    std::vector<Run> runs;
    jamhip_status st = registry_runs(ctx, *g->f, &runs);   // every tensor checked before anything is pinned
    if (st != JAMHIP_OK) return st;
    for (const Run& r : runs) {
        if ((st = pin_range(ctx, base + r.offset, r.type, r.ldw, r.rows, true, true)) != JAMHIP_OK) {
            fail(ctx, st, "gguf pin: run at data offset " + std::to_string(r.offset) + ": " + error_of(ctx));
            break;
        }
        if (n_pinned) *n_pinned += r.members;
        if (bytes_pinned) *bytes_pinned += r.bytes;
    }
    ctx->w_raw.release();
    return st;
}

jamhip_status gguf_evict_impl(jamhip_ctx* ctx, const jamhip_gguf* g, const void* data_base, int64_t* n_evicted) {
    if (!g) return fail(ctx, JAMHIP_EINVAL, "gguf evict: null handle");
    const uint8_t* base = data_base ? static_cast<const uint8_t*>(data_base) : g->f->data;
    Busy guard(ctx);
    if (!guard.ok) return fail(ctx, JAMHIP_EBUSY, "context busy");
    (void) hipSetDevice(ctx->device);
    std::vector<Run> runs;
    const jamhip_status st = registry_runs(ctx, *g->f, &runs);
    if (st != JAMHIP_OK) return st;
    for (const Run& r : runs)
        if (evict_at(ctx, reinterpret_cast<uintptr_t>(base + r.offset)) && n_evicted) *n_evicted += r.members;
    return JAMHIP_OK;
}

}  // namespace
