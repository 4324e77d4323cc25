// Dispatch of the decode / few-token kernels (gemv_impl.h) by weight type; each type's kernels are
// instantiated in gemv_<type>.hip.
#include "gemv_impl.h"

namespace jamhip {

extern template hipError_t gemv_dt<Q4_K>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m, int n, float* c, int ldc, hipStream_t st, float* part, const Epi& ep);
extern template hipError_t gemv_grouped_dt<Q4_K>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, const Groups& g, int E, int cap8, float* c, int ldc, hipStream_t st);
extern template hipError_t rows_float_dt<Q4_K>(const WeightView& w, const float* a, int lda, int k, int r0, int rows, int n, float* c, int ldc, hipStream_t st, const Epi& ep);
extern template hipError_t gemv_dt<Q6_K>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m, int n, float* c, int ldc, hipStream_t st, float* part, const Epi& ep);
extern template hipError_t gemv_grouped_dt<Q6_K>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, const Groups& g, int E, int cap8, float* c, int ldc, hipStream_t st);
extern template hipError_t rows_float_dt<Q6_K>(const WeightView& w, const float* a, int lda, int k, int r0, int rows, int n, float* c, int ldc, hipStream_t st, const Epi& ep);
extern template hipError_t gemv_dt<Q8_0>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m, int n, float* c, int ldc, hipStream_t st, float* part, const Epi& ep);
extern template hipError_t gemv_grouped_dt<Q8_0>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, const Groups& g, int E, int cap8, float* c, int ldc, hipStream_t st);
extern template hipError_t rows_float_dt<Q8_0>(const WeightView& w, const float* a, int lda, int k, int r0, int rows, int n, float* c, int ldc, hipStream_t st, const Epi& ep);
extern template hipError_t gemv_dt<Q4_0>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m, int n, float* c, int ldc, hipStream_t st, float* part, const Epi& ep);
extern template hipError_t gemv_grouped_dt<Q4_0>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, const Groups& g, int E, int cap8, float* c, int ldc, hipStream_t st);
extern template hipError_t rows_float_dt<Q4_0>(const WeightView& w, const float* a, int lda, int k, int r0, int rows, int n, float* c, int ldc, hipStream_t st, const Epi& ep);
extern template hipError_t gemv_dt<MXFP4>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m, int n, float* c, int ldc, hipStream_t st, float* part, const Epi& ep);
extern template hipError_t gemv_grouped_dt<MXFP4>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, const Groups& g, int E, int cap8, float* c, int ldc, hipStream_t st);
extern template hipError_t rows_float_dt<MXFP4>(const WeightView& w, const float* a, int lda, int k, int r0, int rows, int n, float* c, int ldc, hipStream_t st, const Epi& ep);
extern template hipError_t gemv_dt<Q5_K>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m, int n, float* c, int ldc, hipStream_t st, float* part, const Epi& ep);
extern template hipError_t gemv_grouped_dt<Q5_K>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, const Groups& g, int E, int cap8, float* c, int ldc, hipStream_t st);
extern template hipError_t rows_float_dt<Q5_K>(const WeightView& w, const float* a, int lda, int k, int r0, int rows, int n, float* c, int ldc, hipStream_t st, const Epi& ep);
extern template hipError_t gemv_dt<NVFP4>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m, int n, float* c, int ldc, hipStream_t st, float* part, const Epi& ep);
extern template hipError_t gemv_grouped_dt<NVFP4>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, const Groups& g, int E, int cap8, float* c, int ldc, hipStream_t st);
extern template hipError_t rows_float_dt<NVFP4>(const WeightView& w, const float* a, int lda, int k, int r0, int rows, int n, float* c, int ldc, hipStream_t st, const Epi& ep);
extern template hipError_t gemv_dt<Q1_0>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m, int n, float* c, int ldc, hipStream_t st, float* part, const Epi& ep);
extern template hipError_t gemv_grouped_dt<Q1_0>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, const Groups& g, int E, int cap8, float* c, int ldc, hipStream_t st);
extern template hipError_t rows_float_dt<Q1_0>(const WeightView& w, const float* a, int lda, int k, int r0, int rows, int n, float* c, int ldc, hipStream_t st, const Epi& ep);

hipError_t launch_gemv_grouped(int dt, int flavour, const WeightView& w, const ActQ& A, const float* a, int lda,
                               int k, const Groups& g, int E, int cap8, float* c, int ldc, hipStream_t st) {
    if (flavour == 2 && cap8 <= 0) return hipSuccess;
    switch (dt) {
    case Q4_K: return gemv_grouped_dt<Q4_K>(flavour, w, A, a, lda, k, g, E, cap8, c, ldc, st);
    case Q6_K: return gemv_grouped_dt<Q6_K>(flavour, w, A, a, lda, k, g, E, cap8, c, ldc, st);
    case Q8_0: return gemv_grouped_dt<Q8_0>(flavour, w, A, a, lda, k, g, E, cap8, c, ldc, st);
    case Q4_0: return gemv_grouped_dt<Q4_0>(flavour, w, A, a, lda, k, g, E, cap8, c, ldc, st);
    case MXFP4: return gemv_grouped_dt<MXFP4>(flavour, w, A, a, lda, k, g, E, cap8, c, ldc, st);
    case Q5_K: return gemv_grouped_dt<Q5_K>(flavour, w, A, a, lda, k, g, E, cap8, c, ldc, st);
    case NVFP4: return gemv_grouped_dt<NVFP4>(flavour, w, A, a, lda, k, g, E, cap8, c, ldc, st);
    case Q1_0: return gemv_grouped_dt<Q1_0>(flavour, w, A, a, lda, k, g, E, cap8, c, ldc, st);
    default: return hipErrorInvalidValue;
    }
}

// The fused F1 prologue quantizes one K slice of n tokens per workgroup into LDS (at most 4 half-blocks per
// thread); ks = the slice length (gemv_slice(k, n) for a launch_gemv call, k for the grouped kernels).
static bool fusable_slice(int n, int ks, const float* a, int lda) {
    return n < 8 && fuse_lds(n, ks) <= (size_t) kFuseMaxBytes && fuse_hp(n, ks) <= 4 &&
           (reinterpret_cast<uintptr_t>(a) & 15) == 0 && (lda & 3) == 0;
}
bool gemv_fusable(int n, int k, const float* a, int lda) { return fusable_slice(n, gemv_slice(k, n), a, lda); }
bool gemv_grouped_fusable(int k, const float* a, int lda) { return fusable_slice(7, k, a, lda); }

size_t gemv_split_floats(int k, int m, int n) {
    const int ks = gemv_slice(k, n);
    return ks < k ? (size_t) ((k + ks - 1) / ks) * n * m : 0;
}

hipError_t launch_gemv(int dt, int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m,
                       int n, float* c, int ldc, hipStream_t st, float* part, const Epi& ep) {
    switch (dt) {
    case Q4_K: return gemv_dt<Q4_K>(flavour, w, A, a, lda, k, m, n, c, ldc, st, part, ep);
    case Q6_K: return gemv_dt<Q6_K>(flavour, w, A, a, lda, k, m, n, c, ldc, st, part, ep);
    case Q8_0: return gemv_dt<Q8_0>(flavour, w, A, a, lda, k, m, n, c, ldc, st, part, ep);
    case Q4_0: return gemv_dt<Q4_0>(flavour, w, A, a, lda, k, m, n, c, ldc, st, part, ep);
    case MXFP4: return gemv_dt<MXFP4>(flavour, w, A, a, lda, k, m, n, c, ldc, st, part, ep);
    case Q5_K: return gemv_dt<Q5_K>(flavour, w, A, a, lda, k, m, n, c, ldc, st, part, ep);
    case NVFP4: return gemv_dt<NVFP4>(flavour, w, A, a, lda, k, m, n, c, ldc, st, part, ep);
    case Q1_0: return gemv_dt<Q1_0>(flavour, w, A, a, lda, k, m, n, c, ldc, st, part, ep);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_rows_float(int dt, const WeightView& w, const float* a, int lda, int k, int r0, int rows, int n,
                             float* c, int ldc, hipStream_t st, const Epi& ep) {
    if (rows <= 0) return hipSuccess;
    switch (dt) {
    case Q4_K: return rows_float_dt<Q4_K>(w, a, lda, k, r0, rows, n, c, ldc, st, ep);
    case Q6_K: return rows_float_dt<Q6_K>(w, a, lda, k, r0, rows, n, c, ldc, st, ep);
    case Q8_0: return rows_float_dt<Q8_0>(w, a, lda, k, r0, rows, n, c, ldc, st, ep);
    case Q4_0: return rows_float_dt<Q4_0>(w, a, lda, k, r0, rows, n, c, ldc, st, ep);
    case MXFP4: return rows_float_dt<MXFP4>(w, a, lda, k, r0, rows, n, c, ldc, st, ep);
    case Q5_K: return rows_float_dt<Q5_K>(w, a, lda, k, r0, rows, n, c, ldc, st, ep);
    case NVFP4: return rows_float_dt<NVFP4>(w, a, lda, k, r0, rows, n, c, ldc, st, ep);
    case Q1_0: return rows_float_dt<Q1_0>(w, a, lda, k, r0, rows, n, c, ldc, st, ep);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace jamhip
