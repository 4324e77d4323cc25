// The decode / few-token kernels for NVFP4 weights (gemv_impl.h), instantiated in a translation unit of
// their own so the weight types compile in parallel.
#include "gemv_impl.h"

namespace jamhip {
template hipError_t gemv_dt<NVFP4>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, int m, int n, float* c, int ldc, hipStream_t st, float* part, const Epi& ep);
template hipError_t gemv_grouped_dt<NVFP4>(int flavour, const WeightView& w, const ActQ& A, const float* a, int lda, int k, const Groups& g, int E, int cap8, float* c, int ldc, hipStream_t st);
template hipError_t rows_float_dt<NVFP4>(const WeightView& w, const float* a, int lda, int k, int r0, int rows, int n, float* c, int ldc, hipStream_t st, const Epi& ep);
}  // namespace jamhip
