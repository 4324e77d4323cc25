// int8-MFMA prefill GEMM (F2 activations). Filled in per dtype; unsupported dtypes fall back to the
// skinny weight-streaming kernel.
#include "common.h"
#include "launch.h"

namespace jamhip {

hipError_t launch_gemm(int dt, const WeightView& w, const ActQ& A, int k, int m, int n, float* c, int ldc,
                       hipStream_t st) {
    (void) dt; (void) w; (void) A; (void) k; (void) m; (void) n; (void) c; (void) ldc; (void) st;
    return hipErrorNotSupported;
}

}  // namespace jamhip
