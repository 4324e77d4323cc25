// Gated activations that jinfer runs between the FFN's matmuls, in place on the gate rows:
//   act 1  SwiGLU            gate = silu(gate) · up             (Activations.siluMultiply, Llama.java:428-436)
//   act 2  gpt-oss clamped   gate = quickgelu(min(gate, 7)) · (clamp(up, ±7) + 1)
//                                                                (Activations.clampedSwigluMultiply, GptOss.java:306-313)
// Each follows the reference's full-scalar form (jinfer/jinfer-kernels/src/main/java/com/qxotic/jinfer/
// kernels/Ops.java:578-583 and Activations.java:183-187): the arithmetic in double, rounded to f32 where the
// Java code rounds. The bias adds that precede them in gpt-oss run in the producing matmul's epilogue (Epi).
// HBM-bound: 12 bytes per element (gate read + written, up read).
#include "common.h"
#include "launch.h"

namespace jamhip {

__device__ inline float silu_mul(float g, float u) {   // (float) (g / (1.0 + Math.exp(-g)) * u), all double
    return (float) ((double) g / (1.0 + exp(-(double) g)) * (double) u);
}

__device__ inline float clamped_swiglu(float g, float u) {
    const float x = g > 7.0f ? 7.0f : g;                          // Math.min / Math.clamp: NaN stays NaN
    const float y = u < -7.0f ? -7.0f : u > 7.0f ? 7.0f : u;
    const double t = (double) (1.702f * -x);                      // float product, as 1.702f * -x in Java
    return (float) ((double) x / (1.0 + exp(t)) * ((double) y + 1.0));
}

template <int ACT>
__global__ void __launch_bounds__(256) glu_kernel(float* __restrict__ gate, int ldg, const float* __restrict__ up,
                                                  int ldu, int rows, int cols) {
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        float* g = gate + r * ldg;
        const float* u = up + r * ldu;
        for (int i = blockIdx.x * 256 + threadIdx.x; i < cols; i += gridDim.x * 256)
            g[i] = ACT == 1 ? silu_mul(g[i], u[i]) : clamped_swiglu(g[i], u[i]);
    }
}

hipError_t launch_glu(int act, float* gate, int ldg, const float* up, int ldu, int rows, int cols, hipStream_t st) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    const dim3 grid((unsigned) ((cols + 255) / 256 < 64 ? (cols + 255) / 256 : 64), (unsigned) (rows < 65535 ? rows : 65535));
    if (act == 1) glu_kernel<1><<<grid, 256, 0, st>>>(gate, ldg, up, ldu, rows, cols);
    else if (act == 2) glu_kernel<2><<<grid, 256, 0, st>>>(gate, ldg, up, ldu, rows, cols);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace jamhip
