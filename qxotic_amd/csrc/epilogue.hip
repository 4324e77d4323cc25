// Gated activations that jinfer runs between the FFN's matmuls, in place on the gate rows:
//   act 1  SwiGLU            gate = silu(gate) · up             (Activations.siluMultiply, Llama.java:428-436)
//   act 2  gpt-oss clamped   gate = quickgelu(min(gate, 7)) · (clamp(up, ±7) + 1)
//                                                                (Activations.clampedSwigluMultiply, GptOss.java:306-313)
// Each has two forms: the reference's full-scalar form (jinfer/jinfer-kernels/src/main/java/com/qxotic/jinfer/
// kernels/Ops.java:578-583 and Activations.java:183-187: the arithmetic in double, rounded to f32 where the
// Java code rounds), and the Vector API form jinfer runs by default (lanes > 0, below). The bias adds that precede them in gpt-oss run in the producing matmul's epilogue (Epi).
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

// jinfer's default (Vector API) arithmetic: njuffa's minimax rational tanh (Ops.tanhApprox / tanhVec,
// Ops.java:620-663) in f32 with fused multiply-adds, every operation rounded where the Java code rounds
// (explicit _rn intrinsics: nothing is contracted or reassociated). Math.max / Math.min return NaN if
// either operand is NaN.
__device__ inline float jmax(float a, float b) { return (isnan(a) || isnan(b)) ? __builtin_nanf("") : fmaxf(a, b); }
__device__ inline float jmin(float a, float b) { return (isnan(a) || isnan(b)) ? __builtin_nanf("") : fminf(a, b); }

__device__ inline float tanh_approx(float x) {
    const float y = jmax(-5.76110792f, jmin(5.76110792f, x));
    const float y2 = __fmul_rn(y, y);
    const float num = __fmul_rn(__fmaf_rn(__fmaf_rn(-1.60153955e-4f, y2, -9.34448242e-1f), y2, -2.19176636e+1f), y2);
    const float den = __fmaf_rn(__fadd_rn(y2, 29.0915985f), y2, 65.7667847f);
    return __fmaf_rn(__fdiv_rn(num, den), y, y);
}

// The SwiGLU vector body (Ops.java:551-563): g * (tanh(g/2)*0.5 + 0.5) * u.
__device__ inline float silu_mul_vec(float g, float u) {
    const float t = tanh_approx(__fmul_rn(g, 0.5f));
    return __fmul_rn(__fmul_rn(g, __fadd_rn(__fmul_rn(t, 0.5f), 0.5f)), u);
}

// gpt-oss's vector body and its scalar twin clampedSwigluApprox (Activations.java:189-224):
// x*0.5 * (1 + tanh(0.851x)) * (y + 1), x = min(g, 7), y = clamp(u, -7, 7).
__device__ inline float clamped_swiglu_vec(float g, float u) {
    const float x = jmin(g, 7.0f);
    const float y = jmin(jmax(u, -7.0f), 7.0f);
    const float t = tanh_approx(__fmul_rn(x, 0.851f));
    return __fmul_rn(__fmul_rn(__fmul_rn(x, 0.5f), __fadd_rn(1.0f, t)), __fadd_rn(y, 1.0f));
}

// bound = the row's vector-loop bound (cols - cols % lanes, F_SPECIES.loopBound); elements past it take the
// loop's scalar tail: SwiGLU's double formula, gpt-oss's clampedSwigluApprox. bound = 0: the full-scalar forms.
template <int ACT>
__global__ void __launch_bounds__(256) glu_kernel(float* __restrict__ gate, int ldg, const float* __restrict__ up,
                                                  int ldu, int rows, int cols, int bound) {
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        float* g = gate + r * ldg;
        const float* u = up + r * ldu;
        for (int i = blockIdx.x * 256 + threadIdx.x; i < cols; i += gridDim.x * 256) {
            float v;
            if (ACT == 1) v = i < bound ? silu_mul_vec(g[i], u[i]) : silu_mul(g[i], u[i]);
            else if (ACT == 2) v = clamped_swiglu(g[i], u[i]);
            else v = clamped_swiglu_vec(g[i], u[i]);
            g[i] = v;
        }
    }
}

hipError_t launch_glu(int act, float* gate, int ldg, const float* up, int ldu, int rows, int cols, hipStream_t st,
                      int lanes) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    if (lanes < 0) return hipErrorInvalidValue;
    const dim3 grid((unsigned) ((cols + 255) / 256 < 64 ? (cols + 255) / 256 : 64), (unsigned) (rows < 65535 ? rows : 65535));
    const int bound = lanes > 0 ? cols - cols % lanes : 0;
    if (act == 1) glu_kernel<1><<<grid, 256, 0, st>>>(gate, ldg, up, ldu, rows, cols, bound);
    else if (act == 2 && lanes == 0) glu_kernel<2><<<grid, 256, 0, st>>>(gate, ldg, up, ldu, rows, cols, 0);
    else if (act == 2) glu_kernel<3><<<grid, 256, 0, st>>>(gate, ldg, up, ldu, rows, cols, bound);   // body = tail
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace jamhip
