// Activation quantizer kernels (jam's F1 and F2, bit-exact; lane math in quant.h) and the one-time
// weight repack into the device layout.
#include "common.h"
#include "launch.h"
#include "quant.h"

namespace jamhip {

// One lane per activation element; a 32-lane half-wave owns one 32-element block (quant.h).
// k % 32 == 0 is checked by the caller, so whole blocks retire together at the row end.
__global__ void __launch_bounds__(256) quant_f1_kernel(const float* __restrict__ a, int lda, int k,
                                                       int8_t* __restrict__ q, float* __restrict__ d,
                                                       float* __restrict__ asum, int* __restrict__ s16) {
    const int j = blockIdx.y;
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= k) return;
    float db;
    int h16, h32;
    const int v = f1_lane(a[(int64_t) j * lda + e], db, h16, h32);
    q[(int64_t) j * k + e] = (int8_t) v;
    if ((e & 15) == 0) s16[(int64_t) j * (k >> 4) + (e >> 4)] = h16;
    if ((e & 31) == 0) {
        d[(int64_t) j * (k >> 5) + (e >> 5)] = db;
        asum[(int64_t) j * (k >> 5) + (e >> 5)] = (float) h32;
    }
}

__global__ void __launch_bounds__(256) quant_f2_kernel(const float* __restrict__ a, int lda, int k,
                                                       int8_t* __restrict__ q, float* __restrict__ d,
                                                       float* __restrict__ xs) {
    const int j = blockIdx.y;
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= k) return;
    float db, s;
    const int v = f2_lane(a[(int64_t) j * lda + e], db, s);
    q[(int64_t) j * k + e] = (int8_t) v;
    if ((e & 15) == 0) xs[(int64_t) j * (k >> 4) + (e >> 4)] = s;
    if ((e & 31) == 0) d[(int64_t) j * (k >> 5) + (e >> 5)] = db;
}

// Weight repack: raw GGUF rows (stride raw_stride bytes, rb blocks) -> the two-plane device layout
// described in common.h. One thread per block; runs once per pinned tensor.
template <int DT>
__global__ void __launch_bounds__(256) repack_kernel(const uint8_t* __restrict__ raw, int64_t raw_stride,
                                                     int64_t rows, int64_t rb, uint8_t* __restrict__ qs,
                                                     uint8_t* __restrict__ sc) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * rb) return;
    const int64_t r = i / rb, b = i - r * rb;
    const uint8_t* src = raw + r * raw_stride + b * block_bytes(DT);
    uint8_t* dq = qs + i * qs_bytes(DT);
    uint8_t* ds = sc + i * sc_bytes(DT);
    if constexpr (DT == Q8_0 || DT == Q4_0) {          // d fp16 @0, payload @2
        ds[0] = src[0];
        ds[1] = src[1];
        for (int t = 0; t < qs_bytes(DT); t++) dq[t] = src[2 + t];
    } else if constexpr (DT == MXFP4) {                // e8m0 @0, nibbles @1
        ds[0] = src[0];
        for (int t = 0; t < 16; t++) dq[t] = src[1 + t];
    } else if constexpr (DT == Q6_K) {                 // ql/qh/scales @0..207, d fp16 @208
        for (int t = 0; t < 208; t++) dq[t] = src[t];
        ds[0] = src[208];
        ds[1] = src[209];
    }
}

hipError_t launch_quant_f1(const float* a, int lda, int n, int k, int8_t* q, float* d, float* asum, int* s16,
                           hipStream_t st) {
    dim3 grid((k + 255) / 256, n);
    quant_f1_kernel<<<grid, 256, 0, st>>>(a, lda, k, q, d, asum, s16);
    return hipGetLastError();
}

hipError_t launch_quant_f2(const float* a, int lda, int n, int k, int8_t* q, float* d, float* xs,
                           hipStream_t st) {
    dim3 grid((k + 255) / 256, n);
    quant_f2_kernel<<<grid, 256, 0, st>>>(a, lda, k, q, d, xs);
    return hipGetLastError();
}

hipError_t launch_repack(int dt, const uint8_t* raw, int64_t raw_stride, int64_t rows, int64_t rb, uint8_t* qs,
                         uint8_t* sc, hipStream_t st) {
    const int64_t n = rows * rb;
    const dim3 grid((unsigned) ((n + 255) / 256));
    switch (dt) {
    case Q8_0: repack_kernel<Q8_0><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, qs, sc); break;
    case Q4_0: repack_kernel<Q4_0><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, qs, sc); break;
    case MXFP4: repack_kernel<MXFP4><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, qs, sc); break;
    case Q6_K: repack_kernel<Q6_K><<<grid, 256, 0, st>>>(raw, raw_stride, rows, rb, qs, sc); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace jamhip
