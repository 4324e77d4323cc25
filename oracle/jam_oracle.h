/* jam_oracle — CPU restatement of jam's quantized-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (qxotic_amd/, include/) links, loads or calls this
 * code: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only as the
 * checker. Every function names the reference file:line it restates (paths relative to the
 * qxoticai/qxotic repository root).
 *
 * Pinning (what keeps this restatement honest; the tests under tests/ run these checks):
 *   - jo_half2float, jo_e8m0_half            : exhaustive against closed forms (all 65536 / 256 codes).
 *   - jo_quant_f1 / jo_quant_f2              : bit-exact against libjam's own exported quantizers
 *                                             (jam_q8_0_requant, jam_q4k_quant) built from the reference
 *                                             sources into oracle/_ref/, and against committed fixtures.
 *   - jo_dequant_row (all dtypes)            : exact-value weights (integer scales, closed-form values)
 *                                             and brute-force double dots.
 *   - jo_mm_int8 (both flavours, all dtypes) : against libjam's jam_mm at matching n-ranges (same int8
 *                                             semantics, f32 order differs) and fixtures.
 *   - jo_mm_ref                              : closed forms + PRECISION.md bound against libjam.
 */
#ifndef JAM_ORACLE_H
#define JAM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml / jam dtype tags (jam/jam-native/include/jam.h:59-77; jam/jam-core/.../JAM.java:74-84). */
enum { JO_F32 = 0, JO_F16 = 1, JO_Q4_0 = 2, JO_Q8_0 = 8, JO_Q4_K = 12, JO_Q5_K = 13, JO_Q6_K = 14,
       JO_BF16 = 30, JO_MXFP4 = 39, JO_NVFP4 = 40, JO_Q1_0 = 41 };

/* Block geometry: elements and bytes per block (jam/jam-core/.../GGMLType.java:15-26). 0 if unknown. */
int    jo_block_elems(int dtype);
int    jo_block_bytes(int dtype);
/* Byte span of `rows` rows at element stride `stride` with `row_elems` data elements
 * (GGMLType.java:43-54). */
int64_t jo_span_bytes(int dtype, int rows, int stride, int row_elems);

/* IEEE half -> float, exact incl. subnormals/inf/nan (jam/jam-native/src/kernels/jam_fp16.h:8-27). */
float    jo_half2float(uint16_t h);
/* float -> IEEE half, round-to-nearest-even (the repo's own weight quantizers use it). */
uint16_t jo_float2half(float f);
/* E8M0 byte -> 2^(e-128) = 0.5*2^(e-127); e=0 -> 2^-128, e=255 -> +Inf
 * (jam/jam-native/src/kernels/jam_mxfp4.h:17-24). */
float    jo_e8m0_half(uint8_t e);

/* UE4M3 byte -> float as jam_ue4m3_to_float (jam/jam-native/src/kernels/jam_nvfp4.h:19-25): bit 7 ignored
 * but 0x00 and 0x7F (exactly) give 0; normal (1 + m/8)·2^(e-7), subnormal m·2^-9. */
float    jo_ue4m3(uint8_t x);
/* float -> bf16, round to nearest even (NaN kept quiet); what vcvtne2ps2bf16 does to jam's BF16 activations
 * (jam_kernels_bf16_avx512bf16.c). */
uint16_t jo_float2bf16(float f);

/* Decode one weight row of `k` elements (GGUF block layout) to float values
 * (jam_kernels_generic.c:42-321; ScalarJAM.java:95-201). Q4_K/Q6_K/Q5_K values are computed in double
 * and rounded once. */
void jo_dequant_row(int dtype, const uint8_t* wrow, int k, float* out);
void jo_dequant_row_f64(int dtype, const uint8_t* wrow, int k, double* out);

/* The repo's own weight quantizers (f32 -> GGUF blocks). The reference ships none for Q4_0/Q4_K/Q6_K. */
void jo_quantize_row(int dtype, const float* x, int k, uint8_t* out);

/* F1 activation quantizer, per 32-block: amax, d = amax/127, id = d>0 ? 1/d : 0, q = clamp(rint(x*id)),
 * asum = (float)Σq (jam/jam-native/src/kernels/jam_kernels_generic.c:71-94). */
void jo_quant_f1(const float* x, int k, int8_t* q, float* d, float* asum);
/* F2 activation quantizer, per 32-block: d = max/127, inv = max>0 ? 127/max : 0, q = sat8(rne(x*inv)),
 * plus raw f32 sums per 16 in the xor-8/4/2/1 tree of _mm512_reduce_add_ps
 * (jam/jam-native/src/kernels/jam_kernels_q4k_avx512.c:25-37). */
void jo_quant_f2(const float* x, int k, int8_t* q, float* d, float* xsum16);

/* jam's int8 pipeline, C[j*ldc+i] for i<m, j<n. flavour 1 = the n<8 decode decomposition (F1 quant;
 * jam.c:469-481 with the per-dtype kernels named in jam_oracle.c), flavour 2 = the n>=8 band
 * decomposition (F2 quant; jam.c:489-499, 544-560). flavour 0 picks jam's own rule: n<8 -> 1 on every
 * row; n>=8 -> 2 on rows [0, m - m%16) and an exact float dot on the last m%16 rows, as every 16-row
 * band kernel does for its tail (jam_kernels_q4k_avx512.c:185-188).
 * Per-block terms are formed in f32 exactly as jam forms its scale products, and summed in double.
 * Returns 0, or -1 for an unsupported dtype/shape. */
int jo_mm_int8(int dtype, const uint8_t* w, int ldw, const float* a, int lda, float* c, int ldc,
               int m, int n, int k, int flavour);

/* jam's dense paths (F32, F16, BF16 weights; jam.c:596-660) on an AVX-512-BF16 host: F32 and F16 take the
 * f32 activations as they are; BF16 rounds the activations to bf16 (vcvtne2ps2bf16) whenever jam's bf16
 * kernels take the call (n >= 8 with k even, or k % 32 == 0) and keeps them f32 otherwise (the dense
 * convert-and-FMA floor). Products are exact; summed in double. Returns 0, or -1 for another dtype. */
int jo_mm_dense(int dtype, const uint8_t* w, int ldw, const float* a, int lda, float* c, int ldc, int m, int n,
                int k);
/* 1 if jo_mm_dense rounds BF16 activations to bf16 for this (n, k). */
int jo_bf16_rounds_activations(int n, int k);

/* Float reference: C = Σ dequant(W)·A in double, plus sumabs = Σ|w·a| (QuantWeights.refDot contract,
 * jam/jam-vector/src/test/java/com/qxotic/jam/QuantWeights.java:67-75). Either output may be NULL. */
int jo_mm_ref(int dtype, const uint8_t* w, int ldw, const float* a, int lda, double* c, double* sumabs,
              int ldc, int m, int n, int k);

/* Seeded synthetic data: splitmix64 + Box-Muller, x = mean + std*N(0,1). */
void jo_fill_normal(uint64_t seed, float* x, size_t n, float mean, float std);
/* Config-4 activations: N(0,1) with Bernoulli(p) positions replaced by +-mag (random sign). */
void jo_fill_outliers(uint64_t seed, float* x, size_t n, float p, float mag);

#ifdef __cplusplus
}
#endif
#endif
