/*
 * oracle.h -- CPU restatement of Light's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * implementation in light_amd/ and the timed CPU baseline in bench.py.  It
 * is never linked into, loaded by, or called from the product path
 * (light_amd/), which fails loudly when its HIP library is missing.
 *
 * It restates, in plain C (+ AVX2/FMA intrinsics for the parts whose
 * floating-point order matters), the Go / Go-assembly CPU kernels of
 * sushvibez/light.  Every function cites the reference file:line it follows.
 * Light's Go code cannot be compiled here (no Go toolchain), so bit-identity
 * to a Go run is not provable; the restatement is pinned instead by the
 * reference's known-answer tests, exhaustive f16 checks, scalar-vs-AVX2
 * bit-identity (as Light's own TestAVX2DecodersExact does) and an f64 oracle.
 *
 * DType codes are Light's dtype.DType values (dtype/dtype.go:13-37).
 */
#ifndef LIGHT_ORACLE_H
#define LIGHT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  OR_F16 = 0, OR_BF16 = 1, OR_F32 = 2,
  OR_Q4_0 = 13, OR_Q5_0 = 15, OR_Q8_0 = 17, OR_Q8_1 = 18, OR_Q4_K = 21, OR_Q5_K = 22, OR_Q6_K = 23,
};

/* dtype/half.go */
float or_half_to_f32(uint16_t h);
uint16_t or_half_from_f32(float f);
uint16_t or_bf16_from_f32(float f);
void or_half_to_f32_avx2(const uint16_t *src, float *dst, int64_t n); /* F16C, n%8==0 */

/* Row decoders (kernels/cpu/quant_matmul.go:28-88 scalar; qdecode_amd64.s AVX2). */
int or_decode_row(int dt, const uint8_t *raw, int64_t K, float *dst);
int or_decode_row_avx2(int dt, const uint8_t *raw, int64_t K, float *dst);
void or_int4_row(const uint32_t *codes, const float *s, const float *z, float *dst, int64_t K, int G);
void or_int4_row_avx2(const uint32_t *codes, const float *s, const float *z, float *dst, int64_t K, int G);

/* quant.Dequantize (quant/dequant.go:13) for Q8_0 / Q4_K / Q6_K / Q8_1 into F32. */
int or_dequant(int dt, const uint8_t *raw, int64_t n, float *out);
/* ops.DequantizeInt4 CPU kernel (kernels/cpu/int4.go:19-54); out_dt F32 or BF16. */
int or_int4_dequant(const uint32_t *codes, const float *s, const float *z, void *out, int out_dt,
                    int64_t N, int64_t K, int G);

/* internal/simd */
float or_dot_avx2(const float *a, const float *b, int64_t n);
float or_dot_lanes(const float *a, const float *b, int64_t n); /* scalar emulation of the same order */
void or_dot4x3_avx2(const float *a, int64_t lda, const float *w, int64_t ldw, int64_t k, float *out);
void or_mattb(const float *a, int64_t lda, const float *w, int64_t ldw, float *out, int64_t ldo,
              int64_t m, int64_t n, int64_t k);

/* Light's CPU qmatmul: matmulQCPU (kernels/cpu/quant_matmul.go:141-170). threads<=0: all cores. */
int or_matmul_q(const float *x, const uint8_t *w, float *out, int64_t M, int64_t N, int64_t K, int dt,
                int threads);
/* int4MatMulCPU (kernels/cpu/quant_matmul.go:178-203); x F32. */
int or_int4_matmul(const float *x, const uint32_t *codes, const float *s, const float *z, float *out,
                   int64_t M, int64_t N, int64_t K, int G, int threads);

/* MoE: MoERouteFromIDs sort (ops/moe.go:78-99 + kernels/cpu/shape_ops.go:156-184, stable). */
void or_moe_route_from_ids(const int64_t *ids, int64_t M, int64_t *sorted_expts, int64_t *sorted_pairs);
void or_moe_route(const float *probs, int64_t T, int64_t E, int topk, int normalize, int64_t *topk_ids,
                  float *weights, int64_t *sorted_pairs, int64_t *sorted_expts);
/* moeGemmKernel F32 path (kernels/cpu/moe.go:51-96); w is F32 (E, N, K). */
int or_moe_gemm_f32(const float *x, const float *w, const int64_t *pairs, const int64_t *expts,
                    const float *topk_w, float *out, int64_t M, int64_t size_m, int64_t N, int64_t K,
                    int topk, int row_per_pair, int threads);
/* MoEGemmQ on the CPU (ops/moe.go:257-263): dequantize the whole stack, then moeGemmKernel.
 * w_scratch: E*N*K floats (caller-owned); NULL -> allocated internally. */
int or_moe_gemm_q(const float *x, const uint8_t *w, int dt, const int64_t *pairs, const int64_t *expts,
                  const float *topk_w, float *out, int64_t M, int64_t size_m, int64_t E, int64_t N,
                  int64_t K, int topk, int row_per_pair, int threads, float *w_scratch);
/* MoECombine (ops/moe.go:209-240): sum the topk slot rows in slot order. */
void or_moe_combine(const float *pair_out, float *out, int64_t M, int64_t N, int topk);
/* SiLU (act 0) or GeluErf (act 1) of g, times u (kernels/cpu/unary.go:216-222; Mul). */
void or_gated(const float *g, const float *u, float *out, int64_t n, int act);

/* Activation quantizers. */
void or_quantize_q8_0(const float *x, int64_t n, uint8_t *dst);  /* encodeQ8_0, quant/quantize.go:70-86 */
void or_quantize_q8_1(const float *x, int64_t n, uint8_t *dst);  /* q8_1 spec: quant/q8_1.go:10-18 + encodeQ8_0 rounding */

/* f64 dequant-then-matmul oracle: ref[m,n] = sum_k x[m,k]*w[n,k] in f64, mag = sum |x*w|,
 * wnorm[n] = ||w_n||_2, xnorm[m] = ||x_m||_2.  w is F32 (N, K) (dequantized). Any may be NULL. */
void or_matmul_f64(const float *x, const float *w, int64_t M, int64_t N, int64_t K, double *ref,
                   double *mag, double *wnorm, double *xnorm, int threads);

int or_hw_threads(void);

#ifdef __cplusplus
}
#endif
#endif
