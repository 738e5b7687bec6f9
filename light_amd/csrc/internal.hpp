// internal.hpp -- host-side helpers shared by the libhipq entry points.
#pragma once

#include <hip/hip_runtime.h>

#include "common.hpp"

namespace hq {

// Record a failure for hq_last_error() and return `code`.
int fail(int code, const char *call, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
// Map a hipError_t to the return convention (0 or the positive HIP code).
int check(hipError_t e, const char *call);
// Check the most recent kernel launch.
inline int check_launch(const char *call) { return check(hipGetLastError(), call); }
// NULL -> the library's current stream.
hipStream_t resolve(hq_stream_t s);
// Library-owned, grow-on-demand device workspace of the current device.
int workspace(size_t bytes, hipStream_t stream, void **out, const char *call);
// Frees every library-owned workspace (hq_workspace_release).
int workspace_release();

// Trace span: brackets one op call with HIP events while hq_trace_start is active.
struct TraceSpan {
  TraceSpan(const char *name, hipStream_t s);
  ~TraceSpan();
  const char *name;
  hipStream_t stream;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
};

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---- kernel launchers (one translation unit each) ----
int launch_quantize_q8_1(const void *x, int x_dtype, void *dst, int64_t M, int64_t K, hipStream_t s);
int launch_quantize_act(const void *x, int x_dtype, void *dst, int64_t M, int64_t K, hipStream_t s);
int launch_dequant(const void *src, void *dst, int64_t n, int src_dtype, int out_dtype, hipStream_t s);
// Q6_K_R (q6k_repack.hip): GGUF Q6_K (N, K) -> the planar layout, and its row-aware dequant.
int launch_repack_q6k(const void *src, void *dst, int64_t N, int64_t K, hipStream_t s);
int launch_dequant_q6kr(const void *src, void *dst, int64_t N, int64_t K, int out_dtype, hipStream_t s);
// matmul_q: quantizes x (GEMV, M <= kGemvMaxRows) or converts it to bf16 (Q4_K MFMA GEMM)
// in ws, then runs the kernel.
constexpr int64_t kGemvMaxRows = 8;
bool use_gemm(int64_t M, int dt);
// hq_matmul_q_act runs the MFMA GEMM (else the int8 GEMV on the prepared activations).
bool matmul_act_takes_gemm(int64_t M, int64_t K, int dt);
// hq_matmul_q_act runs long rows as K parts (ws: M * N floats).
bool act_long_rows_ok(int64_t M, int64_t N, int64_t K, int dt, const void *w, const void *act);
int launch_gemm_ws_bf16(const uint16_t *xb, const uint16_t *wb, float *out, float *partials, int64_t M, int64_t N,
                        int64_t K, hipStream_t s);
size_t matmul_q_ws_bytes(int64_t M, int64_t N, int64_t K, int dt);
size_t matmul_act_ws_bytes(int64_t M, int64_t N, int64_t K, int dt);
int launch_matmul_q(const float *x, const void *w, float *out, int64_t M, int64_t N, int64_t K, int dt, void *ws,
                    hipStream_t s);
const char *matmul_q_kernel_name(int64_t M, int dt);
// GEMV / GEMM on prepared (planar q8_1) activations.
int launch_gemv_act(const void *act, const void *w, float *out, int64_t M, int64_t N, int64_t K, int dt,
                    hipStream_t s);
int launch_matmul_act(const void *act, const void *w, float *out, int64_t M, int64_t N, int64_t K, int dt,
                      void *ws, hipStream_t s);
bool gemv_fast_ok(int dt, int64_t K, const void *w);
// Q4_K MFMA GEMM on bf16 activations; partials: split-K scratch (gemm_q4k_partial_bytes).
int launch_gemm_q4k_bf16(const uint16_t *xb, const void *w, float *out, float *partials, int64_t M, int64_t N,
                         int64_t K, hipStream_t s);
size_t gemm_q4k_ws_bytes(int64_t M, int64_t K);
// The all-waves Q4_K GEMM (gemm_q4k.hip) for M > 64.
bool gemm_q4k_ok(int64_t M, int64_t N, int64_t K, const void *w, const void *x);
size_t gemm_q4k2_ws_bytes(int64_t M, int64_t N, int64_t K);
int launch_gemm_q4k2(const uint16_t *xb, const void *w, float *out, void *ws, int64_t M, int64_t N, int64_t K,
                     hipStream_t s);
size_t gemm_q4k_partial_bytes(int64_t M, int64_t N, int64_t K);
// src_kind: F32, F16, BF16 (copy) or kActSrc (prepared activations).
constexpr int kActSrc = -1;
int launch_to_bf16(const void *src, int src_kind, uint16_t *dst, int64_t M, int64_t K, hipStream_t s);
size_t gemm_x_bytes(int64_t M, int64_t K);
size_t gemm_partial_bytes(int64_t M, int64_t N, int64_t K, bool f32_out);
int launch_gemm_int4_bf16(const uint16_t *xb, const uint32_t *codes, const float *sc, const float *zr, void *out,
                          int out_dtype, float *partials, int64_t M, int64_t N, int64_t K, int G, hipStream_t s);
int device_cus();
// Ceiling measurements (ceiling.hip).
int launch_ceiling_read(const void *buf, int64_t bytes, int order, int depth, uint32_t *sink, hipStream_t s);
int launch_ceiling_mfma(int64_t iters, float *sink, hipStream_t s);
int64_t ceiling_mfma_flops(int64_t iters);
int launch_ceiling_mix(int mode, int64_t iters, float *sink, hipStream_t s);
bool moe_stream_ok(int64_t rows, int64_t size_m, int64_t N, int64_t K, int64_t gated_I);
int launch_moe_stream_q4k(const uint16_t *xh, const float *xs, const void *w, const int64_t *pairs,
                          const int32_t *offsets, const float *topk_w, float *out, int topk, int64_t size_m, int64_t E,
                          int64_t N, int64_t K, int rpp, int64_t gated_I, int act, hipStream_t s);
// Q4_K GEMV on F32 x quantized in LDS (M <= kGemvMaxRows); w1 != NULL: gated pair,
// out = act(x.w0) * (x.w1), act 0 = SiLU, 1 = GELU (erf).
// x: F32 x or prepared activations (16-byte aligned); w1 may be NULL.
bool q4kx_ok(int64_t M, int64_t N, int64_t K, const void *w0, const void *w1, const void *x, int dt);
int launch_gemv_q4kx(const float *x, const void *w0, const void *w1, float *out, int64_t M, int64_t N, int64_t K,
                     int act, int dt, hipStream_t s);
int launch_gemv_q4kx_act(const void *act_in, const void *w, float *out, int64_t M, int64_t N, int64_t K, int dt,
                         hipStream_t s);
// Q4_K / Q5_K rows of 32768 < K <= 65536 at M <= 8: the act GEMV on each K half, then an add
// (tmp: M * N floats).
bool q4kx_halves_ok(int64_t M, int64_t N, int64_t K, int dt, const void *w, const void *act);
// The Q4_K / Q5_K halves for M >= 2 rows of F32 x: one launch per half for every row of x.
size_t q4kx_halves_x_ws_bytes(int64_t M, int64_t N, int64_t K);
int launch_gemv_q4kx_halves_x(const float *x, const void *w, float *out, void *ws, int64_t M, int64_t N, int64_t K,
                              int dt, hipStream_t s);
// out[i] += tmp[i], i < n (the second and later K parts of a split row).
int launch_add_rows(float *out, const float *tmp, int64_t n, hipStream_t s);
// Q8_0 / Q4_0 / Q5_0 / Q6_K rows too long to stage whole, at M <= 8: the staged GEMV on
// prepared activations over K parts of whole 8-block groups, summed (tmp: M * N floats).
bool staged_parts_ok(int64_t M, int64_t N, int64_t K, int dt, const void *w, const void *x);
int launch_staged_parts(const void *act, const void *w, float *out, float *tmp, int64_t M, int64_t N, int64_t K,
                        int dt, hipStream_t s);
int launch_gemv_q4kx_act_halves(const void *act_in, const void *w, float *out, float *tmp, int64_t M, int64_t N,
                                int64_t K, int dt, hipStream_t s);
// int4 GEMV on x quantized in the kernel (M <= kGemvMaxRows, G % 32 == 0, K % 64 == 0).
bool int4x_ok(int64_t M, int64_t N, int64_t K, int G, const void *codes, const void *x);
// int4 rows of 32768 < K <= 65536 (256 % G == 0) at M <= 8: two K halves + a combine
// (ws: the act layout of x, then 2 * M * N floats).
bool int4_halves_ok(int64_t M, int64_t N, int64_t K, int G, const void *codes, const void *x);
int launch_int4_halves(const void *x, int x_dtype, const uint32_t *codes, const float *sc, const float *zr, void *y,
                       int64_t M, int64_t N, int64_t K, int G, void *ws, hipStream_t s);
int launch_gemv_int4x(const void *x, int x_dtype, const uint32_t *codes, const float *sc, const float *zr, void *y,
                      int64_t M, int64_t N, int64_t K, int G, void *ws, hipStream_t s);
// Whether the decode GEMVs quantize x inside their workgroups at this K.
bool q4kx_xin(int64_t K);
size_t matmul_q_gated_ws_bytes(int64_t M, int64_t N, int64_t K, int dt);
size_t matmul_q_gated_act_ws_bytes(int64_t M, int64_t N, int64_t K, int dt);
int launch_matmul_q_gated_act(const float *x, const void *wg, const void *wu, uint8_t *aout, int64_t M, int64_t N,
                              int64_t K, int dt, int act, void *ws, hipStream_t s);
size_t mlp_q_ws_bytes(int64_t M, int64_t H, int64_t I, int dt);
int launch_mlp_q(const float *x, const void *wg, const void *wu, const void *wd, float *out, int64_t M, int64_t H,
                 int64_t I, int dt, int act, void *ws, hipStream_t s);
int launch_matmul_q_gated(const float *x, const void *wg, const void *wu, float *out, int64_t M, int64_t N, int64_t K,
                          int dt, int act, void *ws, hipStream_t s);
int launch_int4_dequant(const uint32_t *codes, const float *s, const float *z, void *out, int out_dtype,
                        int64_t N, int64_t K, int G, int64_t off, hipStream_t st);
int launch_int4_matmul(const void *x, int x_dtype, const uint32_t *codes, const float *s, const float *z, void *y,
                       int64_t M, int64_t N, int64_t K, int G, void *ws, hipStream_t st);
int launch_gather_cols(const void *x, const int64_t *idx, void *y, int64_t M, int64_t K, int elem_bytes,
                       hipStream_t s);
int i4f16_splits(int64_t N, int64_t K);
// GPTQ / AWQ checkpoint tensors -> canonical quant.Int4 (int4_convert.hip).
int launch_int4_from_gptq(const uint32_t *qw, const uint32_t *qz, const float *sc, const int64_t *perm, int64_t K,
                          int64_t N, int group, bool v2, uint32_t *codes, float *s_out, float *z_out, hipStream_t s);
int launch_int4_from_awq(const uint32_t *qw, const uint32_t *qz, const float *sc, int64_t K, int64_t N, int group,
                         uint32_t *codes, float *s_out, float *z_out, hipStream_t s);
bool i4cu_ok(int64_t M, int64_t N, int64_t K, int G, int x_dtype, const void *x, const void *codes);
int launch_i4cu(const uint16_t *x, const uint32_t *codes, const float *s, const float *z, void *y, int64_t M, int64_t N,
                int64_t K, int G, hipStream_t st);
bool i4f16_small_ok(int64_t M, int64_t N, int64_t K, int G, int x_dtype, const void *x, const void *codes);
int launch_i4f16_small(const uint16_t *x, const uint32_t *codes, const float *s, const float *z, void *y,
                       float *partials, int64_t M, int64_t N, int64_t K, int G, hipStream_t st);
size_t int4_ws_bytes(int64_t M, int64_t N, int64_t K, int G, int x_dtype);
size_t moe_ws_bytes(int64_t rows, int64_t K, int dt);
int launch_moe_combine(const float *pair, float *out, int64_t T, int64_t N, int topk, hipStream_t s);
int launch_moe_q(const float *x, const void *w, const int64_t *pairs, const int64_t *expts, int32_t *counts,
                 int32_t *offsets, const float *topk_w, float *out, int topk, int64_t size_m, int64_t M, int64_t rows,
                 int64_t E, int64_t N, int64_t K, int rpp, int dt, void *ws, hipStream_t s, float *zero_out = nullptr,
                 bool routed = false);
bool moe_x_ok(int64_t K, int dt, const void *w, const void *x);
int launch_moe_gemv_x(const float *x, const void *w, const int64_t *pairs, const int64_t *expts, int32_t *counts,
                      int32_t *offsets, const float *topk_w, float *out, int topk, int64_t size_m, int64_t M,
                      int64_t rows, int64_t E, int64_t N, int64_t K, int rpp, int dt, int act, hipStream_t s);
// On-device MoERoute / MoERouteFromIDs sort (moe_route.hip).
bool moe_route_fits(int64_t M, int64_t E);
// x_f32 / K / xh / xs (optional): each token's row of x is also converted to f16 with its
// power-of-two row scale (what the grouped GEMM's to_f16_rowscale_kernel writes, bit for bit).
int launch_moe_route(const float *probs, int64_t T, int64_t E, int topk, int normalize, int64_t *topk_ids,
                     float *weights, int64_t *sorted_pairs, int64_t *sorted_expts, int32_t *counts, int32_t *offsets,
                     hipStream_t s, const float *x_f32 = nullptr, int64_t K = 0, uint16_t *xh = nullptr,
                     float *xs = nullptr);
int launch_moe_sort_ids(const int64_t *ids, int64_t M, int64_t E, int64_t *sorted_pairs, int64_t *sorted_expts,
                        int32_t *counts, int32_t *offsets, hipStream_t s);
int launch_moe_q_gated(const float *x, const void *w, const int64_t *pairs, const int64_t *expts, int32_t *counts,
                       int32_t *offsets, float *out, int topk, int64_t size_m, int64_t M, int64_t rows, int64_t E,
                       int64_t I, int64_t K, int rpp, int dt, int act, void *ws, hipStream_t s, bool routed = false,
                       bool x_ready = false);
size_t moe_combine_ws_bytes(int64_t M, int64_t E, int64_t N, int64_t K, int dt);
int launch_moe_q_combine(const float *h, const void *w, const int64_t *pairs, const int64_t *expts, int32_t *counts,
                         int32_t *offsets, const float *topk_w, float *y, int topk, int64_t T, int64_t E, int64_t N,
                         int64_t K, int dt, void *ws, hipStream_t s, bool routed = false);
size_t moe_route_gated_ws_bytes(int64_t T, int topk, int64_t E, int64_t I, int64_t K, int dt);
int launch_moe_route_gated_any(const float *probs, const float *x, const void *w, float *h, int64_t T, int64_t E,
                               int topk, int normalize, int64_t I, int64_t K, int dt, int act, int64_t *topk_ids,
                               float *weights, int64_t *sorted_pairs, int64_t *sorted_expts, int32_t *counts,
                               int32_t *offsets, void *ws, hipStream_t s);
bool moe_route_gated_ok(int64_t T, int64_t E, int topk, int64_t K, int dt, const void *w, const void *x);
int launch_moe_route_gated(const float *probs, const float *x, const void *w, float *h, int64_t T, int64_t E,
                           int topk, int normalize, int64_t I, int64_t K, int dt, int act, int64_t *topk_ids,
                           float *weights, int64_t *sorted_pairs, int64_t *sorted_expts, int32_t *counts,
                           int32_t *offsets, hipStream_t s);
int launch_moe_block(const float *probs, const float *x, const void *wgu, const void *wdn, float *h, float *y,
                     int64_t T, int64_t E, int topk, int normalize, int64_t H, int64_t I, int dt, int act,
                     int64_t *topk_ids, float *weights, int64_t *sorted_pairs, int64_t *sorted_expts,
                     int32_t *counts, int32_t *offsets, uint8_t *hact, hipStream_t s);
size_t moe_block_ws_bytes(int64_t T, int topk, int64_t E, int64_t H, int64_t I, int dt);
int moe_block_check(hipStream_t s, const char *call);
void moe_block_set_spin_limit(uint32_t limit);
// A stream that is being destroyed stops owning the one-launch MoE block's barrier.
void moe_block_forget_stream(hipStream_t s);
int launch_moe_block_any(const float *probs, const float *x, const void *wgu, const void *wdn, float *h, float *y,
                         int64_t T, int64_t E, int topk, int normalize, int64_t H, int64_t I, int dt, int act,
                         int64_t *topk_ids, float *weights, int64_t *sorted_pairs, int64_t *sorted_expts,
                         int32_t *counts, int32_t *offsets, void *ws, hipStream_t s);
bool moe_int4_ok(int64_t H, int64_t I, int G, int topk);
size_t moe_int4_ws_bytes(int64_t T, int topk, int64_t I);
int launch_moe_int4(const void *x, int x_dtype, const void *const *tab, int64_t E, const int64_t *ids,
                    const float *w, void *y, int64_t T, int topk, int64_t H, int64_t I, int G, int act, void *ws,
                    hipStream_t s);
bool moe_comb_ok(int64_t M, int64_t T, int topk, int64_t K, int dt, const void *w, const void *x);
int launch_moe_down_combine(const float *h, const void *w, const int64_t *pairs, const int64_t *expts,
                            int32_t *counts, int32_t *offsets, const float *topk_w, float *y, int topk, int64_t T,
                            int64_t E, int64_t N, int64_t K, int dt, hipStream_t s);
size_t moe_gated_ws_bytes(int64_t size_m, int64_t rows, int64_t I, int64_t K, int dt);
int launch_moe_gemv_q4k(const void *act, const void *w, const int64_t *pairs, const int32_t *offsets,
                        const float *topk_w, float *out, int topk, int64_t size_m, int64_t M, int64_t rows,
                        int64_t E, int64_t N, int64_t K, int rpp, hipStream_t s);
// MoE grouped Q4_K GEMM: x (rows, K) F32 converted into xh (f16, rows * K * 2 bytes) and
// xs (rows row scales) in the caller's workspace, then the grouped f16 MFMA kernel.
// x_ready: xh / xs already hold that conversion (written by the routing launch).
int launch_moe_gemm_q4k(const float *x, uint16_t *xh, float *xs, const void *w, const int64_t *pairs,
                        const int32_t *offsets, const float *topk_w, float *out, int topk, int64_t size_m,
                        int64_t rows, int64_t E, int64_t N, int64_t K, int rpp, hipStream_t s, int64_t gated_I = 0,
                        int act = 0, bool x_ready = false);

}  // namespace hq
