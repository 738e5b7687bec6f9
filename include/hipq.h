/*
 * hipq.h -- C ABI of libhipq, the MI355X (gfx950) quantized-weight matmul library.
 *
 * This is the drop-in boundary for Light's quantized matmul path: the
 * functions below are what a cgo layer (kernels/rocm + internal/hiprt in a
 * Light tree) binds in place of the CUDA launchers and internal/cudart calls
 * for this path.  Each declaration cites the reference interface it replaces.
 *
 * Conventions
 *  - Every function returns int: 0 (HQ_OK) on success, a negative HQ_E* code
 *    for argument / support errors, or a positive hipError_t.  The message
 *    of the last failure on the calling thread is hq_last_error(), formatted
 *    like Light's cudart errors: "hipq: <call>: <msg> (code N)"
 *    (internal/cudart/runtime.go:335-337).
 *  - Pointers are device pointers unless stated; sizes are element counts.
 *    Weights are raw GGUF block bytes (dtype/dtype.go:53-60), never repacked.
 *  - `stream` is last; NULL means the library's current stream
 *    (hq_stream_set_current; the null stream until set), as Light issues all
 *    work on one process-wide current stream (internal/cudart/stream.go:22-30).
 *    All op calls are asynchronous, as cuLaunchKernel is in Light.
 *  - dtype codes are Light's dtype.DType values (dtype/dtype.go:13-37).
 *  - Workspace (`ws`, `ws_bytes`): device scratch for the on-GPU q8_1
 *    activation quantization.  Size it with the matching *_ws_bytes().
 *    ws == NULL makes the library use a buffer per (device, stream) that it
 *    allocates and grows on demand; growing retires the old buffer without
 *    freeing it (hq_workspace_release frees them).  During stream capture a
 *    growth fails with HQ_EUNSUPPORTED: pass ws, or use hq_matmul_q_noalloc.
 */
#ifndef HIPQ_H
#define HIPQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *hq_stream_t; /* == hipStream_t */

enum {
  HQ_OK = 0,
  HQ_EINVAL = -1,       /* bad argument (shape, dtype, pointer) */
  HQ_EUNSUPPORTED = -2, /* dtype / layout not handled by this library */
  HQ_ENOMEM = -3,       /* workspace too small or allocation failed */
  HQ_EBARRIER = -4,     /* a one-launch kernel's grid barrier gave up (hq_moe_block_q) */
};

/* dtype.DType codes (dtype/dtype.go:13-37). */
enum {
  HQ_F16 = 0, HQ_BF16 = 1, HQ_F32 = 2,
  HQ_Q4_0 = 13, HQ_Q5_0 = 15, HQ_Q8_0 = 17, HQ_Q8_1 = 18, HQ_Q4_K = 21, HQ_Q5_K = 22, HQ_Q6_K = 23,
  /* Not a Light dtype: the planar load-time layout of Q6_K that hq_repack_q6k writes. */
  HQ_Q6_K_R = 123,
};

/* ---- errors / version ------------------------------------------------- */

/* Thread-local text of the last failure ("" if none).
 * Replaces cudart's error rendering (internal/cudart/runtime.go:335-363). */
const char *hq_last_error(void);
/* Library ABI version (major*10000 + minor*100 + patch). */
int hq_version(void);

/* ---- runtime: the internal/cudart roles this path needs ---------------- */

/* cudart.DeviceCount (device/cuda.go:27-39, internal/cudart/runtime.go:40-50). */
int hq_device_count(int *count);
/* cudart.SetDevice (internal/cudart/runtime.go:52-62). */
int hq_set_device(int device);
/* cudart.Malloc / Free (internal/cudart/runtime.go:64-110); Light's caching
 * pool (storage/cuda.go:115-245) stays on the Go side. */
int hq_malloc(void **ptr, size_t bytes);
int hq_free(void *ptr);
/* cudart.MemcpyHtoD / DtoH / DtoD and Memset (internal/cudart/runtime.go:150-230).
 * h2d and d2h are synchronous with respect to `stream` (the host buffer may be
 * reused on return), as Light's copies are. */
int hq_memcpy_h2d(void *dst, const void *src, size_t bytes, hq_stream_t stream);
int hq_memcpy_d2h(void *dst, const void *src, size_t bytes, hq_stream_t stream);
int hq_memcpy_d2d(void *dst, const void *src, size_t bytes, hq_stream_t stream);
int hq_memset(void *dst, int value, size_t bytes, hq_stream_t stream);
/* cudart stream helpers (internal/cudart/stream.go:12-60). */
int hq_stream_create(hq_stream_t *stream);
/* hq_stream_destroy waits for the stream to drain, frees the library workspace it used for
 * calls with ws == NULL (graphs captured on it with ws == NULL must not be replayed after
 * this), and destroys it. */
int hq_stream_destroy(hq_stream_t stream);
int hq_stream_synchronize(hq_stream_t stream);
int hq_stream_set_current(hq_stream_t stream);
hq_stream_t hq_stream_get_current(void);

/* GPU trace spans (internal/cudart/gputrace.go:24-101): while tracing, every
 * op call is bracketed by a pair of HIP events; hq_trace_stop synchronizes
 * and reports, per kernel family, the call count and total microseconds.
 * names: caller buffer of n_max * 32 chars; returns the number of entries. */
int hq_trace_start(void);
int hq_trace_stop(char *names, int *calls, double *total_us, int n_max);

/* ---- ops ----------------------------------------------------------------- */

/* Pointers: activations (x, act, h) and GGUF weight buffers start 16-byte aligned, F32 outputs
 * 4-byte aligned (hipMalloc and torch allocations are 256-byte aligned); a misaligned base
 * pointer is HQ_EINVAL, never a silent misread.  Row lengths need no alignment: rows whose
 * byte length is not a multiple of 16 take the generic paths named below.  Empty operands
 * (M, N or T = 0) return HQ_OK and launch nothing. */

/* Workspace bytes hq_matmul_q needs for x (M, K), a weight (N, K) and w_dtype. */
size_t hq_matmul_q_ws_bytes(int64_t M, int64_t N, int64_t K, int w_dtype);

/* out (M, N) F32 = x (M, K) F32 contiguous @ dequant(w (N, K))^T.
 * w_dtype: one of the six GGUF formats Light fuses: HQ_Q4_0, HQ_Q5_0, HQ_Q8_0, HQ_Q4_K,
 * HQ_Q5_K or HQ_Q6_K, or HQ_Q6_K_R (a Q6_K weight after hq_repack_q6k).  K must be a
 * multiple of the block size.
 *  - M <= 8, Q4_K / Q5_K / Q6_K_R: the persistent int8-dot GEMV, x quantized to q8_1 inside its
 *    workgroups (K > 8192: into ws first).
 *  - M <= 8, Q8_0 / Q4_0 / Q5_0 / Q6_K: the LDS-staged int8-dot GEMV (x quantized in its
 *    workgroups up to K = 8192, into ws above).
 *  - M > 8 (K % 64 == 0): the bf16 MFMA GEMM; x is rounded to bf16 in ws; Q4_K tiles are
 *    dequantized inside the GEMM, the other formats once to a bf16 copy in ws.
 *  - M <= 8, rows longer than one GEMV team (Q4_K / Q5_K, 32768 < K <= 65536) or one LDS
 *    slice (the staged formats past 16 KB per row): x quantized into ws once, the GEMV over
 *    K parts on the full row stride, the parts' outputs summed in ws.
 *  - Rows whose byte length is not a multiple of 16: a generic F32 GEMV with the bit-exact
 *    decoder.
 * Replaces registry kernel "matmul_q" (ops/matmul_q.go:61-75; CUDA launcher
 * kernels/cuda/matmul_q.go:44-91) and, since it serves every M, the M >= 8
 * dequant + cuBLAS fallback (ops/matmul_q.go:52-59, 85-95). */
int hq_matmul_q(const float *x, const void *w, float *out, int64_t M, int64_t N, int64_t K, int w_dtype,
                void *ws, size_t ws_bytes, hq_stream_t stream);

/* Allocation-free hq_matmul_q: the same kernels and results, with the scratch taken from a
 * device array of HQ_NOALLOC_SCRATCH_BYTES that the library holds on each GPU it runs on
 * (a static device symbol, present from module load until the process ends).  Calls no
 * hipMalloc / hipFree, so it may be used under HIP graph capture, in serving loops, and by
 * harnesses that forbid allocation.  Returns HQ_ENOMEM when hq_matmul_q_ws_bytes(M, N, K,
 * w_dtype) exceeds HQ_NOALLOC_SCRATCH_BYTES (decode GEMVs need kilobytes; the Q4_K GEMM
 * needs 2*M*K bytes plus split-K partials, e.g. M = 512, K = 14336 fits).  Every call on a
 * GPU shares that GPU's scratch: calls that overlap on one GPU (two streams, or two
 * threads) race; serialise them.  No counterpart in Light: it is for callers that cannot
 * allocate. */
#define HQ_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int hq_matmul_q_noalloc(const float *x, const void *w, float *out, int64_t M, int64_t N, int64_t K, int w_dtype,
                        hq_stream_t stream);

/* Frees the library-owned workspaces (ws == NULL calls) after a device synchronisation on
 * each device that has one.  The caller guarantees that no call or captured graph that
 * used them still runs.  cudart has no counterpart: Light's op scratch lives in its Go
 * storage pool (storage/cuda.go:115-245). */
int hq_workspace_release(void);

/* Gated MLP projection (the SwiGLU / GeGLU decode step):
 *   out (M, N) F32 = act(x @ dequant(wg)^T) * (x @ dequant(wu)^T),
 * act HQ_ACT_SILU (x / (1 + exp(-x))) or HQ_ACT_GELU_ERF (0.5 x (1 + erf(x / sqrt 2))).
 * Same x / weight / workspace rules as hq_matmul_q; wg and wu share dtype and shape.
 * For Q4_K with M <= 8 one kernel reads both weights (x quantized in LDS, no workspace
 * used); other cases run the two matmuls and an elementwise epilogue.
 * Light computes this as MatMulQ, MatMulQ, SiLU / GeluErf and Mul (models/llama.go:1306-1328;
 * kernels/cpu/unary.go:216-222); its fused dense counterpart is ops.GatedLinear
 * (ops/gemv.go:80-130).  No quantized counterpart in Light. */
enum { HQ_ACT_SILU = 0, HQ_ACT_GELU_ERF = 1 };
size_t hq_matmul_q_gated_ws_bytes(int64_t M, int64_t N, int64_t K, int w_dtype);
int hq_matmul_q_gated(const float *x, const void *wg, const void *wu, float *out, int64_t M, int64_t N, int64_t K,
                      int w_dtype, int act, void *ws, size_t ws_bytes, hq_stream_t stream);

/* Gated projection that emits prepared activations for the next matmul:
 *   act_out (hq_act_bytes(M, N) bytes) = quantize_act(act(x @ dequant(wg)^T) * (x @ dequant(wu)^T)),
 * the same values hq_quantize_act would write for the F32 gated output.  N % 32 == 0.
 * For Q4_K / Q5_K with M <= 8 this is one kernel: the gated GEMV quantizes each completed
 * 32-row chunk of its output in the epilogue (the first launch of hq_mlp_q).  Other cases
 * run hq_matmul_q_gated into ws, then the quantizer.  Feed act_out to hq_matmul_q_act (the
 * down projection).  Light: models/llama.go:1306-1328 (gate, up, SiLU * up before
 * DownProj); no counterpart op in Light. */
size_t hq_matmul_q_gated_act_ws_bytes(int64_t M, int64_t N, int64_t K, int w_dtype);
int hq_matmul_q_gated_act(const float *x, const void *wg, const void *wu, void *act_out, int64_t M, int64_t N,
                          int64_t K, int w_dtype, int act, void *ws, size_t ws_bytes, hq_stream_t stream);

/* The gated MLP block of a decoder layer:
 *   out (M, H) F32 = (act(x @ dequant(wg)^T) * (x @ dequant(wu)^T)) @ dequant(wd)^T
 * with x (M, H) F32, wg and wu (I, H), wd (H, I), all of w_dtype; act as above.
 * For Q4_K with M <= 8 this is two launches: the gated gate/up GEMV, which writes its
 * output already quantized for the next matmul into ws, and the down GEMV on it.  Other
 * cases run hq_matmul_q_gated into ws and then hq_matmul_q.
 * Light: models/llama.go:1306-1333 (GatedLinear or MatMulQ/SiLU/Mul, then DownProj).
 * No counterpart op in Light. */
size_t hq_mlp_q_ws_bytes(int64_t M, int64_t H, int64_t I, int w_dtype);
int hq_mlp_q(const float *x, const void *wg, const void *wu, const void *wd, float *out, int64_t M, int64_t H,
             int64_t I, int w_dtype, int act, void *ws, size_t ws_bytes, hq_stream_t stream);

/* Prepared activations: hq_matmul_q = hq_quantize_act + hq_matmul_q_act (bit for bit
 * for Q8_0 / Q6_K; the Q4_K GEMV quantizes x inside its own workgroups with
 * reciprocal-based scales, so there the two agree to the activation rounding).
 * A caller that multiplies one activation by several weights (the SwiGLU gate
 * and up projections, models/llama.go:1306-1328) quantizes once and reuses it.
 * No counterpart in Light.  The act buffer (hq_act_bytes(M, K) bytes, 16-byte
 * aligned) holds a two-level int8 quantization of x in a planar layout:
 *   q1 int8 [M][K]            q8_1's quants (d = amax/127), as hq_quantize_q8_1
 *   q2 int8 [M][K]            quants of the residual x - d*q1 at step e = d/254
 *   (d, e) f32 pairs [M][K/32] (d before q8_1's f16 rounding)
 *   sx f32 [M][K/32]          the block sum of x
 * so x = d*q1 + e*q2 to within e/2 (about 2^-15 of the block's amax); offsets are
 * rounded up to 256 bytes.  The decode GEMVs read q1 alone (exactly q8_1) for rows of
 * K >= 4096, where the rounding averages out below the 1e-3 bar; shorter rows and the MoE
 * GEMVs use both levels.  The layout is internal and may change with the version. */
size_t hq_act_bytes(int64_t M, int64_t K);
int hq_quantize_act(const void *x, int x_dtype, void *act, int64_t M, int64_t K, hq_stream_t stream);
/* Workspace hq_matmul_q_act needs beyond the act buffer (0 for the GEMV). */
size_t hq_matmul_q_act_ws_bytes(int64_t M, int64_t N, int64_t K, int w_dtype);
/* out (M, N) F32 = x @ dequant(w)^T from prepared activations.  For M <= 8, and for
 * any M when K is not a multiple of 64, the weight must take the int8 GEMV (16-byte
 * aligned, rows a multiple of 16 bytes; HQ_EUNSUPPORTED otherwise -- hq_matmul_q takes
 * every layout); rows longer than one GEMV team or LDS slice run as K parts, summed in ws
 * (M * N floats). */
int hq_matmul_q_act(const void *act, const void *w, float *out, int64_t M, int64_t N, int64_t K, int w_dtype,
                    void *ws, size_t ws_bytes, hq_stream_t stream);

/* Dequantize n elements of GGUF blocks to F32 or BF16 (bit-exact with Light's
 * CPU decoders; BF16 rounds the F32 value once, RNE).
 * Replaces the "dequant" hook (quant/cuda_hook.go:17-69, kernels/cuda/dequant.go:39-80). */
int hq_dequant(const void *src, void *dst, int64_t n, int src_dtype, int out_dtype, hq_stream_t stream);

/* Bytes of the Q6_K_R copy of a Q6_K weight (N, K): N rows of ceil16(210 * K / 256) bytes. */
size_t hq_repack_q6k_bytes(int64_t N, int64_t K);
/* Load-time repack of a Q6_K weight (N, K) (GGUF blocks of 210 bytes, 2-byte aligned;
 * quant/q6_k.go:10-27) into the Q6_K_R layout, which the decode GEMV reads with aligned
 * 16-byte loads.  Per row (K = 256 nb, P = 4 nb units of 64 weights; unit u = 4 b + v of
 * block b pairs the element groups g = v % 2 and g + 2 of half h = v / 2):
 *   [0, 16 P)      unit u's quant bytes 0..15  (ql[64 h + 32 g + i], i < 16)
 *   [16 P, 32 P)   its quant bytes 16..31
 *   [32 P, 48 P)   its 2-bit highs: dword m, byte t = the highs of element 8m+t (bits 0-1)
 *                  and 8m+4+t (bits 2-3) of group g, then the same two of group g+2
 *   [48 P, 52 P)   its four scales: scales[8h + 2g], [8h + 2g + 1], [8h + 2g + 4], [8h + 2g + 5]
 *   [52 P, 52 P + 2 nb)  d (f16) of each block; then zero padding to the row size.
 * Values are unchanged: hq_dequant_rows of the copy equals hq_dequant of the original, bit
 * for bit.  Light keeps GGUF bytes; a loader that wants the faster Q6_K GEMV calls this once
 * per weight and passes HQ_Q6_K_R to hq_matmul_q.  No counterpart in Light. */
int hq_repack_q6k(const void *src, void *dst, int64_t N, int64_t K, hq_stream_t stream);

/* Dequantize a weight (N, K) of src_dtype (any dtype hq_dequant takes, or HQ_Q6_K_R, whose
 * rows are padded) to F32 or BF16 (N, K), bit-exact as hq_dequant. */
int hq_dequant_rows(const void *src, void *dst, int64_t N, int64_t K, int src_dtype, int out_dtype,
                    hq_stream_t stream);

/* Quantize x (M, K) (F32, BF16 or F16) to q8_1 blocks (M, K/32) x 36 bytes:
 * [f16 d][f16 s][i8 q[32]] (quant/q8_1.go:10-18) with encodeQ8_0's rounding
 * (quant/quantize.go:70-86): d = amax/127, q = RoundToEven(v * (1/d)),
 * s = f16(f32(sum q) * d).  No counterpart in Light (which has no q8_1
 * encoder); bit-exact with the specification. */
int hq_quantize_q8_1(const void *x, int x_dtype, void *dst, int64_t M, int64_t K, hq_stream_t stream);

/* Workspace bytes hq_int4_matmul needs (x (M, K) of x_dtype, weight (N, K), group G). */
size_t hq_int4_matmul_ws_bytes(int64_t M, int64_t N, int64_t K, int G, int x_dtype);

/* y (M, N) = x (M, K) @ W^T for Light's canonical 4-bit layout (quant.Int4,
 * quant/int4.go:11-34): codes U32 (N, K/8), nibble j of word c = W[n, 8c+j];
 * scales / zeros F32 (N, K/G); W = s * (code - z).  x_dtype F32, BF16 or F16;
 * y has x's dtype (F16 is an extension: Light takes F32 or BF16, ops/int4.go:70-72).
 * K % 32 == 0 and G % 32 == 0.  M <= 8 (or G % 64 != 0): x is quantized to q8_1
 * into ws and the int8-dot GEMV runs (K <= 65536; rows past 32768 with 256 % G == 0 as two
 * K halves whose F32 partials are summed in ws); otherwise -- and for longer rows at
 * any M when G % 64 == 0 -- the MFMA GEMMs run (F16 x at 8 < M <= 64 as given, else
 * rounded to bf16 into ws).  G % 64 != 0 with K > 65536 is HQ_EUNSUPPORTED.
 * Replaces registry kernel "int4_gemv" (ops/int4.go:87-99; kernels/cuda/int4.go:76-101)
 * and, since it serves every M, the dequant + GEMM path (ops/int4.go:100-126). */
int hq_int4_matmul(const void *x, int x_dtype, const uint32_t *codes, const float *scales, const float *zeros,
                   void *y, int64_t M, int64_t N, int64_t K, int G, void *ws, size_t ws_bytes,
                   hq_stream_t stream);

/* Expand canonical 4-bit weights to (N, K) F32 or BF16 at element offset
 * out_offset of out: s * (q - z) in F32, rounded once (bit-exact with Light).
 * Replaces registry kernel "int4_dequant" (ops/int4.go:34-56; kernels/cuda/int4.go:43-70). */
int hq_int4_dequant(const uint32_t *codes, const float *scales, const float *zeros, void *out, int out_dtype,
                    int64_t N, int64_t K, int G, int64_t out_offset, hq_stream_t stream);

/* GPTQ checkpoint tensors -> canonical 4-bit weights, on the device (quant.FromGPTQ,
 * quant/int4.go:102-182).  qweight I32 (K/8, N) packed along K (nibble j of qweight[r][n] is
 * row 8r + j); qzeros I32 (K/group, N/8) packed along N, holding zero - 1 ("gptq") or, with
 * v2 != 0, the zero ("gptq_v2"); scales F32 (K/group, N) (the caller casts the checkpoint's
 * F16).  perm: NULL, or I64 (K) for act-order checkpoints -- canonical column k takes input
 * row perm[k] (Light's stable sort of K by g_idx; the host layer computes it).  Writes codes
 * U32 (N, K/8), scales_out / zeros_out F32 (N, K/group).  K and N multiples of 8. */
int hq_int4_from_gptq(const void *qweight, const void *qzeros, const float *scales, const int64_t *perm, int64_t K,
                      int64_t N, int group, int v2, uint32_t *codes, float *scales_out, float *zeros_out,
                      hq_stream_t stream);

/* AutoAWQ (GEMM version) checkpoint tensors -> canonical 4-bit weights, on the device
 * (quant.FromAWQ, quant/int4.go:184-235).  qweight I32 (K, N/8) and qzeros I32 (K/group, N/8)
 * packed along N, nibble i of a word holding column 8c + (0, 2, 4, 6, 1, 3, 5, 7)[i]; scales
 * F32 (K/group, N).  Writes codes U32 (N, K/8), scales_out / zeros_out F32 (N, K/group). */
int hq_int4_from_awq(const void *qweight, const void *qzeros, const float *scales, int64_t K, int64_t N, int group,
                     uint32_t *codes, float *scales_out, float *zeros_out, hq_stream_t stream);

/* Workspace bytes hq_moe_gemm_q needs for `rows` input rows of K elements. */
size_t hq_moe_gemm_q_ws_bytes(int64_t rows, int64_t K, int w_dtype);

/* Grouped expert qmatmul (ops.MoEGemmQ, ops/moe.go:242-265):
 *   out[p, :] = w(p) * x[row(p), :] @ dequant(W[e(p)])^T  for every routed pair p,
 * row(p) = row_per_pair ? p : p / topk, w(p) = topk_w[p] or 1 (topk_w NULL).
 * x F32 (rows, K); W (E, N, K) GGUF blocks; sorted_pairs / sorted_expts I64 (M)
 * expert-sorted (MoERouteFromIDs, ops/moe.go:78-99); counts I32 (E) and
 * offsets I32 (E+1) are scratch the caller zeroes, as Light's op layer
 * allocates them (ops/moe.go:172-179); out F32 (size_m, N) zeroed by the
 * caller; pairs outside [0, size_m) are skipped.
 * Replaces registry kernel "moe_gemm_q" (kernels/cuda/moe.go:78-141). */
int hq_moe_gemm_q(const float *x, const void *w, const int64_t *sorted_pairs, const int64_t *sorted_expts,
                  int32_t *counts, int32_t *offsets, const float *topk_w, float *out, int topk, int64_t size_m,
                  int64_t M, int64_t rows, int64_t E, int64_t N, int64_t K, int row_per_pair, int w_dtype,
                  void *ws, size_t ws_bytes, hq_stream_t stream);

/* MoECombine (ops/moe.go:206-240): out (M/topk, N) F32, out[t] = sum of the topk
 * slot rows of pair_out (M, N) F32, added in slot order as Light's chain of Add ops
 * does (bit-identical). */
int hq_moe_combine(const float *pair_out, float *out, int64_t M, int64_t N, int topk, hq_stream_t stream);

/* The routed down projection with MoECombine in its epilogue:
 *   y (T, N) F32 = MoECombine(MoEGemmQ(h, w, routing, topk_w, topk), topk),
 * h F32 (T*topk, K) per pair (row_per_pair), W (E, N, K) GGUF blocks, routing arguments as
 * hq_moe_gemm_q with size_m = M = T*topk; counts / offsets nullable (written when given).
 * Bit-identical to hq_moe_gemm_q + hq_moe_combine.  For Q4_K / Q5_K decode one kernel
 * computes each (token, output row) over the token's topk experts and adds the slots in
 * slot order; other cases run those two ops through ws.  Light: nn/moe.go:230-235
 * (MoEGemmQ then MoECombine, ops/moe.go:209-265); no counterpart kernel in Light. */
size_t hq_moe_gemm_q_combine_ws_bytes(int64_t T, int topk, int64_t E, int64_t N, int64_t K, int w_dtype);
int hq_moe_gemm_q_combine(const float *h, const void *w, const int64_t *sorted_pairs, const int64_t *sorted_expts,
                          int32_t *counts, int32_t *offsets, const float *topk_w, float *y, int topk, int64_t T,
                          int64_t E, int64_t N, int64_t K, int w_dtype, void *ws, size_t ws_bytes,
                          hq_stream_t stream);

/* On-device MoERoute (ops/moe.go:29-71): probs F32 (T, E) -> topk_ids I64 (T, topk), weights
 * F32 (T*topk) (renormalised per token when normalize != 0: den = left-to-right f32 sum of
 * the k values, then value / den), and the stable expert sort of the T*topk pairs:
 * sorted_pairs / sorted_expts I64 (T*topk).  Top-k ties keep index order (Light's stable
 * descending sort, kernels/cpu/topk.go:52-68); probs must be finite.  counts I32 (E) and
 * offsets I32 (E+1) (nullable) receive moe_gemm_q's scratch for the same routing.
 * Limits: 1 <= topk <= min(E, 64), E <= 1024, T*topk <= 65535 and
 * 2 T topk + 2 ceil(T topk / 64) E + 4 E <= 160 KiB (the sort runs in one workgroup).
 * Replaces ops.MoERoute's TopK / Sum / Div / Sort dispatches (kernels/cuda). */
int hq_moe_route(const float *probs, int64_t T, int64_t E, int topk, int normalize, int64_t *topk_ids,
                 float *weights, int64_t *sorted_pairs, int64_t *sorted_expts, int32_t *counts, int32_t *offsets,
                 hq_stream_t stream);

/* The sort of MoERouteFromIDs (ops/moe.go:78-99: Sort(flat ids, ascending), stable) on the
 * device: ids I64 (M) in [0, E) -> sorted_pairs / sorted_expts I64 (M), plus counts /
 * offsets (nullable) as hq_moe_route.  Same limits with T*topk = M. */
int hq_moe_sort_ids(const int64_t *ids, int64_t M, int64_t E, int64_t *sorted_pairs, int64_t *sorted_expts,
                    int32_t *counts, int32_t *offsets, hq_stream_t stream);

/* Workspace bytes hq_moe_gemm_q_gated needs. */
size_t hq_moe_gemm_q_gated_ws_bytes(int64_t size_m, int64_t rows, int64_t I, int64_t K, int w_dtype);

/* Routed gated gate/up of nn.SparseMoE.runExperts (nn/moe.go:196-236): w is the stacked
 * GateUp (E, 2I, K) quantized (gate rows [0, I), up rows [I, 2I) of each expert), and
 * out (size_m, I) F32 gets h[p] = act(x_row(p) . Wg[e(p)]) * (x_row(p) . Wu[e(p)]) -- the
 * MoEGemmQ, Narrow, SiLU / GeluErf and Mul of that function in one op (one kernel for
 * Q4_K / Q5_K decode).  Routing arguments as hq_moe_gemm_q; act HQ_ACT_SILU or
 * HQ_ACT_GELU_ERF.  No counterpart kernel in Light: these launches fused. */
int hq_moe_gemm_q_gated(const float *x, const void *w, const int64_t *sorted_pairs, const int64_t *sorted_expts,
                        int32_t *counts, int32_t *offsets, float *out, int topk, int64_t size_m, int64_t M,
                        int64_t rows, int64_t E, int64_t I, int64_t K, int row_per_pair, int w_dtype, int act,
                        void *ws, size_t ws_bytes, hq_stream_t stream);

/* MoERoute followed by the routed gated gate/up, the first half of the SparseMoE decode block
 * (nn/moe.go:150-225: MoERoute, then runExperts' MoEGemmQ, Narrow, SiLU / GeluErf, Mul):
 * probs F32 (T, E) -> topk_ids, weights, sorted_pairs, sorted_expts as hq_moe_route, and
 * h F32 (T*topk, I) per pair as hq_moe_gemm_q_gated with x F32 (T, K) per token and the
 * stacked GateUp w (E, 2I, K).  counts / offsets nullable.  Bit-identical to hq_moe_route +
 * hq_moe_gemm_q_gated.  For Q4_K / Q5_K with T <= 8 and T*topk <= 64 one kernel runs both:
 * each workgroup selects the top-k and sorts the pairs itself, so no launch sits between
 * the router and the expert weights.  Limits as hq_moe_route.  No counterpart in Light. */
size_t hq_moe_route_gated_ws_bytes(int64_t T, int topk, int64_t E, int64_t I, int64_t K, int w_dtype);
int hq_moe_route_gated(const float *probs, const float *x, const void *w, float *h, int64_t T, int64_t E, int topk,
                       int normalize, int64_t I, int64_t K, int w_dtype, int act, int64_t *topk_ids, float *weights,
                       int64_t *sorted_pairs, int64_t *sorted_expts, int32_t *counts, int32_t *offsets, void *ws,
                       size_t ws_bytes, hq_stream_t stream);

/* The SparseMoE decode block (nn/moe.go:150-236: MoERoute, runExperts' MoEGemmQ, Narrow,
 * SiLU / GeluErf, Mul, MoEGemmQ with the routing weights, MoECombine): hq_moe_route_gated
 * followed by hq_moe_gemm_q_combine, with their arguments (x F32 (T, H), w_gate_up the
 * stacked GateUp (E, 2I, H), w_down (E, H, I), h F32 (T*topk, I) the per-pair activations it
 * writes on the way, y F32 (T, H)) and the same bits.  For one token (T = 1) of Q4_K / Q5_K
 * one kernel runs the whole block, with a grid barrier between the gate/up and the down
 * projection; that kernel serves the first stream that calls this function on a device
 * (other streams get the two launches), and graph replays of it must not run beside one
 * another.  No counterpart kernel in Light: these launches fused. */
/* The one-launch kernel needs its whole grid resident at once.  It is sized to the
 * occupancy, but kernels of other streams or processes can hold CUs, so its grid barrier is
 * a bounded wait (2^22 polls: 0.1 s to a few seconds).  A workgroup that gives up writes NaN
 * to its rows of y and sets a flag in pinned host memory; the next hq_moe_block_q on the
 * device then returns HQ_EBARRIER without launching anything (or hq_moe_block_q_check does,
 * after synchronizing the stream), and from then on the device takes the two launches. */
size_t hq_moe_block_q_ws_bytes(int64_t T, int topk, int64_t E, int64_t H, int64_t I, int w_dtype);
int hq_moe_block_q(const float *probs, const float *x, const void *w_gate_up, const void *w_down, float *h, float *y,
                   int64_t T, int64_t E, int topk, int normalize, int64_t H, int64_t I, int w_dtype, int act,
                   int64_t *topk_ids, float *weights, int64_t *sorted_pairs, int64_t *sorted_expts, int32_t *counts,
                   int32_t *offsets, void *ws, size_t ws_bytes, hq_stream_t stream);
/* Synchronizes `stream`, then returns HQ_EBARRIER (and clears the flag) if a one-launch MoE
 * block on the current device gave up at its grid barrier since the last report, else HQ_OK.
 * No counterpart in Light (its ops report every failure as an error, ops/moe.go:247-265). */
int hq_moe_block_q_check(hq_stream_t stream);
/* Test hook: the number of s_sleep(1) polls the one-launch block's barrier makes before it
 * gives up (0: give up at once, so every workgroup fails and exits normally; the default is
 * 2^22).  It also re-enables the one launch on the current device after a reported failure
 * and hands the kernel to the next stream that runs the block. */
void hq_debug_moe_block_spin_limit(uint32_t limit);

/* ops.MoEInt4 (ops/int4.go:149-246): the routed gated-MLP expert block with canonical 4-bit
 * experts (GPTQ / AWQ MoE checkpoints):
 *   y[t] (T, H) = sum over j < topk of w[t*topk+j] * down_e(act(gate_e x[t]) * up_e x[t]),
 *   e = topk_ids[t*topk+j], the slots added onto zero in slot order, y at x's dtype.
 * x (T, H) F32 / BF16 / F16.  expert_tab: a DEVICE array of 6*E pointers -- the E gate-up
 * codes (U32 (2I, H/8), gate rows then up rows), their E scales and E zeros (F32 (2I, H/G)),
 * then the E down codes (U32 (H, I/8)), scales and zeros (F32 (H, I/G)).  topk_ids I64 and
 * weights F32 (T*topk) are the routing (MoERouting.TopKIDs / Weights).  Only the routed
 * experts' rows are read: nothing is expanded (Light dequantizes the used experts into its
 * weight scratch, ops/int4.go:199-215).  An id outside [0, E) contributes zero (Light
 * returns "expert out of range").  H and I multiples of 64 with G % 32 == 0 take the int8-dot
 * GEMV kernels (x and h quantized in the workgroups); other shapes a generic F32 kernel. */
size_t hq_moe_int4_ws_bytes(int64_t T, int topk, int64_t I);
int hq_moe_int4(const void *x, int x_dtype, const void *const *expert_tab, int64_t E, const int64_t *topk_ids,
                const float *weights, void *y, int64_t T, int topk, int64_t H, int64_t I, int G, int act, void *ws,
                size_t ws_bytes, hq_stream_t stream);

/* y (M, K) = x[:, idx] for 2- or 4-byte elements (ops.gatherColumns, ops/int4.go:129-147):
 * the act-order (desc_act) permutation of quant.Int4.Perm applied to the activations.
 * Indices outside [0, K) give zeros. */
int hq_gather_cols(const void *x, const int64_t *idx, void *y, int64_t M, int64_t K, int elem_bytes,
                   hq_stream_t stream);

/* ---- ceilings (measurement only; no counterpart in Light) ----------------
 * What the hardware sustains, reported beside the roofline fractions.
 * hq_ceiling_read: one launch that reads `bytes` (16-byte aligned) of `buf` with 16-byte
 * loads, `depth` (1, 2, 4 or 8) in flight per thread, two 512-thread workgroups per CU;
 * order 0 reads a contiguous window that moves through the buffer (grid stride), order 1
 * gives each workgroup its own contiguous slice, order 2 reads order 0's bytes as half cache
 * lines (each load 16 rows x 64 bytes, the other halves a trip later; `bytes` a multiple of
 * 2048).  `sink`: one device word (almost never written).
 * hq_ceiling_mfma: one launch of `iters` rounds of four independent
 * v_mfma_f32_32x32x16_bf16 per wave on register operands, two 256-thread workgroups per CU
 * (two waves per SIMD); *flops receives the launch's flop count.
 * hq_ceiling_mix: one launch of `iters` rounds, one 512-thread workgroup per CU, of
 * mode 0: 20 v_mfma_f32_16x16x32_f16, mode 1: 80 v_pk_fma_f16, mode 2: both (VALU block,
 * then MFMA block) -- time(2) against time(0) + time(1) is how far a SIMD overlaps them. */
int hq_ceiling_read(const void *buf, int64_t bytes, int order, int depth, uint32_t *sink, hq_stream_t stream);
int hq_ceiling_mfma(int64_t iters, float *sink, int64_t *flops, hq_stream_t stream);
int hq_ceiling_mix(int mode, int64_t iters, float *sink, hq_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* HIPQ_H */
