// moe.hip -- MoE grouped expert qmatmul (Light's ops.MoEGemmQ, ops/moe.go:242-265).
//
//   out[p, :] = w(p) * x[row(p), :] @ dequant(W[e(p)])^T   for every routed pair p
//
// with the pairs sorted by expert (MoERouteFromIDs, ops/moe.go:78-99),
// row(p) = rowPerPair ? p : p / topk and w(p) = topkW[p] or 1.
//
//  * Expert segments: offsets[e] = first sorted position with expert >= e, found by
//    a binary search over the sorted expert ids (one thread per expert; no atomics,
//    deterministic); counts[e] = offsets[e+1] - offsets[e].  This fills the counts /
//    offsets scratch Light's launcher computes with an atomic histogram and a serial
//    scan (kernels/cuda/src/moe.cu:28-42).
//  * Q4_K, few pairs per expert (decode): grouped int8-dot GEMV (gemv.hip), up to 4
//    pairs per weight pass.
//  * Q4_K, many pairs per expert (prefill): grouped bf16 MFMA GEMM (gemm.hip) over
//    32-pair chunks.
//  * Other formats / shapes: a generic grouped kernel on F32 activations with the
//    bit-exact block decoder (one wave per weight row).
#include "decode.hpp"
#include "internal.hpp"

#include <algorithm>

namespace hq {

__global__ __launch_bounds__(256) void moe_offsets_kernel(const int64_t *__restrict__ expts, int64_t M, int E,
                                                          int32_t *__restrict__ counts, int32_t *__restrict__ offsets) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e > E) return;
  auto lower = [&](int64_t v) {
    int64_t lo = 0, hi = M;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (expts[mid] < v) lo = mid + 1; else hi = mid;
    }
    return lo;
  };
  const int64_t a = lower(e);
  offsets[e] = (int32_t)a;
  if (e < E) counts[e] = (int32_t)(lower(e + 1) - a);
}

__global__ __launch_bounds__(256) void zero_f32_kernel(float *__restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// The same offsets / counts from one workgroup, for E + 1 offsets that fit in LDS: the sorted
// ids are read once, coalesced (a binary search per expert is a chain of dependent loads),
// and each segment start fills the offsets of the experts up to its own:
// offsets[e] = i for e in (ids[i-1], ids[i]], and M after the last id -- the lower bound of e.
// With zero_out: the rows r < size_m of zero_out (row_len floats each) that no pair of a valid
// expert will write -- pairs routed nowhere, indices the pair list skips -- are zeroed here,
// instead of the whole output before the grouped GEMM.
__global__ __launch_bounds__(1024) void moe_offsets_wg_kernel(const int64_t *__restrict__ expts, int64_t M, int E,
                                                              int32_t *__restrict__ counts,
                                                              int32_t *__restrict__ offsets,
                                                              const int64_t *__restrict__ pairs,
                                                              float *__restrict__ zero_out, int64_t size_m,
                                                              int64_t row_len) {
  extern __shared__ int32_t lo[];
  uint32_t *seen = reinterpret_cast<uint32_t *>(lo + E + 1);  // size_m bits (zero_out only)
  const int t = threadIdx.x, nt = blockDim.x;
  for (int e = t; e <= E; e += nt) lo[e] = (int32_t)M;  // experts past the last id
  if (zero_out)
    for (int64_t w = t; w < (size_m + 31) / 32; w += nt) seen[w] = 0u;
  __syncthreads();
  for (int64_t i = t; i < M; i += nt) {
    const int64_t v = expts[i], p = i > 0 ? expts[i - 1] : -1;
    if (i == 0 || v != p) {
      const int64_t e0 = p + 1 > 0 ? p + 1 : 0, e1 = v < E ? v : E;
      for (int64_t e = e0; e <= e1; e++) lo[e] = (int32_t)i;
    }
    if (zero_out && v >= 0 && v < E) {
      const int64_t r = pairs[i];
      if (r >= 0 && r < size_m) atomicOr(&seen[r >> 5], 1u << (r & 31));
    }
  }
  __syncthreads();
  for (int e = t; e <= E; e += nt) {
    offsets[e] = lo[e];
    if (e < E) counts[e] = lo[e + 1] - lo[e];
  }
  if (zero_out) {
    for (int64_t r = t; r < size_m; r += nt) {  // a row to zero is rare: its thread does it alone
      if (seen[r >> 5] & (1u << (r & 31))) continue;
      for (int64_t c = 0; c < row_len; c++) zero_out[r * row_len + c] = 0.f;
    }
  }
}

// counts / offsets of the sorted expert ids; with zero_out, the rows no valid pair writes are
// zeroed (the one-workgroup kernel when E + 1 offsets and size_m row bits fit in LDS, else a
// whole-output zero first).
static int moe_offsets(const int64_t *expts, int64_t M, int64_t E, int32_t *counts, int32_t *offsets,
                       const int64_t *pairs, float *zero_out, int64_t size_m, int64_t row_len, hipStream_t s) {
  const int64_t lds = 4 * (E + 1) + (zero_out ? 4 * ((size_m + 31) / 32) : 0);
  if (lds <= 64 * 1024) {
    moe_offsets_wg_kernel<<<1, 1024, (size_t)lds, s>>>(expts, M, (int)E, counts, offsets, pairs, zero_out, size_m,
                                                      row_len);
    return check_launch("moe_offsets");
  }
  if (zero_out) {
    zero_f32_kernel<<<(unsigned)cdiv(size_m * row_len, 256), 256, 0, s>>>(zero_out, size_m * row_len);
    if (int rc = check_launch("zero")) return rc;
  }
  moe_offsets_kernel<<<(unsigned)cdiv(E + 1, 256), 256, 0, s>>>(expts, M, (int)E, counts, offsets);
  return check_launch("moe_offsets");
}

template <int DT>
__global__ __launch_bounds__(256) void moe_generic_kernel(const float *__restrict__ x, const uint8_t *__restrict__ w,
                                                          const int64_t *__restrict__ pairs,
                                                          const int32_t *__restrict__ offsets,
                                                          const float *__restrict__ topk_w, float *__restrict__ out,
                                                          int64_t size_m, int64_t N, int64_t K, int topk, int rpp) {
  const int e = blockIdx.y;
  const int seg0 = offsets[e], seg1 = offsets[e + 1];
  if (seg0 >= seg1) return;
  const BlockInfo bi = block_info(DT);
  const int64_t row_bytes = K / bi.elems * bi.bytes;
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  for (int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); n < N; n += nwaves) {
    const uint8_t *rp = w + ((int64_t)e * N + n) * row_bytes;
    for (int i = seg0; i < seg1; i++) {
      const int64_t p = pairs[i];
      if (p < 0 || p >= size_m) continue;
      const float *xr = x + (rpp ? p : p / topk) * K;
      float acc = 0.f;
      for (int64_t t = lane; t < K / 8; t += 64) {
        float y[8];
        decode8<DT>(rp, t, y);
#pragma unroll
        for (int j = 0; j < 8; j++) acc += y[j] * xr[8 * t + j];
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
      if (lane == 0) out[p * N + n] = acc * (topk_w ? topk_w[p] : 1.f);
    }
  }
}

// MoECombine (ops/moe.go:209-240): out[t, n] = ((p[t*topk] + p[t*topk+1]) + ...) in slot
// order, the order of Light's chain of Add ops, so F32 results are bit-identical.
__global__ __launch_bounds__(256) void moe_combine_kernel(const float *__restrict__ pair, float *__restrict__ out,
                                                          int64_t T, int64_t N, int topk) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * N) return;
  const int64_t t = i / N, n = i - t * N;
  const float *p = pair + t * topk * N + n;
  float acc = p[0];
  for (int s = 1; s < topk; s++) acc = __fadd_rn(acc, p[(int64_t)s * N]);
  out[i] = acc;
}

int launch_moe_combine(const float *pair, float *out, int64_t T, int64_t N, int topk, hipStream_t s) {
  moe_combine_kernel<<<(unsigned)cdiv(T * N, 256), 256, 0, s>>>(pair, out, T, N, topk);
  return check_launch("moe_combine");
}

static bool moe_q4k_fast(int dt, int64_t K, const void *w) {
  return dt == Q4_K && ((uintptr_t)w & 15) == 0 && K / 256 <= 128;
}

static bool moe_use_mfma(int64_t M, int64_t E) { return M > 4 * E; }

static int64_t al256m(int64_t b);

size_t moe_ws_bytes(int64_t rows, int64_t K, int dt) {
  if (rows <= 0 || K <= 0 || K % 32) return 0;
  // Q4_K: the decode path's act layout of x, or the grouped GEMM's f16 x and row scales.
  return dt == Q4_K ? (size_t)std::max<int64_t>(act_bytes(rows, K), al256m(2 * rows * K) + 4 * rows) : 0;
}

// zero_out (nullable; = out): rows of out that no valid pair writes are zeroed on the way.
// routed: pairs / expts / counts / offsets come from MoERoute over exactly the pairs [0, M)
// with size_m == M (every pair in one valid expert segment, counts / offsets already written),
// so the grouped GEMM writes every row: no offsets pass, nothing to zero.
int launch_moe_q(const float *x, const void *w, const int64_t *pairs, const int64_t *expts, int32_t *counts,
                 int32_t *offsets, const float *topk_w, float *out, int topk, int64_t size_m, int64_t M, int64_t rows,
                 int64_t E, int64_t N, int64_t K, int rpp, int dt, void *ws, hipStream_t s, float *zero_out,
                 bool routed) {
  if (routed && size_m != M) return fail(HQ_EINVAL, "moe_gemm_q", "routed pairs need size_m == M");
  if (E > INT32_MAX - 1 || M > INT32_MAX || N > INT32_MAX) return fail(HQ_EUNSUPPORTED, "moe_gemm_q", "too large");
  // Decode: one launch finds the segments, writes counts / offsets, quantizes x and streams.
  // (Q5_K takes it at every M: it has no grouped MFMA kernel.)
  if (M > 0 && E <= 65535 && (dt == Q5_K || !moe_use_mfma(M, E)) && moe_x_ok(K, dt, w, x)) {
    if (zero_out && !routed) {
      zero_f32_kernel<<<(unsigned)cdiv(size_m * N, 256), 256, 0, s>>>(zero_out, size_m * N);
      if (int rc = check_launch("zero")) return rc;
    }
    return launch_moe_gemv_x(x, w, pairs, expts, counts, offsets, topk_w, out, topk, size_m, M, rows, E, N, K, rpp,
                             dt, -1, s);
  }
  if (!routed)
    if (int rc = moe_offsets(expts, M, E, counts, offsets, pairs, zero_out, size_m, N, s)) return rc;
  if (moe_q4k_fast(dt, K, w)) {
    if (moe_use_mfma(M, E)) {
      auto *xh = static_cast<uint16_t *>(ws);
      auto *xs = reinterpret_cast<float *>(static_cast<char *>(ws) + al256m(2 * rows * K));
      return launch_moe_gemm_q4k(x, xh, xs, w, pairs, offsets, topk_w, out, topk, size_m, rows, E, N, K, rpp, s);
    }
    if (int rc = launch_quantize_act(x, F32, ws, rows, K, s)) return rc;
    return launch_moe_gemv_q4k(ws, w, pairs, offsets, topk_w, out, topk, size_m, M, rows, E, N, K, rpp, s);
  }
  const int64_t active = M < E ? M : E;
  const int64_t cap = cdiv((int64_t)device_cus() * 8, active > 0 ? active : 1);
  const int64_t wgs = cdiv(N, 4);
  dim3 grid((unsigned)(wgs < cap ? wgs : cap), (unsigned)E);
  auto *wb = static_cast<const uint8_t *>(w);
  switch (dt) {
    case Q4_K: moe_generic_kernel<Q4_K><<<grid, 256, 0, s>>>(x, wb, pairs, offsets, topk_w, out, size_m, N, K, topk, rpp); break;
    case Q8_0: moe_generic_kernel<Q8_0><<<grid, 256, 0, s>>>(x, wb, pairs, offsets, topk_w, out, size_m, N, K, topk, rpp); break;
    case Q4_0: moe_generic_kernel<Q4_0><<<grid, 256, 0, s>>>(x, wb, pairs, offsets, topk_w, out, size_m, N, K, topk, rpp); break;
    case Q5_0: moe_generic_kernel<Q5_0><<<grid, 256, 0, s>>>(x, wb, pairs, offsets, topk_w, out, size_m, N, K, topk, rpp); break;
    case Q5_K: moe_generic_kernel<Q5_K><<<grid, 256, 0, s>>>(x, wb, pairs, offsets, topk_w, out, size_m, N, K, topk, rpp); break;
    case Q6_K: moe_generic_kernel<Q6_K><<<grid, 256, 0, s>>>(x, wb, pairs, offsets, topk_w, out, size_m, N, K, topk, rpp); break;
    default: return fail(HQ_EUNSUPPORTED, "moe_gemm_q", "dtype %d", dt);
  }
  return check_launch("moe_generic");
}

// Gated gate/up (the SwiGLU / GeGLU of nn.SparseMoE.runExperts, nn/moe.go:196-236):
// h[p, n] = act(x_row(p) . Wgu[e(p)][n]) * (x_row(p) . Wgu[e(p)][I + n]) for n < I.  Decode
// shapes run one fused launch; otherwise moe_gemm_q into the workspace (size_m, 2I), then an
// epilogue over its two halves.
__global__ __launch_bounds__(256) void moe_gated_split_kernel(const float *__restrict__ gu, float *__restrict__ out,
                                                              int64_t rows, int64_t I, int act) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * I) return;
  const int64_t r = i / I, n = i - r * I;
  out[i] = gate_act(gu[r * 2 * I + n], act) * gu[r * 2 * I + I + n];
}


static int64_t al256m(int64_t b) { return (b + 255) & ~(int64_t)255; }

size_t moe_gated_ws_bytes(int64_t size_m, int64_t rows, int64_t I, int64_t K, int dt) {
  return (size_t)al256m(4 * size_m * 2 * I) + moe_ws_bytes(rows, K, dt);
}

int launch_moe_q_gated(const float *x, const void *w, const int64_t *pairs, const int64_t *expts, int32_t *counts,
                       int32_t *offsets, float *out, int topk, int64_t size_m, int64_t M, int64_t rows, int64_t E,
                       int64_t I, int64_t K, int rpp, int dt, int act, void *ws, hipStream_t s, bool routed,
                       bool x_ready) {
  if (E > INT32_MAX - 1 || M > INT32_MAX || 2 * I > INT32_MAX)
    return fail(HQ_EUNSUPPORTED, "moe_gemm_q_gated", "too large");
  if (routed && size_m != M) return fail(HQ_EINVAL, "moe_gemm_q_gated", "routed pairs need size_m == M");
  if (M > 0 && E <= 65535 && (dt == Q5_K || !moe_use_mfma(M, E)) && moe_x_ok(K, dt, w, x))
    return launch_moe_gemv_x(x, w, pairs, expts, counts, offsets, nullptr, out, topk, size_m, M, rows, E, I, K, rpp,
                             dt, act, s);
  if (moe_q4k_fast(dt, K, w) && moe_use_mfma(M, E)) {
    // The grouped GEMM with the gated epilogue: h straight from the gate / up tiles.  Rows of
    // pairs outside every expert segment stay zero, as after the split of a zeroed output.
    void *inner = static_cast<char *>(ws) + al256m(4 * size_m * 2 * I);
    if (!routed)
      if (int rc = moe_offsets(expts, M, E, counts, offsets, pairs, out, size_m, I, s)) return rc;
    auto *xh = static_cast<uint16_t *>(inner);
    auto *xs = reinterpret_cast<float *>(static_cast<char *>(inner) + al256m(2 * rows * K));
    return launch_moe_gemm_q4k(x, xh, xs, w, pairs, offsets, nullptr, out, topk, size_m, rows, E, 2 * I, K, rpp, s, I,
                               act, x_ready);
  }
  float *gu = static_cast<float *>(ws);
  void *inner = static_cast<char *>(ws) + al256m(4 * size_m * 2 * I);
  zero_f32_kernel<<<(unsigned)cdiv(size_m * 2 * I, 256), 256, 0, s>>>(gu, size_m * 2 * I);
  if (int rc = check_launch("zero")) return rc;
  if (int rc = launch_moe_q(x, w, pairs, expts, counts, offsets, nullptr, gu, topk, size_m, M, rows, E, 2 * I, K, rpp,
                            dt, inner, s))
    return rc;
  moe_gated_split_kernel<<<(unsigned)cdiv(size_m * I, 256), 256, 0, s>>>(gu, out, size_m, I, act);
  return check_launch("moe_gated_split");
}

// Workspace of the unfused down + combine: the pair rows (M, N) F32, the counts / offsets
// scratch when the caller passes none, then moe_gemm_q's own workspace.
size_t moe_combine_ws_bytes(int64_t M, int64_t E, int64_t N, int64_t K, int dt) {
  return (size_t)al256m(4 * M * N) + (size_t)al256m(4 * (2 * E + 1)) + moe_ws_bytes(M, K, dt);
}

// Down projection + MoECombine: y (T, N) = combine(moe_gemm_q(h, w, routing, topk_w)).  Decode
// shapes whose moe_gemm_q would run the one-launch grouped GEMV take the fused token-major
// kernel (bit-identical to that GEMV + moe_combine); otherwise moe_gemm_q runs into the
// zeroed workspace and moe_combine follows.
int launch_moe_q_combine(const float *h, const void *w, const int64_t *pairs, const int64_t *expts, int32_t *counts,
                         int32_t *offsets, const float *topk_w, float *y, int topk, int64_t T, int64_t E, int64_t N,
                         int64_t K, int dt, void *ws, hipStream_t s, bool routed) {
  const int64_t M = T * topk;
  if (E > INT32_MAX - 1 || M > INT32_MAX || N > INT32_MAX)
    return fail(HQ_EUNSUPPORTED, "moe_gemm_q_combine", "too large");
  if (E <= 65535 && (dt == Q5_K || !moe_use_mfma(M, E)) && moe_x_ok(K, dt, w, h) &&
      moe_comb_ok(M, T, topk, K, dt, w, h))
    return launch_moe_down_combine(h, w, pairs, expts, counts, offsets, topk_w, y, topk, T, E, N, K, dt, s);
  float *po = static_cast<float *>(ws);
  auto *co = reinterpret_cast<int32_t *>(static_cast<char *>(ws) + al256m(4 * M * N));
  void *inner = static_cast<char *>(ws) + al256m(4 * M * N) + al256m(4 * (2 * E + 1));
  // moe_gemm_q writes counts / offsets; without caller buffers they go to the workspace (and
  // are not the route's: the offsets pass runs).
  const bool caller_counts = counts && offsets;
  if (!counts || !offsets) {
    counts = co;
    offsets = co + E;
  }
  // The rows no valid pair writes are zeroed by launch_moe_q (zero_out = po), as Light's
  // zeroed pair output would hold them.
  if (int rc = launch_moe_q(h, w, pairs, expts, counts, offsets, topk_w, po, topk, M, M, M, E, N, K, 1, dt, inner, s,
                            po, routed && caller_counts))
    return rc;
  return launch_moe_combine(po, y, T, N, topk, s);
}

size_t moe_route_gated_ws_bytes(int64_t T, int topk, int64_t E, int64_t I, int64_t K, int dt) {
  return (size_t)al256m(4 * (2 * E + 1)) + moe_gated_ws_bytes(T * topk, T, I, K, dt);
}

// MoERoute, then the routed gated gate/up (h per pair, row(p) = p / topk).  Decode shapes run
// both in one launch (bit-identical to moe_route + moe_gemm_q_gated); otherwise the two run
// in sequence, with counts / offsets in the workspace when the caller passes none.
int launch_moe_route_gated_any(const float *probs, const float *x, const void *w, float *h, int64_t T, int64_t E,
                               int topk, int normalize, int64_t I, int64_t K, int dt, int act, int64_t *topk_ids,
                               float *weights, int64_t *sorted_pairs, int64_t *sorted_expts, int32_t *counts,
                               int32_t *offsets, void *ws, hipStream_t s) {
  if (moe_route_gated_ok(T, E, topk, K, dt, w, x))
    return launch_moe_route_gated(probs, x, w, h, T, E, topk, normalize, I, K, dt, act, topk_ids, weights,
                                  sorted_pairs, sorted_expts, counts, offsets, s);
  auto *co = static_cast<int32_t *>(ws);
  void *inner = static_cast<char *>(ws) + al256m(4 * (2 * E + 1));
  if (!counts || !offsets) {
    counts = co;
    offsets = co + E;
  }
  const int64_t M = T * topk;
  // The grouped-GEMM path converts x to f16 rows first: the routing launch does that on the
  // way (one wave per token), into the places launch_moe_q_gated's grouped GEMM reads.
  const bool fuse_x = moe_q4k_fast(dt, K, w) && moe_use_mfma(M, E) && ((uintptr_t)x & 15) == 0;
  char *gemm_ws = static_cast<char *>(inner) + al256m(4 * M * 2 * I);
  auto *xh = reinterpret_cast<uint16_t *>(gemm_ws);
  auto *xs = reinterpret_cast<float *>(gemm_ws + al256m(2 * T * K));
  if (int rc = launch_moe_route(probs, T, E, topk, normalize, topk_ids, weights, sorted_pairs, sorted_expts, counts,
                                offsets, s, fuse_x ? x : nullptr, K, xh, xs))
    return rc;
  return launch_moe_q_gated(x, w, sorted_pairs, sorted_expts, counts, offsets, h, topk, M, M, T, E, I, K, 0, dt, act,
                            inner, s, /*routed=*/true, fuse_x);
}

// The two halves share the workspace (they do not overlap in time), followed by the counts /
// offsets of the routing when the caller passes none: written by the route, read by both.
size_t moe_block_ws_bytes(int64_t T, int topk, int64_t E, int64_t H, int64_t I, int dt) {
  return std::max(moe_route_gated_ws_bytes(T, topk, E, I, H, dt), moe_combine_ws_bytes(T * topk, E, H, I, dt)) +
         (size_t)al256m(4 * (2 * E + 1));
}

// The SparseMoE decode block: MoERoute, the routed gated gate/up into h, then the down
// projection with MoECombine into y.  One launch for a single token where it applies
// (launch_moe_block); otherwise the route-gated launch and the combine path in sequence, on
// the same workspace (the two do not overlap in time).  Bit-identical either way.
int launch_moe_block_any(const float *probs, const float *x, const void *wgu, const void *wdn, float *h, float *y,
                         int64_t T, int64_t E, int topk, int normalize, int64_t H, int64_t I, int dt, int act,
                         int64_t *topk_ids, float *weights, int64_t *sorted_pairs, int64_t *sorted_expts,
                         int32_t *counts, int32_t *offsets, void *ws, hipStream_t s) {
  // The one-launch kernels use the front of the workspace for h's act blocks (act_bytes(topk, I),
  // well inside the two-launch path's share).
  uint8_t *hact = moe_block_ws_bytes(T, topk, E, H, I, dt) >= (size_t)act_bytes(T * topk, I) + 256
                      ? static_cast<uint8_t *>(ws) : nullptr;
  const int rc = launch_moe_block(probs, x, wgu, wdn, h, y, T, E, topk, normalize, H, I, dt, act, topk_ids, weights,
                                  sorted_pairs, sorted_expts, counts, offsets, hact, s);
  if (rc != 1) return rc;
  if (!counts || !offsets) {
    const size_t tail = std::max(moe_route_gated_ws_bytes(T, topk, E, I, H, dt), moe_combine_ws_bytes(T * topk, E, H, I, dt));
    counts = reinterpret_cast<int32_t *>(static_cast<char *>(ws) + tail);
    offsets = counts + E;
  }
  if (int r = launch_moe_route_gated_any(probs, x, wgu, h, T, E, topk, normalize, I, H, dt, act, topk_ids, weights,
                                         sorted_pairs, sorted_expts, counts, offsets, ws, s))
    return r;
  // The route wrote counts / offsets for exactly the pairs [0, T topk): the down projection
  // needs no offsets pass and no zeroing.
  return launch_moe_q_combine(h, wdn, sorted_pairs, sorted_expts, counts, offsets, weights, y, topk, T, E, H, I, dt,
                              ws, s, /*routed=*/true);
}

}  // namespace hq
