// moe_route.hip -- on-device MoERoute (ops/moe.go:29-71) and the expert sort of
// MoERouteFromIDs (ops/moe.go:78-99).
//
// MoERoute(probs (T, E) F32, topk, normalize):
//   * TopK(probs, topk, largest): Light's CPU kernel is a stable descending sort of each
//     row (kernels/cpu/topk.go:52-68), so equal values keep index order: the selection
//     here takes the largest value, the lowest index among equals.
//   * normalize: den = Sum(vals, axis 1) -- a left-to-right f32 sum from 0
//     (kernels/cpu/reduce.go:76-87) -- then vals / den (IEEE division).
//   * Sort(flat ids, ascending) is sort.SliceStable (kernels/cpu/shape_ops.go:156-184):
//     pairs of one expert keep pair order.  The sort here is a counting sort that keeps
//     that order, and it also produces MoEGemmQ's counts / offsets scratch
//     (kernels/cuda/src/moe.cu:28-42) in the same pass.
//
// Layout of the sort (one 1024-thread workgroup): pairs are taken 64 at a time (a "chunk",
// one wave).  Within a chunk, lanes with equal ids are found by ballots over the id bits,
// giving each pair its rank among equal ids of lower lanes.  Per-chunk counts [W][E] (u16
// in LDS) are turned into exclusive offsets along the chunk axis per expert, the expert
// totals are scanned, and every pair lands at base[e] + chunk offset + rank.
#include <atomic>

#include "internal.hpp"
#include "route.hpp"

namespace hq {

namespace {

constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / 64;
constexpr int kTopkVpl = 16;  // values per lane: E <= 1024

struct RouteArgs {
  const float *probs;      // (T, E), or nullptr when ids come in
  const int64_t *ids_in;   // (M) expert per pair (sort only)
  int64_t *topk_ids;       // (T, topk) out
  float *weights;          // (M) out
  int64_t *sorted_pairs, *sorted_expts;
  int32_t *counts, *offsets;  // nullable
  int T, E, topk, normalize, M, W;
  // Optional: x (T, K) F32 rows converted to f16 (xh) with their power-of-two scales (xs).
  const float *x;
  _Float16 *xh;
  float *xs;
  int64_t K;
};

// Row t of x to f16 divided by 2^e (e = 0 unless max |x| >= 2^15; then e brings the row's
// maximum below 2^15) and xs[t] = 2^e, by one wave: what to_f16_rowscale_kernel writes for
// the row, bit for bit (the same maximum, exponent and conversion).  K % 4 == 0, x 16-byte
// aligned.  K <= 4096: the row is read once, into registers.
__device__ void rowscale_wave(const RouteArgs &a, int t, int lane) {
  const float4 *xr = reinterpret_cast<const float4 *>(a.x + (int64_t)t * a.K);
  const int64_t n4 = a.K / 4;
  typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
  f16x4 *yr = reinterpret_cast<f16x4 *>(a.xh + (int64_t)t * a.K);
  auto amax = [](const float4 v) { return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); };
  auto scale = [](float m) {
    int ex = 0;
    (void)frexpf(m, &ex);  // m < 2^ex
    return ex > 15 && m == m && m < INFINITY ? ex - 15 : 0;
  };
  auto cvt = [](const float4 v, int e) {
    return f16x4{(_Float16)ldexpf(v.x, -e), (_Float16)ldexpf(v.y, -e), (_Float16)ldexpf(v.z, -e),
                 (_Float16)ldexpf(v.w, -e)};
  };
  constexpr int R = 16;  // float4 per lane held in registers
  float m = 0.f;
  if (n4 <= 64 * R) {
    float4 v[R];
#pragma unroll
    for (int j = 0; j < R; j++) {
      const int64_t i = lane + 64 * j;
      v[j] = i < n4 ? xr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int j = 0; j < R; j++) m = fmaxf(m, amax(v[j]));
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    const int e = scale(m);
#pragma unroll
    for (int j = 0; j < R; j++) {
      const int64_t i = lane + 64 * j;
      if (i < n4) yr[i] = cvt(v[j], e);
    }
    if (lane == 0) a.xs[t] = ldexpf(1.f, e);
    return;
  }
  for (int64_t i = lane; i < n4; i += 64) m = fmaxf(m, amax(xr[i]));
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  const int e = scale(m);
  for (int64_t i = lane; i < n4; i += 64) yr[i] = cvt(xr[i], e);
  if (lane == 0) a.xs[t] = ldexpf(1.f, e);
}

// Top-k of token t by one wave, renormalised if asked; writes topk_ids and weights.
template <int VPL>
__device__ void route_token_v(const RouteArgs &a, int t, int lane, uint16_t *lid) {
  float sv, den;
  int si;
  topk_row<VPL>(a.probs + (int64_t)t * a.E, a.E, a.topk, lane, sv, si, den);
  const float w = a.normalize ? __fdiv_rn(sv, den) : sv;
  if (lane < a.topk) {
    const int64_t p = (int64_t)t * a.topk + lane;
    a.topk_ids[p] = si;
    a.weights[p] = w;
    if (lid) lid[p] = (uint16_t)si;
  }
}

__device__ __forceinline__ void route_token(const RouteArgs &a, int t, int lane, uint16_t *lid) {
  if (a.E <= 64)
    route_token_v<1>(a, t, lane, lid);
  else if (a.E <= 128)
    route_token_v<2>(a, t, lane, lid);
  else if (a.E <= 256)
    route_token_v<4>(a, t, lane, lid);
  else if (a.E <= 512)
    route_token_v<8>(a, t, lane, lid);
  else
    route_token_v<16>(a, t, lane, lid);
}


// Mask of lanes holding the same id as this lane (among valid lanes).
__device__ __forceinline__ uint64_t match_id(int id, bool valid, int nbits) {
  uint64_t m = __ballot(valid);
  for (int b = 0; b < nbits; b++) {
    const bool bit = (id >> b) & 1;
    const uint64_t bb = __ballot(bit);
    m &= bit ? bb : ~bb;
  }
  return valid ? m : 0;
}

template <bool TOPK>
__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(RouteArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int nthr = blockDim.x, nwav = nthr >> 6;
  uint16_t *lid = reinterpret_cast<uint16_t *>(smem);                                   // [M]
  uint16_t *wcnt = lid + ((a.M + 7) & ~7);                                              // [W][E]
  uint32_t *base = reinterpret_cast<uint32_t *>(wcnt + (((int64_t)a.W * a.E + 7) & ~7));  // [E]

  for (int64_t i = t; i < (int64_t)a.W * a.E; i += nthr) wcnt[i] = 0;
  if constexpr (TOPK) {
    for (int tok = wave; tok < a.T; tok += nwav) {
      route_token(a, tok, lane, lid);
      if (a.x) rowscale_wave(a, tok, lane);
    }
  } else {
    for (int p = t; p < a.M; p += nthr) {
      int64_t id = a.ids_in[p];
      id = id < 0 ? 0 : (id >= a.E ? a.E - 1 : id);  // ids are in [0, E); clamped for memory safety
      lid[p] = (uint16_t)id;
    }
  }
  __syncthreads();

  int nbits = 1;
  while ((1 << nbits) < a.E) nbits++;
  const uint64_t lt = (1ull << lane) - 1;
  // Phase A: per-chunk counts.
  for (int w = wave; w < a.W; w += nwav) {
    const int p = 64 * w + lane;
    const bool valid = p < a.M;
    const int id = valid ? lid[p] : 0;
    const uint64_t m = match_id(id, valid, nbits);
    if (valid && __popcll(m & lt) == 0) wcnt[w * a.E + id] = (uint16_t)__popcll(m);
  }
  __syncthreads();
  // Phase B: per expert, chunk counts -> exclusive offsets; totals into base.
  for (int e = t; e < a.E; e += nthr) {
    uint32_t run = 0;
    for (int w = 0; w < a.W; w++) {
      const uint32_t c = wcnt[w * a.E + e];
      wcnt[w * a.E + e] = (uint16_t)run;
      run += c;
    }
    base[e] = run;
  }
  __syncthreads();
  // Exclusive scan of the totals by wave 0 (lane l owns a run of consecutive experts).
  if (wave == 0) {
    const int per = (a.E + 63) / 64, e0 = lane * per, e1 = e0 + per < a.E ? e0 + per : a.E;
    uint32_t s = 0;
    for (int e = e0; e < e1; e++) s += base[e];
    uint32_t incl = s;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t o = __shfl_up(incl, off);
      if (lane >= off) incl += o;
    }
    uint32_t run = incl - s;
    for (int e = e0; e < e1; e++) {
      const uint32_t c = base[e];
      if (a.counts) a.counts[e] = (int32_t)c;
      if (a.offsets) a.offsets[e] = (int32_t)run;
      base[e] = run;
      run += c;
    }
    if (lane == 0 && a.offsets) a.offsets[a.E] = a.M;
  }
  __syncthreads();
  // Phase C: placement.
  for (int w = wave; w < a.W; w += nwav) {
    const int p = 64 * w + lane;
    const bool valid = p < a.M;
    const int id = valid ? lid[p] : 0;
    const uint64_t m = match_id(id, valid, nbits);
    if (valid) {
      const uint32_t pos = base[id] + wcnt[w * a.E + id] + (uint32_t)__popcll(m & lt);
      a.sorted_pairs[pos] = p;
      a.sorted_expts[pos] = id;
    }
  }
}

// Top-k for many tokens: one wave per token, blockDim / 64 tokens per workgroup.
__global__ __launch_bounds__(512) void moe_topk_kernel(RouteArgs a) {
  const int tok = blockIdx.x * (int)(blockDim.x >> 6) + (int)(threadIdx.x >> 6);
  if (tok < a.T) {
    route_token(a, tok, threadIdx.x & 63, nullptr);
    if (a.x) rowscale_wave(a, tok, threadIdx.x & 63);
  }
}

size_t route_lds(int64_t M, int64_t E) {
  const int64_t W = (M + 63) / 64;
  return (size_t)(2 * ((M + 7) & ~7) + 2 * ((W * E + 7) & ~7) + 4 * E);
}

int run_route(bool topk, const RouteArgs &a, hipStream_t s) {
  const size_t lds = route_lds(a.M, a.E);
  auto *kern = topk ? &moe_route_kernel<true> : &moe_route_kernel<false>;
  static std::atomic<bool> attr_done[2] = {false, false};  // (idempotent: racing callers both set it)
  if (lds > 64 * 1024 && !attr_done[topk].load(std::memory_order_acquire)) {
    if (int rc = check(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024),
                       "hipFuncSetAttribute"))
      return rc;
    attr_done[topk].store(true, std::memory_order_release);
  }
  // One wave per chunk of 64 pairs (and per token for the top-k), up to 16 waves.
  int64_t waves = a.W > a.T ? a.W : a.T;
  waves = waves < 1 ? 1 : (waves > kRouteWaves ? kRouteWaves : waves);
  kern<<<1, (unsigned)(64 * waves), lds, s>>>(a);
  return check_launch("moe_route");
}

}  // namespace

bool moe_route_fits(int64_t M, int64_t E) {
  return M >= 1 && M <= 65535 && E >= 1 && E <= 64 * kTopkVpl && route_lds(M, E) <= 160 * 1024;
}

int launch_moe_route(const float *probs, int64_t T, int64_t E, int topk, int normalize, int64_t *topk_ids,
                     float *weights, int64_t *sorted_pairs, int64_t *sorted_expts, int32_t *counts, int32_t *offsets,
                     hipStream_t s, const float *x_f32, int64_t K, uint16_t *xh, float *xs) {
  RouteArgs a = {};
  a.probs = probs;
  a.x = x_f32;
  a.xh = reinterpret_cast<_Float16 *>(xh);
  a.xs = xs;
  a.K = K;
  a.topk_ids = topk_ids;
  a.weights = weights;
  a.sorted_pairs = sorted_pairs;
  a.sorted_expts = sorted_expts;
  a.counts = counts;
  a.offsets = offsets;
  a.T = (int)T;
  a.E = (int)E;
  a.topk = topk;
  a.normalize = normalize;
  a.M = (int)(T * topk);
  a.W = (a.M + 63) / 64;
  // Few tokens: top-k and sort in one workgroup; otherwise top-k over the grid first.
  if (T <= 4 * kRouteWaves) return run_route(true, a, s);
  // Converting x too: one token per workgroup, so the rows spread over the CUs.
  const int tpw = a.x ? 1 : 8;
  moe_topk_kernel<<<(unsigned)cdiv(T, tpw), 64 * tpw, 0, s>>>(a);
  if (int rc = check_launch("moe_topk")) return rc;
  a.ids_in = topk_ids;
  return run_route(false, a, s);
}

int launch_moe_sort_ids(const int64_t *ids, int64_t M, int64_t E, int64_t *sorted_pairs, int64_t *sorted_expts,
                        int32_t *counts, int32_t *offsets, hipStream_t s) {
  RouteArgs a = {};
  a.ids_in = ids;
  a.sorted_pairs = sorted_pairs;
  a.sorted_expts = sorted_expts;
  a.counts = counts;
  a.offsets = offsets;
  a.E = (int)E;
  a.M = (int)M;
  a.W = (a.M + 63) / 64;
  return run_route(false, a, s);
}

}  // namespace hq
