// ops.cpp -- MatMulQ, MatMulInt4, DequantizeInt4, MoERouteFromIDs, MoEGemmQ, MoECombine,
// Dequantize: validation, output allocation and registry dispatch as in Light's ops package.
#include "ops.hpp"

#include <algorithm>
#include <numeric>

#include "../../include/hipq.h"
#include "registry.hpp"

namespace light {
namespace ops {

static bool same_device(const Tensor &a, const Tensor &b) { return a.device().SameAs(b.device()); }

// ---- MatMulQ (ops/matmul_q.go:27-76) ----

Tensor MatMulQ(const Tensor &x, const Tensor &w) {
  if (x.Rank() != 2 || w.Rank() != 2)
    Fail("MatMulQ: want x (M,K) and w (N,K); got %s, %s", x.ShapeStr().c_str(), w.ShapeStr().c_str());
  if (x.dtype() != DType::F32) Fail("MatMulQ: x must be F32, got %s", DTypeName(x.dtype()));
  if (!IsQuantized(w.dtype())) Fail("MatMulQ: w must be a quantized dtype, got %s", DTypeName(w.dtype()));
  if (!same_device(x, w)) Fail("MatMulQ: x on %s, w on %s", x.device().str().c_str(), w.device().str().c_str());
  const int64_t M = x.Dim(0), K = x.Dim(1), N = w.Dim(0);
  if (w.Dim(1) != K) Fail("MatMulQ: inner dim mismatch (x K=%lld, w K=%lld)", (long long)K, (long long)w.Dim(1));
  if (K % BlockElems(w.dtype()))
    Fail("MatMulQ: K=%lld not a multiple of %s block size %d", (long long)K, DTypeName(w.dtype()),
         BlockElems(w.dtype()));
  // ensureContig (:48-51) is the identity here: this layer's tensors are always dense
  // row-major (Tensor has no strides).  Light's CUDA-only M >= MatMulQDequantMinRows
  // fallback (:52-59) does not apply: the ROCm kernel serves every M (GEMV for decode, MFMA
  // GEMM for prefill).  A dtype with no fused kernel takes matMulQFallback (:61-71).
  Kernel k;
  try {
    k = Lookup(Key{"matmul_q", x.device().kind, w.dtype()});
  } catch (const Error &e) {
    if (!e.IsKernelNotFound()) throw;
    return MatMulQFallback(x, w);
  }
  Tensor out = Tensor::Empty(DType::F32, {M, N}, x.device());
  Context ctx;
  ctx.inputs = {x, w};
  ctx.output = out;
  k(ctx);
  return out;
}

// matMulQFallback (ops/matmul_q.go:85-95): quant.Dequantize, then the ordinary F32 matmul
// out = x . wf^T through the registry's "matmul" key.  This library registers neither a
// dequant for the formats without a fused kernel nor an F32 matmul, so on ROCm the
// fallback ends in the registry's kernel-not-found error, as Light's does on a device
// whose backend lacks those kernels.
Tensor MatMulQFallback(const Tensor &x, const Tensor &w) {
  Tensor wf = Dequantize(w);
  Kernel mm = Lookup(Key{"matmul", x.device().kind, DType::F32});
  Tensor out = Tensor::Empty(DType::F32, {x.Dim(0), w.Dim(0)}, x.device());
  Context ctx;
  ctx.inputs = {x, wf};
  ctx.output = out;
  ctx.attrs = {{"transpose_b", Attr::Bool(true)}};
  mm(ctx);
  return out;
}

Tensor MatMulQGated(const Tensor &x, const Tensor &wg, const Tensor &wu, bool gelu) {
  if (x.Rank() != 2 || x.dtype() != DType::F32)
    Fail("MatMulQGated: x must be (M, K) F32, got %s %s", DTypeName(x.dtype()), x.ShapeStr().c_str());
  const int64_t M = x.Dim(0), K = x.Dim(1);
  for (const Tensor *w : {&wg, &wu}) {
    if (w->Rank() != 2 || w->Dim(1) != K || w->Dim(0) != wg.Dim(0) || w->dtype() != wg.dtype() ||
        !IsQuantized(w->dtype()) || !same_device(*w, x))
      Fail("MatMulQGated: weights must be (N, %lld) %s on %s, got %s / %s", (long long)K, DTypeName(wg.dtype()),
           x.device().str().c_str(), wg.ShapeStr().c_str(), wu.ShapeStr().c_str());
  }
  if (K % BlockElems(wg.dtype()))
    Fail("MatMulQGated: K=%lld not a multiple of %s block size %d", (long long)K, DTypeName(wg.dtype()),
         BlockElems(wg.dtype()));
  Kernel k = Lookup(Key{"matmul_q_gated", x.device().kind, wg.dtype()});
  Tensor out = Tensor::Empty(DType::F32, {M, wg.Dim(0)}, x.device());
  Context ctx;
  ctx.inputs = {x, wg, wu};
  ctx.output = out;
  ctx.attrs = {{"gelu", Attr::Bool(gelu)}};
  k(ctx);
  return out;
}

bool MatMulQFusedOn(DeviceKind kind, DType dt) {
  try {
    Lookup(Key{"matmul_q", kind, dt});
    return true;
  } catch (const Error &e) {
    if (e.IsKernelNotFound()) return false;
    throw;
  }
}

// ---- int4 (ops/int4.go) ----

static void dequantize_int4_at(const Int4 &w, const Tensor &out, int64_t off) {
  if (w.group <= 0 || w.K() % w.group)
    Fail("ops.DequantizeInt4: group %d does not divide K %lld", w.group, (long long)w.K());
  Kernel k = Lookup(Key{"int4_dequant", w.codes.device().kind, out.dtype()});
  Context ctx;
  ctx.inputs = {w.codes, w.scales, w.zeros};
  ctx.output = out;
  ctx.attrs = {{"group", Attr::Int(w.group)}, {"offset", Attr::Int(off)}};
  k(ctx);
}

Tensor DequantizeInt4(const Int4 &w, DType out_dt) {
  Tensor out = Tensor::Zeros(out_dt, {w.N(), w.K()}, w.codes.device());
  dequantize_int4_at(w, out, 0);
  return out;
}

constexpr int64_t kInt4GEMVMaxM = 8;  // ops/int4.go:58-59

Tensor MatMulInt4(const Tensor &x, const Int4 &w) {
  if (x.Rank() != 2 || x.Dim(1) != w.K())
    Fail("ops.MatMulInt4: x %s, weight (%lld, %lld)", x.ShapeStr().c_str(), (long long)w.N(), (long long)w.K());
  // Light takes F32 or BF16 (:70-72); F16 activations are this library's extension.
  if (x.dtype() != DType::F32 && x.dtype() != DType::BF16 && x.dtype() != DType::F16)
    Fail("ops.MatMulInt4: activations %s, want F32, BF16 or F16", DTypeName(x.dtype()));
  const int64_t M = x.Dim(0), N = w.N();
  Tensor xc = x;
  if (w.perm) {
    // Act-order GPTQ: gather x's columns into the weight's K order (x[:, Perm]).
    xc = Tensor::Empty(x.dtype(), x.shape(), x.device());
    if (x.device().kind != DeviceKind::ROCm) Fail("ops.MatMulInt4: act-order gather needs a ROCm device");
    Check(hq_gather_cols(x.data(), static_cast<const int64_t *>(w.perm->data()), xc.data(), M, w.K(),
                         x.dtype() == DType::F32 ? 4 : 2, nullptr));
  }
  // Light runs the fused kernel for M <= 8 on GPUs (:87-99); the ROCm kernel also serves
  // larger M (its MFMA leg), so ROCm takes it for every M.
  const bool fused_ok = w.K() % 32 == 0 && w.group % 32 == 0;
  if (fused_ok && (M <= kInt4GEMVMaxM || x.device().kind != DeviceKind::CUDA)) {
    Kernel k = Lookup(Key{"int4_gemv", x.device().kind, x.dtype()});
    Tensor out = Tensor::Zeros(x.dtype(), {M, N}, x.device());
    Context ctx;
    ctx.inputs = {xc, w.codes, w.scales, w.zeros};
    ctx.output = out;
    ctx.attrs = {{"group", Attr::Int(w.group)}};
    k(ctx);
    return out;
  }
  Fail("ops.MatMulInt4: K=%lld, group %d: no fused kernel (K and the group must be multiples of 32)",
       (long long)w.K(), w.group);
}

// ---- MoE (ops/moe.go) ----

MoERouting MoERoute(const Tensor &probs, int topk, bool normalize) {
  if (probs.Rank() != 2 || probs.dtype() != DType::F32)
    Fail("moe_route: probs must be (T, E) F32, got %s %s", probs.ShapeStr().c_str(), DTypeName(probs.dtype()));
  const int64_t T = probs.Dim(0), E = probs.Dim(1);
  if (topk < 1 || topk > E) Fail("moe_route: topk %d out of range [1, %lld]", topk, (long long)E);
  Kernel k = Lookup(Key{"moe_route", probs.device().kind, DType::F32});
  MoERouting r;
  r.topk_ids = Tensor::Empty(DType::I64, {T, topk}, probs.device());
  r.weights = Tensor::Empty(DType::F32, {T * topk}, probs.device());
  r.sorted_pairs = Tensor::Empty(DType::I64, {T * topk}, probs.device());
  r.sorted_expts = Tensor::Empty(DType::I64, {T * topk}, probs.device());
  Context ctx;  // outputs beyond the first travel as inputs, as ops.TopK's index output does
  ctx.inputs = {probs, r.topk_ids, r.weights, r.sorted_expts};
  ctx.output = r.sorted_pairs;
  ctx.attrs = {{"k", Attr::Int(topk)}, {"normalize", Attr::Bool(normalize)}};
  k(ctx);
  return r;
}

MoERouting MoERouteFromIDs(const std::vector<int64_t> &ids, const std::vector<float> &weights, int64_t T,
                           int topk, Device dev) {
  const int64_t M = T * topk;
  if ((int64_t)ids.size() != M || (int64_t)weights.size() != M)
    Fail("moe_route: %zu ids / %zu weights for %lld × %d", ids.size(), weights.size(), (long long)T, topk);
  if (dev.kind == DeviceKind::ROCm && M > 0) {
    // Sort(flat, false) on the device ("moe_sort", stable ascending).
    int64_t emax = 0;
    for (int64_t v : ids) {
      if (v < 0) Fail("moe_route: expert id %lld < 0", (long long)v);
      emax = std::max(emax, v);
    }
    MoERouting r;
    r.topk_ids = Tensor::FromHost(ids.data(), 8 * M, DType::I64, {T, topk}, dev);
    r.weights = Tensor::FromHost(weights.data(), 4 * M, DType::F32, {M}, dev);
    r.sorted_pairs = Tensor::Empty(DType::I64, {M}, dev);
    r.sorted_expts = Tensor::Empty(DType::I64, {M}, dev);
    Kernel k = Lookup(Key{"moe_sort", dev.kind, DType::I64});
    Context ctx;
    ctx.inputs = {r.topk_ids, r.sorted_expts};
    ctx.output = r.sorted_pairs;
    ctx.attrs = {{"experts", Attr::Int(emax + 1)}};
    k(ctx);
    return r;
  }
  // Sort(flat, false): a stable ascending sort (kernels/cpu/shape_ops.go:156-184).
  std::vector<int64_t> order(M);
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) { return ids[a] < ids[b]; });
  std::vector<int64_t> sorted(M);
  for (int64_t i = 0; i < M; i++) sorted[i] = ids[order[i]];
  MoERouting r;
  r.topk_ids = Tensor::FromHost(ids.data(), 8 * M, DType::I64, {T, topk}, dev);
  r.weights = Tensor::FromHost(weights.data(), 4 * M, DType::F32, {M}, dev);
  r.sorted_pairs = Tensor::FromHost(order.data(), 8 * M, DType::I64, {M}, dev);
  r.sorted_expts = Tensor::FromHost(sorted.data(), 8 * M, DType::I64, {M}, dev);
  return r;
}

// moeGemmDispatch (ops/moe.go:122-204) for op "moe_gemm_q".
static Tensor moe_gemm_dispatch(const char *op, DType key_dt, const Tensor &input, const Tensor &weights,
                                const MoERouting &routing, const Tensor *topk_weights, int topk) {
  if (input.Rank() != 2 || weights.Rank() != 3)
    Fail("%s: input (rows, K) and weights (E, N, K) required, got %s / %s", op, input.ShapeStr().c_str(),
         weights.ShapeStr().c_str());
  if (!same_device(input, weights) || !same_device(input, routing.sorted_pairs)) Fail("%s: device mismatch", op);
  const int64_t E = weights.Dim(0), N = weights.Dim(1), K = weights.Dim(2);
  if (input.Dim(1) != K) Fail("%s: input K %lld != weights K %lld", op, (long long)input.Dim(1), (long long)K);
  const int64_t M = routing.sorted_pairs.Dim(0);
  if (routing.sorted_expts.Dim(0) != M || routing.sorted_pairs.dtype() != DType::I64 ||
      routing.sorted_expts.dtype() != DType::I64)
    Fail("%s: routing must hold M I64 pair ids and M I64 expert ids", op);
  bool row_per_pair;
  if (input.Dim(0) == M)
    row_per_pair = true;
  else if (input.Dim(0) == M / topk)
    row_per_pair = false;
  else
    Fail("%s: input rows %lld must be M=%lld (per pair) or M/topk=%lld (per token)", op, (long long)input.Dim(0),
         (long long)M, (long long)(M / topk));
  if (topk_weights) {
    if (topk_weights->dtype() != DType::F32 || topk_weights->NumElements() != M)
      Fail("%s: topkWeights must be F32 with %lld elements", op, (long long)M);
    if (!same_device(*topk_weights, input)) Fail("%s: topkWeights device mismatch", op);
  }
  Tensor counts = Tensor::Zeros(DType::I32, {E}, input.device());
  Tensor offsets = Tensor::Zeros(DType::I32, {E + 1}, input.device());
  Tensor out = Tensor::Zeros(input.dtype(), {M, N}, input.device());
  Kernel k = Lookup(Key{op, input.device().kind, key_dt});
  Context ctx;
  ctx.inputs = {input, weights, routing.sorted_pairs, routing.sorted_expts, counts, offsets};
  if (topk_weights) ctx.inputs.push_back(*topk_weights);
  ctx.output = out;
  ctx.attrs = {{"topk", Attr::Int(topk)}, {"row_per_pair", Attr::Bool(row_per_pair)}};
  k(ctx);
  return out;
}

Tensor MoEGemmQ(const Tensor &x, const Tensor &w, const MoERouting &routing, const Tensor *topk_weights, int topk) {
  if (x.dtype() != DType::F32) Fail("moe_gemm_q: x must be F32, got %s", DTypeName(x.dtype()));
  if (!IsQuantized(w.dtype()) || w.Rank() != 3)
    Fail("moe_gemm_q: w must be a quantized (E, N, K) tensor, got %s %s", DTypeName(w.dtype()), w.ShapeStr().c_str());
  if (w.Dim(2) % BlockElems(w.dtype()))
    Fail("moe_gemm_q: K=%lld not a multiple of %s block size %d", (long long)w.Dim(2), DTypeName(w.dtype()),
         BlockElems(w.dtype()));
  return moe_gemm_dispatch("moe_gemm_q", w.dtype(), x, w, routing, topk_weights, topk);
}

Tensor MoEGemmQGated(const Tensor &x, const Tensor &w, const MoERouting &routing, int topk, bool gelu) {
  const char *op = "moe_gemm_q_gated";
  if (x.dtype() != DType::F32) Fail("%s: x must be F32, got %s", op, DTypeName(x.dtype()));
  if (!IsQuantized(w.dtype()) || w.Rank() != 3 || w.Dim(1) % 2)
    Fail("%s: w must be a quantized (E, 2I, K) tensor, got %s %s", op, DTypeName(w.dtype()), w.ShapeStr().c_str());
  if (w.Dim(2) % BlockElems(w.dtype()))
    Fail("%s: K=%lld not a multiple of %s block size %d", op, (long long)w.Dim(2), DTypeName(w.dtype()),
         BlockElems(w.dtype()));
  if (x.Rank() != 2) Fail("%s: input (rows, K) required, got %s", op, x.ShapeStr().c_str());
  if (!same_device(x, w) || !same_device(x, routing.sorted_pairs)) Fail("%s: device mismatch", op);
  const int64_t E = w.Dim(0), I = w.Dim(1) / 2, K = w.Dim(2), M = routing.sorted_pairs.Dim(0);
  if (x.Dim(1) != K) Fail("%s: input K %lld != weights K %lld", op, (long long)x.Dim(1), (long long)K);
  bool row_per_pair;
  if (x.Dim(0) == M)
    row_per_pair = true;
  else if (x.Dim(0) == M / topk)
    row_per_pair = false;
  else
    Fail("%s: input rows %lld must be M=%lld (per pair) or M/topk=%lld (per token)", op, (long long)x.Dim(0),
         (long long)M, (long long)(M / topk));
  Tensor counts = Tensor::Zeros(DType::I32, {E}, x.device());
  Tensor offsets = Tensor::Zeros(DType::I32, {E + 1}, x.device());
  Tensor out = Tensor::Zeros(DType::F32, {M, I}, x.device());
  Kernel k = Lookup(Key{op, x.device().kind, w.dtype()});
  Context ctx;
  ctx.inputs = {x, w, routing.sorted_pairs, routing.sorted_expts, counts, offsets};
  ctx.output = out;
  ctx.attrs = {{"topk", Attr::Int(topk)}, {"row_per_pair", Attr::Bool(row_per_pair)}, {"gelu", Attr::Bool(gelu)}};
  k(ctx);
  return out;
}

Tensor MoECombine(const Tensor &pair_out, int topk) {
  const int64_t M = pair_out.Dim(0), N = pair_out.Dim(1);
  if (topk < 1 || M % topk) Fail("moe_combine: %lld rows not divisible by topk %d", (long long)M, topk);
  if (pair_out.dtype() != DType::F32) Fail("moe_combine: %s rows, want F32", DTypeName(pair_out.dtype()));
  if (pair_out.device().kind != DeviceKind::ROCm)
    Fail("moe_combine: device %s is not supported by this build", pair_out.device().str().c_str());
  Tensor out = Tensor::Empty(DType::F32, {M / topk, N}, pair_out.device());
  Check(hq_moe_combine(static_cast<const float *>(pair_out.data()), static_cast<float *>(out.data()), M, N, topk,
                       nullptr));
  return out;
}

// ---- MoEInt4 (ops/int4.go:149-246) ----

Tensor MoEInt4(const Tensor &x, const std::vector<Int4> &gate_up, const std::vector<Int4> &down,
               const MoERouting &routing, int topk, bool gelu) {
  if (x.Rank() != 2 || gate_up.empty() || gate_up.size() != down.size())
    Fail("ops.MoEInt4: x %s, %zu gate-up / %zu down experts", x.ShapeStr().c_str(), gate_up.size(), down.size());
  const int64_t T = x.Dim(0), H = x.Dim(1), I2 = gate_up[0].N(), I = down[0].K();
  if (gate_up[0].K() != H || down[0].N() != H || I2 != 2 * I)
    Fail("ops.MoEInt4: expert shapes gate-up (%lld, %lld), down (%lld, %lld) for hidden %lld", (long long)I2,
         (long long)gate_up[0].K(), (long long)down[0].N(), (long long)I, (long long)H);
  const int G = gate_up[0].group;
  std::vector<uint64_t> tab(6 * gate_up.size());
  const size_t E = gate_up.size();
  for (size_t e = 0; e < E; e++) {
    const Int4 &gu = gate_up[e], &dn = down[e];
    // The fused kernel reads every expert with expert 0's geometry: all must share it.
    if (gu.N() != I2 || gu.K() != H || dn.N() != H || dn.K() != I || gu.group != G || dn.group != G ||
        gu.perm || dn.perm)
      Fail("ops.MoEInt4: expert %zu differs from expert 0 (shapes, group or act-order)", e);
    for (const Tensor *t : {&gu.codes, &gu.scales, &gu.zeros, &dn.codes, &dn.scales, &dn.zeros})
      if (!same_device(*t, x)) Fail("ops.MoEInt4: expert %zu on %s, x on %s", e, t->device().str().c_str(),
                                    x.device().str().c_str());
    tab[0 * E + e] = (uint64_t)(uintptr_t)gu.codes.data();
    tab[1 * E + e] = (uint64_t)(uintptr_t)gu.scales.data();
    tab[2 * E + e] = (uint64_t)(uintptr_t)gu.zeros.data();
    tab[3 * E + e] = (uint64_t)(uintptr_t)dn.codes.data();
    tab[4 * E + e] = (uint64_t)(uintptr_t)dn.scales.data();
    tab[5 * E + e] = (uint64_t)(uintptr_t)dn.zeros.data();
  }
  if (routing.topk_ids.NumElements() != T * topk || routing.weights.NumElements() != T * topk)
    Fail("ops.MoEInt4: routing holds %lld ids for %lld tokens x topk %d", (long long)routing.topk_ids.NumElements(),
         (long long)T, topk);
  Tensor table = Tensor::FromHost(tab.data(), tab.size() * 8, DType::U64, {(int64_t)tab.size()}, x.device());
  Kernel k = Lookup(Key{"moe_int4", x.device().kind, x.dtype()});
  Tensor out = Tensor::Empty(x.dtype(), {T, H}, x.device());
  Context ctx;
  ctx.inputs = {x, table, routing.topk_ids, routing.weights};
  ctx.output = out;
  ctx.attrs = {{"topk", Attr::Int(topk)}, {"group", Attr::Int(G)}, {"inter", Attr::Int(I)},
               {"gelu", Attr::Bool(gelu)}};
  k(ctx);
  return out;
}

// ---- Dequantize (quant/dequant.go:10-42, dispatchRegistry quant/cuda_hook.go:51-69) ----

Tensor Dequantize(const Tensor &w) {
  if (!IsQuantized(w.dtype())) Fail("quant.Dequantize: %s is not a quantized dtype", DTypeName(w.dtype()));
  if (w.NumElements() % BlockElems(w.dtype()))
    Fail("quant.Dequantize: element count %lld not a multiple of %s block size %d", (long long)w.NumElements(),
         DTypeName(w.dtype()), BlockElems(w.dtype()));
  Kernel k = Lookup(Key{"dequant", w.device().kind, w.dtype()});
  Tensor out = Tensor::Empty(DType::F32, w.shape(), w.device());
  Context ctx;
  ctx.inputs = {w};
  ctx.output = out;
  k(ctx);
  return out;
}

}  // namespace ops
}  // namespace light
