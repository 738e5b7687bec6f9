// quant.cpp -- quant.FromGPTQ / quant.FromAWQ (quant/int4.go:102-235): GPTQ and AutoAWQ
// checkpoint tensors to Light's canonical quant.Int4, with Light's checks and messages.
//
// Light converts on the host into CPU tensors; here the conversion runs on the ROCm device
// (hq_int4_from_gptq / hq_int4_from_awq) and the Int4 it returns lives there: ROCm inputs
// stay on their device, CPU inputs are copied to ROCm device 0 first.  Only the act-order
// permutation (a stable sort of K by g_idx, K entries) is computed on the host, as in Light.
#include <algorithm>
#include <numeric>

#include "../../include/hipq.h"
#include "ops.hpp"

namespace light {
namespace quant {

namespace {

std::string shape_v(const Tensor &t) {  // Go's %v of a []int
  std::string s = "[";
  for (int i = 0; i < t.Rank(); i++) s += (i ? " " : "") + std::to_string(t.Dim(i));
  return s + "]";
}

// u32s (quant/int4.go:39-59): I32 or U32 words.
void need_words(const Tensor &t, const char *name) {
  if (t.dtype() != DType::I32 && t.dtype() != DType::U32)
    Fail("quant: %s is %s, want I32 / U32", name, DTypeName(t.dtype()));
}

// f32s (quant/int4.go:61-73).
void need_f32(const Tensor &t) {
  if (t.dtype() != DType::F32)
    Fail("quant: scales / zeros must be F32 (cast the checkpoint's F16 first), got %s", DTypeName(t.dtype()));
}

Device target(const Tensor &t) { return t.device().kind == DeviceKind::ROCm ? t.device() : ROCm(0); }

Tensor on(const Tensor &t, const Device &dev) {
  if (t.device().SameAs(dev)) return t;
  std::vector<uint8_t> host(t.nbytes());
  t.ToHost(host.data(), host.size());
  return Tensor::FromHost(host.data(), host.size(), t.dtype(), t.shape(), dev);
}

std::vector<int64_t> host_ints(const Tensor &t) {
  std::vector<int64_t> v((size_t)t.NumElements());
  if (t.dtype() == DType::I32 || t.dtype() == DType::U32) {
    std::vector<uint32_t> w(v.size());
    t.ToHost(w.data(), w.size() * 4);
    for (size_t i = 0; i < v.size(); i++) v[i] = (int64_t)w[i];
  } else {
    Fail("quant: g_idx is %s, want I32 / U32", DTypeName(t.dtype()));
  }
  return v;
}

}  // namespace

ops::Int4 FromGPTQ(const Tensor &qweight, const Tensor &qzeros, const Tensor &scales, const Tensor *g_idx, int group,
                   bool v2) {
  if (qweight.Rank() != 2 || qzeros.Rank() != 2 || scales.Rank() != 2)
    Fail("quant.FromGPTQ: rank-2 qweight / qzeros / scales expected");
  const int64_t K = qweight.Dim(0) * 8, N = qweight.Dim(1);
  if (group <= 0) group = (int)K;  // group_size -1: one group over all of K
  if (K % group != 0 || scales.Dim(0) != K / group || scales.Dim(1) != N || qzeros.Dim(0) != K / group ||
      qzeros.Dim(1) * 8 != N)
    Fail("quant.FromGPTQ: qweight %s, qzeros %s, scales %s, group %d inconsistent", shape_v(qweight).c_str(),
         shape_v(qzeros).c_str(), shape_v(scales).c_str(), group);
  // Act order: sort K stably by group so each group is contiguous; Perm records the order.
  std::vector<int64_t> perm;
  if (g_idx) {
    const std::vector<int64_t> gi = host_ints(*g_idx);
    if ((int64_t)gi.size() != K)
      Fail("quant.FromGPTQ: g_idx has %lld entries for K %lld", (long long)gi.size(), (long long)K);
    bool ordered = true;
    for (int64_t k = 0; k < K && ordered; k++) ordered = gi[k] == k / group;
    if (!ordered) {
      perm.resize((size_t)K);
      std::iota(perm.begin(), perm.end(), 0);
      std::stable_sort(perm.begin(), perm.end(), [&](int64_t a, int64_t b) { return gi[a] < gi[b]; });
      for (int64_t kk = 0; kk < K; kk++)
        if (gi[perm[kk]] != kk / group) Fail("quant.FromGPTQ: g_idx groups are not all of size %d", group);
    }
  }
  need_words(qweight, "qweight");
  need_words(qzeros, "qzeros");
  need_f32(scales);
  if (K % 8 || N % 8) Fail("quant.FromGPTQ: K %lld and N %lld must be multiples of 8", (long long)K, (long long)N);
  const Device dev = target(qweight);
  const Tensor qw = on(qweight, dev), qz = on(qzeros, dev), sc = on(scales, dev);
  ops::Int4 w;
  w.group = group;
  w.codes = Tensor::Empty(DType::U32, {N, K / 8}, dev);
  w.scales = Tensor::Empty(DType::F32, {N, K / group}, dev);
  w.zeros = Tensor::Empty(DType::F32, {N, K / group}, dev);
  if (!perm.empty()) w.perm = Tensor::FromHost(perm.data(), perm.size() * 8, DType::I64, {K}, dev);
  Check(hq_int4_from_gptq(qw.data(), qz.data(), static_cast<const float *>(sc.data()),
                          w.perm ? static_cast<const int64_t *>(w.perm->data()) : nullptr, K, N, group, v2 ? 1 : 0,
                          static_cast<uint32_t *>(w.codes.data()), static_cast<float *>(w.scales.data()),
                          static_cast<float *>(w.zeros.data()), nullptr));
  return w;
}

ops::Int4 FromAWQ(const Tensor &qweight, const Tensor &qzeros, const Tensor &scales, int group) {
  if (qweight.Rank() != 2 || qzeros.Rank() != 2 || scales.Rank() != 2)
    Fail("quant.FromAWQ: rank-2 qweight / qzeros / scales expected");
  const int64_t K = qweight.Dim(0), N = qweight.Dim(1) * 8;
  if (group <= 0 || K % group != 0 || scales.Dim(0) != K / group || scales.Dim(1) != N ||
      qzeros.Dim(0) != K / group || qzeros.Dim(1) * 8 != N)
    Fail("quant.FromAWQ: qweight %s, qzeros %s, scales %s, group %d inconsistent", shape_v(qweight).c_str(),
         shape_v(qzeros).c_str(), shape_v(scales).c_str(), group);
  need_words(qweight, "qweight");
  need_words(qzeros, "qzeros");
  need_f32(scales);
  if (K % 8) Fail("quant.FromAWQ: K %lld must be a multiple of 8", (long long)K);
  const Device dev = target(qweight);
  const Tensor qw = on(qweight, dev), qz = on(qzeros, dev), sc = on(scales, dev);
  ops::Int4 w;
  w.group = group;
  w.codes = Tensor::Empty(DType::U32, {N, K / 8}, dev);
  w.scales = Tensor::Empty(DType::F32, {N, K / group}, dev);
  w.zeros = Tensor::Empty(DType::F32, {N, K / group}, dev);
  Check(hq_int4_from_awq(qw.data(), qz.data(), static_cast<const float *>(sc.data()), K, N, group,
                         static_cast<uint32_t *>(w.codes.data()), static_cast<float *>(w.scales.data()),
                         static_cast<float *>(w.zeros.data()), nullptr));
  return w;
}

}  // namespace quant
}  // namespace light
