// kernels_rocm.cpp -- registry entries of the ROCm backend (the role of Light's
// kernels/cuda/*.go init() registrations: matmul_q.go:35-39, int4.go:15-20,
// moe.go:78-82, dequant.go:15-17).  Each kernel unpacks its Context and calls one
// libhipq C-ABI entry point on the library's current stream.
#include "../../include/hipq.h"
#include "registry.hpp"

namespace light {
namespace {

// The six formats Light fuses on CUDA (kernels/cuda/matmul_q.go:17-24, moe.go:78-82).
const DType kGGUF[] = {DType::Q4_0, DType::Q5_0, DType::Q8_0, DType::Q4_K, DType::Q5_K, DType::Q6_K};

void matmul_q(Context &c) {
  const Tensor &x = c.in(0), &w = c.in(1);
  Check(hq_matmul_q(static_cast<const float *>(x.data()), w.data(), static_cast<float *>(c.output.data()), x.Dim(0),
                    w.Dim(0), x.Dim(1), (int)w.dtype(), nullptr, 0, nullptr));
}

void matmul_q_gated(Context &c) {
  const Tensor &x = c.in(0), &wg = c.in(1), &wu = c.in(2);
  Check(hq_matmul_q_gated(static_cast<const float *>(x.data()), wg.data(), wu.data(),
                          static_cast<float *>(c.output.data()), x.Dim(0), wg.Dim(0), x.Dim(1), (int)wg.dtype(),
                          c.attr("gelu") ? HQ_ACT_GELU_ERF : HQ_ACT_SILU, nullptr, 0, nullptr));
}

void int4_gemv(Context &c) {
  const Tensor &x = c.in(0), &codes = c.in(1), &s = c.in(2), &z = c.in(3);
  Check(hq_int4_matmul(x.data(), (int)x.dtype(), static_cast<const uint32_t *>(codes.data()),
                       static_cast<const float *>(s.data()), static_cast<const float *>(z.data()), c.output.data(),
                       x.Dim(0), codes.Dim(0), x.Dim(1), (int)c.attr("group"), nullptr, 0, nullptr));
}

void int4_dequant(Context &c) {
  const Tensor &codes = c.in(0), &s = c.in(1), &z = c.in(2);
  Check(hq_int4_dequant(static_cast<const uint32_t *>(codes.data()), static_cast<const float *>(s.data()),
                        static_cast<const float *>(z.data()), c.output.data(), (int)c.output.dtype(), codes.Dim(0),
                        codes.Dim(1) * 8, (int)c.attr("group"), c.attr("offset"), nullptr));
}

void moe_gemm_q(Context &c) {
  const Tensor &x = c.in(0), &w = c.in(1), &pairs = c.in(2), &expts = c.in(3), &counts = c.in(4),
               &offsets = c.in(5);
  const float *tw = c.has(6) ? static_cast<const float *>(c.in(6).data()) : nullptr;
  const int topk = (int)c.attr("topk");
  Check(hq_moe_gemm_q(static_cast<const float *>(x.data()), w.data(), static_cast<const int64_t *>(pairs.data()),
                      static_cast<const int64_t *>(expts.data()), static_cast<int32_t *>(counts.data()),
                      static_cast<int32_t *>(offsets.data()), tw, static_cast<float *>(c.output.data()), topk,
                      c.output.Dim(0), pairs.Dim(0), x.Dim(0), w.Dim(0), w.Dim(1), w.Dim(2),
                      (int)c.attr("row_per_pair"), (int)w.dtype(), nullptr, 0, nullptr));
}

// ops.MoERoute: inputs {probs, topk_ids, weights, sorted_expts}, output sorted_pairs.
void moe_route(Context &c) {
  const Tensor &probs = c.in(0), &ids = c.in(1), &w = c.in(2), &se = c.in(3);
  Check(hq_moe_route(static_cast<const float *>(probs.data()), probs.Dim(0), probs.Dim(1), (int)c.attr("k"),
                     (int)c.attr("normalize"), static_cast<int64_t *>(ids.data()), static_cast<float *>(w.data()),
                     static_cast<int64_t *>(c.output.data()), static_cast<int64_t *>(se.data()), nullptr, nullptr,
                     nullptr));
}

// MoERouteFromIDs' Sort: inputs {ids, sorted_expts}, output sorted_pairs, attr experts.
void moe_sort(Context &c) {
  const Tensor &ids = c.in(0), &se = c.in(1);
  Check(hq_moe_sort_ids(static_cast<const int64_t *>(ids.data()), ids.NumElements(), c.attr("experts"),
                        static_cast<int64_t *>(c.output.data()), static_cast<int64_t *>(se.data()), nullptr, nullptr,
                        nullptr));
}

void moe_gemm_q_gated(Context &c) {
  const Tensor &x = c.in(0), &w = c.in(1), &pairs = c.in(2), &expts = c.in(3), &counts = c.in(4),
               &offsets = c.in(5);
  Check(hq_moe_gemm_q_gated(static_cast<const float *>(x.data()), w.data(), static_cast<const int64_t *>(pairs.data()),
                            static_cast<const int64_t *>(expts.data()), static_cast<int32_t *>(counts.data()),
                            static_cast<int32_t *>(offsets.data()), static_cast<float *>(c.output.data()),
                            (int)c.attr("topk"), c.output.Dim(0), pairs.Dim(0), x.Dim(0), w.Dim(0), w.Dim(1) / 2,
                            w.Dim(2), (int)c.attr("row_per_pair"), (int)w.dtype(),
                            c.attr("gelu") ? HQ_ACT_GELU_ERF : HQ_ACT_SILU, nullptr, 0, nullptr));
}

// ops.MoEInt4: inputs {x, expert pointer table U64 (6E), topk_ids, weights}.
void moe_int4(Context &c) {
  const Tensor &x = c.in(0), &tab = c.in(1), &ids = c.in(2), &w = c.in(3);
  Check(hq_moe_int4(x.data(), (int)x.dtype(), static_cast<const void *const *>(tab.data()), tab.Dim(0) / 6,
                    static_cast<const int64_t *>(ids.data()), static_cast<const float *>(w.data()), c.output.data(),
                    x.Dim(0), (int)c.attr("topk"), x.Dim(1), c.attr("inter"), (int)c.attr("group"),
                    c.attr("gelu") ? HQ_ACT_GELU_ERF : HQ_ACT_SILU, nullptr, 0, nullptr));
}

void dequant(Context &c) {
  const Tensor &w = c.in(0);
  Check(hq_dequant(w.data(), c.output.data(), w.NumElements(), (int)w.dtype(), HQ_F32, nullptr));
}

struct Registrar {
  Registrar() {
    for (DType dt : kGGUF) {
      Register(Key{"matmul_q", DeviceKind::ROCm, dt}, matmul_q);
      Register(Key{"matmul_q_gated", DeviceKind::ROCm, dt}, matmul_q_gated);
      Register(Key{"moe_gemm_q", DeviceKind::ROCm, dt}, moe_gemm_q);
      Register(Key{"moe_gemm_q_gated", DeviceKind::ROCm, dt}, moe_gemm_q_gated);
      Register(Key{"dequant", DeviceKind::ROCm, dt}, dequant);
    }
    Register(Key{"dequant", DeviceKind::ROCm, DType::Q8_1}, dequant);
    Register(Key{"moe_route", DeviceKind::ROCm, DType::F32}, moe_route);
    Register(Key{"moe_sort", DeviceKind::ROCm, DType::I64}, moe_sort);
    for (DType dt : {DType::F32, DType::BF16, DType::F16}) Register(Key{"int4_gemv", DeviceKind::ROCm, dt}, int4_gemv);
    for (DType dt : {DType::F32, DType::BF16}) Register(Key{"int4_dequant", DeviceKind::ROCm, dt}, int4_dequant);
    for (DType dt : {DType::F32, DType::BF16, DType::F16}) Register(Key{"moe_int4", DeviceKind::ROCm, dt}, moe_int4);
  }
};
const Registrar registrar;

}  // namespace
}  // namespace light
