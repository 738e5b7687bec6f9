// ops.hpp -- Light's public ops for the quantized matmul path (package ops), restated in C++.
//
// Each op validates like Light's Go function (same checks, same messages), allocates its
// output as Light's op layer does, and runs the kernel registered for
// (op, device kind, dtype) -- on ROCm the libhipq kernels of kernels_rocm.cpp.
#pragma once

#include <optional>
#include <vector>

#include "light.hpp"

namespace light {
namespace ops {

// ops.MatMulQ (ops/matmul_q.go:14-76): x F32 (M, K) times a GGUF-quantized weight (N, K)^T -> F32 (M, N).
Tensor MatMulQ(const Tensor &x, const Tensor &w);
// matMulQFallback (ops/matmul_q.go:85-95): Dequantize, then the registry's F32 "matmul".
Tensor MatMulQFallback(const Tensor &x, const Tensor &w);
// ops.MatMulQFusedOn (ops/matmul_q.go:102-106).
bool MatMulQFusedOn(DeviceKind kind, DType dt);
// Gated projection on quantized weights: act(x . wg^T) * (x . wu^T), act = SiLU or GELU (erf)
// -- ops.GatedLinear's contract (ops/gemv.go:80-130: Inputs [x, wg, wu], Attrs {"gelu"}) for
// GGUF weights and F32 x of any M, registry key "matmul_q_gated" keyed by the weight dtype.
Tensor MatMulQGated(const Tensor &x, const Tensor &wg, const Tensor &wu, bool gelu);

// quant.Int4 (quant/int4.go:11-34): Codes U32 (N, K/8), Scales / Zeros F32 (N, K/G), Group,
// Perm I64 (K,) for act-order checkpoints.
struct Int4 {
  Tensor codes, scales, zeros;
  int group = 0;
  std::optional<Tensor> perm;
  int64_t N() const { return codes.Dim(0); }
  int64_t K() const { return codes.Dim(1) * 8; }
};
// ops.DequantizeInt4 (ops/int4.go:13-56).
Tensor DequantizeInt4(const Int4 &w, DType out_dt);
// ops.MatMulInt4 (ops/int4.go:61-127).
Tensor MatMulInt4(const Tensor &x, const Int4 &w);

// ops.MoERouting (ops/moe.go:13-22).
struct MoERouting {
  Tensor topk_ids, weights, sorted_pairs, sorted_expts;
};
// ops.MoERoute (ops/moe.go:24-71): top-k of router probabilities (T, E) F32, optional
// renormalisation, expert sort -- one "moe_route" kernel on ROCm.
MoERouting MoERoute(const Tensor &probs, int topk, bool normalize);
// ops.MoERouteFromIDs (ops/moe.go:73-99).
MoERouting MoERouteFromIDs(const std::vector<int64_t> &ids, const std::vector<float> &weights, int64_t T,
                           int topk, Device dev);
// ops.MoEGemmQ (ops/moe.go:242-265); topk_weights may be absent.
Tensor MoEGemmQ(const Tensor &x, const Tensor &w, const MoERouting &routing, const Tensor *topk_weights, int topk);
// The routed gated gate/up of nn.SparseMoE.runExperts (nn/moe.go:196-236): w (E, 2I, K)
// stacked gate/up, output (M, I) = act(gate) * up ("moe_gemm_q_gated", keyed by w's dtype).
Tensor MoEGemmQGated(const Tensor &x, const Tensor &w, const MoERouting &routing, int topk, bool gelu);
// ops.MoEInt4 (ops/int4.go:149-246): x (T, H) F32 / BF16 / F16, per-expert gate-up (2I, H) and
// down (H, I) canonical 4-bit weights, the routing's TopKIDs / Weights; act = SiLU or GELU
// (erf).  Returns (T, H) at x's dtype ("moe_int4" registry key, keyed by x's dtype).
Tensor MoEInt4(const Tensor &x, const std::vector<Int4> &gate_up, const std::vector<Int4> &down,
               const MoERouting &routing, int topk, bool gelu);
// ops.MoECombine (ops/moe.go:206-240).
Tensor MoECombine(const Tensor &pair_out, int topk);

// quant.Dequantize (quant/dequant.go:10-42) through the "dequant" registry key.
Tensor Dequantize(const Tensor &w);

}  // namespace ops

namespace quant {
// quant.FromGPTQ (quant/int4.go:102-182): AutoGPTQ / GPTQModel qweight I32 (K/8, N), qzeros
// I32 (K/G, N/8), scales F32 (K/G, N), optional g_idx (K,) (act order -> Perm); v2 =
// checkpoint_format "gptq_v2".  Converted on the ROCm device; the Int4 lives there.
ops::Int4 FromGPTQ(const Tensor &qweight, const Tensor &qzeros, const Tensor &scales, const Tensor *g_idx, int group,
                   bool v2);
// quant.FromAWQ (quant/int4.go:184-235): AutoAWQ GEMM qweight I32 (K, N/8), qzeros I32
// (K/G, N/8), scales F32 (K/G, N).
ops::Int4 FromAWQ(const Tensor &qweight, const Tensor &qzeros, const Tensor &scales, int group);
}  // namespace quant
}  // namespace light
