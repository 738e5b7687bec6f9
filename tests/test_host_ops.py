"""Host layer (light_amd._light): registry behaviour and the ops' argument validation.

These mirror Light's Go-side contracts without touching a GPU:
  * internal/registry/registry.go:20-82 -- Key.String, duplicate registration panics,
    Lookup wraps ErrKernelNotFound;
  * ops/matmul_q.go:27-47, ops/int4.go:67-72, ops/moe.go:78-82,122-160,206-214,246-256,
    quant/dequant.go:38-41 -- the checks and messages each op raises before dispatch.
Tensors here are CPU tensors; no CPU kernels are registered in this build, so a
well-formed call on the CPU fails with KernelNotFound (the ROCm keys are the product).
"""
import numpy as np
import pytest

from light_amd import _light as L


def f32(*shape):
    return L.from_numpy(np.zeros(shape, np.float32), "F32", list(shape))


def q(dt, N, K):
    return L.from_numpy(np.zeros(L.byte_size(dt, N * K), np.uint8), dt, [N, K])


GGUF = ["Q4_0", "Q5_0", "Q8_0", "Q4_K", "Q5_K", "Q6_K"]


def test_registered_rocm_keys():
    keys = set(L.registered())
    for dt in GGUF:
        for op in ("matmul_q", "matmul_q_gated", "moe_gemm_q", "moe_gemm_q_gated", "dequant"):
            assert f"{op}/ROCm/{dt}" in keys
    for dt in ("F32", "BF16", "F16"):
        assert f"int4_gemv/ROCm/{dt}" in keys
    for dt in ("F32", "BF16"):
        assert f"int4_dequant/ROCm/{dt}" in keys
    assert "dequant/ROCm/Q8_1" in keys
    assert "moe_route/ROCm/F32" in keys and "moe_sort/ROCm/I64" in keys


def test_duplicate_registration_fails():
    L.register_noop("host_test_op", "CPU", "F32")
    with pytest.raises(L.Error, match="registry: duplicate kernel for host_test_op/CPU/F32"):
        L.register_noop("host_test_op", "CPU", "F32")
    with pytest.raises(L.Error, match="duplicate kernel for matmul_q/ROCm/Q4_K"):
        L.register_noop("matmul_q", "ROCm", "Q4_K")


def test_lookup_not_found():
    with pytest.raises(L.KernelNotFound, match=r"^registry: kernel not found: matmul_q/CPU/Q4_K$"):
        L.lookup("matmul_q", "CPU", "Q4_K")
    L.lookup("matmul_q", "ROCm", "Q4_K")
    assert issubclass(L.KernelNotFound, L.Error)


def test_matmul_q_fused_on():
    for dt in GGUF:
        assert L.matmul_q_fused_on("ROCm", dt)
        assert not L.matmul_q_fused_on("CPU", dt)
    for dt in ("Q4_1", "Q5_1", "Q2_K", "Q3_K", "Q8_K"):  # no fused kernel: ops.MatMulQ falls back
        assert not L.matmul_q_fused_on("ROCm", dt)


def test_tensor_roundtrip_and_sizes():
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    t = L.from_numpy(a, "F32", [3, 4])
    assert t.shape == [3, 4] and t.dtype == "F32" and t.device == "CPU"
    assert np.array_equal(t.numpy(), a)
    assert L.byte_size("Q4_K", 512) == 288 and L.byte_size("Q8_0", 64) == 68 and L.byte_size("Q6_K", 256) == 210
    assert L.byte_size("Q4_0", 64) == 36 and L.byte_size("Q5_0", 64) == 44 and L.byte_size("Q5_K", 512) == 352
    with pytest.raises(L.Error, match="bytes for F32"):
        L.from_numpy(a, "F32", [4, 4])
    assert t.reshape([2, 6]).shape == [2, 6]
    with pytest.raises(L.Error, match="cannot reshape"):
        t.reshape([5])


def test_matmul_q_validation():
    x, w = f32(2, 256), q("Q4_K", 8, 256)
    with pytest.raises(L.Error, match=r"MatMulQ: want x \(M,K\) and w \(N,K\); got \[256\], \[8 256\]"):
        L.matmul_q(f32(256), w)
    with pytest.raises(L.Error, match="MatMulQ: x must be F32, got BF16"):
        L.matmul_q(L.from_numpy(np.zeros((2, 256), np.uint16), "BF16", [2, 256]), w)
    with pytest.raises(L.Error, match="MatMulQ: w must be a quantized dtype, got F32"):
        L.matmul_q(x, f32(8, 256))
    with pytest.raises(L.Error, match=r"MatMulQ: inner dim mismatch \(x K=256, w K=512\)"):
        L.matmul_q(x, q("Q4_K", 8, 512))
    with pytest.raises(L.Error, match="MatMulQ: K=288 not a multiple of Q4_K block size 256"):
        L.matmul_q(f32(1, 288), q("Q4_K", 8, 288))
    # No fused CPU kernel: MatMulQ takes matMulQFallback (ops/matmul_q.go:61-71), whose
    # Dequantize finds no CPU "dequant" kernel in this build.
    with pytest.raises(L.KernelNotFound, match="^registry: kernel not found: dequant/CPU/Q4_K$"):
        L.matmul_q(x, w)


def test_matmul_q_falls_back_for_unfused_formats():
    """A format with no fused kernel (Q3_K) goes through the dequant + matmul fallback rather
    than failing on the matmul_q lookup (ops/matmul_q.go:65-71)."""
    x = f32(1, 256)
    w = q("Q3_K", 4, 256)
    with pytest.raises(L.KernelNotFound, match="^registry: kernel not found: dequant/CPU/Q3_K$"):
        L.matmul_q(x, w)


def test_int4_validation():
    codes = L.from_numpy(np.zeros((4, 32), np.uint32), "U32", [4, 32])
    s = f32(4, 2)
    with pytest.raises(L.Error, match=r"ops.MatMulInt4: x \[1 128\], weight \(4, 256\)"):
        L.matmul_int4(f32(1, 128), codes, s, s, 128)
    with pytest.raises(L.Error, match="ops.MatMulInt4: activations I32"):
        L.matmul_int4(L.from_numpy(np.zeros((1, 256), np.int32), "I32", [1, 256]), codes, s, s, 128)
    with pytest.raises(L.Error, match="ops.DequantizeInt4: group 96 does not divide K 256"):
        L.dequantize_int4(codes, s, s, 96, "F32")
    with pytest.raises(L.KernelNotFound, match="int4_gemv/CPU/F32"):
        L.matmul_int4(f32(1, 256), codes, s, s, 128)


def test_moe_route_from_ids_stable_sort():
    ids = [3, 1, 3, 0, 1, 1]
    r = L.moe_route_from_ids(ids, [0.5] * 6, 3, 2, "CPU")
    assert r.topk_ids.shape == [3, 2]
    assert r.sorted_pairs.numpy().tolist() == [3, 1, 4, 5, 0, 2]  # stable: ties keep pair order
    assert r.sorted_expts.numpy().tolist() == [0, 1, 1, 1, 3, 3]
    with pytest.raises(L.Error, match="moe_route: 5 ids / 6 weights for 3 × 2"):
        L.moe_route_from_ids(ids[:5], [0.5] * 6, 3, 2, "CPU")


def test_moe_gemm_q_validation():
    T, topk, E, N, K = 3, 2, 4, 8, 256
    r = L.moe_route_from_ids([0, 1, 2, 3, 0, 1], [1.0] * 6, T, topk, "CPU")
    w = q("Q4_K", E * N, K).reshape([E, N, K])
    with pytest.raises(L.Error, match="moe_gemm_q: x must be F32, got I32"):
        L.moe_gemm_q(L.from_numpy(np.zeros((T, K), np.int32), "I32", [T, K]), w, r, None, topk)
    with pytest.raises(L.Error, match=r"moe_gemm_q: w must be a quantized \(E, N, K\) tensor, got Q4_K \[32 256\]"):
        L.moe_gemm_q(f32(T, K), q("Q4_K", E * N, K), r, None, topk)
    with pytest.raises(L.Error, match="moe_gemm_q: K=288 not a multiple of Q4_K block size 256"):
        L.moe_gemm_q(f32(T, 288), q("Q4_K", E * N, 288).reshape([E, N, 288]), r, None, topk)
    with pytest.raises(L.Error, match="moe_gemm_q: input K 128 != weights K 256"):
        L.moe_gemm_q(f32(T, 128), w, r, None, topk)
    with pytest.raises(L.Error, match=r"moe_gemm_q: input rows 4 must be M=6 \(per pair\) or M/topk=3 \(per token\)"):
        L.moe_gemm_q(f32(4, K), w, r, None, topk)
    with pytest.raises(L.Error, match="moe_gemm_q: topkWeights must be F32 with 6 elements"):
        L.moe_gemm_q(f32(T, K), w, r, f32(5), topk)
    with pytest.raises(L.KernelNotFound, match="moe_gemm_q/CPU/Q4_K"):
        L.moe_gemm_q(f32(T, K), w, r, f32(6), topk)


def test_moe_combine_and_dequantize_validation():
    with pytest.raises(L.Error, match="moe_combine: 5 rows not divisible by topk 2"):
        L.moe_combine(f32(5, 4), 2)
    with pytest.raises(L.Error, match="quant.Dequantize: F32 is not a quantized dtype"):
        L.dequantize(f32(4))
    with pytest.raises(L.KernelNotFound, match="dequant/CPU/Q6_K"):
        L.dequantize(q("Q6_K", 1, 256))


def test_matmul_q_gated_validation():
    x, w = f32(1, 256), q("Q4_K", 8, 256)
    with pytest.raises(L.Error, match=r"MatMulQGated: x must be \(M, K\) F32"):
        L.matmul_q_gated(f32(256), w, w)
    with pytest.raises(L.Error, match=r"MatMulQGated: weights must be \(N, 256\) Q4_K on CPU"):
        L.matmul_q_gated(x, w, q("Q4_K", 16, 256))
    with pytest.raises(L.KernelNotFound, match="matmul_q_gated/CPU/Q4_K"):
        L.matmul_q_gated(x, w, w)


def test_moe_route_checks():
    """ops.MoERoute's argument checks (ops/moe.go:29-37), then the registry lookup."""
    with pytest.raises(L.Error, match=r"moe_route: probs must be \(T, E\) F32"):
        L.moe_route(L.from_numpy(np.zeros(8, np.float32), "F32", [8]), 2)
    with pytest.raises(L.Error, match=r"moe_route: topk 5 out of range \[1, 4\]"):
        L.moe_route(f32(3, 4), 5)
    with pytest.raises(L.KernelNotFound, match="moe_route/CPU/F32"):
        L.moe_route(f32(3, 4), 2)


def test_moe_int4_validation():
    """ops.MoEInt4's argument checks and messages (ops/int4.go:159-167)."""
    x = f32(2, 64)
    c = L.from_numpy(np.zeros((64, 8), np.uint32), "U32", [64, 8])
    s = f32(64, 2)
    r = L.moe_route_from_ids([0, 0], [1.0, 1.0], 2, 1, "CPU")
    with pytest.raises(L.Error, match=r"ops.MoEInt4: x \[2 64\], 1 gate-up / 0 down experts"):
        L.moe_int4(x, [(c, s, s)], [], r, 1, 32)
    cd = L.from_numpy(np.zeros((64, 4), np.uint32), "U32", [64, 4])
    sd = f32(64, 1)
    c60 = L.from_numpy(np.zeros((60, 8), np.uint32), "U32", [60, 8])
    with pytest.raises(L.Error, match=r"ops.MoEInt4: expert shapes gate-up \(60, 64\), down \(64, 32\) for hidden 64"):
        L.moe_int4(x, [(c60, s, s)], [(cd, sd, sd)], r, 1, 32)
    # Valid shapes on the CPU: this build registers the kernel for ROCm only.
    with pytest.raises(L.KernelNotFound, match="^registry: kernel not found: moe_int4/CPU/F32$"):
        L.moe_int4(x, [(c, s, s)], [(cd, sd, sd)], r, 1, 32)
