"""GGUF tensors loaded straight onto ROCm(0) and consumed by the kernels.

  * gguf/gguf_cuda_test.go:15-74 -- a Q4_0 tensor read from a GGUF stream onto the GPU,
    dequantized there, equals scale * q;
  * models/llama_gguf.go:173-206 -- the MoE expert stacks of a GGUF layer (gate and up
    fused per expert, down row-major) loaded to ROCm and run through MoERoute ->
    MoEGemmQGated -> MoEGemmQ -> MoECombine, checked against the CPU oracle on the same
    bytes.
"""
import struct

import numpy as np
import pytest

import oracle
from _gguf import Writer
from light_amd import _light as L
from light_amd import hipq, synth

pytestmark = pytest.mark.gpu

DEV = "ROCm(0)"


def test_q4_0_tensor_on_rocm():
    print("[case] gguf Q4_0 tensor -> ROCm dequant", flush=True)
    vals = [(i % 16) - 8 for i in range(32)]
    block = struct.pack("<H", int(oracle.half_from_f32(np.float32(0.25))))
    block += bytes(((vals[j] + 8) & 15) | (((vals[j + 16] + 8) & 15) << 4) for j in range(16))
    w = Writer()
    w.add_tensor("w", [32], 2, block)
    f = L.gguf_open_bytes(w.bytes())
    t = f.load_tensor("w", DEV)
    assert t.device == DEV and t.dtype == "Q4_0"
    assert t.numpy().tobytes() == block
    got = L.dequantize(t.reshape([1, 32])).numpy().ravel()
    np.testing.assert_array_equal(got, np.float32(0.25) * np.asarray(vals, np.float32))


@pytest.mark.parametrize("dt,code", [(hipq.Q4_K, 12), (hipq.Q6_K, 14), (hipq.Q8_0, 8)])
def test_gguf_experts_moe_layer(dt, code):
    print(f"[case] gguf experts {hipq.NAMES[dt]} -> MoE layer on ROCm", flush=True)
    g = synth.rng(900 + dt)
    T, E, topk, H, I = 5, 8, 2, 512, 256
    gate = synth.gguf_weight(dt, E * I, H, g)
    up = synth.gguf_weight(dt, E * I, H, g)
    down = synth.gguf_weight(dt, E * H, I, g)
    w = Writer()
    w.add_tensor("blk.3.ffn_gate_exps.weight", [H, I, E], code, gate.tobytes())
    w.add_tensor("blk.3.ffn_up_exps.weight", [H, I, E], code, up.tobytes())
    w.add_tensor("blk.3.ffn_down_exps.weight", [I, H, E], code, down.tobytes())
    f = L.gguf_open_bytes(w.bytes())
    gu, dn = L.gguf_load_experts(f, "blk.3.", DEV)
    assert gu.device == DEV and gu.shape == [E, 2 * I, H] and dn.shape == [E, H, I]

    logits = g.standard_normal((T, E)).astype(np.float32)
    probs = np.exp(logits - logits.max(axis=1, keepdims=True))
    probs = (probs / probs.sum(axis=1, keepdims=True)).astype(np.float32)
    r = L.moe_route(L.from_numpy(probs, "F32", [T, E], DEV), topk, True)
    _, rw, rsp, rse = oracle.moe_route(probs, topk, True)
    x = synth.activations(T, H, g)
    h = L.moe_gemm_q_gated(L.from_numpy(x, "F32", [T, H], DEV), gu, r, topk, False)
    y = L.moe_combine(L.moe_gemm_q(h, dn, r, r.weights, topk), topk).numpy()

    # The oracle's fused (E, 2I, H) stack, built from the file's per-expert slabs.
    slab = gate.nbytes // E
    fused = np.concatenate([np.concatenate([gate.reshape(E, slab)[e], up.reshape(E, slab)[e]]) for e in range(E)])
    gur = oracle.moe_gemm_q(x, fused, dt, E, 2 * I, H, rsp, rse, topk)
    hr = oracle.gated(gur[:, :I], gur[:, I:], hipq.ACT_SILU)
    assert np.max(np.abs(h.numpy() - hr)) <= 1e-3 * np.abs(hr).max()
    want = oracle.moe_combine(oracle.moe_gemm_q(hr, down, dt, E, H, I, rsp, rse, topk, topk_w=rw), topk)
    assert np.max(np.abs(y - want)) <= 5e-3 * np.abs(want).max()
