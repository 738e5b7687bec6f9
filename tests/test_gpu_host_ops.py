"""GPU parity of Light's ops API as restated by the C++ host layer (light_amd._light).

Each test goes through the registry exactly as Light's callers do -- ops.MatMulQ,
ops.MatMulInt4 (incl. act-order Perm), ops.DequantizeInt4, quant.Dequantize,
ops.MoERouteFromIDs -> ops.MoEGemmQ -> ops.MoECombine -- on ROCm(0) tensors, and checks
against the CPU oracle (Light's CPU kernels restated): bit-exact for dequantization and
the combine; max |err| / (||w_n|| ||x_m||) <= 1e-3 for the matmuls.
"""
import numpy as np
import pytest

import oracle
from _util import norm_err
from light_amd import _light as L
from light_amd import hipq, synth

pytestmark = pytest.mark.gpu

DEV = "ROCm(0)"
TOL = 1e-3
NAME = hipq.NAMES


def dev_t(a, dt, shape):
    return L.from_numpy(np.ascontiguousarray(a), dt, list(shape), DEV)


@pytest.mark.parametrize("dt", [hipq.Q4_0, hipq.Q5_0, hipq.Q8_0, hipq.Q4_K, hipq.Q5_K, hipq.Q6_K])
@pytest.mark.parametrize("M", [1, 5, 40])
def test_matmul_q(dt, M):
    print(f"[case] host MatMulQ {NAME[dt]} M={M}", flush=True)
    g = synth.rng(100 + dt + M)
    N, K = 96, 1024
    w = synth.gguf_weight(dt, N, K, g)
    x = synth.activations(M, K, g)
    y = L.matmul_q(dev_t(x, "F32", (M, K)), dev_t(w, NAME[dt], (N, K)))
    assert y.shape == [M, N] and y.dtype == "F32" and y.device == DEV
    got = y.numpy()
    want = oracle.matmul_q(x, w, N, K, dt)
    wd = oracle.dequant(dt, w, N * K).reshape(N, K)
    assert norm_err(got, want, np.linalg.norm(wd, axis=1), np.linalg.norm(x, axis=1)) <= TOL


@pytest.mark.parametrize("dt", [hipq.Q4_0, hipq.Q5_0, hipq.Q8_0, hipq.Q4_K, hipq.Q5_K, hipq.Q6_K])
def test_dequantize_bit_exact(dt):
    g = synth.rng(200 + dt)
    N, K = 16, 512
    w = synth.gguf_weight(dt, N, K, g)
    got = L.dequantize(dev_t(w, NAME[dt], (N, K))).numpy()
    want = oracle.dequant(dt, w, N * K).reshape(N, K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("out_dt", ["F32", "BF16"])
def test_dequantize_int4_bit_exact(out_dt):
    g = synth.rng(300)
    N, K, G = 24, 512, 128
    codes, s, z = synth.int4_weight(N, K, G, g)
    t = L.dequantize_int4(dev_t(codes, "U32", codes.shape), dev_t(s, "F32", s.shape), dev_t(z, "F32", z.shape), G,
                          out_dt)
    want = oracle.int4_dequant(codes, s, z, N, K, G, out_dt=oracle.F32 if out_dt == "F32" else oracle.BF16)
    got = t.numpy()
    assert np.array_equal(got.reshape(-1).view(np.uint8), np.ascontiguousarray(want).reshape(-1).view(np.uint8))


@pytest.mark.parametrize("M", [1, 8, 33])
@pytest.mark.parametrize("act_order", [False, True])
def test_matmul_int4(M, act_order):
    print(f"[case] host MatMulInt4 M={M} act_order={act_order}", flush=True)
    g = synth.rng(400 + M + act_order)
    N, K, G = 80, 1024, 128
    codes, s, z = synth.int4_weight(N, K, G, g)
    x = synth.activations(M, K, g)
    perm = g.permutation(K).astype(np.int64) if act_order else None
    y = L.matmul_int4(dev_t(x, "F32", (M, K)), dev_t(codes, "U32", codes.shape), dev_t(s, "F32", s.shape),
                      dev_t(z, "F32", z.shape), G, None if perm is None else dev_t(perm, "I64", (K,)))
    xg = x[:, perm] if act_order else x
    want = oracle.int4_matmul(np.ascontiguousarray(xg), codes, s, z, N, K, G)
    wd = oracle.int4_dequant(codes, s, z, N, K, G)
    assert norm_err(y.numpy(), want, np.linalg.norm(wd, axis=1), np.linalg.norm(xg, axis=1)) <= TOL


@pytest.mark.parametrize("dt", [hipq.Q4_0, hipq.Q5_0, hipq.Q4_K, hipq.Q5_K, hipq.Q6_K])
@pytest.mark.parametrize("T,E,topk", [(1, 8, 2), (40, 4, 2)])
def test_moe_pipeline(dt, T, E, topk):
    """MoERouteFromIDs -> MoEGemmQ (per-token rows, routing weights) -> MoECombine."""
    print(f"[case] host MoE {NAME[dt]} T={T} E={E} topk={topk}", flush=True)
    g = synth.rng(500 + dt + T)
    N, K = 64, 512
    w = synth.gguf_weight(dt, E * N, K, g)
    ids, tw = synth.moe_routing(T, E, topk, g)
    x = synth.activations(T, K, g)
    r = L.moe_route_from_ids(ids.tolist(), tw.tolist(), T, topk, DEV)
    se, sp = synth.sort_pairs(ids)
    assert np.array_equal(r.sorted_pairs.numpy(), sp) and np.array_equal(r.sorted_expts.numpy(), se)
    pair_out = L.moe_gemm_q(dev_t(x, "F32", (T, K)), dev_t(w, NAME[dt], (E, N, K)), r, r.weights, topk)
    po = pair_out.numpy()
    want = oracle.moe_gemm_q(x, w, dt, E, N, K, sp, se, topk, topk_w=tw)
    wd = oracle.dequant(dt, w, E * N * K).reshape(E, N, K)
    for p in range(T * topk):
        scale = abs(float(tw[p])) * np.linalg.norm(wd[ids[p]], axis=1) * np.linalg.norm(x[p // topk])
        assert np.max(np.abs(po[p] - want[p]) / np.maximum(scale, 1e-30)) <= TOL, p
    out = L.moe_combine(pair_out, topk)
    assert out.shape == [T, N]
    assert np.array_equal(out.numpy().view(np.uint32), oracle.moe_combine(po, topk).view(np.uint32))


@pytest.mark.parametrize("gelu", [False, True])
def test_matmul_q_gated(gelu):
    g = synth.rng(600 + gelu)
    N, K = 300, 2048
    wg = synth.gguf_weight(hipq.Q4_K, N, K, g)
    wu = synth.gguf_weight(hipq.Q4_K, N, K, g)
    x = synth.activations(2, K, g)
    got = L.matmul_q_gated(dev_t(x, "F32", (2, K)), dev_t(wg, "Q4_K", (N, K)), dev_t(wu, "Q4_K", (N, K)), gelu).numpy()
    gr = oracle.matmul_q(x, wg, N, K, hipq.Q4_K)
    ur = oracle.matmul_q(x, wu, N, K, hipq.Q4_K)
    want = oracle.gated(gr, ur, int(gelu))
    xn = np.linalg.norm(x.astype(np.float64), axis=1)[:, None]
    ng = np.linalg.norm(oracle.dequant(hipq.Q4_K, wg, N * K).reshape(N, K).astype(np.float64), axis=1)[None, :]
    nu = np.linalg.norm(oracle.dequant(hipq.Q4_K, wu, N * K).reshape(N, K).astype(np.float64), axis=1)[None, :]
    hg = oracle.gated(gr, np.ones_like(gr), int(gelu)).astype(np.float64)
    bound = TOL * (1.13 * np.abs(ur) * ng * xn + np.abs(hg) * nu * xn) + 1e-30
    assert np.max(np.abs(got - want) / bound) <= 1.0


@pytest.mark.parametrize("gelu", [False, True])
def test_moe_route_and_gated_host(gelu):
    """ops.MoERoute on ROCm, then MoEGemmQGated -> MoEGemmQ (weighted) -> MoECombine."""
    g = synth.rng(700 + gelu)
    T, E, topk, H, I = 3, 32, 4, 512, 256
    logits = g.standard_normal((T, E)).astype(np.float32)
    probs = np.exp(logits - logits.max(axis=1, keepdims=True))
    probs = (probs / probs.sum(axis=1, keepdims=True)).astype(np.float32)
    r = L.moe_route(dev_t(probs, "F32", (T, E)), topk, True)
    rids, rw, rsp, rse = oracle.moe_route(probs, topk, True)
    assert np.array_equal(r.topk_ids.numpy(), rids) and np.array_equal(r.sorted_pairs.numpy(), rsp)
    assert np.array_equal(r.weights.numpy().view(np.uint32), rw.view(np.uint32))
    wgu = synth.gguf_weight(hipq.Q4_K, E * 2 * I, H, g)
    wdn = synth.gguf_weight(hipq.Q4_K, E * H, I, g)
    x = synth.activations(T, H, g)
    h = L.moe_gemm_q_gated(dev_t(x, "F32", (T, H)), dev_t(wgu, "Q4_K", (E, 2 * I, H)), r, topk, gelu)
    assert h.shape == [T * topk, I]
    act = hipq.ACT_GELU_ERF if gelu else hipq.ACT_SILU
    gu = oracle.moe_gemm_q(x, wgu, hipq.Q4_K, E, 2 * I, H, rsp, rse, topk)
    hr = oracle.gated(gu[:, :I], gu[:, I:], act)
    assert np.max(np.abs(h.numpy() - hr)) <= 1e-3 * np.abs(hr).max()
    y = L.moe_combine(L.moe_gemm_q(h, dev_t(wdn, "Q4_K", (E, H, I)), r, r.weights, topk), topk)
    pr = oracle.moe_gemm_q(hr, wdn, hipq.Q4_K, E, H, I, rsp, rse, topk, topk_w=rw)
    want = oracle.moe_combine(pr, topk)
    assert np.max(np.abs(y.numpy() - want)) <= 5e-3 * np.abs(want).max()


@pytest.mark.parametrize("T,E,topk,H,I,G", [(5, 4, 2, 64, 32, 32), (1, 16, 4, 2048, 768, 128)])
def test_moe_int4_host_op(T, E, topk, H, I, G):
    """ops.MoEInt4 through the registry (ROCm "moe_int4") against Light's CPU MoEInt4 restated
    (oracle.moe_int4); the routing comes from ops.MoERouteFromIDs."""
    print(f"[case] host MoEInt4 T={T} E={E} topk={topk} H={H} I={I}", flush=True)
    g = synth.rng(700 + T + H)
    gu = [synth.int4_weight(2 * I, H, G, g) for _ in range(E)]
    dn = [synth.int4_weight(H, I, G, g) for _ in range(E)]
    ids = np.concatenate([g.choice(E, size=topk, replace=False) for _ in range(T)]).astype(np.int64)
    w = g.random(T * topk).astype(np.float32)
    x = g.standard_normal((T, H)).astype(np.float32)
    r = L.moe_route_from_ids(ids.tolist(), w.tolist(), T, topk, DEV)
    wrap = lambda ws: [tuple(dev_t(a, "U32" if a.dtype == np.uint32 else "F32", a.shape) for a in t) for t in ws]
    y = L.moe_int4(dev_t(x, "F32", (T, H)), wrap(gu), wrap(dn), r, topk, G)
    assert y.shape == [T, H] and y.dtype == "F32"
    got = y.numpy()
    want = oracle.moe_int4(x, gu, dn, ids, w, topk, G)
    for t in range(T):
        assert np.max(np.abs(got[t] - want[t])) <= 5e-3 * (np.abs(want[t]).max() + 1e-30), t
