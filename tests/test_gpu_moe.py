"""GPU parity of the MoE grouped expert qmatmul (ops.MoEGemmQ) through the C ABI.

Mirrors TestMoEGemmQCUDAParity (ops/moe_test.go:187-255): per-token input with no
weights and per-pair input with routing weights, against Light's CPU path
(dequantize the expert stack + moeGemmKernel, oracle.moe_gemm_q) and an f64
per-pair oracle.  Bar: max |err| / (w(p) ||W[e(p)]_n|| ||x_row(p)||) <= 1e-3.
Also pins the counts / offsets contract and skipped out-of-range pairs.
"""
import numpy as np
import pytest
import torch

import oracle
from light_amd import hipq, synth

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _run(dev, x, w, dt, E, N, K, ids, tw, topk, weighted, size_m=None):
    se, sp = synth.sort_pairs(ids)
    M = ids.size
    xt = _t(x, dev)
    out = torch.zeros((size_m or M, N), device=dev)
    counts = torch.zeros(E, dtype=torch.int32, device=dev)
    offsets = torch.zeros(E + 1, dtype=torch.int32, device=dev)
    hipq.moe_gemm_q(xt, _t(w, dev), _t(sp, dev), _t(se, dev), E, N, K, dt, topk,
                    topk_w=_t(tw, dev) if weighted else None, out=out, counts=counts, offsets=offsets)
    torch.cuda.synchronize()
    return out.cpu().numpy(), counts.cpu().numpy(), offsets.cpu().numpy(), se, sp


def _check(dev, x, w, dt, E, N, K, ids, tw, topk, weighted, sample=None):
    M = ids.size
    print(f"[case] moe dt={hipq.NAMES[dt]} E={E} N={N} K={K} M={M} rows={x.shape[0]} weighted={weighted}", flush=True)
    got, counts, offsets, se, sp = _run(dev, x, w, dt, E, N, K, ids, tw, topk, weighted)
    assert np.array_equal(counts, np.bincount(ids, minlength=E))
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(np.bincount(ids, minlength=E))]))
    cpu = oracle.moe_gemm_q(x, w, dt, E, N, K, sp, se, topk, topk_w=tw if weighted else None)
    wd = oracle.dequant(dt, w, E * N * K).reshape(E, N, K)
    pairs = range(M) if sample is None else sample
    rpp = x.shape[0] == M
    for p in pairs:
        r = p if rpp else p // topk
        e = ids[p]
        scale = float(tw[p]) if weighted else 1.0
        ref = wd[e].astype(np.float64) @ x[r].astype(np.float64) * scale
        norm = abs(scale) * np.linalg.norm(wd[e].astype(np.float64), axis=1) * np.linalg.norm(x[r].astype(np.float64))
        norm = np.maximum(norm, 1e-30)
        assert np.max(np.abs(got[p] - ref) / norm) <= TOL, f"pair {p} vs f64"
        assert np.max(np.abs(got[p] - cpu[p]) / norm) <= TOL, f"pair {p} vs Light CPU"
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("dt", [hipq.Q4_K, hipq.Q8_0, hipq.Q6_K, hipq.Q4_0, hipq.Q5_0, hipq.Q5_K])
@pytest.mark.parametrize("E", [3, 16])  # E=3: 42 pairs > 4E -> MFMA path for Q4_K; E=16: grouped GEMV
@pytest.mark.parametrize("weighted", [False, True])
def test_moe_gemm_q_light_shapes(dev, dt, E, weighted):
    """TestMoEGemmQCUDAParity shapes: T=21, K=256, N=40, topk=2."""
    g = synth.rng(7 + E + dt)
    T, K, N, topk = 21, 256, 40, 2
    w = synth.gguf_weight(dt, E * N, K, g)
    ids, tw = synth.moe_routing(T, E, topk, g)
    rows = T * topk if weighted else T
    x = (g.standard_normal((rows, K)) * 0.4).astype(np.float32)
    _check(dev, x, w, dt, E, N, K, ids, tw, topk, weighted)


@pytest.mark.parametrize("T,E,topk,N,K", [(1, 8, 2, 64, 512), (5, 32, 4, 300, 1024), (64, 16, 2, 128, 2048),
                                          (33, 64, 8, 256, 768), (200, 8, 2, 96, 256),
                                          # decode kernel: several chunks of pairs per expert; K=4096
                                          # (one-wave teams); K=5120 (falls back to the act GEMV)
                                          (13, 4, 1, 72, 512), (3, 8, 2, 128, 4096), (2, 4, 2, 40, 5120)])
def test_moe_gemm_q4_k_shapes(dev, T, E, topk, N, K):
    g = synth.rng(T * 13 + E + N + K)
    w = synth.gguf_weight(hipq.Q4_K, E * N, K, g)
    ids, tw = synth.moe_routing(T, E, topk, g)
    x = g.standard_normal((T, K)).astype(np.float32)
    _check(dev, x, w, hipq.Q4_K, E, N, K, ids, tw, topk, False)
    xp = g.standard_normal((T * topk, K)).astype(np.float32)
    _check(dev, xp, w, hipq.Q4_K, E, N, K, ids, tw, topk, True)


def test_moe_pairs_outside_size_m_are_skipped(dev):
    """Pairs p >= size_m leave the output untouched (kernels/cuda/moe.go:115, moe_gguf.cu:62)."""
    g = synth.rng(3)
    T, E, topk, N, K = 6, 4, 2, 32, 256
    w = synth.gguf_weight(hipq.Q4_K, E * N, K, g)
    ids, tw = synth.moe_routing(T, E, topk, g)
    x = g.standard_normal((T, K)).astype(np.float32)
    size_m = 7  # only pairs 0..6 of 12 land in the output
    se, sp = synth.sort_pairs(ids)
    out = torch.full((size_m, N), 0.0, device=dev)
    hipq.moe_gemm_q(_t(x, dev), _t(w, dev), _t(sp, dev), _t(se, dev), E, N, K, hipq.Q4_K, topk, out=out)
    full, *_ = _run(dev, x, w, hipq.Q4_K, E, N, K, ids, tw, topk, False)
    assert torch.equal(out.cpu(), torch.from_numpy(full[:size_m]))


@pytest.mark.parametrize("T", [1, 256])
def test_moe_benchmark_configs(dev, T):
    """Qwen3-30B-A3B-like: E=128, topk=8, H=2048, I=768; gate/up per token, down per pair weighted."""
    c = synth.CONFIGS[f"moe_q4_k_t{T}"]
    g = synth.rng(c["cfg"])
    E, topk, H, I = c["E"], c["topk"], c["H"], c["I"]
    wgu = synth.gguf_weight(hipq.Q4_K, E * 2 * I, H, g)
    wdn = synth.gguf_weight(hipq.Q4_K, E * H, I, g)
    ids, tw = synth.moe_routing(T, E, topk, g)
    x = g.standard_normal((T, H)).astype(np.float32)
    h = g.standard_normal((T * topk, I)).astype(np.float32)
    sample = None if T == 1 else list(range(0, T * topk, 37))
    _check(dev, x, wgu, hipq.Q4_K, E, 2 * I, H, ids, tw, topk, False, sample=sample)
    _check(dev, h, wdn, hipq.Q4_K, E, H, I, ids, tw, topk, True, sample=sample)
