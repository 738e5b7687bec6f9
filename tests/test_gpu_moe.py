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


def _moe_norm(wd_rows, ids, w, h):
    """The north-star normaliser of a combined MoE output: for token t and output n,
    sum over its slots j of |w_j| * ||W_dn[e_j]_n|| * ||h_j||  (wd_rows: (E, N) row norms of the
    dequantized down experts; ids, w: (T * topk); h: (T * topk, I))."""
    hn = np.linalg.norm(np.asarray(h, dtype=np.float64), axis=1)
    per_pair = np.abs(np.asarray(w, dtype=np.float64))[:, None] * wd_rows[ids.reshape(-1)] * hn[:, None]
    return per_pair


def _moe_bar(got, want, wd_rows, ids, w, h, topk, tol=1e-3):
    """max over (t, n) of |got - want| / sum_j |w_j| ||W_dn[e_j]_n|| ||h_j|| <= tol."""
    per_pair = _moe_norm(wd_rows, ids, w, h)
    T = per_pair.shape[0] // topk
    norm = per_pair.reshape(T, topk, -1).sum(axis=1) + 1e-30
    err = np.max(np.abs(np.asarray(got, dtype=np.float64) - np.asarray(want, dtype=np.float64)) / norm)
    assert err <= tol, f"max normalised error {err:.3g} > {tol}"
    return err


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
                                          (13, 4, 1, 72, 512), (3, 8, 2, 128, 4096), (2, 4, 2, 40, 5120),
                                          # MFMA path with N % 16 != 0: the tiled grouped GEMM
                                          (64, 4, 2, 200, 512)])
def test_moe_gemm_q4_k_shapes(dev, T, E, topk, N, K):
    g = synth.rng(T * 13 + E + N + K)
    w = synth.gguf_weight(hipq.Q4_K, E * N, K, g)
    ids, tw = synth.moe_routing(T, E, topk, g)
    x = g.standard_normal((T, K)).astype(np.float32)
    _check(dev, x, w, hipq.Q4_K, E, N, K, ids, tw, topk, False)
    xp = g.standard_normal((T * topk, K)).astype(np.float32)
    _check(dev, xp, w, hipq.Q4_K, E, N, K, ids, tw, topk, True)


@pytest.mark.parametrize("big", [1e5, 3e7])
def test_moe_grouped_gemm_rows_beyond_f16_range(dev, big):
    """The grouped MFMA path (more than 4 pairs per expert) runs on f16 x with a power-of-two
    scale per row: rows whose |x| exceeds the f16 range (65504) must not clip.  Rows 0 and 3
    carry outliers of `big`; every pair is checked against the f64 oracle at the 1e-3 bar."""
    g = synth.rng(int(big) % 1000 + 11)
    T, E, topk, N, K = 40, 4, 2, 96, 512
    w = synth.gguf_weight(hipq.Q4_K, E * N, K, g)
    ids, tw = synth.moe_routing(T, E, topk, g)
    x = g.standard_normal((T, K)).astype(np.float32)
    x[0, 5] = big
    x[3] *= np.float32(big / 4)
    _check(dev, x, w, hipq.Q4_K, E, N, K, ids, tw, topk, False)
    xp = g.standard_normal((T * topk, K)).astype(np.float32)
    xp[7] *= np.float32(big)
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
    sample = None if T == 1 else list(range(0, T * topk, 8))
    _check(dev, x, wgu, hipq.Q4_K, E, 2 * I, H, ids, tw, topk, False, sample=sample)
    _check(dev, h, wdn, hipq.Q4_K, E, H, I, ids, tw, topk, True, sample=sample)


# ---- MoERoute on the device ---------------------------------------------

def _probs(g, T, E, ties):
    logits = g.standard_normal((T, E)).astype(np.float32)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p = (p / p.sum(axis=1, keepdims=True)).astype(np.float32)
    if ties and E > 1:  # (one expert: nothing to tie)
        p[:, E // 2] = p[:, 0]
        p[:, E - 1] = p[:, 1]
    return p


@pytest.mark.parametrize("T,E,topk", [(1, 128, 8), (1, 8, 2), (5, 60, 60), (64, 128, 8), (65, 128, 8),
                                      (300, 256, 8), (2048, 128, 8), (3, 1000, 4)])
@pytest.mark.parametrize("normalize", [False, True])
def test_moe_route_bit_exact(dev, T, E, topk, normalize):
    """hq_moe_route against Light's CPU MoERoute (TopK, Sum, Div, Sort): ids, weights and the
    sorted pairs bit for bit, and counts / offsets as moe_gemm_q's scratch."""
    print(f"[case] moe_route T={T} E={E} topk={topk} normalize={normalize}", flush=True)
    g = synth.rng(T * 7 + E + topk)
    probs = _probs(g, T, E, ties=True)
    counts = torch.full((E,), -1, dtype=torch.int32, device=dev)
    offsets = torch.full((E + 1,), -1, dtype=torch.int32, device=dev)
    ids, w, sp, se = hipq.moe_route(_t(probs, dev), topk, normalize, counts=counts, offsets=offsets)
    torch.cuda.synchronize()
    rids, rw, rsp, rse = oracle.moe_route(probs, topk, normalize)
    assert np.array_equal(ids.cpu().numpy(), rids)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), rw.view(np.uint32))
    assert np.array_equal(sp.cpu().numpy(), rsp) and np.array_equal(se.cpu().numpy(), rse)
    bc = np.bincount(rids.reshape(-1), minlength=E)
    assert np.array_equal(counts.cpu().numpy(), bc)
    assert np.array_equal(offsets.cpu().numpy(), np.concatenate([[0], np.cumsum(bc)]))


@pytest.mark.parametrize("M,E", [(1, 1), (16, 4), (1000, 128), (16384, 128), (777, 1000)])
def test_moe_sort_ids(dev, M, E):
    """MoERouteFromIDs' Sort on the device: stable ascending, against the oracle's counting sort."""
    g = synth.rng(M + E)
    ids = g.integers(0, E, size=M).astype(np.int64)
    counts = torch.zeros(E, dtype=torch.int32, device=dev)
    offsets = torch.zeros(E + 1, dtype=torch.int32, device=dev)
    sp, se = hipq.moe_sort_ids(_t(ids, dev), E, counts=counts, offsets=offsets)
    rse, rsp = oracle.moe_route_from_ids(ids)
    assert np.array_equal(sp.cpu().numpy(), rsp) and np.array_equal(se.cpu().numpy(), rse)
    assert np.array_equal(counts.cpu().numpy(), np.bincount(ids, minlength=E))


def test_moe_route_limits(dev):
    probs = torch.rand((4, 8), device=dev)
    with pytest.raises(hipq.HipqError, match="topk 9 out of range"):
        hipq.moe_route(probs, 9)
    with pytest.raises(hipq.HipqError, match="beyond the one-workgroup sort"):
        hipq.moe_route(torch.rand((1, 2000), device=dev), 2)


# ---- routed gated gate/up ---------------------------------------------------

def _check_gated(dev, dt, T, E, topk, I, K, act, rpp=False):
    print(f"[case] moe_gated dt={hipq.NAMES[dt]} T={T} E={E} topk={topk} I={I} K={K} act={act} rpp={rpp}",
          flush=True)
    g = synth.rng(T * 31 + E + I + K + dt + act)
    w = synth.gguf_weight(dt, E * 2 * I, K, g)
    ids, tw = synth.moe_routing(T, E, topk, g)
    se, sp = synth.sort_pairs(ids)
    rows = T * topk if rpp else T
    x = g.standard_normal((rows, K)).astype(np.float32)
    got = hipq.moe_gemm_q_gated(_t(x, dev), _t(w, dev), _t(sp, dev), _t(se, dev), E, I, K, dt, topk, act=act)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    gu = oracle.moe_gemm_q(x, w, dt, E, 2 * I, K, sp, se, topk)
    want = oracle.gated(gu[:, :I], gu[:, I:], act)
    wd = oracle.dequant(dt, w, E * 2 * I * K).reshape(E, 2 * I, K).astype(np.float64)
    M = T * topk
    for p in range(M):
        r = p if rpp else p // topk
        xn = np.linalg.norm(x[r].astype(np.float64))
        ng = np.linalg.norm(wd[ids[p], :I], axis=1) * xn
        nu = np.linalg.norm(wd[ids[p], I:], axis=1) * xn
        hg = oracle.gated(gu[p:p + 1, :I], np.ones((1, I), np.float32), act)[0].astype(np.float64)
        bound = TOL * (1.13 * np.abs(gu[p, I:]) * ng + np.abs(hg) * nu) + 1e-30
        err = np.abs(got[p].astype(np.float64) - want[p]) / bound
        assert err.max() <= 1.0, f"pair {p}: {err.max():.3g}"


@pytest.mark.parametrize("act", [hipq.ACT_SILU, hipq.ACT_GELU_ERF])
def test_moe_gated_decode_config(dev, act):
    """Qwen3-30B-A3B-like decode: E=128, topk=8, H=2048, I=768 -- one fused launch."""
    _check_gated(dev, hipq.Q4_K, 1, 128, 8, 768, 2048, act)


@pytest.mark.parametrize("dt,T,E,topk,I,K,rpp", [(hipq.Q4_K, 5, 16, 4, 96, 512, False),
                                                 (hipq.Q5_K, 3, 8, 2, 64, 1024, True),
                                                 (hipq.Q4_K, 40, 4, 2, 64, 256, False),   # M > 4E: MFMA, gated epilogue
                                                 (hipq.Q4_K, 60, 4, 2, 96, 512, True),    # ragged gate/up tile, rpp
                                                 (hipq.Q4_K, 256, 32, 8, 768, 2048, False),  # configs[4] T = 256
                                                 (hipq.Q8_0, 4, 8, 2, 48, 256, False),    # generic + split
                                                 (hipq.Q4_K, 2, 4, 2, 32, 5120, False),  # K > 4096: fallback
                                                 (hipq.Q4_K, 64, 4, 2, 40, 512, False)])  # I % 16 != 0: tiled GEMM
def test_moe_gated_shapes(dev, dt, T, E, topk, I, K, rpp):
    _check_gated(dev, dt, T, E, topk, I, K, hipq.ACT_SILU, rpp)


def test_moe_decode_pipeline_on_device(dev):
    """Router probs -> hq_moe_route -> gated gate/up -> down (weighted) -> combine, all on the
    device, against Light's CPU chain (MoERoute, MoEGemmQ, SiLU * up, MoEGemmQ, MoECombine)."""
    T, E, topk, H, I = 2, 64, 8, 1024, 512
    g = synth.rng(77)
    wgu = synth.gguf_weight(hipq.Q4_K, E * 2 * I, H, g)
    wdn = synth.gguf_weight(hipq.Q4_K, E * H, I, g)
    x = g.standard_normal((T, H)).astype(np.float32)
    probs = _probs(g, T, E, ties=False)
    ids, w, sp, se = hipq.moe_route(_t(probs, dev), topk, True)
    h = hipq.moe_gemm_q_gated(_t(x, dev), _t(wgu, dev), sp, se, E, I, H, hipq.Q4_K, topk)
    pair = hipq.moe_gemm_q(h, _t(wdn, dev), sp, se, E, H, I, hipq.Q4_K, topk, topk_w=w)
    y = hipq.moe_combine(pair, topk).cpu().numpy()
    rids, rw, rsp, rse = oracle.moe_route(probs, topk, True)
    gu = oracle.moe_gemm_q(x, wgu, hipq.Q4_K, E, 2 * I, H, rsp, rse, topk)
    hr = oracle.gated(gu[:, :I], gu[:, I:], hipq.ACT_SILU)
    pr = oracle.moe_gemm_q(hr, wdn, hipq.Q4_K, E, H, I, rsp, rse, topk, topk_w=rw)
    want = oracle.moe_combine(pr, topk)
    wd_rows = np.linalg.norm(oracle.dequant(hipq.Q4_K, wdn, E * H * I).reshape(E, H, I).astype(np.float64), axis=2)
    _moe_bar(y, want, wd_rows, rids.reshape(-1), rw, hr, topk)


@pytest.mark.parametrize("dt,T,E,topk,H,I,weighted", [
    (hipq.Q4_K, 1, 128, 8, 2048, 768, True),     # Qwen3-30B-A3B-like decode (configs[4], T = 1)
    (hipq.Q4_K, 3, 128, 8, 2048, 768, True),
    (hipq.Q5_K, 2, 64, 4, 1024, 512, True),
    (hipq.Q4_K, 5, 16, 2, 512, 2048, False),     # K = 2048: two-wave-row teams
    (hipq.Q4_K, 2, 8, 4, 256, 4096, True),       # K = 4096: one team per wave
    (hipq.Q8_0, 2, 16, 4, 512, 256, True),       # no fused kernel: gemm + combine through ws
])
def test_moe_down_combine_bit_exact(dev, dt, T, E, topk, H, I, weighted):
    """hq_moe_gemm_q_combine equals hq_moe_gemm_q followed by hq_moe_combine bit for bit, and
    Light's CPU chain (MoEGemmQ, MoECombine) within the bar; counts / offsets as moe_gemm_q."""
    print(f"[case] moe down+combine dt={hipq.NAMES[dt]} T={T} E={E} topk={topk} H={H} I={I}", flush=True)
    g = synth.rng(900 + T + topk + dt)
    wdn = synth.gguf_weight(dt, E * H, I, g)
    ids, tw = synth.moe_routing(T, E, topk, g)
    se, sp = synth.sort_pairs(ids)
    h = synth.activations(T * topk, I, g)
    wt, ht, spt, set_, twt = _t(wdn, dev), _t(h, dev), _t(sp, dev), _t(se, dev), _t(tw, dev)
    kw = dict(topk_w=twt if weighted else None)
    pair = hipq.moe_gemm_q(ht, wt, spt, set_, E, H, I, dt, topk, **kw)
    want = hipq.moe_combine(pair, topk)
    counts = torch.full((E,), -7, dtype=torch.int32, device=dev)
    offsets = torch.full((E + 1,), -7, dtype=torch.int32, device=dev)
    got = hipq.moe_gemm_q_combine(ht, wt, spt, set_, E, H, I, dt, topk, counts=counts, offsets=offsets, **kw)
    torch.cuda.synchronize()
    assert torch.equal(got, want), f"max diff {(got - want).abs().max().item():.3g}"
    bc = np.bincount(ids.ravel(), minlength=E)
    assert np.array_equal(counts.cpu().numpy(), bc)
    assert np.array_equal(offsets.cpu().numpy(), np.concatenate([[0], np.cumsum(bc)]))
    pr = oracle.moe_gemm_q(h, wdn, dt, E, H, I, sp, se, topk, topk_w=tw if weighted else None)
    ref = oracle.moe_combine(pr, topk)
    wd_rows = np.linalg.norm(oracle.dequant(dt, wdn, E * H * I).reshape(E, H, I).astype(np.float64), axis=2)
    tw_used = tw.reshape(-1) if weighted else np.ones(T * topk, dtype=np.float32)
    _moe_bar(got.cpu().numpy(), ref, wd_rows, ids.reshape(-1), tw_used, h, topk)


@pytest.mark.parametrize("dt,T,E,topk", [(hipq.Q4_K, 64, 16, 2), (hipq.Q8_0, 3, 16, 4), (hipq.Q4_K, 1, 128, 8)])
def test_moe_down_combine_without_scratch_buffers(dev, dt, T, E, topk):
    """counts / offsets are optional: the unfused path (here the grouped MFMA GEMM at M > 4E,
    or a format without the fused kernel) keeps them in its workspace."""
    print(f"[case] moe down+combine no counts dt={hipq.NAMES[dt]} T={T} E={E} topk={topk}", flush=True)
    H, I = 256, 512
    g = synth.rng(1200 + T + dt)
    wdn = synth.gguf_weight(dt, E * H, I, g)
    ids, tw = synth.moe_routing(T, E, topk, g)
    se, sp = synth.sort_pairs(ids)
    h = synth.activations(T * topk, I, g)
    wt, ht, spt, set_, twt = _t(wdn, dev), _t(h, dev), _t(sp, dev), _t(se, dev), _t(tw, dev)
    want = hipq.moe_combine(hipq.moe_gemm_q(ht, wt, spt, set_, E, H, I, dt, topk, topk_w=twt), topk)
    got = hipq.moe_gemm_q_combine(ht, wt, spt, set_, E, H, I, dt, topk, topk_w=twt)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("dt,T,E,topk,H,I,ties", [
    (hipq.Q4_K, 1, 128, 8, 2048, 768, False),    # configs[4] decode
    (hipq.Q4_K, 3, 128, 8, 2048, 768, True),
    (hipq.Q5_K, 8, 8, 4, 1024, 512, False),      # experts shared across tokens: fewer segments than slots
    (hipq.Q4_K, 2, 64, 2, 4096, 256, True),      # K = 4096
    (hipq.Q8_0, 2, 16, 4, 512, 256, False),      # no fused kernel: route, then the gated op
])
def test_moe_route_gated_bit_exact(dev, dt, T, E, topk, H, I, ties):
    """hq_moe_route_gated equals hq_moe_route + hq_moe_gemm_q_gated bit for bit (routing
    outputs, counts / offsets and h)."""
    print(f"[case] moe route+gated dt={hipq.NAMES[dt]} T={T} E={E} topk={topk} H={H} I={I}", flush=True)
    g = synth.rng(1500 + T + E + dt)
    wgu = _t(synth.gguf_weight(dt, E * 2 * I, H, g), dev)
    x = _t(synth.activations(T, H, g), dev)
    probs = _t(_probs(g, T, E, ties=ties), dev)
    c0 = torch.zeros(E, dtype=torch.int32, device=dev)
    o0 = torch.zeros(E + 1, dtype=torch.int32, device=dev)
    ids, w, sp, se = hipq.moe_route(probs, topk, True)
    h0 = hipq.moe_gemm_q_gated(x, wgu, sp, se, E, I, H, dt, topk, counts=c0, offsets=o0)
    c1 = torch.full((E,), -5, dtype=torch.int32, device=dev)
    o1 = torch.full((E + 1,), -5, dtype=torch.int32, device=dev)
    ids1, w1, sp1, se1, h1 = hipq.moe_route_gated(probs, x, wgu, E, I, H, dt, topk, counts=c1, offsets=o1)
    torch.cuda.synchronize()
    for a, b, name in ((ids, ids1, "ids"), (w, w1, "weights"), (sp, sp1, "sorted_pairs"), (se, se1, "sorted_expts"),
                       (c0, c1, "counts"), (o0, o1, "offsets"), (h0, h1, "h")):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("dt,T,E,topk,H,I", [
    (hipq.Q4_K, 1, 128, 8, 2048, 768),   # configs[4] decode: the one-launch block
    (hipq.Q5_K, 1, 64, 4, 1024, 512),
    (hipq.Q4_K, 1, 16, 2, 4096, 256),    # K = 4096 gate/up, few pairs
    (hipq.Q4_K, 3, 128, 8, 2048, 768),   # several tokens: the two launches
    (hipq.Q8_0, 1, 16, 4, 512, 256),     # no fused kernel
])
def test_moe_block_equals_route_gated_then_combine(dev, dt, T, E, topk, H, I):
    """hq_moe_block_q equals hq_moe_route_gated followed by hq_moe_gemm_q_combine bit for bit:
    y, h, the routing outputs and counts / offsets -- in one launch (T = 1) as in two.  Three
    calls in a row (the grid barrier's state carries over between launches) all agree."""
    print(f"[case] moe block dt={hipq.NAMES[dt]} T={T} E={E} topk={topk} H={H} I={I}", flush=True)
    g = synth.rng(1700 + T + E + dt)
    wgu = _t(synth.gguf_weight(dt, E * 2 * I, H, g), dev)
    wdn = _t(synth.gguf_weight(dt, E * H, I, g), dev)
    x = _t(synth.activations(T, H, g), dev)
    probs = _t(_probs(g, T, E, ties=False), dev)
    c0 = torch.zeros(E, dtype=torch.int32, device=dev)
    o0 = torch.zeros(E + 1, dtype=torch.int32, device=dev)
    ids, w, sp, se, h = hipq.moe_route_gated(probs, x, wgu, E, I, H, dt, topk, counts=c0, offsets=o0)
    y = hipq.moe_gemm_q_combine(h, wdn, sp, se, E, H, I, dt, topk, topk_w=w)
    for rep in range(3):
        c1 = torch.full((E,), -5, dtype=torch.int32, device=dev)
        o1 = torch.full((E + 1,), -5, dtype=torch.int32, device=dev)
        y1, ids1, w1, sp1, se1, h1 = hipq.moe_block_q(probs, x, wgu, wdn, E, H, I, dt, topk, counts=c1, offsets=o1)
        torch.cuda.synchronize()
        for a, b, name in ((y, y1, "y"), (h, h1, "h"), (ids, ids1, "ids"), (w, w1, "weights"),
                           (sp, sp1, "sorted_pairs"), (se, se1, "sorted_expts"), (c0, c1, "counts"),
                           (o0, o1, "offsets")):
            assert torch.equal(a, b), (name, rep)


@pytest.mark.parametrize("caller_counts", [True, False])
def test_moe_block_grouped_gemm_path_equals_separate_calls(dev, caller_counts):
    """Past 4 E pairs the block runs the grouped MFMA GEMMs on the route's counts / offsets,
    with no offsets pass and no zeroing (every pair of the route is in one expert segment).
    Bit for bit equal to moe_route, moe_gemm_q_gated and moe_gemm_q_combine called separately
    (each with its own offsets pass), with h and the workspace NaN-filled, with the caller's
    counts / offsets and with the workspace's."""
    dt, T, E, topk, H, I = hipq.Q4_K, 80, 128, 8, 2048, 768
    print(f"[case] moe block grouped path T={T} E={E} caller_counts={caller_counts}", flush=True)
    g = synth.rng(1790 + int(caller_counts))
    wgu = _t(synth.gguf_weight(dt, E * 2 * I, H, g), dev)
    wdn = _t(synth.gguf_weight(dt, E * H, I, g), dev)
    x = _t(synth.activations(T, H, g), dev)
    probs = _t(_probs(g, T, E, ties=False), dev)
    ids, w, sp, se = hipq.moe_route(probs, topk)
    h = hipq.moe_gemm_q_gated(x, wgu, sp, se, E, I, H, dt, topk)
    y = hipq.moe_gemm_q_combine(h, wdn, sp, se, E, H, I, dt, topk, topk_w=w)
    nb = hipq.lib().hq_moe_block_q_ws_bytes(T, topk, E, H, I, dt)
    ws = torch.full((nb // 4 + 1,), float("nan"), dtype=torch.float32, device=dev)
    for rep in range(2):
        h1 = torch.full((T * topk, I), float("nan"), dtype=torch.float32, device=dev)
        c1 = torch.full((E,), -5, dtype=torch.int32, device=dev) if caller_counts else None
        o1 = torch.full((E + 1,), -5, dtype=torch.int32, device=dev) if caller_counts else None
        y1, ids1, w1, sp1, se1, h1 = hipq.moe_block_q(probs, x, wgu, wdn, E, H, I, dt, topk, h=h1, counts=c1,
                                                      offsets=o1, ws=ws)
        torch.cuda.synchronize()
        for a, b, name in ((y, y1, "y"), (h, h1, "h"), (ids, ids1, "ids"), (w, w1, "weights"),
                           (sp, sp1, "sorted_pairs"), (se, se1, "sorted_expts")):
            assert torch.equal(a, b), (name, rep)
        if caller_counts:
            cnt = torch.bincount(se, minlength=E).to(torch.int32)
            assert torch.equal(c1, cnt)
            assert torch.equal(o1, torch.cat([torch.zeros(1, dtype=torch.int32, device=dev),
                                              torch.cumsum(cnt, 0).to(torch.int32)]))


@pytest.mark.parametrize("T,N,topk", [(256, 2048, 8), (3, 4096, 1), (5, 1024, 3), (2, 512, 9), (4, 1026, 8)])
def test_moe_combine_bit_exact(dev, T, N, topk):
    """MoECombine (ops/moe.go:209-240): y[t] = pair[t, 0] + pair[t, 1] + ... in slot order, bit
    for bit against the oracle's sequential sum, for pair values spread over 2^-8 .. 2^8, at
    the T = 256 shape and at small, odd and topk > 8 ones."""
    print(f"[case] moe_combine T={T} N={N} topk={topk}", flush=True)
    g = synth.rng(1900 + T + topk)
    pr = (g.standard_normal((T * topk, N)) * np.exp(g.uniform(-8, 8, (T * topk, 1)))).astype(np.float32)
    y = hipq.moe_combine(_t(pr, dev), topk).cpu().numpy()
    want = oracle.moe_combine(pr, topk)
    assert np.array_equal(y.view(np.uint32), np.asarray(want, dtype=np.float32).view(np.uint32))


def test_moe_block_second_stream_and_changing_routes(dev):
    """The one-launch block on its stream and the two-launch path on another stream agree with
    the separate calls, for routings that change from call to call."""
    print("[case] moe block, two streams, 6 routings", flush=True)
    dt, E, topk, H, I = hipq.Q4_K, 128, 8, 2048, 768
    g = synth.rng(1777)
    wgu = _t(synth.gguf_weight(dt, E * 2 * I, H, g), dev)
    wdn = _t(synth.gguf_weight(dt, E * H, I, g), dev)
    x = _t(synth.activations(1, H, g), dev)
    other = torch.cuda.Stream(device=dev)
    for i in range(6):
        probs = _t(_probs(g, 1, E, ties=False), dev)
        ids, w, sp, se, h = hipq.moe_route_gated(probs, x, wgu, E, I, H, dt, topk)
        want = hipq.moe_gemm_q_combine(h, wdn, sp, se, E, H, I, dt, topk, topk_w=w)
        got = hipq.moe_block_q(probs, x, wgu, wdn, E, H, I, dt, topk)[0]
        with torch.cuda.stream(other):
            got2 = hipq.moe_block_q(probs, x, wgu, wdn, E, H, I, dt, topk, stream=other)[0]
        torch.cuda.synchronize()
        assert torch.equal(got, want), i
        assert torch.equal(got2, want), i


def test_moe_grouped_gemm_pairs_routed_nowhere(dev):
    """Pairs whose expert id is outside [0, E) contribute zero rows, in the grouped MFMA paths
    that zero only the rows no valid pair writes: the gated gate/up (h rows of such pairs are
    0 even in a NaN-filled output) and the down + combine (equal bit for bit to moe_gemm_q into
    a zeroed output followed by moe_combine, with a NaN-filled workspace)."""
    print("[case] moe grouped GEMM, pairs routed nowhere", flush=True)
    g = synth.rng(2024)
    T, E, topk, H, I = 48, 4, 2, 512, 256  # M = 96 > 4 E: the grouped MFMA GEMM
    ids, tw = synth.moe_routing(T, E, topk, g)
    ids = ids.copy()
    bad = [3, 17, 50, 95]
    ids.reshape(-1)[bad] = [E, -1, E + 5, E]
    se, sp = synth.sort_pairs(ids)
    wgu = _t(synth.gguf_weight(hipq.Q4_K, E * 2 * I, H, g), dev)
    wdn = _t(synth.gguf_weight(hipq.Q4_K, E * H, I, g), dev)
    x = _t(synth.activations(T, H, g), dev)
    spt, set_, twt = _t(sp, dev), _t(se, dev), _t(tw, dev)
    hz = hipq.moe_gemm_q_gated(x, wgu, spt, set_, E, I, H, hipq.Q4_K, topk,
                               out=torch.zeros((T * topk, I), device=dev))
    hn = hipq.moe_gemm_q_gated(x, wgu, spt, set_, E, I, H, hipq.Q4_K, topk,
                               out=torch.full((T * topk, I), float("nan"), device=dev))
    torch.cuda.synchronize()
    assert torch.equal(hz, hn)
    assert torch.all(hn[bad] == 0)
    h = _t(synth.activations(T * topk, I, g), dev)
    want = hipq.moe_combine(hipq.moe_gemm_q(h, wdn, spt, set_, E, H, I, hipq.Q4_K, topk, topk_w=twt,
                                            out=torch.zeros((T * topk, H), device=dev)), topk)
    nb = hipq.lib().hq_moe_gemm_q_combine_ws_bytes(T, topk, E, H, I, hipq.Q4_K)
    ws = torch.full((nb // 4 + 1,), float("nan"), device=dev)
    got = hipq.moe_gemm_q_combine(h, wdn, spt, set_, E, H, I, hipq.Q4_K, topk, topk_w=twt, ws=ws)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_moe_block_barrier_gives_up_loudly(dev):
    """The one-launch block's grid barrier is a bounded wait.  With the host's test hook set
    to give up at once (every workgroup still arrives, gives up and exits normally), the
    call's y is all NaN, the next hq_moe_block_q on the device returns HQ_EBARRIER without
    launching, later calls take the two launches, and hq_moe_block_q_check reports a failure
    after synchronizing.  Restoring the limit re-enables the one launch, whose results then
    equal the separate calls bit for bit (the barrier state stayed consistent)."""
    print("[case] moe block barrier give-up (spin limit 0)", flush=True)
    dt, E, topk, H, I = hipq.Q4_K, 128, 8, 2048, 768
    g = synth.rng(1811)
    wgu = _t(synth.gguf_weight(dt, E * 2 * I, H, g), dev)
    wdn = _t(synth.gguf_weight(dt, E * H, I, g), dev)
    x = _t(synth.activations(1, H, g), dev)
    probs = _t(_probs(g, 1, E, ties=False), dev)
    ids, w, sp, se, h = hipq.moe_route_gated(probs, x, wgu, E, I, H, dt, topk)
    want = hipq.moe_gemm_q_combine(h, wdn, sp, se, E, H, I, dt, topk, topk_w=w)
    try:
        hipq.debug_moe_block_spin_limit(0)
        y0 = hipq.moe_block_q(probs, x, wgu, wdn, E, H, I, dt, topk)[0]
        torch.cuda.synchronize()
        assert bool(torch.isnan(y0).all()), "a block whose barrier gave up must not return numbers"
        with pytest.raises(hipq.HipqError) as ei:
            hipq.moe_block_q(probs, x, wgu, wdn, E, H, I, dt, topk)
        assert ei.value.code == hipq.HQ_EBARRIER, ei.value
        assert "grid barrier" in str(ei.value)
        # Reported once; the device now takes the two launches (spin limit still 0).
        y1 = hipq.moe_block_q(probs, x, wgu, wdn, E, H, I, dt, topk)[0]
        hipq.moe_block_q_check()
        assert torch.equal(y1, want)
        # Re-enabled with the limit still 0: the failure is reported by the check call too.
        hipq.debug_moe_block_spin_limit(0)
        y2 = hipq.moe_block_q(probs, x, wgu, wdn, E, H, I, dt, topk)[0]
        with pytest.raises(hipq.HipqError) as ei:
            hipq.moe_block_q_check()
        assert ei.value.code == hipq.HQ_EBARRIER
        assert bool(torch.isnan(y2).all())
        hipq.moe_block_q_check()  # reported once
    finally:
        hipq.debug_moe_block_spin_limit()
    for _ in range(2):
        y3 = hipq.moe_block_q(probs, x, wgu, wdn, E, H, I, dt, topk)[0]
        hipq.moe_block_q_check()
        assert torch.equal(y3, want)


@pytest.mark.parametrize("dt", [hipq.Q4_K, hipq.Q8_0])
@pytest.mark.parametrize("T", [3, 64])
def test_moe_out_of_range_expert_ids_are_skipped(dev, dt, T):
    """Expert ids outside [0, E) in a sorted routing (-1 before, E after the valid ones) form no
    expert segment: those pairs read no weights, and every valid pair's row equals the run
    without them (the grouped kernels index experts only through the counts / offsets of
    [0, E), and the segment-search GEMV skips a segment whose expert is out of range)."""
    print(f"[case] moe out-of-range ids dt={hipq.NAMES[dt]} T={T}", flush=True)
    g = synth.rng(40 + T + dt)
    E, topk, N, K = 8, 2, 64, 512
    w = _t(synth.gguf_weight(dt, E * N, K, g), dev)
    ids, tw = synth.moe_routing(T, E, topk, g)
    x = _t(g.standard_normal((T, K)).astype(np.float32), dev)
    se, sp = synth.sort_pairs(ids)
    M = ids.size
    se_bad = se.copy()
    se_bad[0], se_bad[1], se_bad[-1] = -1, -1, E
    se_bad = np.sort(se_bad, kind="stable")  # still sorted: -1s first, E last
    ref = torch.zeros((M, N), device=dev)
    hipq.moe_gemm_q(x, w, _t(sp, dev), _t(se, dev), E, N, K, dt, topk, out=ref)
    out = torch.zeros((M, N), device=dev)
    hipq.moe_gemm_q(x, w, _t(sp, dev), _t(se_bad, dev), E, N, K, dt, topk, out=out)
    torch.cuda.synchronize()
    pos_bad = {0, 1, M - 1}  # sorted positions given out-of-range experts
    good_pairs = [int(sp[i]) for i in range(M) if i not in pos_bad]
    assert torch.equal(out[good_pairs], ref[good_pairs])
