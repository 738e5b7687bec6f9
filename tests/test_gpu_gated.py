"""GPU parity of the fused gated MLP projection hq_matmul_q_gated (SwiGLU / GeGLU decode).

Reference: Light's unfused path, MatMulQ(x, Wg), MatMulQ(x, Wu), SiLU / GeluErf, Mul
(models/llama.go:1306-1328) -- oracle.matmul_q twice and oracle.gated.  Bar: per output,
|h - h_ref| <= 1e-3 * (1.13 |u| ||wg_n|| ||x|| + |act(g)| ||wu_n|| ||x||): the 1e-3 matmul bar
carried through the product (1.13 bounds |act'| for SiLU and GELU).
"""
import numpy as np
import pytest
import torch

import oracle
from light_amd import hipq, synth

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _check(dev, dt, M, N, K, act, seed):
    print(f"[case] gated dt={hipq.NAMES[dt]} M={M} N={N} K={K} act={act}", flush=True)
    g = synth.rng(seed)
    wg = synth.gguf_weight(dt, N, K, g)
    wu = synth.gguf_weight(dt, N, K, g)
    x = synth.activations(M, K, g)
    xt = torch.from_numpy(x).to(dev)
    got = hipq.matmul_q_gated(xt, torch.from_numpy(wg).to(dev), torch.from_numpy(wu).to(dev), N, K, dt, act=act)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    gr = oracle.matmul_q(x, wg, N, K, dt)
    ur = oracle.matmul_q(x, wu, N, K, dt)
    want = oracle.gated(gr, ur, act)
    xn = np.linalg.norm(x.astype(np.float64), axis=1)[:, None]
    ng = np.linalg.norm(oracle.dequant(dt, wg, N * K).reshape(N, K).astype(np.float64), axis=1)[None, :]
    nu = np.linalg.norm(oracle.dequant(dt, wu, N * K).reshape(N, K).astype(np.float64), axis=1)[None, :]
    hg = oracle.gated(gr, np.ones_like(gr), act).astype(np.float64)
    bound = TOL * (1.13 * np.abs(ur) * ng * xn + np.abs(hg) * nu * xn) + 1e-30
    err = np.abs(got.astype(np.float64) - want) / bound
    assert np.all(np.isfinite(got))
    assert err.max() <= 1.0, f"max err / bound {err.max():.3g} at {np.unravel_index(err.argmax(), err.shape)}"


@pytest.mark.parametrize("act", [hipq.ACT_SILU, hipq.ACT_GELU_ERF])
@pytest.mark.parametrize("M", [1, 2, 5, 8])
@pytest.mark.parametrize("K", [256, 2048, 4096, 14336])
def test_gated_q4_k_fused(dev, act, M, K):
    _check(dev, hipq.Q4_K, M, 333, K, act, seed=M * 7 + K + act)


@pytest.mark.parametrize("dt", [hipq.Q4_0, hipq.Q5_0, hipq.Q8_0, hipq.Q5_K, hipq.Q6_K])
@pytest.mark.parametrize("M", [1, 4])
def test_gated_other_formats(dev, dt, M):
    _check(dev, dt, M, 200, 1024, hipq.ACT_SILU, seed=dt + M)


def test_gated_q4_k_prefill(dev):
    """M > 8 takes the GEMM pair + epilogue."""
    _check(dev, hipq.Q4_K, 24, 256, 2048, hipq.ACT_SILU, seed=99)


def test_gated_llama3_shape(dev):
    """Llama-3-8B gate/up at decode: N = 14336, K = 4096."""
    _check(dev, hipq.Q4_K, 1, 14336, 4096, hipq.ACT_SILU, seed=1)


def _check_mlp(dev, dt, M, H, I, act, seed):
    """hq_mlp_q against Light's unfused CPU path.  Bar: the gated bound b_h per element of h
    (as above), carried through the down projection: |y - y_ref| <= ||wd_n|| (||b_h|| +
    1e-3 ||h_ref||)."""
    print(f"[case] mlp dt={hipq.NAMES[dt]} M={M} H={H} I={I} act={act}", flush=True)
    g = synth.rng(seed)
    wg = synth.gguf_weight(dt, I, H, g)
    wu = synth.gguf_weight(dt, I, H, g)
    wd = synth.gguf_weight(dt, H, I, g)
    x = synth.activations(M, H, g)
    t = lambda a: torch.from_numpy(a).to(dev)
    got = hipq.mlp_q(t(x), t(wg), t(wu), t(wd), H, I, dt, act=act)
    torch.cuda.synchronize()
    got = got.cpu().numpy().astype(np.float64)
    gr = oracle.matmul_q(x, wg, I, H, dt)
    ur = oracle.matmul_q(x, wu, I, H, dt)
    h = oracle.gated(gr, ur, act)
    want = oracle.matmul_q(h, wd, H, I, dt).astype(np.float64)
    xn = np.linalg.norm(x.astype(np.float64), axis=1)[:, None]
    ng = np.linalg.norm(oracle.dequant(dt, wg, I * H).reshape(I, H).astype(np.float64), axis=1)[None, :]
    nu = np.linalg.norm(oracle.dequant(dt, wu, I * H).reshape(I, H).astype(np.float64), axis=1)[None, :]
    nd = np.linalg.norm(oracle.dequant(dt, wd, H * I).reshape(H, I).astype(np.float64), axis=1)[None, :]
    hg = oracle.gated(gr, np.ones_like(gr), act).astype(np.float64)
    bh = TOL * (1.13 * np.abs(ur) * ng * xn + np.abs(hg) * nu * xn)
    bound = nd * (np.linalg.norm(bh, axis=1)[:, None] + TOL * np.linalg.norm(h.astype(np.float64), axis=1)[:, None])
    err = np.abs(got - want) / (bound + 1e-30)
    assert np.all(np.isfinite(got))
    assert err.max() <= 1.0, f"max err / bound {err.max():.3g}"


@pytest.mark.parametrize("M", [1, 2, 3, 8])
@pytest.mark.parametrize("act", [hipq.ACT_SILU, hipq.ACT_GELU_ERF])
def test_mlp_q4_k_fused(dev, M, act):
    _check_mlp(dev, hipq.Q4_K, M, 1024, 2816, act, seed=300 + M + act)


@pytest.mark.parametrize("M", [1, 5])
def test_mlp_q5_k_fused(dev, M):
    _check_mlp(dev, hipq.Q5_K, M, 1024, 2816, hipq.ACT_SILU, seed=500 + M)


@pytest.mark.parametrize("H,I", [(4096, 14336), (2048, 768), (512, 256), (256, 1024)])
def test_mlp_q4_k_shapes(dev, H, I):
    _check_mlp(dev, hipq.Q4_K, 1, H, I, hipq.ACT_SILU, seed=H + I)


@pytest.mark.parametrize("dt,M", [(hipq.Q8_0, 1), (hipq.Q6_K, 2), (hipq.Q4_K, 12), (hipq.Q4_0, 1), (hipq.Q5_0, 3)])
def test_mlp_unfused_paths(dev, dt, M):
    _check_mlp(dev, dt, M, 512, 768, hipq.ACT_SILU, seed=dt * 3 + M)


def test_mlp_repeated_calls_agree(dev):
    """Calls at different M (one and two grid rows) interleave on the same weights, and every
    repeat of a call reproduces its first result bit for bit (the decode kernels keep no state
    between calls and sum in a fixed order)."""
    print("[case] mlp repeated calls", flush=True)
    g = synth.rng(77)
    H, I = 1024, 2816
    t = lambda a: torch.from_numpy(a).to(dev)
    wg, wu, wd = (t(synth.gguf_weight(hipq.Q4_K, r, c, g)) for r, c in ((I, H), (I, H), (H, I)))
    xs = {M: t(synth.activations(M, H, g)) for M in (1, 8, 3)}
    first = {}
    for rep in range(3):
        for M, x in xs.items():
            y = hipq.mlp_q(x, wg, wu, wd, H, I, hipq.Q4_K, act=hipq.ACT_SILU)
            torch.cuda.synchronize()
            if rep == 0:
                first[M] = y.clone()
            else:
                assert torch.equal(y, first[M]), (rep, M)


@pytest.mark.parametrize("dt,M,H,I", [(hipq.Q4_K, 1, 4096, 14336), (hipq.Q4_K, 3, 1024, 2816),
                                      (hipq.Q5_K, 2, 1024, 2816), (hipq.Q8_0, 1, 512, 768),
                                      # both unit variants (two-level x below 4096, one level
                                      # from it) on each side; fewer chunks than workgroups
                                      (hipq.Q5_K, 1, 1024, 2816), (hipq.Q4_K, 1, 8192, 1024),
                                      (hipq.Q4_K, 1, 256, 256), (hipq.Q4_K, 1, 2048, 768)])
def test_gated_act_then_down_equals_mlp(dev, dt, M, H, I):
    """hq_matmul_q_gated_act followed by hq_matmul_q_act is hq_mlp_q split at its kernel
    boundary: the same launches, so the same bits (the unfused formats run the same
    gated-then-quantize sequence too)."""
    print(f"[case] gated_act+down dt={hipq.NAMES[dt]} M={M} H={H} I={I}", flush=True)
    g = synth.rng(4000 + dt + M)
    t = lambda a: torch.from_numpy(a).to(dev)
    wg, wu, wd = (t(synth.gguf_weight(dt, r, c, g)) for r, c in ((I, H), (I, H), (H, I)))
    x = t(synth.activations(M, H, g))
    want = hipq.mlp_q(x, wg, wu, wd, H, I, dt, act=hipq.ACT_SILU)
    act = hipq.matmul_q_gated_act(x, wg, wu, I, H, dt, act=hipq.ACT_SILU)
    got = hipq.matmul_q_act(act, wd, M, H, I, dt)
    torch.cuda.synchronize()
    if dt in (hipq.Q4_K, hipq.Q5_K):
        assert torch.equal(got, want)
    else:  # mlp_q's unfused path feeds F32 h to hq_matmul_q; here h is quantized first
        scale = want.abs().max().item()
        assert (got - want).abs().max().item() <= 1e-3 * scale


def test_mlp_streams_and_repeats(dev):
    """hq_mlp_q without a caller workspace keeps one per stream: calls alternating over three
    streams, repeated, reproduce the separate-launch result bit for bit every time."""
    print("[case] mlp three streams", flush=True)
    g = synth.rng(91)
    H, I = 4096, 14336
    t = lambda a: torch.from_numpy(a).to(dev)
    wg, wu, wd = (t(synth.gguf_weight(hipq.Q4_K, r, c, g)) for r, c in ((I, H), (I, H), (H, I)))
    xs = [t(synth.activations(1, H, g)) for _ in range(3)]
    want = [hipq.matmul_q_act(hipq.matmul_q_gated_act(x, wg, wu, I, H, hipq.Q4_K), wd, 1, H, I, hipq.Q4_K)
            for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=dev) for _ in range(3)]
    outs = [[None] * 3 for _ in range(3)]
    for rep in range(20):
        for i, st in enumerate(streams):
            with torch.cuda.stream(st):
                y = hipq.mlp_q(xs[i], wg, wu, wd, H, I, hipq.Q4_K, stream=st)
            if rep < 3:
                outs[i][rep] = y
    torch.cuda.synchronize()
    for i in range(3):
        for rep in range(3):
            assert torch.equal(outs[i][rep], want[i]), (i, rep)
