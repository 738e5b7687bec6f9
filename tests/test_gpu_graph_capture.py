"""Every entry point captured into a HIP graph and replayed: each replay equals the eager call
bit for bit, with the program's own eager work and synchronizations between replays (the
library workspace of the capturing stream is sized by one eager call first; no memset node is
recorded -- the library clears memory with fill kernels)."""
import numpy as np
import pytest
import torch

from light_amd import hipq, synth

pytestmark = pytest.mark.gpu


def _replays_equal(fn, other, reps=4):
    torch.cuda.synchronize()
    want = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # the capturing stream's workspace, sized eagerly
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            outs = fn()
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(reps):
        for o in outs:
            o.fill_(float("nan") if o.is_floating_point() else 0)
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            assert torch.equal(o, w), f"replay {rep}"
        other()  # eager work between replays
        torch.cuda.synchronize()


def _act_regions(a, M, N):
    """The written regions of an act-layout buffer (q1, q2, (d, e), sx); the rounding gaps
    between them are not part of the output."""
    q2o = (M * N + 255) & ~255
    do = 2 * q2o
    so = do + 8 * M * (N // 32)
    return torch.cat([a[0:M * N], a[q2o:q2o + M * N], a[do:so], a[so:so + 4 * M * (N // 32)]])


def _w(dt, N, K, seed, dev):
    return torch.from_numpy(synth.gguf_weight(dt, N, K, synth.rng(seed))).to(dev)


@pytest.mark.parametrize("dt,M,N,K", [
    (hipq.Q4_K, 1, 4096, 4096),      # persistent GEMV, x quantized in-kernel
    (hipq.Q4_K, 2, 4096, 14336),     # x quantized into the workspace, long-row GEMV
    (hipq.Q8_0, 3, 2048, 4096),      # staged GEMV
    (hipq.Q6_K, 1, 1024, 12288),     # staged GEMV on quantized x in the workspace
    (hipq.Q4_K, 512, 4096, 14336),   # MFMA GEMM, K split + reduce
    (hipq.Q8_0, 40, 1024, 2048),     # bf16 weight copy + GEMM
    (hipq.Q4_0, 24, 300, 2784),      # generic GEMV (rows of 1566 bytes)
    (hipq.Q4_K, 1, 2048, 53248),     # long rows: two K halves + an add
    (hipq.Q4_K, 3, 2048, 53248),     # long rows, several x rows: each half's x copied out (memcpy node)
    (hipq.Q6_K, 2, 1024, 53248),     # staged K parts + adds, per x row
])
def test_matmul_q_graph(dev, dt, M, N, K):
    print(f"[case] graph matmul_q dt={hipq.NAMES[dt]} M={M} N={N} K={K}", flush=True)
    w = _w(dt, N, K, M + K, dev)
    x = torch.randn(M, K, device=dev)
    _replays_equal(lambda: (hipq.matmul_q(x, w, N, K, dt),), lambda: hipq.matmul_q(x[:1], w, N, K, dt))


@pytest.mark.parametrize("M", [1, 3, 16])
def test_gated_and_mlp_graph(dev, M):
    print(f"[case] graph gated/mlp M={M}", flush=True)
    H, I = 2048, 5632
    wg, wu, wd = _w(hipq.Q4_K, I, H, 1, dev), _w(hipq.Q4_K, I, H, 2, dev), _w(hipq.Q4_K, H, I, 3, dev)
    x = torch.randn(M, H, device=dev)
    _replays_equal(lambda: (hipq.matmul_q_gated(x, wg, wu, I, H, hipq.Q4_K),
                            hipq.mlp_q(x, wg, wu, wd, H, I, hipq.Q4_K),
                            _act_regions(hipq.matmul_q_gated_act(x, wg, wu, I, H, hipq.Q4_K), M, I)),
                   lambda: hipq.mlp_q(x[:1], wg, wu, wd, H, I, hipq.Q4_K))


@pytest.mark.parametrize("M,N,K,xdt", [(1, 18944, 3584, torch.float16), (3, 3584, 18944, torch.float32),
                                       (64, 18944, 3584, torch.float16), (64, 3584, 18944, torch.float16),
                                       (16, 2048, 1024, torch.bfloat16)])
def test_int4_graph(dev, M, N, K, xdt):
    print(f"[case] graph int4 M={M} N={N} K={K} x={xdt}", flush=True)
    gen = torch.Generator(device="cpu").manual_seed(M + N)
    G = 128
    codes = torch.randint(0, 2 ** 31, (N, K // 8), dtype=torch.int32, generator=gen).to(dev)
    s = (torch.rand(N, K // G, generator=gen) * 0.02 + 1e-3).to(dev)
    z = torch.randint(0, 16, (N, K // G), generator=gen).float().to(dev)
    x = torch.randn(M, K, generator=gen).to(xdt).to(dev)
    _replays_equal(lambda: (hipq.int4_matmul(x, codes, s, z, G),), lambda: hipq.int4_matmul(x[:1], codes, s, z, G))


@pytest.mark.parametrize("T", [1, 4, 256])
def test_moe_graph(dev, T):
    """Route + gated gate/up + down + combine in hq_moe_block_q: one launch at T = 1, the routed
    GEMVs at T = 4 and the grouped MFMA GEMMs at T = 256."""
    print(f"[case] graph moe T={T}", flush=True)
    E, topk, H, I, dt = 128, 8, 2048, 768, hipq.Q4_K
    g = synth.rng(50 + T)
    wgu = torch.from_numpy(synth.gguf_weight(dt, E * 2 * I, H, g)).to(dev)
    wdn = torch.from_numpy(synth.gguf_weight(dt, E * H, I, g)).to(dev)
    x = torch.from_numpy(synth.activations(T, H, g)).to(dev)
    logits = torch.from_numpy(g.standard_normal((T, E)).astype(np.float32)).to(dev)
    probs = torch.softmax(logits, dim=1)

    def block():
        y, ids, w, sp, se, h = hipq.moe_block_q(probs, x, wgu, wdn, E, H, I, dt, topk)
        return y, ids, w, sp, se, h

    _replays_equal(block, lambda: hipq.moe_block_q(probs[:1], x[:1], wgu, wdn, E, H, I, dt, topk))
