"""The allocation-free entry point hq_matmul_q_noalloc against hq_matmul_q.

Both run the same kernels (the GEMV, or the bf16 MFMA GEMM with its fixed-order split-K
reduce), so the outputs must agree bit for bit.  Each case calls the no-alloc entry point
twice in a row, the second time on a smaller input, because every call shares the one
static scratch array of the device and must not depend on what the last call left there.
"""
import ctypes

import numpy as np
import pytest
import torch

from _util import random_blocks
from light_amd import hipq, synth

pytestmark = pytest.mark.gpu


def _pair(dev, dt, M, N, K, seed):
    g = synth.rng(seed)
    w = torch.from_numpy(synth.gguf_weight(dt, N, K, g)).to(dev)
    x = torch.from_numpy(synth.activations(M, K, g)).to(dev)
    return x, w


def _noalloc(x, w, N, K, dt):
    out = torch.full((x.shape[0], N), float("nan"), device=x.device)
    return hipq.matmul_q_noalloc(x, w, N, K, dt, out=out)


@pytest.mark.parametrize("dt,big,small", [
    (hipq.Q4_K, (4, 14336, 4096), (1, 4096, 14336)),      # GEMV: x quantized in-kernel, then into scratch
    (hipq.Q6_K, (1, 4096, 4096), (1, 1024, 2048)),        # staged GEMV
    (hipq.Q8_0, (3, 4096, 4096), (1, 512, 10240)),        # staged GEMV, K > 8192: quantize into scratch
    (hipq.Q4_K, (512, 4096, 14336), (64, 2048, 4096)),    # MFMA GEMM: bf16 x and split-K partials in scratch
    (hipq.Q6_K, (96, 1024, 4096), (16, 512, 2048)),       # bf16 weight copy in scratch, then the GEMM
    (hipq.Q5_K, (1, 4096, 4096), (12, 1024, 2048)),       # Q5_K GEMV, then the GEMM on a bf16 copy
    (hipq.Q4_0, (2, 2048, 4096), (32, 512, 1024)),        # staged Q4_0 GEMV, then the GEMM
    (hipq.Q4_K, (2, 1024, 12288), (1, 512, 9216)),        # K > 8192 at small M: x quantized into scratch
    (hipq.Q5_K, (1, 2048, 10240), (3, 512, 8448)),
    (hipq.Q4_K, (1, 4096, 53248), (3, 512, 40960)),       # long rows: two K halves + their sum in scratch
    (hipq.Q6_K, (1, 2048, 53248), (2, 256, 20480)),       # staged K parts + their sums in scratch
])
def test_noalloc_matches_matmul_q(dev, dt, big, small):
    for i, (M, N, K) in enumerate((big, small)):
        print(f"[case] noalloc dt={hipq.NAMES[dt]} M={M} N={N} K={K} call {i}", flush=True)
        x, w = _pair(dev, dt, M, N, K, 100 + i)
        want = hipq.matmul_q(x, w, N, K, dt)
        got = _noalloc(x, w, N, K, dt)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {i}: max diff {(got - want).abs().max().item():.3g}"


def test_noalloc_q6k_r_matches_matmul_q(dev):
    """Q6_K_R (repacked once by hq_repack_q6k) at decode and prefill sizes, two calls in a row."""
    for i, (M, N, K) in enumerate(((1, 4096, 4096), (24, 1024, 2048))):
        print(f"[case] noalloc dt=Q6_K_R M={M} N={N} K={K} call {i}", flush=True)
        x, raw = _pair(dev, hipq.Q6_K, M, N, K, 200 + i)
        w = hipq.repack_q6k(raw, N, K)
        want = hipq.matmul_q(x, w, N, K, hipq.Q6_K_R)
        got = _noalloc(x, w, N, K, hipq.Q6_K_R)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {i}: max diff {(got - want).abs().max().item():.3g}"


def _random_pairs(n, seed):
    rng = np.random.default_rng(seed)
    fmts = (hipq.Q4_0, hipq.Q5_0, hipq.Q8_0, hipq.Q4_K, hipq.Q5_K, hipq.Q6_K)
    block = {hipq.Q4_0: 32, hipq.Q5_0: 32, hipq.Q8_0: 32, hipq.Q4_K: 256, hipq.Q5_K: 256, hipq.Q6_K: 256}
    ms = (1, 2, 3, 5, 8, 9, 16, 24, 33, 64, 100)
    out = []
    for i in range(n):
        dt = fmts[i % len(fmts)]
        shapes = []
        for _ in range(2):
            M = int(rng.choice(ms))
            K = block[dt] * int(rng.integers(1, 16384 // block[dt] + 1))
            N = int(rng.integers(1, 4000))
            shapes.append((M, N, K))
        out.append((dt, shapes[0], shapes[1]))
    return out


@pytest.mark.parametrize("dt,first,second", _random_pairs(18, 5151))
def test_noalloc_random_shape_pairs(dev, dt, first, second):
    """Two calls in a row at random shapes: each equals hq_matmul_q bit for bit, or is refused
    with HQ_ENOMEM exactly when its workspace exceeds the scratch array."""
    for i, (M, N, K) in enumerate((first, second)):
        print(f"[case] noalloc random dt={hipq.NAMES[dt]} M={M} N={N} K={K} call {i}", flush=True)
        rng = np.random.default_rng(M * 7919 + N * 31 + K + dt + i)
        w = torch.from_numpy(random_blocks(rng, dt, N, K)).to(dev)
        x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(dev)
        need = hipq.lib().hq_matmul_q_ws_bytes(M, N, K, dt)
        want = hipq.matmul_q(x, w, N, K, dt)
        if need > hipq.NOALLOC_SCRATCH_BYTES:
            with pytest.raises(hipq.HipqError) as ei:
                _noalloc(x, w, N, K, dt)
            assert ei.value.code == hipq.HQ_ENOMEM
            continue
        got = _noalloc(x, w, N, K, dt)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {i}: max diff {(got - want).abs().max().item():.3g}"


def test_noalloc_rejects_beyond_scratch(dev):
    x, w = _pair(dev, hipq.Q4_K, 8, 256, 256, 7)
    big_m = 4096
    with pytest.raises(hipq.HipqError) as ei:
        hipq.lib()  # the size check happens before any device work
        rc = hipq.lib().hq_matmul_q_noalloc(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(w.data_ptr()),
                                            ctypes.c_void_p(x.data_ptr()), big_m, 4096, 14336, hipq.Q4_K, None)
        hipq.check(rc)
    assert ei.value.code == hipq.HQ_ENOMEM


def test_noalloc_under_graph_capture(dev):
    """No allocation inside: the call can be captured and replayed; every replay equals eager."""
    M, N, K, dt = 1, 14336, 4096, hipq.Q4_K
    x, w = _pair(dev, dt, M, N, K, 3)
    out = torch.empty((M, N), device=dev)
    want = hipq.matmul_q(x, w, N, K, dt)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        hipq.matmul_q_noalloc(x, w, N, K, dt, out=out, stream=s)  # warm (module load)
        with torch.cuda.graph(g, stream=s):
            hipq.matmul_q_noalloc(x, w, N, K, dt, out=out, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep}"
        hipq.matmul_q(x, w, N, K, dt)  # eager work between replays
        torch.cuda.synchronize()
