"""GPU tests of the Q6_K_R load-time layout (hq_repack_q6k) and the decode GEMV that reads it.

The repack is value-preserving: hq_dequant_rows of the copy must equal hq_dequant of the GGUF
bytes bit for bit (those are pinned to Light's decoder by test_dequant_bit_exact and the KATs),
which pins the layout.  MatMulQ on the copy is held to the same 1e-3 bar as the GGUF formats,
against Light's CPU qmatmul on the original bytes and the f64 oracle.
"""
import numpy as np
import pytest
import torch

import oracle
from _util import norm_err, random_blocks
from light_amd import hipq, synth

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _repack(dev, w, N, K):
    r = hipq.repack_q6k(_t(w, dev), N, K)
    torch.cuda.synchronize()
    return r


@pytest.mark.parametrize("N,K", [(33, 1024), (5, 3584), (7, 256), (3, 14336)])
@pytest.mark.parametrize("odt", [hipq.F32, hipq.BF16])
def test_repack_dequant_bit_exact(dev, N, K, odt):
    print(f"[case] repack dequant N={N} K={K} odt={odt}", flush=True)
    g = np.random.default_rng(N + K)
    raw = random_blocks(g, hipq.Q6_K, N, K)
    r = _repack(dev, raw, N, K)
    rb = -(-(K // 256 * 210) // 16) * 16
    assert r.numel() == N * rb
    got = hipq.dequant_rows(r, N, K, hipq.Q6_K_R, odt)
    want = hipq.dequant(_t(raw, dev), N * K, hipq.Q6_K, odt).reshape(N, K)
    if odt == hipq.F32:
        assert torch.equal(got.view(torch.int32), want.view(torch.int32))
        ref = oracle.dequant(hipq.Q6_K, raw, N * K).reshape(N, K)
        assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    else:
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # Every row's padding is zero.
    pad = r.view(N, rb)[:, K // 256 * 210:]
    assert int(pad.abs().sum()) == 0


def test_dequant_rows_gguf_matches_dequant(dev):
    g = np.random.default_rng(2)
    N, K = 9, 512
    raw = random_blocks(g, hipq.Q4_K, N, K)
    a = hipq.dequant_rows(_t(raw, dev), N, K, hipq.Q4_K)
    b = hipq.dequant(_t(raw, dev), N * K, hipq.Q4_K).reshape(N, K)
    assert torch.equal(a, b)


def _check(dev, x, w, N, K, label):
    print(f"[case] matmul_q Q6_K_R {label} M={x.shape[0]} N={N} K={K}", flush=True)
    r = _repack(dev, w, N, K)
    got = hipq.matmul_q(_t(x, dev), r, N, K, hipq.Q6_K_R)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    cpu = oracle.matmul_q(x, w, N, K, hipq.Q6_K)
    wd = oracle.dequant(hipq.Q6_K, w, N * K).reshape(N, K)
    ref, _, wn, xn = oracle.matmul_f64(x, wd)
    assert np.all(np.isfinite(got))
    e_cpu, e_f64 = norm_err(got, cpu, wn, xn), norm_err(got, ref, wn, xn)
    assert e_cpu <= TOL, f"{label}: vs Light CPU {e_cpu:.3g}"
    assert e_f64 <= TOL, f"{label}: vs f64 {e_f64:.3g}"


@pytest.mark.parametrize("M", [1, 2, 3, 8])
@pytest.mark.parametrize("N,K", [(1, 256), (64, 512), (130, 2048), (257, 4096), (70, 6144), (65, 12288),
                                 (33, 3584), (20, 14336)])
def test_matmul_q6kr_shapes(dev, M, N, K):
    g = np.random.default_rng(N * 7 + K + M)
    x = synth.activations(M, K, g)
    w = synth.gguf_weight(hipq.Q6_K, N, K, g)
    _check(dev, x, w, N, K, "shapes")


@pytest.mark.parametrize("M", [1, 4])
def test_matmul_q6kr_random_blocks(dev, M):
    """Random bytes: every scale and high-bit pattern, including scales of -128."""
    g = np.random.default_rng(11 + M)
    N, K = 45, 1792 + 256
    x = (g.random((M, K)) * 2 - 1).astype(np.float32)
    w = random_blocks(g, hipq.Q6_K, N, K)
    _check(dev, x, w, N, K, "random_blocks")


def test_matmul_q6kr_gemm_path(dev):
    g = np.random.default_rng(21)
    N, K = 96, 1024
    x = synth.activations(16, K, g)
    w = synth.gguf_weight(hipq.Q6_K, N, K, g)
    _check(dev, x, w, N, K, "gemm M=16")


@pytest.mark.parametrize("name", ["q6_k_gemv_attn_out_4096x4096", "q6_k_gemv_lm_head_128256x4096"])
def test_matmul_q6kr_benchmark_configs(dev, name):
    c = synth.CONFIGS[name]
    g = synth.rng(c["cfg"])
    w = synth.gguf_weight(c["dt"], c["N"], c["K"], g)
    x = synth.activations(c["M"], c["K"], g)
    _check(dev, x, w, c["N"], c["K"], name)


def test_repack_errors(dev):
    w = torch.zeros(210 * 4, dtype=torch.uint8, device=dev)
    with pytest.raises(hipq.HipqError):
        hipq.repack_q6k(w, 4, 200)
    x = torch.zeros((1, 256), device=dev)
    r = hipq.repack_q6k(w, 4, 256)
    with pytest.raises(hipq.HipqError):  # M > 8 is fine, but a misaligned weight is refused
        hipq.matmul_q(x, r[1:], 4, 256, hipq.Q6_K_R)
