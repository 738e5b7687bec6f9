"""GPU parity of the GGUF path through the C ABI: quantizer, dequant, MatMulQ.

Bars (from the build's north star): dequantized weights and quantized
activations bit-exact; float outputs within max |err| / (||w_n|| * ||x_m||)
<= 1e-3 of Light's CPU qmatmul (oracle.matmul_q) and of the f64
dequant-then-matmul oracle.  Shapes follow TestCUDAMatMulQParity
(ops/matmul_q_test.go:105-146) plus the benchmark shapes.
"""
import numpy as np
import pytest
import torch

import oracle
from _util import norm_err, random_blocks
from light_amd import hipq, synth

pytestmark = pytest.mark.gpu

TOL = 1e-3  # max |err| / (||w_n|| ||x_m||)
FMTS = [hipq.Q4_0, hipq.Q5_0, hipq.Q8_0, hipq.Q4_K, hipq.Q5_K, hipq.Q6_K]


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _check_matmul(dev, dt, x, w, N, K, label, got=None):
    print(f"[case] matmul_q {label} dt={hipq.NAMES[dt]} M={x.shape[0]} N={N} K={K}", flush=True)
    if got is None:
        y = hipq.matmul_q(_t(x, dev), _t(w, dev), N, K, dt)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
    cpu = oracle.matmul_q(x, w, N, K, dt)
    wd = oracle.dequant(dt, w, N * K).reshape(N, K)
    ref, _, wn, xn = oracle.matmul_f64(x, wd)
    e_cpu = norm_err(got, cpu, wn, xn)
    e_f64 = norm_err(got, ref, wn, xn)
    assert np.all(np.isfinite(got))
    assert e_cpu <= TOL, f"{label}: vs Light CPU {e_cpu:.3g}"
    assert e_f64 <= TOL, f"{label}: vs f64 {e_f64:.3g}"
    return e_cpu


# ---- q8_1 activation quantizer -------------------------------------------

@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16, torch.float16])
def test_quantize_q8_1_bit_exact(dev, xdt):
    g = np.random.default_rng(1)
    M, K = 7, 4096
    x = (g.standard_normal((M, K)) * np.repeat(10.0 ** g.uniform(-9, 3, size=(M, K // 32)), 32, axis=1))
    x = x.astype(np.float32)
    x[0, :32] = 0.0
    x[1, :32] = 5e-6  # d in Light's f16 flush-to-zero range
    xt = torch.from_numpy(x).to(xdt)
    xw = xt.float().numpy()  # the exact widened values the CPU quantizer sees
    got = hipq.quantize_q8_1(xt.to(dev)).cpu().numpy()
    want = oracle.quantize_q8_1(xw)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"first mismatch at byte {bad[:8]}"


# ---- dequant -------------------------------------------------------------

@pytest.mark.parametrize("dt", FMTS)
@pytest.mark.parametrize("odt", [hipq.F32, hipq.BF16])
def test_dequant_bit_exact(dev, dt, odt):
    g = np.random.default_rng(dt)
    N, K = 33, 1024
    raw = random_blocks(g, dt, N, K)
    got = hipq.dequant(_t(raw, dev), N * K, dt, odt)
    want = oracle.dequant(dt, raw, N * K)
    if odt == hipq.F32:
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))
    else:
        wb = torch.from_numpy(want).to(torch.bfloat16).view(torch.int16)
        assert torch.equal(got.cpu().view(torch.int16), wb)


def test_dequant_golden_known_answers(dev):
    import json
    import os
    cases = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "dequant_kat.json")))["cases"]
    for c in cases:
        dt = {n: d for d, n in hipq.NAMES.items()}[c["dtype"]]
        raw = np.frombuffer(bytes.fromhex(c["blocks"]), np.uint8).copy()
        got = hipq.dequant(_t(raw, dev), c["n"], dt).cpu().numpy()
        if c["checks"] == "all":
            assert np.array_equal(got, np.array(c["want"], np.float32)), c["name"]
        else:
            for i, v in c["want"].items():
                assert got[int(i)] == np.float32(v), c["name"]


def test_dequant_q8_1_roundtrip(dev):
    g = np.random.default_rng(9)
    x = g.standard_normal((3, 256)).astype(np.float32)
    q = hipq.quantize_q8_1(_t(x, dev))
    y = hipq.dequant(q, 3 * 256, hipq.Q8_1).cpu().numpy()
    assert np.array_equal(y, oracle.dequant(oracle.Q8_1, q.cpu().numpy(), 3 * 256))


# ---- MatMulQ ---------------------------------------------------------------

@pytest.mark.parametrize("dt", FMTS)
@pytest.mark.parametrize("M", [1, 4, 9])
@pytest.mark.parametrize("K", [1024, 1792])
def test_matmul_q_parity_light_shapes(dev, dt, M, K):
    """TestCUDAMatMulQParity shapes: M in {1,4,9}, K in {1024,1792}, N=13, random blocks."""
    g = np.random.default_rng(5 * M + K + dt)
    N = 13
    if K % oracle.BLOCK[dt][0]:
        pytest.skip("K not a block multiple")
    x = (g.random((M, K)) * 2 - 1).astype(np.float32)
    w = random_blocks(g, dt, N, K)
    _check_matmul(dev, dt, x, w, N, K, "light_shapes")


@pytest.mark.parametrize("dt", FMTS)
@pytest.mark.parametrize("N,K", [(1, 256), (64, 512), (130, 2048), (257, 4096), (70, 6144), (65, 12288)])
def test_matmul_q_shapes(dev, dt, N, K):
    g = np.random.default_rng(N * 7 + K + dt)
    x = synth.activations(1, K, g)
    w = synth.gguf_weight(dt, N, K, g)
    _check_matmul(dev, dt, x, w, N, K, "shapes")


@pytest.mark.parametrize("name", ["q8_0_gemv_4096x4096", "q4_k_gemv_gate_14336x4096", "q4_k_gemv_down_4096x14336",
                                  "q6_k_gemv_attn_out_4096x4096", "q6_k_gemv_lm_head_128256x4096"])
def test_matmul_q_benchmark_configs(dev, name):
    c = synth.CONFIGS[name]
    g = synth.rng(c["cfg"])
    w = synth.gguf_weight(c["dt"], c["N"], c["K"], g)
    x = synth.activations(c["M"], c["K"], g)
    _check_matmul(dev, c["dt"], x, w, c["N"], c["K"], name)


def test_matmul_q_zero_and_large_activations(dev):
    g = np.random.default_rng(3)
    N, K = 40, 2048
    w = synth.gguf_weight(hipq.Q4_K, N, K, g)
    x = np.zeros((2, K), np.float32)
    x[1] = g.standard_normal(K).astype(np.float32) * 1e4
    x[1, :256] = 0
    y = hipq.matmul_q(_t(x, dev), _t(w, dev), N, K, hipq.Q4_K).cpu().numpy()
    assert np.all(y[0] == 0)
    _check_matmul(dev, hipq.Q4_K, x[1:], w, N, K, "large")


def test_matmul_q_explicit_workspace_and_stream(dev):
    g = np.random.default_rng(4)
    N, K = 96, 4096
    w = _t(synth.gguf_weight(hipq.Q6_K, N, K, g), dev)
    x = _t(synth.activations(2, K, g), dev)
    ws = torch.empty(hipq.matmul_q_ws_bytes(2, N, K, hipq.Q6_K), dtype=torch.uint8, device=dev)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        y1 = hipq.matmul_q(x, w, N, K, hipq.Q6_K, ws=ws)
    s.synchronize()
    y2 = hipq.matmul_q(x, w, N, K, hipq.Q6_K)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    small = torch.empty(16, dtype=torch.uint8, device=dev)
    with pytest.raises(hipq.HipqError):
        hipq.matmul_q(x, w, N, K, hipq.Q6_K, ws=small)


def test_prepared_activations_match_q8_1(dev):
    """The act layout: level 1 is exactly q8_1 (quants and f32 d), level 2 quantizes the
    residual at e = d / 254, and sx is the block sum of x."""
    g = np.random.default_rng(12)
    M, K = 3, 2048
    x = (g.standard_normal((M, K)) * 3).astype(np.float32)
    x[1, :32] = 0.0
    xt = _t(x, dev)
    act = hipq.quantize_act(xt).cpu().numpy()
    q81 = oracle.quantize_q8_1(x).reshape(-1, 36)
    nb = M * K // 32
    q2_off = (M * K + 255) & ~255
    d_off = 2 * q2_off
    s_off = d_off + 8 * nb
    q1 = act[:M * K].reshape(-1, 32)
    q2 = act[q2_off:q2_off + M * K].view(np.int8).reshape(-1, 32).astype(np.float64)
    de = act[d_off:d_off + 8 * nb].view(np.float32).reshape(-1, 2)
    sx = act[s_off:s_off + 4 * nb].view(np.float32)
    assert np.array_equal(q1, q81[:, 4:])
    amax = np.abs(x.reshape(-1, 32)).max(1)
    assert np.array_equal(de[:, 0], amax / np.float32(127))
    assert np.array_equal(de[:, 0].astype(np.float16).view(np.uint16), q81[:, 0:2].copy().view("<u2")[:, 0])
    assert np.array_equal(de[:, 1], de[:, 0] / np.float32(254))
    assert np.all(np.abs(q2) <= 127)
    recon = q1.view(np.int8).astype(np.float64) * de[:, :1] + q2 * de[:, 1:]
    err = np.abs(recon - x.reshape(-1, 32))
    assert np.all(err <= de[:, 1:] * 0.5 * (1 + 1e-3) + 1e-30)
    assert np.allclose(sx, x.reshape(-1, 32).sum(1), rtol=1e-5, atol=1e-5)
    assert np.all(de[32 // 32 * (K // 32)] == 0)  # the all-zero block


@pytest.mark.parametrize("dt", FMTS)
@pytest.mark.parametrize("M", [1, 2, 3, 5, 8])
def test_matmul_q_act_equals_matmul_q(dev, dt, M):
    g = np.random.default_rng(M + dt)
    N, K = 200, 4096
    w = _t(synth.gguf_weight(dt, N, K, g), dev)
    x = _t(synth.activations(M, K, g), dev)
    y1 = hipq.matmul_q(x, w, N, K, dt)
    act = hipq.quantize_act(x)
    y2 = hipq.matmul_q_act(act, w, M, N, K, dt)
    torch.cuda.synchronize()
    # At K <= 8192 the decode GEMVs quantize x inside their workgroups (reciprocal-based
    # scales), hq_quantize_act with IEEE divisions: a q1 that rounds the other way at a tie
    # moves its element by one step d (no second level to absorb it from K = 4096), so the two
    # paths agree to a few such steps, far inside the bar (each is checked against it below).
    ref = torch.from_numpy(oracle.matmul_q(x.cpu().numpy(), w.cpu().numpy(), N, K, dt)).to(dev)
    ratio = ((y1 - y2).abs().max() / ref.abs().max()).item()
    print(f"[diff] {hipq.NAMES[dt]} M={M}: max |y1 - y2| / max |y| = {ratio:.3g}", flush=True)
    assert ratio <= (1e-4 if K < 4096 else 1e-3)
    _check_matmul(dev, dt, x.cpu().numpy(), w.cpu().numpy(), N, K, "act")
    _check_matmul(dev, dt, x.cpu().numpy(), w.cpu().numpy(), N, K, "act", got=y2.cpu().numpy())


@pytest.mark.parametrize("dt", [hipq.Q4_0, hipq.Q5_0, hipq.Q5_K])
@pytest.mark.parametrize("M", [1, 3, 8, 12, 40])
def test_matmul_q_added_formats_rows(dev, dt, M):
    """Q4_0 / Q5_0 / Q5_K (kernels/cuda/matmul_q.go:17-24) at decode and small prefill rows,
    against Light's CPU path (Q5_K: its dequant + MatMul fallback)."""
    g = np.random.default_rng(70 + M + dt)
    N, K = 96, 2048
    w = synth.gguf_weight(dt, N, K, g)
    x = synth.activations(M, K, g)
    _check_matmul(dev, dt, x, w, N, K, "added_formats")


@pytest.mark.parametrize("dt", [hipq.Q4_0, hipq.Q5_0, hipq.Q8_0, hipq.Q5_K, hipq.Q6_K])
@pytest.mark.parametrize("M,N,K", [(9, 13, 1024), (100, 200, 2048), (300, 130, 512), (512, 256, 4096)])
def test_gemm_dequant_bf16_formats(dev, dt, M, N, K):
    """M > 8, formats without an in-GEMM dequant: bit-exact bf16 dequant into the workspace,
    then the MFMA GEMM on bf16 weights (Light's prefill is dequant + GEMM too,
    ops/matmul_q.go:52-59)."""
    g = np.random.default_rng(M + N + K + dt)
    w = synth.gguf_weight(dt, N, K, g)
    x = synth.activations(M, K, g)
    _check_matmul(dev, dt, x, w, N, K, "gemm_bf16")


def test_matmul_q_many_rows_k_not_64(dev):
    """K % 64 != 0 (Q8_0 K = 96) keeps the GEMV at M > 8."""
    g = np.random.default_rng(12)
    N, K, M = 20, 96, 12
    w = synth.gguf_weight(hipq.Q8_0, N, K, g)
    x = synth.activations(M, K, g)
    _check_matmul(dev, hipq.Q8_0, x, w, N, K, "k96")


def test_matmul_q_q5_0_high_bits_only(dev):
    """Q5_0 with zero nibbles and every fifth bit set (q5 = 16 -> 0) or clear (-16): pins the
    qh bit order in the GEMV against the closed form."""
    g = np.random.default_rng(4)
    N, K = 8, 256
    nb = N * K // 32
    q = 16 * g.integers(0, 2, size=(nb, 32))
    d = synth._f16_bits(np.full(nb, 0.5, np.float32))
    w = synth.pack_q5_0(d, q)
    x = synth.activations(1, K, g)
    wd = 0.5 * (q.reshape(N, K) - 16).astype(np.float64)
    want = wd @ x[0].astype(np.float64)
    got = hipq.matmul_q(_t(x, dev), _t(w, dev), N, K, hipq.Q5_0).cpu().numpy()[0]
    assert np.max(np.abs(got - want) / (np.linalg.norm(wd, axis=1) * np.linalg.norm(x[0]))) <= TOL
    _check_matmul(dev, hipq.Q5_0, x, w, N, K, "q5_0_high_bits")


# ---- Q4_K prefill GEMM (MFMA) ----------------------------------------------

@pytest.mark.parametrize("M,N,K", [(9, 13, 1024), (17, 128, 256), (100, 200, 2048), (256, 256, 4096),
                                   (300, 130, 1024), (64, 4096, 4096), (513, 384, 2560)])
def test_gemm_q4_k_shapes(dev, M, N, K):
    g = np.random.default_rng(M * 31 + N + K)
    x = synth.activations(M, K, g)
    w = synth.gguf_weight(hipq.Q4_K, N, K, g)
    _check_matmul(dev, hipq.Q4_K, x, w, N, K, "gemm")


@pytest.mark.parametrize("name", ["q4_k_gemm_m512_14336x4096", "q4_k_gemm_m512_4096x14336"])
def test_gemm_q4_k_benchmark_configs(dev, name):
    """Full M=512 configs on the GPU against Light's CPU path and the f64 oracle, every row."""
    c = synth.CONFIGS[name]
    g = synth.rng(c["cfg"])
    M, N, K = c["M"], c["N"], c["K"]
    w = synth.gguf_weight(hipq.Q4_K, N, K, g)
    x = synth.activations(M, K, g)
    print(f"[case] gemm {name}", flush=True)
    y = hipq.matmul_q(_t(x, dev), _t(w, dev), N, K, hipq.Q4_K).cpu().numpy()
    rows = np.arange(M)
    cpu = oracle.matmul_q(x[rows], w, N, K, hipq.Q4_K)
    wd = oracle.dequant(hipq.Q4_K, w, N * K).reshape(N, K)
    ref, _, wn, xn = oracle.matmul_f64(x[rows], wd)
    assert norm_err(y[rows], cpu, wn, xn) <= TOL
    assert norm_err(y[rows], ref, wn, xn) <= TOL
    assert np.all(np.isfinite(y))


def test_gemm_act_path_matches(dev):
    """hq_matmul_q_act at M > 8 (act -> bf16 -> GEMM) stays within tolerance of the F32 path."""
    g = np.random.default_rng(77)
    M, N, K = 40, 300, 2048
    x = synth.activations(M, K, g)
    w = synth.gguf_weight(hipq.Q4_K, N, K, g)
    xt, wt = _t(x, dev), _t(w, dev)
    act = hipq.quantize_act(xt)
    ws = torch.empty(hipq.lib().hq_matmul_q_act_ws_bytes(M, N, K, hipq.Q4_K), dtype=torch.uint8, device=dev)
    y = hipq.matmul_q_act(act, wt, M, N, K, hipq.Q4_K, ws=ws).cpu().numpy()
    wd = oracle.dequant(hipq.Q4_K, w, N * K).reshape(N, K)
    ref, _, wn, xn = oracle.matmul_f64(x, wd)
    assert norm_err(y, ref, wn, xn) <= TOL


@pytest.mark.parametrize("dt", [hipq.Q4_K, hipq.Q5_K])
@pytest.mark.parametrize("K,amp", [(4096, 10.0), (4096, 30.0), (8192, 10.0), (8192, 30.0), (14336, 10.0)])
def test_matmul_q_single_level_outlier_blocks(dev, dt, K, amp):
    """Rows of K >= 4096 quantize x to q1 alone (q8_1): its error is largest when one element
    per 32-block sets the step.  One outlier of `amp` sigma in every block, 2048 rows."""
    g = np.random.default_rng(int(amp) + K + dt)
    N = 2048
    x = g.standard_normal((1, K)).astype(np.float32)
    pos = np.arange(0, K, 32) + g.integers(0, 32, K // 32)
    x[0, pos] = (amp * np.sign(g.standard_normal(K // 32))).astype(np.float32)
    w = synth.gguf_weight(dt, N, K, g)
    e = _check_matmul(dev, dt, x, w, N, K, f"outliers amp={amp}")
    print(f"[err] single-level K={K} amp={amp}: {e:.3g}", flush=True)
