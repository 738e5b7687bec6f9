"""Seeded random shapes through every dispatch path of MatMulQ (GGUF bytes, the Q6_K_R layout
and prepared activations), dequant, MatMulInt4 (with DequantizeInt4 and the GPTQ / AWQ
conversions), MoEGemmQ, the fused gated projection and MLP, MoERoute, the fused MoE blocks and
MoEInt4.

Each entry point picks among several kernels by M, N, K, the group size and the x dtype
(decode GEMVs, staged GEMVs, the one-launch and split-K int4 kernels, the MFMA GEMMs).  The
shapes below are drawn once from a fixed seed over ragged N, K up to 16-20 K and M from 1 to
100 (and, for the int4 kernels that need the chip filled, N up to 24 K with sampled rows;
for MoEGemmQ, random expert counts, top-k and token counts), so every path meets shapes its
own tests do not name; each call must succeed and stay within the north-star bar of Light's
CPU path and the f64 oracle (ops/matmul_q_test.go:105-146, ops/int4_test.go:15-31 and
ops/moe_test.go for the input distributions).
"""
import numpy as np
import pytest
import torch

import oracle
from _util import norm_err, random_blocks
from light_amd import hipq, synth
from test_gpu_gated import _check as check_gated, _check_mlp as check_mlp
from test_gpu_int4 import _check as check_int4, light_int4
from test_gpu_matmul_q import _check_matmul
from test_gpu_int4 import test_moe_int4_vs_light_cpu as check_moe_int4
from test_gpu_int4_convert import test_from_awq_bit_exact as check_awq
from test_gpu_int4_convert import test_from_gptq_bit_exact as check_gptq
from test_gpu_moe import _check as check_moe
from test_gpu_moe import test_moe_block_equals_route_gated_then_combine as check_moe_block
from test_gpu_moe import test_moe_route_bit_exact as check_route
from test_gpu_moe import test_moe_route_gated_bit_exact as check_route_gated
from test_gpu_q6k_repack import _check as check_q6kr

pytestmark = pytest.mark.gpu

_MS = (1, 2, 3, 5, 8, 9, 12, 16, 17, 24, 33, 40, 48, 64, 65, 100)
_GGUF = (hipq.Q4_0, hipq.Q5_0, hipq.Q8_0, hipq.Q4_K, hipq.Q5_K, hipq.Q6_K)
_BLOCK = {hipq.Q4_0: 32, hipq.Q5_0: 32, hipq.Q8_0: 32, hipq.Q4_K: 256, hipq.Q5_K: 256, hipq.Q6_K: 256}
_WORK = 2.5e8  # M * N * K per case: the CPU oracle finishes each in about a second


def _gguf_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        dt = _GGUF[i % len(_GGUF)]
        M = int(rng.choice(_MS))
        K = _BLOCK[dt] * int(rng.integers(1, 20480 // _BLOCK[dt] + 1))
        N = int(rng.integers(1, 6000))
        while M * N * K > _WORK and N > 1:
            N //= 2
        out.append((dt, M, N, K))
    return out


def _int4_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        xdt = (hipq.F32, hipq.F16, hipq.BF16)[i % 3]
        G = int(rng.choice((32, 64, 128, 256)))
        M = int(rng.choice(_MS))
        K = G * int(rng.integers(1, 16384 // G + 1))
        N = int(rng.integers(1, 20000))
        while M * N * K > _WORK and N > 1:
            N //= 2
        out.append((xdt, M, N, K, G))
    return out


@pytest.mark.parametrize("dt,M,N,K", _gguf_cases(36, 2024))
def test_matmul_q_random_shape(dev, dt, M, N, K):
    rng = np.random.default_rng(M * 7919 + N * 31 + K + dt)
    w = random_blocks(rng, dt, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    _check_matmul(dev, dt, x, w, N, K, "random shape")


@pytest.mark.parametrize("xdt,M,N,K,G", _int4_cases(30, 4048))
def test_int4_matmul_random_shape(dev, xdt, M, N, K, G):
    rng = np.random.default_rng(M * 7919 + N * 31 + K + G)
    codes, s, z = light_int4(rng, N, K, G)
    x = rng.standard_normal((M, K)).astype(np.float32)
    check_int4(dev, x, codes, s, z, G, xdt)


def _int4_wide_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        xdt = (hipq.F16, hipq.F32, hipq.BF16, hipq.F16)[i % 4]
        G = int(rng.choice((64, 128, 256)))
        M = int(rng.integers(9, 65))
        K = G * int(rng.integers(1, 8192 // G + 1))
        N = int(rng.integers(15000, 24000))
        out.append((xdt, M, N, K, G))
    return out


@pytest.mark.parametrize("xdt,M,N,K,G", _int4_wide_cases(12, 8096))
def test_int4_matmul_random_wide_shape(dev, xdt, M, N, K, G):
    """N large enough for the one-launch F16 kernel; four rows checked (first, last, two inside)."""
    rng = np.random.default_rng(M * 7919 + N * 31 + K + G)
    codes, s, z = light_int4(rng, N, K, G)
    x = rng.standard_normal((M, K)).astype(np.float32)
    rows = sorted({0, M - 1, int(rng.integers(0, M)), int(rng.integers(0, M))})
    check_int4(dev, x, codes, s, z, G, xdt, rows=rows)


def _moe_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        dt = _GGUF[i % len(_GGUF)]
        E = int(rng.integers(2, 65))
        topk = int(rng.integers(1, min(E, 8) + 1))
        T = int(rng.choice((1, 2, 3, 7, 16, 33, 64, 100, 256)))
        K = _BLOCK[dt] * int(rng.integers(1, 6144 // _BLOCK[dt] + 1))
        N = int(rng.integers(1, 700))
        while (T * topk * N * K > _WORK or E * N * K > 6e7) and N > 1:  # oracle time and memory
            N //= 2
        out.append((dt, T, E, topk, N, K, bool(i % 2)))
    return out


@pytest.mark.parametrize("dt,T,E,topk,N,K,weighted", _moe_cases(24, 6072))
def test_moe_gemm_q_random_shape(dev, dt, T, E, topk, N, K, weighted):
    g = synth.rng(T * 131 + E * 17 + topk + N + K + dt)
    w = synth.gguf_weight(dt, E * N, K, g)
    ids, tw = synth.moe_routing(T, E, topk, g)
    rows = T * topk if weighted else T
    x = g.standard_normal((rows, K)).astype(np.float32)
    M = T * topk
    sample = None if M <= 64 else list(range(0, M, max(1, M // 64))) + [M - 1]
    check_moe(dev, x, w, dt, E, N, K, ids, tw, topk, weighted, sample=sample)


def _gated_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        dt = _GGUF[i % len(_GGUF)]
        M = int(rng.choice(_MS))
        K = _BLOCK[dt] * int(rng.integers(1, 16384 // _BLOCK[dt] + 1))
        N = int(rng.integers(1, 6000))
        while 2 * M * N * K > _WORK and N > 1:
            N //= 2
        out.append((dt, M, N, K, (hipq.ACT_SILU, hipq.ACT_GELU_ERF)[i % 2]))
    return out


@pytest.mark.parametrize("dt,M,N,K,act", _gated_cases(24, 9120))
def test_gated_random_shape(dev, dt, M, N, K, act):
    check_gated(dev, dt, M, N, K, act, seed=M * 7919 + N * 31 + K + dt)


def _mlp_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        dt = _GGUF[i % len(_GGUF)]
        M = int(rng.choice(_MS))
        H = _BLOCK[dt] * int(rng.integers(1, 6144 // _BLOCK[dt] + 1))
        I = _BLOCK[dt] * int(rng.integers(1, 16384 // _BLOCK[dt] + 1))
        while 3 * M * H * I > _WORK and I > _BLOCK[dt]:
            I = max(_BLOCK[dt], (I // 2) // _BLOCK[dt] * _BLOCK[dt])
        out.append((dt, M, H, I, (hipq.ACT_SILU, hipq.ACT_GELU_ERF)[i % 2]))
    return out


@pytest.mark.parametrize("dt,M,H,I,act", _mlp_cases(18, 10144))
def test_mlp_random_shape(dev, dt, M, H, I, act):
    check_mlp(dev, dt, M, H, I, act, seed=M * 7919 + H * 31 + I + dt)


def _route_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        E = int(rng.choice((1, 2, 7, 16, 60, 64, 65, 128, 200, 256, 513, 1024)))
        topk = int(rng.integers(1, min(E, 64) + 1))
        # the one-workgroup sort holds a 16-bit count per (64-pair chunk, expert) in LDS
        T = int(rng.integers(1, max(2, min(3000, 4_000_000 // (topk * E)))))
        out.append((T, E, topk, bool(i % 2)))
    return out


@pytest.mark.parametrize("T,E,topk,normalize", _route_cases(16, 11168))
def test_moe_route_random_shape(dev, T, E, topk, normalize):
    check_route(dev, T, E, topk, normalize)


def _moe_fused_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        dt = (hipq.Q4_K, hipq.Q5_K, hipq.Q4_K, hipq.Q8_0, hipq.Q6_K, hipq.Q4_0)[i % 6]
        T = int(rng.choice((1, 1, 1, 2, 3, 5, 16, 40)))
        E = int(rng.integers(2, 161))
        topk = int(rng.integers(1, min(E, 8) + 1))
        H = _BLOCK[dt] * int(rng.integers(1, 4096 // _BLOCK[dt] + 1))
        I = _BLOCK[dt] * int(rng.integers(1, 2048 // _BLOCK[dt] + 1))
        while E * 3 * I * H > 1.2e8 and E > 2:
            E = max(2, E // 2)
        topk = min(topk, E)
        out.append((dt, T, E, topk, H, I))
    return out


@pytest.mark.parametrize("dt,T,E,topk,H,I", _moe_fused_cases(18, 12192))
def test_moe_fused_random_shape(dev, dt, T, E, topk, H, I):
    """Route + gated equals the separate calls, and the whole block equals route + gated +
    combine, bit for bit (the separate calls are held to the oracle by their own tests)."""
    check_route_gated(dev, dt, T, E, topk, H, I, False)
    check_moe_block(dev, dt, T, E, topk, H, I)


def _moe_int4_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        G = int(rng.choice((32, 64, 128)))
        T = int(rng.choice((1, 2, 3, 7)))
        E = int(rng.integers(2, 33))
        topk = int(rng.integers(1, min(E, 8) + 1))
        H = G * int(rng.integers(1, 2048 // G + 1))
        I = G * int(rng.integers(1, 1536 // G + 1))
        out.append((T, E, topk, H, I, G, (torch.float32, torch.float16, torch.bfloat16)[i % 3]))
    return out


@pytest.mark.parametrize("T,E,topk,H,I,G,xdt", _moe_int4_cases(9, 13216))
def test_moe_int4_random_shape(dev, T, E, topk, H, I, G, xdt):
    check_moe_int4(dev, T, E, topk, H, I, G, xdt)


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("dt,M,N,K", [(hipq.Q6_K, M, N, K) for (_, M, N, K) in _gguf_cases(18, 14240)])
def test_matmul_q6kr_random_shape(dev, dt, M, N, K):
    """The Q6_K_R layout (repacked on the device) against Light's CPU path on the GGUF bytes."""
    rng = np.random.default_rng(M * 7919 + N * 31 + K)
    K = 256 * max(1, K // 256)
    w = random_blocks(rng, hipq.Q6_K, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    check_q6kr(dev, x, w, N, K, "random shape")


@pytest.mark.parametrize("dt,M,N,K", _gguf_cases(24, 15264))
@pytest.mark.parametrize("odt", [hipq.F32, hipq.BF16])
def test_dequant_random_shape(dev, dt, M, N, K, odt):
    """Bit-exact dequant of N rows of K at random sizes (M unused)."""
    print(f"[case] dequant dt={hipq.NAMES[dt]} N={N} K={K} odt={odt}", flush=True)
    raw = random_blocks(np.random.default_rng(N * 31 + K + dt), dt, N, K)
    got = hipq.dequant(_t(raw, dev), N * K, dt, odt)
    want = oracle.dequant(dt, raw, N * K)
    if odt == hipq.F32:
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))
    else:
        assert torch.equal(got.cpu().view(torch.int16), torch.from_numpy(want).to(torch.bfloat16).view(torch.int16))


@pytest.mark.parametrize("dt,M,N,K", _gguf_cases(24, 16288))
def test_matmul_q_act_random_shape(dev, dt, M, N, K):
    """Prepared activations (hq_quantize_act, then hq_matmul_q_act) against the f64 oracle.
    Calls that take the GEMV (M <= 8, or K not a multiple of 64) need a weight layout the int8
    GEMV reads (rows of whole 16-byte pieces); any other is refused with HQ_EUNSUPPORTED, never
    run (hq_matmul_q takes those, and test_matmul_q_random_shape covers it)."""
    print(f"[case] matmul_q_act dt={hipq.NAMES[dt]} M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M * 7919 + N * 31 + K + dt + 1)
    w = random_blocks(rng, dt, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    act = hipq.quantize_act(_t(x, dev))
    ws = torch.empty(max(1, hipq.lib().hq_matmul_q_act_ws_bytes(M, N, K, dt)), dtype=torch.uint8, device=dev)
    takes_gemv = M <= 8 or K % 64 != 0
    try:
        got = hipq.matmul_q_act(act, _t(w, dev), M, N, K, dt, ws=ws).cpu().numpy()
    except hipq.HipqError as e:
        assert e.code == hipq.HQ_EUNSUPPORTED and takes_gemv, str(e)
        return
    wd = oracle.dequant(dt, w, N * K).reshape(N, K)
    ref, _, wn, xn = oracle.matmul_f64(x, wd)
    assert np.all(np.isfinite(got))
    assert norm_err(got, ref, wn, xn) <= 1e-3


@pytest.mark.parametrize("dt,M,N,K,act", [(dt, M, 32 * max(1, N // 32), K, a)
                                          for (dt, M, N, K, a) in _gated_cases(24, 17312)])
def test_gated_act_random_shape(dev, dt, M, N, K, act):
    """hq_matmul_q_gated_act writes what hq_quantize_act writes for hq_matmul_q_gated's F32
    output: the same bytes (N % 32 == 0)."""
    print(f"[case] gated_act dt={hipq.NAMES[dt]} M={M} N={N} K={K} act={act}", flush=True)
    rng = np.random.default_rng(M * 7919 + N * 31 + K + dt + 2)
    wg = _t(random_blocks(rng, dt, N, K), dev)
    wu = _t(random_blocks(rng, dt, N, K), dev)
    x = _t(rng.standard_normal((M, K)).astype(np.float32), dev)
    got = hipq.matmul_q_gated_act(x, wg, wu, N, K, dt, act=act)
    h = hipq.matmul_q_gated(x, wg, wu, N, K, dt, act=act)
    want = hipq.quantize_act(h)
    torch.cuda.synchronize()
    assert got.shape == want.shape
    # The defined regions of the act layout (q1, q2, (d, e), sx); the rounding gaps between
    # them are not written.
    q2o = (M * N + 255) & ~255
    do = 2 * q2o
    so = do + 8 * M * (N // 32)
    for name, a, b in (("q1", 0, M * N), ("q2", q2o, q2o + M * N), ("de", do, so), ("sx", so, so + 4 * M * (N // 32))):
        assert torch.equal(got[a:b], want[a:b]), name


def _int4_layout_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        G = int(rng.choice((32, 64, 128)))
        K = G * int(rng.integers(1, 12288 // G + 1))
        N = 8 * int(rng.integers(1, 3000))
        out.append((K, N, G, bool(i % 2), bool((i // 2) % 2)))
    return out


@pytest.mark.parametrize("K,N,G,v2,act_order", _int4_layout_cases(12, 18336))
def test_from_gptq_random_shape(dev, K, N, G, v2, act_order):
    check_gptq(dev, K, N, G, v2, act_order)


@pytest.mark.parametrize("K,N,G,v2,act_order", _int4_layout_cases(8, 19360))
def test_from_awq_random_shape(dev, K, N, G, v2, act_order):
    check_awq(dev, K, N, G)


@pytest.mark.parametrize("K,N,G,v2,act_order", _int4_layout_cases(10, 20384))
@pytest.mark.parametrize("odt", [hipq.F32, hipq.BF16])
def test_dequantize_int4_random_shape(dev, K, N, G, v2, act_order, odt):
    """Bit-exact DequantizeInt4 at random sizes (v2 / act_order unused)."""
    print(f"[case] int4_dequant N={N} K={K} G={G} odt={odt}", flush=True)
    rng = np.random.default_rng(N * 31 + K + G)
    codes, sc, z = light_int4(rng, N, K, G)
    got = hipq.int4_dequant(_t(codes, dev), _t(sc, dev), _t(z, dev), G, odt).cpu()
    want = oracle.int4_dequant(codes, sc, z, N, K, G, odt)
    if odt == hipq.F32:
        assert np.array_equal(got.numpy().view(np.uint32), want.view(np.uint32))
    else:
        assert np.array_equal(got.view(torch.int16).numpy().view(np.uint16), want)


@pytest.mark.parametrize("dt", _GGUF)
@pytest.mark.parametrize("K", [32768, 33024, 40960, 53248, 65536, 73728])
@pytest.mark.parametrize("M", [1, 3, 8, 16])
def test_matmul_q_long_rows(dev, dt, K, M):
    """Rows past the decode kernels' team sizes (Llama-3-405B's FFN is K = 53248): each path
    takes a kernel that covers them, within the bar."""
    rng = np.random.default_rng(M * 7919 + K + dt)
    N = 64
    w = random_blocks(rng, dt, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    _check_matmul(dev, dt, x, w, N, K, "long rows")
    # The prepared-activation entry: the same bar (long rows run as K parts), HQ_EUNSUPPORTED
    # only at M <= 8 for rows the int8 GEMV cannot read: Q4_K / Q5_K past two teams, or a row
    # whose byte length is not a multiple of 16.
    bpb = {hipq.Q4_0: 18, hipq.Q5_0: 22, hipq.Q8_0: 34, hipq.Q4_K: 144, hipq.Q5_K: 176, hipq.Q6_K: 210}[dt]
    refusable = (K // _BLOCK[dt] * bpb) % 16 != 0 or (dt in (hipq.Q4_K, hipq.Q5_K) and K > 65536)
    act = hipq.quantize_act(_t(x, dev))
    ws = torch.empty(max(1, hipq.lib().hq_matmul_q_act_ws_bytes(M, N, K, dt)), dtype=torch.uint8, device=dev)
    try:
        got = hipq.matmul_q_act(act, _t(w, dev), M, N, K, dt, ws=ws).cpu().numpy()
    except hipq.HipqError as e:
        assert e.code == hipq.HQ_EUNSUPPORTED and M <= 8 and refusable, str(e)
        return
    wd = oracle.dequant(dt, w, N * K).reshape(N, K)
    ref, _, wn, xn = oracle.matmul_f64(x, wd)
    assert norm_err(got, ref, wn, xn) <= 1e-3


@pytest.mark.parametrize("K", [53248, 73728])
@pytest.mark.parametrize("M", [1, 3, 16])
@pytest.mark.parametrize("xdt", [hipq.F32, hipq.F16])
def test_int4_long_rows(dev, K, M, xdt):
    rng = np.random.default_rng(M + K + xdt)
    codes, s, z = light_int4(rng, 64, K, 128)
    x = rng.standard_normal((M, K)).astype(np.float32)
    check_int4(dev, x, codes, s, z, 128, xdt)


@pytest.mark.parametrize("dt", [hipq.Q4_K, hipq.Q6_K, hipq.Q8_0])
@pytest.mark.parametrize("K", [32768, 53248])
@pytest.mark.parametrize("T", [1, 3, 64])
def test_moe_gemm_q_long_rows(dev, dt, K, T):
    g = synth.rng(T + K + dt)
    E, topk, N = 4, 2, 64
    w = synth.gguf_weight(dt, E * N, K, g)
    ids, tw = synth.moe_routing(T, E, topk, g)
    x = g.standard_normal((T, K)).astype(np.float32)
    check_moe(dev, x, w, dt, E, N, K, ids, tw, topk, False)


@pytest.mark.parametrize("H,I", [(32768, 256), (256, 53248)])
@pytest.mark.parametrize("T", [1, 3])
def test_moe_int4_long_rows(dev, H, I, T):
    check_moe_int4(dev, T, 4, 2, H, I, 128, torch.float32)


@pytest.mark.parametrize("dt,M,H,I", [(hipq.Q4_K, 1, 4096, 53248), (hipq.Q4_K, 3, 16384, 2048),
                                      (hipq.Q6_K, 1, 16384, 4096), (hipq.Q8_0, 2, 2048, 40960)])
def test_mlp_long_rows(dev, dt, M, H, I):
    """Llama-3-405B-sized rows (H = 16384, I = 53248) through the gated projection and the MLP."""
    check_gated(dev, dt, M, min(I, 8192), H, hipq.ACT_SILU, seed=M + H + I)
    check_mlp(dev, dt, M, H, I, hipq.ACT_SILU, seed=M + H + I)
