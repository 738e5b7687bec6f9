"""GPU parity of the GPTQ / AWQ int4 path (Light's quant.Int4) through the C ABI.

Mirrors TestDequantizeInt4 (ops/int4_test.go:47-81: bit-exact F32 and BF16) and
TestMatMulInt4 (ops/int4_test.go:83-145: M in {1, 3, 8, 9}) plus the
Qwen2.5-7B MLP shapes of the benchmark.  Float bar: max |err| / (||w_n|| ||x_m||)
<= 1e-3 against Light's CPU int4MatMulCPU (oracle.int4_matmul) and the f64
oracle, plus the output dtype's rounding (half an ulp of |y|) for BF16 / F16 y.
"""
import numpy as np
import pytest
import torch

import oracle
from _util import norm_err
from light_amd import hipq, synth

pytestmark = pytest.mark.gpu

TOL = 1e-3
TDT = {hipq.F32: torch.float32, hipq.BF16: torch.bfloat16, hipq.F16: torch.float16}
ULP = {hipq.F32: 0.0, hipq.BF16: 2.0 ** -8, hipq.F16: 2.0 ** -11}


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def light_int4(rng, N, K, G):
    """randomInt4 (ops/int4_test.go:15-31): codes uniform, s in [1e-3, 0.021), z in [0, 15]."""
    codes = rng.integers(0, 2 ** 32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = (rng.random((N, K // G)) * 0.02 + 1e-3).astype(np.float32)
    z = rng.integers(0, 16, size=(N, K // G)).astype(np.float32)
    return codes, s, z


def _check(dev, x, codes, s, z, G, xdt, rows=None):
    M, K = x.shape
    N = codes.shape[0]
    print(f"[case] int4 M={M} N={N} K={K} G={G} x={hipq.NAMES[xdt]}", flush=True)
    xt = torch.from_numpy(x).to(TDT[xdt])
    xw = xt.float().numpy()  # exact widened activations
    y = hipq.int4_matmul(xt.to(dev), _t(codes, dev), _t(s, dev), _t(z, dev), G)
    torch.cuda.synchronize()
    assert y.dtype == TDT[xdt] and tuple(y.shape) == (M, N)
    got = y.float().cpu().numpy()
    if rows is not None:
        got, xw = got[rows], xw[rows]
    cpu = oracle.int4_matmul(xw, codes, s, z, N, K, G)
    wd = oracle.int4_dequant(codes, s, z, N, K, G)
    ref, _, wn, xn = oracle.matmul_f64(xw, wd)
    slack = ULP[xdt] * np.abs(ref) / np.maximum(np.outer(xn, wn), 1e-30)
    e = np.abs(got - ref) / np.maximum(np.outer(xn, wn), 1e-30) - slack
    assert np.all(np.isfinite(got))
    assert float(e.max()) <= TOL, f"vs f64 {e.max():.3g}"
    e2 = np.abs(got - cpu) / np.maximum(np.outer(xn, wn), 1e-30) - slack
    assert float(e2.max()) <= TOL, f"vs Light CPU {e2.max():.3g}"


@pytest.mark.parametrize("odt", [hipq.F32, hipq.BF16])
def test_dequantize_int4_bit_exact(dev, odt):
    rng = np.random.default_rng(3)
    N, K, G = 24, 256, 64
    codes, s, z = light_int4(rng, N, K, G)
    got = hipq.int4_dequant(_t(codes, dev), _t(s, dev), _t(z, dev), G, odt).cpu()
    want = oracle.int4_dequant(codes, s, z, N, K, G, odt)
    if odt == hipq.F32:
        assert np.array_equal(got.numpy().view(np.uint32), want.view(np.uint32))
    else:
        assert np.array_equal(got.view(torch.int16).numpy().view(np.uint16), want)


def test_dequantize_int4_offset_slot(dev):
    """The offset argument writes one slot of a stacked buffer (ops/int4.go:31-56)."""
    rng = np.random.default_rng(5)
    N, K, G = 8, 128, 32
    codes, s, z = light_int4(rng, N, K, G)
    out = torch.full((3 * N * K,), -1.0, device=dev)
    hipq.int4_dequant(_t(codes, dev), _t(s, dev), _t(z, dev), G, hipq.F32, out=out, out_offset=N * K)
    o = out.cpu().numpy()
    assert np.all(o[:N * K] == -1) and np.all(o[2 * N * K:] == -1)
    assert np.array_equal(o[N * K:2 * N * K], oracle.int4_dequant(codes, s, z, N, K, G).ravel())


@pytest.mark.parametrize("M", [1, 3, 8, 9])
@pytest.mark.parametrize("xdt", [hipq.F32, hipq.BF16, hipq.F16])
def test_matmul_int4_light_shapes(dev, M, xdt):
    """TestMatMulInt4 shapes: N=96, K=256, G=64."""
    rng = np.random.default_rng(4 + M)
    N, K, G = 96, 256, 64
    codes, s, z = light_int4(rng, N, K, G)
    x = rng.standard_normal((M, K)).astype(np.float32)
    _check(dev, x, codes, s, z, G, xdt)


@pytest.mark.parametrize("M,N,K,G", [(1, 1, 32, 32), (2, 300, 512, 32), (5, 77, 1024, 128), (16, 256, 4096, 128),
                                     (33, 130, 2048, 64), (64, 512, 3584, 128), (70, 200, 1536, 96),
                                     (4, 64, 32768, 128), (3, 77, 16384, 128),
                                     # 8 < M <= 64 with G % 64 != 0 (a scale per 8-column slice),
                                     # ragged N and M, and K split 16 ways
                                     (24, 96, 1024, 32), (40, 136, 1536, 96), (48, 256, 8192, 32)])
def test_matmul_int4_shapes(dev, M, N, K, G):
    rng = np.random.default_rng(M * 7 + N + K)
    codes, s, z = light_int4(rng, N, K, G)
    x = rng.standard_normal((M, K)).astype(np.float32)
    _check(dev, x, codes, s, z, G, hipq.F32)


@pytest.mark.parametrize("zkind", ["frac", "wide"])
def test_matmul_int4_f16_nonintegral_zeros(dev, zkind):
    """Zero points that are not the integers 0..15 of a checkpoint (quant.Int4 holds them as
    f32): fractional, or integral beyond 64.  The f16 MFMA path for 8 < M <= 64 takes its
    second-add branch for these; results stay within tolerance of the f64 reference."""
    rng = np.random.default_rng(11 if zkind == "frac" else 12)
    M, N, K, G = 64, 512, 3584, 128
    codes, s, _ = light_int4(rng, N, K, G)
    if zkind == "frac":
        z = (rng.random((N, K // G)) * 15).astype(np.float32)
    else:
        z = rng.integers(60, 100, size=(N, K // G)).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[:, ::7] *= 1e-4  # small activations: the x pairs staged / 16 go subnormal in f16
    _check(dev, x, codes, s, z, G, hipq.F16)


@pytest.mark.parametrize("name", ["int4_m1_18944x3584", "int4_m1_3584x18944", "int4_m64_18944x3584",
                                  "int4_m64_3584x18944"])
def test_matmul_int4_benchmark_configs(dev, name):
    c = synth.CONFIGS[name]
    g = synth.rng(c["cfg"])
    M, N, K, G = c["M"], c["N"], c["K"], c["G"]
    codes, s, z = synth.int4_weight(N, K, G, g)
    x = synth.activations(M, K, g)
    _check(dev, x, codes, s, z, G, hipq.F16)  # every row


def _int4_experts(g, E, N, K, G, dev):
    host = [synth.int4_weight(N, K, G, g) for _ in range(E)]
    return host, [tuple(torch.from_numpy(a).to(dev) for a in w) for w in host]


@pytest.mark.parametrize("T,E,topk,H,I,G,xdt", [
    (5, 4, 2, 64, 32, 32, torch.float32),        # TestMoEInt4MatchesDense's shape: the generic kernel
    (1, 16, 4, 2048, 768, 128, torch.float16),   # decode: the int8-dot GEMV kernels
    (1, 16, 4, 2048, 768, 128, torch.float32),
    (3, 8, 2, 1024, 512, 64, torch.bfloat16),
    (2, 8, 8, 512, 256, 32, torch.float32),      # topk 8: four rows x eight slots per workgroup
])
def test_moe_int4_vs_light_cpu(dev, T, E, topk, H, I, G, xdt):
    """hq_moe_int4 against the restated CPU MoEInt4 (oracle.moe_int4, ops/int4.go:284-343) and
    an f64 dense block on the dequantized experts.  Bar (the north star's, for a combined MoE
    output): |y[t, n] - ref[t, n]| <= 1e-3 * sum_j |w_j| ||W_dn[e_j]_n|| ||h_j|| for every
    token and output, with h_j the f64 gated activations of slot j."""
    print(f"[case] moe_int4 T={T} E={E} topk={topk} H={H} I={I} G={G} x={xdt}", flush=True)
    g = synth.rng(3000 + T + H + I)
    gu_h, gu_d = _int4_experts(g, E, 2 * I, H, G, dev)
    dn_h, dn_d = _int4_experts(g, E, H, I, G, dev)
    ids = np.concatenate([g.choice(E, size=topk, replace=False) for _ in range(T)]).astype(np.int64)
    w = g.random(T * topk).astype(np.float32)
    x = g.standard_normal((T, H)).astype(np.float32)
    xt = torch.from_numpy(x).to(xdt)
    xw = xt.float().numpy()
    got = hipq.moe_int4(xt.to(dev), gu_d, dn_d, torch.from_numpy(ids).to(dev), torch.from_numpy(w).to(dev), topk, G)
    torch.cuda.synchronize()
    got = got.float().cpu().numpy()
    want = oracle.moe_int4(xw, gu_h, dn_h, ids, w, topk, G)
    # f64 dense on the dequantized experts, and the normaliser
    ref = np.zeros((T, H))
    norm = np.zeros((T, H))
    wdn = {}
    for t in range(T):
        for j in range(topk):
            e = ids[t * topk + j]
            wg = oracle.int4_dequant(*gu_h[e], 2 * I, H, G).astype(np.float64)
            if e not in wdn:
                wdn[e] = oracle.int4_dequant(*dn_h[e], H, I, G).astype(np.float64)
            gg, uu = wg[:I] @ xw[t].astype(np.float64), wg[I:] @ xw[t].astype(np.float64)
            hj = gg / (1 + np.exp(-gg)) * uu
            ref[t] += float(w[t * topk + j]) * (wdn[e] @ hj)
            norm[t] += abs(float(w[t * topk + j])) * np.linalg.norm(wdn[e], axis=1) * np.linalg.norm(hj)
    norm += 1e-30
    err_cpu = np.max(np.abs(got - want) / norm)
    err_f64 = np.max(np.abs(got - ref) / norm)
    assert err_cpu <= 1e-3, f"vs Light CPU: {err_cpu:.3g}"
    assert err_f64 <= 1e-3, f"vs f64: {err_f64:.3g}"


@pytest.mark.parametrize("M,N,K,G,kind", [
    (24, 15400, 1024, 128, "light"),   # two 16-row x tiles, a 40-row last column tile
    (40, 16000, 512, 256, "light"),    # four chunks over eight waves (some own none), G > 128
    (9, 20480, 2048, 128, "light"),    # one x tile, rows past M clamped
    (64, 15400, 768, 128, "frac"),     # non-integral zero points: the second FMA subtracts z s'
    (64, 15400, 768, 128, "wide"),     # integral zero points beyond 64
    (48, 15400, 1536, 128, "tiny"),    # scales 1e-7 .. 1e-4 in a row: the per-row exponent
    (40, 15400, 8192, 128, "light"),   # K / G = 64 groups: every lane stages one group's scale
])
def test_matmul_int4_f16_one_launch(dev, M, N, K, G, kind):
    """F16 x, 8 < M <= 64, 80-row column tiles filling the chip: the one-launch kernel (one
    workgroup per CU over all of K) against the f64 reference and Light's CPU path."""
    rng = np.random.default_rng(M * 3 + N + K + G)
    codes, s, z = light_int4(rng, N, K, G)
    if kind == "frac":
        z = (rng.random((N, K // G)) * 15).astype(np.float32)
    elif kind == "wide":
        z = rng.integers(60, 100, size=(N, K // G)).astype(np.float32)
    elif kind == "tiny":
        s = (10.0 ** rng.uniform(-7, -4, size=(N, K // G))).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    _check(dev, x, codes, s, z, G, hipq.F16)


@pytest.mark.parametrize("M,N,K,G", [
    (33, 1000, 1024, 128), (64, 18944, 3584, 128), (17, 300, 2048, 256),
    (64, 15400, 8192, 128),  # 17 groups per split: scales / zeros past 64 KB of LDS
])
def test_matmul_int4_f16_split_k_streams_and_repeats(dev, M, N, K, G):
    """F16 x, 8 < M <= 64, split over K: matches the f64 reference, and repeated calls -- on the
    default stream and on twenty other streams (each with its own library workspace) -- give
    the same bits."""
    rng = np.random.default_rng(M + N + K)
    codes, s, z = light_int4(rng, N, K, G)
    x = rng.standard_normal((M, K)).astype(np.float32)
    _check(dev, x, codes, s, z, G, hipq.F16)
    xt = torch.from_numpy(x).to(torch.float16).to(dev)
    ct, st, zt = _t(codes, dev), _t(s, dev), _t(z, dev)
    first = hipq.int4_matmul(xt, ct, st, zt, G)
    again = [hipq.int4_matmul(xt, ct, st, zt, G) for _ in range(3)]
    other = torch.cuda.Stream(device=dev)
    outs = []
    for i in range(20):
        st2 = torch.cuda.Stream(device=dev) if i else other
        with torch.cuda.stream(st2):
            outs.append(hipq.int4_matmul(xt, ct, st, zt, G, stream=st2))
    torch.cuda.synchronize()
    for y in again + outs:
        assert torch.equal(y, first)
