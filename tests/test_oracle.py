"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each check is chosen so a plausible restatement mistake (wrong nibble, wrong
scale index, fused vs unfused rounding, dropped min term, wrong summation
order) fails at least one of them.  Mirrors Light's own CPU tests:
quant/q4_k_test.go, quant/q6_k_test.go, kernels/cpu/qdecode_test.go,
ops/matmul_q_cpu_test.go, ops/matmul_q_test.go, ops/int4_test.go, ops/moe_test.go.
"""
import json
import os

import numpy as np
import pytest

import oracle
from _util import light_bound_ok, max_rel, random_blocks

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "dequant_kat.json")
DT = {"Q4_0": oracle.Q4_0, "Q5_0": oracle.Q5_0, "Q8_0": oracle.Q8_0, "Q4_K": oracle.Q4_K, "Q5_K": oracle.Q5_K,
      "Q6_K": oracle.Q6_K}


# ---- dtype/half.go -------------------------------------------------------

def test_half_to_f32_exhaustive():
    """All 65536 f16 patterns widen like IEEE (TestF16RowF16C, kernels/cpu/qdecode_test.go:116-138)."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    scalar = np.array([oracle.half_to_f32(b) for b in bits], np.float32)
    avx = oracle.half_to_f32_avx2(bits)
    fin = np.isfinite(want) | np.isinf(want)
    assert np.array_equal(scalar[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.array_equal(avx[fin].view(np.uint32), want[fin].view(np.uint32))
    nan = ~fin
    # Half.ToF32 canonicalises NaN to 0x7fc00000 with the sign kept.
    assert np.all((scalar[nan].view(np.uint32) & 0x7fffffff) == 0x7fc00000)


def test_half_from_f32_rne():
    g = np.random.default_rng(1)
    u = g.integers(0, 2 ** 32, size=1 << 16, dtype=np.uint64).astype(np.uint32)
    # plus exact ties at every f16 exponent and the subnormal range
    ties = (np.arange(0, 31, dtype=np.uint32) + 112) << 23 | 0x1000
    sub = np.float32(2.0 ** -26) * np.arange(1, 4000, dtype=np.float32)
    f = np.concatenate([u.view(np.float32), ties.view(np.float32), sub, -sub])
    f = f[np.isfinite(f)]
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    # Light's HalfFromF32 flushes |x| < 2^-24 to signed zero (dtype/half.go:43-46),
    # where IEEE would round (2^-25, 2^-24) up to the smallest subnormal.
    tiny = np.abs(f) < np.float32(2.0 ** -24)
    want = np.where(tiny, np.where(np.signbit(f), 0x8000, 0).astype(np.uint16), want)
    got = np.array([oracle.half_from_f32(v) for v in f], np.uint16)
    assert np.array_equal(got, want)
    assert tiny.sum() > 0


def test_bf16_from_f32_rne():
    import torch
    g = np.random.default_rng(2)
    u = g.integers(0, 2 ** 32, size=1 << 15, dtype=np.uint64).astype(np.uint32)
    ties = (g.integers(1, 254, size=4096).astype(np.uint32) << 23) | 0x8000 | (
        g.integers(0, 2, size=4096).astype(np.uint32) << 16)
    f = np.concatenate([u, ties]).view(np.float32)
    f = f[np.isfinite(f)]
    want = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([oracle.bf16_from_f32(v) for v in f], np.uint16)
    assert np.array_equal(got, want)
    nan = np.array([0x7f800001, 0xffc00001], np.uint32).view(np.float32)
    for v, b in zip(nan, [0x7fc0, 0xffc0]):
        assert oracle.bf16_from_f32(v) == b  # quiet bit set, top bits kept


# ---- known answers (golden fixtures from Light's tests) -----------------

def _kat_cases():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _kat_cases(), ids=lambda c: c["name"])
@pytest.mark.parametrize("avx2", [False, True])
def test_dequant_known_answers(case, avx2):
    raw = np.frombuffer(bytes.fromhex(case["blocks"]), np.uint8)
    got = oracle.decode_row(DT[case["dtype"]], raw, case["n"], avx2=avx2)
    if case["checks"] == "all":
        want = np.array(case["want"], np.float32)
        assert np.array_equal(got, want), np.nonzero(got != want)
    else:
        for idx, want in case["want"].items():
            assert got[int(idx)] == np.float32(want)


# ---- decoders: scalar vs AVX2 bit identity + closed forms ---------------

@pytest.mark.parametrize("dt", [oracle.Q4_0, oracle.Q5_0, oracle.Q8_0, oracle.Q4_K, oracle.Q6_K])
def test_avx2_decoders_exact(dt):
    """TestAVX2DecodersExact (kernels/cpu/qdecode_test.go:38-82)."""
    g = np.random.default_rng(dt)
    K = 2048
    raw = random_blocks(g, dt, 4, K)
    rb = len(raw) // 4
    for n in range(4):
        a = oracle.decode_row(dt, raw[n * rb:(n + 1) * rb], K)
        b = oracle.decode_row(dt, raw[n * rb:(n + 1) * rb], K, avx2=True)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q4_k_closed_forms():
    """q = 0 gives exactly -(dmin*m); sc = 0 and m = 0 gives 0; the nibble order is pinned by q = index."""
    from light_amd import synth
    g = np.random.default_rng(5)
    d = np.float16(0.0123).view(np.uint16)
    dmin = np.float16(0.0071).view(np.uint16)
    sc = g.integers(0, 64, size=(1, 8))
    mn = g.integers(0, 64, size=(1, 8))
    blk = synth.pack_q4_k(np.array([d]), np.array([dmin]), sc, mn, np.zeros((1, 256)))
    y = oracle.decode_row(oracle.Q4_K, blk, 256)
    dm = np.float32(np.float16(0.0071))
    want = np.repeat(-(dm * mn[0].astype(np.float32)), 32)
    assert np.array_equal(y, want.astype(np.float32))
    q = (np.arange(256) % 16).reshape(1, 256)
    blk = synth.pack_q4_k(np.array([d]), np.array([dmin]), np.ones((1, 8)), np.zeros((1, 8)), q)
    y = oracle.decode_row(oracle.Q4_K, blk, 256)
    assert np.array_equal(y, np.float32(np.float16(0.0123)) * q[0].astype(np.float32))


def test_q6_k_closed_forms():
    """Element order and scale index: raw = element index mod 64, sc[s] = s - 8."""
    from light_amd import synth
    d = np.float16(0.5).view(np.uint16)
    raw = (np.arange(256) % 64).reshape(1, 256)
    sc = (np.arange(16) - 8).reshape(1, 16)
    blk = synth.pack_q6_k(np.array([d]), sc, raw)
    y = oracle.decode_row(oracle.Q6_K, blk, 256)
    i = np.arange(256)
    want = (np.float32(0.5) * (i // 16 - 8).astype(np.float32)) * ((i % 64) - 32).astype(np.float32)
    assert np.array_equal(y, want.astype(np.float32))


def test_q4_0_q5_0_closed_forms():
    """Element order (low nibbles 0..15, high 16..31; qh bit j = element j) pinned by q = index."""
    from light_amd import synth
    d = np.array([np.float16(0.375).view(np.uint16)])
    q = np.arange(32).reshape(1, 32)
    y = oracle.decode_row(oracle.Q4_0, synth.pack_q4_0(d, q % 16), 32)
    assert np.array_equal(y, np.float32(0.375) * ((q[0] % 16) - 8).astype(np.float32))
    y = oracle.decode_row(oracle.Q5_0, synth.pack_q5_0(d, q), 32)
    assert np.array_equal(y, np.float32(0.375) * (q[0] - 16).astype(np.float32))
    # qh bits only: q = 16 * (index odd) -> every odd element 0, even -16 d.
    q = (16 * (np.arange(32) % 2)).reshape(1, 32)
    y = oracle.decode_row(oracle.Q5_0, synth.pack_q5_0(d, q), 32, avx2=True)
    assert np.array_equal(y, np.float32(0.375) * (q[0] - 16).astype(np.float32))


def test_q5_k_reduces_to_q4_k():
    """Q5_K with every fifth bit clear equals Q4_K on the same header and nibbles; a set fifth
    bit adds exactly 16 (d sc) before the min is subtracted."""
    from light_amd import synth
    g = np.random.default_rng(9)
    nb = 6
    d = synth._f16_bits(np.abs(g.standard_normal(nb)) * 1e-2)
    dmin = synth._f16_bits(np.abs(g.standard_normal(nb)) * 1e-2)
    sc = g.integers(0, 64, size=(nb, 8))
    mn = g.integers(0, 64, size=(nb, 8))
    q = g.integers(0, 16, size=(nb, 256))
    a = oracle.decode_row(oracle.Q5_K, synth.pack_q5_k(d, dmin, sc, mn, q), nb * 256)
    b = oracle.decode_row(oracle.Q4_K, synth.pack_q4_k(d, dmin, sc, mn, q), nb * 256)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    c = oracle.decode_row(oracle.Q5_K, synth.pack_q5_k(d, dmin, sc, mn, q + 16), nb * 256)
    df = d.view(np.float16).astype(np.float32)
    dm = dmin.view(np.float16).astype(np.float32)
    j = np.arange(256) // 32
    for b_ in range(nb):
        ds = df[b_] * sc[b_, j].astype(np.float32)
        want = ds * (q[b_] + 16).astype(np.float32) - dm[b_] * mn[b_, j].astype(np.float32)
        assert np.array_equal(c[b_ * 256:(b_ + 1) * 256], want.astype(np.float32))


def test_q8_0_closed_form():
    from light_amd import synth
    qs = (np.arange(32) - 16).reshape(1, 32).astype(np.int8)
    blk = synth.pack_q8_0(np.array([np.float16(0.25).view(np.uint16)]), qs)
    y = oracle.decode_row(oracle.Q8_0, blk, 32)
    assert np.array_equal(y, 0.25 * (np.arange(32) - 16).astype(np.float32))


def test_int4_rows_exact():
    g = np.random.default_rng(7)
    for G in (32, 64, 128):
        K = 512
        codes = g.integers(0, 2 ** 32, size=K // 8, dtype=np.uint64).astype(np.uint32)
        s = (g.random(K // G) * 0.02 + 1e-3).astype(np.float32)
        z = g.integers(0, 16, size=K // G).astype(np.float32)
        a = oracle.int4_row(codes, s, z, K, G)
        b = oracle.int4_row(codes, s, z, K, G, avx2=True)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        # closed form: nibble j of word c is element 8c + j; W = s * (q - z)
        q = (codes[:, None] >> (4 * np.arange(8, dtype=np.uint32))[None, :]) & 15
        want = np.repeat(s, G) * (q.reshape(-1).astype(np.float32) - np.repeat(z, G))
        assert np.array_equal(a, want.astype(np.float32))


def test_int4_dequant_bf16_rounds_once():
    """TestDequantizeInt4 (ops/int4_test.go:47-81): BF16 = BF16FromF32(F32 value)."""
    import torch
    g = np.random.default_rng(3)
    N, K, G = 24, 256, 64
    codes = g.integers(0, 2 ** 32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = (g.random((N, K // G)) * 0.02 + 1e-3).astype(np.float32)
    z = g.integers(0, 16, size=(N, K // G)).astype(np.float32)
    f32 = oracle.int4_dequant(codes, s, z, N, K, G, oracle.F32)
    b16 = oracle.int4_dequant(codes, s, z, N, K, G, oracle.BF16)
    want = torch.from_numpy(f32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(b16, want)


# ---- simd order -----------------------------------------------------------

@pytest.mark.parametrize("n", [0, 1, 7, 8, 9, 31, 32, 33, 63, 100, 257, 4096])
def test_dot_order(n):
    g = np.random.default_rng(n)
    a = g.standard_normal(n).astype(np.float32)
    b = g.standard_normal(n).astype(np.float32)
    x = oracle.dot(a, b)
    y = oracle.dot(a, b, lanes=True)
    assert np.float32(x).view(np.uint32) == np.float32(y).view(np.uint32)
    ref = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
    assert abs(float(x) - ref) <= 1e-5 * (1 + float(np.sum(np.abs(a.astype(np.float64) * b))))


def test_mattb_tiles_match_dot():
    """MatTB's 4x3 tiles and its Dot edges give the same result as f64 within Light's bound."""
    g = np.random.default_rng(11)
    a = g.standard_normal((9, 64)).astype(np.float32)
    w = g.standard_normal((7, 64)).astype(np.float32)
    out = oracle.mattb(a, w)
    ref = a.astype(np.float64) @ w.astype(np.float64).T
    mag = np.abs(a.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    assert light_bound_ok(out, ref, mag)
    # the Dot edges (row 8, col 6) equal dotAVX2 bit for bit
    assert out[8, 6] == oracle.dot(a[8], w[6])


# ---- Light's CPU qmatmul ------------------------------------------------

@pytest.mark.parametrize("dt", [oracle.Q4_0, oracle.Q5_0, oracle.Q8_0, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K])
@pytest.mark.parametrize("M", [1, 9])
def test_matmul_q_vs_f64(dt, M):
    """TestMatMulQCPUKernels (ops/matmul_q_cpu_test.go:19-81): N=37, K=512, bound 1e-5 (1 + sum|xw|)."""
    g = np.random.default_rng(100 + dt + M)
    N, K = 37, 512
    raw = random_blocks(g, dt, N, K)
    x = g.standard_normal((M, K)).astype(np.float32)
    y = oracle.matmul_q(x, raw, N, K, dt)
    wd = oracle.dequant(dt, raw, N * K).reshape(N, K)
    ref, mag, _, _ = oracle.matmul_f64(x, wd)
    assert light_bound_ok(y, ref, mag)


@pytest.mark.parametrize("dt", [oracle.Q4_0, oracle.Q5_0, oracle.Q8_0, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K])
def test_matmul_q_matches_dequant_matmul(dt):
    """TestMatMulQCPUMatchesDequant (ops/matmul_q_test.go:75-103): rel 1e-5 vs dequant + MatMul."""
    g = np.random.default_rng(3 + dt)
    M, N, K = 5, 7, 512
    x = (g.random((M, K)) * 2 - 1).astype(np.float32)
    raw = random_blocks(g, dt, N, K)
    got = oracle.matmul_q(x, raw, N, K, dt)
    wd = oracle.dequant(dt, raw, N * K).reshape(N, K)
    assert max_rel(got, oracle.mattb(x, wd)) <= 1e-5
    # threading does not change bits
    assert np.array_equal(got, oracle.matmul_q(x, raw, N, K, dt, threads=1))


def test_int4_matmul_vs_f64():
    """TestMatMulInt4 (ops/int4_test.go:83-145) CPU leg, tol 1e-4 relative."""
    g = np.random.default_rng(4)
    N, K, G = 96, 256, 64
    codes = g.integers(0, 2 ** 32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = (g.random((N, K // G)) * 0.02 + 1e-3).astype(np.float32)
    z = g.integers(0, 16, size=(N, K // G)).astype(np.float32)
    wd = oracle.int4_dequant(codes, s, z, N, K, G)
    for M in (1, 3, 8, 9):
        x = g.standard_normal((M, K)).astype(np.float32)
        y = oracle.int4_matmul(x, codes, s, z, N, K, G)
        ref, _, _, _ = oracle.matmul_f64(x, wd)
        scale = np.maximum(1.0, np.abs(ref))
        assert np.max(np.abs(y - ref) / scale) <= 1e-4


# ---- MoE -------------------------------------------------------------------

def test_moe_routing_invariants():
    """ops/moe_test.go:63-88: sorted experts non-decreasing; pairs a permutation; stable."""
    from light_amd import synth
    g = synth.rng(4)
    ids, w = synth.moe_routing(37, 16, 4, g)
    assert np.allclose(w.reshape(37, 4).sum(1), 1, atol=1e-6)
    se, sp = oracle.moe_route_from_ids(ids)
    assert np.all(np.diff(se) >= 0)
    assert np.array_equal(np.sort(sp), np.arange(ids.size))
    assert np.array_equal(ids[sp], se)
    for e in np.unique(se):  # stable: pair ids increase inside each expert segment
        assert np.all(np.diff(sp[se == e]) > 0)
    se2, sp2 = synth.sort_pairs(ids)
    assert np.array_equal(se, se2) and np.array_equal(sp, sp2)


@pytest.mark.parametrize("per_pair", [False, True])
def test_moe_gemm_q_vs_expert_loop(per_pair):
    """MoEGemmQ CPU = dequant + MoEGemm, against the per-expert loop of ops/moe_test.go:16-50 in f64."""
    from light_amd import synth
    g = synth.rng(21)
    T, E, K, N, topk = 21, 3, 256, 40, 2
    w = synth.gguf_weight(oracle.Q4_K, E * N, K, g)
    ids, tw = synth.moe_routing(T, E, topk, g)
    se, sp = oracle.moe_route_from_ids(ids)
    rows = T * topk if per_pair else T
    x = g.standard_normal((rows, K)).astype(np.float32)
    got = oracle.moe_gemm_q(x, w, oracle.Q4_K, E, N, K, sp, se, topk, topk_w=tw if per_pair else None)
    wd = oracle.dequant(oracle.Q4_K, w, E * N * K).reshape(E, N, K).astype(np.float64)
    for p in range(T * topk):
        r = p if per_pair else p // topk
        ref = wd[ids[p]] @ x[r].astype(np.float64) * (tw[p] if per_pair else 1.0)
        mag = np.abs(wd[ids[p]]) @ np.abs(x[r].astype(np.float64))
        assert np.all(np.abs(got[p] - ref) <= 1e-5 * (1 + mag))
    comb = oracle.moe_combine(got, topk)
    assert np.array_equal(comb, (got.reshape(T, topk, N)[:, 0] + got.reshape(T, topk, N)[:, 1]))


# ---- q8_1 quantizer (specification-pinned) ---------------------------------

def test_quantize_q8_1_spec():
    g = np.random.default_rng(8)
    x = (g.standard_normal(32 * 512) * np.repeat(g.random(512) * 10, 32)).astype(np.float32)
    x[:32] = 0  # all-zero block
    x[32:64] = np.linspace(-3, 3, 32, dtype=np.float32)
    q1 = oracle.quantize_q8_1(x).reshape(-1, 36)
    q0 = oracle.quantize_q8_0(x).reshape(-1, 34)
    d = q1[:, 0:2].copy().view("<u2").view(np.float16).astype(np.float32)[:, 0]
    s = q1[:, 2:4].copy().view("<u2").view(np.float16).astype(np.float32)[:, 0]
    q = q1[:, 4:].view(np.int8).astype(np.int32)
    # same d and q as Light's Q8_0 encoder (the rounding rule q8_1 adopts)
    assert np.array_equal(q1[:, 0:2], q0[:, 0:2])
    assert np.array_equal(q1[:, 4:], q0[:, 2:])
    assert np.all(np.abs(q) <= 127)
    assert np.all(q1[0] == 0)
    blocks = x.reshape(-1, 32)
    amax = np.abs(blocks).max(1)
    dd = amax / np.float32(127)
    # round trip within d/2 (+1 ulp slack for the f16 storage of d)
    recon = q.astype(np.float64) * dd[:, None]
    assert np.all(np.abs(recon - blocks) <= dd[:, None] * 0.5 * (1 + 1e-6) + 1e-30)
    # at least one element of every non-zero block saturates to +-127
    nz = amax > 0
    assert np.all(np.abs(q[nz]).max(1) == 127)
    # s = f16(sum q * d): within half an f16 ulp of the exact product
    exact = q.sum(1).astype(np.float64) * dd
    assert np.all(np.abs(s - exact) <= np.abs(exact) * 2.0 ** -11 + 2.0 ** -25)
    assert np.all(np.abs(d - dd) <= dd * 2.0 ** -11 + 2.0 ** -25)


def test_gated_tail_closed_forms():
    """or_gated: SiLU = x * sigmoid(x) and GELU = 0.5 x (1 + erf(x / sqrt 2)) (f64 closed forms)."""
    from scipy.special import erf
    g = np.concatenate([np.array([0.0, -0.0, 1e-30, 30.0, -30.0, 88.0, -88.0], np.float32),
                        (np.random.default_rng(5).standard_normal(4096) * 4).astype(np.float32)])
    u = np.random.default_rng(6).standard_normal(g.size).astype(np.float32)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    silu = oracle.gated(g, u, 0)
    want = g64 / (1.0 + np.exp(-g64)) * u64
    assert np.allclose(silu, want, rtol=2e-6, atol=1e-30)
    gelu = oracle.gated(g, u, 1)
    want = 0.5 * g64 * (1.0 + erf(g64 / np.sqrt(2.0))) * u64
    assert np.allclose(gelu, want, rtol=2e-6, atol=1e-30)
    assert silu[0] == 0.0 and gelu[0] == 0.0
    assert abs(silu[4]) < 1e-10 and gelu[4] == 0.0  # x = -30: SiLU ~ -2.8e-12 * u, GELU underflows to 0


# ---- MoERoute -------------------------------------------------------------

@pytest.mark.parametrize("T,E,topk", [(1, 8, 2), (7, 4, 2), (33, 128, 8), (5, 60, 60)])
@pytest.mark.parametrize("normalize", [False, True])
def test_moe_route_pinned(T, E, topk, normalize):
    """TestMoEGemmMatchesExpertLoop's routing checks (ops/moe_test.go:63-88) plus an independent
    encoding: numpy's stable argsort of -probs (TopK keeps index order on ties), a float32
    loop for Sum, and numpy's stable argsort of the flat ids (Sort)."""
    g = np.random.default_rng(T * 100 + E + topk)
    logits = g.standard_normal((T, E)).astype(np.float32)
    probs = np.exp(logits - logits.max(axis=1, keepdims=True))
    probs = (probs / probs.sum(axis=1, keepdims=True)).astype(np.float32)
    probs[:, E // 2] = probs[:, 0]  # ties
    ids, w, sp, se = oracle.moe_route(probs, topk, normalize)
    want_ids = np.argsort(-probs, axis=1, kind="stable")[:, :topk]
    assert np.array_equal(ids, want_ids)
    vals = np.take_along_axis(probs, want_ids, axis=1)
    if normalize:
        for t in range(T):
            den = np.float32(0)
            for j in range(topk):
                den = np.float32(den + vals[t, j])
            vals[t] = vals[t] / den
        assert np.allclose(w.reshape(T, topk).sum(axis=1), 1, atol=1e-5)
    assert np.array_equal(w.view(np.uint32), vals.reshape(-1).view(np.uint32))
    order = np.argsort(ids.reshape(-1), kind="stable")
    assert np.array_equal(sp, order) and np.array_equal(se, ids.reshape(-1)[order])
    assert np.all(np.diff(se) >= 0) and np.array_equal(np.sort(sp), np.arange(T * topk))


def _light_int4(g, N, K, G):
    """randomInt4 of ops/int4_test.go:16-32: random code words, s ~ U[1e-3, 2.1e-2), z ~ U{0..15}."""
    codes = g.integers(0, 2 ** 32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = (g.random((N, K // G)) * 0.02 + 1e-3).astype(np.float32)
    z = g.integers(0, 16, size=(N, K // G)).astype(np.float32)
    return codes, s, z


@pytest.mark.parametrize("seed", [7, 8])
def test_moe_int4_matches_dense(seed):
    """TestMoEInt4MatchesDense (ops/int4_test.go:150-206): the restated CPU MoEInt4 against
    sum_j w_j * down_e(silu(gate_e x) * up_e x) in f64 on the dequantized experts, within
    Light's 1e-4 (1 + |want|)."""
    T, H, I, E, topk, G = 5, 64, 32, 4, 2, 32
    g = np.random.default_rng(seed)
    gu = [_light_int4(g, 2 * I, H, G) for _ in range(E)]
    dn = [_light_int4(g, H, I, G) for _ in range(E)]
    x = g.standard_normal((T, H)).astype(np.float32)
    ids = np.array([0, 2, 2, 1, 3, 0, 2, 3, 1, 2], np.int64)
    ws = g.random(T * topk).astype(np.float32)
    got = oracle.moe_int4(x, gu, dn, ids, ws, topk, G)
    for t in range(T):
        want = np.zeros(H)
        for j in range(topk):
            e = ids[t * topk + j]
            wg = oracle.int4_dequant(*gu[e], 2 * I, H, G).astype(np.float64)
            wd = oracle.int4_dequant(*dn[e], H, I, G).astype(np.float64)
            gg = wg[:I] @ x[t].astype(np.float64)
            uu = wg[I:] @ x[t].astype(np.float64)
            h = gg / (1 + np.exp(-gg)) * uu
            want += float(ws[t * topk + j]) * (wd @ h)
        assert np.all(np.abs(got[t] - want) <= 1e-4 * (1 + np.abs(want))), t


def test_moe_int4_slot_order_sum():
    """The pair rows are added onto zero in slot order (moeInt4Rows' o[k] += p[k]): with one
    expert routed twice per token the result is exactly 0 + w0 y + w1 y in f32."""
    T, H, I, E, topk, G = 2, 64, 64, 2, 2, 32
    g = np.random.default_rng(3)
    gu = [_light_int4(g, 2 * I, H, G) for _ in range(E)]
    dn = [_light_int4(g, H, I, G) for _ in range(E)]
    x = g.standard_normal((T, H)).astype(np.float32)
    ids = np.array([1, 1, 0, 0], np.int64)
    ws = np.array([0.25, 0.75, 0.5, 0.125], np.float32)
    got = oracle.moe_int4(x, gu, dn, ids, ws, topk, G)
    for t, e in ((0, 1), (1, 0)):
        gu_e = oracle.int4_matmul(x[t:t + 1], *gu[e], 2 * I, H, G)
        h = oracle.gated(gu_e[:, :I].copy(), gu_e[:, I:].copy(), 0)
        y = oracle.int4_matmul(h, *dn[e], H, I, G)[0]
        want = (np.float32(0) + ws[2 * t] * y).astype(np.float32)
        want = (want + ws[2 * t + 1] * y).astype(np.float32)
        assert np.array_equal(got[t], want)
