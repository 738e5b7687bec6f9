"""CPU oracle for Light's quantized-matmul path -- TEST INFRASTRUCTURE ONLY.

A ctypes front end over ``liboracle.so`` (built from ``oracle.c`` by the
Makefile beside it).  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or the timed CPU baseline; the product path (``light_amd``) never
does.

Parity status of each function (how it is pinned):

* ``half_to_f32`` / ``half_from_f32`` / ``bf16_from_f32``: all 65536 f16
  patterns against numpy's IEEE conversion; f32 -> f16 / bf16 on 2^20 random
  patterns plus ties against numpy / torch round-to-nearest-even.
* ``decode_row`` / ``dequant`` (Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K): Light's
  known-answer tests (quant/q4_0_test.go, quant/others_test.go,
  quant/q4_k_test.go, quant/q5_k_test.go, quant/q6_k_test.go) as golden
  fixtures, scalar vs AVX2 bit identity (Light's TestAVX2DecodersExact),
  closed forms on special blocks (q = 0, scale = 0, min = 0), and Q5_K with
  every fifth bit clear against Q4_K on the same header and nibbles.
* ``int4_row`` / ``int4_dequant``: scalar vs AVX2 bit identity; closed forms
  (codes all equal, z = q) and the BF16 round-once rule.
* ``dot`` / ``mattb``: intrinsics vs a lane-by-lane scalar encoding of the same
  order (bit identity), and the f64 bound 1e-5 (1 + sum|x w|).
* ``matmul_q`` / ``int4_matmul``: the f64 oracle with Light's own bound
  (ops/matmul_q_cpu_test.go:66-76).
* ``moe_gemm_q`` / ``moe_route_from_ids`` / ``moe_combine``: Light's routing
  invariants (ops/moe_test.go:63-88) and a per-expert loop in f64.
* ``moe_route``: numpy's stable argsort of -probs (top-k with index-order ties),
  a float32 loop for the renormalisation, Light's invariants (weights sum to 1,
  sorted experts non-decreasing, pairs a permutation), on rows with ties.
* ``gated``: SiLU against x * sigmoid(x) in f64 and GELU against scipy's erf
  (closed forms), at special points (0, large |x|) and on random data.
* ``int4_from_gptq`` / ``int4_from_awq`` (numpy restatements of quant.FromGPTQ /
  quant.FromAWQ): PARITY UNPINNED against Light itself -- its only tests of them
  (quant/int4_test.go:80-114) read real checkpoints, absent offline.  They are
  checked against the producers' published packing rules (AutoGPTQ: qweight
  packed along K, qzeros along N storing zero - 1; AutoAWQ: order
  0, 2, 4, 6, 1, 3, 5, 7), written independently in the tests as packers, by
  round trips and single-nibble known answers.
* ``quantize_q8_1``: specification only (Light has no q8_1 encoder): layout,
  |q| <= 127, round trip within d/2, all-zero block, and the q8_0 encoder
  (same rounding rule) on the same data.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

F16, BF16, F32 = 0, 1, 2
Q4_0, Q5_0, Q8_0, Q8_1, Q4_K, Q5_K, Q6_K = 13, 15, 17, 18, 21, 22, 23
BLOCK = {Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q8_1: (32, 36), Q4_K: (256, 144), Q5_K: (256, 176),
         Q6_K: (256, 210)}

_lib = None


def build():
    """Compile liboracle.so with make (gcc)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


P = ctypes.c_void_p
I64 = ctypes.c_int64
I = ctypes.c_int


def _declare(L):
    sig = {
        "or_half_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "or_half_from_f32": (ctypes.c_uint16, [ctypes.c_float]),
        "or_bf16_from_f32": (ctypes.c_uint16, [ctypes.c_float]),
        "or_half_to_f32_avx2": (None, [P, P, I64]),
        "or_decode_row": (I, [I, P, I64, P]),
        "or_decode_row_avx2": (I, [I, P, I64, P]),
        "or_int4_row": (None, [P, P, P, P, I64, I]),
        "or_int4_row_avx2": (None, [P, P, P, P, I64, I]),
        "or_dequant": (I, [I, P, I64, P]),
        "or_int4_dequant": (I, [P, P, P, P, I, I64, I64, I]),
        "or_dot_avx2": (ctypes.c_float, [P, P, I64]),
        "or_dot_lanes": (ctypes.c_float, [P, P, I64]),
        "or_mattb": (None, [P, I64, P, I64, P, I64, I64, I64, I64]),
        "or_matmul_q": (I, [P, P, P, I64, I64, I64, I, I]),
        "or_int4_matmul": (I, [P, P, P, P, P, I64, I64, I64, I, I]),
        "or_moe_route_from_ids": (None, [P, I64, P, P]),
        "or_moe_route": (None, [P, I64, I64, I, I, P, P, P, P]),
        "or_moe_gemm_f32": (I, [P, P, P, P, P, P, I64, I64, I64, I64, I, I, I]),
        "or_moe_gemm_q": (I, [P, P, I, P, P, P, P, I64, I64, I64, I64, I64, I, I, I, P]),
        "or_moe_combine": (None, [P, P, I64, I64, I]),
        "or_gated": (None, [P, P, P, I64, I]),
        "or_quantize_q8_0": (None, [P, I64, P]),
        "or_quantize_q8_1": (None, [P, I64, P]),
        "or_matmul_f64": (None, [P, P, I64, I64, I64, P, P, P, P, I]),
        "or_hw_threads": (I, []),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def hw_threads():
    return lib().or_hw_threads()


def half_to_f32(h):
    return lib().or_half_to_f32(int(h))


def half_from_f32(f):
    return lib().or_half_from_f32(float(f))


def bf16_from_f32(f):
    return lib().or_bf16_from_f32(float(f))


def half_to_f32_avx2(h):
    h = _c(h, np.uint16)
    out = np.zeros(h.size, np.float32)
    lib().or_half_to_f32_avx2(_p(h), _p(out), h.size)
    return out


def decode_row(dt, raw, K, avx2=False):
    raw = _c(raw, np.uint8)
    out = np.zeros(K, np.float32)
    f = lib().or_decode_row_avx2 if avx2 else lib().or_decode_row
    if f(dt, _p(raw), K, _p(out)) != 0:
        raise ValueError("decode_row: bad dtype or K")
    return out


def dequant(dt, raw, n):
    raw = _c(raw, np.uint8)
    out = np.zeros(n, np.float32)
    if lib().or_dequant(dt, _p(raw), n, _p(out)) != 0:
        raise ValueError("dequant: bad dtype or n")
    return out


def int4_row(codes, s, z, K, G, avx2=False):
    codes, s, z = _c(codes, np.uint32), _c(s, np.float32), _c(z, np.float32)
    out = np.zeros(K, np.float32)
    f = lib().or_int4_row_avx2 if avx2 else lib().or_int4_row
    f(_p(codes), _p(s), _p(z), _p(out), K, G)
    return out


def int4_dequant(codes, s, z, N, K, G, out_dt=F32):
    codes, s, z = _c(codes, np.uint32), _c(s, np.float32), _c(z, np.float32)
    out = np.zeros(N * K, np.float32 if out_dt == F32 else np.uint16)
    if lib().or_int4_dequant(_p(codes), _p(s), _p(z), _p(out), out_dt, N, K, G) != 0:
        raise ValueError("int4_dequant: bad args")
    return out.reshape(N, K)


def dot(a, b, lanes=False):
    a, b = _c(a, np.float32), _c(b, np.float32)
    f = lib().or_dot_lanes if lanes else lib().or_dot_avx2
    return np.float32(f(_p(a), _p(b), a.size))


def mattb(a, w):
    """out = a @ w.T with Light's MatTB order; a (m, k), w (n, k)."""
    a, w = _c(a, np.float32), _c(w, np.float32)
    m, k = a.shape
    n = w.shape[0]
    out = np.zeros((m, n), np.float32)
    lib().or_mattb(_p(a), k, _p(w), k, _p(out), n, m, n, k)
    return out


def matmul_q(x, w_raw, N, K, dt, threads=0):
    """Light's CPU MatMulQ: x (M, K) f32 times dequant(W)^T -> (M, N) f32."""
    x = _c(x, np.float32)
    w_raw = _c(w_raw, np.uint8)
    M = x.size // K
    out = np.zeros((M, N), np.float32)
    if lib().or_matmul_q(_p(x), _p(w_raw), _p(out), M, N, K, dt, threads) != 0:
        raise ValueError("matmul_q: bad args")
    return out


def int4_matmul(x, codes, s, z, N, K, G, threads=0):
    x = _c(x, np.float32)
    codes, s, z = _c(codes, np.uint32), _c(s, np.float32), _c(z, np.float32)
    M = x.size // K
    out = np.zeros((M, N), np.float32)
    if lib().or_int4_matmul(_p(x), _p(codes), _p(s), _p(z), _p(out), M, N, K, G, threads) != 0:
        raise ValueError("int4_matmul: bad args")
    return out


def moe_route_from_ids(ids):
    ids = _c(ids, np.int64).ravel()
    se = np.zeros(ids.size, np.int64)
    sp = np.zeros(ids.size, np.int64)
    lib().or_moe_route_from_ids(_p(ids), ids.size, _p(se), _p(sp))
    return se, sp


def moe_route(probs, topk, normalize=True):
    """Light's CPU MoERoute: (topk_ids (T, topk), weights (T*topk,), sorted_pairs, sorted_expts)."""
    probs = _c(probs, np.float32)
    T, E = probs.shape
    ids = np.zeros((T, topk), np.int64)
    w = np.zeros(T * topk, np.float32)
    sp = np.zeros(T * topk, np.int64)
    se = np.zeros(T * topk, np.int64)
    lib().or_moe_route(_p(probs), T, E, topk, int(bool(normalize)), _p(ids), _p(w), _p(sp), _p(se))
    return ids, w, sp, se


def moe_gemm_q(x, w_raw, dt, E, N, K, sorted_pairs, sorted_expts, topk, topk_w=None, threads=0,
               scratch=None):
    """Light's CPU MoEGemmQ: dequantize the (E, N, K) stack, then moeGemmKernel."""
    x = _c(x, np.float32)
    w_raw = _c(w_raw, np.uint8)
    sp, se = _c(sorted_pairs, np.int64), _c(sorted_expts, np.int64)
    M = sp.size
    rows = x.shape[0]
    if rows == M:
        rpp = 1
    elif rows == M // topk:
        rpp = 0
    else:
        raise ValueError("moe_gemm_q: input rows must be M or M/topk")
    tw = None if topk_w is None else _c(topk_w, np.float32)
    out = np.zeros((M, N), np.float32)
    if scratch is not None:
        assert scratch.dtype == np.float32 and scratch.size >= E * N * K
    rc = lib().or_moe_gemm_q(_p(x), _p(w_raw), dt, _p(sp), _p(se), _p(tw), _p(out), M, M, E, N, K, topk, rpp,
                             threads, _p(scratch))
    if rc != 0:
        raise ValueError("moe_gemm_q: bad args")
    return out


def moe_gemm_f32(x, w, sorted_pairs, sorted_expts, topk, topk_w=None, threads=0):
    x, w = _c(x, np.float32), _c(w, np.float32)
    E, N, K = w.shape
    sp, se = _c(sorted_pairs, np.int64), _c(sorted_expts, np.int64)
    M = sp.size
    rpp = 1 if x.shape[0] == M else 0
    tw = None if topk_w is None else _c(topk_w, np.float32)
    out = np.zeros((M, N), np.float32)
    lib().or_moe_gemm_f32(_p(x), _p(w), _p(sp), _p(se), _p(tw), _p(out), M, M, N, K, topk, rpp, threads)
    return out


def moe_combine(pair_out, topk):
    pair_out = _c(pair_out, np.float32)
    M, N = pair_out.shape
    out = np.zeros((M // topk, N), np.float32)
    lib().or_moe_combine(_p(pair_out), _p(out), M, N, topk)
    return out


def gated(g, u, act=0):
    """Light's unfused gated tail: SiLU (act 0) or GeluErf (act 1) of g, times u, in f32."""
    g = _c(g, np.float32)
    u = _c(u, np.float32)
    out = np.empty_like(g)
    lib().or_gated(_p(g), _p(u), _p(out), g.size, act)
    return out


def quantize_q8_0(x):
    x = _c(x, np.float32).ravel()
    out = np.zeros(x.size // 32 * 34, np.uint8)
    lib().or_quantize_q8_0(_p(x), x.size, _p(out))
    return out


def quantize_q8_1(x):
    x = _c(x, np.float32).ravel()
    out = np.zeros(x.size // 32 * 36, np.uint8)
    lib().or_quantize_q8_1(_p(x), x.size, _p(out))
    return out


def matmul_f64(x, w, threads=0):
    """f64 oracle: returns (ref, mag, wnorm, xnorm) for x (M, K) and dequantized w (N, K)."""
    x, w = _c(x, np.float32), _c(w, np.float32)
    M, K = x.shape
    N = w.shape[0]
    ref = np.zeros((M, N), np.float64)
    mag = np.zeros((M, N), np.float64)
    wn = np.zeros(N, np.float64)
    xn = np.zeros(M, np.float64)
    lib().or_matmul_f64(_p(x), _p(w), M, N, K, _p(ref), _p(mag), _p(wn), _p(xn), threads)
    return ref, mag, wn, xn


def moe_int4(x, gate_up, down, ids, w, topk, G, act=0, threads=0):
    """Light's CPU MoEInt4 with F32 activations (moeInt4Rows, ops/int4.go:284-343): for each
    expert in first-use order, its routed rows of x through the fused int4 MatMulInt4
    (gate-up, (R, 2I)), act(gate) * up, MatMulInt4 with down, times the pair's weight; then
    per token out = 0 + pair[slot 0] + pair[slot 1] + ... in slot order.
    gate_up / down: lists of (codes, scales, zeros) numpy arrays per expert."""
    x = _c(x, np.float32)
    T, H = x.shape
    ids = np.asarray(ids, np.int64).ravel()
    w = np.asarray(w, np.float32).ravel()
    I = down[0][0].shape[1] * 8
    used = list(dict.fromkeys(int(e) for e in ids))
    pair = np.zeros((ids.size, H), np.float32)
    for e in used:
        r = [i for i, v in enumerate(ids) if v == e]
        xg = np.ascontiguousarray(x[[i // topk for i in r]])
        c, sc, zr = gate_up[e]
        gu = int4_matmul(xg, c, sc, zr, 2 * I, H, G, threads)
        h = gated(np.ascontiguousarray(gu[:, :I]), np.ascontiguousarray(gu[:, I:]), act)
        c, sc, zr = down[e]
        y = int4_matmul(h, c, sc, zr, H, I, G, threads)
        for j, i in enumerate(r):
            pair[i] = (w[i] * y[j]).astype(np.float32)
    out = np.zeros((T, H), np.float32)
    for t in range(T):
        for j in range(topk):
            out[t] = (out[t] + pair[t * topk + j]).astype(np.float32)
    return out


def _gos(shape):
    """A shape as Go's %v prints an []int."""
    return "[" + " ".join(str(int(d)) for d in shape) + "]"


def _nib(w, j):
    return (np.asarray(w, np.uint32) >> np.uint32(4 * j)) & np.uint32(0xF)


def _canon(code):
    """Pack codes (N, K) uint8 into canonical words: nibble j of word (n, c) is code (n, 8c + j)
    (build, quant/int4.go:75-101)."""
    N, K = code.shape
    c = code.reshape(N, K // 8, 8).astype(np.uint32)
    return np.bitwise_or.reduce(c << (np.arange(8, dtype=np.uint32) * 4), axis=2).astype(np.uint32)


def int4_from_gptq(qweight, qzeros, scales, group, g_idx=None, v2=False):
    """quant.FromGPTQ (quant/int4.go:102-182) on numpy arrays: qweight (K/8, N) and qzeros
    (K/G, N/8) as int32 / uint32, scales (K/G, N) F32, g_idx (K,) or None.  Returns (codes
    (N, K/8) uint32, scales (N, K/G), zeros (N, K/G), perm (K,) int64 or None); raises
    ValueError with Light's messages."""
    qw = np.asarray(qweight).view(np.uint32)
    qz = np.asarray(qzeros).view(np.uint32)
    sc = np.asarray(scales, np.float32)
    K, N = qw.shape[0] * 8, qw.shape[1]
    if group <= 0:
        group = K
    if K % group or sc.shape != (K // group, N) or qz.shape[0] != K // group or qz.shape[1] * 8 != N:
        raise ValueError(f"quant.FromGPTQ: qweight {_gos(qw.shape)}, qzeros {_gos(qz.shape)}, scales "
                         f"{_gos(sc.shape)}, group {group} inconsistent")
    perm = None
    if g_idx is not None:
        gi = np.asarray(g_idx).astype(np.int64).ravel()
        if gi.size != K:
            raise ValueError(f"quant.FromGPTQ: g_idx has {gi.size} entries for K {K}")
        if not np.array_equal(gi, np.arange(K) // group):
            perm = np.argsort(gi, kind="stable").astype(np.int64)
            if not np.array_equal(gi[perm], np.arange(K) // group):
                raise ValueError(f"quant.FromGPTQ: g_idx groups are not all of size {group}")
    G = K // group
    n = np.arange(N)
    zeros = _nib(qz[:, n // 8], n % 8).astype(np.float32)  # (G, N)
    if not v2:
        zeros = zeros + np.float32(1)
    src = perm if perm is not None else np.arange(K)
    code = _nib(qw[src // 8][:, n], (src % 8)[:, None])  # (K, N): code of (n, k)
    return _canon(code.T.astype(np.uint8)), np.ascontiguousarray(sc.T), np.ascontiguousarray(zeros.T), perm


_AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def int4_from_awq(qweight, qzeros, scales, group):
    """quant.FromAWQ (quant/int4.go:184-235) on numpy arrays: qweight (K, N/8) and qzeros
    (K/G, N/8) int32 / uint32, scales (K/G, N) F32.  Returns (codes, scales, zeros)."""
    qw = np.asarray(qweight).view(np.uint32)
    qz = np.asarray(qzeros).view(np.uint32)
    sc = np.asarray(scales, np.float32)
    K, N = qw.shape[0], qw.shape[1] * 8
    if group <= 0 or K % group or sc.shape != (K // group, N) or qz.shape[0] != K // group or qz.shape[1] * 8 != N:
        raise ValueError(f"quant.FromAWQ: qweight {_gos(qw.shape)}, qzeros {_gos(qz.shape)}, scales "
                         f"{_gos(sc.shape)}, group {group} inconsistent")
    inv = np.zeros(8, np.int64)
    for i, o in enumerate(_AWQ_ORDER):
        inv[o] = i
    n = np.arange(N)
    zeros = _nib(qz[:, n // 8], inv[n % 8]).astype(np.float32)
    code = _nib(qw[:, n // 8], inv[n % 8])  # (K, N)
    return _canon(code.T.astype(np.uint8)), np.ascontiguousarray(sc.T), np.ascontiguousarray(zeros.T)
