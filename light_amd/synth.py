"""Seeded synthetic inputs for the five benchmark configurations.

Blocks are written directly from their fields (never produced by a quantizer),
so every dequantized value is known exactly.  The packers follow Light's block
layouts and its test builders (buildQ4_KBlock, quant/q4_k_test.go:20-46;
buildQ6_KBlock, quant/q6_k_test.go:20-59).  Distributions:

* Q8_0:  qs ~ U[-127, 127], d = f16(|N(0,1)| * 0.02 / 127).
* Q4_K:  6-bit sc, m ~ U[0, 63], q ~ U[0, 15], d and dmin = f16(|N(0,1)| * 1e-3)
         (the configs leave the Q4_K d / dmin distribution open; this is the
         stated choice, the same law as Q6_K's d).
* Q6_K:  raw ~ U[0, 63], int8 sc ~ U[-32, 31], d = f16(|N(0,1)| * 1e-3).
* Q4_0 / Q5_0 (not benchmark configs; parity cases): q ~ U over the format's
         range, d = f16(|N(0,1)| * 0.02 / 8) and f16(|N(0,1)| * 0.02 / 16).
* Q5_K:  as Q4_K with q5 ~ U[0, 31].
* int4:  codes u32 uniform, s = f16(|N(0,1)| * 0.01) widened to F32,
         z ~ U[0, 15] as F32, group 128.
* MoE:   expert ids uniform without replacement per token, routing weights
         softmax(N(0,1)) over the topk slots, pairs sorted by expert.
* Activations ~ N(0,1) (F32, or F16 for int4).
"""
import numpy as np

Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 13, 15, 17, 21, 22, 23


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def _f16_bits(v):
    return np.asarray(v, dtype=np.float32).astype(np.float16).view(np.uint16)


def pack_q8_0(d_bits, qs):
    """d_bits (nb,) uint16, qs (nb, 32) int8 -> (nb*34,) uint8."""
    nb = d_bits.shape[0]
    out = np.empty((nb, 34), np.uint8)
    out[:, 0:2] = d_bits.astype("<u2").view(np.uint8).reshape(nb, 2)
    out[:, 2:] = qs.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def pack_q4_k(d_bits, dmin_bits, sc, mn, q):
    """sc, mn (nb, 8) in [0, 63]; q (nb, 256) in [0, 15] -> (nb*144,) uint8."""
    nb = d_bits.shape[0]
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    out = np.empty((nb, 144), np.uint8)
    out[:, 0:2] = d_bits.astype("<u2").view(np.uint8).reshape(nb, 2)
    out[:, 2:4] = dmin_bits.astype("<u2").view(np.uint8).reshape(nb, 2)
    s12 = np.empty((nb, 12), np.uint8)
    s12[:, 0:4] = (sc[:, 0:4] & 0x3F) | ((sc[:, 4:8] & 0x30) << 2)
    s12[:, 4:8] = (mn[:, 0:4] & 0x3F) | ((mn[:, 4:8] & 0x30) << 2)
    s12[:, 8:12] = (sc[:, 4:8] & 0x0F) | ((mn[:, 4:8] & 0x0F) << 4)
    out[:, 4:16] = s12
    q = q.astype(np.uint8).reshape(nb, 4, 2, 32)  # (p, lo/hi, l)
    out[:, 16:] = (q[:, :, 0, :] | (q[:, :, 1, :] << 4)).reshape(nb, 128)
    return out.reshape(-1)


def pack_q4_0(d_bits, q):
    """q (nb, 32) in [0, 15] (stored nibbles; value = q - 8) -> (nb*18,) uint8 (quant/q4_0.go:18-27)."""
    nb = d_bits.shape[0]
    q = q.astype(np.uint8)
    out = np.empty((nb, 18), np.uint8)
    out[:, 0:2] = d_bits.astype("<u2").view(np.uint8).reshape(nb, 2)
    out[:, 2:] = (q[:, :16] & 0x0F) | ((q[:, 16:] & 0x0F) << 4)
    return out.reshape(-1)


def pack_q5_0(d_bits, q):
    """q (nb, 32) in [0, 31] (value = q - 16) -> (nb*22,) uint8 (quant/q5_0.go:11-20)."""
    nb = d_bits.shape[0]
    q = q.astype(np.uint32)
    out = np.empty((nb, 22), np.uint8)
    out[:, 0:2] = d_bits.astype("<u2").view(np.uint8).reshape(nb, 2)
    qh = (((q >> 4) & 1) << np.arange(32, dtype=np.uint32)[None, :]).sum(axis=1).astype("<u4")
    out[:, 2:6] = qh.view(np.uint8).reshape(nb, 4)
    out[:, 6:] = ((q[:, :16] & 0x0F) | ((q[:, 16:] & 0x0F) << 4)).astype(np.uint8)
    return out.reshape(-1)


def pack_q5_k(d_bits, dmin_bits, sc, mn, q):
    """q (nb, 256) in [0, 31] -> (nb*176,) uint8: Q4_K's header, qh[32], Q4_K's qs (quant/q5_k.go:11-22)."""
    nb = d_bits.shape[0]
    q = q.astype(np.uint8)
    q4 = pack_q4_k(d_bits, dmin_bits, sc, mn, q & 0x0F).reshape(nb, 144)
    hb = ((q >> 4) & 1).reshape(nb, 4, 2, 32)  # (p, lo/hi, l) -> bit 2p + lo/hi of qh[l]
    sh = (2 * np.arange(4)[:, None] + np.arange(2)[None, :]).astype(np.uint8)
    qh = (hb << sh[None, :, :, None]).sum(axis=(1, 2)).astype(np.uint8)
    out = np.empty((nb, 176), np.uint8)
    out[:, 0:16] = q4[:, 0:16]
    out[:, 16:48] = qh
    out[:, 48:] = q4[:, 16:]
    return out.reshape(-1)


def pack_q6_k(d_bits, sc, raw):
    """sc (nb, 16) int8; raw (nb, 256) in [0, 63] -> (nb*210,) uint8."""
    nb = d_bits.shape[0]
    raw = raw.astype(np.uint8).reshape(nb, 2, 4, 32)  # (half, group, l)
    out = np.empty((nb, 210), np.uint8)
    r1, r2, r3, r4 = raw[:, :, 0], raw[:, :, 1], raw[:, :, 2], raw[:, :, 3]
    ql = np.empty((nb, 2, 64), np.uint8)
    ql[:, :, :32] = (r1 & 0x0F) | ((r3 & 0x0F) << 4)
    ql[:, :, 32:] = (r2 & 0x0F) | ((r4 & 0x0F) << 4)
    qh = ((r1 >> 4) & 3) | (((r2 >> 4) & 3) << 2) | (((r3 >> 4) & 3) << 4) | (((r4 >> 4) & 3) << 6)
    out[:, 0:128] = ql.reshape(nb, 128)
    out[:, 128:192] = qh.reshape(nb, 64)
    out[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    out[:, 208:210] = d_bits.astype("<u2").view(np.uint8).reshape(nb, 2)
    return out.reshape(-1)


def gguf_weight(dt, N, K, g):
    """Random (N, K) weight in format dt with the config distributions; returns uint8 bytes."""
    if dt == Q8_0:
        nb = N * K // 32
        d = _f16_bits(np.abs(g.standard_normal(nb, dtype=np.float32)) * np.float32(0.02 / 127))
        qs = g.integers(-127, 128, size=(nb, 32), dtype=np.int8)
        return pack_q8_0(d, qs)
    if dt == Q4_K:
        nb = N * K // 256
        d = _f16_bits(np.abs(g.standard_normal(nb, dtype=np.float32)) * np.float32(1e-3))
        dmin = _f16_bits(np.abs(g.standard_normal(nb, dtype=np.float32)) * np.float32(1e-3))
        sc = g.integers(0, 64, size=(nb, 8), dtype=np.uint8)
        mn = g.integers(0, 64, size=(nb, 8), dtype=np.uint8)
        q = g.integers(0, 16, size=(nb, 256), dtype=np.uint8)
        return pack_q4_k(d, dmin, sc, mn, q)
    if dt == Q6_K:
        nb = N * K // 256
        d = _f16_bits(np.abs(g.standard_normal(nb, dtype=np.float32)) * np.float32(1e-3))
        sc = g.integers(-32, 32, size=(nb, 16), dtype=np.int8)
        raw = g.integers(0, 64, size=(nb, 256), dtype=np.uint8)
        return pack_q6_k(d, sc, raw)
    if dt in (Q4_0, Q5_0):
        nb = N * K // 32
        hi = 16 if dt == Q4_0 else 32
        d = _f16_bits(np.abs(g.standard_normal(nb, dtype=np.float32)) * np.float32(0.02 / (hi // 2)))
        q = g.integers(0, hi, size=(nb, 32), dtype=np.uint8)
        return pack_q4_0(d, q) if dt == Q4_0 else pack_q5_0(d, q)
    if dt == Q5_K:
        nb = N * K // 256
        d = _f16_bits(np.abs(g.standard_normal(nb, dtype=np.float32)) * np.float32(1e-3))
        dmin = _f16_bits(np.abs(g.standard_normal(nb, dtype=np.float32)) * np.float32(1e-3))
        sc = g.integers(0, 64, size=(nb, 8), dtype=np.uint8)
        mn = g.integers(0, 64, size=(nb, 8), dtype=np.uint8)
        q = g.integers(0, 32, size=(nb, 256), dtype=np.uint8)
        return pack_q5_k(d, dmin, sc, mn, q)
    raise ValueError(f"dtype {dt}")


def activations(M, K, g, dtype=np.float32):
    return g.standard_normal((M, K), dtype=np.float32).astype(dtype)


def int4_weight(N, K, G, g):
    """Canonical quant.Int4 tensors: codes u32 (N, K/8), scales / zeros f32 (N, K/G)."""
    codes = g.integers(0, 2 ** 32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = (np.abs(g.standard_normal((N, K // G), dtype=np.float32)) * np.float32(0.01)).astype(np.float16)
    s = s.astype(np.float32)
    z = g.integers(0, 16, size=(N, K // G)).astype(np.float32)
    return codes, s, z


def moe_routing(T, E, topk, g):
    """ids (T*topk,) int64 uniform without replacement per token, weights (T*topk,) f32 softmax(N(0,1))."""
    ids = np.empty((T, topk), np.int64)
    for t in range(T):
        ids[t] = g.choice(E, size=topk, replace=False)
    logits = g.standard_normal((T, topk)).astype(np.float32)
    e = np.exp(logits - logits.max(axis=1, keepdims=True))
    w = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids.reshape(-1), w.reshape(-1)


def sort_pairs(ids):
    """Stable expert sort of the flat ids (MoERouteFromIDs): (sorted_expts, sorted_pairs)."""
    order = np.argsort(ids, kind="stable")
    return ids[order].astype(np.int64), order.astype(np.int64)


# Named single-GPU workloads of the five configs (seed = config index).
CONFIGS = {
    "q8_0_gemv_4096x4096": dict(cfg=0, kind="gguf", dt=Q8_0, M=1, N=4096, K=4096),
    "q4_k_gemv_gate_14336x4096": dict(cfg=1, kind="gguf", dt=Q4_K, M=1, N=14336, K=4096),
    "q4_k_gemv_down_4096x14336": dict(cfg=1, kind="gguf", dt=Q4_K, M=1, N=4096, K=14336),
    "q6_k_gemv_attn_out_4096x4096": dict(cfg=1, kind="gguf", dt=Q6_K, M=1, N=4096, K=4096),
    "q6_k_gemv_lm_head_128256x4096": dict(cfg=1, kind="gguf", dt=Q6_K, M=1, N=128256, K=4096),
    # The same Q6_K weights after the load-time planar repack (Q6_K_R), as a model would run them.
    "q6_k_r_gemv_attn_out_4096x4096": dict(cfg=1, kind="gguf", dt=Q6_K, M=1, N=4096, K=4096, repack=True),
    "q6_k_r_gemv_lm_head_128256x4096": dict(cfg=1, kind="gguf", dt=Q6_K, M=1, N=128256, K=4096, repack=True),
    "q4_k_gemm_m512_14336x4096": dict(cfg=2, kind="gguf", dt=Q4_K, M=512, N=14336, K=4096),
    "q4_k_gemm_m512_4096x14336": dict(cfg=2, kind="gguf", dt=Q4_K, M=512, N=4096, K=14336),
    "int4_m1_18944x3584": dict(cfg=3, kind="int4", M=1, N=18944, K=3584, G=128),
    "int4_m1_3584x18944": dict(cfg=3, kind="int4", M=1, N=3584, K=18944, G=128),
    "int4_m64_18944x3584": dict(cfg=3, kind="int4", M=64, N=18944, K=3584, G=128),
    "int4_m64_3584x18944": dict(cfg=3, kind="int4", M=64, N=3584, K=18944, G=128),
    "moe_q4_k_t1": dict(cfg=4, kind="moe", dt=Q4_K, T=1, E=128, topk=8, H=2048, I=768),
    "moe_q4_k_t256": dict(cfg=4, kind="moe", dt=Q4_K, T=256, E=128, topk=8, H=2048, I=768),
}

# Not benchmark configurations: the remaining fused formats at the Llama-3-8B gate shape
# (decode) and Q8_0 / Q6_K / Q5_K prefill, timed by bench.py --table only.
EXTRA_CONFIGS = {
    "q4_0_gemv_14336x4096": dict(cfg=5, kind="gguf", dt=Q4_0, M=1, N=14336, K=4096),
    "q5_0_gemv_14336x4096": dict(cfg=5, kind="gguf", dt=Q5_0, M=1, N=14336, K=4096),
    "q5_k_gemv_14336x4096": dict(cfg=5, kind="gguf", dt=Q5_K, M=1, N=14336, K=4096),
    "q8_0_gemm_m512_14336x4096": dict(cfg=5, kind="gguf", dt=Q8_0, M=512, N=14336, K=4096),
    "q6_k_gemm_m512_14336x4096": dict(cfg=5, kind="gguf", dt=Q6_K, M=512, N=14336, K=4096),
    "q5_k_gemm_m512_14336x4096": dict(cfg=5, kind="gguf", dt=Q5_K, M=512, N=14336, K=4096),
}
