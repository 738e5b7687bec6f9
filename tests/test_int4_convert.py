"""quant.FromGPTQ / quant.FromAWQ (quant/int4.go:102-235): the oracle's restatement against the
producers' published packing (tests/_ckpt.py), and the host layer's argument checks.

Light's own tests of these converters read real checkpoints (quant/int4_test.go:80-114), which
are not available offline: parity to Light is unpinned.  What pins the restatement here:
round trips through independently written AutoGPTQ / AutoAWQ packers (v1 and v2 zero points,
act order), single-nibble known answers for both layouts, and the Int4 contract -- the
canonical weight's column k is the checkpoint's input row Perm[k].
"""
import numpy as np
import pytest

import oracle
from _ckpt import AWQ_ORDER, pack_awq, pack_gptq, random_checkpoint, unpack_canonical
from light_amd import _light as L


@pytest.mark.parametrize("v2", [False, True])
@pytest.mark.parametrize("K,N,G", [(256, 64, 128), (512, 40, 64), (128, 8, 128)])
def test_gptq_round_trip(K, N, G, v2):
    g = np.random.default_rng(K + N + G + v2)
    q, z, s, _ = random_checkpoint(g, K, N, G)
    qw, qz = pack_gptq(q, z, v2)
    codes, so, zo, perm = oracle.int4_from_gptq(qw, qz, s, G, v2=v2)
    assert perm is None and codes.shape == (N, K // 8) and codes.dtype == np.uint32
    assert np.array_equal(unpack_canonical(codes), q.T)
    assert np.array_equal(zo, z.T.astype(np.float32)) and np.array_equal(so, s.T)


def test_gptq_act_order():
    """Canonical column k is input row perm[k]; perm sorts K stably by group; every group's rows
    keep that group's scale and zero."""
    K, N, G = 512, 32, 128
    g = np.random.default_rng(7)
    q, z, s, gidx = random_checkpoint(g, K, N, G, act_order=True)
    qw, qz = pack_gptq(q, z)
    codes, so, zo, perm = oracle.int4_from_gptq(qw, qz, s, G, g_idx=gidx)
    assert perm is not None and np.array_equal(np.sort(perm), np.arange(K))
    assert np.all(np.diff(gidx[perm]) >= 0) and np.array_equal(gidx[perm], np.arange(K) // G)
    # stable: rows of one group stay in input order
    for grp in range(K // G):
        rows = perm[grp * G:(grp + 1) * G]
        assert np.all(np.diff(rows) > 0)
    assert np.array_equal(unpack_canonical(codes), q[perm].T)
    # W[n, k] = s[n, k / G] (code - z[n, k / G]) == the checkpoint's row perm[k] in its group
    w_canon = so[:, np.arange(K) // G] * (unpack_canonical(codes).astype(np.float32) - zo[:, np.arange(K) // G])
    w_ckpt = s[gidx[perm]].T * (q[perm].T.astype(np.float32) - z[gidx[perm]].T.astype(np.float32))
    assert np.array_equal(w_canon, w_ckpt)


def test_gptq_ordered_g_idx_gives_no_perm():
    K, N, G = 256, 16, 64
    g = np.random.default_rng(3)
    q, z, s, _ = random_checkpoint(g, K, N, G)
    qw, qz = pack_gptq(q, z)
    a = oracle.int4_from_gptq(qw, qz, s, G, g_idx=(np.arange(K) // G).astype(np.int32))
    b = oracle.int4_from_gptq(qw, qz, s, G)
    assert a[3] is None and all(np.array_equal(x, y) for x, y in zip(a[:3], b[:3]))


def test_gptq_single_nibble():
    """qweight[1, 3] = 5 << 8 (nibble 2) is input row 8 * 1 + 2 = 10 of column 3: canonical
    codes[3, 1] = 5 << 8; qzeros[0, 0] = 6 << 4 (nibble 1) is column 1's zero - 1 = 6."""
    K, N, G = 64, 8, 64
    qw = np.zeros((K // 8, N), np.int32)
    qw[1, 3] = 5 << 8
    qz = np.zeros((1, 1), np.int32)
    qz[0, 0] = 6 << 4
    codes, so, zo, _ = oracle.int4_from_gptq(qw, qz, np.ones((1, N), np.float32), G)
    want = np.zeros((N, K // 8), np.uint32)
    want[3, 1] = 5 << 8
    assert np.array_equal(codes, want)
    assert zo[1, 0] == 7 and zo[0, 0] == 1 and np.all(np.delete(zo[:, 0], 1) == 1)


@pytest.mark.parametrize("K,N,G", [(256, 64, 128), (128, 16, 32)])
def test_awq_round_trip(K, N, G):
    g = np.random.default_rng(K * N + G)
    q, z, s, _ = random_checkpoint(g, K, N, G)
    qw, qz = pack_awq(q, z)
    codes, so, zo = oracle.int4_from_awq(qw, qz, s, G)
    assert np.array_equal(unpack_canonical(codes), q.T)
    assert np.array_equal(zo, z.T.astype(np.float32)) and np.array_equal(so, s.T)


def test_awq_single_nibble():
    """qweight[5, 0] = 7 << 4 (nibble 1) holds column 8 * 0 + order[1] = 2 of input row 5."""
    assert AWQ_ORDER[1] == 2
    K, N, G = 64, 8, 64
    qw = np.zeros((K, N // 8), np.int32)
    qw[5, 0] = 7 << 4
    codes, _, _ = oracle.int4_from_awq(qw, np.zeros((1, 1), np.int32), np.ones((1, N), np.float32), G)
    want = np.zeros((N, K // 8), np.uint32)
    want[2, 0] = 7 << (4 * 5)
    assert np.array_equal(codes, want)


def test_oracle_messages():
    with pytest.raises(ValueError, match=r"quant.FromGPTQ: qweight \[8 16\], qzeros \[1 2\], scales \[2 16\], "
                                         r"group 64 inconsistent"):
        oracle.int4_from_gptq(np.zeros((8, 16), np.int32), np.zeros((1, 2), np.int32), np.zeros((2, 16), np.float32), 64)
    with pytest.raises(ValueError, match="g_idx groups are not all of size 32"):
        gi = np.zeros(64, np.int32)  # every row in group 0
        oracle.int4_from_gptq(np.zeros((8, 8), np.int32), np.zeros((2, 1), np.int32), np.zeros((2, 8), np.float32),
                              32, g_idx=gi)


# ---- host layer: Light's checks and messages, before any device work (CPU tensors) ----

def t(a, dt):
    a = np.ascontiguousarray(a)
    return L.from_numpy(a, dt, list(a.shape))


def test_host_from_gptq_validation():
    qw, qz, s = np.zeros((8, 16), np.int32), np.zeros((1, 2), np.int32), np.zeros((1, 16), np.float32)
    with pytest.raises(L.Error, match=r"quant.FromGPTQ: rank-2 qweight / qzeros / scales expected"):
        L.from_gptq(t(np.zeros(8, np.int32), "I32"), t(qz, "I32"), t(s, "F32"), None, 64)
    with pytest.raises(L.Error, match=r"quant.FromGPTQ: qweight \[8 16\], qzeros \[1 2\], scales \[1 16\], "
                                      r"group 32 inconsistent"):
        L.from_gptq(t(qw, "I32"), t(qz, "I32"), t(s, "F32"), None, 32)
    with pytest.raises(L.Error, match="quant.FromGPTQ: g_idx has 10 entries for K 64"):
        L.from_gptq(t(qw, "I32"), t(qz, "I32"), t(s, "F32"), t(np.zeros(10, np.int32), "I32"), 64)
    with pytest.raises(L.Error, match="quant.FromGPTQ: g_idx groups are not all of size 32"):
        L.from_gptq(t(qw, "I32"), t(np.zeros((2, 2), np.int32), "I32"), t(np.zeros((2, 16), np.float32), "F32"),
                    t(np.zeros(64, np.int32), "I32"), 32)
    with pytest.raises(L.Error, match="quant: qweight is F32, want I32 / U32"):
        L.from_gptq(t(qw.astype(np.float32), "F32"), t(qz, "I32"), t(s, "F32"), None, 64)
    with pytest.raises(L.Error, match=r"quant: scales / zeros must be F32 \(cast the checkpoint's F16 first\), got F16"):
        L.from_gptq(t(qw, "I32"), t(qz, "I32"), t(s.astype(np.float16), "F16"), None, 64)


def test_host_from_awq_validation():
    with pytest.raises(L.Error, match=r"quant.FromAWQ: qweight \[64 2\], qzeros \[1 2\], scales \[1 16\], "
                                      r"group 0 inconsistent"):
        L.from_awq(t(np.zeros((64, 2), np.int32), "I32"), t(np.zeros((1, 2), np.int32), "I32"),
                   t(np.zeros((1, 16), np.float32), "F32"), 0)
    with pytest.raises(L.Error, match="quant: qzeros is U8, want I32 / U32"):
        L.from_awq(t(np.zeros((64, 2), np.int32), "I32"), t(np.zeros((1, 2), np.uint8), "U8"),
                   t(np.zeros((1, 16), np.float32), "F32"), 64)
