"""GPU: the device conversion of GPTQ / AWQ checkpoint tensors to canonical quant.Int4
(hq_int4_from_gptq / hq_int4_from_awq, and the host layer's quant.FromGPTQ / FromAWQ on top)
against the oracle's restatement of quant.FromGPTQ / quant.FromAWQ, bit for bit; then the
converted weight through ops.MatMulInt4 (act order included) against the dequantized
checkpoint at the 1e-3 bar.  Shapes: configs[3]'s Qwen2.5-7B MLP (K = 3584, N = 18944, G = 128)
and small ragged ones."""
import numpy as np
import pytest
import torch

import oracle
from _ckpt import pack_awq, pack_gptq, random_checkpoint, unpack_canonical
from _util import norm_err
from light_amd import _light as L
from light_amd import hipq

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("act_order", [False, True])
@pytest.mark.parametrize("v2", [False, True])
@pytest.mark.parametrize("K,N,G", [(3584, 18944, 128), (256, 40, 64), (128, 8, 128)])
def test_from_gptq_bit_exact(dev, K, N, G, v2, act_order):
    print(f"[case] from_gptq K={K} N={N} G={G} v2={v2} act_order={act_order}", flush=True)
    g = np.random.default_rng(K + N + G + 2 * v2 + act_order)
    q, z, s, gidx = random_checkpoint(g, K, N, G, act_order)
    qw, qz = pack_gptq(q, z, v2)
    want = oracle.int4_from_gptq(qw, qz, s, G, g_idx=gidx, v2=v2)
    perm = None if want[3] is None else _t(want[3], dev)
    codes, so, zo = hipq.int4_from_gptq(_t(qw, dev), _t(qz, dev), _t(s, dev), G, perm=perm, v2=v2)
    torch.cuda.synchronize()
    assert np.array_equal(codes.cpu().numpy().view(np.uint32), want[0])
    assert np.array_equal(so.cpu().numpy(), want[1]) and np.array_equal(zo.cpu().numpy(), want[2])


@pytest.mark.parametrize("K,N,G", [(3584, 18944, 128), (18944, 3584, 128), (128, 16, 32)])
def test_from_awq_bit_exact(dev, K, N, G):
    print(f"[case] from_awq K={K} N={N} G={G}", flush=True)
    g = np.random.default_rng(K * 3 + N + G)
    q, z, s, _ = random_checkpoint(g, K, N, G)
    qw, qz = pack_awq(q, z)
    want = oracle.int4_from_awq(qw, qz, s, G)
    codes, so, zo = hipq.int4_from_awq(_t(qw, dev), _t(qz, dev), _t(s, dev), G)
    torch.cuda.synchronize()
    assert np.array_equal(codes.cpu().numpy().view(np.uint32), want[0])
    assert np.array_equal(so.cpu().numpy(), want[1]) and np.array_equal(zo.cpu().numpy(), want[2])


@pytest.mark.parametrize("fmt", ["gptq", "gptq_act_order", "awq"])
def test_host_convert_then_matmul(fmt):
    """quant.FromGPTQ / FromAWQ on CPU tensors (converted on ROCm(0)), then ops.MatMulInt4:
    y = x . W^T with W the checkpoint's own dequantized weight (input rows in Perm order)."""
    print(f"[case] host convert {fmt}", flush=True)
    K, N, G, M = 1024, 96, 128, 3
    g = np.random.default_rng(len(fmt))
    q, z, s, gidx = random_checkpoint(g, K, N, G, act_order=fmt == "gptq_act_order")
    cpu = lambda a, dt: L.from_numpy(np.ascontiguousarray(a), dt, list(np.shape(a)))
    if fmt == "awq":
        qw, qz = pack_awq(q, z)
        codes, sc, zr, group, perm = L.from_awq(cpu(qw, "I32"), cpu(qz, "I32"), cpu(s, "F32"), G)
    else:
        qw, qz = pack_gptq(q, z)
        codes, sc, zr, group, perm = L.from_gptq(cpu(qw, "I32"), cpu(qz, "I32"), cpu(s, "F32"),
                                                 None if gidx is None else cpu(gidx, "I32"), G)
    assert codes.device == "ROCm(0)" and codes.shape == [N, K // 8] and group == G
    assert (perm is None) == (gidx is None)
    # The checkpoint's weight over ITS input rows: W[n, k] = s[g(k), n] (q[k, n] - z[g(k), n]).
    grp = (np.arange(K) // G) if gidx is None else gidx
    w_ckpt = (s[grp] * (q.astype(np.float32) - z[grp].astype(np.float32))).T  # (N, K)
    x = np.random.default_rng(5).standard_normal((M, K)).astype(np.float32)
    y = L.matmul_int4(L.from_numpy(x, "F32", [M, K], "ROCm(0)"), codes, sc, zr, G, perm).numpy()
    want = x.astype(np.float64) @ w_ckpt.T.astype(np.float64)
    assert norm_err(y, want, np.linalg.norm(w_ckpt, axis=1), np.linalg.norm(x, axis=1)) <= 1e-3
    if perm is not None:
        assert np.array_equal(unpack_canonical(codes.numpy()), q[perm.numpy()].T)
