"""Writers of GPTQ / AWQ checkpoint tensors from a known 4-bit weight, following the producers'
published packing (test infrastructure).

* AutoGPTQ / GPTQModel ``pack``: ``qweight[r, n] |= q[8r + j, n] << 4j`` (K packed along rows),
  ``qzeros[g, c] |= (z[g, 8c + j] - 1) << 4j`` ("gptq"; "gptq_v2" stores z itself), scales
  (K/G, N); act order assigns input row k to group ``g_idx[k]``.
* AutoAWQ GEMM ``pack``: ``qweight[k, c] |= q[k, 8c + order[i]] << 4i`` with
  ``order = (0, 2, 4, 6, 1, 3, 5, 7)``, qzeros likewise, scales (K/G, N).

q here is indexed (input row k, output column n), as the checkpoints store the transposed weight.
"""
import numpy as np

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def pack_gptq(q_kn, z_gn, v2=False):
    K, N = q_kn.shape
    qw = np.zeros((K // 8, N), np.uint32)
    for j in range(8):
        qw |= q_kn[j::8].astype(np.uint32) << np.uint32(4 * j)
    zs = z_gn.astype(np.int64) - (0 if v2 else 1)
    G = z_gn.shape[0]
    qz = np.zeros((G, N // 8), np.uint32)
    for j in range(8):
        qz |= (zs[:, j::8] & 0xF).astype(np.uint32) << np.uint32(4 * j)
    return qw.view(np.int32), qz.view(np.int32)


def pack_awq(q_kn, z_gn):
    K, N = q_kn.shape
    qw = np.zeros((K, N // 8), np.uint32)
    G = z_gn.shape[0]
    qz = np.zeros((G, N // 8), np.uint32)
    for i, o in enumerate(AWQ_ORDER):
        qw |= q_kn[:, o::8].astype(np.uint32) << np.uint32(4 * i)
        qz |= z_gn[:, o::8].astype(np.uint32) << np.uint32(4 * i)
    return qw.view(np.int32), qz.view(np.int32)


def unpack_canonical(codes):
    """Canonical codes (N, K/8) words -> (N, K) nibbles: nibble j of word c is column 8c + j."""
    c = np.asarray(codes).view(np.uint32)
    N, W = c.shape
    return np.stack([(c >> np.uint32(4 * j)) & np.uint32(0xF) for j in range(8)], axis=2).reshape(N, 8 * W)


def random_checkpoint(g, K, N, G, act_order=False):
    """A random 4-bit weight: q (K, N), zeros (K/G, N) in [0, 15], scales (K/G, N) and, with act
    order, g_idx (K,) assigning each input row to a group (every group holds G rows)."""
    q = g.integers(0, 16, (K, N), dtype=np.uint8)
    z = g.integers(1, 16, (K // G, N), dtype=np.uint8)  # "gptq" stores z - 1 >= 0
    s = (np.abs(g.standard_normal((K // G, N))) * 0.01).astype(np.float32)
    gidx = None
    if act_order:
        gidx = np.empty(K, np.int32)
        gidx[g.permutation(K)] = np.arange(K) // G
    return q, z, s, gidx
