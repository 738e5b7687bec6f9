"""Shared comparison helpers for the parity tests."""
import numpy as np


def norm_err(got, want, wnorm, xnorm):
    """max_{m,n} |got - want| / (||w_n|| * ||x_m||): the north-star normalisation."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = np.outer(xnorm, wnorm)
    scale = np.where(scale == 0, 1.0, scale)
    return float(np.max(np.abs(got - want) / scale)) if got.size else 0.0


def light_bound_ok(got, ref64, mag, tol=1e-5):
    """Light's CPU kernel bound: |got - ref| <= tol * (1 + sum |x w|) (ops/matmul_q_cpu_test.go:66-76)."""
    return bool(np.all(np.abs(np.asarray(got, np.float64) - ref64) <= tol * (1.0 + mag)))


def max_rel(got, want):
    """Light's maxRelErr (ops/matmul_q_test.go:61-73): max |a-b| / max |b|."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.max(np.abs(want)) if want.size else 0.0
    num = np.max(np.abs(got - want)) if want.size else 0.0
    return num / den if den else num


def random_blocks(rng, dt, N, K):
    """Light's randomQuantBlocks (ops/matmul_q_test.go:16-56): random bytes, f16 scale fields in [2^-6, 2^-5)."""
    be, bb = {13: (32, 18), 15: (32, 22), 17: (32, 34), 21: (256, 144), 22: (256, 176), 23: (256, 210)}[dt]
    nb = N * K // be
    buf = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)

    def small():
        v = (0x2400 | rng.integers(0, 0x400, size=nb)).astype("<u2")
        return v.view(np.uint8).reshape(nb, 2)

    if dt in (13, 15, 17):
        buf[:, 0:2] = small()
    elif dt in (21, 22):
        buf[:, 0:2] = small()
        buf[:, 2:4] = small()
    else:
        buf[:, 208:210] = small()
    return buf.reshape(-1)
