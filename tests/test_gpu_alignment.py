"""Misaligned operands through the C ABI: a base pointer of x or of a GGUF weight that is not
16-byte aligned is refused with HQ_EINVAL (never read through a path that assumes alignment);
int4 codes at any 4-byte offset take a path that reads them as they lie, within the bar."""
import numpy as np
import pytest
import torch

from light_amd import hipq, synth

pytestmark = pytest.mark.gpu


def _off(t, elems):
    """A copy of t whose storage starts `elems` elements past an aligned allocation."""
    buf = torch.empty(t.numel() + elems, dtype=t.dtype, device=t.device)
    v = buf[elems:].view(t.shape)
    v.copy_(t)
    return v


@pytest.mark.parametrize("dt,K", [(hipq.Q4_K, 4096), (hipq.Q8_0, 4096), (hipq.Q6_K, 2048), (hipq.Q4_0, 14336)])
@pytest.mark.parametrize("M", [1, 16])
def test_misaligned_x_or_w_is_einval(dev, dt, K, M):
    print(f"[case] misaligned dt={hipq.NAMES[dt]} K={K} M={M}", flush=True)
    g = synth.rng(K + M + dt)
    N = 96
    w = torch.from_numpy(synth.gguf_weight(dt, N, K, g)).to(dev)
    x = torch.randn(M, K, device=dev)
    for xx, ww in ((_off(x, 1), w), (x, _off(w, 1)), (x, _off(w, 4))):
        with pytest.raises(hipq.HipqError) as ei:
            hipq.matmul_q(xx, ww, N, K, dt)
        assert ei.value.code == hipq.HQ_EINVAL
        with pytest.raises(hipq.HipqError) as ei:
            hipq.matmul_q_gated(xx, ww, ww, N, K, dt)
        assert ei.value.code == hipq.HQ_EINVAL
    torch.cuda.synchronize()


@pytest.mark.parametrize("M", [1, 3, 16, 64])
@pytest.mark.parametrize("xdt", [torch.float32, torch.float16])
def test_int4_misaligned(dev, M, xdt):
    print(f"[case] int4 misaligned M={M} x={xdt}", flush=True)
    N, K, G = 300, 2048, 128
    gen = torch.Generator(device="cpu").manual_seed(M)
    codes = torch.randint(0, 2 ** 31, (N, K // 8), dtype=torch.int32, generator=gen).to(dev)
    s = (torch.rand(N, K // G, generator=gen) * 0.02 + 1e-3).to(dev)
    z = torch.randint(0, 16, (N, K // G), generator=gen).float().to(dev)
    x = torch.randn(M, K, generator=gen).to(xdt).to(dev)
    with pytest.raises(hipq.HipqError) as ei:
        hipq.int4_matmul(_off(x, 1), codes, s, z, G)
    assert ei.value.code == hipq.HQ_EINVAL
    got = hipq.int4_matmul(x, _off(codes, 1), s, z, G).double()
    wd = hipq.int4_dequant(codes, s, z, G).double()  # bit-exact with the oracle
    xd = x.double()
    ref = xd @ wd.T
    norm = torch.outer(xd.norm(dim=1), wd.norm(dim=1)).clamp_min(1e-30)
    assert float(((got - ref).abs() / norm).max()) <= 1e-3
