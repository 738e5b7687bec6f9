"""Non-finite activations: a NaN or Inf in row m of x makes every output of row m non-finite,
as Light's F32 arithmetic does (kernels/cpu/quant_matmul.go: the dequantized dot of that row),
and leaves every other row bit-identical to the call without it.  The int8 paths quantize x
per 32-block, where a max that ignores NaN would otherwise hide it behind finite codes."""
import pytest
import torch

from light_amd import hipq, synth

pytestmark = pytest.mark.gpu


def _rows_check(y_bad, y_ok):
    assert not torch.isfinite(y_bad[0]).any(), "row 0 holds a non-finite x but has finite outputs"
    assert torch.equal(y_bad[1:], y_ok[1:]), "other rows changed"


@pytest.mark.parametrize("dt,K", [(hipq.Q4_K, 2048), (hipq.Q4_K, 4096), (hipq.Q4_K, 14336), (hipq.Q5_K, 4096),
                                  (hipq.Q8_0, 4096), (hipq.Q8_0, 1024), (hipq.Q6_K, 4096), (hipq.Q4_0, 12288),
                                  (hipq.Q5_0, 2048)])
@pytest.mark.parametrize("M", [2, 3, 16])
@pytest.mark.parametrize("bad", [float("nan"), float("inf"), float("-inf")])
def test_matmul_q_nonfinite_row(dev, dt, K, M, bad):
    print(f"[case] nonfinite matmul_q dt={hipq.NAMES[dt]} K={K} M={M} x={bad}", flush=True)
    g = synth.rng(K + M + dt)
    N = 96
    w = torch.from_numpy(synth.gguf_weight(dt, N, K, g)).to(dev)
    x = torch.randn(M, K, device=dev)
    ok = hipq.matmul_q(x, w, N, K, dt)
    x[0, 37] = bad
    _rows_check(hipq.matmul_q(x, w, N, K, dt), ok)
    act = hipq.quantize_act(x)
    y = hipq.matmul_q_act(act, w, M, N, K, dt)
    assert not torch.isfinite(y[0]).any()
    assert torch.isfinite(y[1:]).all()


@pytest.mark.parametrize("M", [1, 2, 16])
def test_gated_and_mlp_nonfinite_row(dev, M):
    print(f"[case] nonfinite gated/mlp M={M}", flush=True)
    g = synth.rng(90 + M)
    H, I = 1024, 2816
    t = lambda a: torch.from_numpy(a).to(dev)
    wg, wu, wd = (t(synth.gguf_weight(hipq.Q4_K, r, c, g)) for r, c in ((I, H), (I, H), (H, I)))
    x = torch.randn(max(M, 2), H, device=dev)
    ok_g = hipq.matmul_q_gated(x, wg, wu, I, H, hipq.Q4_K)
    ok_m = hipq.mlp_q(x, wg, wu, wd, H, I, hipq.Q4_K)
    x[0, 5] = float("nan")
    _rows_check(hipq.matmul_q_gated(x, wg, wu, I, H, hipq.Q4_K), ok_g)
    _rows_check(hipq.mlp_q(x, wg, wu, wd, H, I, hipq.Q4_K), ok_m)


@pytest.mark.parametrize("M", [2, 16, 64])
@pytest.mark.parametrize("xdt", [torch.float32, torch.float16])
def test_int4_nonfinite_row(dev, M, xdt):
    print(f"[case] nonfinite int4 M={M} x={xdt}", flush=True)
    gen = torch.Generator(device="cpu").manual_seed(M)
    N, K, G = 200, 2048, 128
    codes = torch.randint(0, 2 ** 31, (N, K // 8), dtype=torch.int32, generator=gen).to(dev)
    s = (torch.rand(N, K // G, generator=gen) * 0.02 + 1e-3).to(dev)
    z = torch.randint(0, 16, (N, K // G), generator=gen).float().to(dev)
    x = torch.randn(M, K, generator=gen).to(dev)
    ok = hipq.int4_matmul(x.to(xdt), codes, s, z, G)
    x[0, 100] = float("nan")
    _rows_check(hipq.int4_matmul(x.to(xdt), codes, s, z, G), ok)
