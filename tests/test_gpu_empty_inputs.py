"""Empty inputs through the C ABI on the GPU: zero rows, zero output columns, zero tokens.

Light's ops return empty results for empty operands (an M = 0 MatMulQ is an (0, N) tensor);
every entry point here must return HQ_OK with correctly shaped empty outputs and launch
nothing that reads past them.
"""
import pytest
import torch

from light_amd import hipq, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def q4k(dev):
    g = synth.rng(1)
    t = lambda a: torch.from_numpy(a).to(dev)
    return dict(w=t(synth.gguf_weight(hipq.Q4_K, 512, 256, g)), wd=t(synth.gguf_weight(hipq.Q4_K, 256, 512, g)),
                we=t(synth.gguf_weight(hipq.Q4_K, 4 * 64, 256, g)))


def test_matmul_q_empty(dev, q4k):
    w = q4k["w"]
    assert tuple(hipq.matmul_q(torch.empty((0, 256), device=dev), w, 512, 256, hipq.Q4_K).shape) == (0, 512)
    assert tuple(hipq.matmul_q(torch.randn(3, 256, device=dev), w[:0], 0, 256, hipq.Q4_K).shape) == (3, 0)
    x0 = torch.empty((0, 256), device=dev)
    assert tuple(hipq.matmul_q_gated(x0, w, w, 512, 256, hipq.Q4_K).shape) == (0, 512)
    assert hipq.matmul_q_gated_act(x0, w, w, 512, 256, hipq.Q4_K).numel() == 0
    assert hipq.quantize_act(x0).numel() == 0
    assert hipq.dequant(w, 0, hipq.Q4_K).numel() == 0
    assert tuple(hipq.mlp_q(x0, w, w, q4k["wd"], 256, 512, hipq.Q4_K).shape) == (0, 256)
    torch.cuda.synchronize()


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
def test_int4_empty(dev, xdt):
    codes = torch.zeros((64, 32), dtype=torch.int32, device=dev)
    s, z = torch.ones((64, 2), device=dev), torch.zeros((64, 2), device=dev)
    assert tuple(hipq.int4_matmul(torch.empty((0, 256), device=dev, dtype=xdt), codes, s, z, 128).shape) == (0, 64)
    assert tuple(hipq.int4_matmul(torch.randn(3, 256, device=dev).to(xdt), codes[:0], s[:0], z[:0], 128).shape) == (3, 0)
    assert tuple(hipq.int4_dequant(codes[:0], s[:0], z[:0], 128).shape) == (0, 256)
    torch.cuda.synchronize()


def test_moe_empty(dev, q4k):
    ids, w, sp, se = hipq.moe_route(torch.empty((0, 8), device=dev), 2)
    assert tuple(ids.shape) == (0, 2) and w.numel() == sp.numel() == se.numel() == 0
    e64 = torch.empty(0, dtype=torch.int64, device=dev)
    y = hipq.moe_gemm_q(torch.empty((0, 256), device=dev), q4k["we"], e64, e64, 4, 64, 256, hipq.Q4_K, 2)
    assert tuple(y.shape) == (0, 64)
    torch.cuda.synchronize()
