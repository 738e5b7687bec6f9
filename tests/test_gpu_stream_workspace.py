"""A stream's library workspace goes with the stream: hq_stream_destroy frees the buffers
that calls with ws == NULL grew on it, and the MoE block's one-launch kernel passes to the
next stream that runs it (its barrier words belong to one stream at a time)."""
import ctypes

import pytest
import torch

from light_amd import hipq, synth

pytestmark = pytest.mark.gpu


class _Stream:
    """A HIP stream made by the library (hq_stream_create), usable where _stream() is."""

    def __init__(self):
        p = ctypes.c_void_p()
        hipq.check(hipq.lib().hq_stream_create(ctypes.byref(p)))
        self.cuda_stream = p.value

    def destroy(self):
        hipq.check(hipq.lib().hq_stream_destroy(ctypes.c_void_p(self.cuda_stream)))


def test_stream_destroy_frees_its_workspace(dev):
    print("[case] stream destroy frees workspace", flush=True)
    M, N, K, dt = 512, 4096, 14336, hipq.Q4_K  # the M = 512 GEMM: bf16 x and split-K slices
    g = synth.rng(61)
    w = torch.from_numpy(synth.gguf_weight(dt, N, K, g)).to(dev)
    x = torch.from_numpy(synth.activations(M, K, g)).to(dev)
    want = hipq.matmul_q(x, w, N, K, dt)
    need = hipq.matmul_q_ws_bytes(M, N, K, dt)
    assert need > (32 << 20)
    torch.cuda.synchronize()
    for rep in range(3):
        s = _Stream()
        got = hipq.matmul_q(x, w, N, K, dt, stream=s)
        hipq.check(hipq.lib().hq_stream_synchronize(ctypes.c_void_p(s.cuda_stream)))
        assert torch.equal(got, want), rep
        free_before = torch.cuda.mem_get_info()[0]
        s.destroy()
        free_after = torch.cuda.mem_get_info()[0]
        assert free_after - free_before >= need - (4 << 20), (rep, free_before, free_after, need)


def test_moe_block_owner_moves_to_next_stream(dev):
    """The stream that ran the one-launch block is destroyed; the next stream to call it runs it
    (same bits as the two launches either way)."""
    print("[case] moe block owner after stream destroy", flush=True)
    dt, E, topk, H, I = hipq.Q4_K, 128, 8, 2048, 768
    g = synth.rng(62)
    wgu = torch.from_numpy(synth.gguf_weight(dt, E * 2 * I, H, g)).to(dev)
    wdn = torch.from_numpy(synth.gguf_weight(dt, E * H, I, g)).to(dev)
    x = torch.from_numpy(synth.activations(1, H, g)).to(dev)
    probs = torch.softmax(torch.from_numpy(g.standard_normal((1, E)).astype("float32")), dim=1).to(dev)
    ids, w, sp, se, h = hipq.moe_route_gated(probs, x, wgu, E, I, H, dt, topk)
    want = hipq.moe_gemm_q_combine(h, wdn, sp, se, E, H, I, dt, topk, topk_w=w)
    torch.cuda.synchronize()
    hipq.debug_moe_block_spin_limit()  # (also hands the kernel to the next stream that calls it)
    for rep in range(2):
        s = _Stream()
        y = hipq.moe_block_q(probs, x, wgu, wdn, E, H, I, dt, topk, stream=s)[0]
        hipq.moe_block_q_check(stream=s)
        assert torch.equal(y, want), rep
        s.destroy()
