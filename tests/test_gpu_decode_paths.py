"""The one-token decode kernels against the many-row kernels they sit beside, bit for bit.

At M = 1 the library takes kernels laid out for one token (one workgroup per CU:
gate_cu_kernel for the MLP's gated gate/up with the quantized-h epilogue, gemv_rows_kernel
for rows longer than a wave on prepared activations, gemv_cu_kernel for 8-16 rows per CU);
at M = 2 it takes the persistent gemv_q4kx_kernel.  Each output row is computed by the same
instruction sequence in both (the same activation quantization per row, unit dots, team sums
in the same order), so row 0 of an M = 2 call equals the M = 1 call on that row, bit for bit.
The shapes cover the benchmark's (14336 / 4096 rows: two chunks per CU; K = 14336: eight rows
per team) and smaller ones (one chunk per CU, one to four rows per team).
"""
import numpy as np
import pytest
import torch

from light_amd import hipq, synth

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("dt,H,I", [(hipq.Q4_K, 4096, 14336), (hipq.Q4_K, 4096, 4096), (hipq.Q5_K, 4096, 8192),
                                    (hipq.Q4_K, 3072, 8192), (hipq.Q4_K, 4096, 2048),
                                    # more 32-row chunks than CUs, at most two per CU (gate_cu_kernel<2>)
                                    (hipq.Q5_K, 4096, 12288), (hipq.Q4_K, 3840, 14336), (hipq.Q4_K, 3072, 16384),
                                    (hipq.Q4_K, 2048, 10240)])
def test_mlp_one_token_kernels_equal_persistent(dev, dt, H, I):
    """gated gate/up (quantized h) then the down projection: M = 1 against row 0 of M = 2."""
    print(f"[case] decode paths mlp dt={hipq.NAMES[dt]} H={H} I={I}", flush=True)
    g = synth.rng(7100 + H + I + dt)
    wg, wu, wd = (_t(synth.gguf_weight(dt, r, c, g), dev) for r, c in ((I, H), (I, H), (H, I)))
    x2 = _t(synth.activations(2, H, g), dev)
    x1 = x2[:1].contiguous()
    a1 = hipq.matmul_q_gated_act(x1, wg, wu, I, H, dt)
    a2 = hipq.matmul_q_gated_act(x2, wg, wu, I, H, dt)
    y1 = hipq.matmul_q_act(a1, wd, 1, H, I, dt)
    y2 = hipq.matmul_q_act(a2, wd, 2, H, I, dt)
    m1 = hipq.mlp_q(x1, wg, wu, wd, H, I, dt)
    torch.cuda.synchronize()
    assert torch.equal(y1[0], y2[0])
    assert torch.equal(m1[0], y2[0])
    # Graph replays of the call reproduce it.
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    out = torch.empty_like(m1)
    ws = torch.empty(hipq.mlp_q_ws_bytes(1, H, I, dt), dtype=torch.uint8, device=dev)
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            hipq.mlp_q(x1, wg, wu, wd, H, I, dt, out=out, ws=ws)
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[0], y2[0])


@pytest.mark.parametrize("dt,N,K", [(hipq.Q4_K, 4096, 14336), (hipq.Q4_K, 1024, 14336), (hipq.Q5_K, 4096, 8192),
                                    (hipq.Q4_K, 300, 28672)])
def test_rows_kernel_equals_persistent(dev, dt, N, K):
    """hq_matmul_q_act on prepared activations, K > 4096: M = 1 against row 0 of M = 2."""
    print(f"[case] decode paths rows dt={hipq.NAMES[dt]} N={N} K={K}", flush=True)
    g = synth.rng(7200 + N + dt)
    w = _t(synth.gguf_weight(dt, N, K, g), dev)
    x2 = _t(synth.activations(2, K, g), dev)
    a1 = hipq.quantize_act(x2[:1].contiguous())
    a2 = hipq.quantize_act(x2)
    y1 = hipq.matmul_q_act(a1, w, 1, N, K, dt)
    y2 = hipq.matmul_q_act(a2, w, 2, N, K, dt)
    torch.cuda.synchronize()
    assert torch.equal(y1[0], y2[0])


@pytest.mark.parametrize("dt,N,K", [(hipq.Q6_K_R, 4096, 4096), (hipq.Q4_K, 2048, 4096), (hipq.Q5_K, 3072, 3072)])
def test_cu_kernel_equals_persistent(dev, dt, N, K):
    """hq_matmul_q (x quantized in the kernel) at 8-16 rows per CU: M = 1 against row 0 of M = 2,
    and the gated projection with F32 output the same way."""
    print(f"[case] decode paths cu dt={hipq.NAMES[dt]} N={N} K={K}", flush=True)
    g = synth.rng(7300 + N + dt)
    src = hipq.Q6_K if dt == hipq.Q6_K_R else dt
    raw = [_t(synth.gguf_weight(src, N, K, g), dev) for _ in range(2)]
    w = [hipq.repack_q6k(r, N, K) for r in raw] if dt == hipq.Q6_K_R else raw
    x2 = _t(synth.activations(2, K, g), dev)
    x1 = x2[:1].contiguous()
    y1 = hipq.matmul_q(x1, w[0], N, K, dt)
    y2 = hipq.matmul_q(x2, w[0], N, K, dt)
    torch.cuda.synchronize()
    assert torch.equal(y1[0], y2[0])
    if dt != hipq.Q6_K_R:  # (the gated projection takes GGUF formats only)
        h1 = hipq.matmul_q_gated(x1, w[0], w[1], N, K, dt)
        h2 = hipq.matmul_q_gated(x2, w[0], w[1], N, K, dt)
        torch.cuda.synchronize()
        assert torch.equal(h1[0], h2[0])


@pytest.mark.parametrize("N,K,xdt", [(3584, 3584, torch.float16), (2048, 4096, torch.float32),
                                     (4096, 2560, torch.bfloat16),
                                     # rows longer than a wave: gemv_rows_kernel (one and two levels)
                                     (3584, 18944, torch.float16), (1000, 10240, torch.float32),
                                     (2048, 6144, torch.bfloat16)])
def test_int4_cu_kernel_equals_persistent(dev, N, K, xdt):
    """int4 GEMV at one token (8-16 rows per CU with x quantized in the kernel, or rows longer
    than a wave on prepared activations): M = 1 against row 0 of M = 2."""
    print(f"[case] decode paths int4 N={N} K={K} x={xdt}", flush=True)
    g = synth.rng(7400 + N + K)
    G = 128
    codes, s, z = synth.int4_weight(N, K, G, g)
    ct, st, zt = (_t(a, dev) for a in (codes, s, z))
    x2 = torch.from_numpy(synth.activations(2, K, g)).to(xdt).to(dev)
    y1 = hipq.int4_matmul(x2[:1].contiguous(), ct, st, zt, G)
    y2 = hipq.int4_matmul(x2, ct, st, zt, G)
    torch.cuda.synchronize()
    assert torch.equal(y1[0], y2[0])


@pytest.mark.parametrize("dt,N,K", [(hipq.Q4_K, 4096, 14336), (hipq.Q5_K, 1000, 12288), (hipq.Q4_K, 300, 16384),
                                    (hipq.Q4_K, 2048, 8448), (hipq.Q5_K, 700, 28672)])
def test_long_rows_f32_x_equals_prepared_activations(dev, dt, N, K):
    """hq_matmul_q at one token with rows longer than 8192 (past the kernels that quantize x
    themselves) equals hq_quantize_act followed by hq_matmul_q_act bit for bit."""
    print(f"[case] long rows f32 x dt={hipq.NAMES[dt]} N={N} K={K}", flush=True)
    g = synth.rng(7500 + N + dt)
    w = _t(synth.gguf_weight(dt, N, K, g), dev)
    x = _t(synth.activations(1, K, g), dev)
    want = hipq.matmul_q_act(hipq.quantize_act(x), w, 1, N, K, dt)
    got = hipq.matmul_q(x, w, N, K, dt)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("N,K,xdt", [(3584, 18944, torch.float16), (1000, 10240, torch.float32),
                                     (2048, 8192, torch.bfloat16)])
def test_int4_long_rows_one_token_equals_two(dev, N, K, xdt):
    """int4 GEMV with K >= 8192 (a quantize launch, then the long-row kernel on single-level
    activations): M = 1 equals row 0 of M = 2 bit for bit."""
    print(f"[case] int4 long rows N={N} K={K} x={xdt}", flush=True)
    g = synth.rng(7600 + N + K)
    G = 128
    codes, s, z = synth.int4_weight(N, K, G, g)
    ct, st, zt = (_t(a, dev) for a in (codes, s, z))
    x2 = torch.from_numpy(synth.activations(2, K, g)).to(xdt).to(dev)
    y1 = hipq.int4_matmul(x2[:1].contiguous(), ct, st, zt, G)
    y2 = hipq.int4_matmul(x2, ct, st, zt, G)
    torch.cuda.synchronize()
    assert torch.equal(y1[0], y2[0])
