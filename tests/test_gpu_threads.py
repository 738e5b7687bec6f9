"""Host threads calling the library at once, each on its own stream with its own library
workspace (no ws argument): every result equals the single-threaded one bit for bit (the
one-launch MoE block included: it equals the two launches other streams take).  The
ctypes calls release the GIL, so the C ABI's calls overlap on the host (workspace map,
per-stream state, error text, first-use kernel attributes)."""
import threading

import pytest
import torch

from light_amd import hipq, synth

pytestmark = pytest.mark.gpu


def test_threads_on_own_streams(dev):
    print("[case] 8 host threads x 25 mixed calls", flush=True)
    g = synth.rng(77)
    t = lambda a: torch.from_numpy(a).to(dev)
    w4k = t(synth.gguf_weight(hipq.Q4_K, 4096, 4096, g))
    w80 = t(synth.gguf_weight(hipq.Q8_0, 2048, 4096, g))
    wdn = t(synth.gguf_weight(hipq.Q4_K, 4096, 14336, g))
    codes = torch.randint(0, 2 ** 31, (3584, 18944 // 8), dtype=torch.int32, device=dev)
    sc = torch.rand(3584, 18944 // 128, device=dev) * 0.02 + 1e-3
    zr = torch.full((3584, 18944 // 128), 8.0, device=dev)
    x1 = torch.randn(1, 4096, device=dev)
    x64 = torch.randn(64, 4096, device=dev)
    xl = torch.randn(2, 14336, device=dev)
    xi = torch.randn(16, 18944, device=dev).half()
    probs = torch.softmax(torch.randn(64, 128, device=dev), dim=1)
    wgu = t(synth.gguf_weight(hipq.Q4_K, 128 * 2 * 768, 2048, g))
    wmd = t(synth.gguf_weight(hipq.Q4_K, 128 * 2048, 768, g))
    xm = torch.randn(1, 2048, device=dev)
    calls = [
        lambda s: hipq.matmul_q(x1, w4k, 4096, 4096, hipq.Q4_K, stream=s),
        lambda s: hipq.matmul_q(x64, w4k, 4096, 4096, hipq.Q4_K, stream=s),
        lambda s: hipq.matmul_q(x1, w80, 2048, 4096, hipq.Q8_0, stream=s),
        lambda s: hipq.matmul_q(xl, wdn, 4096, 14336, hipq.Q4_K, stream=s),
        lambda s: hipq.int4_matmul(xi, codes, sc, zr, 128, stream=s),
        lambda s: hipq.moe_route(probs, 8, True, stream=s)[3],
        lambda s: hipq.matmul_q_gated(x1, w4k, w4k, 4096, 4096, hipq.Q4_K, stream=s),
        lambda s: hipq.mlp_q(x1, w4k, w4k, w4k, 4096, 4096, hipq.Q4_K, stream=s),
        # one token: the one-launch block on its owner stream, the two launches on the others
        lambda s: hipq.moe_block_q(probs[:1], xm, wgu, wmd, 128, 2048, 768, hipq.Q4_K, 8, stream=s)[0],
    ]
    want = [c(torch.cuda.current_stream()) for c in calls]
    torch.cuda.synchronize()
    errors = []

    def worker(k):
        try:
            s = torch.cuda.Stream(device=dev)
            outs = []
            with torch.cuda.stream(s):
                for i in range(25):
                    j = (i + k) % len(calls)
                    outs.append((j, calls[j](s)))
            s.synchronize()
            for j, o in outs:
                if not torch.equal(o, want[j]):
                    errors.append((k, j))
        except Exception as e:  # reported below
            errors.append((k, repr(e)))

    th = [threading.Thread(target=worker, args=(k,)) for k in range(8)]
    for x in th:
        x.start()
    for x in th:
        x.join(timeout=120)
    assert not any(x.is_alive() for x in th)
    assert not errors, errors[:5]
