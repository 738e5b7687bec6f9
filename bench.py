"""Benchmark of the MI355X quantized-matmul path (BASELINE.json metric).

Headline metric: "Q4_K GEMV GB/s (% of HBM peak) + Q4_K M=512 GEMM TFLOPS", Llama-3-8B
shapes.  Both halves are measured in the default run.

* `value` (GB/s): one "step" is one MLP decode pass through the hot path at M = 1, as
  Light's decoder runs it (models/llama.go:1306-1333), one hq_mlp_q call = two kernels:
      h = SiLU(x . Wgate^T) * (x . Wup^T)   gate/up 14336x4096 Q4_K (h emitted quantized)
      y = h . Wdown^T                        down 4096x14336 Q4_K
  value = algorithmic bytes of a step (the three weights as stored + F32 x in + F32 y out)
  / GPU time of the K timed steps, run back to back (HIP events around them, the host's
  enqueueing hidden behind a spin kernel; `graph_us_per_step`: the same steps replayed from a
  captured HIP graph, for reference).
* `roofline`: the step's dominant kernel, its first launch (hq_matmul_q_gated_act: the gated
  GEMV with the quantized-h epilogue), timed per launch with HIP events on its stream.
  `second_kernel` is the step's down GEMV, timed the same way.
* `gemm`: the Q4_K M = 512 prefill GEMM at both shapes, hq_matmul_q per call
  (the bf16 conversion of x plus the MFMA GEMM), TFLOP/s and fraction of the 2.5 PFLOP/s
  dense bf16 MFMA peak, with Light's CPU path beside it.
* `cpu_baseline`: Light's AVX2 CPU path (the C restatement in oracle/: MatMulQ, MatMulQ,
  SiLU, Mul, MatMulQ) on the same step, on the host cores available to this process.
* `table`: every named configuration (the GEMV / GEMM / int4 / MoE shapes and the added
  formats): µs per call, GB/s, TFLOP/s and fraction of HBM peak, with Light's CPU path for
  the same call beside it (a bounded sample where the whole call would take too long).

Inputs are synthetic (seeded, BASELINE distributions) and resident in HBM; every weight is
rotated over enough copies that the working set exceeds the 256 MB Infinity Cache.

Usage: python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-table] [--no-cpu]
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "int8": 5000.0}
MALL_BYTES = 256 << 20


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--table", action="store_true", help="also print the per-config table to stderr")
    p.add_argument("--no-table", action="store_true", help="leave the per-config table out of the line")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--launches", type=int, default=200, help="per-kernel timed launches for the roofline")
    p.add_argument("--gemm-launches", type=int, default=100, help="timed calls per M=512 GEMM shape")
    p.add_argument("--probe", action="store_true",
                   help="counter probe for rocprofv3 --pmc: a 64 MiB device copy, then the step's two GEMVs "
                        "and the M=512 GEMMs (no timing, no JSON line)")
    p.add_argument("--probe-int4", action="store_true",
                   help="counter probe: a 64 MiB device copy, then 5 calls of int4 M=64 at both Qwen2.5-7B shapes")
    return p.parse_args()


def copies_for(nbytes):
    return max(2, math.ceil(2 * MALL_BYTES / nbytes))


class Weight:
    """A GGUF weight with `n` rotated device copies."""

    def __init__(self, raw, dt, N, K, dev):
        import torch
        self.raw, self.dt, self.N, self.K = raw, dt, N, K
        base = torch.from_numpy(raw).to(dev)
        self.copies = [base] + [base.clone() for _ in range(copies_for(raw.nbytes) - 1)]

    def __getitem__(self, i):
        return self.copies[i % len(self.copies)]


def mlp_inputs(dev):
    """Llama-3-8B MLP decode at M = 1, config 1 (seed 1)."""
    import torch
    from light_amd import hipq, synth
    g = synth.rng(1)
    H, I = 4096, 14336
    gate = Weight(synth.gguf_weight(hipq.Q4_K, I, H, g), hipq.Q4_K, I, H, dev)
    up = Weight(synth.gguf_weight(hipq.Q4_K, I, H, g), hipq.Q4_K, I, H, dev)
    down = Weight(synth.gguf_weight(hipq.Q4_K, H, I, g), hipq.Q4_K, H, I, dev)
    x = synth.activations(1, H, g)
    h = synth.activations(1, I, g)
    return gate, up, down, x, h


def step_bytes(gate, up, down, M=1):
    """Algorithmic bytes of one MLP decode step: the three weights as stored, F32 x in and
    F32 y out (h stays inside the step)."""
    return gate.raw.nbytes + up.raw.nbytes + down.raw.nbytes + 4 * M * gate.K + 4 * M * down.N


def run_gpu(args):
    import torch
    from light_amd import hipq

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gate, up, down, x_np, h_np = mlp_inputs(dev)
    x = torch.from_numpy(x_np).to(dev)
    H, I = 4096, 14336
    ws = torch.empty(hipq.mlp_q_ws_bytes(1, H, I, hipq.Q4_K), dtype=torch.uint8, device=dev)
    y = torch.empty((1, H), device=dev)
    rot = max(len(gate.copies), len(down.copies))

    def step(i):
        hipq.mlp_q(x, gate[i], up[i], down[i], H, I, hipq.Q4_K, act=hipq.ACT_SILU, out=y, ws=ws)

    # Eager reference output of copy 0.
    step(0)
    torch.cuda.synchronize()
    eager = y.clone()

    # The timed steps: back-to-back hq_mlp_q calls rotating over the weight copies, timed by a
    # HIP event pair on the stream.  A spin kernel queued first keeps the GPU busy while the
    # host enqueues all K calls, so the interval is the K steps' own GPU time whatever the
    # host's per-call cost (a profiler's, say).
    def run_steps(n):
        for i in range(n):
            step(i % rot)

    run_steps(args.warmup)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(3e5 * args.steps))
    e0.record()
    run_steps(args.steps)
    e1.record()
    torch.cuda.synchronize()
    dt = e0.elapsed_time(e1) * 1e-3
    if not torch.equal(y, eager):  # copies hold identical bytes
        raise RuntimeError("a timed step differs from the eager step")
    nbytes = step_bytes(gate, up, down)
    ms_per_step = dt * 1e3 / args.steps
    value = nbytes * args.steps / dt / 1e9

    # The same steps captured as one HIP graph (a step per weight copy) and replayed, for
    # reference: on this stack a replay runs the step's two kernels about 1 us slower than
    # back-to-back launches.  Replays must reproduce the eager result.
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        full = torch.cuda.CUDAGraph()
        with torch.cuda.graph(full, stream=cap):
            for i in range(rot):
                step(i)
    torch.cuda.current_stream().wait_stream(cap)
    full.replay()
    torch.cuda.synchronize()
    if not torch.equal(y, eager):
        raise RuntimeError("graph replay differs from the eager step")
    nrep = max(1, args.steps // rot)
    t0 = time.perf_counter()
    for _ in range(nrep):
        full.replay()
    torch.cuda.synchronize()
    graph_us = (time.perf_counter() - t0) * 1e6 / (nrep * rot)

    roof = gemv_roofline(args, gate, up, x, dev)
    h = torch.from_numpy(h_np).to(dev)
    down_k = down_kernel(args, down, h, dev)
    return dict(value=value, ms_per_step=ms_per_step, step_bytes=nbytes, roofline=roof, down=down_k, graph_us=graph_us,
                inputs=(gate, up, down, x_np, h_np))


def time_launches(fn, n, rot):
    """Average per-launch duration (us): one HIP event pair on torch's current stream around n
    back-to-back launches, all queued behind a spin kernel so that host launch latency is hidden."""
    import torch
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    for i in range(min(n, 10)):
        fn(i)
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2e8))
    a.record()
    for i in range(n):
        fn(i)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / n


def gemv_roofline(args, gate, up, x, dev):
    """Roofline of the step's dominant kernel: its first launch, the fused gate/up Q4_K GEMV
    that quantizes h into the act layout in its epilogue (hq_matmul_q_gated_act, the call
    hq_mlp_q makes), x F32 quantized inside the kernel."""
    import torch
    from light_amd import hipq
    N, K = gate.N, gate.K
    ab = hipq.lib().hq_act_bytes(1, N)
    out = torch.empty(ab, dtype=torch.uint8, device=dev)
    us = time_launches(lambda i: hipq.matmul_q_gated_act(x, gate[i], up[i], N, K, hipq.Q4_K, out=out),
                       args.launches, len(gate.copies))
    alg = gate.raw.nbytes + up.raw.nbytes + 4 * K + ab  # both weights + F32 x + quantized h
    achieved = alg / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(f"gated_act N={N} K={K} M=1"),
            "kernel": "gemv_q4kx_kernel (gated, quantized-h epilogue)", "shape": f"gate+up N={N} K={K} M=1",
            "alg_bytes_per_launch": alg, "avg_launch_us": round(us, 3)}


def down_kernel(args, down, h, dev):
    """The step's second kernel: the down projection GEMV on prepared activations
    (gemv_q4kx_kernel, act input)."""
    import torch
    from light_amd import hipq
    N, K = down.N, down.K
    out = torch.empty((1, N), device=dev)
    act = hipq.quantize_act(h)
    us = time_launches(lambda i: hipq.matmul_q_act(act, down[i], 1, N, K, hipq.Q4_K, out=out), args.launches,
                       len(down.copies))
    alg = down.raw.nbytes + hipq.lib().hq_act_bytes(1, K) + 4 * N
    gbs = alg / (us * 1e-6) / 1e9
    return {"kernel": "gemv_q4kx_kernel (act input)", "shape": f"down N={N} K={K} M=1", "avg_launch_us": round(us, 3),
            "achieved": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "alg_bytes_per_launch": alg,
            "traffic": measured_traffic(f"down act N={N} K={K} M=1")}


def ceilings(args, dev, step_us, kernel_bytes):
    """What the hardware sustains on this box, measured in this run (context for the roofline
    fractions, never their denominator): hq_ceiling_read, a plain streaming read launch of the
    step's kernel sizes and of the whole step's bytes, rotating over a 640 MB buffer (beyond
    the 256 MB MALL), in two access orders with two 16-byte loads in flight per thread, and
    the 268 MB read once more as half cache lines; hq_ceiling_mfma, back-to-back
    register-operand v_mfma_f32_32x32x16_bf16; and hq_ceiling_mix, how far a SIMD overlaps
    MFMA and VALU work."""
    import ctypes
    import torch
    from light_amd import hipq
    L = hipq.lib()
    big = torch.empty(640 << 20, dtype=torch.uint8, device=dev)
    big.fill_(1)
    sink = torch.zeros(64, dtype=torch.int32, device=dev)
    base = big.data_ptr()

    def read_us(nbytes, order, n=60, rotate=True):
        nbytes = nbytes // 2048 * 2048
        nwin = big.numel() // nbytes if rotate else 1

        def fn(i):
            hipq.check(L.hq_ceiling_read(ctypes.c_void_p(base + (i % nwin) * nbytes), nbytes, order, 2,
                                         ctypes.c_void_p(sink.data_ptr()), None))
        return time_launches(fn, n, nwin)

    sizes = sorted(set(kernel_bytes) | {sum(kernel_bytes), 268435456})
    reads = []
    for nb in sizes:
        for order, name in ((0, "window"), (1, "slice")):
            us = read_us(nb, order)
            reads.append({"bytes": nb, "order": name, "loads_in_flight_per_thread": 2, "us": round(us, 2),
                          "GBs": round(nb / us / 1e3, 1), "frac": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)})
    half = read_us(268435456, 2)
    reads.append({"bytes": 268435456, "order": "half_lines", "loads_in_flight_per_thread": 2, "us": round(half, 2),
                  "GBs": round(268435456 / half / 1e3, 1), "frac": round(268435456 / half / 1e3 / HBM_PEAK_GBS, 4)})
    best = {nb: min(r["us"] for r in reads if r["bytes"] == nb and r["order"] != "half_lines") for nb in sizes}
    # The same 16 MB read again and again: after the first launch it sits in the XCDs' L2s, so
    # the CUs' request rate, not HBM, bounds it -- whole lines against half lines.
    l2 = []
    for order, name in ((0, "window"), (2, "half_lines")):
        us = read_us(16 << 20, order, rotate=False)
        l2.append({"bytes": 16 << 20, "order": name, "us": round(us, 2), "GBs": round((16 << 20) / us / 1e3, 1)})
    two = sum(best[nb] for nb in kernel_bytes)
    flops = ctypes.c_int64()
    sf = torch.zeros(16, device=dev)
    iters = 20000
    hipq.check(L.hq_ceiling_mfma(iters, ctypes.c_void_p(sf.data_ptr()), ctypes.byref(flops), None))
    us = time_launches(lambda i: hipq.check(L.hq_ceiling_mfma(iters, ctypes.c_void_p(sf.data_ptr()),
                                                               ctypes.byref(flops), None)), 5, 1)
    tf = flops.value / us / 1e6
    mix_iters = 4000
    mix = [time_launches(lambda i, m=m: hipq.check(L.hq_ceiling_mix(m, mix_iters, ctypes.c_void_p(sf.data_ptr()), None)),
                         5, 1) * 1e3 / mix_iters for m in (0, 1, 2)]
    del big
    torch.cuda.empty_cache()
    return {"read": reads,
            "read_l2_resident": l2,
            "step_kernels_read_us": round(two, 2),
            "step_vs_read_ceiling": round(two / step_us, 4),
            "step_one_launch_read_us": best[sum(kernel_bytes)],
            "mfma_bf16": {"TFLOPS": round(tf, 1), "frac_of_peak": round(tf / 2500.0, 4),
                          "kernel": "4 independent v_mfma_f32_32x32x16_bf16 chains per wave, register operands, "
                                    "2 waves per SIMD"},
            "mfma_valu_mix": {"ns_per_round": {"mfma": round(mix[0], 2), "valu": round(mix[1], 2), "both": round(mix[2], 2)},
                              "overlap": round((mix[0] + mix[1] - mix[2]) / min(mix[0], mix[1]), 3),
                              "round": "20 v_mfma_f32_16x16x32_f16 and/or 80 v_pk_fma_f16 per wave, 2 waves per SIMD; "
                                       "overlap 1 = the shorter hidden entirely, 0 = none"}}


GEMM_SHAPES = ((512, 14336, 4096), (512, 4096, 14336))


def gemm_records(args, dev, cpu=True):
    """Q4_K prefill GEMM at M = 512, both shapes, per hq_matmul_q call (x F32 ->
    bf16 conversion launch + the MFMA GEMM), weights rotated past the Infinity Cache."""
    import torch
    from light_amd import hipq, synth
    out = []
    for idx, (M, N, K) in enumerate(GEMM_SHAPES):
        g = synth.rng(20 + idx)
        w = Weight(synth.gguf_weight(hipq.Q4_K, N, K, g), hipq.Q4_K, N, K, dev)
        x_np = synth.activations(M, K, g)
        x = torch.from_numpy(x_np).to(dev)
        y = torch.empty((M, N), device=dev)
        ws = torch.empty(hipq.matmul_q_ws_bytes(M, N, K, hipq.Q4_K), dtype=torch.uint8, device=dev)
        us = time_launches(lambda i: hipq.matmul_q(x, w[i], N, K, hipq.Q4_K, out=y, ws=ws), args.gemm_launches,
                           len(w.copies))
        flops = 2 * M * N * K
        tflops = flops / (us * 1e-6) / 1e12
        kern = "to_bf16_kernel + gemm_q4k_kernel<112>" if N % 112 == 0 else \
            "to_bf16_kernel + gemm_q4k_kernel<128> (K split 4) + splitk_reduce_kernel"
        rec = {"shape": f"M={M} N={N} K={K}", "kernel": kern,
               "us_per_call": round(us, 2), "TFLOPS": round(tflops, 1), "peak": MFMA_PEAK_TFLOPS["bf16"],
               "peak_unit": "TFLOP/s (dense bf16 MFMA)", "frac": round(tflops / MFMA_PEAK_TFLOPS["bf16"], 4),
               "flops_per_call": flops,
               "traffic": measured_traffic(f"gemm M={M} N={N} K={K}" + ("" if N % 112 == 0 else " (K split 4)"))}
        if cpu:
            t, th, smp = cpu_gguf_row(x_np, w.raw, N, K, hipq.Q4_K)
            rec["cpu"] = {"us_per_call": round(t * 1e6, 1), "TFLOPS": round(flops / t / 1e12, 4), "cores": th,
                          "kind": "port", "sample": smp}
        out.append(rec)
        del w, x, y, ws
        torch.cuda.empty_cache()
    return out


def measured_traffic(shape):
    """HBM bytes per launch of one reported kernel from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE runs (profiles/q4k_traffic.md gives the commands and the copy-kernel scaling)."""
    path = os.path.join(ROOT, "profiles", "q4k_traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return None
    for r in d.get("kernels", []):
        if r.get("shape") == shape:
            return r.get("traffic_bytes")
    return None


def table(args, dev):
    """Per-config µs/call, GB/s, TFLOPS and roofline fraction (stderr)."""
    import numpy as np
    import torch
    from light_amd import hipq, synth
    rows = []
    for name, c in list(synth.CONFIGS.items()) + list(synth.EXTRA_CONFIGS.items()):
        g = synth.rng(c["cfg"])
        try:
            if c["kind"] == "gguf":
                M, N, K, dt = c["M"], c["N"], c["K"], c["dt"]
                w = Weight(synth.gguf_weight(dt, N, K, g), dt, N, K, dev)
                x = torch.from_numpy(synth.activations(M, K, g)).to(dev)
                out = torch.empty((M, N), device=dev)
                kdt = dt
                if c.get("repack"):  # Q6_K_R: the load-time planar copy; bytes per call as stored in GGUF
                    w.copies = [hipq.repack_q6k(cp, N, K) for cp in w.copies]
                    kdt = hipq.Q6_K_R
                ws = torch.empty(max(hipq.matmul_q_ws_bytes(M, N, K, kdt), 256), dtype=torch.uint8, device=dev)
                us = time_launches(lambda i: hipq.matmul_q(x, w[i], N, K, kdt, out=out, ws=ws), 100,
                                   len(w.copies))
                nbytes = w.raw.nbytes + 4 * M * K + 4 * M * N
                flops = 2 * M * N * K
            elif c["kind"] == "int4":
                M, N, K, G = c["M"], c["N"], c["K"], c["G"]
                codes, s, z = synth.int4_weight(N, K, G, g)
                xt = torch.from_numpy(synth.activations(M, K, g, np.float16)).to(dev)
                ct, st, zt = (torch.from_numpy(a).to(dev) for a in (codes, s, z))
                reps = copies_for(codes.nbytes)
                cs = [ct] + [ct.clone() for _ in range(reps - 1)]
                out = torch.empty((M, N), dtype=torch.float16, device=dev)
                us = time_launches(lambda i: hipq.int4_matmul(xt, cs[i % reps], st, zt, G, out=out), 100, reps)
                nbytes = codes.nbytes + s.nbytes + z.nbytes + 2 * M * K + 2 * M * N
                flops = 2 * M * N * K
            else:
                rows.extend(moe_rows(c, name, g, dev, cpu=not args.no_cpu))
                continue
        except hipq.HipqError as e:
            rows.append(dict(config=name, error=str(e)))
            continue
        gbs = nbytes / (us * 1e-6) / 1e9
        tfl = flops / (us * 1e-6) / 1e12
        row = dict(config=name, us=round(us, 2), GBs=round(gbs, 1), TFLOPS=round(tfl, 2),
                   hbm_frac=round(gbs / HBM_PEAK_GBS, 3))
        if not args.no_cpu:
            import oracle
            if c["kind"] == "gguf":
                t, th, smp = cpu_gguf_row(x.cpu().numpy(), w.raw, N, K, dt)
            else:
                xf = xt.cpu().float().numpy()
                th = _cpu_threads()
                t, smp = _cpu_median(lambda: oracle.int4_matmul(xf, codes, s, z, N, K, G, th), 1), "whole call"
            row.update(cpu_us=round(t * 1e6, 1), cpu_threads=th, cpu_sample=smp, gpu_over_cpu=round(t * 1e6 / us, 1))
        rows.append(row)
        torch.cuda.empty_cache()
    return rows


def moe_rows(c, name, g, dev, cpu=False):
    """MoE gate/up (per token) and down (per pair, weighted) Q4_K grouped GEMMs of one layer.
    Routing rotates over 16 draws so consecutive calls touch different experts (the stacks,
    340 MB, then exceed the 256 MB Infinity Cache)."""
    import numpy as np
    import torch
    from light_amd import hipq, synth
    E, topk, H, I, T = c["E"], c["topk"], c["H"], c["I"], c["T"]
    dt = hipq.Q4_K
    wgu_np = synth.gguf_weight(dt, E * 2 * I, H, g)
    wdn_np = synth.gguf_weight(dt, E * H, I, g)
    wgu, wdn = torch.from_numpy(wgu_np).to(dev), torch.from_numpy(wdn_np).to(dev)
    routes = []
    for _ in range(16):
        ids, tw = synth.moe_routing(T, E, topk, g)
        se, sp = synth.sort_pairs(ids)
        routes.append((ids, torch.from_numpy(se).to(dev), torch.from_numpy(sp).to(dev), torch.from_numpy(tw).to(dev)))
    M = T * topk
    x = torch.from_numpy(synth.activations(T, H, g)).to(dev)
    h = torch.from_numpy(synth.activations(M, I, g)).to(dev)
    ogu = torch.zeros((M, 2 * I), device=dev)
    odn = torch.zeros((M, H), device=dev)
    counts = torch.zeros(E, dtype=torch.int32, device=dev)
    offsets = torch.zeros(E + 1, dtype=torch.int32, device=dev)
    ws = torch.empty(max(hipq.moe_gemm_q_ws_bytes(T, H, dt), hipq.moe_gemm_q_ws_bytes(M, I, dt), 256),
                     dtype=torch.uint8, device=dev)
    ebytes_gu, ebytes_dn = 2 * I * (H // 256) * 144, H * (I // 256) * 144
    out = []
    for leg, fn, eb, flops_n, flops_k, xb, ob in (
            ("gate_up", lambda r: hipq.moe_gemm_q(x, wgu, r[2], r[1], E, 2 * I, H, dt, topk, out=ogu, counts=counts,
                                                   offsets=offsets, ws=ws), ebytes_gu, 2 * I, H, 4 * T * H, 4 * M * 2 * I),
            ("down", lambda r: hipq.moe_gemm_q(h, wdn, r[2], r[1], E, H, I, dt, topk, topk_w=r[3], out=odn,
                                                counts=counts, offsets=offsets, ws=ws), ebytes_dn, H, I, 4 * M * I, 4 * M * H)):
        us = time_launches(lambda i: fn(routes[i % 16]), 64, 16)
        used = float(np.mean([len(np.unique(r[0])) for r in routes]))
        nbytes = used * eb + xb + ob
        flops = 2.0 * M * flops_n * flops_k
        gbs = nbytes / (us * 1e-6) / 1e9
        row = dict(config=f"{name}_{leg}", us=round(us, 2), GBs=round(gbs, 1),
                   TFLOPS=round(flops / (us * 1e-6) / 1e12, 2), hbm_frac=round(gbs / HBM_PEAK_GBS, 3))
        if cpu:
            ids, se_np, sp_np, tw_np = routes[0][0], *(r.cpu().numpy() for r in routes[0][1:])
            if leg == "gate_up":
                t, th, smp = cpu_moe_leg(x.cpu().numpy(), wgu_np, dt, E, 2 * I, H, sp_np, se_np, topk)
            else:
                t, th, smp = cpu_moe_leg(h.cpu().numpy(), wdn_np, dt, E, H, I, sp_np, se_np, topk, tw_np)
            row.update(cpu_us=round(t * 1e6, 1), cpu_threads=th, cpu_sample=smp, gpu_over_cpu=round(t * 1e6 / us, 1))
        out.append(row)
    # The whole routed block on the device (hq_moe_block_q): router probs -> routing + gated
    # gate/up (SiLU * up) -> down (routing-weighted) with the combine in its epilogue, in one
    # launch for a single token.  Probs rotate over 16 draws.
    probs = []
    for _ in range(16):
        lg = torch.from_numpy(g.standard_normal((T, E)).astype(np.float32))
        probs.append(torch.softmax(lg, dim=1).to(dev))
    hg = torch.zeros((M, I), device=dev)
    ws_g = torch.empty(max(hipq.moe_gemm_q_gated_ws_bytes(M, T, I, H, dt), 256), dtype=torch.uint8, device=dev)
    yb = torch.empty((T, H), device=dev)

    ws_b = torch.empty(max(hipq.lib().hq_moe_block_q_ws_bytes(T, topk, E, H, I, dt), 256), dtype=torch.uint8,
                       device=dev)

    def block(i):  # hq_moe_block_q: one launch for a single token, else route-gated + combine
        hipq.moe_block_q(probs[i % 16], x, wgu, wdn, E, H, I, dt, topk, out=yb, h=hg, ws=ws_b)

    us = time_launches(block, 64, 16)
    used = float(np.mean([len(np.unique(torch.topk(p_, topk, dim=1).indices.cpu().numpy())) for p_ in probs]))
    nbytes = used * (ebytes_gu + ebytes_dn) + 4 * T * E + 4 * T * H * 2
    gbs = nbytes / (us * 1e-6) / 1e9
    brow = dict(config=f"{name}_block", us=round(us, 2), GBs=round(gbs, 1),
                TFLOPS=round(2.0 * M * (2 * I * H + H * I) / (us * 1e-6) / 1e12, 2),
                hbm_frac=round(gbs / HBM_PEAK_GBS, 3))
    legs = [r for r in out if r["config"] in (f"{name}_gate_up", f"{name}_down") and "cpu_us" in r]
    if cpu and len(legs) == 2:
        # Light's CPU block is its routing (a top-k and a sort of T x E values, negligible here)
        # plus the two MoEGemmQ legs (the SiLU * up and the combine are O(T topk I) adds): the
        # sum of the two legs' CPU times above.
        t = sum(r["cpu_us"] for r in legs)
        brow.update(cpu_us=round(t, 1), cpu_threads=legs[0]["cpu_threads"],
                    cpu_sample="sum of the gate_up and down rows' CPU times", gpu_over_cpu=round(t / us, 1))
    out.append(brow)
    return out


def _cpu_threads():
    """Host cores this process may use (the GOMAXPROCS / hardware_concurrency role): the CPU
    affinity set, capped by a cgroup CPU quota when one is set."""
    n = len(os.sched_getaffinity(0))
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            n = min(n, max(1, math.ceil(int(quota) / int(period))))
    except (OSError, ValueError):
        pass
    return max(1, n)


def _cpu_median(fn, reps=3):
    """Median wall time (s) of `reps` calls after one warm-up."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_gguf_row(x, raw, N, K, dt):
    """Light's CPU MatMulQ (oracle restatement) on a bounded sample of one table config: all of
    it when it is small; a slice of the weight rows, or of the activation rows for M > 8, scaled
    back linearly otherwise (the sample says which)."""
    import oracle
    M = x.shape[0]
    th = _cpu_threads()
    bb = oracle.BLOCK[dt][1] * (K // oracle.BLOCK[dt][0])  # bytes per weight row
    if M > 8:
        ms = 32
        t = _cpu_median(lambda: oracle.matmul_q(x[:ms], raw, N, K, dt, th), 1) * (M / ms)
        return t, th, f"M={ms} of {M} rows x {M // ms}"
    if N * K > (64 << 20):
        ns = N // 8
        t = _cpu_median(lambda: oracle.matmul_q(x, raw[:ns * bb], ns, K, dt, th)) * (N / ns)
        return t, th, f"{ns} of {N} weight rows x 8"
    return _cpu_median(lambda: oracle.matmul_q(x, raw, N, K, dt, th)), th, "whole call"


def cpu_moe_leg(x, w_raw, dt, E, N, K, sp, se, topk, tw=None):
    """Light's CPU MoEGemmQ: dequantize the whole (E, N, K) stack (single thread, as
    quant.Dequantize), then moeGemmKernel over the pairs.  The dequant is timed on 16 experts and
    scaled to E; the pair dots run in full on a 16-expert stack with expert ids folded mod 16
    (the same number of dot products)."""
    import numpy as np
    import oracle
    th = _cpu_threads()
    es = min(16, E)
    nb = w_raw.size // E
    sub = np.ascontiguousarray(w_raw.reshape(E, nb)[:es]).ravel()
    t_deq = _cpu_median(lambda: oracle.dequant(dt, sub, es * N * K), 1) * (E / es)
    wf = oracle.dequant(dt, sub, es * N * K).reshape(es, N, K)
    se_f = np.asarray(se) % es
    order = np.argsort(se_f, kind="stable")
    t_gemm = _cpu_median(lambda: oracle.moe_gemm_f32(x, wf, np.asarray(sp)[order], se_f[order], topk, tw, th), 1)
    return t_deq + t_gemm, th, f"dequant {t_deq * 1e3:.1f} ms (16 of {E} experts x {E // es}) + dots {t_gemm * 1e3:.1f} ms"


def cpu_baseline(inputs):
    """Light's AVX2 CPU path (oracle C restatement: MatMulQ, MatMulQ, SiLU, Mul, MatMulQ) on the same
    step; median of 5 after a warm-up."""
    import oracle
    gate, up, down, x, _ = inputs
    threads = _cpu_threads()

    def run():
        g = oracle.matmul_q(x, gate.raw, gate.N, gate.K, gate.dt, threads)
        u = oracle.matmul_q(x, up.raw, up.N, up.K, up.dt, threads)
        h = oracle.gated(g, u, 0)
        oracle.matmul_q(h, down.raw, down.N, down.K, down.dt, threads)

    run()
    ts = []
    for _ in range(5):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    nbytes = step_bytes(gate, up, down)
    return {"value": round(nbytes / t / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"5 timed MLP decode steps (gate, up, SiLU*up, down; Q4_K, M=1), median {t * 1e3:.2f} ms/step",
            "cpu": _cpu_model()}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def probe(dev):
    """Known-size copy (reference for the counters' scale), then the kernels the JSON line
    reports: the step's first launch (gated GEMV, quantized-h epilogue) x20, its down GEMV on
    prepared activations x20 and the M = 512 GEMM at both shapes x5 each."""
    import torch
    from light_amd import hipq, synth
    src = torch.ones(64 << 18, dtype=torch.float32, device=dev)  # 64 MiB
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    gate, up, down, x_np, h_np = mlp_inputs(dev)
    x = torch.from_numpy(x_np).to(dev)
    out = torch.empty(hipq.lib().hq_act_bytes(1, gate.N), dtype=torch.uint8, device=dev)
    for i in range(20):
        hipq.matmul_q_gated_act(x, gate[i], up[i], gate.N, gate.K, hipq.Q4_K, out=out)
    act = hipq.quantize_act(torch.from_numpy(h_np).to(dev))
    y = torch.empty((1, down.N), device=dev)
    for i in range(20):
        hipq.matmul_q_act(act, down[i], 1, down.N, down.K, hipq.Q4_K, out=y)
    torch.cuda.synchronize()
    del gate, up, down
    torch.cuda.empty_cache()
    for idx, (M, N, K) in enumerate(GEMM_SHAPES):
        g = synth.rng(20 + idx)
        w = Weight(synth.gguf_weight(hipq.Q4_K, N, K, g), hipq.Q4_K, N, K, dev)
        xg = torch.from_numpy(synth.activations(M, K, g)).to(dev)
        yg = torch.empty((M, N), device=dev)
        ws = torch.empty(hipq.matmul_q_ws_bytes(M, N, K, hipq.Q4_K), dtype=torch.uint8, device=dev)
        for i in range(5):
            hipq.matmul_q(xg, w[i], N, K, hipq.Q4_K, out=yg, ws=ws)
        torch.cuda.synchronize()
        del w
        torch.cuda.empty_cache()
    print("probe: copy 67108864 B x3; gated_act N=14336 K=4096 x20; down act N=4096 K=14336 x20; "
          "gemm M=512 (14336x4096, 4096x14336) x5 each", file=sys.stderr)


def probe_int4(dev):
    """Known-size copy, then configs[3]'s M = 64 int4 matmul (f16 x) at both shapes, 5 calls each."""
    import numpy as np
    import torch
    from light_amd import hipq, synth
    src = torch.ones(64 << 18, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    for name in ("int4_m64_18944x3584", "int4_m64_3584x18944"):
        c = synth.CONFIGS[name]
        g = synth.rng(c["cfg"])
        M, N, K, G = c["M"], c["N"], c["K"], c["G"]
        codes, s, z = synth.int4_weight(N, K, G, g)
        x = torch.from_numpy(synth.activations(M, K, g, np.float16)).to(dev)
        ct, st, zt = (torch.from_numpy(a).to(dev) for a in (codes, s, z))
        out = torch.empty((M, N), dtype=torch.float16, device=dev)
        for _ in range(5):
            hipq.int4_matmul(x, ct, st, zt, G, out=out)
        torch.cuda.synchronize()
    print("probe: copy 67108864 B x3; int4 M=64 (18944x3584, 3584x18944) x5 each", file=sys.stderr)


def main():
    args = parse()
    if args.probe_int4:
        import torch
        probe_int4(torch.device("cuda:0"))
        return
    if args.probe:
        import torch
        probe(torch.device("cuda:0"))
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "sharding the weights' N rows across GPUs is designed but not built", file=sys.stderr)
        sys.exit(2)
    res = run_gpu(args)
    line = {
        "metric": "Q4_K GEMV GB/s (% of HBM peak) + Q4_K M=512 GEMM TFLOPS, Llama-3-8B shapes",
        "value": round(res["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 5),
        "graph_us_per_step": round(res["graph_us"], 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k x q8_1 -> f32 (int8 dot, f32 accumulate)",
        "data": "synthetic (seeded, BASELINE.json distributions; weights rotated over >512 MB)",
        "config": {"workload": "llama3_8b_mlp_decode_q4_k", "M": 1, "hidden": 4096, "intermediate": 14336,
                   "matmuls": ["gate+up 2x14336x4096 (fused, SiLU*up, h quantized in the epilogue)",
                               "down 4096x14336"],
                   "step_bytes": res["step_bytes"]},
        "roofline": res["roofline"],
        "second_kernel": res["down"],
    }
    import torch
    line["ceilings"] = ceilings(args, torch.device("cuda:0"), res["ms_per_step"] * 1e3,
                                [res["roofline"]["alg_bytes_per_launch"], res["down"]["alg_bytes_per_launch"]])
    line["gemm"] = gemm_records(args, torch.device("cuda:0"), cpu=not args.no_cpu)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(res["inputs"])
    if args.table or not args.no_table:
        line["table"] = table(args, torch.device("cuda:0"))
        if args.table:
            print(json.dumps({"table": line["table"]}), file=sys.stderr)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
