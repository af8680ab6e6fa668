"""Benchmark of the bfp16-weight GEMM path on one MI355X.

Workload (one step): the DiT FFN pair at M = 4352 tokens, hidden 3072, FF 12288 with bfp16 weights ~N(0, 0.02) and
bf16 activations ~N(0, 1), seed 0:
  quantize  x (4352 x 3072 bf16) -> bfp16 packed bytes + decoded bf16 (bit-exact to the CPU packer)
  up GEMM   4352 x 3072 x (2 x 12288), SwiGLU on the [gate 64 | proj 64] interleave, output re-quantized to bfp16
  down GEMM 4352 x 12288 x 3072, out = residual + gate[n] * acc
The metric is the step's GEMM throughput (2MNK summed over both GEMMs, quantize time included) in TFLOP/s, the step
captured once as a HIP graph and replayed (its eager time, launched from Python, is reported beside it). The
roofline object is for the dominant kernel, the up GEMM (657.13 GFLOP per call), against the dense bf16 MFMA peak; the
library runs that call as two launches (the 4-wave kernel over rows 0..4095 in 512 x 128 tiles, six full rounds of the
256 CUs, then the same kernel over the last 256 rows in 256 x 128 tiles), timed together. Kernel times are medians of
HIP-event intervals on the launch stream. Before the warmup steps the step runs untimed for SETTLE_S seconds, so that
the timed steps see the sustained clock rather than power management's first tens of milliseconds.
Also reported: the adaLN modulation GEMV (M=1, K=3072, N=18432, SiLU) in GB/s against HBM (8 TB/s), timed over six
rotating weight copies so that the 256 MB MALL cannot hold them; the residual + LayerNorm + modulate pass that
produces the up GEMM's A (4352 x 3072) and the QKV post pass (4352 tokens x 24 heads) in GB/s against HBM; attention
over 4352 tokens x 24 heads in TFLOP/s (torch's SDPA beside it); the GEMMs of the other reference configurations
(1, 2, 4 and 5: see configs_bench) in TFLOP/s; and the CPU baseline (the oracle's numpy restatement of the reference
CPU path on a row sample of the same workload).

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--no-cpu] [--copy-probe MB] [--sustain SECONDS]
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "redline-tiny_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (vendor figure)
PEAK_HBM_GBPS = 8000.0     # MI355X HBM3E
# HBM bytes per up-GEMM call (its two launches) from rocprofv3 FETCH_SIZE (x2) and WRITE_SIZE (x1), the factors that make a 256 MB
# device-to-device copy read and write 256 MB (profiles/gemm_dit_ffn_counters.md); re-measured when the kernel changes
UP_GEMM_TRAFFIC_BYTES = 853128984
M, K, FF = 4352, 3072, 12288
GEMV_K, GEMV_N = 3072, 18432
# seconds of untimed runs before each timed region (the clock settles within ~50 ms of load); RLBFP_BENCH_SETTLE_S
# overrides it (0 for counter-collection runs, where every extra dispatch is profiled)
SETTLE_S = float(os.environ.get("RLBFP_BENCH_SETTLE_S", "0.3"))


def flops_up():
    return 2.0 * M * K * 2 * FF


def flops_down():
    return 2.0 * M * FF * K


def make_inputs(dev):
    import numpy as np
    import torch

    from rlbfp import ops

    rng = np.random.default_rng(0)
    x = rng.standard_normal((M, K), dtype=np.float32)                      # activations first
    w_gate = rng.standard_normal((FF, K), dtype=np.float32) * 0.02         # then weights
    w_proj = rng.standard_normal((FF, K), dtype=np.float32) * 0.02
    w_down = rng.standard_normal((K, FF), dtype=np.float32) * 0.02
    res = rng.standard_normal((M, K), dtype=np.float32)                    # then epilogue vectors
    gate = rng.standard_normal(K, dtype=np.float32)
    t = lambda a, dt: torch.from_numpy(a).to(dev).to(dt)
    up = ops.pack_weight(ops.interleave_up(t(w_gate, torch.float32), t(w_proj, torch.float32)).contiguous())
    down = ops.pack_weight(t(w_down, torch.float32))
    return {"x": t(x, torch.bfloat16), "up": up, "down": down, "res": t(res, torch.bfloat16),
            "gate": t(gate, torch.float32)}, (x, w_gate, w_proj, w_down, res, gate)


class Timer:
    """HIP events on torch's current stream (the stream the kernels are launched on) around each kernel."""

    def __init__(self):
        import torch
        self.torch = torch
        self.ev = {}

    def mark(self, name):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        self.ev.setdefault(name, []).append(e)

    def median_ms(self, a, b):
        ts = sorted(x.elapsed_time(y) for x, y in zip(self.ev[a], self.ev[b]))
        n = len(ts)
        return ts[n // 2] if n % 2 else 0.5 * (ts[n // 2 - 1] + ts[n // 2])


def gpu_bench(steps, warmup, no_configs=False):
    import torch

    from rlbfp import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    inp, host = make_inputs(dev)
    h = torch.empty((M, FF), dtype=torch.bfloat16, device=dev)
    y = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    xq = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    xp = torch.empty(M * K // 8 * 9, dtype=torch.uint8, device=dev)
    from rlbfp import _lib as L
    import ctypes
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def quantize():
        L.check(L.lib().rl_bfp16_quantize(ctypes.c_void_p(inp["x"].data_ptr()), L.RL_DTYPE_BF16, M, K, K,
                                          L.RL_ORDER_ROWBLOCK, ctypes.c_void_p(xp.data_ptr()),
                                          ctypes.c_void_p(xq.data_ptr()), stream()))

    def step(tm=None):
        if tm:
            tm.mark("q0")
        quantize()
        if tm:
            tm.mark("up0")
        ops.gemm(xq, inp["up"], 2 * FF, K, act="swiglu", quantize_out=True, out=h)
        if tm:
            tm.mark("down0")
        ops.gemm(h, inp["down"], K, FF, gate=inp["gate"], residual=inp["res"], out=y)
        if tm:
            tm.mark("end")

    settle(step)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    tm = Timer()
    t0 = time.perf_counter()
    for _ in range(steps):
        step(tm)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_q, ms_up, ms_down = tm.median_ms("q0", "up0"), tm.median_ms("up0", "down0"), tm.median_ms("down0", "end")
    ms_step_eager = wall * 1e3 / steps
    y_eager = y.clone()

    # The step as one HIP graph (its four launches enqueued back to back, as the reference submits its merged program
    # asynchronously), replayed `steps` times between synchronisations; every replay recomputes all outputs, and the
    # last one must equal the eager result bit for bit.
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            step()
    torch.cuda.current_stream().wait_stream(side)
    settle(graph.replay)
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g0.record()
    for _ in range(steps):
        graph.replay()
    g1.record()
    torch.cuda.synchronize()
    ms_step = g0.elapsed_time(g1) / steps
    assert torch.equal(y, y_eager), "graph replay of the step differs from the eager result"
    h_step = h.clone()
    v9a = v9a_bench(inp, xq, h_step)

    # the quantize pass alone: a ~12 us kernel whose event interval inside the eager step also holds a kernel
    # boundary, so it is timed like the GEMV, in graph replays rotating over 4 inputs and outputs (274 MB > MALL)
    qx = [inp["x"]] + [torch.randn((M, K), generator=torch.Generator(device=dev).manual_seed(50 + c),
                                   device=dev).to(torch.bfloat16) for c in range(3)]
    qp = [torch.empty_like(xp) for _ in range(4)]
    qq = [torch.empty_like(xq) for _ in range(4)]

    def quantize_rot(i):
        j = i % 4
        L.check(L.lib().rl_bfp16_quantize(ctypes.c_void_p(qx[j].data_ptr()), L.RL_DTYPE_BF16, M, K, K,
                                          L.RL_ORDER_ROWBLOCK, ctypes.c_void_p(qp[j].data_ptr()),
                                          ctypes.c_void_p(qq[j].data_ptr()), stream()))

    us_q_alone = graph_us(quantize_rot, 8, 40, 5)
    assert torch.equal(qq[0], xq), "the quantize pass in graph replays differs from the step's"

    # the same pass with the packed output only (to_bfp16 alone: 2 bytes read, 9/8 written per value)
    def quantize_packed_rot(i):
        j = i % 4
        L.check(L.lib().rl_bfp16_quantize(ctypes.c_void_p(qx[j].data_ptr()), L.RL_DTYPE_BF16, M, K, K,
                                          L.RL_ORDER_ROWBLOCK, ctypes.c_void_p(qp[j].data_ptr()), None, stream()))

    us_q_packed = graph_us(quantize_packed_rot, 8, 40, 5)
    assert torch.equal(qp[0], xp), "the packed-only quantize pass differs from the step's packed bytes"
    del qx, qp, qq

    # GEMV: M = 1 adaLN modulation, weights rotated over 6 copies (382 MB > 256 MB MALL)
    rng_x = torch.randn((1, GEMV_K), generator=torch.Generator().manual_seed(0)).to(dev, torch.bfloat16)
    copies = []
    for c in range(6):
        g = torch.Generator(device=dev).manual_seed(100 + c)
        copies.append(ops.pack_weight(torch.randn((GEMV_N, GEMV_K), generator=g, device=dev) * 0.02))
    ym = torch.empty((1, GEMV_N), dtype=torch.bfloat16, device=dev)
    for i in range(12):
        ops.gemv(rng_x, copies[i % 6], GEMV_N, out=ym)
    torch.cuda.synchronize()
    # a ~10 us kernel launched from Python one call at a time measures the launch path, not the kernel: capture the
    # rotation over the copies in a HIP graph and time its replays (no memset nodes; the GEMV writes every output)
    per_graph = 60
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for i in range(per_graph):
                ops.gemv(rng_x, copies[i % 6], GEMV_N, out=ym)
    torch.cuda.current_stream().wait_stream(side)
    graph.replay()
    torch.cuda.synchronize()
    ref = ops.gemv(rng_x, copies[(per_graph - 1) % 6], GEMV_N)
    assert torch.equal(ref, ym), "graph replay of the GEMV differs from the eager result"
    settle(graph.replay)
    reps = 4
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us_gemv = e0.elapsed_time(e1) * 1e3 / (reps * per_graph)
    gemv_bytes = GEMV_K * GEMV_N * 9 / 8 + GEMV_K * 2 + GEMV_N * 2
    return {
        "host": host, "p_up": inp["up"].cpu().numpy(), "p_down": inp["down"].cpu().numpy(),
        "wall_s": wall, "ms_step": ms_step, "ms_step_eager": ms_step_eager,
        "ms_q": ms_q, "us_q_alone": us_q_alone, "us_q_packed": us_q_packed, "ms_up": ms_up, "ms_down": ms_down,
        "us_gemv": us_gemv,
        "gemv_gbps": gemv_bytes / (us_gemv * 1e-6) / 1e9, "gemv_bytes": gemv_bytes,
        "v9a": v9a,
        "v9_ops": v9_oplist_bench(dev),
        "ln": ln_bench(dev),
        "qkv": qkv_bench(dev),
        "attn": attn_bench(dev),
        "configs": None if no_configs else configs_bench(dev),
    }


def v9a_bench(inp, xq, h_step, per_graph=10, reps=3):
    """The up GEMM with A as the reference passes it, the a_layout bfp16 stream (V9), beside the same GEMM on the bf16
    A of the quantize pass, both as HIP-graph replays: the library decodes the stream into a bf16 copy in the
    workspace (one HBM-bound launch), then runs the bf16-A kernels. Both must give the step's H bit for bit."""
    import torch

    from rlbfp import ops

    xa, _ = ops.quantize(inp["x"], order="a_layout")
    h = torch.empty_like(h_step)
    out = {}
    for name, a, kw in (("bf16", xq, {}), ("v9a_staged", xa, {"M": M, "a_fmt": "packed_a_layout"})):
        def call(i):
            ops.gemm(a, inp["up"], 2 * FF, K, act="swiglu", quantize_out=True, out=h, **kw)
        us = graph_us(call, 3, per_graph, reps)
        assert torch.equal(h, h_step), f"up GEMM with {name} A differs from the step's"
        out[name + "_us"] = round(us, 2)
    return out


def ln_bench(dev, sets=4, per_graph=40, reps=4):
    """The residual + LayerNorm + modulate pass that produces the up GEMM's A (M x hidden = 4352 x 3072), in two
    configurations, each as HIP-graph replays of `per_graph` launches rotating over `sets` input sets (4 x 53 MB of
    inputs plus the outputs exceed the 256 MB MALL):
      native:  bf16 x, bf16 branch (a GEMM output) -> x' bf16 and A as bf16 (the next GEMM's operand): 8 B per value
      packed:  bf16 x, bfp16 branch (row blocks) -> x' bf16 and A as bfp16 (the reference's formats): 6.25 B per value
    Algorithmic bytes are those reads and writes once each; the 2 x 2D bf16 parameters are not counted."""
    import ctypes

    import torch

    from rlbfp import _lib as L
    from rlbfp import ops

    g = torch.Generator(device=dev).manual_seed(7)
    xs = [torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16) for _ in range(sets)]
    brs = [torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16) for _ in range(sets)]
    brp = [ops.quantize(b)[0] for b in brs]
    params = torch.cat([torch.tanh(torch.randn((2, K), generator=g, device=dev)),
                        1 + 0.3 * torch.randn((2, K), generator=g, device=dev)], 1).to(torch.bfloat16).contiguous()
    xo = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    a_d = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    a_p = torch.empty(M * K // 8 * 9, dtype=torch.uint8, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)

    def call(i, packed):
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        br, fmt = (brp[i % sets], L.RL_BRANCH_PACKED) if packed else (brs[i % sets], L.RL_BRANCH_BF16)
        L.check(L.lib().rl_ln_modulate(P(xs[i % sets]), K, P(br), fmt, K, P(params), 0, L.RL_NORM_LAYER, P(xo), K,
                                       P(a_p if packed else None), L.RL_ORDER_ROWBLOCK, P(None if packed else a_d),
                                       K, M, K, st))

    out = {"shape": [M, K], "norm": "layer", "sets": sets}
    for name, packed, bpv in (("native", False, 8.0), ("packed", True, 2 + 9 / 8 + 2 + 9 / 8)):
        us = graph_us(lambda i: call(i, packed), 2 * sets, per_graph, reps)
        gbps = M * K * bpv / (us * 1e-6) / 1e9
        out[name] = {"us": round(us, 2), "bytes": int(M * K * bpv), "gbps": round(gbps, 1),
                     "frac_hbm": round(gbps / PEAK_HBM_GBPS, 4)}
    return out


def graph_us(call, warm, per_graph, reps):
    """Microseconds per call(i): `warm` eager calls, then `per_graph` calls captured in one HIP graph (i = 0, 1, ...)
    and replayed `reps` times between two events."""
    import torch

    for i in range(warm):
        call(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for i in range(per_graph):
                call(i)
    torch.cuda.current_stream().wait_stream(side)
    graph.replay()
    torch.cuda.synchronize()
    settle(graph.replay)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * per_graph)


def settle(run, seconds=None):
    """Runs `run()` untimed for SETTLE_S seconds (a synchronisation every tenth call) right before a timed region.
    On an MI355X that was idle, even for a few ms of host work between two timed regions, power management takes some
    tens of ms of load to settle the clock: the first ~50 FFN steps from cold run the up GEMM at ~537 us, then
    518-522 us for seconds on the same box, and a step graph replayed right after host work measured 8% slower than
    the settled eager steps before it."""
    import torch

    t = time.perf_counter()
    n = 0
    while time.perf_counter() - t < (SETTLE_S if seconds is None else seconds):
        run()
        n += 1
        if n % 10 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def attn_bench(dev, heads=24, per_graph=10, reps=3):
    """Attention over the benchmark's M (4352 tokens, 24 heads of 128 = hidden 3072): Q (score scale folded in), K,
    V^T bf16 in, bf16 O out (4 * heads * M^2 * 128 FLOP); HIP-graph replays. `us` is the default launch (the last
    partial round split along the keys, with its combine launch); `whole_tasks_us` runs every task whole. torch's bf16
    scaled_dot_product_attention of the same shape is timed beside it as a reference point."""
    import torch

    from rlbfp import ops

    g = torch.Generator(device=dev).manual_seed(13)
    q = (torch.randn((heads, M, 128), generator=g, device=dev) * 0.1275).to(torch.bfloat16)
    k = torch.randn((heads, M, 128), generator=g, device=dev).to(torch.bfloat16)
    vt = torch.randn((heads, 128, M), generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty((M, heads * 128), dtype=torch.bfloat16, device=dev)
    # 20 warm-up calls each: the clocks take a few milliseconds of this load to settle
    us = graph_us(lambda i: ops.attention(q, k, vt, out=out), 20, per_graph, reps)
    us_whole = graph_us(lambda i: ops.attention(q, k, vt, out=out, split=False), 20, per_graph, reps)
    flops = 4.0 * heads * M * M * 128
    qs, ks, vs = q.unsqueeze(0), k.unsqueeze(0), vt.transpose(1, 2).contiguous().unsqueeze(0)
    f = torch.nn.functional.scaled_dot_product_attention
    for _ in range(3):
        f(qs, ks, vs)
    settle(lambda: f(qs, ks, vs))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(per_graph):
        f(qs, ks, vs)
    e1.record()
    torch.cuda.synchronize()
    us_t = e0.elapsed_time(e1) * 1e3 / per_graph
    tf = flops / (us * 1e-6) / 1e12
    return {"shape": [heads, M, M, 128], "us": round(us, 2), "tflops": round(tf, 1),
            "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4), "whole_tasks_us": round(us_whole, 2),
            "torch_sdpa_us": round(us_t, 2),
            "torch_sdpa_tflops": round(flops / (us_t * 1e-6) / 1e12, 1)}


def configs_bench(dev, per_graph=10, reps=3):
    """The other reference configurations' GEMMs, timed like the FFN pair (HIP-graph replays, A already quantized
    along K): config 1 (4096 x 3072 x 3072, no epilogue), config 2 (QKV 4352 x 3072 x 9216 with bias and 1% outlier
    channels), config 4 (text-encoder MLP, M = 512: up K = 4096, N = 2 x 12288 SwiGLU re-quantized, down K = 12288,
    N = 4096) and config 5 (one DiT block's GEMMs for the image (M = 4096) and text (M = 256) streams with separate
    weights: QKV, out-projection, SwiGLU up and down, each op one grouped launch of both streams). Synthetic data of
    those shapes; weights ~N(0, 0.02) packed on the GPU. FLOP = 2 M N K, N counting both SwiGLU halves."""
    import torch

    from rlbfp import ops

    g = torch.Generator(device=dev).manual_seed(0)

    def act(M, K, outliers=0.0):
        a = torch.randn((M, K), generator=g, device=dev)
        if outliers:
            idx = torch.randperm(K, generator=g, device=dev)[: round(outliers * K)]
            a[:, idx] *= 20
        return ops.quantize(a.to(torch.bfloat16), deq=True)[1]

    def weight(N, K):
        return ops.pack_weight(torch.randn((N, K), generator=g, device=dev) * 0.02)

    def up_weight(F_, K):
        return ops.pack_weight(ops.interleave_up(torch.randn((F_, K), generator=g, device=dev) * 0.02,
                                                 torch.randn((F_, K), generator=g, device=dev) * 0.02))

    def line(us, flop):
        tf = flop / (us * 1e-6) / 1e12
        return {"us": round(us, 2), "tflops": round(tf, 1), "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4),
                "gflop": round(flop / 1e9, 2)}

    out = {}
    a1, w1 = act(4096, 3072), weight(3072, 3072)
    c1 = torch.empty((4096, 3072), dtype=torch.bfloat16, device=dev)
    out["cfg1"] = line(graph_us(lambda i: ops.gemm(a1, w1, 3072, 3072, out=c1), 5, per_graph, reps),
                       2.0 * 4096 * 3072 * 3072)
    a2, w2 = act(4352, 3072, outliers=0.01), weight(9216, 3072)
    b2 = torch.randn(9216, generator=g, device=dev) * 0.02
    c2 = torch.empty((4352, 9216), dtype=torch.bfloat16, device=dev)
    out["cfg2"] = line(graph_us(lambda i: ops.gemm(a2, w2, 9216, 3072, bias=b2, out=c2), 5, per_graph, reps),
                       2.0 * 4352 * 3072 * 9216)
    x4 = act(512, 4096)
    up4, dn4 = up_weight(12288, 4096), weight(4096, 12288)
    h4 = torch.empty((512, 12288), dtype=torch.bfloat16, device=dev)
    y4 = torch.empty((512, 4096), dtype=torch.bfloat16, device=dev)

    def cfg4(i):
        ops.gemm(x4, up4, 2 * 12288, 4096, act="swiglu", quantize_out=True, out=h4)
        ops.gemm(h4, dn4, 4096, 12288, out=y4)

    out["cfg4"] = line(graph_us(cfg4, 5, per_graph, reps), 2.0 * 512 * 4096 * 24576 + 2.0 * 512 * 12288 * 4096)
    # config 5: per stream the four ops' inputs and weights (the ops are not chained here: timing only)
    K = 3072
    ops5 = []
    for N, Kop, kind in ((9216, K, None), (K, K, None), (2 * 12288, K, "swiglu"), (K, 12288, None)):
        specs = []
        for M in (4096, 256):
            a = act(M, Kop)
            w = up_weight(12288, Kop) if kind == "swiglu" else weight(N, Kop)
            specs.append(ops.GemmSpec(a, w, N, Kop, act=kind, quantize_out=kind == "swiglu"))
        ops5.append(specs)

    def cfg5(i):
        for specs in ops5:
            ops.gemm_grouped(specs)

    out["cfg5"] = line(graph_us(cfg5, 5, per_graph, reps), 2.0 * 4352 * K * (9216 + K + 2 * 12288 + 12288))
    return out


def v9_oplist_bench(dev, per_graph=5, reps=3):
    """The DiT block's GEMMs in the order CachedStep.blocks issues them (redline/forward.py:240-254: qkv, o,
    up_swiglu, down), through the NPU.run mirror on the reference's own buffers: A as the V9 a_layout stream, C as the
    ATB bfp16 stream, H in the down GEMM's A layout (each GEMM's epilogue writes the packed blocks itself; a V9 A is
    staged as bf16 in a workspace first). Beside them: the same GEMMs on the native operands (bf16 A and C), and
    bf16 A with the V9 C (the cost of the packed output alone). Hidden 3072, FF 12288, M = 4608: the 4352 tokens of
    the benchmark padded to a multiple of 512, as the reference's ATB artifacts need (its cfg2 note). HIP-graph
    replays; every V9 output is checked against the quantize pass over the native output."""
    import torch

    from rlbfp import forward as FW
    from rlbfp import ops

    Mp, H, Fh = 4608, K, FF
    g = torch.Generator(device=dev).manual_seed(21)
    w = {"qkv": ops.pack_weight(torch.randn((3 * H, H), generator=g, device=dev) * 0.02),
         "o": ops.pack_weight(torch.randn((H, H), generator=g, device=dev) * 0.02),
         "up": ops.pack_weight(ops.interleave_up(torch.randn((Fh, H), generator=g, device=dev) * 0.02,
                                                 torch.randn((Fh, H), generator=g, device=dev) * 0.02).contiguous()),
         "down": ops.pack_weight(torch.randn((H, Fh), generator=g, device=dev) * 0.02)}
    # the V9 A streams encode the raw activations; the native bf16 A holds their values
    x_raw = torch.randn((Mp, H), generator=g, device=dev).to(torch.bfloat16)
    o_raw = torch.randn((Mp, H), generator=g, device=dev).to(torch.bfloat16)
    x, o = ops.quantize(x_raw, deq=True)[1], ops.quantize(o_raw, deq=True)[1]
    a9, o9 = ops.quantize(x_raw, order="a_layout")[0], ops.quantize(o_raw, order="a_layout")[0]
    npu = FW.NPU(kn={"qkv": (H, 3 * H), "o": (H, H), "up": (H, 2 * Fh), "down": (Fh, H)})
    c_qkv9, c9, h9 = FW.v9(Mp * 3 * H, dev), FW.v9(Mp * H, dev), FW.v9(Mp * Fh, dev)
    c_qkv, c, h = (torch.empty((Mp, n), dtype=torch.bfloat16, device=dev) for n in (3 * H, H, Fh))
    h_a9 = torch.empty_like(h9)
    # (op, V9 call, native call, V9 C from the native bf16 A, check: V9 output against the native one)
    ops_ = {
        "qkv": (lambda: npu._gemm("qkv", "atb3d2-qkv", a9, w["qkv"], c_qkv9),
                lambda: ops.gemm(x, w["qkv"], 3 * H, H, out=c_qkv),
                lambda: ops.gemm(x, w["qkv"], 3 * H, H, packed_out=c_qkv9),
                lambda: torch.equal(c_qkv9, ops.quantize(c_qkv, order="c_atb")[0])),
        "o": (lambda: npu._gemm("o", "atb3d2-4096", o9, w["o"], c9),
              lambda: ops.gemm(o, w["o"], H, H, out=c),
              lambda: ops.gemm(o, w["o"], H, H, packed_out=c9),
              lambda: torch.equal(c9, ops.quantize(c, order="c_atb")[0])),
        # H as the reference pushes it: the bfp16 blocks of the bf16 SwiGLU output; the native H (re-quantized in
        # the epilogue) holds their values
        "up_swiglu": (lambda: npu._gemm("up_swiglu", "atb3sw2-m4608", a9, w["up"], h9),
                      lambda: ops.gemm(x, w["up"], 2 * Fh, H, act="swiglu", quantize_out=True, out=h),
                      lambda: ops.gemm(x, w["up"], 2 * Fh, H, act="swiglu", packed_out=h9, packed_order="a_layout"),
                      lambda: torch.equal(ops.dequantize(h9, Mp, Fh, order="a_layout", dtype=torch.bfloat16), h)),
        "down": (lambda: npu._gemm("down", "atb3d2-down", h_a9, w["down"], c9),
                 lambda: ops.gemm(h, w["down"], H, Fh, out=c),
                 lambda: ops.gemm(h, w["down"], H, Fh, packed_out=c9),
                 lambda: torch.equal(c9, ops.quantize(c, order="c_atb")[0])),
    }
    out = {"M": Mp, "hidden": H, "ff": Fh}
    tot = {"v9": 0.0, "native": 0.0, "v9c_bf16a": 0.0}
    for name, (v9call, native, v9c, check) in ops_.items():
        if name == "down":
            h_a9.copy_(h9)  # the down GEMM's V9 A: H as up_swiglu pushed it
        us_n = graph_us(lambda i: native(), 2, per_graph, reps)
        us_c = graph_us(lambda i: v9c(), 2, per_graph, reps)
        assert check(), f"{name}: the V9 C from bf16 A differs from the quantize pass over the bf16 C"
        us_v = graph_us(lambda i: v9call(), 2, per_graph, reps)
        assert check(), f"{name}: the V9 op differs from the quantize pass over the native output"
        out[name] = {"v9_us": round(us_v, 2), "native_us": round(us_n, 2), "v9c_bf16a_us": round(us_c, 2),
                     "v9c_vs_bf16c": round(us_c / us_n, 4)}
        tot["v9"] += us_v
        tot["native"] += us_n
        tot["v9c_bf16a"] += us_c
    out["total"] = {k + "_us": round(v, 2) for k, v in tot.items()}
    out["total"]["v9_vs_native"] = round(tot["v9"] / tot["native"], 4)
    return out


def qkv_bench(dev, heads=24, sets=3, per_graph=30, reps=4):
    """The QKV post pass on the QKV GEMM output of the benchmark's M (4352 tokens x 3 x 24 heads of 128 = hidden 3072):
    bf16 C in, the attention Q / K / V tiles (bfp16) out; HIP-graph replays rotating over `sets` copies of C
    (3 x 80 MB with the outputs exceed the 256 MB MALL). Algorithmic bytes: C read once (2 B per value) and the tiles
    written once (9/8 B per value); the cos/sin rows (1.1 MB) and weights are not counted."""
    import ctypes

    import torch

    from rlbfp import _lib as L

    g = torch.Generator(device=dev).manual_seed(11)
    n = 3 * heads * 128
    Cs = [torch.randn((M, n), generator=g, device=dev).to(torch.bfloat16) for _ in range(sets)]
    ang = torch.rand((M, 64), generator=g, device=dev) * 6.2832
    cos, sin = torch.cos(ang).to(torch.bfloat16), torch.sin(ang).to(torch.bfloat16)
    wq = (1 + 0.1 * torch.randn(128, generator=g, device=dev)).to(torch.bfloat16)
    wk = (1 + 0.1 * torch.randn(128, generator=g, device=dev)).to(torch.bfloat16)
    qt = torch.empty((heads, M // 64, 9216), dtype=torch.uint8, device=dev)
    kvt = torch.empty((heads, M // 64, 2, 9216), dtype=torch.uint8, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)

    def call(i):
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        L.check(L.lib().rl_qkv_post(P(Cs[i % sets]), n, M, heads, P(cos), P(sin), P(wq), P(wk), P(qt), P(kvt),
                                    P(None), P(None), P(None), st))

    us = graph_us(call, 2 * sets, per_graph, reps)
    nbytes = M * n * (2 + 9 / 8)
    gbps = nbytes / (us * 1e-6) / 1e9
    return {"shape": [M, heads, 128], "us": round(us, 2), "bytes": int(nbytes), "gbps": round(gbps, 1),
            "frac_hbm": round(gbps / PEAK_HBM_GBPS, 4), "sets": sets}


def cpu_baseline(host, p_up, p_down, rows=M, runs=3):
    """The oracle's numpy restatement of the reference CPU path on the first `rows` rows of the same workload:
    to_bfp16 of the activations, from_bfp16 of the activations and of the pre-packed weights (the same bytes the GPU
    uses; packing is an offline cost and is not timed), float32 BLAS matmul, SwiGLU, bf16 rounding, re-quantize,
    down matmul, gate * acc + residual, bf16 rounding."""
    import numpy as np

    from oracle import bfp16 as F

    x, _wg, _wp, _wd, res, gate = host
    x = F.bf16_round(x[:rows])
    res = F.bf16_round(res[:rows])

    def one():
        t0 = time.perf_counter()
        xq = F.quantize_rows(x)
        acc = xq @ F.decode_b(p_up, K, 2 * FF)
        gt = acc.reshape(rows, -1, 2, 64)
        hv = gt[:, :, 0] / (1 + np.exp(-gt[:, :, 0])) * gt[:, :, 1]
        hq = F.quantize_rows(F.bf16_round(hv.reshape(rows, FF).astype(np.float32)))
        out = F.bf16_round((res + gate * (hq @ F.decode_b(p_down, FF, K))).astype(np.float32))
        assert out.shape == (rows, K)
        return time.perf_counter() - t0

    # the BLAS pool is set to the host cores this process may use: the CPU share the environment states
    # (OMP_NUM_THREADS), else the affinity mask
    visible = len(os.sched_getaffinity(0))
    cores = min(visible, int(os.environ.get("OMP_NUM_THREADS") or visible))
    blas, blas_threads = "unknown", None
    try:
        from threadpoolctl import threadpool_info, threadpool_limits
        limiter = threadpool_limits(limits=cores, user_api="blas")
        pools = [i for i in threadpool_info() if i.get("user_api") == "blas"]
        if pools:
            blas = f"{pools[0].get('internal_api')} {pools[0].get('version')} ({os.path.basename(pools[0].get('filepath', ''))})"
            blas_threads = pools[0].get("num_threads")
    except Exception:
        limiter = None
    one()                                        # warm-up
    dt = sorted(one() for _ in range(runs))[runs // 2]
    if limiter is not None:
        limiter.restore_original_limits()
    flops = 2.0 * rows * K * 2 * FF + 2.0 * rows * FF * K
    return {"value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": blas_threads or cores, "kind": "port",
            "blas": blas, "blas_threads": blas_threads, "cpu_model": _cpu_model(), "cpus_visible": visible,
            "sample": f"the full FFN pair step ({rows} rows, weights decoded from the packed bytes each run), median "
                      f"of {runs} runs after a warm-up, {dt:.2f} s per step; numpy float32 BLAS matmuls on "
                      f"{blas_threads or cores} threads"}


def _cpu_model():
    """The host CPU's model name from /proc/cpuinfo (None if unreadable)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def copy_probe(mb, reps=10):
    """D2D copies of `mb` MB: a kernel whose HBM bytes are known (mb MB read + mb MB written per launch)."""
    import torch
    n = mb * 2**20
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    print(json.dumps({"copy_probe_mb": mb, "bytes_read": n, "bytes_written": n, "us": round(us, 2),
                      "gbps_rw": round(2 * n / us / 1e3, 1)}), flush=True)


def _smi_sample():
    """One `amd-smi metric -p -c` reading of GPU 0: (socket power W, mean graphics clock MHz over the XCDs), or
    (None, None) when the tool is absent or prints something else."""
    import re
    import subprocess
    try:
        txt = subprocess.run(["amd-smi", "metric", "-p", "-c", "-g", "0"], capture_output=True, text=True,
                             timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        return None, None
    pw = re.search(r"SOCKET_POWER:\s*([0-9.]+)\s*W", txt)
    clks = [float(c) for c in re.findall(r"GFX_\d+:\s*\n\s*CLK:\s*([0-9.]+)\s*MHz", txt)]
    return (float(pw.group(1)) if pw else None), (sum(clks) / len(clks) if clks else None)


def sustain(seconds):
    """Runs the up GEMM back to back for `seconds`, then torch's bf16 linear of the same shape (hipBLASLt, no decode,
    no epilogue) for as long, while a thread reads socket power and graphics clock with amd-smi. One JSON line per
    kernel: time per call and the power/clock readings taken while it ran."""
    import threading

    import torch

    from rlbfp import ops

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    w_up = torch.randn((2 * FF, K), generator=g, device=dev) * 0.02
    packed = ops.pack_weight(ops.interleave_up(w_up[:FF], w_up[FF:]))
    a_q = ops.quantize(a, deq=True)[1]
    h = torch.empty((M, FF), dtype=torch.bfloat16, device=dev)
    w_bf = w_up.to(torch.bfloat16)
    runs = {"up GEMM + SwiGLU (bfp16 weights)":
            lambda: ops.gemm(a_q, packed, 2 * FF, K, act="swiglu", quantize_out=True, out=h),
            "torch bf16 linear, same shape": lambda: torch.nn.functional.linear(a_q, w_bf)}
    for name, fn in runs.items():
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        samples, stop = [], threading.Event()

        def sampler():
            time.sleep(min(1.0, seconds / 4))  # past the first launches
            while not stop.is_set():
                samples.append(_smi_sample())
                time.sleep(0.25)

        th = threading.Thread(target=sampler)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n, t0 = 0, time.time()
        th.start()
        e0.record()
        while time.time() - t0 < seconds:
            for _ in range(100):
                fn()
            n += 100
            torch.cuda.synchronize()
        e1.record()
        torch.cuda.synchronize()
        stop.set()
        th.join()
        pw = [p for p, _ in samples if p is not None]
        ck = [c for _, c in samples if c is not None]
        print(json.dumps({"sustain": name, "shape": [M, K, 2 * FF], "calls": n,
                          "us_per_call": round(e0.elapsed_time(e1) * 1e3 / n, 2),
                          "tflops": round(flops_up() * n / (e0.elapsed_time(e1) * 1e-3) / 1e12, 1),
                          "socket_power_w": pw, "gfx_clock_mhz": [round(c) for c in ck]}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the other configurations' GEMM timings")
    ap.add_argument("--sustain", type=float, default=0, metavar="SECONDS",
                    help="only run the up GEMM, then torch's bf16 linear of the same shape, back to back for SECONDS "
                         "each while amd-smi reads socket power and graphics clock; print one line per kernel and exit")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MB",
                    help="only run device-to-device copies of MB megabytes (calibrates rocprofv3 FETCH_SIZE and "
                         "WRITE_SIZE against a transfer of known size), print their bandwidth and exit")
    args = ap.parse_args()
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.sustain:
        sustain(args.sustain)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the path would shard by weight "
              "columns across GPUs, which is not built)", file=sys.stderr)
        sys.exit(2)
    r = gpu_bench(args.steps, args.warmup, args.no_configs)
    ms_step = r["ms_step"]
    step_flops = flops_up() + flops_down()
    up_tflops = flops_up() / (r["ms_up"] * 1e-3) / 1e12
    line = {
        "metric": "bfp16-weight GEMM TFLOP/s and % bf16 MFMA peak at DiT FFN shape; GEMV GB/s",
        "value": round(step_flops / (ms_step * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "settle_s": SETTLE_S,
        "ms_per_step": round(ms_step, 4),
        "ms_per_step_eager": round(r["ms_step_eager"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "dit_ffn_pair", "M": M, "hidden": K, "ff": FF,
                   "step": "quantize x + up GEMM (SwiGLU, re-quantized H) + down GEMM (gate*acc + residual)",
                   "weights": "bfp16ebs8 ~N(0,0.02)", "activations": "bf16 ~N(0,1)", "seed": 0},
        "roofline": {"bound": "mfma", "achieved": round(up_tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(up_tflops / PEAK_BF16_TFLOPS, 4), "traffic": UP_GEMM_TRAFFIC_BYTES,
                     "kernel": "up GEMM 4352x3072x24576 + SwiGLU: gemm4w_kernel<1,8,false,true> rows 0..4095 + gemm4w_kernel<1,4,false,true> rows 4096..4351 (register epilogue)",
                     "us": round(r["ms_up"] * 1e3, 2)},
        "kernels": {
            # the kernel alone (graph replays); algorithmic bytes: bf16 read + packed written (the pass also writes
            # the decoded bf16 copy the GEMM reads, not counted)
            "quantize_us": round(r["us_q_alone"], 2),
            "quantize_gbps": round(M * K * (2 + 9 / 8) / (r["us_q_alone"] * 1e-6) / 1e9, 1),
            "quantize_packed_only_us": round(r["us_q_packed"], 2),
            "quantize_packed_only_frac_hbm": round(M * K * (2 + 9 / 8) / (r["us_q_packed"] * 1e-6) / 1e9
                                                   / PEAK_HBM_GBPS, 4),
            "quantize_in_step_us": round(r["ms_q"] * 1e3, 2),
            "up_us": round(r["ms_up"] * 1e3, 2), "up_tflops": round(up_tflops, 2),
            "down_us": round(r["ms_down"] * 1e3, 2),
            "down_tflops": round(flops_down() / (r["ms_down"] * 1e-3) / 1e12, 2),
            # the up GEMM in graph replays, fed bf16 A, then the reference's a_layout A stream (same H bits)
            "up_graph_us": r["v9a"]["bf16_us"],
            "up_v9a_staged_us": r["v9a"]["v9a_staged_us"],
            "up_v9a_vs_bf16": round(r["v9a"]["v9a_staged_us"] / r["v9a"]["bf16_us"], 4),
        },
        "gemv": {"shape": [1, GEMV_K, GEMV_N], "us": round(r["us_gemv"], 2), "gbps": round(r["gemv_gbps"], 1),
                 "frac_hbm": round(r["gemv_gbps"] / PEAK_HBM_GBPS, 4), "bytes": int(r["gemv_bytes"]),
                 "copies": 6},
        "v9_oplist": r["v9_ops"],
        "ln_modulate": r["ln"],
        "qkv_post": r["qkv"],
        "attention": r["attn"],
        "configs": r["configs"],
    }
    line["cpu_baseline"] = None if args.no_cpu else cpu_baseline(r["host"], r["p_up"], r["p_down"])
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
