"""Benchmark of the fused Qwen3 layer operators on one MI355X.

Headline workload: prefill n = 2811 at Qwen3-1.7B shape
(H = 2048, 16 q heads, 8 kv heads, head_dim 128, I = 6144), all 28 layers, each
layer with its own seeded buffers and weights. One step = for every layer:
  residual add + RMSNorm      [n, H]              (rpg_op_add_rms_norm)
  q/k norm + RoPE + fp16 KV   [n, 16|8, 128]      (rpg_op_qk_norm_rope_kv)
  SwiGLU                      [n, I]              (rpg_op_silu_mul_inplace)
`value` = algorithmic bytes of the step / step time (GB/s); per-kernel averages
come from HIP events attached to every kernel dispatch of the timed steps
(librpg_ops launch profiling, hipExtLaunchKernel). The 28 layers'
buffers total ~9 GB, far above the 256 MB Infinity Cache, so every launch reads
from HBM. Also reported: decode n = 1 (us per layer, eager and HIP graph), the
Q4_K / Q6_K embedding gather at n = 2811, a streaming-copy ceiling, same-size
ceilings (a copy moving each op's bytes, a fill writing its output bytes) timed
the same way as the ops, and the CPU oracle on the host cores as a baseline.

python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

METRIC = "fused layer-op HBM GB/s (% of MI355X peak) at n=1 decode and n=2811 prefill"
PEAK_GBPS = 8000.0

H, HQ, HKV, D, INTER, LAYERS = 2048, 16, 8, 128, 6144, 28
MAX_SEQ, EPS, THETA = 4096, 1e-6, 1e6
N_PREFILL = 2811
VOCAB = 151936
CALIB_BYTES = 256 << 20


def bytes_add_rms(n, h=H):
    return 16 * n * h + 4 * h


def bytes_qk(n, hq=HQ, hkv=HKV, d=D):
    return n * (8 * hq * d + 12 * hkv * d + 4 * d) + 8 * d


def bytes_swiglu(n, inter=INTER):
    return 12 * n * inter


def bytes_gather(n, bb, h=H):
    return n * (4 + (h // 256) * bb + 4 * h)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


QWEN3_1_7B = dict(hidden=H, n_heads=HQ, n_kv_heads=HKV, inter=INTER, layers=LAYERS)
QWEN3_4B = dict(hidden=2560, n_heads=32, n_kv_heads=8, inter=9728, layers=36)


_SPIN = {"cycles_per_us": None}


def hold_launches(torch, n_launches, host_us_per_launch=40.0):
    """Queue a bounded spin kernel (torch.cuda._sleep) on the stream the library
    launches on, long enough for the host to enqueue the next `n_launches`
    profiled launches behind it; the GPU then runs those kernels back to back, as
    it does in the timed region and in the engine's forward pass. Launched one by
    one from Python, each kernel would instead start on a GPU that has just gone
    idle, which adds up to ~0.5 us to a 5 us kernel (measured on MI355X: the Q4_K
    gather 4.9-5.5 us after launch gaps, 4.5-4.6 us queued). The spin only counts
    clock cycles; it waits on nothing."""
    if _SPIN["cycles_per_us"] is None:
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1 << 20)
        e0.record()
        torch.cuda._sleep(4 << 20)
        e1.record()
        torch.cuda.synchronize()
        _SPIN["cycles_per_us"] = (4 << 20) / max(e0.elapsed_time(e1) * 1e3, 1.0)
    torch.cuda._sleep(int((100.0 + host_us_per_launch * n_launches) * _SPIN["cycles_per_us"]))


def back_to_back_us(torch, ops, launch, n=100, trials=3):
    """Per-launch GPU time of `launch(i)` run n times back to back: the n launches are
    captured into one HIP graph (on the library's stream), and the graph's replays
    are timed with stream events (best of `trials`). This is the cost of one more
    launch in a graph-replayed decode loop. Dispatch-attached events put a floor of
    ~4 us under any kernel, and launches issued one by one from Python are bound by
    the host (~3.3 us each), so neither shows the difference between two short
    kernels. `launch` must not allocate or stage anything (it is captured)."""
    for i in range(8):
        launch(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        with ops.ScopedEngineStream(st):
            g.capture_begin()
            for i in range(n):
                launch(i)
            g.capture_end()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(trials):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        best = min(best, a.elapsed_time(b) * 1e3 / n)
    del g
    return best


def launch_floor_us(torch, ops):
    """The same for a one-workgroup kernel (a 4 KiB fill): what any launch in a graph costs."""
    buf = torch.empty(1024, dtype=torch.float32, device="cuda")
    return back_to_back_us(torch, ops, lambda i: ops.GpuStreamFill(buf, 4096, 0), n=200)


def batch_us(torch, launch, count, trials=5, start=0):
    """Per-launch GPU time of `count` launches run back to back, median over
    `trials` batches: the reference's BenchItem method (tools/matmul_bench.cu:114-132:
    launches issued back to back, one clock read around the batch), with stream
    events in place of the host clock. Each batch queues behind a bounded spin
    kernel (hold_launches) and the start event follows it, so the kernels run
    with no idle gap and no per-dispatch event packets between them, as the
    product runs them. launch(i) receives a running index (continued across
    batches from `start`) so callers can rotate through distinct buffers.
    Returns (median us per launch, [us per launch of each batch])."""
    import statistics

    samples = []
    i = start
    for _ in range(trials):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        hold_launches(torch, count)
        e0.record()
        for _ in range(count):
            launch(i)
            i += 1
        e1.record()
        torch.cuda.synchronize()
        samples.append(e0.elapsed_time(e1) * 1e3 / count)
    return statistics.median(samples), samples


class Layer:
    """One layer's device buffers (all distinct per layer)."""

    def __init__(self, torch, n, gen, shape=QWEN3_1_7B):
        f32 = dict(dtype=torch.float32, device="cuda")
        hid, hq, hkv, inter = shape["hidden"], shape["n_heads"], shape["n_kv_heads"], shape["inter"]
        self.n, self.hid, self.hq, self.hkv, self.inter = n, hid, hq, hkv, inter
        self.x = torch.randn((n, hid), generator=gen, **f32)
        self.d = torch.randn((n, hid), generator=gen, **f32)
        self.h = torch.empty((n, hid), **f32)
        self.w = 1.0 + 0.1 * torch.randn(hid, generator=gen, **f32)
        self.q = torch.randn((n, hq, D), generator=gen, **f32)
        self.k = torch.randn((n, hkv, D), generator=gen, **f32)
        self.v = torch.randn((n, hkv, D), generator=gen, **f32)
        self.qn = 1.0 + 0.1 * torch.randn(D, generator=gen, **f32)
        self.kn = 1.0 + 0.1 * torch.randn(D, generator=gen, **f32)
        self.kc = torch.zeros(hkv * MAX_SEQ * D, dtype=torch.int16, device="cuda")
        self.vc = torch.zeros_like(self.kc)
        self.gate = torch.randn((n, inter), generator=gen, **f32)
        self.up = torch.randn((n, inter), generator=gen, **f32)


def run_layer(ops, L, n, tab, pos0):
    ops.GpuAddRmsNorm(L.x, L.d, L.w, n, L.hid, EPS, L.h)
    ops.GpuQkNormRopeKv(L.q, L.k, L.v, L.qn, L.kn, L.hq, L.hkv, D, tab, MAX_SEQ, pos0, n, EPS, L.kc, L.vc, MAX_SEQ)
    ops.GpuSiluMulInPlace(L.gate, L.up, n * L.inter)


def op_launchers(ops, n, tab, pos0=0):
    """One launch of each layer op on a layer's buffers, keyed by op name."""
    return {
        "add_rms_norm": lambda L: ops.GpuAddRmsNorm(L.x, L.d, L.w, n, L.hid, EPS, L.h),
        "qk_norm_rope_kv": lambda L: ops.GpuQkNormRopeKv(L.q, L.k, L.v, L.qn, L.kn, L.hq, L.hkv, D, tab, MAX_SEQ,
                                                         pos0, n, EPS, L.kc, L.vc, MAX_SEQ),
        "swiglu": lambda L: ops.GpuSiluMulInPlace(L.gate, L.up, n * L.inter),
    }


def op_batches(torch, ops, layers, tab, n, trials=5):
    """Each op timed alone the way the product runs it: one launch per layer's
    buffers (28 or 36 distinct buffer sets, far beyond the Infinity Cache), all
    back to back, one event pair around the batch, median of `trials` batches."""
    out = {}
    for name, fn in op_launchers(ops, n, tab).items():
        fn(layers[0])
        med, samples = batch_us(torch, lambda i, fn=fn: fn(layers[i % len(layers)]), len(layers), trials)
        out[name] = (med, samples)
    return out


def layer_bytes(n, shape):
    return (bytes_add_rms(n, shape["hidden"]) + bytes_qk(n, shape["n_heads"], shape["n_kv_heads"]) +
            bytes_swiglu(n, shape["inter"]))


OP_NAMES = ("add_rms_norm", "qk_norm_rope_kv", "swiglu")
# the kernels the n = 2811 prefill launches; add + RMSNorm runs persistent (AddRmsNormRowsKernel) when the rows
# are at least twice its grid of four workgroups per CU, else one workgroup per row
KERNEL_NAMES = {"add_rms_norm": ("AddRmsNormRowsKernel", "AddRmsNormRowBlockKernel"),
                "qk_norm_rope_kv": ("QkNormRopeKvKernel",), "swiglu": ("SiluMulKernel",)}


def launched_kernel(report, op):
    """The name under which `op`'s kernel appears in a launch-profile report."""
    for name in KERNEL_NAMES[op]:
        if name in report:
            return name
    raise KeyError(f"no kernel of {op} in the launch profile ({sorted(report)})")


def timed_prefill(torch, ops, layers, tab, n, steps, warmup):
    """K steps over all layers, bracketed by stream events, twice: once as the
    product runs (this pass gives ms_per_step and `value`), then again with
    dispatch-attached HIP events on every launch (ops.profile_*), which give each
    kernel's execution time; in that pass every step's launches are queued behind
    a spin kernel (hold_launches) so the kernels still run back to back.
    Returns (ms_per_step, summed kernel time per step of the profiled pass, per-kernel report)."""
    for _ in range(warmup):
        for L in layers:
            run_layer(ops, L, n, tab, 0)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()

    def timed():
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record(stream)
        for _ in range(steps):
            for L in layers:
                run_layer(ops, L, n, tab, 0)
        t1.record(stream)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / steps

    def profiled():
        # each step's launches queue behind a spin kernel, so the step's kernels run
        # back to back as in the timed pass
        ops.profile_start(steps * len(layers) * 3)
        for _ in range(steps):
            hold_launches(torch, len(layers) * 3)
            for L in layers:
                run_layer(ops, L, n, tab, 0)
        torch.cuda.synchronize()
        ops.profile_stop()
        report = ops.profile_report()
        return sum(k["total_us"] for k in report.values()) * 1e-3 / steps, report

    ms_plain = timed()
    ms_prof, report = profiled()
    return ms_plain, ms_prof, report


def measure_decode(torch, ops, tab, steps):
    """n = 1 decode at a random position: us per layer for the 3 fused ops, eager and as a HIP graph."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    layers = [Layer(torch, 1, gen) for _ in range(LAYERS)]
    pos = 2731
    for _ in range(5):
        for L in layers:
            run_layer(ops, L, 1, tab, pos)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        for L in layers:
            run_layer(ops, L, 1, tab, pos)
    torch.cuda.synchronize()
    eager_us = (time.perf_counter() - t0) * 1e6 / (steps * LAYERS)

    graph_us = None
    try:
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with ops.ScopedEngineStream(s):
                g.capture_begin()
                for L in layers:
                    run_layer(ops, L, 1, tab, pos)
                g.capture_end()
        torch.cuda.synchronize()
        ops.stage_pos0(pos)
        torch.cuda.synchronize()
        for _ in range(5):
            g.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        graph_us = e0.elapsed_time(e1) * 1e3 / (steps * LAYERS)
    except Exception as exc:  # graph capture unavailable: report eager only
        log(f"decode graph capture failed: {exc}")
    b = layer_bytes(1, QWEN3_1_7B)
    return {"us_per_layer_eager": round(eager_us, 3),
            "us_per_layer_graph": None if graph_us is None else round(graph_us, 3),
            "bytes_per_layer": b, "position": pos, "launches_per_layer": 3}


def measure_prefill_4b(torch, ops, tab, steps=5, warmup=2):
    """Prefill n = 4096 at Qwen3-4B shape, 36 layers (the 4096-slot caches are filled):
    the chain's step time, then each op's 36 launches back to back (median of 5
    batches) and, secondary, each op's average under dispatch-attached events."""
    return measure_prefill_shape(torch, ops, tab, 4096, QWEN3_4B, 4, steps, warmup)


# One GPU's share of Qwen3-1.7B under tensor parallelism over 8 GPUs: the hidden
# size replicated (add + RMSNorm unchanged), 2 q heads and 1 kv head (with its
# cache slice), 768 of the 6144 intermediate columns.
QWEN3_1_7B_TP8 = dict(hidden=H, n_heads=HQ // 8, n_kv_heads=HKV // 8, inter=INTER // 8, layers=LAYERS)


def measure_shard_tp8(torch, ops, tab, steps=5, warmup=2):
    """The n = 2811 chain at one GPU's TP=8 shard shape (QWEN3_1_7B_TP8), measured
    like the 4B section. The sharded ops are small launches (10-26 MB)."""
    out = measure_prefill_shape(torch, ops, tab, N_PREFILL, QWEN3_1_7B_TP8, 8, steps, warmup)
    out["shape"] = QWEN3_1_7B_TP8
    return out


def measure_prefill_shape(torch, ops, tab, n, shape, seed, steps=5, warmup=2):
    """The chain at (n, shape): step time, each op's launches back to back (median
    of 5 batches) and each op's average under dispatch-attached events."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    layers = [Layer(torch, n, gen, shape) for _ in range(shape["layers"])]
    for _ in range(warmup):
        for L in layers:
            run_layer(ops, L, n, tab, 0)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        for L in layers:
            run_layer(ops, L, n, tab, 0)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    b = shape["layers"] * layer_bytes(n, shape)
    hid, hq, hkv, inter = shape["hidden"], shape["n_heads"], shape["n_kv_heads"], shape["inter"]
    op_bytes = {"add_rms_norm": bytes_add_rms(n, hid), "qk_norm_rope_kv": bytes_qk(n, hq, hkv),
                "swiglu": bytes_swiglu(n, inter)}
    batches = op_batches(torch, ops, layers, tab, n)
    ops.profile_start(3 * len(layers))
    hold_launches(torch, 3 * len(layers))
    for L in layers:
        run_layer(ops, L, n, tab, 0)
    ops.profile_stop()
    report = ops.profile_report()
    per_op = {}
    for name in OP_NAMES:
        us, samples = batches[name]
        kname = launched_kernel(report, name)
        ev = report[kname]["avg_us"]
        per_op[name] = {"us": round(us, 2), "pct_peak": round(op_bytes[name] / us / 1e3 / PEAK_GBPS * 100, 1),
                        "GBps": round(op_bytes[name] / us / 1e3, 1), "batch_us": [round(x, 2) for x in samples],
                        "us_event": round(ev, 2),
                        "pct_peak_event": round(op_bytes[name] / ev / 1e3 / PEAK_GBPS * 100, 1),
                        "bytes": op_bytes[name], "kernel": kname}
    del layers
    torch.cuda.empty_cache()
    return {"ms_per_step": round(ms, 4), "GBps": round(b / (ms * 1e-3) / 1e9, 1),
            "pct_of_peak": round(b / (ms * 1e-3) / 1e9 / PEAK_GBPS * 100, 2), "bytes_per_step": b,
            "us_per_layer": round(ms * 1e3 / shape["layers"], 2), "layers": shape["layers"], "n_tokens": n,
            "ops": per_op}


def gather_table(torch, ops, ggml_type, gen):
    """A [151936, 2048] token_embd of configs[1]'s distributions on the device:
    Q4_K: fp16 d, dmin = |N(0, 0.01)|, the 12 scale bytes and the 4-bit quants
    uniform random bytes; Q6_K: fp16 d = |N(0, 0.01)|, int8 scales uniform over
    -32..31, the 6-bit quants (ql, qh) uniform random bytes."""
    bb = 144 if ggml_type == ops.GGML_Q4_K else 210
    blocks_n = VOCAB * (H // 256)
    blob = torch.randint(0, 256, (blocks_n * bb,), dtype=torch.uint8, device="cuda", generator=gen)
    blocks = blob.view(blocks_n, bb)

    def f16_bytes():
        d = (torch.randn(blocks_n, generator=gen, device="cuda") * 0.01).abs().half()
        return d.view(torch.uint8).view(blocks_n, 2)

    if ggml_type == ops.GGML_Q4_K:
        blocks[:, 0:2] = f16_bytes()
        blocks[:, 2:4] = f16_bytes()
    else:
        sc = torch.randint(-32, 32, (blocks_n, 16), dtype=torch.int8, device="cuda", generator=gen)
        blocks[:, 192:208] = sc.view(torch.uint8)
        blocks[:, 208:210] = f16_bytes()
    return blob


def measure_gather(torch, ops, ggml_type, bb, copies=4, id_sets=64, reps=20):
    """n = 2811 ids gathered from a [151936, 2048] table. Launch i reads table copy
    i % copies with id set i % id_sets (each set uniform over the vocabulary, so
    each launch's rows are cold) and writes output window i % windows of a 1 GiB
    span, so no launch finds its rows or its output in the 256 MB Infinity Cache.
    `us`: median of 5 batches of `reps` launches back to back (batch_us);
    `us_event`: the same launches under dispatch-attached events;
    `us_idle_start`: each launch issued from Python after the previous one ended."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(10 + ggml_type)
    tables = [gather_table(torch, ops, ggml_type, gen) for _ in range(copies)]
    ids = [torch.randint(0, VOCAB, (N_PREFILL,), dtype=torch.int32, device="cuda", generator=gen)
           for _ in range(id_sets)]
    out_floats = N_PREFILL * H
    windows = max(2, -(-(1 << 30) // (4 * out_floats)))
    span = torch.empty(windows * out_floats, dtype=torch.float32, device="cuda")
    outs = [span[w * out_floats:(w + 1) * out_floats] for w in range(windows)]
    embs = [ops.GpuTensor(t, ggml_type, VOCAB, H) for t in tables]

    def launch(i):
        ops.GpuEmbeddingLookup(embs[i % copies], ids[i % id_sets], N_PREFILL, outs[i % windows])

    for i in range(copies):
        launch(i)
    torch.cuda.synchronize()
    name = "GatherQ4KKernel" if ggml_type == ops.GGML_Q4_K else "GatherQ6KKernel"
    us, samples = batch_us(torch, launch, reps, trials=5, start=copies)
    nxt = copies + 5 * reps

    def evented(queued, start):
        ops.profile_start(reps)
        if queued:
            hold_launches(torch, reps)
        for r in range(reps):
            launch(start + r)
        ops.profile_stop()
        return ops.profile_report()[name]

    ev = evented(True, nxt)
    idle = evented(False, nxt + reps)
    nbytes = bytes_gather(N_PREFILL, bb)
    del tables, outs, span
    torch.cuda.empty_cache()
    return {"us": round(us, 2), "GBps": round(nbytes / us / 1e3, 1),
            "pct_peak": round(nbytes / us / 1e3 / PEAK_GBPS * 100, 1), "batch_us": [round(x, 2) for x in samples],
            "bytes": nbytes, "kernel": name, "us_event": round(ev["avg_us"], 2),
            "us_idle_start": round(idle["avg_us"], 2), "table_copies": copies, "id_sets": id_sets,
            "output_windows": windows,
            "timing": "us: median of 5 batches of 20 launches back to back, one event pair per batch; "
                      "us_event: dispatch-attached events, launches queued; us_idle_start: each launch issued "
                      "from Python after the previous kernel ended"}


def measure_ceilings(torch, ops, sizes, reps=20):
    """Same-size streaming ceilings, timed like the ops (batch_us: `reps` launches
    back to back, one event pair per batch, median of 5). For each (label,
    total_bytes, write_bytes, read_bytes): a StreamCopyKernel moving total_bytes
    (half read, half written), a StreamFillKernel writing write_bytes and a
    StreamReadKernel reading read_bytes (a 0 skips that probe). Launches walk
    through 1 GiB source / destination spans, so no launch finds its window in
    the 256 MB Infinity Cache."""
    span = 1 << 30
    src = torch.empty(span // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    out = {}

    def timed(per_launch, launch):
        windows = max(2, span // per_launch)
        launch(0)
        us, _ = batch_us(torch, lambda i: launch(i % windows), reps, trials=5, start=1)
        return us

    for label, total, written, read in sizes:
        res = {}
        half = (total // 2) // 16 * 16
        if half > 0:
            def copy(i, half=half):
                off = i * half // 4
                ops.GpuStreamCopy(src[off:off + half // 4], dst[off:off + half // 4], half)

            res["copy_us"] = round(timed(half, copy), 2)
            res["copy_GBps"] = round(2 * half / res["copy_us"] / 1e3, 1)
        w = written // 16 * 16
        if w > 0:
            def fill(i, w=w):
                off = i * w // 4
                ops.GpuStreamFill(dst[off:off + w // 4], w, 0x3F800000)

            res["fill_us"] = round(timed(w, fill), 2)
            res["fill_GBps"] = round(w / res["fill_us"] / 1e3, 1)
        rd = read // 16 * 16
        if rd > 0:
            def rdl(i, rd=rd):
                off = i * rd // 4
                ops.GpuStreamRead(src[off:off + rd // 4], rd, sink)

            res["read_us"] = round(timed(rd, rdl), 2)
            res["read_GBps"] = round(rd / res["read_us"] / 1e3, 1)
        out[label] = res
    assert int(sink.item()) == 0, "the read probe's key was hit"
    del src, dst
    torch.cuda.empty_cache()
    return out


def measure_stream_read(torch, ops, nbytes=1 << 30, reps=10):
    """Read-only streaming ceiling over 1 GiB (StreamReadKernel, the reference's BwReadKernel probe)."""
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.GpuStreamRead(src, nbytes, sink)
    torch.cuda.synchronize()
    us, _ = batch_us(torch, lambda i: ops.GpuStreamRead(src, nbytes, sink), reps, trials=3)
    del src
    return round(nbytes / us / 1e3, 1)


def measure_copy(torch, ops, nbytes=1 << 30, reps=10):
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    ops.GpuStreamCopy(src, dst, nbytes)
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        ops.GpuStreamCopy(src, dst, nbytes)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    del src, dst
    return round(2 * nbytes / (ms * 1e-3) / 1e9, 1)


def profile_traffic(kernel_tag):
    """HBM bytes per launch of `kernel_tag` from the committed rocprofv3 counter summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by the calibration copy), if present."""
    path = os.path.join(REPO, "profiles", "pmc_traffic_prefill_n2811.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        m = re.match(r"\s*traffic_bytes_per_launch\[(.+?)\]\s*=\s*([0-9.eE+]+)", line)
        if m and m.group(1) == kernel_tag:
            return float(m.group(2))
    return None


# Qwen3-1.7B decode matrices as a Q4_K_M file stores them (attn_v / ffn_down in Q6_K
# on the layers that get more bits; the output projection in Q6_K).
DECODE_MATRICES = [
    ("attn_q", 12, 2048, 2048), ("attn_k", 12, 1024, 2048), ("attn_v", 14, 1024, 2048),
    ("attn_output", 12, 2048, 2048), ("ffn_gate", 12, INTER, 2048), ("ffn_up", 12, INTER, 2048),
    ("ffn_down", 14, 2048, INTER),
]
OUTPUT_MATRIX = ("output", 14, VOCAB, 2048)


def measure_matmul_decode(torch, ops, reps=20, span=768 << 20):
    """GpuMatMulQuant at n = 1 on each decode matrix: weight copies rotated so that a
    launch never finds its matrix in the 256 MB Infinity Cache; kernel time from
    dispatch-attached events. Bytes = weights + x + out."""
    res = {}
    layer_us = 0.0
    for name, t, rows, cols in DECODE_MATRICES + [OUTPUT_MATRIX]:
        rb = (cols // 256) * (144 if t == 12 else 210)
        wbytes = rows * rb
        copies = max(2, min(512, span // wbytes + 1))
        gen = torch.Generator(device="cuda")
        gen.manual_seed(20 + rows + cols + t)
        blob = torch.randint(0, 256, (copies * wbytes,), dtype=torch.uint8, device="cuda", generator=gen)
        # keep the fp16 scales finite: clear the exponent's top bit of every d / dmin
        blocks = blob.view(-1, 144 if t == 12 else 210)
        if t == 12:
            blocks[:, 1] &= 0x3B
            blocks[:, 3] &= 0x3B
        else:
            blocks[:, 209] &= 0x3B
        x = torch.randn((1, cols), dtype=torch.float32, device="cuda", generator=gen)
        out = torch.empty((1, rows), dtype=torch.float32, device="cuda")
        mats = [ops.GpuTensor(blob[i * wbytes:(i + 1) * wbytes], t, rows, cols) for i in range(copies)]
        for i in range(min(copies, 4)):
            ops.GpuMatMulQuant(mats[i], x, 1, out)
        torch.cuda.synchronize()
        ops.profile_start(reps)
        hold_launches(torch, reps)
        for r in range(reps):
            ops.GpuMatMulQuant(mats[r % copies], x, 1, out)
        ops.profile_stop()
        rep = ops.profile_report()
        kname, k = next(iter(rep.items()))
        nbytes = wbytes + 4 * cols + 4 * rows
        us = k["avg_us"]
        b2b = back_to_back_us(torch, ops, lambda i: ops.GpuMatMulQuant(mats[i % copies], x, 1, out))
        res[name] = {"type": "Q4_K" if t == 12 else "Q6_K", "rows": rows, "cols": cols, "us": round(us, 2),
                     "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "pct_peak": round(nbytes / (us * 1e-6) / 1e9 / PEAK_GBPS * 100, 1), "kernel": kname,
                     "bytes": nbytes, "us_back_to_back": round(b2b, 2),
                     "GBps_back_to_back": round(nbytes / (b2b * 1e-6) / 1e9, 1)}
        if name != OUTPUT_MATRIX[0]:
            layer_us += us
        del blob, blocks, mats, x, out
        torch.cuda.empty_cache()
    token_us = LAYERS * layer_us + res[OUTPUT_MATRIX[0]]["us"]
    grouped = measure_matmul_decode_grouped(torch, ops, reps, span)
    return {"matrices": res, "launch_floor_us_back_to_back": round(launch_floor_us(torch, ops), 2),
            "layer_us": round(layer_us, 2), "token_matmul_us": round(token_us, 1),
            "grouped": grouped,
            "token_matmul_us_grouped": round(LAYERS * grouped["layer_us"] + res[OUTPUT_MATRIX[0]]["us"], 1),
            "note": "n = 1, Qwen3-1.7B Q4_K_M layout; token_matmul_us = 28 layers + output projection, "
                    "matmuls only; _grouped = with q/k/v and gate/up fused per layer (GpuMatMulQuantGroup); "
                    "us: dispatch-attached events (a ~4 us floor under any kernel); us_back_to_back: 100 "
                    "launches captured in one HIP graph, replays timed with stream events (the per-launch "
                    "cost in a graph-replayed decode loop), beside launch_floor_us_back_to_back for a "
                    "one-workgroup kernel"}


def measure_matmul_decode_grouped(torch, ops, reps, span):
    """One 1.7B layer's decode matmuls as GpuMatMulQuantGroup launches: [q, k, v] (Q4_K,
    Q4_K, Q6_K in one launch), [o], [gate, up], [down]; copies rotated past the Infinity
    Cache. `forward` times the same matrices in the launches the decode step issues: the
    attention and FFN norms formed inside the q / k / v and gate / up launches
    (GpuNormMatMulQuantGroup, GpuNormMatMulQuantSwiGLU, the latter writing silu(gate) * up),
    then o and down."""
    mats = {name: (t, rows, cols) for name, t, rows, cols in DECODE_MATRICES}
    groups = [["attn_q", "attn_k", "attn_v"], ["attn_output"], ["ffn_gate", "ffn_up"], ["ffn_down"]]
    res, layer_us, layer_b2b, forward = {}, 0.0, 0.0, {}
    for grp in groups:
        specs = [mats[n] for n in grp]
        sizes = [rows * (cols // 256) * (144 if t == 12 else 210) for t, rows, cols in specs]
        copies = max(2, min(256, span // sum(sizes) + 1))
        gen = torch.Generator(device="cuda")
        gen.manual_seed(60 + sum(sizes))
        sets = []
        for _ in range(copies):
            ts = []
            for (t, rows, cols), nbytes in zip(specs, sizes):
                blob = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda", generator=gen)
                blocks = blob.view(-1, 144 if t == 12 else 210)
                if t == 12:
                    blocks[:, 1] &= 0x3B
                    blocks[:, 3] &= 0x3B
                else:
                    blocks[:, 209] &= 0x3B
                ts.append(ops.GpuTensor(blob, t, rows, cols))
            sets.append(ts)
        cols = specs[0][2]
        x = torch.randn((1, cols), device="cuda", generator=gen)
        outs = [torch.empty((1, rows), device="cuda") for _, rows, _ in specs]
        for i in range(min(copies, 4)):
            ops.GpuMatMulQuantGroup(sets[i], x, 1, outs)
        torch.cuda.synchronize()
        ops.profile_start(reps * len(grp))
        hold_launches(torch, reps * len(grp))
        for r in range(reps):
            ops.GpuMatMulQuantGroup(sets[r % copies], x, 1, outs)
        ops.profile_stop()
        rep = ops.profile_report()
        us = sum(k["total_us"] for k in rep.values()) / reps
        nbytes = sum(sizes) + 4 * cols + 4 * sum(r for _, r, _ in specs)
        b2b = back_to_back_us(torch, ops, lambda i: ops.GpuMatMulQuantGroup(sets[i % copies], x, 1, outs))
        res["+".join(grp)] = {"us": round(us, 2), "launches": int(sum(k["count"] for k in rep.values()) // reps),
                              "GBps": round(nbytes / us / 1e3, 1), "bytes": nbytes,
                              "us_back_to_back": round(b2b, 2), "GBps_back_to_back": round(nbytes / b2b / 1e3, 1)}
        layer_us += us
        layer_b2b += b2b
        if grp[0] in ("attn_q", "ffn_gate"):
            # the same group with the norm formed inside the launch, as the decode step runs it
            d = torch.randn((1, cols), device="cuda", generator=gen)
            nw = torch.randn((1, cols), device="cuda", generator=gen)
            x_out = torch.empty_like(x)
            if grp[0] == "attn_q":
                def launch(i):
                    assert ops.GpuNormMatMulQuantGroup(x, d, nw, 1e-6, x_out, sets[i % copies], outs)
            else:
                def launch(i):
                    st = sets[i % copies]
                    assert ops.GpuNormMatMulQuantSwiGLU(x, d, nw, 1e-6, x_out, st[0], st[1], outs[0], outs[1])
            forward[grp[0]] = round(back_to_back_us(torch, ops, launch), 2)
        else:
            forward[grp[0]] = round(b2b, 2)
        del sets, x, outs
        torch.cuda.empty_cache()
    return {"groups": res, "layer_us": round(layer_us, 2), "layer_us_back_to_back": round(layer_b2b, 2),
            "forward_back_to_back": {"norm+attn_q+attn_k+attn_v": forward["attn_q"],
                                     "attn_output": forward["attn_output"],
                                     "norm+ffn_gate+ffn_up+swiglu": forward["ffn_gate"],
                                     "ffn_down": forward["ffn_down"],
                                     "layer_us": round(sum(forward.values()), 2)}}


def measure_matmul_prefill(torch, ops, n=N_PREFILL, reps=3):
    """GpuMatMulQuant at prefill size (n = 2811) on the Qwen3-1.7B layer matrices:
    the matrix-core GEMM. Each matrix alone (its own activation split), then the
    layer as the forward runs it (GpuMatMulQuantGroup: q / k / v and gate / up
    share one split). Reported as useful TFLOP/s (2 n rows cols) against
    MI355X's dense fp16 peak; the matrix cores execute 2x that for Q4_K (two
    fp16 activation terms) and 4x for Q6_K (two weight terms as well)."""
    res = {}
    layer_us = 0.0
    mats = {}
    for name, t, rows, cols in DECODE_MATRICES:
        rb = (cols // 256) * (144 if t == 12 else 210)
        gen = torch.Generator(device="cuda")
        gen.manual_seed(40 + rows + cols + t)
        blob = torch.randint(0, 256, (rows * rb,), dtype=torch.uint8, device="cuda", generator=gen)
        blocks = blob.view(-1, 144 if t == 12 else 210)
        if t == 12:
            blocks[:, 1] &= 0x3B
            blocks[:, 3] &= 0x3B
        else:
            blocks[:, 209] &= 0x3B
        x = torch.randn((n, cols), dtype=torch.float32, device="cuda", generator=gen)
        out = torch.empty((n, rows), dtype=torch.float32, device="cuda")
        mat = ops.GpuTensor(blob, t, rows, cols)
        mats[name] = (mat, blob, x, out)
        ops.GpuMatMulQuant(mat, x, n, out)
        torch.cuda.synchronize()
        ops.profile_start(4 * reps)
        hold_launches(torch, 4 * reps)
        for _ in range(reps):
            ops.GpuMatMulQuant(mat, x, n, out)
        ops.profile_stop()
        rep = ops.profile_report()
        us = sum(k["total_us"] for k in rep.values()) / reps
        flops = 2.0 * n * rows * cols
        res[name] = {"type": "Q4_K" if t == 12 else "Q6_K", "rows": rows, "cols": cols, "us": round(us, 1),
                     "TFLOPs": round(flops / us / 1e6, 1),
                     "kernels": {kn: round(k["avg_us"], 1) for kn, k in rep.items()}}
        layer_us += us
    groups = (("attn_q", "attn_k", "attn_v"), ("attn_output",), ("ffn_gate", "ffn_up"), ("ffn_down",))

    def layer():
        for g in groups:
            x = mats[g[0]][2]
            ops.GpuMatMulQuantGroup([mats[k][0] for k in g], x, n, [mats[k][3] for k in g])

    layer()
    torch.cuda.synchronize()
    ops.profile_start(32 * reps)
    hold_launches(torch, 16 * reps)
    for _ in range(reps):
        layer()
    ops.profile_stop()
    rep = ops.profile_report()
    grouped_us = sum(k["total_us"] for k in rep.values()) / reps
    del mats
    torch.cuda.empty_cache()
    total_flops = sum(2.0 * n * r * c for _, _, r, c in DECODE_MATRICES)
    return {"n_tokens": n, "matrices": res, "layer_us": round(grouped_us, 1),
            "layer_TFLOPs": round(total_flops / grouped_us / 1e6, 1),
            "layer_us_matrix_by_matrix": round(layer_us, 1),
            "layer_kernels": {kn: {"count": k["count"] // reps, "avg_us": round(k["avg_us"], 1)}
                              for kn, k in rep.items()},
            "roofline": {"bound": "mfma", "peak": 2500.0, "unit": "TFLOP/s",
                         "note": "useful fp32-accurate TFLOP/s against the dense fp16 peak; the matrix cores "
                                 "execute 2x that for Q4_K (two fp16 activation terms) and 4x for Q6_K (even / odd "
                                 "scale parts as well)"}}


def measure_attention(torch, ops, reps=20):
    """GpuAttentionFromCache on the Qwen3-1.7B cache (16 q heads, 8 kv heads, d 128,
    max_seq 4096). Decode (one token at pos0) over rotating cache copies whose
    total exceeds 2x the Infinity Cache; bytes = the K and V rows read
    (2 * n_kv * (pos0 + 1) * 128 * 2) plus q and out. Prefill n = 2811 from
    position 0: useful TFLOP/s = 4 * d * heads * sum over tokens of keys."""
    nh, nkv, d, max_seq = HQ, HKV, D, MAX_SEQ
    layer_elems = nkv * max_seq * d
    copies = 32
    gen = torch.Generator(device="cuda")
    gen.manual_seed(77)
    kc = torch.randn((copies, layer_elems), generator=gen, device="cuda").half()
    vc = torch.randn((copies, layer_elems), generator=gen, device="cuda").half()
    out = {"decode": {}}
    q1 = torch.randn((1, nh, d), generator=gen, device="cuda")
    o1 = torch.empty_like(q1)
    for pos0 in (511, 2047, 4095):
        for i in range(4):
            ops.GpuAttentionFromCache(nh, nkv, d, pos0, q1, 1, kc[i], vc[i], max_seq, o1)
        torch.cuda.synchronize()
        ops.profile_start(2 * reps)
        hold_launches(torch, 2 * reps)
        for r in range(reps):
            ops.GpuAttentionFromCache(nh, nkv, d, pos0, q1, 1, kc[r % copies], vc[r % copies], max_seq, o1)
        ops.profile_stop()
        rep = ops.profile_report()
        us = sum(k["total_us"] for k in rep.values()) / reps
        nbytes = 2 * nkv * (pos0 + 1) * d * 2 + 2 * 4 * nh * d
        # a captured launch reads its position from the staging scalar on every replay
        ops.stage_pos0(pos0)
        torch.cuda.synchronize()
        b2b = back_to_back_us(torch, ops, lambda i: ops.GpuAttentionFromCache(
            nh, nkv, d, pos0, q1, 1, kc[i % copies], vc[i % copies], max_seq, o1))
        out["decode"][f"pos{pos0}"] = {"us": round(us, 2), "GBps": round(nbytes / us / 1e3, 1),
                                       "pct_peak": round(nbytes / us / 1e3 / PEAK_GBPS * 100, 1),
                                       "kernels": {n: round(k["avg_us"], 2) for n, k in rep.items()},
                                       "bytes": nbytes, "us_back_to_back": round(b2b, 2),
                                       "GBps_back_to_back": round(nbytes / b2b / 1e3, 1)}
    n = N_PREFILL
    qp = torch.randn((n, nh, d), generator=gen, device="cuda")
    op = torch.empty_like(qp)
    ops.GpuAttentionFromCache(nh, nkv, d, 0, qp, n, kc[0], vc[0], max_seq, op)
    torch.cuda.synchronize()
    ops.profile_start(6)
    hold_launches(torch, 6)
    for r in range(3):
        ops.GpuAttentionFromCache(nh, nkv, d, 0, qp, n, kc[r + 1], vc[r + 1], max_seq, op)
    ops.profile_stop()
    rep = ops.profile_report()
    us = sum(k["total_us"] for k in rep.values()) / 3
    flops = 4.0 * d * nh * (n * (n + 1) / 2)
    out["prefill_n2811"] = {"us": round(us, 1), "TFLOPs": round(flops / us / 1e6, 2),
                            "kernels": {n_: round(k["avg_us"], 1) for n_, k in rep.items()}}
    del kc, vc
    torch.cuda.empty_cache()
    return out


def measure_sampler(torch, ops, reps=50):
    """Device argmax and sampling over Qwen3's vocabulary (151936 logits, the
    reference's synthetic logits seed 5): kernel microseconds per call (sum of
    the launches, dispatch-attached events), the stream's wall time per call, and
    us_back_to_back: the call (its device-counter form, as a graph-replayed decode
    loop runs it) captured 100 times in one HIP graph, per call. Latency-bound: a
    few MB of traffic per call."""
    n = VOCAB
    x = torch.rand(n, generator=torch.Generator(device="cuda").manual_seed(5), device="cuda") * 16 - 8
    probs = torch.empty(n, device="cuda")
    idx = torch.empty(1, dtype=torch.int32, device="cuda")
    ops.GpuSamplerWarmup()
    counter = torch.zeros(1, dtype=torch.int64, device="cuda")
    graph_forms = {
        "argmax": lambda i: ops.GpuArgMax(x, n, idx),
        "sample_T0.7_topp0.95": lambda i: ops.GpuSampleTokenDev(x, n, ops.SampleOptions(0.7, 0, 0.95), 1, counter,
                                                                probs, idx),
        "sample_T0.7_topk20_topp0.95": lambda i: ops.GpuSampleTokenDev(x, n, ops.SampleOptions(0.7, 20, 0.95), 1,
                                                                       counter, probs, idx),
        "sample_T1": lambda i: ops.GpuSampleTokenDev(x, n, ops.SampleOptions(1.0, 0, 1.0), 1, counter, probs, idx),
    }
    cases = {
        "argmax": lambda: ops.GpuArgMax(x, n, idx),
        "sample_T0.7_topp0.95": lambda: ops.GpuSampleToken(x, n, ops.SampleOptions(0.7, 0, 0.95), 1, 3, probs, idx),
        "sample_T0.7_topk20_topp0.95": lambda: ops.GpuSampleToken(x, n, ops.SampleOptions(0.7, 20, 0.95), 1, 3,
                                                                  probs, idx),
        "sample_T1": lambda: ops.GpuSampleToken(x, n, ops.SampleOptions(1.0, 0, 1.0), 1, 3, probs, idx),
    }
    res = {}
    for name, fn in cases.items():
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        ops.profile_start(16 * reps)
        for _ in range(reps):
            fn()
        ops.profile_stop()
        rep = ops.profile_report()
        kus = sum(k["total_us"] for k in rep.values()) / reps
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        res[name] = {"kernel_us": round(kus, 2), "wall_us": round(e0.elapsed_time(e1) * 1e3 / reps, 2),
                     "us_back_to_back": round(back_to_back_us(torch, ops, graph_forms[name]), 2),
                     "launches": int(sum(k["count"] for k in rep.values()) // reps),
                     "kernels": {k_: round(v["avg_us"], 2) for k_, v in rep.items()}}
    return {"vocab": n, **res}


def measure_gguf_upload(torch, ops, reps=3):
    """GpuModel::Load of a Qwen3-1.7B-shaped Q4_K_M GGUF (1.15 GB, random bytes,
    written to the local temp directory first): file bytes per second from the
    start of the upload to the last byte on the device (page cache warm), against
    the PCIe 5.0 x16 host link (64 GB/s per direction). Beside it, the
    reference's way -- one synchronous pageable copy per tensor out of the
    mapping (src/gpu_model.cu:40-50) -- done with torch on the same file."""
    import tempfile

    import numpy as np

    sys.path.insert(0, os.path.join(REPO, "tests"))
    import gguf_writer

    kv, specs = gguf_writer.qwen3_1_7b_specs(tied=True)
    rng = np.random.default_rng(9)
    tmpdir = os.environ.get("TMPDIR") or tempfile.gettempdir()
    path = os.path.join(tmpdir, "rpg_bench_qwen3_1_7b.gguf")
    size = gguf_writer.write_file(path, kv, specs, lambda name, n: rng.bytes(n))
    try:
        runs = []
        for _ in range(reps):
            m = ops.GpuModel(path, 4096)
            runs.append(m.upload_stats())
            desc = m.describe()
            m.free()
            torch.cuda.synchronize()
        best = min(runs, key=lambda r: r["upload_seconds"])
        nbytes = best["bytes"]
        # reference-style: per tensor, one pageable copy from the mapping
        with ops.GgufFile(path) as g:
            tensors = g.tensors()
        ref_times = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            mm = np.memmap(path, dtype=np.uint8, mode="r")  # mapped per load, as the reference does
            outs = [torch.from_numpy(np.array(mm[t["file_offset"]:t["file_offset"] + t["n_bytes"]], copy=False))
                    .to("cuda") for t in tensors]
            torch.cuda.synchronize()
            ref_times.append(time.perf_counter() - t0)
            del outs, mm
        torch.cuda.empty_cache()
        gbps = nbytes / best["upload_seconds"] / 1e9
        ref = sum(t["n_bytes"] for t in tensors) / min(ref_times) / 1e9
        return {"file_bytes": size, "uploaded_bytes": nbytes, "upload_s": round(best["upload_seconds"], 4),
                "parse_s": round(best["parse_seconds"], 4), "GBps": round(gbps, 2),
                "pct_of_pcie5_x16": round(gbps / 64.0 * 100, 1),
                "runs_s": [round(r["upload_seconds"], 4) for r in runs],
                "per_tensor_pageable_GBps": round(ref, 2), "describe": desc}
    finally:
        os.remove(path)


def measure_model_e2e(torch, ops, reps=3, decode_tokens=128):
    """The whole Qwen3-1.7B through the library: a Q4_K_M-layout GGUF with
    zero-mean, trained-weight-sized synthetic weights (tied embeddings), loaded
    with rpg_model_load, then
      * prefill (GpuForwardFull with the cache, logits for every position as the
        reference computes them) of 21 and 2811 tokens;
      * greedy decoding (GpuGenerate) after those prompts, with the HIP-graph loop
        and with per-step launches; one sampled run (T 0.7, top_k 40, top_p 0.9).
    Wall-clock times with the device synchronised; medians of `reps`."""
    import tempfile

    import numpy as np

    sys.path.insert(0, os.path.join(REPO, "tests"))
    import gguf_writer

    kv_meta, specs = gguf_writer.qwen3_1_7b_specs(tied=True)
    shapes = {name: (dims, t) for name, dims, t in specs}
    rng = np.random.default_rng(17)

    def fill(name, n):
        dims, t = shapes[name]
        raw = gguf_writer.random_tensor(rng, t, dims, model_like=True)
        assert len(raw) == n, (name, len(raw), n)
        return raw

    tmpdir = os.environ.get("TMPDIR") or tempfile.gettempdir()
    path = os.path.join(tmpdir, "rpg_bench_qwen3_1_7b_model.gguf")
    t0 = time.perf_counter()
    gguf_writer.write_file(path, kv_meta, specs, fill, chunk=1 << 40)
    gen_s = time.perf_counter() - t0
    try:
        m = ops.GpuModel(path, 4096)
        vocab = m.meta()["vocab"]
        s = ops.GpuScratch()
        kv = ops.GpuKvCache(m, 4096)
        out = {"model": "Qwen3-1.7B shape, 28 layers, Q4_K_M layout (Q6_K token_embd / attn_v / ffn_down), tied",
               "weights": "synthetic zero-mean Q4_K / Q6_K blocks (std ~0.04), N(1, 0.1) norms",
               "file_gen_s": round(gen_s, 1), "device_bytes": m.upload_stats()["bytes"]}

        def prefill(n):
            toks = np.random.default_rng(n).integers(0, vocab, size=n).astype(np.int32)
            times = []
            for _ in range(reps + 1):
                kv.reset()
                torch.cuda.synchronize()
                t = time.perf_counter()
                ops.GpuForwardFull(m, toks, s, want_logits=False, kv=kv)
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t)
            return float(np.median(times[1:]))

        def decode(n_prompt, use_graph, sample=None):
            prompt_s = prefill(n_prompt)
            first = s.logits_dev() + 4 * vocab * (n_prompt - 1)
            opt = ops.GpuGenerateOptions(max_tokens=decode_tokens, use_graph=use_graph, seed=7,
                                         sample=sample or ops.SampleOptions(0.0))
            times = []
            for _ in range(reps + 1):
                kv.set_len(n_prompt)
                torch.cuda.synchronize()
                t = time.perf_counter()
                ids, _ = ops.GpuGenerate(m, kv, s, first, opt)
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t)
                assert len(ids) == decode_tokens
            sec = float(np.median(times[1:]))
            return prompt_s, sec

        for n in (21, N_PREFILL):
            sec = prefill(n)
            out[f"prefill_n{n}"] = {"ms": round(sec * 1e3, 2), "tok_per_s": round(n / sec, 1)}
        for n_prompt in (21, N_PREFILL):
            for use_graph in (True, False):
                _, sec = decode(n_prompt, use_graph)
                out[f"decode_after_{n_prompt}_{'graph' if use_graph else 'per_step'}"] = {
                    "tokens": decode_tokens, "ms_per_token": round(sec / decode_tokens * 1e3, 3),
                    "tok_per_s": round(decode_tokens / sec, 1)}
        _, sec = decode(21, True, ops.SampleOptions(0.7, 40, 0.9))
        out["decode_after_21_graph_sampled"] = {"tokens": decode_tokens,
                                                "ms_per_token": round(sec / decode_tokens * 1e3, 3),
                                                "tok_per_s": round(decode_tokens / sec, 1)}
        kv.free()
        s.free()
        m.free()
        torch.cuda.empty_cache()
        return out
    finally:
        os.remove(path)


def host_cpu():
    """(threads this process may use, logical CPUs of the host, CPU model)."""
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return usable, os.cpu_count() or usable, model


# CPU threads of the baseline: every thread the process may use, capped at the
# 16-thread CPU share a one-GPU job gets on the GPU boxes (the host itself can
# have many more logical CPUs; both counts are reported).
CPU_SHARE = 16


def cpu_baseline():
    """The oracle's C restatement of one layer of the chain (n = 2811, 1.7B shape,
    the benchmark's input distributions) on the host cores, median of 5; plus
    per-op and single-thread figures. A reported baseline only."""
    from oracle import pyoracle

    usable, host_cpus, model = host_cpu()
    threads = max(1, min(usable, CPU_SHARE))
    args = (N_PREFILL, H, HQ, HKV, INTER)
    sec = pyoracle.bench_layer_chain(threads, *args, 5)
    if sec <= 0:
        return None
    b = layer_bytes(N_PREFILL, QWEN3_1_7B)
    per_op = {}
    for op, name, nbytes in ((1, "add_rms_norm", bytes_add_rms(N_PREFILL)), (2, "qk_norm_rope_kv", bytes_qk(N_PREFILL)),
                             (3, "swiglu", bytes_swiglu(N_PREFILL))):
        t = pyoracle.bench_layer_op(op, threads, *args, 3)
        per_op[name] = {"ms": round(t * 1e3, 3), "GBps": round(nbytes / t / 1e9, 2)}
    t1 = pyoracle.bench_layer_chain(1, *args, 1)
    gq4 = pyoracle.bench_gather(threads, pyoracle.Q4_K, VOCAB, H, N_PREFILL, 3)
    gref = pyoracle.ref_bench_gather(pyoracle.Q4_K, VOCAB, H, N_PREFILL, 3)  # the reference's own quant.cc
    mm = pyoracle.bench_matmul(pyoracle.Q6_K, 4096, 2048, 3)
    return {"value": round(b / sec / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "host_logical_cpus": host_cpus, "usable_cpus": usable, "cpu_model": model,
            "sample": f"one layer of the n={N_PREFILL} chain (add+RMSNorm, qk-norm+RoPE+fp16 KV, SwiGLU; "
                      f"{b} B; activations N(0,1), norm weights N(1,0.1)) by the C oracle, rows split over "
                      f"{threads} threads, median of 5 runs ({sec * 1e3:.1f} ms each)",
            "per_op": per_op, "single_thread_GBps": round(b / t1 / 1e9, 2),
            "gather_q4k_GBps": round(bytes_gather(N_PREFILL, 144) / gq4 / 1e9, 2),
            "gather_q4k_reference_1thread_GBps": (round(bytes_gather(N_PREFILL, 144) / gref / 1e9, 2)
                                                  if gref else None),
            "gather_reference_sample": "the reference's own src/quant.cc DequantizeRow per token row (the CPU "
                                       "engine's gather), built into oracle/_ref, one thread, 2811 random rows of "
                                       "the [151936, 2048] Q4_K table (fp16 d, dmin |N(0,0.01)|), best of 3",
            "matmul_q6k_n1_GBps": round((4096 * 8 * 210 + 4 * 2048 + 4 * 4096) / mm / 1e9, 3),
            "matmul_sample": "4096 x 2048 Q6_K rows times one fp32 vector by the oracle's float64 "
                             "restatement, one thread"}


def calibration_copy(torch, ops):
    """Calibration dispatch for the rocprofv3 counter runs: one StreamCopyKernel of
    exactly CALIB_BYTES read + CALIB_BYTES written, whose FETCH_SIZE / WRITE_SIZE
    give the counters' scale against known traffic."""
    src = torch.empty(CALIB_BYTES // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    ops.GpuStreamCopy(src, dst, CALIB_BYTES)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()


# Secondary measurements that --only can run alone.
SECTIONS = {
    "model_e2e": lambda torch, ops: measure_model_e2e(torch, ops),
    "matmul_prefill_n2811": lambda torch, ops: measure_matmul_prefill(torch, ops),
    "matmul_decode_n1": lambda torch, ops: measure_matmul_decode(torch, ops),
    "attention": lambda torch, ops: measure_attention(torch, ops),
    "sampler": lambda torch, ops: measure_sampler(torch, ops),
    "gather": lambda torch, ops: {"q4k": measure_gather(torch, ops, ops.GGML_Q4_K, 144),
                                  "q6k": measure_gather(torch, ops, ops.GGML_Q6_K, 210)},
    "shard_tp8_n2811": lambda torch, ops: measure_shard_tp8(
        torch, ops, torch.from_numpy(ops.build_rope_table(D, THETA, MAX_SEQ)).cuda()),
    "prefill_4b_n4096": lambda torch, ops: measure_prefill_4b(
        torch, ops, torch.from_numpy(ops.build_rope_table(D, THETA, MAX_SEQ)).cuda()),
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-extras", action="store_true", help="only the headline prefill workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-model", action="store_true",
                    help="skip the whole-model measurement (~1M kernel launches; for kernel-trace runs)")
    ap.add_argument("--only", choices=sorted(SECTIONS), default=None,
                    help="run one secondary measurement alone and print its JSON (for profiling runs); "
                         "not the benchmark line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from rpgbarenginecuda_amd import ops

    ops.load_library()
    ops.init()
    ops.set_stream(torch.cuda.current_stream())
    ok, desc = ops.device_info()
    log(desc)
    if args.only is not None:
        result = SECTIONS[args.only](torch, ops)
        calibration_copy(torch, ops)
        print(json.dumps({args.only: result}), flush=True)
        return

    tab = torch.from_numpy(ops.build_rope_table(D, THETA, MAX_SEQ)).cuda()

    log(f"allocating {LAYERS} layers of prefill buffers (n={N_PREFILL})")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2026)
    layers = [Layer(torch, N_PREFILL, gen) for _ in range(LAYERS)]
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps after {args.warmup} warmup")
    ms_step, ms_prof, report = timed_prefill(torch, ops, layers, tab, N_PREFILL, args.steps, args.warmup)
    log(f"ms/step {ms_step:.4f} (kernel sum {ms_prof:.4f} in the profiled pass); kernels: {json.dumps(report)}")
    step_bytes = LAYERS * layer_bytes(N_PREFILL, QWEN3_1_7B)
    value = step_bytes / (ms_step * 1e-3) / 1e9
    op_bytes = {"add_rms_norm": bytes_add_rms(N_PREFILL), "qk_norm_rope_kv": bytes_qk(N_PREFILL),
                "swiglu": bytes_swiglu(N_PREFILL)}
    log("per-op batches: each op's 28 launches back to back, median of 5")
    batches = op_batches(torch, ops, layers, tab, N_PREFILL)
    op_stats = {}
    for name in OP_NAMES:
        kname = launched_kernel(report, name)
        k = report[kname]
        assert k["count"] == args.steps * LAYERS, (name, k)
        us, samples = batches[name]
        op_stats[name] = {"us": round(us, 2), "GBps": round(op_bytes[name] / us / 1e3, 1),
                          "pct_peak": round(op_bytes[name] / us / 1e3 / PEAK_GBPS * 100, 1),
                          "batch_us": [round(x, 2) for x in samples],
                          "us_event": round(k["avg_us"], 2),
                          "pct_peak_event": round(op_bytes[name] / k["avg_us"] / 1e3 / PEAK_GBPS * 100, 1),
                          "bytes": op_bytes[name], "kernel": kname, "launches_event_pass": k["count"]}
    dominant = max(OP_NAMES, key=lambda k: op_stats[k]["us"])
    achieved = op_bytes[dominant] / op_stats[dominant]["us"] / 1e3
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / PEAK_GBPS, 4), "traffic": profile_traffic(op_stats[dominant]["kernel"]),
                "kernel": op_stats[dominant]["kernel"], "algorithmic_bytes_per_launch": op_bytes[dominant],
                "timing": "median of 5 batches of the kernel's 28 launches (one per layer's buffers) back to back, "
                          "one stream-event pair around each batch",
                "achieved_event_pass": round(op_bytes[dominant] / op_stats[dominant]["us_event"] / 1e3, 1)}
    del layers
    torch.cuda.empty_cache()

    calibration_copy(torch, ops)

    extras = {}
    if not args.no_extras:
        log("decode n=1")
        extras["decode_n1"] = measure_decode(torch, ops, tab, max(20, args.steps))
        log("prefill n=4096 at the 4B shape, 36 layers")
        extras["prefill_4b_n4096"] = measure_prefill_4b(torch, ops, tab)
        log("prefill n=2811 at one GPU's TP=8 shard of the 1.7B shape")
        extras["shard_tp8_n2811"] = measure_shard_tp8(torch, ops, tab)
        log("decode matmuls (GpuMatMulQuant, n = 1)")
        extras["matmul_decode_n1"] = measure_matmul_decode(torch, ops)
        log("prefill matmuls (GpuMatMulQuant, n = 2811)")
        extras["matmul_prefill_n2811"] = measure_matmul_prefill(torch, ops)
        log("attention from the fp16 cache (decode, prefill n=2811)")
        extras["attention"] = measure_attention(torch, ops)
        log("argmax / sampler over the 151936-entry vocabulary")
        extras["sampler"] = measure_sampler(torch, ops)
        if not args.no_model:
            log("whole model: Qwen3-1.7B prefill and decode through rpg_forward / rpg_generate")
            extras["model_e2e"] = measure_model_e2e(torch, ops)
        log("GGUF upload (Qwen3-1.7B-shaped file)")
        extras["gguf_upload"] = measure_gguf_upload(torch, ops)
        log("gather Q4_K / Q6_K")
        extras["gather_q4k_n2811"] = measure_gather(torch, ops, ops.GGML_Q4_K, 144)
        extras["gather_q6k_n2811"] = measure_gather(torch, ops, ops.GGML_Q6_K, 210)
        log("stream copy / read ceilings (1 GiB)")
        extras["stream_copy_GBps"] = measure_copy(torch, ops)
        extras["stream_read_GBps"] = measure_stream_read(torch, ops)
        log("same-size copy / fill / read ceilings")
        out_bytes = 4 * N_PREFILL * H
        ceil_sizes = [
            ("add_rms_norm", op_bytes["add_rms_norm"], 8 * N_PREFILL * H, 0),
            ("qk_norm_rope_kv", op_bytes["qk_norm_rope_kv"], N_PREFILL * (4 * HQ * D + 4 * HKV * D), 0),
            ("swiglu", op_bytes["swiglu"], 4 * N_PREFILL * INTER, 0),
            ("gather_q4k", bytes_gather(N_PREFILL, 144), out_bytes, bytes_gather(N_PREFILL, 144) - out_bytes),
            ("gather_q6k", 0, 0, bytes_gather(N_PREFILL, 210) - out_bytes)]
        mm = extras.get("matmul_decode_n1")
        if mm:
            for name, m in mm["matrices"].items():
                ceil_sizes.append((f"matvec_{name}", 0, 0, m["bytes"]))
            for name, g in mm["grouped"]["groups"].items():
                ceil_sizes.append((f"matvec_group_{name}", 0, 0, g["bytes"]))
        ceil = measure_ceilings(torch, ops, ceil_sizes)
        for name in OP_NAMES:
            c = ceil[name]
            op_stats[name]["copy_ceiling_us"] = c["copy_us"]
            op_stats[name]["pct_of_copy_ceiling"] = round(c["copy_us"] / op_stats[name]["us"] * 100, 1)
        for key, label in (("gather_q4k_n2811", "gather_q4k"), ("gather_q6k_n2811", "gather_q6k")):
            g = extras[key]
            g["write_ceiling_us"] = ceil["gather_q4k"]["fill_us"]
            g["pct_of_write_ceiling"] = round(ceil["gather_q4k"]["fill_us"] / g["us"] * 100, 1)
            g["table_read_ceiling_us"] = ceil[label]["read_us"]
        if mm:
            for name, m in mm["matrices"].items():
                m["read_ceiling_us"] = ceil[f"matvec_{name}"]["read_us"]
                m["pct_of_read_ceiling"] = round(m["read_ceiling_us"] / m["us_back_to_back"] * 100, 1)
            for name, g in mm["grouped"]["groups"].items():
                g["read_ceiling_us"] = ceil[f"matvec_group_{name}"]["read_us"]
                g["pct_of_read_ceiling"] = round(g["read_ceiling_us"] / g["us_back_to_back"] * 100, 1)
        extras["ceilings"] = ceil
    cpu = None if args.no_cpu else cpu_baseline()

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "kernel_ms_per_step_profiled_pass": round(ms_prof, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch.randn activations and N(1,0.1) norm weights per layer)",
        "config": {"workload": "configs[3]: prefill n=2811, Qwen3-1.7B shape, 28 layers with independent buffers; "
                               "per layer residual+RMSNorm, q/k-norm+RoPE+fp16 KV write, SwiGLU",
                   "n_tokens": N_PREFILL, "layers": LAYERS, "hidden": H, "n_heads": HQ, "n_kv_heads": HKV,
                   "head_dim": D, "intermediate": INTER, "max_seq": MAX_SEQ, "bytes_per_step": step_bytes},
        "pct_of_peak": round(value / PEAK_GBPS * 100, 2),
        "ops": op_stats,
        "roofline": roofline,
        "cpu_baseline": cpu,
        **extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
