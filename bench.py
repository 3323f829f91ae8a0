#!/usr/bin/env python3
"""Benchmark of the int8 quantized-linear hot path on one MI355X.

Headline (BASELINE.json `metric`, configs[1]): decode dequant-GEMV, W int8
[4096, 4096] with per-row f32 scales, X fp16 [1, 4096], Y fp16.  One step is
one GEMV over one weight copy; 96 distinct copies (1.6 GB, > 6x the 256 MB
Infinity Cache) rotate so every step reads its weight from HBM.  The timed
region is exactly `--steps` launches, replayed from HIP graphs on the context's
stream (see time_steps).

Printed JSON (one line, stdout):
  value            whole-job GB/s = algorithmic bytes x steps / timed wall time
  roofline         dominant kernel (the GEMV): algorithmic bytes / mean launch
                   duration (device wall-clock stamps on the launch stream
                   around the timed launches, back to back), vs 8 TB/s
  floor            the same weight bytes read without the GEMV's arithmetic
                   (and with its output store): the one-launch floor
  cpu_baseline     the reference's per-token path on host cores: k-ascending
                   f32 GEMV on the load-time-dequantized f32 weight (oracle port);
                   `legs`: the same path at configs[0] and at the configs[3]
                   prefill shape (a bounded sample of its tokens)
  prefill          dequant-GEMM TFLOPS at M=2048 for the three configs[3] shapes
  prefill_mid      the same GEMM at M=256 and 512 (4096x4096), not a configs[] shape
  decode_gemv      GB/s at M=1/4/16 and the SwiGLU shapes (configs[1], [2]), the
                   reference's affine format (u8 codes, scale+bias per 64), and
                   f32 activations (the reference's dtype) at M=1/4/16
  prefill_affine   the dequant-GEMM on affine weights, fp16 and f32 activations
  swiglu           configs[2]: the fused SwiGLU MLP (gate+up pass, then down)
                   at the 7B shape, M=1 and M=8, GB/s of its algorithmic bytes
  decode_tok_s     configs[4]: 1.1B int8 Llama, 512-token prompt, then 128
                   greedy decode steps timed (HIP events), tokens/s; `decode`
                   also holds the batched prefill of that prompt (tokens/s,
                   TFLOPS of its GEMM + attention work) next to the stepwise one;
                   `decode_affine` the same on the reference's affine u8 weights
  ops              the path's other operations, each against its roofline: the
                   reference's two dequantize kernels (4096^2 elements), its f32
                   tiled matmul (k-ascending, bit-exact with the reference's order;
                   configs[0] and 4096^3, the shape the reference publishes:
                   120.71 GFLOPS on an Apple M2), the frozen-weight input gradient
                   and Linear::forward with a LoRA adapter

Algorithmic bytes per GEMV = N*K (codes) + 4*N (scales) + 2*M*K (X) + 2*M*N (Y).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0
COPIES = 96
METRIC = "int8 GEMV GB/s (% HBM peak) at 4096² M=1; prefill TFLOPS; decode tok/s"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemv_bytes(m: int, n: int, k: int) -> int:
    return n * k + 4 * n + 2 * m * k + 2 * m * n


class GemvWorkload:
    """COPIES rotating int8 weights [n, k] plus X [m, k], Y [m, n] fp16.  Per-row
    codes with one f32 scale per row (the configs), or with `affine` the
    reference's format: u8 codes with an f32 scale and bias per 64 elements."""

    def __init__(self, ctx, m: int, n: int, k: int, seed: int = 0, copies: int = COPIES, affine: bool = False,
                 x_f32: bool = False):
        from rusty_amd import DType, UnifiedTensor, _lib, synth

        self.ctx, self.m, self.n, self.k, self.copies = ctx, m, n, k, copies
        g = synth.rng(seed)
        if affine:
            q, s, b = synth.affine_weight(g, n, k, 64)
        else:
            (q, s), b = synth.rowwise_weight(g, n, k), None
        x = synth.activations(g, m, k)
        ns = s.size  # scales (and biases) per copy
        self.codes = UnifiedTensor.empty(ctx, [copies, n, k], DType.U8)
        self.scales = UnifiedTensor.empty(ctx, [copies, ns], DType.FP32)
        self.biases = UnifiedTensor.empty(ctx, [copies, ns], DType.FP32) if affine else None
        first = UnifiedTensor.new(ctx, q.view(np.uint8), dtype=DType.U8)
        fs = UnifiedTensor.new(ctx, s)
        fb = UnifiedTensor.new(ctx, b) if affine else None
        for c in range(copies):
            _lib.call("rq_memcpy_d2d", ctx.handle, self.codes.ptr + c * n * k, first.ptr, n * k, None)
            _lib.call("rq_memcpy_d2d", ctx.handle, self.scales.ptr + c * ns * 4, fs.ptr, ns * 4, None)
            if affine:
                _lib.call("rq_memcpy_d2d", ctx.handle, self.biases.ptr + c * ns * 4, fb.ptr, ns * 4, None)
        ctx.sync()
        self.x_dtype = 0 if x_f32 else 1  # RQ_F32 / RQ_F16: f32 is the reference's activation dtype
        self.x = UnifiedTensor.new(ctx, x.astype(np.float32), dtype=DType.FP32) if x_f32 else \
            UnifiedTensor.new(ctx, x, dtype=DType.FP16)
        self.y = UnifiedTensor.empty(ctx, [m, n], DType.FP16)
        fmt = _lib.RQ_Q_AFFINE_U8 if affine else _lib.RQ_Q_ROWWISE_I8
        self.desc = [_lib.rq_qweight(self.codes.ptr + c * n * k, self.scales.ptr + c * ns * 4,
                                     self.biases.ptr + c * ns * 4 if affine else None, n, k, fmt, 64 if affine else 0)
                     for c in range(copies)]
        self._fn = _lib.lib().rq_qmatmul
        self._h = ctx.handle
        self.bytes = gemv_bytes(m, n, k) + (4 * n * k // 64 * 2 - 4 * n if affine else 0) + (2 * m * k if x_f32 else 0)

    def launch(self, i: int) -> None:
        st = self._fn(self._h, ctypes.byref(self.desc[i % self.copies]), self.x.ptr, self.x_dtype, self.y.ptr, 1,
                      self.m, None)
        if st != 0:
            from rusty_amd import _lib
            _lib.check(st, "rq_qmatmul")


class DeviceClock:
    """Two device timestamps (rq_device_clock: the device's constant-rate wall
    clock stored by a one-wave kernel on the stream) that can sit inside a
    captured graph, around exactly the launches to be timed."""

    def __init__(self, ctx):
        from rusty_amd import DType, UnifiedTensor, _lib

        self.ctx = ctx
        self.buf = UnifiedTensor.new(ctx, np.zeros(2, np.uint64).view(np.uint8), dtype=DType.U8)
        hz = ctypes.c_uint64()
        _lib.call("rq_device_clock", ctx.handle, self.buf.ptr, ctypes.byref(hz), None)
        ctx.sync()
        self.hz = hz.value

    def stamp(self, i: int) -> None:
        from rusty_amd import _lib

        _lib.call("rq_device_clock", self.ctx.handle, self.buf.ptr + 8 * i, None, None)

    def elapsed_ms(self) -> float:
        t = self.buf.to_vec().view(np.uint64)
        return float(int(t[1]) - int(t[0])) / self.hz * 1e3


class ProbeWorkload:
    """The headline GEMV's weight stream without its arithmetic (rq_stream_probe
    over the same rotating copies, same grid: 2 rows of 4096 B per block of
    256 threads, one 16-byte non-temporal load per thread and row); with
    `store`, one 2-byte value per row is written, as the GEMV writes Y."""

    def __init__(self, wl: GemvWorkload, store: bool):
        from rusty_amd import _lib

        self.wl, self.copies, self.store = wl, wl.copies, store
        self._fn = _lib.lib().rq_stream_probe
        self._h = wl.ctx.handle
        self.bytes = wl.n * wl.k + (2 * wl.n if store else 0)

    def launch(self, i: int) -> None:
        wl = self.wl
        st = self._fn(self._h, wl.codes.ptr + (i % self.copies) * wl.n * wl.k, wl.k, wl.n, 2, wl.y.ptr,
                      1 if self.store else 0, None)
        if st != 0:
            from rusty_amd import _lib
            _lib.check(st, "rq_stream_probe")


def floor_probe(ctx, wl: GemvWorkload, steps: int, use_graph: bool = True) -> dict:
    """Mean launch time of the headline GEMV beside the bare read of its weight
    bytes and the read plus its output store, each over the same rotating
    copies and timed the same way: the one-launch floor the GEMV sits on."""
    out = {}
    for name, w in (("gemv", wl), ("read", ProbeWorkload(wl, False)), ("read_store", ProbeWorkload(wl, True))):
        ms, _ = time_steps(ctx, w, steps, wl.copies, use_graph=use_graph)
        out[f"{name}_us"] = round(ms / steps * 1e3, 3)
    out["gemv_over_read_store"] = round(out["gemv_us"] / out["read_store_us"], 4)
    out["read_gbs"] = round(wl.n * wl.k / (out["read_us"] * 1e-6) / 1e9, 1)
    out["what"] = ("16 MiB weight read by rq_stream_probe with the GEMV's grid (2048 blocks x 256 threads, 2 rows "
                   "each), without and with the 8 KB output store, vs the GEMV itself; same copies, same timing")
    return out


def time_steps(ctx, wl, steps: int, warmup: int, use_graph: bool = True):
    """Times exactly `steps` launches on the context stream; returns
    (elapsed ms, description of what the timed region launched).

    Graph mode: one captured graph holds an untimed rotation over all `copies`
    weight copies, a device timestamp, `steps` launches over copies 0, 1, ...
    (mod copies), and a second timestamp.  Both timestamps are kernels on the
    launch stream inside the graph (rq_device_clock), so the timed region is
    exactly the `steps` dispatches, back to back, plus one kernel boundary,
    with neither the graph's launch nor the host in it; the lead-in rotation
    keeps the device at its sustained clock and leaves copy 0 the least
    recently used.  elapsed / steps is the mean kernel duration as well as the
    whole-job time per step.  (HIP events cannot be graph nodes here; events
    around a graph of 20 launches read 5.3 us per launch where 2000 read 4.7,
    the difference being the graph launch's own cost, which time_steps also
    reports as `graph_launch_ms`.)  Direct mode (tracers that do not follow
    graph launches): batches of `copies` launches, each queued behind a device
    delay, between HIP events; the timed region then includes the delays."""
    from rusty_amd.hiprt import Event, Graph

    stream = ctx.stream
    C = wl.copies
    t0, t1 = Event(), Event()
    if use_graph:
        clock = DeviceClock(ctx)
        rotation = Graph(stream, lambda: [wl.launch(i) for i in range(C)])

        def body():
            for i in range(C):
                wl.launch(i)
            clock.stamp(0)
            for i in range(steps):
                wl.launch(i)
            clock.stamp(1)

        timed = Graph(stream, body)
        desc = (f"one HIP graph: an untimed rotation over all {C} weight copies, then {steps} launches over copies "
                f"0, 1, ... (mod {C}) between two device wall-clock stamps on the launch stream")
    else:
        rotation = _Direct(ctx, lambda: [wl.launch(i) for i in range(C)], C)
        q, r = divmod(steps, C)
        batches = [rotation] * q + ([_Direct(ctx, lambda: [wl.launch(i) for i in range(r)], r)] if r else [])
        desc = (f"direct launches in batches of <= {C}, each batch queued behind a device delay, between HIP "
                f"events (for tracers; the timed region includes the delays)")

    # W warm-up steps, and at least 0.25 s of them: the clock ramps out of
    # idle over tens of ms, and the timed steps should see the sustained clock
    for _ in range(max(1, -(-warmup // C))):
        rotation.launch()
    ctx.sync()
    t_end = time.perf_counter() + 0.25
    while time.perf_counter() < t_end:
        rotation.launch()
        ctx.sync()
    t0.record(stream)
    if use_graph:
        timed.launch()
    else:
        for b in batches:
            b.launch()
    t1.record(stream)
    t1.synchronize()
    events_ms = t0.elapsed_ms(t1)
    if not use_graph:
        return events_ms, desc
    time_steps.graph_launch_ms = round(events_ms, 4)  # whole graph launch incl. the rotation, for reference
    return clock.elapsed_ms(), desc


HOST_US_PER_LAUNCH = 80  # generous host cost of one direct launch under a tracer


def device_delay(ctx, us: float) -> None:
    """Queues a bounded device-side wait on the context stream: launches the
    host issues meanwhile line up behind it and then run back to back."""
    from rusty_amd import _lib

    _lib.call("rq_device_delay", ctx.handle, int(min(us, 100000)), None)


class _Direct:
    """Stands in for a captured graph: launch() queues a device delay, then
    issues the calls directly, so they run back to back as from the graph
    (profiling runs whose tracer does not follow graph launches)."""

    def __init__(self, ctx, fn, launches: int):
        self.ctx, self.fn, self.launches = ctx, fn, launches

    def launch(self) -> None:
        device_delay(self.ctx, HOST_US_PER_LAUNCH * self.launches)
        self.fn()


def _replays(ctx, fn, launches: int, use_graph: bool, reps: int = 3) -> list:
    """Elapsed ms of `reps` timed runs of the work `fn` enqueues, after >= 0.25 s
    of warm-up runs.  Graph mode: fn is captured between two device
    wall-clock stamps (rq_device_clock), so each timed run is exactly fn's
    dispatches, back to back, without the graph launch; each run starts after a
    host wait (a burst, as a prompt arrives).  Direct mode: fn's launches
    queued behind a device delay, between HIP events."""
    from rusty_amd.hiprt import Event, Graph

    if use_graph:
        clock = DeviceClock(ctx)

        def body():
            clock.stamp(0)
            fn()
            clock.stamp(1)
        graph = Graph(ctx.stream, body)
    else:
        a, b = Event(), Event()
        graph = _Direct(ctx, lambda: (a.record(ctx.stream), fn(), b.record(ctx.stream)), launches)
    t_end = time.perf_counter() + 0.25
    while time.perf_counter() < t_end:
        graph.launch()
        ctx.sync()
    times = []
    for _ in range(reps):
        graph.launch()
        ctx.sync()
        times.append(clock.elapsed_ms() if use_graph else a.elapsed_ms(b))
    return times


def prefill(ctx, engine, n: int, k: int, m: int = 2048, steps: int = 30, warmup: int = 5,
            use_graph: bool = True, operands: str = "random", affine: bool = False, x_f32: bool = False):
    """configs[3] dequant-GEMM.  `operands` other than "random" (the benchmark
    data) zero the activations or the weight codes: the same kernel and
    instruction stream on data that switches fewer bits, to show how much of
    the time is the chip's power limit (a diagnostic, never the headline).
    `affine`: the reference's weight format (u8 codes, f32 scale and bias per
    64 elements); `x_f32`: f32 activations (the reference's dtype), cast to
    fp16 on the device inside the timed call."""
    from rusty_amd import DType, QuantizedTensor, UnifiedTensor, synth

    g = synth.rng(n + k)
    if affine:
        q, s, b = synth.affine_weight(g, n, k, 64)
    else:
        (q, s), b = synth.rowwise_weight(g, n, k), None
    xa = synth.activations(g, m, k, sigma=0.5, dtype=np.float32 if x_f32 else np.float16)
    if operands == "zero-activations":
        xa = np.zeros_like(xa)
    elif operands == "zero-weights":
        q = np.zeros_like(q)
    w = QuantizedTensor.affine(ctx, q, s, b, 64) if affine else QuantizedTensor.rowwise(ctx, q, s)
    x = UnifiedTensor.new(ctx, xa, dtype=DType.FP32 if x_f32 else DType.FP16)
    y = UnifiedTensor.empty(ctx, [m, n], DType.FP16)
    # the launches are replayed from a HIP graph: back to back on the device,
    # with no host call in between (a Python call per launch costs ~40 us).
    # Warm-up is time-based (>= 0.25 s of replays) so the timed replays run at
    # the sustained clock, not the ramp out of idle; median of 3 replays, each
    # a burst after a host wait (back-to-back replays with no wait measured
    # ~6 % slower at 2048x4096x4096: the MFMA clock is power-limited).
    for _ in range(warmup):
        engine.qmatmul(ctx, x, w, y)
    fn = lambda: [engine.qmatmul(ctx, x, w, y) for _ in range(steps)]  # noqa: E731
    times = _replays(ctx, fn, steps, use_graph)
    times = [t / steps for t in times]
    ms = sorted(times)[1]
    tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    out = {"shape": f"{m}x{n}x{k}", "ms": round(ms, 5), "tflops": round(tflops, 2),
           "frac_of_fp16_peak": round(tflops / FP16_MFMA_PEAK_TFLOPS, 4)}
    if operands != "random":
        out["operands"] = operands
    if affine or x_f32:
        out["weights"] = ("affine u8, scale+bias per 64, scale table prepared at load (rq_qweight_prepare)"
                          if affine else "per-row int8")
        out["activations"] = "f32 (cast on device)" if x_f32 else "fp16"
    return out


def swiglu(ctx, engine, m: int, copies: int = 4, launches: int = 60, use_graph: bool = True) -> dict:
    """y = down(silu(gate.x) * (up.x)), gate/up int8 [11008,4096],
    down int8 [4096,11008], per-row scales; x fp16 [m,4096].  Bytes per MLP =
    3*I*H codes + 4*(2I+H) scales + 2mH (x) + 2*2mI (h written, read) + 4mH (y f32)."""
    from rusty_amd import DType, QuantizedTensor, UnifiedTensor, synth

    I, H = 11008, 4096
    g = synth.rng(2)
    mats = [[QuantizedTensor.rowwise(ctx, *synth.rowwise_weight(g, I, H)),
             QuantizedTensor.rowwise(ctx, *synth.rowwise_weight(g, I, H)),
             QuantizedTensor.rowwise(ctx, *synth.rowwise_weight(g, H, I))] for _ in range(copies)]
    x = UnifiedTensor.new(ctx, synth.activations(g, m, H), dtype=DType.FP16)
    y = UnifiedTensor.empty(ctx, [m, H], DType.FP32)  # |y| ~1e5 at these statistics: past fp16 range
    h = UnifiedTensor.empty(ctx, [2, m, I], DType.FP16)
    for i in range(2 * copies):
        engine.mlp_swiglu(ctx, x, *mats[i % copies], y, h)
    # replayed from a HIP graph (no host call between MLPs), after >= 0.25 s
    # of warm-up replays; median of 3 timed replays
    fn = lambda: [engine.mlp_swiglu(ctx, x, *mats[i % copies], y, h) for i in range(launches)]  # noqa: E731
    times = [t / launches * 1e3 for t in _replays(ctx, fn, 2 * launches, use_graph)]
    us = sorted(times)[1]
    nbytes = 3 * I * H + 4 * (2 * I + H) + 2 * m * H + 2 * 2 * m * I + 4 * m * H
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"m": m, "us_per_mlp": round(us, 2), "gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "bytes": nbytes, "launches": "gate+up pass, down pass (2 kernels)"}


REF_MATMUL_4096_GFLOPS = 120.71  # f32 matmul 4096^3 on an Apple M2, benchmarks/RESULTS.md:21
FP32_PEAK_TFLOPS = 157.3  # MI355X fp32 (packed FMA; one-wide VALU FMA issue gives half)


def ops_bench(ctx, engine, use_graph: bool = True) -> list:
    """The path's remaining operations, each timed like the GEMMs (captured,
    after >= 0.25 s of warm-up replays, median of 3) against its roofline:
      dequantize          a2, kernels.wgsl:153-166: 1 B read + 4 B written per element
      affine_dequantize   a1, kernels.wgsl:379-400: + 8 B (scale, bias) per 64 elements
      matmul_f32          a3, kernels.wgsl:7-54: 2 m k n flops, fp32 VALU; at configs[0]'s few
                          outputs the bound is the k-long dependent fma chain of each output,
                          reported as the one-launch time of one wave's chain of k fmas
      qmatmul_dx          f-4, MatMulNode::backward: dX = dY . deq(W), 2 m n k flops, fp32 VALU
      qmatmul_lora        a7 with an adapter, lib.rs:69-83: the fused product plus (x.A).B
    The dequantize kernels rotate 8 inputs and 4 outputs (384 MB, past the
    256 MB Infinity Cache)."""
    from rusty_amd import DType, QuantizedTensor, UnifiedTensor, _lib, synth

    g = synth.rng(5)
    out = []

    def timed(fn, calls):
        return sorted(t / calls * 1e3 for t in _replays(ctx, fn, calls, use_graph))[1]  # us per call

    probe_out = UnifiedTensor.empty(ctx, [64], DType.FP32)

    def chain_floor(steps):  # us: one launch of one wave's `steps` dependent fmas
        return timed(lambda: [_lib.call("rq_fma_chain_probe", ctx.handle, steps, probe_out.ptr, None)
                              for _ in range(4)], 4)

    n = 4096 * 4096
    words = [UnifiedTensor.new(ctx, g.integers(0, 256, n, dtype=np.uint8), dtype=DType.U8) for _ in range(8)]
    outs = [UnifiedTensor.empty(ctx, [n], DType.FP32) for _ in range(4)]
    fn = lambda: [engine.dequantize(ctx, words[i], outs[i % 4]) for i in range(8)]  # noqa: E731
    us = timed(fn, 8)
    nb = 5 * n
    out.append({"op": "dequantize", "ref": "kernels.wgsl:153-166", "elements": n, "us": round(us, 2),
                "bytes": nb, "gbs": round(nb / us / 1e3, 1), "frac_hbm": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)})
    sc = [UnifiedTensor.new(ctx, g.uniform(0.001, 0.02, n // 64).astype(np.float32)) for _ in range(8)]
    bi = [UnifiedTensor.new(ctx, g.uniform(-2.5, -0.1, n // 64).astype(np.float32)) for _ in range(8)]
    fn = lambda: [engine.affine_dequantize(ctx, words[i], sc[i], bi[i], outs[i % 4]) for i in range(8)]  # noqa: E731
    us = timed(fn, 8)
    nb = 5 * n + 8 * n // 64
    out.append({"op": "affine_dequantize", "ref": "kernels.wgsl:379-400", "elements": n, "us": round(us, 2),
                "bytes": nb, "gbs": round(nb / us / 1e3, 1), "frac_hbm": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)})
    del words, outs, sc, bi

    for m, k, nn, calls in ((8, 1024, 1024, 20), (4096, 4096, 4096, 1)):
        a = UnifiedTensor.new(ctx, g.standard_normal((m, k)).astype(np.float32))
        b = UnifiedTensor.new(ctx, g.standard_normal((k, nn)).astype(np.float32))
        c = UnifiedTensor.empty(ctx, [m, nn], DType.FP32)
        us = timed(lambda: [engine.matmul(ctx, a, b, c) for _ in range(calls)], calls)
        gf = 2 * m * k * nn / us / 1e3
        e = {"op": "matmul_f32", "ref": "kernels.wgsl:7-54", "m": m, "k": k, "n": nn, "us": round(us, 2),
             "gflops": round(gf, 1), "frac_fp32_peak": round(gf / 1e3 / FP32_PEAK_TFLOPS, 4)}
        if (m, k, nn) == (4096, 4096, 4096):
            e["vs_published_m2"] = round(gf / REF_MATMUL_4096_GFLOPS, 1)
        else:
            e["chain_floor_us"] = round(chain_floor(k), 2)
        out.append(e)
        del a, b, c

    w = QuantizedTensor.rowwise(ctx, *synth.rowwise_weight(g, 4096, 4096))
    m = 512
    dy = UnifiedTensor.new(ctx, synth.activations(g, m, 4096), dtype=DType.FP16)
    dx = UnifiedTensor.empty(ctx, [m, 4096], DType.FP32)
    us = timed(lambda: [engine.qmatmul_dx(ctx, dy, w, dx) for _ in range(4)], 4)
    gf = 2 * m * 4096 * 4096 / us / 1e3
    w.dx_table(ctx)  # built once per weight, outside the timed calls
    dws = UnifiedTensor.empty(ctx, [int(_lib.lib().rq_qmatmul_dx_mfma_workspace(m, 4096))], DType.U8)
    us_mfma = timed(lambda: [engine.qmatmul_dx(ctx, dy, w, dx, mfma=True, workspace=dws) for _ in range(4)], 4)
    gf_mfma = 2 * m * 4096 * 4096 / us_mfma / 1e3
    out.append({"op": "qmatmul_dx", "ref": "rusty-autograd/src/lib.rs:152-158", "m": m, "n_out": 4096, "k_in": 4096,
                "us": round(us, 2), "gflops": round(gf, 1), "frac_fp32_peak": round(gf / 1e3 / FP32_PEAK_TFLOPS, 4),
                "us_mfma": round(us_mfma, 2), "gflops_mfma": round(gf_mfma, 1),
                "frac_fp16_peak_mfma": round(2 * gf_mfma / 1e3 / FP16_MFMA_PEAK_TFLOPS, 4),
                "what": "us: f32 fma chain in ascending n_out (the reference's bits); us_mfma: rq_qmatmul_dx_mfma, "
                        "dY . s split into two fp16 halves against the transposed codes (twice the MFMA work of "
                        "one fp16 product; frac_fp16_peak_mfma counts both halves)"})

    rank = 16
    la = UnifiedTensor.new(ctx, (g.standard_normal((4096, rank)) * 0.01).astype(np.float32))
    lb = UnifiedTensor.new(ctx, (g.standard_normal((rank, 4096)) * 0.01).astype(np.float32))
    for m in (1, 512):
        x = UnifiedTensor.new(ctx, synth.activations(g, m, 4096), dtype=DType.FP16)
        y = UnifiedTensor.empty(ctx, [m, 4096], DType.FP16)
        need = max(_lora_workspace(m, 4096, 4096, rank, tree) for tree in (False, True))
        ws = UnifiedTensor.empty(ctx, [need], DType.U8)
        us = timed(lambda: [engine.qmatmul_lora(ctx, x, w, la, lb, y, ws) for _ in range(4)], 4)
        us_tree = timed(lambda: [engine.qmatmul_lora(ctx, x, w, la, lb, y, ws, tree=True) for _ in range(4)], 4)
        base = timed(lambda: [engine.qmatmul(ctx, x, w, y) for _ in range(4)], 4)
        out.append({"op": "qmatmul_lora", "ref": "rusty-graph/src/lib.rs:69-83", "m": m, "n_out": 4096, "k_in": 4096,
                    "rank": rank, "us": round(us, 2), "us_tree": round(us_tree, 2), "us_without_adapter": round(base, 2),
                    "adapter_chain_floor_us": round(chain_floor(4096), 2),
                    "what": "y fp16 = x . deq(W)^T + (x . A) . B; the same weight every call (L2/MALL-resident); "
                            "us: x . A in the reference's k-ascending chain (its bits), us_tree: as a fixed-order "
                            "reduction tree (RQ_LORA_TREE, f32 rounding of the same product)"})
    return out


def _lora_workspace(m, k, n, rank, tree=False):
    from rusty_amd import _lib

    return int(_lib.lib().rq_qmatmul_lora_ex_workspace(m, k, n, rank, 1, 1, _lib.RQ_LORA_TREE if tree else 0))


def decode_loop(ctx, prompt_len: int = 512, steps: int = 128, reps: int = 2, eager: bool = False,
                affine_group: int = 0) -> dict:
    """1.1B int8 Llama greedy decode, from captured HIP graphs (four
    steps per launch, the runner's default).
    Algorithmic bytes per token = int8 codes + f32 scales of every Linear and
    the lm_head + the fp16 KV cache rows attention reads (positions 0..pos,
    once per KV head) + one fp16 embedding row.  With ``affine_group`` every
    Linear is in the reference's affine u8 format (f32 scale and bias per
    group), whose scale and bias bytes count instead."""
    from rusty_amd.hiprt import Event
    from rusty_amd.llama import LLAMA_1B, LlamaRunner, synth_weights

    cfg = LLAMA_1B
    runner = LlamaRunner(ctx, cfg, synth_weights(cfg, seed=0, affine_group=affine_group))
    if eager:
        runner.set_graph(False)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, prompt_len)
    best = best_pf = None
    for _ in range(reps):
        a, b, c = Event(), Event(), Event()
        a.record(ctx.stream)
        runner.prefill(prompt)
        b.record(ctx.stream)
        runner.decode(steps)
        c.record(ctx.stream)
        c.synchronize()
        ms, pf = b.elapsed_ms(c), a.elapsed_ms(b)
        best = ms if best is None else min(best, ms)
        best_pf = pf if best_pf is None else min(best_pf, pf)
    toks = runner.tokens()
    # the same prompt one position at a time through the decode step graph
    runner.set_prefill(0)
    a, b = Event(), Event()
    a.record(ctx.stream)
    runner.prefill(prompt)
    b.record(ctx.stream)
    b.synchronize()
    stepwise_ms = a.elapsed_ms(b)
    runner.close()
    # prefill work as performed: every Linear over the prompt's rows and causal
    # attention (q.k and p.v over positions 0..s for every head) in all but
    # the last layer; there q/k/v over every row (the KV cache), attention for
    # the last query tile of 32 positions, the other Linears for the last row;
    # one lm_head row
    shapes = cfg.linear_shapes()
    lin = sum(n * k for n, k in shapes.values())
    lin_qkv = sum(shapes[nm][0] * shapes[nm][1] for nm in ("q", "k", "v"))
    t0 = 32 * ((prompt_len - 1) // 32)
    attn_pos = 4 * cfg.n_heads * cfg.head_dim  # flops per (query, key) pair
    pf_flops = (2 * prompt_len * lin * (cfg.n_layers - 1) + 2 * prompt_len * lin_qkv + 2 * (lin - lin_qkv)
                + 2 * cfg.vocab * cfg.hidden
                + (cfg.n_layers - 1) * attn_pos * prompt_len * (prompt_len + 1) // 2
                + attn_pos * sum(p + 1 for p in range(t0, prompt_len)))
    kv_row = cfg.n_kv_heads * cfg.head_dim * 2 * 2  # K and V, fp16, one position
    kv = cfg.n_layers * kv_row * sum(prompt_len + i + 1 for i in range(steps)) / steps
    per_tok = cfg.weight_bytes(affine_group) + kv + cfg.hidden * 2
    tok_s = steps / (best * 1e-3)
    gbs = per_tok * tok_s / 1e9
    return {"tok_s": round(tok_s, 1), "ms_per_token": round(best / steps, 4), "bytes_per_token": int(per_tok),
            "gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "config": "1.1B: 22 layers, hidden 2048, 32/4 heads x 64, SwiGLU 5632, vocab 32000; "
                      f"{prompt_len}-token random prompt, {steps} greedy steps timed, best of {reps}",
            "weights": (f"affine u8, f32 scale + bias per {affine_group} (the reference's format)" if affine_group
                        else "per-row int8, f32 scale per row"),
            "launch": ("direct kernel launches" if eager else
                       "captured step graphs: four steps per graph launch, a one-step graph for the rest"),
            "generated_head": [int(t) for t in toks[prompt_len:prompt_len + 8]],
            "prefill": {"tok_s": round(prompt_len / (best_pf * 1e-3), 1), "ms": round(best_pf, 3),
                        "tflops": round(pf_flops / (best_pf * 1e-3) / 1e12, 1),
                        "frac_of_fp16_peak": round(pf_flops / (best_pf * 1e-3) / 1e12 / FP16_MFMA_PEAK_TFLOPS, 4),
                        "stepwise_ms": round(stepwise_ms, 3),
                        "what": f"{prompt_len}-token prompt in one batched chunk ([{prompt_len}, H] GEMMs, causal "
                                "prefill attention, last-row lm_head + greedy pick), token upload included; "
                                "stepwise: the same prompt one position at a time through the step graph"}}


def decode_probe(ctx, prompt_len: int = 512, steps: int = 8) -> dict:
    """The configs[4] runner's kernels for counter passes: the bench's 512-token
    prompt through the batched prefill, then `steps` single decode steps as
    direct launches, one progress line per step (a counter pass serialises
    every dispatch; the full decode loop's ~100k are too slow for that)."""
    from rusty_amd.llama import LLAMA_1B, LlamaRunner, synth_weights

    cfg = LLAMA_1B
    runner = LlamaRunner(ctx, cfg, synth_weights(cfg, seed=0))
    runner.set_graph(False)
    log("decode probe: runner created")
    runner.prefill(np.random.default_rng(1).integers(0, cfg.vocab, prompt_len))
    runner.tokens()
    log("decode probe: prefill done")
    for i in range(steps):
        runner.decode(1)
        runner.tokens()
        log(f"decode probe: step {i + 1}")
    toks = runner.tokens()
    runner.close()
    return {"prompt": prompt_len, "steps": steps, "generated": [int(t) for t in toks[prompt_len:]]}


def traffic_from_profile(kernel: str):
    """HBM bytes per launch of the headline kernel, from the committed rocprofv3
    PMC summary (FETCH_SIZE and WRITE_SIZE passes, each calibrated against a
    plain 16 MiB copy); None if the summary is absent or names another kernel."""
    import pathlib
    import re

    p = pathlib.Path(__file__).resolve().parent / "profiles" / "gemv_decode_m1_4096x4096_pmc.md"
    if not p.exists():
        return None
    text = p.read_text()
    m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", text)
    return int(m.group(1)) if m and kernel in text else None


def cpu_baseline(seconds: float):
    """The reference's per-token Linear step on host cores (oracle port)."""
    from oracle import oracle as orc
    from rusty_amd import synth

    g = synth.rng(0)
    q, s = synth.rowwise_weight(g, 4096, 4096)
    x = synth.activations(g, 1, 4096).astype(np.float32)
    ref = orc.RefLinear(q, s, None, 0)  # load-time dequantization (untimed, as in the reference)
    y = np.empty((1, 4096), np.float32)
    _, threads = ref.forward(x, y)  # warm
    steps, t0 = 0, time.perf_counter()
    while True:
        ref.forward(x, y)
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    gbs = gemv_bytes(1, 4096, 4096) * steps / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": int(threads), "kind": "port",
            "sample": (f"{steps} per-token steps of the reference path (k-ascending f32 fma GEMV on the "
                       f"load-time-dequantized f32 weight, configs[1] shape 4096x4096 M=1) in {el:.1f} s; "
                       f"bytes counted as the int8 algorithmic bytes of the GPU step"),
            "legs": [cpu_leg_config0(seconds / 2), cpu_leg_config3(seconds / 2), cpu_leg_config4(seconds / 2)]}


def cpu_leg_config4(seconds: float) -> dict:
    """configs[4] on host cores: the reference's per-token Linear path
    (load-time f32 dequantization, then matmul_tiled's k-ascending f32 sums at
    M = 1) through one LlamaBlock's seven Linears (q, k, v, o, gate, up, down
    at the 1.1B shape) and the lm_head, each token timed; tokens/s =
    1 / (22 x block + lm_head).  Attention, norms, RoPE and the pick are left
    out (under 1 % of the work at 640 positions)."""
    from oracle import oracle as orc
    from rusty_amd import synth
    from rusty_amd.llama import LLAMA_1B

    cfg = LLAMA_1B
    g = synth.rng(0)
    refs = [orc.RefLinear(*synth.rowwise_weight(g, n, k), None, 0) for n, k in cfg.linear_shapes().values()]
    head = orc.RefLinear(*synth.rowwise_weight(g, cfg.vocab, cfg.hidden), None, 0)
    xs = {k: synth.activations(g, 1, k, dtype=np.float32) for k in {k for _, k in cfg.linear_shapes().values()}}

    def block():
        threads = 1
        for r in refs:
            threads = r.forward(xs[r.k])[1]
        return threads

    block()
    head.forward(xs[cfg.hidden])
    n, tb, t0 = 0, 0.0, time.perf_counter()
    while time.perf_counter() - t0 < seconds * 0.8:
        a = time.perf_counter()
        threads = block()
        tb += time.perf_counter() - a
        n += 1
    nh, th, t1 = 0, 0.0, time.perf_counter()
    while time.perf_counter() - t1 < seconds * 0.2 or nh == 0:
        a = time.perf_counter()
        head.forward(xs[cfg.hidden])
        th += time.perf_counter() - a
        nh += 1
    per_tok = cfg.n_layers * tb / n + th / nh
    return {"config": "configs[4]", "value": round(1.0 / per_tok, 3), "unit": "tok/s", "cores": int(threads),
            "kind": "port",
            "sample": f"one 1.1B block's 7 Linears timed over {n} tokens ({tb / n * 1e3:.1f} ms each) and the "
                      f"lm_head over {nh} ({th / nh * 1e3:.1f} ms each), M = 1, f32 on the load-time-dequantized "
                      f"weights; per token = 22 blocks + lm_head = {per_tok * 1e3:.0f} ms"}


def _timed_forward(ref, x, y, seconds):
    _, threads = ref.forward(x, y)  # warm
    steps, t0 = 0, time.perf_counter()
    while True:
        ref.forward(x, y)
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            return steps, el, threads


def cpu_leg_config0(seconds: float) -> dict:
    """configs[0] on host cores: the reference's Linear (load-time f32
    dequantization, then matmul_tiled's k-ascending f32 sum) at X f32 [8, 1024]
    . W [1024, 1024], GFLOPS of 2 M N K per step."""
    from oracle import oracle as orc
    from rusty_amd import synth

    g = synth.rng(0)
    q, s = synth.rowwise_weight(g, 1024, 1024)
    x = synth.activations(g, 8, 1024, dtype=np.float32)
    ref = orc.RefLinear(q, s, None, 0)
    y = np.empty((8, 1024), np.float32)
    steps, el, threads = _timed_forward(ref, x, y, seconds)
    gf = 2 * 8 * 1024 * 1024 * steps / el / 1e9
    return {"config": "configs[0]", "value": round(gf, 3), "unit": "GFLOPS", "cores": int(threads), "kind": "port",
            "sample": f"{steps} steps of Y f32 [8,1024] = X . deq(W)^T, W int8 [1024,1024] per-row scale, "
                      f"in {el:.1f} s (the whole configs[0] workload per step)"}


def cpu_leg_config3(seconds: float, rows: int = 64) -> dict:
    """configs[3] on host cores: the same reference path at the prefill shape
    (W [4096, 4096]), timed on a bounded sample of the 2048 tokens (``rows``
    of them per step: each output is one k-ascending chain, so the rate per
    token does not depend on how many tokens a step holds); TFLOPS of 2 rows
    N K per step."""
    from oracle import oracle as orc
    from rusty_amd import synth

    g = synth.rng(0)
    q, s = synth.rowwise_weight(g, 4096, 4096)
    x = synth.activations(g, rows, 4096, sigma=0.5, dtype=np.float32)
    ref = orc.RefLinear(q, s, None, 0)
    y = np.empty((rows, 4096), np.float32)
    steps, el, threads = _timed_forward(ref, x, y, seconds)
    tf = 2 * rows * 4096 * 4096 * steps / el / 1e12
    return {"config": "configs[3]", "value": round(tf, 5), "unit": "TFLOPS", "cores": int(threads), "kind": "port",
            "sample": f"{steps} steps of {rows} of the 2048 prefill tokens, X f32 [{rows},4096] . deq(W)^T, "
                      f"W int8 [4096,4096] per-row scale, in {el:.1f} s; the full 2048-token step would take "
                      f"{2048 / rows * el / steps:.1f} s"}


def vendor_gemm(reps: int = 5) -> list:
    """Comparison only: the vendor's fp16 GEMM (torch.matmul, hipBLASLt on this
    image) on the prefill shapes with random fp16 operands and no dequantization,
    Y = X . W^T, 40 launches over 8 weight copies per captured graph, HIP events
    around the graph replay, best of `reps`."""
    import torch

    out = []
    g0 = torch.Generator(device="cuda").manual_seed(0)
    for m, n, k in ((2048, 4096, 4096), (2048, 11008, 4096), (2048, 4096, 11008), (512, 4096, 4096)):
        a = torch.randn(m, k, device="cuda", dtype=torch.float16, generator=g0)
        ws = [torch.randn(n, k, device="cuda", dtype=torch.float16, generator=g0) for _ in range(8)]
        for _ in range(50):
            a @ ws[0].T
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(40):
                a @ ws[i % 8].T
        graph.replay()
        torch.cuda.synchronize()
        best = None
        for _ in range(reps):
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record()
            graph.replay()
            t1.record()
            t1.synchronize()
            ms = t0.elapsed_time(t1) / 40
            best = ms if best is None else min(best, ms)
        tf = 2 * m * n * k / (best * 1e-3) / 1e12
        out.append({"shape": f"{m}x{n}x{k}", "us": round(best * 1e3, 1), "tflops": round(tf, 1),
                    "frac_of_fp16_peak": round(tf / FP16_MFMA_PEAK_TFLOPS, 4),
                    "library": str(torch.backends.cuda.preferred_blas_library())})
        log(f"vendor fp16 GEMM {out[-1]}")
        del a, ws, graph
    return out


GEMV_SHAPES = ((4, 4096, 4096, False, False), (16, 4096, 4096, False, False),
               (1, 11008, 4096, False, False), (8, 11008, 4096, False, False),
               (1, 4096, 11008, False, False), (8, 4096, 11008, False, False),
               (1, 4096, 4096, True, False), (4, 4096, 4096, True, False),
               (16, 4096, 4096, True, False), (1, 4096, 4096, False, True),
               (4, 4096, 4096, False, True), (16, 4096, 4096, False, True))


def decode_gemv_extra(ctx, use_graph: bool = True, shapes=GEMV_SHAPES, reps: int = 20) -> dict:
    """configs[1] at M = 4, 16 and the SwiGLU-shaped GEMVs at M = 1, 8, each
    over enough rotating weight copies to stay out of the Infinity Cache
    (`reps` timed rotations over the copies)."""
    extra = {}
    for m, n, k, aff, xf in shapes:
        copies = max(2, min(COPIES, (1200 << 20) // (n * k)))
        w2 = GemvWorkload(ctx, m, n, k, copies=copies, affine=aff, x_f32=xf)
        wms, _ = time_steps(ctx, w2, reps * copies, 2 * copies, use_graph=use_graph)
        kms = wms / (reps * copies)
        key = f"m{m}_{n}x{k}" + ("_affine" if aff else "") + ("_x_f32" if xf else "")
        extra[key] = {"gbs": round(w2.bytes / (kms * 1e-3) / 1e9, 1), "us_per_launch": round(kms * 1e3, 2),
                      "frac_hbm": round(w2.bytes / (kms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes": w2.bytes}
        if aff:
            extra[key]["weights"] = "affine u8, f32 scale+bias per 64 (the reference's format)"
        if xf:
            extra[key]["activations"] = "f32 (the reference's dtype), kept to f32 accuracy"
        log(f"GEMV {key}: {extra[key]}")
        del w2
    return extra


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--prefill-steps", type=int, default=30)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch every GEMV/prefill/SwiGLU step directly, no HIP graph (for tracers that do not "
                         "follow graph launches; the decode loop has --decode-eager)")
    ap.add_argument("--quick", action="store_true", help="headline GEMV only (for profiling runs)")
    ap.add_argument("--only", choices=["gemv", "gemv_skinny", "prefill", "prefill_affine", "swiglu", "decode",
                                       "decode_probe", "floor", "vendor", "ops"],
                    help="run one extra workload alone, no headline (for profiling runs)")
    ap.add_argument("--prefill-operands", choices=["random", "zero-activations", "zero-weights"], default="random",
                    help="with --only prefill: zero one operand (same kernel, fewer switching bits) to measure "
                         "the power limit; diagnostic only")
    ap.add_argument("--decode-eager", action="store_true",
                    help="decode steps as direct launches instead of graph replays (for tools that "
                         "do not trace graphs)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build's hot path runs on a single MI355X and has no "
              "multi-GPU mode (the path would shard along the weight's output rows, one shard per GPU). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    from rusty_amd import ComputeEngine, WgpuContext

    ctx = WgpuContext(0)
    engine = ComputeEngine(ctx)
    log(f"device 0: {ctx.num_cus} CUs")

    if args.only:
        out = {"only": args.only}
        if args.only == "gemv":
            out["decode_gemv"] = decode_gemv_extra(ctx, use_graph=not args.no_graph)
        elif args.only == "gemv_skinny":  # counter passes: M = 4 and 16 at 4096^2, two rotations each
            out["decode_gemv"] = decode_gemv_extra(ctx, use_graph=not args.no_graph, shapes=GEMV_SHAPES[:2], reps=2)
        elif args.only == "floor":
            out["floor"] = floor_probe(ctx, GemvWorkload(ctx, 1, 4096, 4096), args.steps, use_graph=not args.no_graph)
        elif args.only == "prefill":
            out["prefill"] = [prefill(ctx, engine, n, k, steps=args.prefill_steps, use_graph=not args.no_graph,
                                      operands=args.prefill_operands)
                              for n, k in ((4096, 4096), (11008, 4096), (4096, 11008))]
        elif args.only == "prefill_affine":
            # 4096x4096 at M = 2048: per-row codes, then affine codes with fp16 and f32 activations
            out["prefill"] = [prefill(ctx, engine, 4096, 4096, steps=args.prefill_steps, use_graph=not args.no_graph)]
            out["prefill_affine"] = [prefill(ctx, engine, 4096, 4096, steps=args.prefill_steps, affine=True, x_f32=f,
                                             use_graph=not args.no_graph) for f in (False, True)]
        elif args.only == "decode_probe":
            out["decode_probe"] = decode_probe(ctx)
        elif args.only == "swiglu":
            out["swiglu"] = [swiglu(ctx, engine, m, use_graph=not args.no_graph) for m in (1, 8)]
        elif args.only == "vendor":
            out["vendor_gemm"] = vendor_gemm()
        elif args.only == "ops":
            out["ops"] = ops_bench(ctx, engine, use_graph=not args.no_graph)
        else:
            out["decode"] = decode_loop(ctx, eager=args.decode_eager)
            out["decode_affine"] = decode_loop(ctx, eager=args.decode_eager, affine_group=64)
        log(f"{out}")
        ctx.close()
        print(json.dumps(out), flush=True)
        return 0

    wl = GemvWorkload(ctx, 1, 4096, 4096)
    log("headline: GEMV 4096x4096 M=1, %d rotating copies" % wl.copies)
    wall_ms, launch_desc = time_steps(ctx, wl, args.steps, args.warmup, use_graph=not args.no_graph)
    ms_per_step = wall_ms / args.steps
    value = wl.bytes * args.steps / (wall_ms * 1e-3) / 1e9
    kern_ms = ms_per_step  # back-to-back graph launches: mean launch duration
    achieved = wl.bytes / (kern_ms * 1e-3) / 1e9
    log(f"GEMV M=1: {value:.1f} GB/s whole-job, {kern_ms * 1e3:.3f} us per launch")

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights x fp16 activations, fp32 accumulate",
        "data": "synthetic (seeded numpy PCG64: int8 codes U[-127,127], scales U(0.001,0.02), X ~ N(0,1) fp16)",
        "config": {"workload": (f"configs[1]: decode dequant-GEMV W int8 [4096,4096] per-row f32 scale, "
                                f"X fp16 [1,4096], Y fp16; {wl.copies} weight copies "
                                f"({wl.copies * wl.n * wl.k / 1e9:.2f} GB > 256 MB MALL), timed steps "
                                f"touch min(steps, {wl.copies}) of them"),
                   "m": 1, "n": 4096, "k": 4096, "bytes_per_step": wl.bytes, "launch": launch_desc},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profile("k_gemv_decode<M=1,CPT=1,TPR=256,R=2,ROWWISE>"),
                     "traffic_profile": "profiles/gemv_decode_m1_4096x4096_pmc.md (FETCH_SIZE + WRITE_SIZE passes, copy-kernel calibrated)",
                     "kernel": "k_gemv_decode<M=1,CPT=1,TPR=256,R=2,ROWWISE>",
                     "mean_launch_us": round(kern_ms * 1e3, 3),
                     "timing": ("device wall clock (rq_device_clock, 100 MHz) stamped on the launch stream "
                                "before and after the timed launches inside one graph, / steps"
                                if not args.no_graph else "HIP events around the timed region / steps"),
                     "graph_launch_ms_with_events": getattr(time_steps, "graph_launch_ms", None)},
    }

    result["floor"] = floor_probe(ctx, wl, args.steps, use_graph=not args.no_graph)
    log(f"floor {result['floor']}")
    if not args.quick:
        result["decode_gemv"] = decode_gemv_extra(ctx)
        pf = []
        for n, k in ((4096, 4096), (11008, 4096), (4096, 11008)):
            pf.append(prefill(ctx, engine, n, k, steps=args.prefill_steps))
            log(f"prefill {pf[-1]}")
        result["prefill"] = pf
        # mid-size m (a short prompt, or a batch of decode streams): not a configs[] shape
        result["prefill_mid"] = [prefill(ctx, engine, 4096, 4096, m=m, steps=args.prefill_steps) for m in (256, 512)]
        log(f"prefill (mid-size m) {result['prefill_mid']}")
        # the reference's own inputs: affine u8 weights (MLX, group 64), fp16 and f32 activations
        result["prefill_affine"] = [prefill(ctx, engine, 4096, 4096, steps=args.prefill_steps, affine=True, x_f32=f)
                                    for f in (False, True)]
        log(f"prefill (affine weights) {result['prefill_affine']}")
        sw = [swiglu(ctx, engine, m) for m in (1, 8)]
        for e in sw:
            log(f"swiglu {e}")
        result["swiglu"] = sw
        dec = decode_loop(ctx, eager=args.decode_eager)
        log(f"decode {dec}")
        result["decode_tok_s"] = dec["tok_s"]
        result["prefill_tok_s"] = dec["prefill"]["tok_s"]
        result["decode"] = dec
        # configs[4] on the reference's own weight format (affine u8, group 64)
        result["decode_affine"] = decode_loop(ctx, affine_group=64)
        log(f"decode (affine weights) {result['decode_affine']}")
        result["ops"] = ops_bench(ctx, engine)
        for e in result["ops"]:
            log(f"op {e}")

    if not args.no_cpu_baseline:
        log(f"CPU baseline (~{args.cpu_seconds:.0f} s)")
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    ctx.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
