#!/usr/bin/env python3
"""Benchmark of the GPTQ int4 quantized-linear hot path on one MI355X.

Headline (BASELINE.json metric): microseconds per Qwen2.5-0.5B-shaped decode step - the 168 GPTQ
int4 linears (24 layers x q,k,v,o,gate,up,down; group 128) at M = 1, each on its own fp32
activations ~N(0,1) as the benchmark config states them, weights resident in HBM, issued as ONE
persistent launch (ql_seq_create over a strip plan); one step = one ql_seq_run, issued back to
back on the context stream (a one-launch graph replay measured 4.9 us slower per step: the
replay's own dispatch gap). Inputs are synthetic (random nibbles, zero 8, fp16 scales |N(0,1)|*0.01,
x ~ N(0,1)); no checkpoint is available offline.

Also measured (reported under "extra"): the same step after a read-only pass over 1 GiB has
evicted the 256 MB MALL; the linears chained through their outputs (one launch, device-ordered
passes) and as per-linear launches; the 7B-shaped step (140 linears, 3.34 GB, HBM-bound) at
M = 1, 2, 4, 8, 16; the M sweep {1,2,4,8,16}; prefill GEMM at M = 128, 512 (TFLOP/s); the
load-time unpack of all 168 tensors; the lm_head GEMV, elementwise ops and decode attention.
The CPU baseline is the reference CPU path (dequantizeGptqInt4 + gemmNTRef) restated for Node and
run single-threaded on this host over all 168 linears of the timed step on the same inputs, every
output checked against the GPU's; --only cpu runs the rest of the CPU plan (config 1 with the GPU
beside it, variant (ii), config 4 as one 7B layer x28, config 5's fp16 unpack).
"""
from __future__ import annotations

import argparse
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from webllm_amd import qlinear as ql  # noqa: E402
from webllm_amd import synth  # noqa: E402

METRIC = "int4 dequant-GEMV µs per Qwen-0.5B decode step; achieved HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
SEQ_KERNEL_NAMES = {ql.SEQ_TILES: "tiles", ql.SEQ_STRIPS: "strips", ql.SEQ_PREFILL: "prefill",
                    ql.SEQ_STRIP_PASSES: "strip_passes", ql.SEQ_PREFILL_PASSES: "prefill_passes"}
F16_PEAK_TFLOPS = 2500.0
GROUP = 128

LAYER_LAUNCHES_05B = [("q", "k", "v"), ("o",), ("gate", "up"), ("down",)]
LAYER_LAUNCHES_7B = [("q",), ("o",), ("gate", "up"), ("down",)]
# one layer of a linear sequence: (proj, the proj whose output it reads; None = the layer input)
SEQ_LAYER_05B = [("q", None), ("k", None), ("v", None), ("o", "q"), ("gate", "o"), ("up", "o"),
                 ("down", "gate")]
SEQ_LAYER_7B = [("q", None), ("o", "q"), ("gate", "o"), ("up", "o"), ("down", "gate")]
NORM_EPS = 1e-6          # Qwen2.5's rms_norm_eps


def step_inputs(shape: str, M: int, chained: bool) -> list[tuple[int, int, tuple]]:
    """The external inputs SeqStep writes, in its order, as (linear index, K, synth key): the
    first linear's input (the layer-0 residual stream when chained) has key (0, 0, M); in the step
    as written (chained=False) every further linear has an input of its own, key (layer + 1, i, M)
    for linear i of each layer. Host only; tests/golden/make_digests.py hashes the same list."""
    seq = SEQ_LAYER_05B if shape == "0.5b" else SEQ_LAYER_7B
    K = {p: k for p, k, _ in (synth.PROJ_05B if shape == "0.5b" else synth.PROJ_7B)}
    layers = synth.QWEN05_LAYERS if shape == "0.5b" else synth.QWEN7_LAYERS
    out = [(0, K[seq[0][0]], (0, 0, M))]
    if not chained:
        for layer in range(layers):
            for i, (proj, _) in enumerate(seq):
                n = layer * len(seq) + i
                if n > 0:
                    out.append((n, K[proj], (layer + 1, i, M)))
    return out


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def linear_bytes(K, N, M):
    """Algorithmic HBM bytes of one linear: packed weights, zeros, scales, x and y."""
    return K * N // 2 + K * N // 256 + K * N // 64 + M * K * 4 + M * N * 4


class Model:
    """All linears of one model shape packed into a single weight arena."""

    def __init__(self, ctx, shape: str, seed: int, keep_tensors: bool = False):
        """keep_tensors: keep every linear's host tensors (self.tensors[(layer, proj)]) for a
        full-size check against the oracle; otherwise only layer 0's are kept."""
        self.shape = shape
        self.seed = seed
        self.linears = synth.model_linears(shape)
        self.layers = synth.QWEN05_LAYERS if shape == "0.5b" else synth.QWEN7_LAYERS
        lay = ql.ArenaLayout()
        self.descs = {}
        self.tensors_for_cpu = {}
        self.tensors = {}
        plan = []
        for (layer, proj, K, N) in self.linears:
            qw, qz, sc = ql.gptq_sizes(K, N, GROUP)
            offs = (lay.take(qw), lay.take(qz), lay.take(sc))
            plan.append((layer, proj, K, N, offs))
        # the layers' RMSNorm weights (before q/k/v and before gate/up), fp32 [C] each:
        # 1 + 0.1 N(0,1) stands in for trained values near 1
        C = self.linears[0][2]
        self.norm_offs = {(layer, k): lay.take(C * 4) for layer in range(self.layers) for k in range(2)}
        self.arena = ctx.arena(lay.used)
        for (layer, k), off in self.norm_offs.items():
            w = 1.0 + 0.1 * synth.activations(1, C, seed=seed + 3, key=(layer, k))[0]
            self.arena.write(off, w.astype(np.float32))
        self.weight_bytes = 0
        for (layer, proj, K, N, offs) in plan:
            t = synth.gptq_linear(K, N, GROUP, seed=seed, key=(layer, synth.PROJ_INDEX[proj]))
            self.arena.write(offs[0], t.qweight)
            self.arena.write(offs[1], t.qzeros)
            self.arena.write(offs[2], t.scales)
            self.weight_bytes += t.nbytes
            self.descs[(layer, proj)] = ql.make_desc(offs[0], offs[1], offs[2], K, N, GROUP)
            if layer == 0:
                self.tensors_for_cpu[proj] = t
            if keep_tensors:
                self.tensors[(layer, proj)] = t
        self.shapes = {(l, p): (K, N) for (l, p, K, N) in self.linears}


class Step:
    """One decode (or prefill) step over a Model: launch groups, activations, scratch, graph.

    layered=True issues each layer's linears as the model's dependencies allow (q,k,v | o |
    gate,up | down: one launch per group, each group on one input). layered=False is the
    benchmark config as written: every linear on its own input, so any 8 of them can share a
    launch (ql_linear_batch), 8 consecutive linears per launch."""

    def __init__(self, ctx, model: Model, M: int, x_dtype: int = ql.DTYPE_F32, seed: int = 0x5EED,
                 layered: bool = True):
        self.ctx, self.model, self.M, self.x_dtype = ctx, model, M, x_dtype
        groups = LAYER_LAUNCHES_05B if model.shape == "0.5b" else LAYER_LAUNCHES_7B
        es = 4 if x_dtype == ql.DTYPE_F32 else 2
        lay = ql.ArenaLayout()
        self.launches = []
        if layered:
            for layer in range(model.layers):
                for gi, projs in enumerate(groups):
                    descs = [model.descs[(layer, p)] for p in projs]
                    K = descs[0].K
                    x_off = lay.take(M * K * es)
                    y_offs = [lay.take(M * d.N * 4) for d in descs]
                    scratch = ql.plan_batch(descs, M)
                    s_off = lay.take(max(scratch, 16))
                    self.launches.append((layer, gi, projs, descs, [x_off] * len(descs), y_offs, s_off))
        else:
            keys = [(l, p) for (l, p, _, _) in model.linears]
            for b0 in range(0, len(keys), 8):
                part = keys[b0:b0 + 8]
                descs = [model.descs[k] for k in part]
                x_offs = [lay.take(M * d.K * es) for d in descs]
                y_offs = [lay.take(M * d.N * 4) for d in descs]
                s_off = lay.take(max(ql.plan_batch(descs, M), 16))
                self.launches.append((b0, 0, [p for (_, p) in part], descs, x_offs, y_offs, s_off))
        self.act = ctx.arena(lay.used)
        for (layer, gi, projs, descs, x_offs, _, _) in self.launches:
            for i, x_off in enumerate(x_offs if not layered else x_offs[:1]):
                x = synth.activations(M, descs[i].K, seed=seed, key=(layer, gi, M, i))
                if x_dtype == ql.DTYPE_F16:
                    x = x.astype(np.float16).view(np.uint16)
                self.act.write(x_off, x)
        self.bytes = sum(linear_bytes(model.shapes[(l, p)][0], model.shapes[(l, p)][1], M)
                         for (l, p, _, _) in model.linears)
        self.flops = sum(2 * M * K * N for (_, _, K, N) in model.linears)
        self.graph = None

    def issue(self):
        for (_, _, projs, descs, x_offs, y_offs, s_off) in self.launches:
            if len(descs) == 1:
                self.ctx.linear(descs[0], self.model.arena, self.act, x_offs[0], self.x_dtype, self.M,
                                y_offs[0], s_off)
            else:
                self.ctx.linear_batch(descs, self.model.arena, self.act, x_offs,
                                      self.x_dtype, self.M, y_offs, s_off)

    def capture(self):
        self.issue()                      # eager run first (validates every launch)
        self.ctx.sync()
        self.ctx.graph_begin()
        self.issue()
        self.graph = self.ctx.graph_end()

    def run(self, steps: int) -> float:
        """Issues `steps` graph replays between two events; returns total milliseconds."""
        self.ctx.sync()
        self.ctx.timer_start()
        for _ in range(steps):
            self.graph.launch()
        return self.ctx.timer_stop()

    def release(self):
        if self.graph:
            self.graph.destroy()
        self.act.release()


class SeqStep:
    """A step of the model's linears as one sequence (ql_seq_*), enqueued by one ql_seq_run.

    chained=False: the benchmark config as written, every linear on its own input (one strip
    launch at M <= 16, one prefill launch above).
    chained=True: the layer's data flow (src/model/qwen.ts:398-482) with its elementwise work
    folded in (ql_seq_create_fused): q/k/v <- rmsnorm(h); h1 = h + o(q) (o reads q in
    attention's place); gate/up <- rmsnorm(h1); h2 = h1 + down(silu(gate) * up); the next
    layer's h = h2. Each linear runs after what it reads, as after a pass break in the reference
    (qwen.ts:556-559): on the device inside one persistent launch (dependency-ordered tiles), or
    pass by pass in stream order (streamed weights at M = 2..16: K-part strips and part sums;
    M > 16: one GEMM launch per pass); info.kernel says which, info.launches how many."""

    def __init__(self, ctx, model: Model, M: int, seed: int = 0x5EED, chained: bool = True):
        self.ctx, self.model, self.M, self.x_dtype = ctx, model, M, ql.DTYPE_F32
        self.chained = chained
        lay = ql.ArenaLayout()
        descs, xs, ys = [], [], []
        self.order = []
        ext = {n: (K, key) for n, K, key in step_inputs(model.shape, M, chained)}
        inputs = []          # (offset, K, key) of every externally written input, in ext's order
        C = model.shapes[(0, "q")][0]
        h0 = lay.take(M * C * 4)
        inputs.append((h0,) + ext[0])
        h = h0
        fuse = []
        for layer in range(model.layers):
            y = {}
            for i, (proj, src) in enumerate(SEQ_LAYER_05B if model.shape == "0.5b" else SEQ_LAYER_7B):
                d = model.descs[(layer, proj)]
                if chained:
                    if proj in ("q", "k", "v"):
                        x_off = h
                        fuse.append(ql.make_fuse(norm_w_off=model.norm_offs[(layer, 0)], norm_eps=NORM_EPS))
                    elif proj == "o":
                        x_off = y["q"]
                        fuse.append(ql.make_fuse(res_off=h))
                    elif proj in ("gate", "up"):
                        x_off = y["o"]
                        fuse.append(ql.make_fuse(norm_w_off=model.norm_offs[(layer, 1)], norm_eps=NORM_EPS))
                    else:
                        x_off = y["gate"]
                        fuse.append(ql.make_fuse(x2_off=y["up"], res_off=y["o"]))
                else:
                    # the benchmark configs as written: every linear has its own x ~ N(0,1)
                    n = len(self.order)
                    x_off = h0 if n == 0 else lay.take(M * d.K * 4)
                    if n > 0:
                        assert ext[n][0] == d.K
                        inputs.append((x_off,) + ext[n])
                y[proj] = lay.take(M * d.N * 4)
                descs.append(d)
                xs.append(x_off)
                ys.append(y[proj])
                self.order.append((layer, proj))
            h = y["down"]
        self.act = ctx.arena(lay.used)
        for off, K, key in inputs:
            self.act.write(off, synth.activations(M, K, seed=seed, key=key))
        self.x_offs, self.y_offs = xs, ys
        self.fuse = fuse if chained else None
        self.seq = ctx.seq(descs, model.arena, self.act, xs, ql.DTYPE_F32, M, ys, fuse=self.fuse)
        self.info = self.seq.info
        self.bytes = sum(linear_bytes(model.shapes[lp][0], model.shapes[lp][1], M) for lp in self.order)
        self.flops = sum(2 * M * model.shapes[lp][0] * model.shapes[lp][1] for lp in self.order)
        # layer-0 view for the CPU baseline: (layer, group, projs, descs, x_off, y_offs, scratch)
        self.launches = []
        for i, (layer, proj) in enumerate(self.order):
            if layer == 0:
                self.launches.append((0, i, (proj,), [descs[i]], xs[i], [ys[i]], 0))
        self.graph = None

    def capture(self):
        self.seq.run()
        self.seq.status()
        self.ctx.graph_begin()
        self.seq.run()
        self.graph = self.ctx.graph_end()

    def finite(self) -> bool:
        """Every output of the last run is finite (a chained step carries its values across all
        layers)."""
        self.ctx.sync()
        return all(bool(np.isfinite(self.act.read(yo, (self.M, self.model.shapes[lp][1]), np.float32)).all())
                   for yo, lp in zip(self.y_offs, self.order))

    def kernel_ms(self, reps: int, per_graph: int = 10) -> float:
        """Device time per launch with the replay gap amortized: a graph of `per_graph`
        consecutive launches, replayed and timed with HIP events on the context stream."""
        self.ctx.graph_begin()
        for _ in range(per_graph):
            self.seq.run()
        g = self.ctx.graph_end()
        g.launch()
        self.ctx.sync()
        self.ctx.timer_start()
        n = max(1, reps // per_graph)
        for _ in range(n):
            g.launch()
        ms = self.ctx.timer_stop() / (n * per_graph)
        self.seq.status()
        g.destroy()
        return ms

    def run(self, steps: int) -> float:
        """`steps` launches issued directly (ql_seq_run) between two events; total milliseconds.
        A persistent launch needs no graph: replaying a one-launch graph only adds its own
        dispatch gap."""
        self.ctx.sync()
        self.ctx.timer_start()
        for _ in range(steps):
            self.seq.run()
        ms = self.ctx.timer_stop()
        self.seq.status()
        return ms

    def release(self):
        if self.graph:
            self.graph.destroy()
        self.seq.destroy()
        self.act.release()


class PrefillStep:
    """The prefill step as configured (config 3): all linears of the model, each on its own fp16
    activations [M, K] ~ N(0,1), as ONE persistent prefill GEMM launch (ql_seq_* at M > 16: tasks
    of 128 x 256 output tiles over all of K, planned longest first onto one workgroup per CU).
    x_dtype=DTYPE_F32: the same activations as fp32, rounded to fp16 inside the launch as the
    reference's gemm_nt_f16_from_f32.wgsl does."""

    def __init__(self, ctx, model: Model, M: int, seed: int = 0x5EED, x_dtype: int = ql.DTYPE_F16):
        self.ctx, self.model, self.M = ctx, model, M
        lay = ql.ArenaLayout()
        descs, xs, ys = [], [], []
        self.order = []
        es = 4 if x_dtype == ql.DTYPE_F32 else 2
        for (layer, proj, K, N) in model.linears:
            descs.append(model.descs[(layer, proj)])
            xs.append(lay.take(M * K * es))
            ys.append(lay.take(M * N * 4))
            self.order.append((layer, proj))
        self.act = ctx.arena(lay.used)
        for i, (layer, proj) in enumerate(self.order):
            K = model.shapes[(layer, proj)][0]
            x = synth.activations(M, K, seed=seed, key=(layer, synth.PROJ_INDEX[proj], M))
            self.act.write(xs[i], x if es == 4 else x.astype(np.float16).view(np.uint16))
        self.x_offs, self.y_offs = xs, ys
        self.seq = ctx.seq(descs, model.arena, self.act, xs, x_dtype, M, ys)
        self.info = self.seq.info
        self.flops = sum(2 * M * model.shapes[lp][0] * model.shapes[lp][1] for lp in self.order)
        self.graph = None

    capture = SeqStep.capture
    kernel_ms = SeqStep.kernel_ms
    run = SeqStep.run
    release = SeqStep.release


def timed(step, steps: int, warmup: int) -> float:
    if step.graph is None and not isinstance(step, (SeqStep, PrefillStep)):
        step.capture()      # launch groups replay as one graph; a persistent launch runs directly
    if warmup:
        step.run(warmup)
    return step.run(steps) / steps


def flushed_step_ms(ctx, step: Step, reps: int = 5) -> float:
    """Step time with the MALL (256 MB) evicted first by a read-only pass: an fp16 GEMV over a
    1 GiB matrix (1 GiB read, 512 KB written) precedes each step, so the step starts with none of
    its weights cached and no dirty lines left to write back while it runs."""
    N, K = 131072, 4096
    flush = ctx.arena(N * K * 2)
    fx = ctx.arena(K * 4 + N * 4 + 256)
    y_off = (K * 4 + 255) // 256 * 256
    fx.write(0, np.zeros(K, np.float32))
    times = []
    for _ in range(reps):
        ctx.gemv_f16w(flush, 0, None, fx, 0, 1, N, K, y_off)
        ctx.sync()
        times.append(step.run(1))
    fx.release()
    flush.release()
    return float(np.median(times))


def unpack_all(ctx, model: Model, steps: int):
    lay = ql.ArenaLayout()
    offs = {k: lay.take(d.N * d.K * 2) for k, d in model.descs.items()}
    out = ctx.arena(lay.used)

    keys = list(model.descs)
    descs = [model.descs[k] for k in keys]
    out_offs = [offs[k] for k in keys]

    def issue():
        # the whole weight set through the batched entry point (six launches of 28 tensors)
        ctx.unpack_f16_batch(descs, model.arena, out, out_offs)

    issue()
    ctx.sync()
    ctx.graph_begin()
    issue()
    g = ctx.graph_end()
    g.launch()
    ctx.sync()
    ctx.timer_start()
    for _ in range(steps):
        g.launch()
    ms = ctx.timer_stop() / steps
    g.destroy()
    out.release()
    read = model.weight_bytes
    write = sum(d.N * d.K * 2 for d in model.descs.values())
    return ms, read + write


def node_run(items, min_seconds: float, plan=None):
    """The reference CPU path (oracle/js/gptq_ref.js, Node, one thread) over the linears in
    items [(tensors, x [M, K] f32)]: returns its timing record and the outputs y [M, N]."""
    node = shutil.which("node")
    if not node:
        raise RuntimeError("node not found: the CPU baseline runs the reference path under Node")
    with tempfile.TemporaryDirectory() as d:
        meta = {"linears": [], "plan": plan or {}}
        for i, (t, x) in enumerate(items):
            t.qweight.tofile(os.path.join(d, f"qw_{i}"))
            t.qzeros.tofile(os.path.join(d, f"qz_{i}"))
            t.scales.tofile(os.path.join(d, f"sc_{i}"))
            np.ascontiguousarray(x, dtype=np.float32).tofile(os.path.join(d, f"x_{i}"))
            meta["linears"].append({"K": t.K, "N": t.N, "group": GROUP, "M": x.shape[0],
                                    "qweight": f"qw_{i}", "qzeros": f"qz_{i}", "scales": f"sc_{i}",
                                    "x": f"x_{i}"})
        json.dump(meta, open(os.path.join(d, "meta.json"), "w"))
        r = subprocess.run([node, os.path.join(ROOT, "oracle", "js", "gptq_ref.js"), d, str(min_seconds)],
                           capture_output=True, text=True, timeout=1200)
        if r.returncode != 0:
            raise RuntimeError(f"node baseline failed: {r.stderr[-2000:]}")
        res = json.loads(r.stdout.strip().splitlines()[-1])
        ys = [np.fromfile(os.path.join(d, f"y_{i}.f32"), dtype=np.float32).reshape(x.shape[0], t.N)
              for i, (t, x) in enumerate(items)]
    return res, ys


def gpu_cpu_check(gpu_y, cpu_y, xs):
    """|d| <= atol + 1e-4 |ref| with atol = 1e-5 * rms(x) (the reference's 1e-5 for N(0,1)
    inputs); returns (ok, the largest |d| / (atol / 1e-4 + |ref|))."""
    ok, worst = True, 0.0
    for g, c, x in zip(gpu_y, cpu_y, xs):
        a = 1e-5 * max(1.0, float(np.sqrt(np.mean(x.astype(np.float64) ** 2))))
        d = np.abs(g - c)
        ok = ok and bool(np.all(d <= a + 1e-4 * np.abs(c)))
        worst = max(worst, float(np.max(d / (a / 1e-4 + np.abs(c)))))
    return ok, worst


def step_items(model: Model, step):
    """(tensors, x) of every linear of a step, the tensors regenerated from the model's seed."""
    items = []
    for i, (layer, proj) in enumerate(step.order):
        K, N = model.shapes[(layer, proj)]
        t = synth.gptq_linear(K, N, GROUP, seed=model.seed, key=(layer, synth.PROJ_INDEX[proj]))
        items.append((t, step.act.read(step.x_offs[i], (step.M, K), np.float32)))
    return items


def cpu_baseline(model: Model, step, min_seconds: float):
    """The reference CPU path on config 2 in full: all 168 linears of the timed step on the same
    inputs (weights dequantized once, as the reference loads them; the matvecs timed), every
    output checked against the GPU's."""
    items = step_items(model, step)
    res, cpu_y = node_run(items, min_seconds)
    gpu_y = [step.act.read(step.y_offs[i], (step.M, t.N), np.float32) for i, (t, _) in enumerate(items)]
    ok, rel = gpu_cpu_check(gpu_y, cpu_y, [x for _, x in items])
    macs = res["macs"]
    return {
        "value": round(res["matvec_median_ms"] * 1e3, 1), "unit": "us/step", "cores": 1, "kind": "port",
        "sample": (f"config 2 in full: all {len(items)} linears ({macs/1e6:.1f} M MACs) of the timed step "
                   f"on its inputs, variant (i) (weights dequantized once, {res['dequant_ms']:.0f} ms, as "
                   f"the reference loads them; matvecs timed): median of {res['reps']} steps; Node "
                   f"{res['node']} restatement of quant.ts dequantizeGptqInt4 + qwen-ref.ts gemmNTRef"),
        "mean_us": round(res["matvec_ms"] * 1e3, 1),
        "host_cpu": res.get("cpu", ""), "host_threads": res.get("cpus"),
        "dequant_ms": round(res["dequant_ms"], 1),
        "gpu_vs_cpu_ok": bool(ok), "gpu_vs_cpu_max_rel_atol": rel, "linears_checked": len(items),
    }


def cpu_plan(ctx, min_seconds: float):
    """The CPU baseline plan beyond the headline: config 1 in full with the GPU beside it,
    config 2 variant (ii), config 4 (one 7B layer, extrapolated x28) and config 5 (the fp16
    unpack of all 168 tensors)."""
    out = {}
    # config 1: the 0.5B gate_proj shape alone, M = 1
    K, N = 896, 4864
    t = synth.gptq_linear(K, N, GROUP, seed=0xC0F1, key=(0,))
    x = synth.activations(1, K, seed=0xC0F2, key=(0,))
    res, cpu_y = node_run([(t, x)], min(min_seconds, 3.0), {"fused_reps": 9})
    wl, al = ql.ArenaLayout(), ql.ArenaLayout()
    offs = (wl.take(t.qweight.nbytes), wl.take(t.qzeros.nbytes), wl.take(t.scales.nbytes))
    xo, yo = al.take(K * 4), al.take(N * 4)
    so = al.take(max(ql.plan_linear(1, N, K, GROUP).scratch_bytes, 16))
    w = ctx.arena(wl.used)
    act = ctx.arena(al.used)
    w.write(offs[0], t.qweight)
    w.write(offs[1], t.qzeros)
    w.write(offs[2], t.scales)
    act.write(xo, x)
    desc = ql.make_desc(offs[0], offs[1], offs[2], K, N, GROUP)
    ctx.linear(desc, w, act, xo, ql.DTYPE_F32, 1, yo, so)
    ctx.sync()
    ctx.graph_begin()
    ctx.linear(desc, w, act, xo, ql.DTYPE_F32, 1, yo, so)
    g = ctx.graph_end()
    for _ in range(5):
        g.launch()
    ctx.timer_start()
    for _ in range(200):
        g.launch()
    gpu_us = ctx.timer_stop() / 200 * 1e3
    gy = act.read(yo, (1, N), np.float32)
    g.destroy()
    w.release()
    act.release()
    ok, rel = gpu_cpu_check([gy], cpu_y, [x])
    nbytes = linear_bytes(K, N, 1)
    out["config1"] = {"gpu_us": round(gpu_us, 2), "gpu_gbs": round(nbytes / (gpu_us * 1e-6) / 1e9, 1),
                      "cpu_matvec_us": round(res["matvec_median_ms"] * 1e3, 1),
                      "cpu_dequant_ms": round(res["dequant_ms"], 2),
                      "cpu_fused_us": round(res["fused_ms"] * 1e3, 1), "gpu_vs_cpu_ok": ok,
                      "gpu_vs_cpu_max_rel_atol": rel,
                      "note": "gate 896->4864, M=1, one ql_linear launch (graph-replayed, 200 reps); CPU "
                              "variant (i) matvec median and variant (ii) dequant+matvec median of 9"}
    # config 2 variant (ii) and config 5: the 168 linears of the 0.5B step
    m05 = Model(ctx, "0.5b", seed=0x9EF0)
    items = []
    for (layer, proj, K, N) in m05.linears:
        items.append((synth.gptq_linear(K, N, GROUP, seed=m05.seed, key=(layer, synth.PROJ_INDEX[proj])),
                      synth.activations(1, K, seed=0x5EED, key=(layer, synth.PROJ_INDEX[proj], 1))))
    m05.arena.release()
    res, _ = node_run(items, 1.0, {"fused_reps": 3, "f16_reps": 3})
    out["config2_variant_ii"] = {"us": round(res["fused_ms"] * 1e3, 1),
                                 "variant_i_us": round(res["matvec_median_ms"] * 1e3, 1),
                                 "dequant_ms": round(res["dequant_ms"], 1),
                                 "note": "all 168 linears, dequant + matvec per call, median of 3"}
    out["config5"] = {"cpu_ms": round(res["f16_ms"], 1),
                      "note": "dequantizeGptqInt4 + f32ToF16Bits of all 168 tensors ([N,K] fp16), median of 3"}
    del items
    # config 4: one 7B-shaped layer (q, o 3584->3584; gate, up 3584->18944; down 18944->3584)
    items = []
    for (layer, proj, K, N) in synth.model_linears("7b"):
        if layer == 0:
            items.append((synth.gptq_linear(K, N, GROUP, seed=0x7B, key=(0, synth.PROJ_INDEX[proj])),
                          synth.activations(1, K, seed=0x5EED, key=(0, synth.PROJ_INDEX[proj], 1))))
    L7 = synth.QWEN7_LAYERS
    res, _ = node_run(items, min(min_seconds, 5.0), {"fused_reps": 3})
    out["config4_m1_extrapolated"] = {
        "us": round(res["matvec_median_ms"] * 1e3 * L7, 1),
        "variant_ii_us": round(res["fused_ms"] * 1e3 * L7, 1),
        "dequant_ms": round(res["dequant_ms"] * L7, 1),
        "layer_us": round(res["matvec_median_ms"] * 1e3, 1), "layers": L7,
        "note": f"one layer's {len(items)} linears timed in full (variant (i) median, variant (ii) median of 3), "
                f"x{L7} layers: extrapolated"}
    out["host_cpu"] = res.get("cpu", "")
    out["cores"] = 1
    out["node"] = res.get("node", "")
    return out


def traffic_from_profiles(workload: str):
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(p):
        return None
    return json.load(open(p)).get(workload)


def blas_reference(steps: int) -> dict:
    """hipBLASLt's fp16 GEMM (torch.matmul, fp32 accumulation) on the 0.5B prefill shapes, beside
    prefill_kernel: the 168 linears at M = 128 and 512 as dense fp16 weights (one library call
    each, graph-replayed; the library's rate per call on these shapes) and one 8192^3 GEMM (what
    it reaches where the shape is easy). A reference point for the MFMA fraction only: nothing
    here runs on the int4 path."""
    import torch
    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    shapes = [(K, N) for (_, _, K, N) in synth.model_linears("0.5b")[:7]]
    out = {}
    for M in (128, 512):
        xs = {K: torch.randn(M, K, device=dev, dtype=torch.float16) for K in {k for k, _ in shapes}}
        ws = [torch.randn(N, K, device=dev, dtype=torch.float16) * 0.02 for K, N in shapes]
        ys = [torch.empty(M, N, device=dev, dtype=torch.float16) for K, N in shapes]

        def layer():
            for (K, N), w, y in zip(shapes, ws, ys):
                torch.matmul(xs[K], w.t(), out=y)
        layer()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(24):
                layer()
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            g.replay()
        torch.cuda.synchronize()
        us = (time.perf_counter() - t0) / steps * 1e6
        flops = 24 * sum(2 * M * K * N for K, N in shapes)
        out[f"{M}_step"] = {"us": round(us, 1), "tflops": round(flops / us / 1e6, 1),
                            "frac": round(flops / us / 1e6 / F16_PEAK_TFLOPS, 4), "calls": 168}
    a = torch.randn(8192, 8192, device=dev, dtype=torch.float16)
    b = torch.randn(8192, 8192, device=dev, dtype=torch.float16)
    for _ in range(3):
        a @ b
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(10):
        a @ b
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) / 10 * 1e6
    out["8192_cube"] = {"us": round(us, 1), "tflops": round(2 * 8192 ** 3 / us / 1e6, 1),
                        "frac": round(2 * 8192 ** 3 / us / 1e6 / F16_PEAK_TFLOPS, 4)}
    out["note"] = ("torch.matmul fp16 x fp16 -> fp16 (hipBLASLt), dense fp16 weights of the 0.5B shapes "
                   "(not int4): the library's rate on the prefill step's GEMMs and on a large square one")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", default="all",
                    help="all | step05 | headline | step7b | north | sweep | prefill | prefill_one | unpack | lmhead | "
                         "attn | elem | cpu | blas "
                         "(subsets for profiling: headline = the 0.5B step and its MALL-flushed "
                         "timing only; north = the 7B-shaped step at M=1 only)")
    ap.add_argument("--m7b", default="1,2,4,8,16", help="decode batch sizes for the 7B-shaped step")
    ap.add_argument("--prefill-m", default="128,512", help="prefill rows for the one-launch prefill step")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-flush", action="store_true",
                    help="skip the MALL-flushed timing (profiling runs of the headline kernel)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="end with one 512 MiB device-to-device copy: the known-size kernel that "
                         "scales FETCH_SIZE / WRITE_SIZE counter passes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus "
              f"{args.gpus}. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.only == "blas":
        print(json.dumps({"partial": "blas", "extra": {"blas_f16": blas_reference(max(10, args.steps))}}))
        return

    ctx = ql.Context(0)
    info = ctx.info()
    log(f"device: {info['name']} CUs={info['cu_count']}")
    extra = {}
    only = args.only

    m05 = None
    if only in ("all", "step05", "headline", "sweep", "prefill", "prefill_one", "unpack"):
        t0 = time.time()
        m05 = Model(ctx, "0.5b", seed=0x9EF0)
        log(f"0.5B weights: {m05.weight_bytes/1e6:.1f} MB uploaded in {time.time()-t0:.1f}s")

    value = ms_step = None
    roof = None
    step1 = None
    if only in ("all", "step05", "headline"):
        # the benchmark config as written: 168 linears back to back, each on its own fp32
        # activations ~ N(0,1), as one persistent launch per step
        step1 = SeqStep(ctx, m05, 1, chained=False)
        ms_step = timed(step1, args.steps, args.warmup)
        value = ms_step * 1e3
        si = step1.info
        kms = step1.kernel_ms(args.steps)
        gbs = step1.bytes / (kms * 1e-3) / 1e9
        log(f"0.5B step M=1 (one launch): {value:.1f} us/step, kernel {kms*1e3:.1f} us, "
            f"{gbs:.0f} GB/s; plan {si.as_dict()}")
        flushed = None if args.no_flush else flushed_step_ms(ctx, step1)
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4),
                "traffic": traffic_from_profiles("strip05_m1_indep" if si.kernel == ql.SEQ_STRIPS else "seq05_m1_indep"),
                "kernel": ("strip_kernel<1,2,8,1,2,%d,%s>" % (si.split, "true" if si.stream else "false")
                           if si.kernel == ql.SEQ_STRIPS else "seq_kernel<1,2,4,2,8,true>"),
                "launches_per_step": 1,
                "bytes_per_launch": step1.bytes,
                "avg_launch_us": round(kms * 1e3, 3),
                "tiles": si.tiles, "reduces": si.reduces, "grid": si.grid,
                "balance": round(si.balance, 4),
                "mall_resident": True,
                "flushed": None if flushed is None else {
                    "us": round(flushed * 1e3, 1),
                    "achieved": round(step1.bytes / (flushed * 1e-3) / 1e9, 1),
                    "frac": round(step1.bytes / (flushed * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
                "note": "one persistent launch per step (168 linears, each on its own input); "
                        "launch duration = HIP-event time of graphs of 10 consecutive launches on "
                        "the context stream / launches (value = one ql_seq_run per step, back to "
                        "back, so it also carries the gap between launches). The 0.5B weights (186 MB) stay in the "
                        "256 MB MALL across replays, so achieved/frac are HBM+MALL bandwidth over "
                        "the HBM peak; 'flushed' is one step after a read-only pass over 1 GiB has "
                        "evicted them (HBM-fed, includes launch latency). 'traffic' is not measured "
                        "in this run: it is the calibrated FETCH_SIZE + WRITE_SIZE bytes per launch of "
                        "this kernel on this step from separate rocprofv3 counter passes, read from "
                        "profiles/traffic.json"}
        if flushed is not None:
            extra["step05_m1_flushed_us"] = round(flushed * 1e3, 1)
            extra["step05_m1_flushed_gbs"] = round(step1.bytes / (flushed * 1e-3) / 1e9, 1)
            log(f"0.5B step M=1 MALL-flushed: {flushed*1e3:.1f} us")
    if only in ("all", "step05"):
        ch = SeqStep(ctx, m05, 1, chained=True)
        ms = timed(ch, args.steps, args.warmup)
        extra["step05_m1_chained"] = {
            "us": round(ms * 1e3, 1), "gbs": round(ch.bytes / (ms * 1e-3) / 1e9, 1),
            "passes": ch.info.passes, "tiles": ch.info.tiles, "reduces": ch.info.reduces,
            "launches": ch.info.launches, "finite": ch.finite(),
            "note": "the same 168 linears as a layer consumes them, with the layer's elementwise "
                    "work folded into the one launch: (q,k,v) <- rmsnorm(h), h1 = h + o(q), "
                    "(gate,up) <- rmsnorm(h1), h2 = h1 + down(silu(gate) * up); 96 dependent "
                    "passes ordered on the device (o reads q in attention's place)"}
        log(f"0.5B step M=1 chained: {ms*1e3:.1f} us")
        ch.release()
        st = Step(ctx, m05, 1)
        ms = timed(st, args.steps, args.warmup)
        extra["step05_m1_per_linear_launches"] = {
            "us": round(ms * 1e3, 1), "gbs": round(st.bytes / (ms * 1e-3) / 1e9, 1),
            "launches": len(st.launches),
            "note": "same linears as ql_linear / ql_linear_batch launches (q,k,v | o | gate,up | "
                    "down per layer) on independent inputs, graph-replayed"}
        log(f"0.5B step M=1 per-linear launches: {ms*1e3:.1f} us ({len(st.launches)} launches)")
        st.release()

    if only in ("all", "sweep"):
        sweep = {}
        for M in (1, 2, 4, 8, 16):
            st = SeqStep(ctx, m05, M, chained=False)
            ms = timed(st, max(10, args.steps // 2), 2)
            sweep[str(M)] = {"us": round(ms * 1e3, 1), "gbs": round(st.bytes / (ms * 1e-3) / 1e9, 1),
                             "kernel": "strip"}
            st.release()
        # past 16 rows the MFMA GEMM takes over (fp16 activations, one persistent launch)
        for M in (32, 64):
            st = PrefillStep(ctx, m05, M)
            ms = timed(st, max(10, args.steps // 2), 10)
            sweep[str(M)] = {"us": round(ms * 1e3, 1), "tflops": round(st.flops / (ms * 1e-3) / 1e12, 1),
                             "kernel": "prefill"}
            st.release()
        sweep["note"] = ("M <= 16: the decode sequence (strip_kernel, fp32 x); M = 32, 64: the prefill "
                         "GEMM launch (fp16 x, 128-row tiles). Two 16-row decode steps against one "
                         "32-row prefill step place the crossover")
        extra["step05_m_sweep"] = sweep
        log(f"M sweep: {sweep}")

    if only in ("all", "prefill", "prefill_one"):
        pre = {}
        for M in [int(v) for v in args.prefill_m.split(",")]:
            st = PrefillStep(ctx, m05, M)
            # the first launches after an idle period run up to 20% slow (clock ramp): warm up longer
            ms = timed(st, max(20, args.steps // 2), 30)
            kms = st.kernel_ms(max(10, args.steps // 2))
            tf = st.flops / (kms * 1e-3) / 1e12
            pre[f"{M}_one_launch"] = {
                "us": round(ms * 1e3, 1), "kernel_us": round(kms * 1e3, 1), "tflops": round(tf, 2),
                "mfma_frac": round(tf / F16_PEAK_TFLOPS, 4), "launches": 1, "tasks": st.info.tiles,
                "balance": round(st.info.balance, 4)}
            log(f"prefill M={M} one launch: {pre[f'{M}_one_launch']}")
            st.release()
            # fp32 activations into the same launch (rounded to fp16 as staged)
            st = PrefillStep(ctx, m05, M, x_dtype=ql.DTYPE_F32)
            kms = st.kernel_ms(max(10, args.steps // 2))
            tf = st.flops / (kms * 1e-3) / 1e12
            pre[f"{M}_one_launch_f32x"] = {"kernel_us": round(kms * 1e3, 1), "tflops": round(tf, 2),
                                          "mfma_frac": round(tf / F16_PEAK_TFLOPS, 4)}
            st.release()
        for layered in ((False, True) if only != "prefill_one" else ()):
            for M in (128, 512):
                st = Step(ctx, m05, M, x_dtype=ql.DTYPE_F16, layered=layered)
                ms = timed(st, max(5, args.steps // 5), 2)
                tf = st.flops / (ms * 1e-3) / 1e12
                pre[f"{M}{'_layered' if layered else ''}"] = {
                    "us": round(ms * 1e3, 1), "tflops": round(tf, 2),
                    "mfma_frac": round(tf / F16_PEAK_TFLOPS, 4), "launches": len(st.launches)}
                st.release()
        if only != "prefill_one":
            # the model's dependency order with the layer's elementwise work, as one sequence
            # (runForward(M = T)): pass by pass, one prefill launch per pass
            for M in (128, 512):
                st = SeqStep(ctx, m05, M, chained=True)
                ms = timed(st, max(5, args.steps // 5), 2)
                tf = st.flops / (ms * 1e-3) / 1e12
                pre[f"{M}_chained"] = {
                    "us": round(ms * 1e3, 1), "tflops": round(tf, 2), "mfma_frac": round(tf / F16_PEAK_TFLOPS, 4),
                    "passes": st.info.passes, "launches": st.info.launches,
                    "chunked_passes": st.info.variant, "tiles": st.info.tiles, "finite": st.finite()}
                st.release()
        pre["note"] = ("M x 168 linears, fp16 x, fp32 y. _one_launch: the config as written (each linear "
                       "on its own input) as one persistent prefill launch (tflops from the kernel "
                       "time: graphs of 10 launches, HIP events); _one_launch_f32x: the same launch fed "
                       "fp32 x, rounded to fp16 as staged. Plain M: the same as ql_linear_batch "
                       "launches of 8 linears. _layered: the model's dependency order, one launch per "
                       "(q,k,v | o | gate,up | down) group (96 launches). _chained: the model's "
                       "dependency order as one sequence with the layer's RMSNorms, SiLU-mul and "
                       "residuals (ql_seq_create_fused, fp32 x): per pass one GEMM launch (96: the "
                       "prefill kernel where its tiles fill the device, else the chunked split-K "
                       "GEMM), a part-sum launch after each chunked pass with K split, and one "
                       "launch per RMSNorm (48) or SiLU-mul input (24; none where the gate/up pass's "
                       "part-sum launch writes it)")
        extra["prefill05"] = pre
        log(f"prefill: {pre}")

    if only in ("all", "lmhead"):
        # the tied lm_head / embedding GEMV of the 0.5B model (qwen.ts:488-489): fp16 [151936, 896]
        V, C = 151936, 896
        rng = np.random.default_rng(0x1E4D)
        wl = ctx.arena(V * C * 2)
        wl.write(0, (rng.standard_normal((V, C), dtype=np.float32) * 0.02).astype(np.float16).view(np.uint16))
        lm = {}
        for M in (1, 4, 16):
            act = ctx.arena(M * C * 4 + M * V * 4 + 256)
            y_off = (M * C * 4 + 255) // 256 * 256
            act.write(0, synth.activations(M, C, seed=0x1E4E, key=(M,)))
            issue = lambda: ctx.gemv_f16w(wl, 0, None, act, 0, M, V, C, y_off)
            issue()
            ctx.sync()
            nbytes = V * C * 2 + M * C * 4 + M * V * 4
            row = {"bytes": nbytes}
            # one launch per graph replay (what a decode step pays), then ten per replay (the
            # kernel's own time, replay overhead spread over ten)
            for per, key in ((1, ""), (10, "kernel_")):
                ctx.graph_begin()
                for _ in range(per):
                    issue()
                g = ctx.graph_end()
                for _ in range(3):
                    g.launch()
                reps = max(20, args.steps) if per == 1 else max(4, args.steps // 5)
                ctx.timer_start()
                for _ in range(reps):
                    g.launch()
                ms = ctx.timer_stop() / (reps * per)
                g.destroy()
                row[key + "us"] = round(ms * 1e3, 1)
                row[key + "frac"] = round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
            lm[str(M)] = row
            act.release()
        wl.release()
        lm["note"] = ("fp16 W [151936, 896] (272 MB, read once per launch), fp32 x and y. us/frac: one "
                      "launch per graph replay; kernel_us/kernel_frac: graphs of 10 launches. M=1 runs "
                      "the fp32-FMA kernel, M >= 2 the matrix-core one (16 rows per pass)")
        extra["lmhead05"] = lm
        log(f"lm_head GEMV: {lm}")

    if only in ("all", "elem"):
        # the elementwise work of a decode layer: residual add + RMSNorm (twice per layer) and
        # SiLU-mul, at the 0.5B and 7B widths, M = 1, every layer of a step
        el = {}
        for name, L, C, I in (("05b", 24, 896, 4864), ("7b", 28, 3584, 18944)):
            rng = np.random.default_rng(0xE1)
            wa = ctx.arena(C * 4)
            wa.write(0, rng.standard_normal(C).astype(np.float32))
            rb, ib = (C * 4 + 255) // 256 * 256, (I * 4 + 255) // 256 * 256
            act = ctx.arena(4 * rb + 3 * ib)
            act.write(0, rng.standard_normal(C).astype(np.float32))
            act.write(rb, rng.standard_normal(C).astype(np.float32))
            act.write(4 * rb, rng.standard_normal(I).astype(np.float32))
            act.write(4 * rb + ib, rng.standard_normal(I).astype(np.float32))

            def issue():
                for _ in range(L):
                    ctx.add_rmsnorm(act, 0, rb, wa, 0, 1e-6, 1, C, 3 * rb, 2 * rb)
                    ctx.add_rmsnorm(act, 0, rb, wa, 0, 1e-6, 1, C, 3 * rb, 2 * rb)
                    ctx.silu_mul(act, 4 * rb, 4 * rb + ib, I, 4 * rb + 2 * ib)
            issue()
            ctx.sync()
            ctx.graph_begin()
            issue()
            g = ctx.graph_end()
            for _ in range(3):
                g.launch()
            ctx.timer_start()
            reps = max(20, args.steps)
            for _ in range(reps):
                g.launch()
            ms = ctx.timer_stop() / reps
            nbytes = L * (2 * (5 * C * 4) + 3 * I * 4)
            el[name] = {"us_per_step": round(ms * 1e3, 1), "us_per_layer": round(ms * 1e3 / L, 2),
                        "launches_per_layer": 3, "bytes": nbytes}
            g.destroy()
            act.release()
            wa.release()
        el["note"] = ("per layer: two fused residual-add + RMSNorm launches (x, d, w read; sum, y "
                      "written) and one SiLU-mul; the reference runs 5 launches for the same work")
        extra["elem"] = el
        log(f"elementwise: {el}")

    if only in ("all", "attn"):
        # decode attention over the KV cache, every layer of a step (qwen.ts:424-442): the
        # 0.5B model at its full 128-position cache, the 7B shape at 4096 positions
        at = {}
        for name, L, H, KV, D, T in (("05b_t128", 24, 14, 2, 64, 128), ("7b_t4096", 28, 28, 4, 128, 4096)):
            rng = np.random.default_rng(0xA7)
            region = T * KV * D * 4
            cache = ctx.arena(2 * L * region)
            for i in range(2 * L):
                cache.write(i * region, rng.standard_normal((T, KV * D)).astype(np.float32))
            qb = H * D * 4
            act = ctx.arena(2 * L * qb)
            act.write(0, rng.standard_normal((L, H * D)).astype(np.float32))

            def issue():
                for l in range(L):
                    ctx.attention_decode(act, l * qb, cache, 2 * l * region, (2 * l + 1) * region, T, 1, H, KV,
                                         D, T - 1, (L + l) * qb)
            issue()
            ctx.sync()
            ctx.graph_begin()
            issue()
            g = ctx.graph_end()
            for _ in range(3):
                g.launch()
            ctx.timer_start()
            reps = max(20, args.steps)
            for _ in range(reps):
                g.launch()
            ms = ctx.timer_stop() / reps
            nbytes = L * (2 * region + 2 * qb)
            at[name] = {"us_per_step": round(ms * 1e3, 1), "us_per_layer": round(ms * 1e3 / L, 2),
                        "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                        "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes": nbytes,
                        "layers": L, "heads": H, "kv_heads": KV, "head_dim": D, "positions": T}
            g.destroy()
            act.release()
            cache.release()
        at["note"] = ("M = 1 at the last position; one launch per layer (grid heads x 1), graph-replayed; "
                      "bytes = the K and V caches once plus q and out")
        extra["attn"] = at
        log(f"decode attention: {at}")

    if only == "cpu":
        extra["cpu_plan"] = cpu_plan(ctx, args.cpu_seconds)
        log(f"cpu plan: {extra['cpu_plan']}")

    if only in ("all", "unpack"):
        ms, nbytes = unpack_all(ctx, m05, max(5, args.steps // 5))
        extra["unpack05"] = {"us": round(ms * 1e3, 1), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                             "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                             "bytes": nbytes}
        log(f"unpack 168 tensors: {extra['unpack05']}")

    cpu = None
    if only in ("all", "step05", "headline") and not args.no_cpu:
        cpu = cpu_baseline(m05, step1, args.cpu_seconds)
        log(f"cpu baseline: {cpu}")

    if step1 is not None:
        step1.release()
    if m05 is not None:
        m05.arena.release()

    if only == "north":
        m7 = Model(ctx, "7b", seed=0x7B)
        st = SeqStep(ctx, m7, 1, chained=False)
        ms = timed(st, args.steps, args.warmup)
        gbs = st.bytes / (ms * 1e-3) / 1e9
        extra["north_star_7b"] = {"1": {"us": round(ms * 1e3, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                                        "bytes": st.bytes, "tiles": st.info.tiles,
                                        "reduces": st.info.reduces, "balance": round(st.info.balance, 4)}}
        log(f"7B step M=1: {extra['north_star_7b']}")
        st.release()
        # one 512 MiB device copy: the counter calibration kernel for traffic passes
        flush = ctx.arena(1 << 30)
        ctx.copy(flush, 0, flush, 1 << 29, 1 << 29)
        ctx.sync()
        flush.release()
        m7.arena.release()

    if only in ("all", "step7b"):
        t0 = time.time()
        m7 = Model(ctx, "7b", seed=0x7B)
        log(f"7B weights: {m7.weight_bytes/1e9:.2f} GB uploaded in {time.time()-t0:.1f}s")
        s7 = {}
        for chained in (False, True):
            for M in [int(v) for v in args.m7b.split(",")]:
                st = SeqStep(ctx, m7, M, chained=chained)
                ms = timed(st, max(10, args.steps // 2), 2)
                gbs = st.bytes / (ms * 1e-3) / 1e9
                roof_us = st.bytes / (HBM_PEAK_GBS * 1e9) * 1e6
                s7[f"{M}{'_chained' if chained else ''}"] = {
                    "us": round(ms * 1e3, 1), "gbs": round(gbs, 1),
                    "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": st.bytes,
                    "roofline_us": round(roof_us, 1), "target_us_70pct": round(roof_us / 0.7, 1),
                    "launches": st.info.launches, "passes": st.info.passes, "tiles": st.info.tiles,
                    "reduces": st.info.reduces, "kernel": SEQ_KERNEL_NAMES.get(st.info.kernel, "?")}
                if chained:
                    s7[f"{M}_chained"]["finite"] = st.finite()
                st.release()
        st = Step(ctx, m7, 1)
        ms = timed(st, max(10, args.steps // 2), 2)
        s7["1_per_linear_launches"] = {"us": round(ms * 1e3, 1),
                                       "gbs": round(st.bytes / (ms * 1e-3) / 1e9, 1),
                                       "launches": len(st.launches)}
        st.release()
        extra["step7b"] = s7
        if "1" in s7:
            # the north-star target: the 7B-shaped config (cache-exceeding) at >= 70% of HBM roofline
            extra["north_star_7b"] = {M: {"us": s7[M]["us"], "frac": s7[M]["frac"],
                                          "target_us": s7[M]["target_us_70pct"]}
                                      for M in s7 if M.isdigit()}
        log(f"7B step: {s7}")
        m7.arena.release()

    # the per-linear launches carry no elementwise work, the chained steps carry it inside their
    # launch: add the measured elementwise launches per step for the like-for-like figure
    if "elem" in extra:
        pl = extra.get("step05_m1_per_linear_launches")
        if pl:
            pl["plus_elem_us"] = round(pl["us"] + extra["elem"]["05b"]["us_per_step"], 1)
        pl = extra.get("step7b", {}).get("1_per_linear_launches")
        if pl:
            pl["plus_elem_us"] = round(pl["us"] + extra["elem"]["7b"]["us_per_step"], 1)

    if args.calib_copy:
        flush = ctx.arena(1 << 30)
        ctx.copy(flush, 0, flush, 1 << 29, 1 << 29)
        ctx.sync()
        flush.release()

    ctx.destroy()
    if value is None:
        print(json.dumps({"partial": only, "extra": extra}))
        return
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "us/step", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "int4xf32", "data": "synthetic",
        "config": {"workload": "Qwen2.5-0.5B-shaped decode step: 168 GPTQ int4 linears "
                               "(group 128) back to back, M=1, each on its own fp32 activations "
                               "~N(0,1), one persistent launch per step (ql_seq_run)",
                   "global_batch": 1, "seq_len": 1, "parallelism": "none (1 GPU)",
                   "launches_per_step": roof["launches_per_step"] if roof else None},
        "roofline": roof, "cpu_baseline": cpu, "extra": extra,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
