"""GPU parity of linear sequences (ql_seq_*): decode linears chained through their outputs, run
as one persistent launch, against the CPU oracle.

Each linear is checked on its own: the oracle (gemmNTRef over quant.ts weights,
src/reference/qwen-ref.ts:126-145) is applied to the input the GPU actually used — the external
x, or the producer's GPU output — so every linear meets the single-GEMV bar
|d| <= atol + 1e-4|ref|. Chained inputs grow (x1.4 to x6 per linear), so atol = 1e-5 * rms(input),
which is the reference's 1e-5 for the N(0,1) inputs its own tests use (kernels.ts:67).
"""
import sys

import numpy as np
import pytest

from webllm_amd import synth

pytestmark = pytest.mark.gpu

RTOL = 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class SeqModel:
    """Linears of a Qwen-shaped chain in one weight arena; activations in one arena.

    layers of (q,k,v) <- h, o <- q, (gate,up) <- o, down <- gate, next h = down (attention and
    the elementwise ops between linears are not part of the sequence)."""

    def __init__(self, ql, ctx, M, layers, C, I, KV, group=128, x_dtype=0, seed=0x5E0,
                 sym_every=3, bias_qkv=True):
        self.ql, self.ctx, self.M, self.group, self.x_dtype = ql, ctx, M, group, x_dtype
        wl, al = ql.ArenaLayout(), ql.ArenaLayout()
        es = 4 if x_dtype == 0 else 2
        self.x = synth.activations(M, C, seed=seed, key=(M,))
        if x_dtype == 1:
            self.x = self.x.astype(np.float16)
        self.x_off = al.take(self.x.nbytes)
        self.lin = []            # dicts: t, bias, qzeros(used), desc offsets, x_off, y_off, src
        h = (self.x_off, -1)
        idx = 0
        for layer in range(layers):
            plan = [("q", C, C, h), ("k", C, KV, h), ("v", C, KV, h)]
            for key, K, N, (xo, src) in plan:
                self._add(wl, al, layer, key, K, N, xo, src, idx, seed, sym_every, bias_qkv)
                idx += 1
            q = (self.lin[-3]["y_off"], len(self.lin) - 3)
            self._add(wl, al, layer, "o", C, C, q[0], q[1], idx, seed, sym_every, False)
            idx += 1
            o = (self.lin[-1]["y_off"], len(self.lin) - 1)
            self._add(wl, al, layer, "gate", C, I, o[0], o[1], idx, seed, sym_every, False)
            idx += 1
            g = (self.lin[-1]["y_off"], len(self.lin) - 1)
            self._add(wl, al, layer, "up", C, I, o[0], o[1], idx, seed, sym_every, False)
            idx += 1
            self._add(wl, al, layer, "down", I, C, g[0], g[1], idx, seed, sym_every, False)
            idx += 1
            h = (self.lin[-1]["y_off"], len(self.lin) - 1)
        self.weights = ctx.arena(wl.used)
        self.act = ctx.arena(al.used)
        for L in self.lin:
            t = L["t"]
            self.weights.write(L["qw"], t.qweight)
            if L["qz"] is not None:
                self.weights.write(L["qz"], t.qzeros)
            self.weights.write(L["sc"], t.scales)
            if L["bias"] is not None:
                self.weights.write(L["b"], L["bias"])
        self.act.write(self.x_off, self.x)
        self.descs = [ql.make_desc(L["qw"], L["qz"], L["sc"], L["t"].K, L["t"].N, group, L["b"])
                      for L in self.lin]
        self.seq = ctx.seq(self.descs, self.weights, self.act, [L["x_off"] for L in self.lin],
                           x_dtype, M, [L["y_off"] for L in self.lin])

    def _add(self, wl, al, layer, key, K, N, x_off, src, idx, seed, sym_every, biased):
        sym = sym_every and idx % sym_every == 1          # some linears without qzeros (zero 8)
        zero = 7 if idx % 2 == 0 else None
        t = synth.gptq_linear(K, N, self.group, seed=seed, key=(layer, idx), stored_zero=zero)
        bias = synth.activations(1, N, seed=seed + 1, key=(layer, idx))[0] if biased else None
        L = {"t": t, "bias": bias, "qw": wl.take(t.qweight.nbytes),
             "qz": None if sym else wl.take(t.qzeros.nbytes), "sc": wl.take(t.scales.nbytes),
             "b": None if bias is None else wl.take(bias.nbytes), "x_off": x_off,
             "y_off": al.take(self.M * N * 4), "src": src, "name": f"L{layer}.{key}"}
        L["qzeros"] = None if sym else t.qzeros
        self.lin.append(L)

    def outputs(self):
        return [self.act.read(L["y_off"], (self.M, L["t"].N), np.float32) for L in self.lin]

    def inputs(self, ys):
        xs = []
        for L in self.lin:
            if L["src"] < 0:
                xs.append(self.x.astype(np.float32))
            else:
                xs.append(ys[L["src"]])
        return xs

    def release(self):
        self.seq.destroy()
        self.weights.release()
        self.act.release()


def check_all(orc, model: SeqModel, ys, label):
    xs = model.inputs(ys)
    worst = 0.0
    for L, x, y in zip(model.lin, xs, ys):
        t = L["t"]
        ref = orc.gptq_linear(t.qweight, L["qzeros"], t.scales, x, L["bias"], model.group)
        atol = 1e-5 * max(1.0, float(np.sqrt(np.mean(x.astype(np.float64) ** 2))))
        ok, max_abs, max_rel = orc.check_tolerance(y, ref, atol, RTOL)
        norm = float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))
        worst = max(worst, norm)
        assert ok, f"{label} {L['name']}: maxAbs {max_abs:.3e} (atol {atol:.2e}) maxRel {max_rel:.3e}"
    say(f"  {label}: {len(ys)} linears within bar, worst normwise {worst:.3e}")


@pytest.mark.parametrize("M", [1, 4, 16])
def test_seq_qwen05_two_layers(ql, ctx, orc, M):
    m = SeqModel(ql, ctx, M, layers=2, C=896, I=4864, KV=128)
    info = m.seq.info
    say(f"seq 0.5B x2 M={M}: {info.as_dict()}")
    assert info.passes == 8
    m.seq.run()
    m.seq.status()
    check_all(orc, m, m.outputs(), f"0.5B x2 M={M}")
    m.release()


def test_seq_qwen7b_layer(ql, ctx, orc):
    m = SeqModel(ql, ctx, 1, layers=1, C=3584, I=18944, KV=512, bias_qkv=False)
    say(f"seq 7B x1 M=1: {m.seq.info.as_dict()}")
    m.seq.run()
    m.seq.status()
    check_all(orc, m, m.outputs(), "7B x1 M=1")
    m.release()


def test_seq_qwen7b_layer_m16(ql, ctx, orc):
    m = SeqModel(ql, ctx, 16, layers=1, C=3584, I=18944, KV=512, bias_qkv=False)
    say(f"seq 7B x1 M=16: {m.seq.info.as_dict()}")
    m.seq.run()
    m.seq.status()
    check_all(orc, m, m.outputs(), "7B x1 M=16")
    m.release()


@pytest.mark.parametrize("group,M", [(64, 3), (256, 8)])
def test_seq_group_sizes(ql, ctx, orc, group, M):
    m = SeqModel(ql, ctx, M, layers=2, C=1024, I=2048, KV=256, group=group)
    m.seq.run()
    m.seq.status()
    check_all(orc, m, m.outputs(), f"group {group} M={M}")
    m.release()


def test_seq_f16_external_input(ql, ctx, orc):
    m = SeqModel(ql, ctx, 2, layers=1, C=896, I=4864, KV=128, x_dtype=1)
    m.seq.run()
    m.seq.status()
    check_all(orc, m, m.outputs(), "f16 x")
    m.release()


def test_seq_deterministic_and_graph_replay(ql, ctx, orc):
    """Runs reuse the exchange buffers with a new epoch each time: outputs are bit-identical
    across eager runs and graph replays (with eager work and syncs between the replays)."""
    m = SeqModel(ql, ctx, 1, layers=3, C=896, I=4864, KV=128)
    m.seq.run()
    m.seq.status()
    first = m.outputs()
    check_all(orc, m, first, "eager run 1")
    zero = np.zeros((m.M, m.lin[-1]["t"].N), np.float32)
    for r in range(3):
        m.act.write(m.lin[-1]["y_off"], zero)       # stale outputs must be rewritten
        m.seq.run()
        m.seq.status()
        for a, b in zip(first, m.outputs()):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"eager run {r + 2}"
    ctx.graph_begin()
    m.seq.run()
    g = ctx.graph_end()
    for r in range(4):
        m.act.write(m.lin[-1]["y_off"], zero)
        g.launch()
        m.seq.status()
        for a, b in zip(first, m.outputs()):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"graph replay {r}"
        m.seq.run()                                  # eager run between replays
        m.seq.status()
    g.destroy()
    m.release()


def test_seq_agrees_with_single_linears(ql, ctx, orc):
    """The sequence and ql_linear on the same inputs agree to the GEMV bar (they split K
    differently, so the last bits may differ)."""
    m = SeqModel(ql, ctx, 4, layers=1, C=896, I=4864, KV=128)
    m.seq.run()
    m.seq.status()
    ys = m.outputs()
    xs = m.inputs(ys)
    for i, (L, x, y) in enumerate(zip(m.lin, xs, ys)):
        t = L["t"]
        plan = ql.plan_linear(m.M, t.N, t.K, m.group)
        lay = ql.ArenaLayout()
        xo, yo, so = lay.take(x.nbytes), lay.take(m.M * t.N * 4), lay.take(max(plan.scratch_bytes, 16))
        act = ctx.arena(lay.used)
        act.write(xo, x)
        ctx.linear(m.descs[i], m.weights, act, xo, 0, m.M, yo, so)
        y1 = act.read(yo, (m.M, t.N), np.float32)
        act.release()
        atol = 1e-5 * max(1.0, float(np.sqrt(np.mean(x.astype(np.float64) ** 2))))
        ok, max_abs, _ = orc.check_tolerance(y, y1, atol, RTOL)
        assert ok, f"{L['name']}: seq vs ql_linear maxAbs {max_abs:.3e}"
    m.release()


class IndependentModel:
    """Independent 7B-shaped linears (q, o, gate, up, down per layer), each on its own input, in
    one weight arena: `layers` x 120 MB, so three layers exceed the 256 MB from which an
    independent sequence at M >= 2 runs as column strips."""

    SHAPES = [(3584, 3584), (3584, 3584), (3584, 18944), (3584, 18944), (18944, 3584)]

    def __init__(self, ql, ctx, layers=3, seed=0x57A):
        wl = ql.ArenaLayout()
        self.lin = []
        for layer in range(layers):
            for p, (K, N) in enumerate(self.SHAPES):
                idx = len(self.lin)
                t = synth.gptq_linear(K, N, 128, seed=seed, key=(layer, p),
                                      stored_zero=7 if idx % 2 == 0 else None)
                sym = idx % 3 == 1                         # some without qzeros (zero 8)
                bias = synth.activations(1, N, seed=seed + 1, key=(idx,))[0] if p == 0 else None
                self.lin.append({"t": t, "qw": wl.take(t.qweight.nbytes),
                                 "qz": None if sym else wl.take(t.qzeros.nbytes),
                                 "sc": wl.take(t.scales.nbytes),
                                 "b": None if bias is None else wl.take(bias.nbytes),
                                 "bias": bias, "qzeros": None if sym else t.qzeros})
        self.weights = ctx.arena(wl.used)
        for L in self.lin:
            t = L["t"]
            self.weights.write(L["qw"], t.qweight)
            if L["qz"] is not None:
                self.weights.write(L["qz"], t.qzeros)
            self.weights.write(L["sc"], t.scales)
            if L["b"] is not None:
                self.weights.write(L["b"], L["bias"])
        self.descs = [ql.make_desc(L["qw"], L["qz"], L["sc"], L["t"].K, L["t"].N, 128, L["b"])
                      for L in self.lin]


@pytest.fixture(scope="module")
def indep7b(ql, ctx):
    m = IndependentModel(ql, ctx)
    yield m
    m.weights.release()


# M = 5 and 11 leave the last 16-row digit tile partly past the rows (those rows' loads clamp)
@pytest.mark.parametrize("M", [1, 2, 5, 8, 11, 16])
def test_strips_7b_independent(ql, ctx, orc, indep7b, M):
    """Fifteen independent 7B-shaped linears (360 MB, each on its own fp32 input) at M rows run
    as column strips (no K split, nothing reduced): linears with bias, without qzeros and the
    18944-deep down projection meet the GEMV bar against the oracle, and repeated runs and
    graph replays are bit-identical."""
    m = indep7b
    al = ql.ArenaLayout()
    x_offs = [al.take(M * L["t"].K * 4) for L in m.lin]
    y_offs = [al.take(M * L["t"].N * 4) for L in m.lin]
    act = ctx.arena(al.used)
    xs = []
    for i, (L, xo) in enumerate(zip(m.lin, x_offs)):
        x = synth.activations(M, L["t"].K, seed=0x57B, key=(M, i))
        act.write(xo, x)
        xs.append(x)
    seq = ctx.seq(m.descs, m.weights, act, x_offs, 0, M, y_offs)
    info = seq.info
    say(f"strips 7B x3 M={M}: {info.as_dict()}")
    assert info.kernel == ql.SEQ_STRIPS and info.passes == 1 and info.reduces == 0 and info.max_split == 1
    seq.run()
    seq.status()
    ys = [act.read(yo, (M, L["t"].N), np.float32) for L, yo in zip(m.lin, y_offs)]
    for i in (0, 1, 3, 4, 14):              # q + bias, o without qzeros, up, down, last down
        L, t = m.lin[i], m.lin[i]["t"]
        ref = orc.gptq_linear(t.qweight, L["qzeros"], t.scales, xs[i], L["bias"], 128)
        ok, max_abs, max_rel = orc.check_tolerance(ys[i], ref, 1e-5, RTOL)
        say(f"  linear {i} K={t.K} N={t.N}: maxAbs {max_abs:.3e} maxRel {max_rel:.3e}")
        assert ok, f"M={M} linear {i}: maxAbs {max_abs:.3e} maxRel {max_rel:.3e}"
    for i in range(len(m.lin)):
        assert np.isfinite(ys[i]).all() and np.abs(ys[i]).max() > 0, f"linear {i} not written"
    zero = np.zeros((M, m.lin[-1]["t"].N), np.float32)
    act.write(y_offs[-1], zero)
    seq.run()
    seq.status()
    for L, yo, y in zip(m.lin, y_offs, ys):
        assert np.array_equal(act.read(yo, (M, L["t"].N), np.float32).view(np.uint32), y.view(np.uint32))
    ctx.graph_begin()
    seq.run()
    g = ctx.graph_end()
    for r in range(3):
        act.write(y_offs[-1], zero)
        g.launch()
        seq.status()
        for L, yo, y in zip(m.lin, y_offs, ys):
            assert np.array_equal(act.read(yo, (M, L["t"].N), np.float32).view(np.uint32),
                                  y.view(np.uint32)), f"graph replay {r}"
    g.destroy()
    seq.destroy()
    act.release()


@pytest.mark.parametrize("M", [1, 4, 6, 13, 16])
def test_strips_05b_split_blocks(ql, ctx, orc, M):
    """Two layers of 0.5B-shaped independent linears: strips of 4 blocks with two waves per block
    (each wave takes alternate groups of every chunk; part sums added in LDS in part order).
    Every linear, including the 4864-deep down projection and the biased q/k/v, meets the GEMV
    bar; repeated runs are bit-identical."""
    shapes = [(896, 896, True), (896, 128, True), (896, 128, True), (896, 896, False),
              (896, 4864, False), (896, 4864, False), (4864, 896, False)] * 2
    wl, al = ql.ArenaLayout(), ql.ArenaLayout()
    lins = []
    for i, (K, N, biased) in enumerate(shapes):
        t = synth.gptq_linear(K, N, 128, seed=0x5B2, key=(i,), stored_zero=7 if i % 2 else None)
        bias = synth.activations(1, N, seed=0x5B3, key=(i,))[0] if biased else None
        sym = i % 3 == 2
        lins.append({"t": t, "bias": bias, "qw": wl.take(t.qweight.nbytes),
                     "qz": None if sym else wl.take(t.qzeros.nbytes), "sc": wl.take(t.scales.nbytes),
                     "b": None if bias is None else wl.take(bias.nbytes),
                     "x": al.take(M * K * 4), "y": al.take(M * N * 4)})
    w = ctx.arena(wl.used)
    act = ctx.arena(al.used)
    xs = []
    for i, L in enumerate(lins):
        t = L["t"]
        w.write(L["qw"], t.qweight)
        if L["qz"] is not None:
            w.write(L["qz"], t.qzeros)
        w.write(L["sc"], t.scales)
        if L["b"] is not None:
            w.write(L["b"], L["bias"])
        x = synth.activations(M, t.K, seed=0x5B4, key=(M, i))
        act.write(L["x"], x)
        xs.append(x)
    descs = [ql.make_desc(L["qw"], L["qz"], L["sc"], L["t"].K, L["t"].N, 128, L["b"]) for L in lins]
    seq = ctx.seq(descs, w, act, [L["x"] for L in lins], 0, M, [L["y"] for L in lins])
    info = seq.info
    say(f"strips 0.5B x2 M={M}: {info.as_dict()}")
    assert info.kernel == ql.SEQ_STRIPS and info.split == 2 and info.reduces == 0
    seq.run()
    seq.status()
    ys = [act.read(L["y"], (M, L["t"].N), np.float32) for L in lins]
    for i, (L, x, y) in enumerate(zip(lins, xs, ys)):
        t = L["t"]
        qz = None if L["qz"] is None else t.qzeros
        ref = orc.gptq_linear(t.qweight, qz, t.scales, x, L["bias"], 128)
        ok, max_abs, max_rel = orc.check_tolerance(y, ref, 1e-5, RTOL)
        assert ok, f"M={M} linear {i} K={t.K} N={t.N}: maxAbs {max_abs:.3e} maxRel {max_rel:.3e}"
    seq.run()
    seq.status()
    for L, y in zip(lins, ys):
        assert np.array_equal(act.read(L["y"], (M, L["t"].N), np.float32).view(np.uint32), y.view(np.uint32))
    seq.destroy()
    act.release()
    w.release()
