"""GPU parity of the prefill GEMM launch (QL_SEQ_PREFILL and the batch form of ql_linear_batch):
y = f16(x) . f16(W)^T + bias in fp32, the reference's M > 1 path (gemm_nt_f16_from_f32.wgsl),
against the oracle's gemmNTRef over the fp16-rounded x and the uploaded fp16 weights with the bar
|d| <= 1e-5 + 2e-3 |ref|.

Cases: 0.5B-shaped layers (q/k/v with bias, o, gate/up, the 4864-deep down projection; some
linears without qzeros, random stored zeros), M = 128 and 512 (whole 128-row tiles) and 70 and
300 (ragged), a 256-wide group, N = 128 (half a 256-column tile); repeated runs and graph replays
are bit-identical; the full 168-linear config-3 step as bench.py builds it at M = 128 and 512,
every linear checked on a sample of 64-column blocks."""
import sys

import numpy as np
import pytest

import bench
from webllm_amd import synth

ATOL, RTOL = 1e-5, 2e-3


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def x16(x):
    return x.astype(np.float16).astype(np.float32)


class PrefillSet:
    """Independent linears in one weight arena, each with its own fp16 input (x32: fp32 input,
    which the launch rounds to fp16; the oracle reads the fp16-rounded values)."""

    def __init__(self, ql, ctx, shapes, M, seed, group=128, x32=False):
        wl, al = ql.ArenaLayout(), ql.ArenaLayout()
        self.lin = []
        for i, (K, N, biased, g) in enumerate(shapes):
            gs = g or group
            t = synth.gptq_linear(K, N, gs, seed=seed, key=(i,), stored_zero=7 if i % 2 else None)
            bias = synth.activations(1, N, seed=seed + 1, key=(i,))[0] if biased else None
            sym = i % 3 == 2
            x_in = synth.activations(M, K, seed=seed + 2, key=(i, M))
            x = x16(x_in)
            self.lin.append({"t": t, "bias": bias, "group": gs, "x": x, "x_in": x_in,
                             "qw": wl.take(t.qweight.nbytes), "qz": None if sym else wl.take(t.qzeros.nbytes),
                             "sc": wl.take(t.scales.nbytes), "b": None if bias is None else wl.take(bias.nbytes),
                             "xo": al.take(M * K * (4 if x32 else 2)), "yo": al.take(M * N * 4),
                             "qzeros": None if sym else t.qzeros})
        self.w = ctx.arena(wl.used)
        self.act = ctx.arena(al.used)
        for L in self.lin:
            t = L["t"]
            self.w.write(L["qw"], t.qweight)
            if L["qz"] is not None:
                self.w.write(L["qz"], t.qzeros)
            self.w.write(L["sc"], t.scales)
            if L["b"] is not None:
                self.w.write(L["b"], L["bias"])
            self.act.write(L["xo"], L["x_in"] if x32 else L["x"].astype(np.float16).view(np.uint16))
        self.descs = [ql.make_desc(L["qw"], L["qz"], L["sc"], L["t"].K, L["t"].N, L["group"], L["b"])
                      for L in self.lin]
        self.M = M

    def outputs(self):
        return [self.act.read(L["yo"], (self.M, L["t"].N), np.float32) for L in self.lin]

    def check(self, orc, ys, label):
        worst = 0.0
        for i, (L, y) in enumerate(zip(self.lin, ys)):
            t = L["t"]
            ref = orc.gptq_linear_cols(t.qweight, L["qzeros"], t.scales, L["x"], np.arange(t.N), L["bias"],
                                       L["group"], w_f16=True)
            ok, max_abs, max_rel = orc.check_tolerance(y, ref, ATOL, RTOL)
            assert ok, f"{label} linear {i} K={t.K} N={t.N}: maxAbs {max_abs:.3e} maxRel {max_rel:.3e}"
            worst = max(worst, float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30)))
        say(f"  {label}: {len(ys)} linears within bar, worst normwise {worst:.3e}")

    def release(self):
        self.w.release()
        self.act.release()


LAYER = [(896, 896, True, None), (896, 128, True, None), (896, 128, True, None), (896, 896, False, None),
         (896, 4864, False, None), (896, 4864, False, None), (4864, 896, False, None)]


@pytest.mark.gpu
@pytest.mark.parametrize("M", [128, 512, 70, 300])
def test_prefill_seq_layers(ql, ctx, orc, M):
    """Two 0.5B-shaped layers (14 independent linears) as one prefill launch."""
    s = PrefillSet(ql, ctx, LAYER * 2, M, seed=0x9F00)
    seq = ctx.seq(s.descs, s.w, s.act, [L["xo"] for L in s.lin], ql.DTYPE_F16, M, [L["yo"] for L in s.lin])
    info = seq.info
    say(f"prefill seq M={M}: {info.as_dict()}")
    assert info.kernel == ql.SEQ_PREFILL and info.passes == 1 and info.reduces == 0
    seq.run()
    seq.status()
    ys = s.outputs()
    s.check(orc, ys, f"prefill M={M}")
    # repeat and graph replay: bit-identical
    zero = np.zeros((M, s.lin[-1]["t"].N), np.float32)
    s.act.write(s.lin[-1]["yo"], zero)
    seq.run()
    seq.status()
    for a, b in zip(ys, s.outputs()):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    ctx.graph_begin()
    seq.run()
    g = ctx.graph_end()
    for r in range(3):
        s.act.write(s.lin[-1]["yo"], zero)
        g.launch()
        seq.status()
        for a, b in zip(ys, s.outputs()):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"graph replay {r}"
    g.destroy()
    seq.destroy()
    s.release()


@pytest.mark.gpu
@pytest.mark.parametrize("M", [128, 300])
def test_prefill_seq_f32_input(ql, ctx, orc, M):
    """fp32 x into the prefill launch, rounded to fp16 (nearest even) as it is staged, as the
    reference's tile load does (gemm_nt_f16_from_f32.wgsl:60); the oracle reads the same
    fp16-rounded x. Also the single-linear entry (QuantLinearModel.gemm's ql_linear) on a batch
    that fills the device."""
    s = PrefillSet(ql, ctx, LAYER * 2, M, seed=0x9F20, x32=True)
    seq = ctx.seq(s.descs, s.w, s.act, [L["xo"] for L in s.lin], ql.DTYPE_F32, M, [L["yo"] for L in s.lin])
    assert seq.info.kernel == ql.SEQ_PREFILL
    seq.run()
    seq.status()
    ys = s.outputs()
    s.check(orc, ys, f"prefill f32 x M={M}")
    # gate and up (K = 896) through ql_linear_batch on fp32 x, against the oracle
    pick = (4, 5)
    lay = ql.ArenaLayout()
    xo = [lay.take(M * 896 * 4) for _ in pick]
    yo = [lay.take(M * s.lin[i]["t"].N * 4) for i in pick]
    so = lay.take(max(256, ql.plan_batch([s.descs[i] for i in pick], M)))
    act2 = ctx.arena(lay.used)
    for o, i in zip(xo, pick):
        act2.write(o, s.lin[i]["x_in"])
    ctx.linear_batch([s.descs[i] for i in pick], s.w, act2, xo, ql.DTYPE_F32, M, yo, so)
    ctx.sync()
    for o, i in zip(yo, pick):
        y = act2.read(o, (M, s.lin[i]["t"].N), np.float32)
        t = s.lin[i]["t"]
        ref = orc.gptq_linear_cols(t.qweight, s.lin[i]["qzeros"], t.scales, s.lin[i]["x"], np.arange(t.N),
                                   s.lin[i]["bias"], s.lin[i]["group"], w_f16=True)
        ok, ma, mr = orc.check_tolerance(y, ref, ATOL, RTOL)
        assert ok, (i, ma, mr)
    act2.release()
    seq.destroy()
    s.release()


@pytest.mark.gpu
def test_prefill_group_256_and_narrow(ql, ctx, orc):
    """A 256-wide group (two chunks per scale), N = 128 and N = 260 (partial tiles), K = 128."""
    shapes = [(2048, 516, True, 256), (1024, 128, False, 128), (128, 260, True, 128), (1024, 4864, False, 256)]
    s = PrefillSet(ql, ctx, shapes, 200, seed=0x9F10)
    seq = ctx.seq(s.descs, s.w, s.act, [L["xo"] for L in s.lin], ql.DTYPE_F16, 200, [L["yo"] for L in s.lin])
    assert seq.info.kernel == ql.SEQ_PREFILL
    seq.run()
    seq.status()
    s.check(orc, s.outputs(), "group 256 / narrow")
    seq.destroy()
    s.release()


@pytest.mark.gpu
def test_prefill_batch_form(ql, ctx, orc):
    """gate and up (M = 512, 152 tiles) through ql_linear_batch take the prefill launch's batch form
    (tiles numbered across the batch); each single ql_linear (76 tiles) takes the split-K GEMM. Both
    meet the bar against the oracle."""
    M = 512
    s = PrefillSet(ql, ctx, [(896, 4864, False, None), (896, 4864, True, None)], M, seed=0x9F20)
    scratch = max([ql.plan_batch(s.descs, M), 16] +
                  [ql.plan_linear(M, L["t"].N, L["t"].K, 128).scratch_bytes for L in s.lin])
    so = (s.act.size + 255) // 256 * 256
    act2 = ctx.arena(so + scratch)
    ctx.copy(act2, 0, s.act, 0, s.act.size)
    ctx.linear_batch(s.descs, s.w, act2, [L["xo"] for L in s.lin], ql.DTYPE_F16, M, [L["yo"] for L in s.lin], so)
    ys = [act2.read(L["yo"], (M, L["t"].N), np.float32) for L in s.lin]
    s.check(orc, ys, "batch form M=512")
    for i, L in enumerate(s.lin):
        plan = ql.plan_linear(M, L["t"].N, L["t"].K, 128)
        ctx.linear(s.descs[i], s.w, act2, L["xo"], ql.DTYPE_F16, M, L["yo"], so)
        y1 = act2.read(L["yo"], (M, L["t"].N), np.float32)
        ok, ma, _ = orc.check_tolerance(y1, ys[i], ATOL, RTOL)
        assert ok, f"single launch {i} (split {plan.split}) vs batch: maxAbs {ma:.3e}"
    act2.release()
    s.release()


def _cols_sample(N, count=4):
    nb = N // 64
    picks = sorted(set([0, nb - 1] + [int(round(i * (nb - 1) / (count - 1))) for i in range(count)]))
    return np.concatenate([np.arange(b * 64, b * 64 + 64) for b in picks]).astype(np.int32)


@pytest.fixture(scope="module")
def model05(ql, ctx):
    m = bench.Model(ctx, "0.5b", seed=0x9EF0, keep_tensors=True)
    yield m
    m.arena.release()


@pytest.mark.gpu
@pytest.mark.parametrize("M", [128, 512])
def test_prefill_config3_full_step(ql, ctx, orc, model05, M):
    """The timed config-3 launch: all 168 linears of the 0.5B step, each on its own fp16 input, as
    bench.py builds and replays it; every linear checked on 4 blocks of 64 columns."""
    st = bench.PrefillStep(ctx, model05, M)
    info = st.info
    say(f"config 3 M={M}: {info.as_dict()}")
    assert info.kernel == ql.SEQ_PREFILL and info.linears == 168
    st.capture()
    st.run(2)
    worst = 0.0
    for i, (layer, proj) in enumerate(st.order):
        t = model05.tensors[(layer, proj)]
        x = st.act.read(st.x_offs[i], (M, t.K), np.uint16).view(np.float16).astype(np.float32)
        y = st.act.read(st.y_offs[i], (M, t.N), np.float32)
        cols = _cols_sample(t.N)
        ref = orc.gptq_linear_cols(t.qweight, t.qzeros, t.scales, x, cols, None, bench.GROUP, w_f16=True)
        got = np.ascontiguousarray(y[:, cols])
        ok, max_abs, max_rel = orc.check_tolerance(got, ref, ATOL, RTOL)
        assert ok, f"M={M} linear {i} ({layer} {proj}): maxAbs {max_abs:.3e} maxRel {max_rel:.3e}"
        assert np.isfinite(y).all()
        worst = max(worst, float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)))
    say(f"  config 3 M={M}: 168 linears within bar, worst normwise {worst:.3e}")
    st.release()


def flip_bound(x, w_cols):
    """Per output [M, len(cols)]: the most that fp16 rounding of an fp32 activation computed
    slightly differently (within 16 fp32 ulps) can move y = f16(x) . W^T: sum over the
    activations within that distance of an fp16 rounding midpoint of one fp16 ulp times |w|."""
    x = np.asarray(x, dtype=np.float32)
    h = x.astype(np.float16)
    ulp16 = np.spacing(np.abs(h)).astype(np.float32)
    slack = ulp16 / 2 - np.abs(x - h.astype(np.float32))
    amb = slack <= 16 * np.spacing(np.abs(x))
    d = np.where(amb, ulp16, 0.0).astype(np.float64)
    return d @ np.abs(np.asarray(w_cols, dtype=np.float64)).T


@pytest.mark.gpu
@pytest.mark.parametrize("M", [128, 300])
def test_prefill_chained_step(ql, ctx, orc, model05, M):
    """The 0.5B step in the model's dependency order at M > 16 (runForward(M = T),
    qwen.ts:398-482) as one sequence: q/k/v <- rmsnorm(h), h1 = h + o(q), gate/up <- rmsnorm(h1),
    h2 = h1 + down(silu(gate) * up), 24 layers, run pass by pass (96 prefill launches with the
    RMSNorm and SiLU-mul launches between them, the residuals added at the stores). Every linear
    on sampled blocks against the oracle on the inputs the GPU produced: its RMSNorm or SiLU-mul
    in fp32, rounded to fp16 as the launch stages it, fp16 weights, the bar 1e-5 x the input's rms
    + 2e-3 |ref| plus the rounding ambiguity: the GPU's fp32 RMSNorm or SiLU-mul can differ from
    the oracle's in the last bits, and an activation within 16 fp32 ulps of an fp16 midpoint can
    round either way, moving each output by up to one fp16 ulp of that activation times |w|
    (flip_bound). Outputs stay finite to the last layer; a graph replay is bit-identical."""
    st = bench.SeqStep(ctx, model05, M, chained=True)
    info = st.info
    say(f"chained prefill M={M}: {info.as_dict()}")
    assert info.kernel == ql.SEQ_PREFILL_PASSES and info.passes == 96 and info.linears == 168
    st.run(2)
    assert st.finite()
    ql_none = (1 << 64) - 1
    y_of = {yo: i for i, yo in enumerate(st.y_offs)}
    ys = [st.act.read(yo, (M, model05.shapes[lp][1]), np.float32) for yo, lp in zip(st.y_offs, st.order)]

    def value(off, width):
        return ys[y_of[off]] if off in y_of else st.act.read(off, (M, width), np.float32)

    worst = 0.0
    for i, (lp, f) in enumerate(zip(st.order, st.fuse)):
        K, N = model05.shapes[lp]
        t = model05.tensors[lp]
        x = value(st.x_offs[i], K)
        if f.norm_w_off != ql_none:
            w = model05.arena.read(f.norm_w_off, (K,), np.float32)
            x = orc.add_rmsnorm(x, w, f.norm_eps)[1]
        if f.x2_off != ql_none:
            x = orc.silu_mul(x, value(f.x2_off, K))
        cols = _cols_sample(N)
        ref = orc.gptq_linear_cols(t.qweight, t.qzeros, t.scales, x16(x), cols, None, bench.GROUP, w_f16=True)
        if f.res_off != ql_none:
            ref = ref + value(f.res_off, N)[:, cols]
        got = np.ascontiguousarray(ys[i][:, cols])
        atol = 1e-5 * max(1.0, float(np.sqrt(np.mean(x.astype(np.float64) ** 2))))
        bar = atol + RTOL * np.abs(ref)
        if f.norm_w_off != ql_none or f.x2_off != ql_none:
            w16 = orc.dequantize_gptq_int4_f16(t.qweight, t.qzeros, t.scales, K, N, bench.GROUP)
            bar = bar + flip_bound(x, orc.f16_bits_to_f32(w16[cols]))
        err = np.abs(got.astype(np.float64) - ref)
        worst = max(worst, float(err.max() / max(np.abs(ref).max(), 1e-30)))
        k = np.unravel_index(np.argmax(err - bar), err.shape)
        assert (err <= bar).all(), (f"M={M} linear {i} {lp}: |d| {err[k]:.3e} > bar {bar[k]:.3e} at {k} "
                                    f"(ref {ref[k]:.3e})")
    say(f"  chained prefill M={M}: 168 linears within bar, worst normwise {worst:.3e}")
    # a graph replay of the whole pass-by-pass run gives the same bits
    ctx.graph_begin()
    st.seq.run()
    g = ctx.graph_end()
    for r in range(2):
        g.launch()
        st.seq.status()
        for a, (yo, lp) in zip(ys, zip(st.y_offs, st.order)):
            b = st.act.read(yo, (M, model05.shapes[lp][1]), np.float32)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"graph replay {r}"
    g.destroy()
    st.release()
