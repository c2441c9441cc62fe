"""GPU parity of fused sequences (ql_seq_create_fused): the Qwen layer's elementwise work folded
into one persistent launch of its linears, as the reference's layer runs it
(src/model/qwen.ts:403-478: rmsnorm -> q/k/v, o -> vec_add, rmsnorm -> gate/up -> silu_mul ->
down -> vec_add; o reads q in attention's place).

Every linear is checked on the inputs the GPU actually used (its producers' GPU outputs), against
the oracle's composition: rmsNormRef (orc_add_rmsnorm) or siluMulRef (orc_silu_mul) of those
inputs, then gemmNTRef over the quant.ts weights, plus the residual (vec_add in fp32), with the
single-GEMV bar |d| <= atol + 1e-4 |ref|, atol = 1e-5 * max(1, rms(input))."""
import sys

import numpy as np
import pytest

from webllm_amd import synth

pytestmark = pytest.mark.gpu

RTOL = 1e-4
EPS = 1e-6


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class FusedModel:
    """`layers` Qwen-shaped layers as one fused sequence: q/k/v <- rmsnorm(h, ln1);
    h1 = h + o(q); gate/up <- rmsnorm(h1, ln2); h2 = h1 + down(silu(gate) * up)."""

    def __init__(self, ql, ctx, M, layers, C, I, KV, seed=0xF05E, group=128):
        self.ql, self.M, self.group = ql, M, group
        wl, al = ql.ArenaLayout(), ql.ArenaLayout()
        self.h0 = synth.activations(M, C, seed=seed, key=(M,))
        self.h0_off = al.take(self.h0.nbytes)
        self.lin, self.norms = [], []
        fuse = []
        h = (self.h0_off, -1)
        for layer in range(layers):
            ln = []
            for k in range(2):
                w = 1.0 + 0.1 * synth.activations(1, C, seed=seed + 7, key=(layer, k))[0]
                ln.append((wl.take(w.nbytes), w))
            self.norms.extend(ln)
            for key, N in (("q", C), ("k", KV), ("v", KV)):
                self._add(wl, al, layer, key, C, N, h, {"norm": ln[0]}, biased=True)
                fuse.append(ql.make_fuse(norm_w_off=ln[0][0], norm_eps=EPS))
            q = self._ref(-3)
            self._add(wl, al, layer, "o", C, C, q, {"res": h})
            fuse.append(ql.make_fuse(res_off=h[0]))
            h1 = self._ref(-1)
            for key in ("gate", "up"):
                self._add(wl, al, layer, key, C, I, h1, {"norm": ln[1]})
                fuse.append(ql.make_fuse(norm_w_off=ln[1][0], norm_eps=EPS))
            g, u = self._ref(-2), self._ref(-1)
            self._add(wl, al, layer, "down", I, C, g, {"x2": u, "res": h1})
            fuse.append(ql.make_fuse(x2_off=u[0], res_off=h1[0]))
            h = self._ref(-1)
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
        for off, w in self.norms:
            self.weights.write(off, w.astype(np.float32))
        self.act.write(self.h0_off, self.h0)
        self.descs = [ql.make_desc(L["qw"], L["qz"], L["sc"], L["t"].K, L["t"].N, group, L["b"])
                      for L in self.lin]
        self.fuse = fuse
        self.seq = ctx.seq(self.descs, self.weights, self.act, [L["x"][0] for L in self.lin], 0, M,
                           [L["y_off"] for L in self.lin], fuse=fuse)

    def _ref(self, i):
        return (self.lin[i]["y_off"], len(self.lin) + i)

    def _add(self, wl, al, layer, key, K, N, x, extra, biased=False):
        idx = len(self.lin)
        sym = idx % 3 == 1
        t = synth.gptq_linear(K, N, self.group, seed=0xF05F, key=(layer, idx), stored_zero=7 if idx % 2 else None)
        bias = synth.activations(1, N, seed=0xF060, key=(layer, idx))[0] if biased else None
        L = {"t": t, "bias": bias, "qw": wl.take(t.qweight.nbytes),
             "qz": None if sym else wl.take(t.qzeros.nbytes), "sc": wl.take(t.scales.nbytes),
             "b": None if bias is None else wl.take(bias.nbytes), "x": x,
             "y_off": al.take(self.M * N * 4), "name": f"L{layer}.{key}", **extra}
        L["qzeros"] = None if sym else t.qzeros
        self.lin.append(L)

    def outputs(self):
        return [self.act.read(L["y_off"], (self.M, L["t"].N), np.float32) for L in self.lin]

    def value(self, ref, ys):
        off, src = ref
        return self.h0 if src < 0 else ys[src]

    def release(self):
        self.seq.destroy()
        self.weights.release()
        self.act.release()


def check_fused(orc, m: FusedModel, ys, label, cols_for=None):
    worst = 0.0
    for L, y in zip(m.lin, ys):
        t = L["t"]
        x = m.value(L["x"], ys)
        if "norm" in L:
            x = orc.add_rmsnorm(x, L["norm"][1], EPS)[1]
        if "x2" in L:
            x = orc.silu_mul(x, m.value(L["x2"], ys))
        if cols_for is None:
            cols = np.arange(t.N, dtype=np.int32)
            ref = orc.gptq_linear(t.qweight, L["qzeros"], t.scales, x, L["bias"], m.group)
        else:
            cols = cols_for(t.N)
            ref = orc.gptq_linear_cols(t.qweight, L["qzeros"], t.scales, x, cols, L["bias"], m.group)
        if "res" in L:
            ref = ref + m.value(L["res"], ys)[:, cols]        # vec_add in fp32
        got = np.ascontiguousarray(y[:, cols])
        atol = 1e-5 * max(1.0, float(np.sqrt(np.mean(x.astype(np.float64) ** 2))))
        ok, max_abs, max_rel = orc.check_tolerance(got, ref, atol, RTOL)
        assert np.isfinite(y).all(), f"{label} {L['name']}: non-finite output"
        worst = max(worst, float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)))
        assert ok, f"{label} {L['name']}: maxAbs {max_abs:.3e} (atol {atol:.2e}) maxRel {max_rel:.3e}"
    say(f"  {label}: {len(ys)} linears within bar, worst normwise {worst:.3e}")


@pytest.mark.parametrize("M", [1, 4, 8, 16])
def test_fused_layers_05b(ql, ctx, orc, M):
    """Two 0.5B-shaped layers (14 linears, 8 dependent passes) in one fused launch; repeated runs
    and graph replays are bit-identical (fixed reduction orders, epochs instead of clears)."""
    m = FusedModel(ql, ctx, M, 2, 896, 4864, 128)
    info = m.seq.info
    say(f"fused 0.5B x2 M={M}: {info.as_dict()}")
    assert info.kernel == ql.SEQ_TILES and info.passes == 8 and info.linears == 14
    m.seq.run()
    m.seq.status()
    ys = m.outputs()
    check_fused(orc, m, ys, f"fused 0.5B M={M}")
    last = m.lin[-1]
    zero = np.zeros((M, last["t"].N), np.float32)
    m.act.write(last["y_off"], zero)
    m.seq.run()
    m.seq.status()
    for a, b in zip(ys, m.outputs()):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    ctx.graph_begin()
    m.seq.run()
    g = ctx.graph_end()
    for r in range(3):
        m.act.write(last["y_off"], zero)
        g.launch()
        m.seq.status()
        for a, b in zip(ys, m.outputs()):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"graph replay {r}"
    g.destroy()
    m.release()


@pytest.mark.parametrize("M", [1, 16])
def test_fused_silu_mul_external_operand(ql, ctx, orc, M):
    """The SiLU-mul second operand from an external [M, I] buffer (x2_off not another linear's
    output): gate and up run as one pass, down reads silu(gate) * up_ext where up_ext was written
    by the host; every output against siluMulRef + gemmNTRef on the GPU's gate output."""
    C, I = 896, 4864
    wl, al = ql.ArenaLayout(), ql.ArenaLayout()
    tg = synth.gptq_linear(C, I, 128, seed=0xE2A, key=(0,))
    td = synth.gptq_linear(I, C, 128, seed=0xE2A, key=(1,))
    offs = []
    for t in (tg, td):
        offs.append((wl.take(t.qweight.nbytes), wl.take(t.qzeros.nbytes), wl.take(t.scales.nbytes)))
    x = synth.activations(M, C, seed=0xE2B, key=(M,))
    up = synth.activations(M, I, seed=0xE2C, key=(M,))
    x_off, g_off, u_off, y_off = al.take(x.nbytes), al.take(M * I * 4), al.take(up.nbytes), al.take(M * C * 4)
    w = ctx.arena(wl.used)
    for t, (a, b, c) in zip((tg, td), offs):
        w.write(a, t.qweight)
        w.write(b, t.qzeros)
        w.write(c, t.scales)
    act = ctx.arena(al.used)
    act.write(x_off, x)
    act.write(u_off, up)
    descs = [ql.make_desc(*offs[0], C, I, 128), ql.make_desc(*offs[1], I, C, 128)]
    fuse = [ql.make_fuse(), ql.make_fuse(x2_off=u_off)]
    seq = ctx.seq(descs, w, act, [x_off, g_off], 0, M, [g_off, y_off], fuse=fuse)
    assert seq.info.kernel == ql.SEQ_TILES and seq.info.passes == 2
    seq.run()
    seq.status()
    g = act.read(g_off, (M, I), np.float32)
    y = act.read(y_off, (M, C), np.float32)
    ok, ma, mr = orc.check_tolerance(g, orc.gptq_linear(tg.qweight, tg.qzeros, tg.scales, x), 1e-5, RTOL)
    assert ok, ("gate", ma, mr)
    h = orc.silu_mul(g, up)
    ref = orc.gptq_linear(td.qweight, td.qzeros, td.scales, h)
    atol = 1e-5 * max(1.0, float(np.sqrt(np.mean(h.astype(np.float64) ** 2))))
    ok, ma, mr = orc.check_tolerance(y, ref, atol, RTOL)
    assert ok, ("down", ma, mr)
    seq.destroy()
    w.release()
    act.release()


def _sample(N, count=4):
    nb = N // 64
    picks = sorted(set([0, nb - 1] + [int(round(i * (nb - 1) / (count - 1))) for i in range(count)]))
    return np.concatenate([np.arange(b * 64, b * 64 + 64) for b in picks]).astype(np.int32)


@pytest.mark.parametrize("M", [1, 16])
def test_fused_layer_7b(ql, ctx, orc, M):
    """One 7B-shaped layer (q/o 3584, gate/up 18944, down 18944 -> 3584, 4 KV heads of 128 for
    k/v): RMSNorm over 3584-wide rows, SiLU-mul over 18944, both residuals; sampled columns."""
    m = FusedModel(ql, ctx, M, 1, 3584, 18944, 512)
    info = m.seq.info
    say(f"fused 7B x1 M={M}: {info.as_dict()}")
    assert info.kernel == ql.SEQ_TILES and info.passes == 4
    m.seq.run()
    m.seq.status()
    check_fused(orc, m, m.outputs(), f"fused 7B M={M}", cols_for=_sample)
    m.release()


def check_step(orc, model, st, cols_for, label):
    """A chained bench step (bench.SeqStep(chained=True)): every linear against the oracle's
    composition on the inputs the GPU used, its fusion read from the step's own fuse list."""
    ql_none = (1 << 64) - 1
    y_of = {yo: i for i, yo in enumerate(st.y_offs)}
    ys = [st.act.read(yo, (st.M, model.shapes[lp][1]), np.float32) for yo, lp in zip(st.y_offs, st.order)]

    def value(off, width):
        return ys[y_of[off]] if off in y_of else st.act.read(off, (st.M, width), np.float32)

    worst = 0.0
    for i, (lp, f) in enumerate(zip(st.order, st.fuse)):
        K, N = model.shapes[lp]
        t = model.tensors[lp]
        x = value(st.x_offs[i], K)
        if f.norm_w_off != ql_none:
            w = model.arena.read(f.norm_w_off, (K,), np.float32)
            x = orc.add_rmsnorm(x, w, f.norm_eps)[1]
        if f.x2_off != ql_none:
            x = orc.silu_mul(x, value(f.x2_off, K))
        cols = cols_for(N)
        ref = orc.gptq_linear_cols(t.qweight, t.qzeros, t.scales, x, cols, None, 128)
        if f.res_off != ql_none:
            ref = ref + value(f.res_off, N)[:, cols]
        got = np.ascontiguousarray(ys[i][:, cols])
        atol = 1e-5 * max(1.0, float(np.sqrt(np.mean(x.astype(np.float64) ** 2))))
        ok, max_abs, max_rel = orc.check_tolerance(got, ref, atol, RTOL)
        assert np.isfinite(ys[i]).all(), f"{label} linear {i} {lp}: non-finite output"
        worst = max(worst, float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)))
        assert ok, f"{label} linear {i} {lp}: maxAbs {max_abs:.3e} (atol {atol:.2e}) maxRel {max_rel:.3e}"
    say(f"  {label}: {len(ys)} linears within bar, worst normwise {worst:.3e}")


@pytest.fixture(scope="module")
def bench_mod():
    import bench
    return bench


def test_chained_step_05b_full_size(ql, ctx, orc, bench_mod):
    """The bench's chained 0.5B step (24 fused layers, 96 passes, one launch) at M=1: every
    linear's every column against the oracle; the values stay finite to the last layer."""
    model = bench_mod.Model(ctx, "0.5b", seed=0x9EF0, keep_tensors=True)
    st = bench_mod.SeqStep(ctx, model, 1, chained=True)
    say(f"chained 0.5B step: {st.info.as_dict()}")
    assert st.info.kernel == ql.SEQ_TILES and st.info.passes == 96 and st.info.linears == 168
    st.run(2)
    assert st.finite()
    check_step(orc, model, st, lambda N: np.arange(N, dtype=np.int32), "chained 0.5B M=1")
    st.release()
    model.arena.release()


def test_chained_step_05b_bounded_waits_abort(ql, ctx, orc, bench_mod):
    """The pass-break contract (qwen.ts:556-559) made safe: with a spin limit of 64 polls the
    kernel's own bounded waits give up on the chained 0.5B step (96 dependent passes), every
    workgroup exits, and ql_seq_status reports QL_E_STATE; after the default limit is restored the
    next run completes and matches the oracle."""
    model = bench_mod.Model(ctx, "0.5b", seed=0x9EF0, keep_tensors=True)
    st = bench_mod.SeqStep(ctx, model, 1, chained=True)
    assert st.info.kernel == ql.SEQ_TILES and st.info.passes == 96
    st.seq.set_spin_limit(64)
    say("chained 0.5B step, spin limit 64: expecting an abort")
    st.seq.run()
    with pytest.raises(ql.QlError) as exc:
        st.seq.status()
    assert exc.value.name == "QL_E_STATE", exc.value
    say(f"  aborted as expected: {exc.value}")
    st.seq.set_spin_limit(1 << 22)
    st.seq.run()
    st.seq.status()
    assert st.finite()
    check_step(orc, model, st, lambda N: np.arange(N, dtype=np.int32), "chained 0.5B M=1 after abort")
    st.release()
    model.arena.release()


@pytest.fixture(scope="module")
def model7b_chained(ctx, bench_mod):
    m = bench_mod.Model(ctx, "7b", seed=0x7B, keep_tensors=True)
    yield m
    m.arena.release()


@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
def test_chained_step_7b_full_size(ql, ctx, orc, bench_mod, model7b_chained, M):
    """The bench's chained 7B step (28 fused layers, 112 passes, 3.35 GB) at every M bench times
    it: one launch of dependency-ordered tiles at M = 1, pass by pass at M >= 2 (K-part strips
    that RMSNorm-weight or SiLU-mul their activations as they stage them, then part sums with the
    row's 1/rms, bias, residual and the next norm's row sums of squares); every linear on a sample
    of 64-column blocks; finite to the last layer."""
    model = model7b_chained
    st = bench_mod.SeqStep(ctx, model, M, chained=True)
    say(f"chained 7B step M={M}: {st.info.as_dict()}")
    assert st.info.kernel == (ql.SEQ_STRIP_PASSES if M >= 2 else ql.SEQ_TILES) and st.info.passes == 112
    st.run(2)
    assert st.finite()
    check_step(orc, model, st, _sample, f"chained 7B M={M}")
    st.release()
