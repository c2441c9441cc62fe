"""GPU parity: libqlinear.so (called through its C ABI) against the CPU oracle on the same bytes.

Bars: dequant bit-exact; GEMV |d| <= 1e-5 + 1e-4*|ref| against fp32
weights with double accumulation (gemmNTRef, src/reference/qwen-ref.ts:126-145); MFMA GEMM
|d| <= 1e-5 + 2e-3*|ref| against the oracle on fp16-rounded x and W.
"""
import sys

import numpy as np
import pytest

from webllm_amd import synth

pytestmark = pytest.mark.gpu

GEMV_ATOL, GEMV_RTOL = 1e-5, 1e-4
GEMM_ATOL, GEMM_RTOL = 1e-5, 2e-3


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class Linear:
    """One GPTQ linear uploaded to its own weight arena."""

    def __init__(self, ql, ctx, t: synth.GptqTensors, bias=None, no_qzeros=False):
        lay = ql.ArenaLayout()
        qw_off = lay.take(t.qweight.nbytes)
        qz_off = None if no_qzeros else lay.take(t.qzeros.nbytes)
        sc_off = lay.take(t.scales.nbytes)
        b_off = None if bias is None else lay.take(bias.nbytes)
        self.arena = ctx.arena(lay.used)
        self.arena.write(qw_off, t.qweight)
        if qz_off is not None:
            self.arena.write(qz_off, t.qzeros)
        self.arena.write(sc_off, t.scales)
        if bias is not None:
            self.arena.write(b_off, bias)
        self.desc = ql.make_desc(qw_off, qz_off, sc_off, t.K, t.N, t.group, b_off)
        self.t = t
        self.bias = bias
        self.qzeros = None if no_qzeros else t.qzeros


def run_linear(ql, ctx, lin: Linear, x: np.ndarray, x_dtype=0):
    M, K = x.shape
    N = lin.t.N
    plan = ql.plan_linear(M, N, K, lin.t.group)
    lay = ql.ArenaLayout()
    x_off = lay.take(x.nbytes)
    y_off = lay.take(M * N * 4)
    s_off = lay.take(max(plan.scratch_bytes, 16))
    act = ctx.arena(lay.used)
    act.write(x_off, x)
    ctx.linear(lin.desc, lin.arena, act, x_off, x_dtype, M, y_off, s_off)
    y = act.read(y_off, (M, N), np.float32)
    act.release()
    return y, plan


def oracle_gemv(orc, lin: Linear, x):
    return orc.gptq_linear(lin.t.qweight, lin.qzeros, lin.t.scales, x, lin.bias, lin.t.group)


def assert_close(orc, got, ref, atol, rtol, label):
    ok, max_abs, max_rel = orc.check_tolerance(got, ref, atol, rtol)
    norm = float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))
    say(f"  {label}: maxAbs={max_abs:.3e} maxRel={max_rel:.3e} normwise={norm:.3e}")
    assert ok, f"{label}: |d| > {atol} + {rtol}|ref| (maxAbs {max_abs:.3e})"


# ------------------------------------------------------------------------- load-time unpack

UNPACK_CASES = [
    # (K, N, group, stored_zero, no_qzeros, label)
    (896, 4864, 128, 7, False, "0.5B gate"),
    (4864, 896, 128, None, False, "0.5B down, random zeros"),
    (896, 128, 128, 7, True, "0.5B k, no qzeros"),
    (16, 5, 8, None, False, "reference KAT shape"),
    (20, 13, 8, None, False, "K%8!=0, N%8!=0 (generic)"),
    (136, 12, 8, 15, False, "zero 16"),
    (256, 64, 64, None, False, "group 64"),
]


@pytest.mark.parametrize("K,N,group,zero,noqz,label", UNPACK_CASES)
def test_unpack_bitexact(ql, ctx, orc, K, N, group, zero, noqz, label):
    say(f"unpack {label}: K={K} N={N} group={group}")
    t = synth.gptq_linear(K, N, group, seed=0x7A11, key=(K, N), stored_zero=zero)
    lin = Linear(ql, ctx, t, no_qzeros=noqz)
    out = ctx.arena(N * K * 2 + 256)
    ctx.unpack_f16(lin.desc, lin.arena, out, 0)
    got = out.read(0, (N, K), np.uint16)
    want = orc.dequantize_gptq_int4_f16(t.qweight, lin.qzeros, t.scales, K, N, group)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} mismatches, first at {bad[:4]}"


def test_unpack_subnormal_overflow_scales(ql, ctx, orc):
    """fp16-subnormal scales (about 0.5% of |N(0,1)|*0.01), the smallest subnormal, and large
    scales whose products overflow to +-Inf, all bit-exact."""
    K, N = 512, 256
    t = synth.gptq_linear(K, N, 128, seed=0x5AB, stored_zero=None)
    s = t.scales.view(np.float16).copy()
    s[0, :64] = np.float16(2.0 ** -20)
    s[1, :32] = np.float16(2.0 ** -24)
    s[1, 32:64] = np.float16(6.1e-5)
    s[2, :16] = np.float16(8192.0)
    s[3, :16] = np.float16(65504.0)
    t.scales = s.view(np.uint16)
    lin = Linear(ql, ctx, t)
    out = ctx.arena(N * K * 2)
    ctx.unpack_f16(lin.desc, lin.arena, out, 0)
    got = out.read(0, (N, K), np.uint16)
    want = orc.dequantize_gptq_int4_f16(t.qweight, t.qzeros, t.scales, K, N, 128)
    assert np.array_equal(got, want)
    assert np.any(got == 0x7C00) or np.any(got == 0xFC00)


def test_unpack_all_168_tensors_05b(ql, ctx, orc):
    """Config 5: every int4 tensor of a Qwen2.5-0.5B-shaped model into one fp16 [N,K] arena."""
    linears = synth.model_linears("0.5b")
    lay = ql.ArenaLayout()
    tensors, offs = [], []
    for (layer, proj, K, N) in linears:
        t = synth.gptq_linear(K, N, 128, seed=0xC5, key=(layer, synth.PROJ_INDEX[proj]))
        tensors.append(t)
        offs.append((lay.take(t.qweight.nbytes), lay.take(t.qzeros.nbytes), lay.take(t.scales.nbytes)))
    w = ctx.arena(lay.used)
    olay = ql.ArenaLayout()
    out_offs = [olay.take(t.N * t.K * 2) for t in tensors]
    out = ctx.arena(olay.used)
    say(f"unpack 168 tensors: packed {lay.used/1e6:.1f} MB -> fp16 {olay.used/1e6:.1f} MB")
    descs = []
    for t, (a, b, c), o in zip(tensors, offs, out_offs):
        w.write(a, t.qweight); w.write(b, t.qzeros); w.write(c, t.scales)
        descs.append(ql.make_desc(a, b, c, t.K, t.N, 128))
        ctx.unpack_f16(descs[-1], w, out, o)
    ctx.sync()
    wants = []
    for i, (t, o) in enumerate(zip(tensors, out_offs)):
        got = out.read(o, (t.N, t.K), np.uint16)
        wants.append(orc.dequantize_gptq_int4_f16(t.qweight, t.qzeros, t.scales, t.K, t.N, 128))
        assert np.array_equal(got, wants[i]), f"tensor {i} {linears[i]}"
    # the batched entry point (the loader's whole weight set in six launches) into a cleared arena
    out.release()
    out = ctx.arena(olay.used)
    out.write(0, np.full(olay.used // 2, 0xFFFF, np.uint16))
    ctx.unpack_f16_batch(descs, w, out, out_offs)
    ctx.sync()
    for i, (t, o) in enumerate(zip(tensors, out_offs)):
        got = out.read(o, (t.N, t.K), np.uint16)
        assert np.array_equal(got, wants[i]), f"batched: tensor {i} {linears[i]}"
    out.release()
    w.release()


def test_unpack_batch_mixed_shapes(ql, ctx, orc):
    """The batched unpack over tensors the tile path takes and tensors it does not (ragged K or N,
    no qzeros, group 32/64/256, an odd output offset) in one call: each bit-exact, nothing written
    outside its [N,K] range."""
    shapes = [  # (K, N, group, no_qzeros, out_misalign)
        (896, 4864, 128, False, 0), (128, 64, 128, True, 0), (1000, 96, 8, False, 0),
        (896, 130, 128, False, 0), (256, 4, 32, False, 0), (512, 68, 64, True, 0),
        (2048, 516, 256, False, 0), (896, 128, 128, False, 2), (24, 12, 8, False, 0),
    ] * 5   # 45 tensors: more than one launch's worth
    lay = ql.ArenaLayout()
    tensors, offs = [], []
    for i, (K, N, group, noqz, _) in enumerate(shapes):
        t = synth.gptq_linear(K, N, group, seed=0xB0 + i)
        tensors.append((t, noqz))
        offs.append((lay.take(t.qweight.nbytes), None if noqz else lay.take(t.qzeros.nbytes),
                     lay.take(t.scales.nbytes)))
    w = ctx.arena(lay.used)
    olay = ql.ArenaLayout()
    out_offs = [olay.take(t.N * t.K * 2 + 16) + mis for (t, _), (_, _, _, _, mis) in zip(tensors, shapes)]
    out = ctx.arena(olay.used)
    out.write(0, np.full(olay.used // 2, 0xFFFF, np.uint16))
    descs = []
    for (t, noqz), (a, b, c) in zip(tensors, offs):
        w.write(a, t.qweight)
        if b is not None:
            w.write(b, t.qzeros)
        w.write(c, t.scales)
        descs.append(ql.make_desc(a, b, c, t.K, t.N, t.group))
    say(f"unpack batch: {len(descs)} tensors, {olay.used/1e6:.1f} MB out")
    ctx.unpack_f16_batch(descs, w, out, out_offs)
    ctx.sync()
    for i, ((t, noqz), o) in enumerate(zip(tensors, out_offs)):
        got = out.read(o, (t.N, t.K), np.uint16)
        want = orc.dequantize_gptq_int4_f16(t.qweight, None if noqz else t.qzeros, t.scales, t.K,
                                            t.N, t.group)
        assert np.array_equal(got, want), f"tensor {i} {shapes[i]}"
        tail = out.read(o + t.N * t.K * 2, (8 - (o % 16) // 2,), np.uint16)
        assert np.all(tail == 0xFFFF), f"tensor {i}: write past its end"
    out.release()
    w.release()


# ------------------------------------------------------------------------- decode GEMV

GEMV_CASES = [
    # (K, N, M, stored_zero, bias, label)
    (896, 4864, 1, 7, False, "cfg1 gate M=1"),
    (896, 4864, 2, 7, False, "gate M=2"),
    (896, 4864, 4, None, False, "gate M=4 random zeros"),
    (896, 4864, 8, 7, False, "gate M=8"),
    (896, 4864, 16, None, False, "gate M=16 random zeros"),
    (896, 896, 1, 7, True, "q +bias"),
    (896, 128, 1, 7, True, "k +bias"),
    (4864, 896, 1, None, False, "down"),
    (4864, 896, 9, 7, False, "down M=9"),
    (3584, 18944, 1, 7, False, "7B gate M=1"),
    (18944, 3584, 4, 7, False, "7B down M=4"),
    (3584, 3584, 16, None, False, "7B q M=16"),
]


@pytest.mark.parametrize("K,N,M,zero,with_bias,label", GEMV_CASES)
def test_gemv_parity(ql, ctx, orc, K, N, M, zero, with_bias, label):
    t = synth.gptq_linear(K, N, 128, seed=0x9EF0, key=(K, N), stored_zero=zero)
    bias = synth.activations(1, N, seed=0xB1A5, key=(N,))[0] if with_bias else None
    x = synth.activations(M, K, seed=0x9EF1, key=(K, M))
    lin = Linear(ql, ctx, t, bias=bias)
    plan = ql.plan_linear(M, N, K)
    say(f"gemv {label}: M={M} K={K} N={N} kind={plan.kind_name} split={plan.split}")
    y, _ = run_linear(ql, ctx, lin, x)
    ref = oracle_gemv(orc, lin, x)
    assert plan.kind_name == "gemv_mfma"
    assert_close(orc, y, ref, GEMV_ATOL, GEMV_RTOL, label)


@pytest.mark.parametrize("group,M", [(32, 1), (64, 3), (256, 2), (32, 7), (64, 12), (256, 16)])
def test_gemv_group_sizes(ql, ctx, orc, group, M):
    """GPTQ group sizes 64/256 on the MFMA path (1, 2 and 4 row tiles); group 32 (smaller than
    one 64-k MFMA block) on the generic kernel."""
    K, N = 1024, 512
    t = synth.gptq_linear(K, N, group, seed=0x6A, key=(group, M), stored_zero=None)
    x = synth.activations(M, K, seed=0x6B, key=(group, M))
    lin = Linear(ql, ctx, t)
    y, plan = run_linear(ql, ctx, lin, x)
    assert plan.kind_name == ("gemv_simple" if group == 32 else "gemv_mfma")
    assert_close(orc, y, oracle_gemv(orc, lin, x), GEMV_ATOL, GEMV_RTOL, f"group {group} M={M}")


def test_gemv_activation_range(ql, ctx, orc):
    """Per-group power-of-two range normalisation: huge, tiny and zero activation groups."""
    K, N, M = 1024, 256, 2
    t = synth.gptq_linear(K, N, 128, seed=0x6C)
    x = synth.activations(M, K, seed=0x6D)
    x[0, :128] *= 3.0e4          # |x| up to ~1e5, beyond fp16 range
    x[0, 128:256] *= 1e-6
    x[1, 256:384] = 0.0
    x[1, 384:512] *= 1e-30
    lin = Linear(ql, ctx, t)
    for M_ in (1, 2):
        y, _ = run_linear(ql, ctx, lin, np.ascontiguousarray(x[:M_]))
        ref = oracle_gemv(orc, lin, x[:M_])
        assert_close(orc, y, ref, GEMV_ATOL, GEMV_RTOL, f"range M={M_}")
    xb = np.concatenate([x] * 4)            # M = 8: prepared-activation path
    y, _ = run_linear(ql, ctx, lin, xb)
    assert_close(orc, y, oracle_gemv(orc, lin, xb), GEMV_ATOL, GEMV_RTOL, "range M=8")


def test_gemv_f16_activations(ql, ctx, orc):
    K, N, M = 896, 896, 3
    t = synth.gptq_linear(K, N, 128, seed=0x16)
    x16 = synth.activations(M, K, seed=0x17).astype(np.float16)
    lin = Linear(ql, ctx, t)
    y, _ = run_linear(ql, ctx, lin, x16.view(np.uint16), x_dtype=1)
    ref = oracle_gemv(orc, lin, x16.astype(np.float32))
    assert_close(orc, y, ref, GEMV_ATOL, GEMV_RTOL, "f16 x")


def test_gemv_deterministic(ql, ctx):
    """Split-K partials are reduced in fixed ascending order: repeated runs are bit-identical."""
    K, N, M = 18944, 3584, 2
    t = synth.gptq_linear(K, N, 128, seed=0xDE7)
    x = synth.activations(M, K, seed=0xDE8)
    lin = Linear(ql, ctx, t)
    assert ql.plan_linear(M, N, K).split > 1
    ys = [run_linear(ql, ctx, lin, x)[0] for _ in range(3)]
    assert all(np.array_equal(ys[0].view(np.uint32), y.view(np.uint32)) for y in ys[1:])


def test_batch_matches_single(ql, ctx, orc):
    """q/k/v on one input in one launch == three separate launches (bit-identical)."""
    K = 896
    ts = [synth.gptq_linear(K, n, 128, seed=0xBA7, key=(i,)) for i, n in enumerate((896, 128, 128))]
    biases = [synth.activations(1, t.N, seed=0xBA8, key=(i,))[0] for i, t in enumerate(ts)]
    lins = [Linear(ql, ctx, t, bias=b) for t, b in zip(ts, biases)]
    # one shared weight arena is required by the batch entry point: repack
    lay = ql.ArenaLayout()
    descs, parts = [], []
    for t, b in zip(ts, biases):
        a, z, s, bo = lay.take(t.qweight.nbytes), lay.take(t.qzeros.nbytes), lay.take(t.scales.nbytes), lay.take(b.nbytes)
        parts.append((a, z, s, bo, t, b))
        descs.append(ql.make_desc(a, z, s, K, t.N, 128, bo))
    w = ctx.arena(lay.used)
    for a, z, s, bo, t, b in parts:
        w.write(a, t.qweight); w.write(z, t.qzeros); w.write(s, t.scales); w.write(bo, b)
    for M in (1, 5, 16):
        x = synth.activations(M, K, seed=0xBA9, key=(M,))
        scratch = ql.plan_batch(descs, M)
        alay = ql.ArenaLayout()
        x_off = alay.take(x.nbytes)
        y_offs = [alay.take(M * t.N * 4) for t in ts]
        s_off = alay.take(scratch)
        act = ctx.arena(alay.used)
        act.write(x_off, x)
        ctx.linear_batch(descs, w, act, [x_off] * 3, 0, M, y_offs, s_off)
        for lin, yo, t in zip(lins, y_offs, ts):
            yb = act.read(yo, (M, t.N), np.float32)
            ys, _ = run_linear(ql, ctx, lin, x)
            assert np.array_equal(yb.view(np.uint32), ys.view(np.uint32))
            assert_close(orc, yb, oracle_gemv(orc, lin, x), GEMV_ATOL, GEMV_RTOL, f"batch M={M} N={t.N}")


# ------------------------------------------------------------------------- prefill GEMM

GEMM_CASES = [
    (896, 4864, 128, 7, "cfg3 gate M=128"),
    (4864, 896, 64, None, "down M=64"),
    (896, 896, 512, 7, "q M=512"),
    (896, 128, 17, 7, "k M=17 (ragged tiles)"),
    (896, 4864, 100, None, "gate M=100 ragged"),
]


@pytest.mark.parametrize("K,N,M,zero,label", GEMM_CASES)
def test_gemm_parity(ql, ctx, orc, K, N, M, zero, label):
    t = synth.gptq_linear(K, N, 128, seed=0x6E33, key=(K, N, M), stored_zero=zero)
    bias = synth.activations(1, N, seed=0x6E34, key=(N,))[0]
    x = synth.activations(M, K, seed=0x6E35, key=(K, M))
    lin = Linear(ql, ctx, t, bias=bias)
    plan = ql.plan_linear(M, N, K)
    say(f"gemm {label}: M={M} K={K} N={N} kind={plan.kind_name}")
    assert plan.kind_name == "gemm_mfma"
    for x_dtype in (0, 1):
        xin = x if x_dtype == 0 else x.astype(np.float16).view(np.uint16)
        y, _ = run_linear(ql, ctx, lin, xin, x_dtype)
        W16 = orc.f16_bits_to_f32(orc.dequantize_gptq_int4_f16(t.qweight, t.qzeros, t.scales, K, N, 128))
        x16 = orc.f16_bits_to_f32(orc.f32_to_f16_bits(x))
        ref = orc.gemm_nt(x16, W16, bias)
        assert_close(orc, y, ref, GEMM_ATOL, GEMM_RTOL, f"{label} x_dtype={x_dtype}")
        ref32 = oracle_gemv(orc, lin, x)   # against the pure-fp32 oracle, reported only
        say(f"    vs fp32 oracle normwise={np.abs(y-ref32).max()/np.abs(ref32).max():.3e}")


def _gemm_ref(orc, t, x, bias, qzeros):
    W16 = orc.f16_bits_to_f32(orc.dequantize_gptq_int4_f16(t.qweight, qzeros, t.scales, t.K, t.N, t.group))
    x16 = orc.f16_bits_to_f32(orc.f32_to_f16_bits(x))
    return orc.gemm_nt(x16, W16, bias)


GEMM_SHAPE_CASES = [
    # (K, N, M, group, no_qzeros, label): K steps per group 1, 2, 8; absent qzeros; 128-row tiles
    (512, 320, 40, 32, False, "group 32"),
    (1024, 708, 65, 64, False, "group 64, N % 256 != 0"),
    (2048, 516, 96, 256, True, "group 256, no qzeros"),
    (256, 4864, 1800, 128, False, "128-row tiles, ragged M"),
]


@pytest.mark.parametrize("K,N,M,group,noqz,label", GEMM_SHAPE_CASES)
def test_gemm_shapes(ql, ctx, orc, K, N, M, group, noqz, label):
    t = synth.gptq_linear(K, N, group, seed=0x6E40, key=(K, N, M, group))
    bias = synth.activations(1, N, seed=0x6E41, key=(N,))[0]
    x = synth.activations(M, K, seed=0x6E42, key=(K, M))
    lin = Linear(ql, ctx, t, bias=bias, no_qzeros=noqz)
    plan = ql.plan_linear(M, N, K, group)
    say(f"gemm {label}: M={M} K={K} N={N} group={group} split={plan.split} grid={plan.grid_x}")
    assert plan.kind_name == "gemm_mfma"
    ref = _gemm_ref(orc, t, x, bias, lin.qzeros)
    for x_dtype in (0, 1):
        xin = x if x_dtype == 0 else x.astype(np.float16).view(np.uint16)
        y, _ = run_linear(ql, ctx, lin, xin, x_dtype)
        assert_close(orc, y, ref, GEMM_ATOL, GEMM_RTOL, f"{label} x_dtype={x_dtype}")


def test_gemm_batch_and_determinism(ql, ctx, orc):
    """q/k/v (M=128, f16 input) as one batched GEMM launch: each output matches its own launch
    bit for bit, split-K results repeat exactly, and all meet the GEMM bar."""
    K, M = 896, 128
    ts = [synth.gptq_linear(K, n, 128, seed=0x6E50, key=(i,)) for i, n in enumerate((896, 128, 128))]
    biases = [synth.activations(1, t.N, seed=0x6E51, key=(i,))[0] for i, t in enumerate(ts)]
    lay = ql.ArenaLayout()
    descs, parts = [], []
    for t, b in zip(ts, biases):
        a, z, s_, bo = lay.take(t.qweight.nbytes), lay.take(t.qzeros.nbytes), lay.take(t.scales.nbytes), lay.take(b.nbytes)
        parts.append((a, z, s_, bo, t, b))
        descs.append(ql.make_desc(a, z, s_, K, t.N, 128, bo))
    w = ctx.arena(lay.used)
    for a, z, s_, bo, t, b in parts:
        w.write(a, t.qweight); w.write(z, t.qzeros); w.write(s_, t.scales); w.write(bo, b)
    assert any(ql.plan_linear(M, t.N, K).split > 1 for t in ts)
    x = synth.activations(M, K, seed=0x6E52)
    x16 = x.astype(np.float16).view(np.uint16)
    scratch = ql.plan_batch(descs, M)
    alay = ql.ArenaLayout()
    x_off = alay.take(x16.nbytes)
    y_offs = [alay.take(M * t.N * 4) for t in ts]
    s_off = alay.take(max(scratch, 16))
    act = ctx.arena(alay.used)
    act.write(x_off, x16)
    ctx.linear_batch(descs, w, act, [x_off] * 3, 1, M, y_offs, s_off)
    first = [act.read(yo, (M, t.N), np.float32) for yo, t in zip(y_offs, ts)]
    for _ in range(3):
        ctx.linear_batch(descs, w, act, [x_off] * 3, 1, M, y_offs, s_off)
        for yo, t, f in zip(y_offs, ts, first):
            assert np.array_equal(act.read(yo, (M, t.N), np.float32).view(np.uint32), f.view(np.uint32))
    for d, yo, t, b, f in zip(descs, y_offs, ts, biases, first):
        ctx.linear(d, w, act, x_off, 1, M, yo, s_off)
        assert np.array_equal(act.read(yo, (M, t.N), np.float32).view(np.uint32), f.view(np.uint32))
        assert_close(orc, f, _gemm_ref(orc, t, x, b, t.qzeros), GEMM_ATOL, GEMM_RTOL, f"batch N={t.N}")


def test_gemm_batch_fills_device_without_split(ql, ctx, orc):
    """Eight linears on their own f16 inputs in one launch whose tiles together fill the device:
    no linear splits K (each would alone), every output meets the GEMM bar, and repeats are
    bit-identical."""
    K, N, M = 512, 4096, 64
    assert ql.plan_linear(M, N, K).split > 1
    ts = [synth.gptq_linear(K, N, 128, seed=0x6E60, key=(i,), stored_zero=None) for i in range(8)]
    lay = ql.ArenaLayout()
    descs = []
    for t in ts:
        a, z, s_ = lay.take(t.qweight.nbytes), lay.take(t.qzeros.nbytes), lay.take(t.scales.nbytes)
        descs.append((a, z, s_, t))
    w = ctx.arena(lay.used)
    for a, z, s_, t in descs:
        w.write(a, t.qweight); w.write(z, t.qzeros); w.write(s_, t.scales)
    descs = [ql.make_desc(a, z, s_, K, N, 128) for a, z, s_, _ in descs]
    xs = [synth.activations(M, K, seed=0x6E61, key=(i,)) for i in range(8)]
    alay = ql.ArenaLayout()
    x_offs = [alay.take(M * K * 2) for _ in ts]
    y_offs = [alay.take(M * N * 4) for _ in ts]
    s_off = alay.take(max(ql.plan_batch(descs, M), 16))
    act = ctx.arena(alay.used)
    for xo, x in zip(x_offs, xs):
        act.write(xo, x.astype(np.float16).view(np.uint16))
    say(f"gemm batch: 8 x (M={M} K={K} N={N}), f16 x")
    ctx.linear_batch(descs, w, act, x_offs, 1, M, y_offs, s_off)
    first = [act.read(yo, (M, N), np.float32) for yo in y_offs]
    ctx.linear_batch(descs, w, act, x_offs, 1, M, y_offs, s_off)
    for yo, f in zip(y_offs, first):
        assert np.array_equal(act.read(yo, (M, N), np.float32).view(np.uint32), f.view(np.uint32))
    for i, (t, x, f) in enumerate(zip(ts, xs, first)):
        assert_close(orc, f, _gemm_ref(orc, t, x, None, t.qzeros), GEMM_ATOL, GEMM_RTOL, f"batch[{i}]")
    act.release()
    w.release()


# ------------------------------------------------------------------------- generic paths

def test_simple_paths_reference_kat_shape(ql, ctx, orc):
    """Shapes outside the MFMA kernels' constraints (N % 4 != 0, K % 32 != 0) still run on the GPU
    (one lane per column) and meet the same bars."""
    K, N = 20, 13
    t = synth.gptq_linear(K, N, 8, seed=0x51, stored_zero=None)
    lin = Linear(ql, ctx, t, bias=synth.activations(1, N, seed=0x52)[0])
    for M in (1, 3):
        x = synth.activations(M, K, seed=0x53, key=(M,))
        y, plan = run_linear(ql, ctx, lin, x)
        assert plan.kind_name == "gemv_simple"
        assert_close(orc, y, oracle_gemv(orc, lin, x), GEMV_ATOL, GEMV_RTOL, f"simple gemv M={M}")
    x = synth.activations(40, K, seed=0x54)
    y, plan = run_linear(ql, ctx, lin, x)
    assert plan.kind_name == "gemm_simple"
    W16 = orc.f16_bits_to_f32(orc.dequantize_gptq_int4_f16(t.qweight, t.qzeros, t.scales, K, N, 8))
    ref = orc.gemm_nt(orc.f16_bits_to_f32(orc.f32_to_f16_bits(x)), W16, lin.bias)
    assert_close(orc, y, ref, GEMM_ATOL, GEMM_RTOL, "simple gemm")


def test_misaligned_offsets_fall_back_correctly(ql, ctx, orc):
    """x at a 4-byte (not 16-byte) offset uses the generic kernel, same bar."""
    K, N, M = 896, 256, 2
    t = synth.gptq_linear(K, N, 128, seed=0xA1)
    lin = Linear(ql, ctx, t)
    x = synth.activations(M, K, seed=0xA2)
    act = ctx.arena(1 << 20)
    act.write(4, x)
    ctx.linear(lin.desc, lin.arena, act, 4, 0, M, 65536, 131072)
    y = act.read(65536, (M, N), np.float32)
    assert_close(orc, y, oracle_gemv(orc, lin, x), GEMV_ATOL, GEMV_RTOL, "misaligned x")


def test_range_errors_raise(ql, ctx):
    t = synth.gptq_linear(128, 64, 128, seed=0xE1)
    lin = Linear(ql, ctx, t)
    act = ctx.arena(4096)
    with pytest.raises(ql.QlError) as e:
        ctx.linear(lin.desc, lin.arena, act, 0, 0, 1, 4000, 0)    # y runs past the arena
    assert e.value.name == "QL_E_RANGE"
    with pytest.raises(ql.QlError) as e:
        ctx.linear(lin.desc, lin.arena, act, 0, 2, 1, 1024, 0)    # bad dtype
    assert e.value.name == "QL_E_INVALID"
    bad = ql.make_desc(lin.desc.qweight_off, lin.desc.qzeros_off, lin.desc.scales_off, 128, 64, 128, bits=3)
    with pytest.raises(ql.QlError) as e:
        ctx.linear(bad, lin.arena, act, 0, 0, 1, 1024, 2048)
    assert e.value.name == "QL_E_BITS"


# ------------------------------------------------------------------------- graph replay

def test_graph_replay_matches_eager(ql, ctx):
    """A captured sequence (two dependent linears, the second split-K) replayed several times,
    with eager work between replays, gives the eager result every time."""
    K1, N1, K2, N2 = 896, 4864, 4864, 896
    t1 = synth.gptq_linear(K1, N1, 128, seed=0x61)
    t2 = synth.gptq_linear(K2, N2, 128, seed=0x62)
    lay = ql.ArenaLayout()
    o1 = (lay.take(t1.qweight.nbytes), lay.take(t1.qzeros.nbytes), lay.take(t1.scales.nbytes))
    o2 = (lay.take(t2.qweight.nbytes), lay.take(t2.qzeros.nbytes), lay.take(t2.scales.nbytes))
    w = ctx.arena(lay.used)
    for t, o in ((t1, o1), (t2, o2)):
        w.write(o[0], t.qweight); w.write(o[1], t.qzeros); w.write(o[2], t.scales)
    d1 = ql.make_desc(*o1, K1, N1, 128)
    d2 = ql.make_desc(*o2, K2, N2, 128)
    p1, p2 = ql.plan_linear(1, N1, K1), ql.plan_linear(1, N2, K2)
    assert p2.split > 1
    alay = ql.ArenaLayout()
    x_off = alay.take(K1 * 4); h_off = alay.take(N1 * 4); y_off = alay.take(N2 * 4)
    s1 = alay.take(p1.scratch_bytes); s2 = alay.take(p2.scratch_bytes)
    act = ctx.arena(alay.used)
    x = synth.activations(1, K1, seed=0x63)
    act.write(x_off, x)

    def step():
        ctx.linear(d1, w, act, x_off, 0, 1, h_off, s1)
        ctx.linear(d2, w, act, h_off, 0, 1, y_off, s2)

    step()
    eager = act.read(y_off, (1, N2), np.float32)
    ctx.graph_begin()
    step()
    g = ctx.graph_end()
    for i in range(4):
        act.write(y_off, np.zeros(N2, np.float32))
        g.launch()
        ctx.sync()
        got = act.read(y_off, (1, N2), np.float32)
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {i}"
        step()                     # eager work between replays
        ctx.sync()
    g.destroy()


# ------------------------------------------------------------------------- fp16-weight GEMV

F16W_CASES = [
    # (M, N, K, bias, subnormal share of W, x spread, label)
    (1, 151936, 896, False, 0, False, "0.5B tied lm_head M=1 (fp32-FMA kernel)"),
    (4, 151936, 896, False, 0, False, "0.5B tied lm_head M=4 (matrix cores)"),
    (16, 20000, 896, True, 0, False, "M=16: one pass, bias"),
    (3, 4100, 896, True, 0, False, "M=3, ragged N, bias"),
    (6, 1000, 1024, False, 0, False, "M=6"),
    (2, 300, 200, True, 0, False, "K % 32 != 0, bias"),
    (21, 2048, 896, True, 0, False, "M=21: prefill rows, two passes over the weights"),
    (16, 8192, 896, False, 0.1, False, "10% subnormal weights"),
    (3, 4100, 896, True, 0.02, True, "x past fp16's range and in its subnormals, 2% subnormal W"),
    (5, 777, 3584, True, 0.01, True, "K=3584 (7B width), x past fp16's range and in its subnormals"),
]


def f16w_case(M, N, K, biased, sub, spread):
    """W ~ 0.02 N(0,1) in fp16 (about 0.24% of it subnormal by itself), with a share `sub` set to
    uniform subnormals; x ~ N(0,1) per row, with `spread` setting x[0, 5] = 1e5 (past fp16's range,
    so unscaled fp16 parts of x would overflow) and scaling row 1 by 1e-6 (into fp16's
    subnormals)."""
    rng = np.random.default_rng(0xF16 + N)
    W = rng.standard_normal((N, K), dtype=np.float32) * 0.02
    if sub:
        mask = rng.random((N, K)) < sub
        W[mask] = (rng.random(int(mask.sum())) * 2 - 1).astype(np.float32) * 6.0e-5
    W16 = W.astype(np.float16)
    bias = synth.activations(1, N, seed=0xF17)[0] if biased else None
    x = synth.activations(M, K, seed=0xF18, key=(M,))
    if spread:
        x[0, 5] = 1e5
        if M > 1:
            x[1] *= 1e-6
    return W16, bias, x


@pytest.mark.parametrize("M,N,K,biased,sub,spread,label", F16W_CASES)
def test_gemv_f16w_matches_oracle(ql, ctx, orc, M, N, K, biased, sub, spread, label):
    """The tied lm_head product (qwen.ts:488-489, gemm_gemv_f16.wgsl): fp32 x, fp16 W [N,K],
    fp32 accumulation, against gemmNTRef on the fp16-decoded weights (double accumulation) at the
    GEMV bar; repeats are bit-identical. The spread cases exercise the matrix-core kernel's per-row,
    per-step scaling of x into fp16 parts."""
    W16, bias, x = f16w_case(M, N, K, biased, sub, spread)
    lay = ql.ArenaLayout()
    w_off = lay.take(W16.nbytes)
    b_off = lay.take(N * 4) if biased else None
    w = ctx.arena(lay.used)
    w.write(w_off, W16.view(np.uint16))
    if biased:
        w.write(b_off, bias)
    alay = ql.ArenaLayout()
    x_off, y_off = alay.take(x.nbytes), alay.take(M * N * 4)
    act = ctx.arena(alay.used)
    act.write(x_off, x)
    say(f"gemv_f16w {label}: M={M} N={N} K={K}")
    ctx.gemv_f16w(w, w_off, b_off, act, x_off, M, N, K, y_off)
    y = act.read(y_off, (M, N), np.float32)
    ref = orc.gemm_nt(x, W16.astype(np.float32), bias)
    assert_close(orc, y, ref, GEMV_ATOL, GEMV_RTOL, label)
    ctx.gemv_f16w(w, w_off, b_off, act, x_off, M, N, K, y_off)
    assert np.array_equal(act.read(y_off, (M, N), np.float32).view(np.uint32), y.view(np.uint32))
    with pytest.raises(ql.QlError):
        ctx.gemv_f16w(w, w_off, b_off, act, x_off, M, N + 1 << 20, K, y_off)
    act.release()
    w.release()


# ------------------------------------------------------------------------- embedding lookup

EMBED_CASES = [
    # (vocab, D, rows, out offset pad, label)
    (151936, 896, 5, 0, "0.5B table (151936 x 896), 5 tokens incl. the first and last id"),
    (4096, 3584, 16, 0, "7B row width, 16 rows"),
    (65536, 16, 300, 0, "all 2^16 fp16 patterns as rows of 16, 300 rows"),
    (1000, 20, 7, 4, "D % 8 != 0 and a 4-byte output offset: one value per load"),
]


@pytest.mark.parametrize("vocab,D,rows,pad,label", EMBED_CASES)
def test_embed_f16_bit_exact(ql, ctx, orc, vocab, D, rows, pad, label):
    """The embedding lookup (embedding_f16.wgsl, dispatched at qwen.ts:392): out[r, :] =
    f16BitsToF32(W[tokens[r], :]) bit for bit (the oracle's decode is pinned over all 2^16
    patterns); a token id >= vocab gives a zero row."""
    rng = np.random.default_rng(0xE3B + vocab + D)
    if vocab * D == 1 << 20:
        table = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).repeat(16).reshape(vocab, D)
    else:
        table = rng.integers(0, 1 << 16, size=(vocab, D), dtype=np.uint32).astype(np.uint16)
    tokens = rng.integers(0, vocab, size=rows, dtype=np.uint32)
    tokens[0] = 0
    tokens[-1] = vocab - 1
    if rows > 2:
        tokens[1] = vocab            # out of range: zeros
    lay = ql.ArenaLayout()
    e_off = lay.take(table.nbytes)
    w = ctx.arena(lay.used)
    w.write(e_off, table)
    alay = ql.ArenaLayout()
    t_off = alay.take(rows * 4)
    o_off = alay.take(rows * D * 4 + pad) + pad
    act = ctx.arena(alay.used)
    act.write(t_off, tokens)
    say(f"embed {label}: vocab={vocab} D={D} rows={rows}")
    ctx.embed_f16(w, e_off, vocab, D, act, t_off, rows, o_off)
    got = act.read(o_off, (rows, D), np.float32)
    want = np.zeros((rows, D), np.float32)
    ok = tokens < vocab
    want[ok] = orc.f16_bits_to_f32(table[tokens[ok]].reshape(-1)).reshape(-1, D)
    g, r = got.view(np.uint32), want.view(np.uint32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan), label
    assert np.array_equal(g[~nan], r[~nan]), label
    with pytest.raises(ql.QlError):          # table past the arena
        ctx.embed_f16(w, e_off, vocab + 1, D, act, t_off, rows, o_off)
    with pytest.raises(ql.QlError):          # tokens and out overlap
        ctx.embed_f16(w, e_off, vocab, D, act, t_off, rows, t_off)
    act.release()
    w.release()


def test_embed_through_host(ql, ctx, orc):
    """QuantLinearModel.embed over an fp16 table uploaded as the loader does (upload_f16_bits)."""
    from webllm_amd import gptq
    vocab, C, M = 512, 896, 3
    rng = np.random.default_rng(0xE3C)
    table = (rng.standard_normal((vocab, C), dtype=np.float32) * 0.02).astype(np.float16)
    model = gptq.QuantLinearModel(ctx, table.nbytes + 4096, scratch_capacity=4096)
    model.upload_f16_bits("embed", table.view(np.uint16), (vocab, C))
    pool = gptq.ActivationArena(ctx, 1 << 20)
    toks = pool.alloc((M,), "u32")
    out = pool.alloc((M, C))
    ids = np.array([7, 0, vocab - 1], np.uint32)
    toks.write(ids)
    model.embed(toks, out, M)
    assert np.array_equal(out.read(), table[ids].astype(np.float32))
    with pytest.raises(ValueError):
        model.embed(out, out, M)
    pool.arena.release()
    model.release()
