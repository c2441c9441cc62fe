"""ql_linear_noalloc: ql_linear with its split-K partial sums in the library's static per-GPU
array instead of caller scratch. It runs the same kernels on the same plan, so its outputs must
be bit-identical to ql_linear's; checked on two calls in a row, the second with a smaller input
(the array keeps the first call's contents), and against the oracle's bar."""
import sys

import numpy as np
import pytest

from webllm_amd import synth

ATOL, RTOL = 1e-5, 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _linear(ql, ctx, K, N, M, seed, bias=False, x_dtype=0):
    t = synth.gptq_linear(K, N, 128, seed=seed, key=(K, N))
    b = synth.activations(1, N, seed=seed + 1)[0] if bias else None
    wl = ql.ArenaLayout()
    qw, qz, sc = wl.take(t.qweight.nbytes), wl.take(t.qzeros.nbytes), wl.take(t.scales.nbytes)
    bo = wl.take(b.nbytes) if bias else None
    w = ctx.arena(wl.used)
    w.write(qw, t.qweight); w.write(qz, t.qzeros); w.write(sc, t.scales)
    if bias:
        w.write(bo, b)
    desc = ql.make_desc(qw, qz, sc, K, N, 128, bo)
    x = synth.activations(M, K, seed=seed + 2)
    if x_dtype == 1:
        x = x.astype(np.float16)
    plan = ql.plan_linear(M, N, K, 128)
    al = ql.ArenaLayout()
    xo, y1, y2 = al.take(x.nbytes), al.take(M * N * 4), al.take(M * N * 4)
    so = al.take(max(plan.scratch_bytes, 16))
    act = ctx.arena(al.used)
    act.write(xo, x)
    return t, b, desc, w, act, x, plan, xo, y1, y2, so


def _one_call(ql, ctx, orc, K, N, M, seed, bias=False, x_dtype=0):
    t, b, desc, w, act, x, plan, xo, y1, y2, so = _linear(ql, ctx, K, N, M, seed, bias, x_dtype)
    say(f"no-alloc K={K} N={N} M={M} x_dtype={x_dtype}: plan {plan.kind_name} split {plan.split} "
        f"scratch {plan.scratch_bytes} B")
    assert plan.scratch_bytes <= ql.NOALLOC_SCRATCH_BYTES
    ctx.linear(desc, w, act, xo, x_dtype, M, y1, so)
    ctx.linear_noalloc(desc, w, act, xo, x_dtype, M, y2)
    ctx.sync()
    a = act.read(y1, (M, N), np.float32)
    c = act.read(y2, (M, N), np.float32)
    assert np.array_equal(a.view(np.uint32), c.view(np.uint32)), "no-alloc output differs from ql_linear"
    if x_dtype == 0:
        ref = orc.gptq_linear(t.qweight, t.qzeros, t.scales, x, b, 128)
        ok, max_abs, max_rel = orc.check_tolerance(c, ref, ATOL, RTOL)
        assert ok, f"maxAbs {max_abs:.3e} maxRel {max_rel:.3e}"
    w.release()
    act.release()
    return plan


@pytest.mark.gpu
def test_noalloc_matches_linear_two_calls(ql, ctx, orc):
    """A split-K 7B down projection at M=16 (6.6 MiB of partials), then a smaller split-K
    0.5B gate linear at M=1 reusing the array."""
    p1 = _one_call(ql, ctx, orc, 18944, 3584, 16, 0xA110, bias=True)
    assert p1.split > 1 and p1.scratch_bytes > 4 << 20
    p2 = _one_call(ql, ctx, orc, 896, 4864, 1, 0xA111)
    assert p2.split > 1 and p2.scratch_bytes < p1.scratch_bytes


@pytest.mark.gpu
def test_noalloc_prefill_gemm(ql, ctx, orc):
    """An M=64 f16 prefill product whose GEMM plan splits K within the array's size."""
    p = _one_call(ql, ctx, orc, 4864, 896, 64, 0xA112, x_dtype=1)
    assert p.kind_name == "gemm_mfma"


@pytest.mark.gpu
def test_noalloc_rejects_oversized_plan_on_device(ql, ctx):
    """A prefill plan needing 16 MiB of partials is refused on the host (QL_E_RANGE, nothing
    enqueued); ql_linear with caller scratch remains the entry point for it."""
    M, N, K = 128, 4096, 18944
    p = ql.plan_linear(M, N, K, 128)
    assert p.scratch_bytes > ql.NOALLOC_SCRATCH_BYTES
    qw, qz, sc = ql.gptq_sizes(K, N, 128)
    wl = ql.ArenaLayout()
    desc = ql.make_desc(wl.take(qw), wl.take(qz), wl.take(sc), K, N, 128)
    w = ctx.arena(wl.used)
    al = ql.ArenaLayout()
    xo, yo = al.take(M * K * 2), al.take(M * N * 4)
    act = ctx.arena(al.used)
    with pytest.raises(ql.QlError) as e:
        ctx.linear_noalloc(desc, w, act, xo, 1, M, yo)
    assert e.value.code == -11 and "static scratch" in str(e.value)
    w.release()
    act.release()
