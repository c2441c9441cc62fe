"""GPU parity of the elementwise work around the linears: the residual add fused with the next
RMSNorm (vec_add.wgsl + rmsnorm.wgsl, qwen.ts:401-405, :453-458) and SiLU-mul (silu_mul.wgsl,
qwen.ts:468-469), against the oracle's rmsNormRef / siluMulRef restatements. Bar: the reference's
own tolerance for these kernels, 1e-4 (tests/kernels.ts:230, :1154), applied as
|got - ref| <= 1e-5 + 1e-4 |ref|; the stored residual sum is an fp32 add and is bit-exact."""
import sys

import numpy as np
import pytest

from webllm_amd import gptq

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-5, 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


NORM_CASES = [
    # (M, C, residual, store_sum, x offset pad (bytes), label)
    (1, 896, True, True, 0, "0.5B decode: add after o_proj, norm before gate/up"),
    (1, 896, False, False, 0, "0.5B: plain RMSNorm (layer input)"),
    (16, 3584, True, True, 0, "7B width, 16 rows (row kept in registers)"),
    (2, 8192, True, True, 0, "C = 8192: rows read twice"),
    (3, 900, True, False, 0, "C % 4 != 0: scalar path"),
    (2, 896, True, True, 4, "4-byte aligned offsets: scalar path"),
]


@pytest.mark.parametrize("M,C,residual,store,pad,label", NORM_CASES)
def test_add_rmsnorm_matches_oracle(ql, ctx, orc, M, C, residual, store, pad, label):
    say(f"add_rmsnorm {label}: M={M} C={C}")
    rng = np.random.default_rng(M * 7 + C)
    x = rng.standard_normal((M, C)).astype(np.float32)
    d = rng.standard_normal((M, C)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    lay = ql.ArenaLayout()
    xo, do, so, yo = (lay.take(M * C * 4 + 16) + pad for _ in range(4))
    act = ctx.arena(lay.used)
    wl = ql.ArenaLayout()
    wo = wl.take(C * 4)
    wa = ctx.arena(wl.used)
    wa.write(wo, w)
    act.write(xo, x)
    act.write(do, d)
    ctx.add_rmsnorm(act, xo, do if residual else None, wa, wo, 1e-6, M, C, yo, so if store else None)
    s_ref, y_ref = orc.add_rmsnorm(x, w, 1e-6, d if residual else None)
    y = act.read(yo, (M, C), np.float32)
    ok, ma, mr = orc.check_tolerance(y, y_ref, ATOL, RTOL)
    assert ok, (label, ma, mr)
    if store:
        assert np.array_equal(act.read(so, (M, C), np.float32).view(np.uint32), s_ref.view(np.uint32))
    ctx.add_rmsnorm(act, xo, do if residual else None, wa, wo, 1e-6, M, C, yo, so if store else None)
    assert np.array_equal(act.read(yo, (M, C), np.float32).view(np.uint32), y.view(np.uint32))
    with pytest.raises(ql.QlError):               # y overlapping x
        ctx.add_rmsnorm(act, xo, None, wa, wo, 1e-6, M, C, xo)
    act.release()
    wa.release()


@pytest.mark.parametrize("M,C,pad,into,label", [
    (2, 8192, 0, "x", "C = 8192, sum over x: two-pass vector path"),
    (2, 8192, 0, "d", "C = 8192, sum over d"),
    (3, 900, 0, "x", "C % 4 != 0, sum over x: scalar two-pass path"),
    (2, 896, 4, "x", "4-byte aligned, sum over x: scalar path"),
    (4, 896, 0, "x", "0.5B width, sum over x: rows in registers"),
])
def test_add_rmsnorm_sum_in_place(ql, ctx, orc, M, C, pad, into, label):
    """The residual stream updated in place (sum_off == x_off or d_off): the stored sum is
    bit-exact and y meets the bar on every path, including the two-pass ones that read the row
    back; a sum that only partly overlaps x or d is refused."""
    say(f"add_rmsnorm in place {label}: M={M} C={C}")
    rng = np.random.default_rng(M * 11 + C)
    x = rng.standard_normal((M, C)).astype(np.float32)
    d = rng.standard_normal((M, C)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    lay = ql.ArenaLayout()
    xo, do, yo = (lay.take(M * C * 4 + 16) + pad for _ in range(3))
    act = ctx.arena(lay.used)
    wa = ctx.arena(C * 4)
    wa.write(0, w)
    act.write(xo, x)
    act.write(do, d)
    so = xo if into == "x" else do
    ctx.add_rmsnorm(act, xo, do, wa, 0, 1e-6, M, C, yo, so)
    s_ref, y_ref = orc.add_rmsnorm(x, w, 1e-6, d)
    ok, ma, mr = orc.check_tolerance(act.read(yo, (M, C), np.float32), y_ref, ATOL, RTOL)
    assert ok, (label, ma, mr)
    assert np.array_equal(act.read(so, (M, C), np.float32).view(np.uint32), s_ref.view(np.uint32))
    with pytest.raises(ql.QlError, match="partly overlaps"):
        ctx.add_rmsnorm(act, xo, do, wa, 0, 1e-6, M, C, yo, xo + 4 * C if M > 1 else xo + 64)
    act.release()
    wa.release()


@pytest.mark.parametrize("n", [4864, 18944 * 16, 4863, 3])
def test_silu_mul_matches_oracle(ql, ctx, orc, n):
    say(f"silu_mul n={n}")
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    lay = ql.ArenaLayout()
    go, uo, yo = (lay.take(n * 4) for _ in range(3))
    act = ctx.arena(lay.used)
    act.write(go, g)
    act.write(uo, u)
    ctx.silu_mul(act, go, uo, n, yo)
    ok, ma, mr = orc.check_tolerance(act.read(yo, (n,), np.float32), orc.silu_mul(g, u), ATOL, RTOL)
    assert ok, (n, ma, mr)
    act.release()


def test_model_norm_and_silu_through_host(ql, ctx, orc):
    """The host mirror: model.rmsnorm over an uploaded norm weight (the reference's f32 weights by
    name, qwen.ts:640-645), with the residual add fused, and model.silu_mul."""
    model = gptq.QuantLinearModel(ctx, 1 << 20)
    rng = np.random.default_rng(5)
    w = rng.standard_normal(896).astype(np.float32)
    model.upload_f32("L0.postNorm", w)
    pool = gptq.ActivationArena(ctx, 4 << 20)
    x, p, xa, n2 = (pool.alloc((2, 896)) for _ in range(4))
    xv, pv = rng.standard_normal((2, 896)).astype(np.float32), rng.standard_normal((2, 896)).astype(np.float32)
    x.write(xv)
    p.write(pv)
    model.rmsnorm(x, "L0.postNorm", n2, 2, 896, 1e-6, residual=p, sum_out=xa)
    s_ref, y_ref = orc.add_rmsnorm(xv, w, 1e-6, pv)
    assert np.array_equal(xa.read(), s_ref)
    ok, ma, _ = orc.check_tolerance(n2.read(), y_ref, ATOL, RTOL)
    assert ok, ma
    g, u, a = (pool.alloc((2, 4864)) for _ in range(3))
    gv, uv = rng.standard_normal((2, 4864)).astype(np.float32), rng.standard_normal((2, 4864)).astype(np.float32)
    g.write(gv)
    u.write(uv)
    model.silu_mul(g, u, a, 2 * 4864)
    ok, ma, _ = orc.check_tolerance(a.read(), orc.silu_mul(gv, uv), ATOL, RTOL)
    assert ok, ma
    with pytest.raises(ValueError, match="missing f32 weight"):
        model.rmsnorm(x, "L9.inNorm", n2, 2, 896, 1e-6)
