"""GPU parity of the launches bench.py times, at the size it times them.

bench.py's Model and SeqStep build the step here, with bench.py's seeds, so the launch under
test is the timed one: the 0.5B-shaped decode step (168 independent linears, one persistent
launch) at M = 1, 2, 4, 8, 16 and the 7B-shaped step (140 linears, 3.34 GB of packed weights)
at M = 1, 2, 4, 8, 16. The step is run the way bench.py runs it (captured into a graph and
replayed), then every linear's output is compared with the oracle (gemmNTRef over quant.ts
weights, src/reference/qwen-ref.ts:126-145) on the input the launch read, with the reference's
GEMV bar |d| <= 1e-5 + 1e-4|ref| (src/tests/kernels.ts:67, :1390) for these N(0,1) inputs.

0.5B: every output column of every linear, at every M. 7B: every column of every linear at M=1;
at M > 1 a fixed sample of 64-column blocks of every linear (first, last and strided ones), the
launch itself staying full size.
"""
import sys

import numpy as np
import pytest

import bench

ATOL, RTOL = 1e-5, 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def sample_blocks(N: int, count: int = 8) -> np.ndarray:
    """Columns of `count` 64-column blocks: the first, the last and evenly strided ones."""
    nb = N // 64
    picks = sorted(set([0, nb - 1] + [int(round(i * (nb - 1) / (count - 1))) for i in range(count)]))
    return np.concatenate([np.arange(b * 64, min(N, b * 64 + 64)) for b in picks]).astype(np.int32)


def check_step(orc, model, st, cols_for, label):
    """Compares every linear of the step with the oracle on the columns cols_for(N)."""
    M = st.M
    worst_norm, worst_rel, checked = 0.0, 0.0, 0
    for i, (layer, proj) in enumerate(st.order):
        t = model.tensors[(layer, proj)]
        x = st.act.read(st.x_offs[i], (M, t.K), np.float32)
        y = st.act.read(st.y_offs[i], (M, t.N), np.float32)
        cols = cols_for(t.N)
        ref = orc.gptq_linear_cols(t.qweight, t.qzeros, t.scales, x, cols, None, bench.GROUP)
        got = np.ascontiguousarray(y[:, cols])
        ok, max_abs, max_rel = orc.check_tolerance(got, ref, ATOL, RTOL)
        assert ok, (f"{label} linear {i} (layer {layer} {proj}, K={t.K} N={t.N}): maxAbs {max_abs:.3e} "
                    f"maxRel {max_rel:.3e}")
        assert np.isfinite(y).all(), f"{label} linear {i}: non-finite output"
        worst_norm = max(worst_norm, float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)))
        worst_rel = max(worst_rel, float(np.max(np.abs(got - ref) / (ATOL / RTOL + np.abs(ref)))))
        checked += got.size
    say(f"  {label}: {len(st.order)} linears, {checked} outputs within bar; worst normwise "
        f"{worst_norm:.3e}, worst |d|/(atol/rtol+|ref|) {worst_rel:.3e}")


def run_as_benched(st):
    """bench.timed(): direct launches back to back; then one graph replay, as a caller that
    captures the launch would run it (the checks read the replay's outputs)."""
    st.run(2)
    st.capture()
    st.graph.launch()
    st.seq.status()


@pytest.fixture(scope="module")
def model05(ql, ctx):
    m = bench.Model(ctx, "0.5b", seed=0x9EF0, keep_tensors=True)
    yield m
    m.arena.release()


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
def test_headline_step_05b_full_size(ql, ctx, orc, model05, M):
    """The headline launch: 24 layers x 7 linears, each on its own input, one strip launch."""
    st = bench.SeqStep(ctx, model05, M, chained=False)
    info = st.info
    say(f"0.5B step M={M}: {info.as_dict()}")
    assert info.linears == 168 and info.passes == 1 and info.reduces == 0
    assert info.kernel == ql.SEQ_STRIPS
    run_as_benched(st)
    check_step(orc, model05, st, lambda N: np.arange(N, dtype=np.int32), f"0.5B M={M}")
    st.release()


@pytest.fixture(scope="module")
def model7b(ql, ctx):
    m = bench.Model(ctx, "7b", seed=0x7B, keep_tensors=True)
    yield m
    m.arena.release()


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
def test_north_star_step_7b_full_size(ql, ctx, orc, model7b, M):
    """The north-star launch: 28 layers x (q, o, gate, up, down), 3.34 GB streamed from HBM."""
    st = bench.SeqStep(ctx, model7b, M, chained=False)
    info = st.info
    say(f"7B step M={M}: {info.as_dict()}")
    assert info.linears == 140 and info.passes == 1 and info.reduces == 0
    assert info.kernel == ql.SEQ_STRIPS
    run_as_benched(st)
    if M == 1:
        cols_for = lambda N: np.arange(N, dtype=np.int32)  # noqa: E731
    else:
        cols_for = sample_blocks
    check_step(orc, model7b, st, cols_for, f"7B M={M}")
    st.release()


def test_sample_blocks_cover_ends():
    c = sample_blocks(18944)
    assert c[0] == 0 and c[-1] == 18943 and len(c) % 64 == 0 and np.all(np.diff(c) > 0)
    assert len(sample_blocks(896)) == 8 * 64
