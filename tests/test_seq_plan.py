"""Linear sequences, host side (no GPU): dependency inference from arena offsets, validation and
plan figures of ql_plan_seq. The reference separates dependent dispatches with pass breaks
(src/model/qwen.ts:556-559, src/gpu/pipeline.ts:71-116); here the passes come from offsets."""
import pytest

from webllm_amd import qlinear as ql


class Chain:
    """Builds descriptor / offset lists: weights in one layout, activations in another."""

    def __init__(self, M=1, group=128):
        self.M, self.group = M, group
        self.w, self.a = ql.ArenaLayout(), ql.ArenaLayout()
        self.descs, self.x, self.y = [], [], []

    def ext(self, K, es=4):
        return self.a.take(self.M * K * es)

    def add(self, K, N, x_off, qzeros=True):
        qw, qz, sc = ql.gptq_sizes(K, N, self.group)
        d = ql.make_desc(self.w.take(qw), self.w.take(qz) if qzeros else None, self.w.take(sc), K,
                         N, self.group)
        y = self.a.take(self.M * N * 4)
        self.descs.append(d)
        self.x.append(x_off)
        self.y.append(y)
        return y

    def plan(self, grid=256, x_dtype=ql.DTYPE_F32):
        return ql.plan_seq(self.descs, self.M, self.x, self.y, grid, x_dtype)


def fed(c: Chain, K: int, N: int):
    """A K x N linear that consumes a small producer's output (128 -> K): the sequence is chained,
    so it is planned as dependency-ordered tiles, not column strips."""
    y0 = c.add(128, K, c.ext(128))
    return c.add(K, N, y0)


def qwen_layers(c: Chain, layers: int, C=896, I=4864, KV=128):
    h = c.ext(C)
    for _ in range(layers):
        q = c.add(C, C, h)
        c.add(C, KV, h)
        c.add(C, KV, h)
        o = c.add(C, C, q)
        g = c.add(C, I, o)
        c.add(C, I, o)
        h = c.add(I, C, g)
    return c


def test_passes_follow_the_chain():
    info = qwen_layers(Chain(), 24).plan()
    assert info.linears == 168
    assert info.passes == 24 * 4            # (q,k,v) -> o -> (gate,up) -> down, per layer
    assert info.grid == 256


def test_independent_linears_share_one_pass():
    c = Chain(M=4)
    x = c.ext(896)
    for _ in range(5):
        c.add(896, 4864, x)
    info = c.plan()
    assert info.passes == 1 and info.linears == 5


def test_tiles_cover_every_column_and_segment():
    c = Chain()
    fed(c, 3584, 18944)
    info = c.plan(grid=512)
    # 296 blocks x 28 groups = 8288 block-groups on 512 workgroups: runs of about 16 groups, so a
    # block is cut where a run boundary falls inside it (at most 3 parts) and reduced. The
    # weights (34 MB) fit the MALL, where a tile is priced at a quarter of the mean run (4
    # block-groups): a run with fewer tiles takes up to that many more groups. The producer
    # (56 block-groups) adds at most one.
    assert info.passes == 2 and info.total_units == 296 * 28 + 56
    assert info.busiest_units <= 8288 // 512 + 4 + 1
    assert 2 <= info.max_split <= 3
    assert 0 < info.reduces <= 296
    assert info.device_bytes > 0 and info.lds_bytes > 0


def test_split_respects_lds_for_16_rows():
    c = Chain(M=16, group=128)
    fed(c, 18944, 3584)
    info = c.plan(grid=8)
    # 16 rows: 104 KiB of digit LDS per workgroup, 8320 B per group, so a tile covers at most
    # 12 groups and K (148 groups) splits into 13 segments; 7-block chunks walk all segments
    # before the next chunk, one chunk per run (plus the producer's 8 tiles of 37 block-groups)
    assert info.lds_bytes <= 104 << 10
    assert info.max_split == 13
    assert info.tiles == 8 * 13 + 8
    assert info.busiest_units == 56 * 148 // 8 + 296 // 8
    assert info.reduces == 8                 # each run reduces its own 7 blocks in one task


def test_lds_budget_of_few_rows():
    c = Chain(M=4)
    fed(c, 3584, 3584)
    info = c.plan(grid=8)
    # 4 rows: 104 KiB of digits (2080 B per group): 28 groups fit, so no block is split and
    # nothing is reduced
    assert info.lds_bytes <= 104 << 10
    assert info.max_split == 1 and info.reduces == 0


def qwen7b(c: Chain, layers: int, chained: bool, C=3584, I=18944):
    """The 7B-shaped linears (q, o, gate, up, down per layer), chained through their outputs or
    each with its own input as the benchmark configs define."""
    h = c.ext(C)
    for _ in range(layers):
        q = c.add(C, C, h if chained else c.ext(C))
        o = c.add(C, C, q if chained else c.ext(C))
        g = c.add(C, I, o if chained else c.ext(C))
        c.add(C, I, o if chained else c.ext(C))
        h = c.add(I, C, g if chained else c.ext(I))
    return c


@pytest.mark.parametrize("M,grid", [(1, 512), (4, 512), (16, 256)])
def test_balance_7b_independent(M, grid):
    info = qwen7b(Chain(M=M), 28, chained=False).plan(grid=grid)
    assert info.passes == 1 and info.linears == 140
    # independent: column strips of 8 whole blocks over all of K (or of 4, two waves per block,
    # when 8-block strips leave the workgroups more than 6% off balance), dealt longest first,
    # with no K split and nothing to reduce
    def per_layer(strip):
        return 2 * (18944 // 64 // strip) + 3 * (3584 // 64 // strip)
    strip = 8 if info.tiles == 28 * per_layer(8) else 4
    assert info.tiles == 28 * per_layer(strip)
    assert info.reduces == 0 and info.max_split == 1
    assert info.busiest_units <= info.total_units // grid + strip * 148
    assert info.balance < 1.07


def test_strips_for_independent_sequences_only(monkeypatch):
    """Independent linears run as column strips (nothing reduced, no K split across workgroups):
    the 0.5B step at M = 1 is planned as strips of 4 blocks with two waves per block (8-block
    strips of the 4864-deep down projection would outweigh a workgroup's share); a chained
    sequence keeps the dependency-ordered tiles (a streamed one at M >= 2 only with the
    pass-by-pass form switched off)."""
    monkeypatch.setenv("QL_SEQ_PASSES", "0")
    info = qwen7b(Chain(M=16), 28, chained=True).plan(grid=256)
    assert info.kernel == ql.SEQ_TILES and info.passes == 28 * 4 and info.reduces > 0
    monkeypatch.delenv("QL_SEQ_PASSES")
    c = Chain(M=1)
    for _ in range(24):
        for K, N in ((896, 896), (896, 128), (896, 128), (896, 896), (896, 4864), (896, 4864), (4864, 896)):
            c.add(K, N, c.ext(K))
    info = c.plan(grid=256)
    # 4-block strips per layer: q 4, k 1, v 1, o 4, gate 19, up 19, down 4
    assert info.passes == 1 and info.reduces == 0 and info.max_split == 1
    assert info.tiles == 24 * (4 + 1 + 1 + 4 + 19 + 19 + 4)


@pytest.mark.parametrize("M", [2, 4, 5, 8, 16])
def test_chained_streamed_runs_pass_by_pass(M):
    """A chained sequence of streamed weights (the 7B shape, 3.35 GB) at M = 2..16 runs one strip
    launch per pass: 112 passes (q; o; gate, up; down per layer), the independent step's 2660
    strips of 8 blocks, each cut into K parts of whole 512-k chunks that a part-sum launch adds, so
    nothing is reduced across workgroups inside a launch. At M = 1, or on weights the MALL keeps (two 0.5B layers), it keeps the
    dependency-ordered tiles."""
    info = qwen7b(Chain(M=M), 28, chained=True).plan(grid=256)
    assert info.kernel == ql.SEQ_STRIP_PASSES and info.passes == 112 and info.linears == 140
    assert info.tiles == 28 * (7 + 7 + 37 + 37 + 7) and info.reduces == 0 and info.max_split == 1
    assert info.stream == 1 and info.variant == 1 and info.grid == 256
    # every 8-block strip of every linear over all of K: 8 blocks x K/128 groups
    assert info.total_units == 28 * 8 * (7 * 28 + 7 * 28 + 74 * 28 + 7 * 148)
    assert qwen7b(Chain(M=1), 28, chained=True).plan(grid=256).kernel == ql.SEQ_TILES
    c = Chain(M=M)
    h = c.ext(896)
    for _ in range(2):
        q = c.add(896, 896, h)
        o = c.add(896, 896, q)
        g = c.add(896, 4864, o)
        h = c.add(4864, 896, g)
    assert c.plan(grid=256).kernel == ql.SEQ_TILES


def test_05b_independent_prices_tiles():
    """The 0.5B step's 168 linears as one streaming pass of the tile planner (here fed by two small
    producers, so the sequence is chained; 186 MB: MALL-resident). With a tile priced at a
    quarter of the mean run, workgroups whose runs cross many small linears (q/k/v/o) take fewer
    block-groups, and runs stay in whole blocks (almost no K splits to reduce)."""
    c = Chain()
    x = c.ext(128)
    ya, yb = c.add(128, 896, x), c.add(128, 4864, x)
    for _ in range(24):
        for K, N in ((896, 896), (896, 128), (896, 128), (896, 896), (896, 4864), (896, 4864), (4864, 896)):
            c.add(K, N, ya if K == 896 else yb)
    info = c.plan()
    assert info.passes == 2 and info.total_units == 43680 + 14 + 76
    mean = info.total_units / info.grid
    assert mean < info.busiest_units <= mean + 2 * (mean // 4)
    assert info.tiles <= 420 + 90 and info.reduces <= 16


def test_balance_7b_chained():
    info = qwen7b(Chain(), 4, chained=True).plan(grid=512)
    assert info.passes == 16
    # streaming passes are balanced to one group each; q/o passes are latency-bound
    assert info.balance < 1.15


@pytest.mark.parametrize("seed", range(6))
def test_random_plans_verify(seed):
    """Random shapes, batch rows, group sizes, grids and dependency graphs: ql_plan_seq checks
    each plan (coverage, parts, reductions, pass order) and raises on a violation."""
    import random
    rng = random.Random(0x5EC0 + seed)
    for _ in range(25):
        group = rng.choice([64, 128, 256])
        M = rng.choice([1, 2, 3, 4, 8, 16])
        c = Chain(M=M, group=group)
        outs = []
        for _ in range(rng.randint(1, 12)):
            K = group * rng.randint(1, 160)
            N = 4 * rng.randint(1, 1200)
            srcs = [y for y, n in outs if n == K]
            x = rng.choice(srcs) if srcs and rng.random() < 0.6 else c.ext(K)
            outs.append((c.add(K, N, x), N))
        info = c.plan(grid=rng.choice([1, 2, 7, 64, 256, 512, 600]))
        assert info.total_units > 0 and info.max_split <= 4096


@pytest.mark.parametrize("group", [64, 256])
def test_other_group_sizes(group):
    info = qwen_layers(Chain(group=group), 2, C=1024, I=4096).plan()
    assert info.passes == 8


def test_f16_external_input():
    c = Chain(M=2)
    x = c.ext(896, es=2)
    q = c.add(896, 896, x)
    c.add(896, 896, q)
    assert c.plan(x_dtype=ql.DTYPE_F16).passes == 2


def _err(c, **kw):
    with pytest.raises(ql.QlError) as e:
        c.plan(**kw)
    return e.value


def test_reject_overlapping_outputs():
    c = Chain()
    x = c.ext(896)
    c.add(896, 896, x)
    c.add(896, 896, x)
    c.y[1] = c.y[0] + 256
    assert _err(c).name == "QL_E_INVALID"


def test_reject_input_overlapping_an_output():
    c = Chain()
    x = c.ext(896)
    y = c.add(896, 896, x)
    c.add(896, 128, y + 512)          # not the producer's start: partial overlap
    assert _err(c).name == "QL_E_INVALID"


def test_reject_reading_a_later_output():
    c = Chain()
    x = c.ext(896)
    c.add(896, 896, x)
    y1 = c.add(896, 896, x)
    c.x[0] = y1                       # linear 0 would read linear 1's output
    assert _err(c).name == "QL_E_INVALID"


def test_reject_width_mismatch():
    c = Chain()
    x = c.ext(896)
    g = c.add(896, 4864, x)
    c.add(896, 896, g)                # K=896 cannot read a 4864-wide output
    assert _err(c).name == "QL_E_INVALID"


def test_reject_shapes_outside_the_sequence_kernel():
    # M > 16 is the prefill launch, for fp32 x (rounded to fp16 as staged) as for fp16 x
    c = Chain(M=17)
    c.add(896, 896, c.ext(896))
    assert c.plan().kernel == ql.SEQ_PREFILL
    assert c.plan(x_dtype=ql.DTYPE_F16).kernel == ql.SEQ_PREFILL
    c = Chain(M=17)
    c.add(896, 898, c.ext(896))       # N % 4 != 0: no prefill tile form
    assert _err(c).name == "QL_E_INVALID"
    c = Chain()
    x = c.ext(896)
    c.add(896, 896, x)
    c.descs.append(ql.make_desc(0, None, 0, 896, 896, 64))   # mixed group sizes
    c.x.append(x)
    c.y.append(c.a.take(896 * 4))
    assert _err(c).name == "QL_E_INVALID"
    c = Chain()
    c.add(896, 898, c.ext(896))       # N % 4 != 0
    assert _err(c).name == "QL_E_INVALID"


def test_reject_misaligned_offsets():
    c = Chain()
    x = c.ext(896)
    c.add(896, 896, x)
    c.x[0] = x + 4
    assert _err(c).name == "QL_E_ALIGN"


def test_reject_bad_counts():
    with pytest.raises(ql.QlError):
        ql.plan_seq([], 1, [], [], 256)
    c = Chain()
    c.add(896, 896, c.ext(896))
    assert _err(c, grid=0).name == "QL_E_INVALID"


def test_gptq_validation_applies_per_linear():
    c = Chain()
    c.add(896, 896, c.ext(896))
    c.descs[0].bits = 3
    assert _err(c).name == "QL_E_BITS"


def test_strips_stream_weights_the_mall_cannot_keep():
    """Strips read the packed weights with streaming loads when the launch's weights exceed what
    the MALL keeps between steps (the 7B step, 3.3 GB), and with ordinary loads when they fit
    (the 0.5B step, 186 MB, which the next step then finds in the MALL)."""
    c = Chain(M=1)
    for _ in range(24):
        for K, N in ((896, 896), (896, 128), (896, 128), (896, 896), (896, 4864), (896, 4864), (4864, 896)):
            c.add(K, N, c.ext(K))
    small = c.plan(grid=512)
    assert small.kernel == ql.SEQ_STRIPS and small.stream == 0
    big = qwen7b(Chain(M=1), 28, chained=False).plan(grid=256)
    assert big.kernel == ql.SEQ_STRIPS and big.stream == 1 and big.variant == 0
    # M 5..16 on the streamed 7B shapes: the no-padding strip kernel; the 0.5B step (MALL-resident,
    # K = 896 is 7 groups) keeps the general one
    for M in (5, 8, 9, 16):
        wide = qwen7b(Chain(M=M), 28, chained=False).plan(grid=256)
        assert wide.kernel == ql.SEQ_STRIPS and wide.stream == 1 and wide.variant == 1, M
        # the wide kernel has one block per wave: every strip is 8 whole 64-column blocks
        # (140 linears' 21,280 blocks), never the 4-block strips of split 2
        assert wide.split == 1 and wide.tiles == 21280 // 8, (M, wide.split, wide.tiles)
        assert wide.grid == 256, (M, wide.grid)
    for M in (1, 4):
        assert qwen7b(Chain(M=M), 28, chained=False).plan(grid=256).variant == 0
    # chained sequences (dependency-ordered tiles) report no streaming
    assert qwen7b(Chain(M=1), 2, chained=True).plan(grid=256).stream == 0


def test_seq_info_struct_matches_the_library():
    """ql_plan_seq writes exactly sizeof(SeqInfo) bytes: a guard area after the ctypes struct stays
    untouched and the struct's last field (variant) comes back zeroed."""
    import ctypes
    c = Chain(M=1)
    c.add(896, 896, c.ext(896))
    n = len(c.descs)
    size = ctypes.sizeof(ql.SeqInfo)
    buf = (ctypes.c_uint8 * (size + 64))(*([0xAA] * (size + 64)))
    rc = ql.lib().ql_plan_seq(n, (ql.GptqDesc * n)(*c.descs), 1, (ctypes.c_uint64 * n)(*c.x), ql.DTYPE_F32,
                              (ctypes.c_uint64 * n)(*c.y), 256, ctypes.cast(buf, ctypes.POINTER(ql.SeqInfo)))
    assert rc == 0
    assert bytes(buf[size:]) == b"\xaa" * 64
    info = ql.SeqInfo.from_buffer_copy(bytes(buf[:size]))
    assert info.variant == 0 and info.linears == 1


def fused_layers(c: Chain, layers: int, C=896, I=4864, KV=128):
    """The Qwen layer's data flow as a fused sequence (o reads q in attention's place):
    q/k/v <- rmsnorm(h); h1 = h + o(q); gate/up <- rmsnorm(h1); h2 = h1 + down(silu(gate) * up)."""
    fuse = []
    h = c.ext(C)
    for _ in range(layers):
        ln1, ln2 = c.w.take(C * 4), c.w.take(C * 4)
        q = c.add(C, C, h)
        fuse.append(ql.make_fuse(norm_w_off=ln1))
        c.add(C, KV, h)
        fuse.append(ql.make_fuse(norm_w_off=ln1))
        c.add(C, KV, h)
        fuse.append(ql.make_fuse(norm_w_off=ln1))
        h1 = c.add(C, C, q)
        fuse.append(ql.make_fuse(res_off=h))
        g = c.add(C, I, h1)
        fuse.append(ql.make_fuse(norm_w_off=ln2))
        u = c.add(C, I, h1)
        fuse.append(ql.make_fuse(norm_w_off=ln2))
        h = c.add(I, C, g)
        fuse.append(ql.make_fuse(x2_off=u, res_off=h1))
    return c, fuse


def test_fused_layers_plan_as_chained_tiles():
    """Norms, residuals and SiLU-mul folded in: the layer's 4 dependent passes (q/k/v, o,
    gate/up, down), every linear's producers (input, GLU operand, residual) in earlier passes;
    a fused sequence never takes strips, even when no linear reads another's input."""
    c, fuse = fused_layers(Chain(), 2)
    info = ql.plan_seq(c.descs, c.M, c.x, c.y, 256, fuse=fuse)
    assert info.kernel == ql.SEQ_TILES and info.linears == 14 and info.passes == 8
    # independent linears with a norm on their external inputs: still tiles
    c2 = Chain()
    w = c2.w.take(896 * 4)
    f2 = []
    for _ in range(4):
        c2.add(896, 896, c2.ext(896))
        f2.append(ql.make_fuse(norm_w_off=w))
    assert ql.plan_seq(c2.descs, 1, c2.x, c2.y, 256).kernel == ql.SEQ_STRIPS
    i2 = ql.plan_seq(c2.descs, 1, c2.x, c2.y, 256, fuse=f2)
    assert i2.kernel == ql.SEQ_TILES and i2.passes == 1
    # no fusion at all through the fused entry point: the same plan as ql_plan_seq
    none = [ql.make_fuse() for _ in c2.descs]
    assert ql.plan_seq(c2.descs, 1, c2.x, c2.y, 256, fuse=none).kernel == ql.SEQ_STRIPS


@pytest.mark.parametrize("M", [128, 512])
def test_fused_prefill_launches(M):
    """The fused 0.5B layers at M > 16: per layer 4 GEMM passes and 2 RMSNorm launches, a
    part-sum launch after each chunked pass, and a SiLU-mul launch only where gate and up do not
    share one: at M = 128 the gate/up pass's part-sum launch writes silu(gate) * up (the down
    linear's input) beside the two outputs; at M = 512 gate/up runs on the prefill kernel (no part
    sums) and the SiLU-mul keeps its launch."""
    c, fuse = fused_layers(Chain(M=M), 24)
    info = ql.plan_seq(c.descs, M, c.x, c.y, 256, fuse=fuse)
    assert info.kernel == ql.SEQ_PREFILL_PASSES and info.passes == 96 and info.linears == 168
    if M == 128:
        assert info.variant == 96 and info.launches == 24 * (4 + 2 + 4)
    else:
        assert info.variant == 72 and info.launches == 24 * (4 + 2 + 3 + 1)


def test_fused_residual_counts_as_a_dependency():
    """A linear whose only link to an earlier one is its residual runs in a later pass."""
    c = Chain()
    y0 = c.add(896, 896, c.ext(896))
    c.add(896, 896, c.ext(896))
    fuse = [ql.make_fuse(), ql.make_fuse(res_off=y0)]
    info = ql.plan_seq(c.descs, 1, c.x, c.y, 256, fuse=fuse)
    assert info.kernel == ql.SEQ_TILES and info.passes == 2


def test_fused_validation():
    """Norm and GLU exclude each other; producers must run earlier and have the operand's width;
    norm weights are 16-byte aligned with eps in [0, 1]; an external residual must not overlap an
    output; a fused prefill sequence (M > 16) takes fp32 x like any fused sequence."""
    c = Chain()
    h = c.ext(896)
    w = c.w.take(896 * 4)
    y0 = c.add(896, 896, h)
    c.add(896, 896, y0)

    def code(fuse, M=1, descs=None):
        d = descs or c.descs
        with pytest.raises(ql.QlError) as e:
            ql.plan_seq(d, M, c.x[:len(d)], c.y[:len(d)], 256, fuse=fuse)
        return e.value.name

    f = ql.make_fuse
    assert code([f(norm_w_off=w, x2_off=y0), f()]) == "QL_E_INVALID"          # norm and GLU both
    # fused staging reads fp32 words: fp16 x is refused
    with pytest.raises(ql.QlError) as e16:
        ql.plan_seq(c.descs, 1, c.x, c.y, 256, ql.DTYPE_F16, fuse=[f(norm_w_off=w), f()])
    assert e16.value.name == "QL_E_INVALID" and "fp32 x" in str(e16.value)
    assert code([f(res_off=c.y[1]), f()]) == "QL_E_INVALID"                      # residual from a later linear
    assert code([f(), f(norm_w_off=w + 4)]) == "QL_E_ALIGN"                      # norm weight alignment
    assert code([f(), f(norm_w_off=w, norm_eps=-1.0)]) == "QL_E_INVALID"
    # an external residual that overlaps an output
    assert code([f(), f(res_off=y0 + 64)]) == "QL_E_INVALID"
    # a GLU operand from a producer of the wrong width
    c2 = Chain()
    hh = c2.ext(896)
    a = c2.add(896, 128, hh)
    c2.add(896, 896, hh)
    with pytest.raises(ql.QlError) as e:
        ql.plan_seq(c2.descs, 1, c2.x, c2.y, 256, fuse=[f(), f(x2_off=a)])
    assert e.value.name == "QL_E_INVALID"
    # fp16 x is refused at M > 16 too
    c3 = Chain(M=32)
    ww = c3.w.take(896 * 4)
    c3.add(896, 896, c3.ext(896, es=2))
    with pytest.raises(ql.QlError) as e:
        ql.plan_seq(c3.descs, 32, c3.x, c3.y, 256, x_dtype=ql.DTYPE_F16, fuse=[f(norm_w_off=ww)])
    assert e.value.name == "QL_E_INVALID"


@pytest.mark.parametrize("M", [17, 128, 512])
def test_chained_prefill_runs_pass_by_pass(M):
    """The model's dependency order at M > 16 (runForward(M = T)): the 0.5B layers chained
    through their outputs plan as one GEMM launch per pass, 96 passes for 24 layers: the prefill
    kernel for a pass whose 128 x 256 tiles reach 128 (gate/up at M = 512: 4 x 19 x 2), else the
    chunked GEMM with K split (variant counts those passes); fp16 x is refused for a chained
    prefill (the producers' outputs are fp32); independent linears keep the one-launch prefill.
    Launches: one per pass plus a part-sum launch after each chunked pass with K split (every
    chunked pass here: K = 896 splits 3 ways, K = 4864 19 ways)."""
    info = qwen_layers(Chain(M=M), 24).plan()
    assert info.kernel == ql.SEQ_PREFILL_PASSES and info.passes == 96 and info.linears == 168
    assert info.variant == (72 if M == 512 else 96)
    assert info.launches == 96 + info.variant
    # output tiles: 256 columns by 64 rows on the chunked GEMM at these M, 128 rows on the prefill
    t64 = lambda N: -(-M // 64) * -(-N // 256)
    t128 = lambda N: -(-M // 128) * -(-N // 256)
    gu = 2 * (t128(4864) if M == 512 else t64(4864))
    assert info.tiles == 24 * (t64(896) + 2 * t64(128) + t64(896) + gu + t64(896))
    c = Chain(M=M)
    y = c.add(896, 896, c.ext(896, es=2))
    c.add(896, 896, y)
    with pytest.raises(ql.QlError) as e:
        c.plan(x_dtype=ql.DTYPE_F16)
    assert e.value.name == "QL_E_INVALID" and "fp32 x" in str(e.value)
    c = Chain(M=M)
    for _ in range(3):
        c.add(896, 896, c.ext(896))
    assert c.plan().kernel == ql.SEQ_PREFILL and c.plan().passes == 1
