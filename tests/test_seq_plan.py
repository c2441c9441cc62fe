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
    x = c.ext(3584)
    c.add(3584, 18944, x)
    info = c.plan(grid=512)
    # 296 blocks of 64 columns per K segment, dealt as runs to at most 512 workgroups
    assert 296 <= info.tiles <= 512 + 296 * info.max_split
    assert info.max_split <= 64
    assert info.reduces == (296 if info.max_split > 1 else 0)
    assert info.device_bytes > 0 and info.lds_bytes > 0


def test_split_respects_lds_for_16_rows():
    c = Chain(M=16, group=128)
    x = c.ext(18944)
    c.add(18944, 3584, x)
    info = c.plan(grid=8)
    groups = 18944 // 128
    assert info.max_split >= 1
    # each segment's activation digits fit the 48 KiB budget
    assert info.lds_bytes <= 49152
    # 56 blocks per segment on 8 workgroups: runs of whole blocks, at most one cut per row
    assert 8 <= info.tiles <= 8 + info.max_split
    assert info.max_split <= min(groups, 64)


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
    c = Chain(M=17)
    c.add(896, 896, c.ext(896))
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
