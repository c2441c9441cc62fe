"""C-ABI checks that need no GPU: the library loads, exports every declared symbol, and its
host-only entry points (sizes, validation, planning) behave as the reference's contracts say."""
import ctypes

import numpy as np
import pytest


def test_library_exports_every_header_symbol(ql):
    names = ql.header_functions()
    assert len(names) >= 25
    L = ql.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_gptq_sizes_match_reference_layout(ql):
    # quant.ts:54-56: packRows = ceil(in/8), packCols = ceil(out/8), groups = ceil(in/group)
    assert ql.gptq_sizes(896, 4864, 128) == (112 * 4864 * 4, 7 * 608 * 4, 7 * 4864 * 2)
    assert ql.gptq_sizes(18944, 3584, 128) == (2368 * 3584 * 4, 148 * 448 * 4, 148 * 3584 * 2)
    assert ql.gptq_sizes(20, 13, 8) == (3 * 13 * 4, 3 * 2 * 4, 3 * 13 * 2)


def _desc(ql, K=16, N=8, group=8, bits=4, qz=True, bias=False):
    qw, qzb, sc = (ql.gptq_sizes(max(K, 1), max(N, 1), max(group, 1)))
    off = 0
    qweight_off = off; off += qw
    qzeros_off = off if qz else None; off += qzb
    scales_off = off; off += sc
    bias_off = None
    if bias:
        bias_off = (off + 3) // 4 * 4; off = bias_off + 4 * N
    return ql.make_desc(qweight_off, qzeros_off, scales_off, K, N, group, bias_off, bits), off


@pytest.mark.parametrize("mut,code", [
    (dict(bits=3), "QL_E_BITS"), (dict(group=0), "QL_E_GROUP"), (dict(K=0), "QL_E_DIMS"),
    (dict(N=-2), "QL_E_DIMS"), (dict(bits=8, group=-1), "QL_E_BITS"),
    (dict(group=12, K=24), "QL_E_GROUP_PACK"),
])
def test_validate_error_classes(ql, mut, code):
    kw = dict(K=16, N=8, group=8, bits=4)
    kw.update(mut)
    d, size = _desc(ql, **kw)
    assert ql.ERROR_NAMES[ql.validate(d, size + 64)] == code


def test_validate_ranges_in_reference_order(ql):
    d, size = _desc(ql, K=256, N=64, group=128, bias=True)
    assert ql.validate(d, size) == 0
    # qweight checked first (quant.ts:58), then scales (:62), then qzeros (:69)
    assert ql.ERROR_NAMES[ql.validate(d, d.qweight_off + 10)] == "QL_E_QWEIGHT_SHORT"
    d2 = ql.make_desc(0, size - 8, 256 * 64 // 2, 256, 64, 128)   # qzeros at the very end
    assert ql.ERROR_NAMES[ql.validate(d2, size)] == "QL_E_QZEROS_SHORT"
    d3 = ql.make_desc(0, None, size - 8, 256, 64, 128)
    assert ql.ERROR_NAMES[ql.validate(d3, size)] == "QL_E_SCALES_SHORT"
    # group % 8 is checked after the byte lengths (quant.ts:76)
    d4 = ql.make_desc(0, None, 0, 24, 8, 12)
    assert ql.ERROR_NAMES[ql.validate(d4, 4)] == "QL_E_QWEIGHT_SHORT"
    d5 = ql.make_desc(2, None, 4096, 16, 8, 8)
    assert ql.ERROR_NAMES[ql.validate(d5, 1 << 20)] == "QL_E_ALIGN"
    d6 = ql.make_desc(0, None, 4096, 16, 8, 8, bias_off=(1 << 20) - 8)
    assert ql.ERROR_NAMES[ql.validate(d6, 1 << 20)] == "QL_E_RANGE"


def test_validate_matches_oracle_classes(ql, orc):
    """Same class as the oracle's quant.ts restatement for a sweep of shape/bits/group errors
    and for well-formed inputs (byte-length errors are covered in reference order above)."""
    name_map = {"bits": "QL_E_BITS", "group": "QL_E_GROUP", "dims": "QL_E_DIMS",
                "group_pack": "QL_E_GROUP_PACK"}
    rng = np.random.default_rng(3)
    seen = set()
    for _ in range(400):
        K = int(rng.integers(-2, 40)); N = int(rng.integers(-2, 20))
        group = int(rng.choice([-8, 0, 4, 8, 12, 16, 32])); bits = int(rng.choice([4, 4, 4, 3]))
        Kp, Np, gp = max(K, 1), max(N, 1), max(group, 1)
        P, G, NC = (Kp + 7) // 8, (Kp + gp - 1) // gp, (Np + 7) // 8
        qw_b, qz_b, sc_b = P * Np * 4, G * NC * 4, G * Np * 2
        rc_o, _ = orc.dequantize_gptq_int4(np.zeros(qw_b, np.uint8), np.zeros(qz_b, np.uint8),
                                           np.zeros(G * Np, np.float32), K, N, group, bits)
        # one arena: qweight | qzeros | scales, each exactly as long as the layout needs
        d = ql.make_desc(0, qw_b, qw_b + qz_b, K, N, group, None, bits)
        rc_q = ql.validate(d, qw_b + qz_b + sc_b)
        want = name_map[orc.ERRORS[rc_o]] if rc_o else None
        assert (ql.ERROR_NAMES.get(rc_q) if rc_q else None) == want, (K, N, group, bits)
        seen.add(want)
    assert seen == {None, "QL_E_BITS", "QL_E_GROUP", "QL_E_DIMS", "QL_E_GROUP_PACK"}


def test_plan_kinds_and_determinism(ql):
    p = ql.plan_linear(1, 4864, 896, 128)
    assert p.kind_name == "gemv_mfma" and p.block == 256
    assert p.ref_split == 16                       # reference planGemvSplit for gate (qwen.ts:58)
    assert ql.plan_linear(1, 128, 896).ref_split == 64
    assert ql.plan_linear(1, 151936, 896).ref_split == 1
    assert ql.plan_linear(16, 18944, 3584).kind_name == "gemv_mfma"
    assert ql.plan_linear(17, 18944, 3584).kind_name == "gemm_mfma"
    assert ql.plan_linear(1, 5, 16, 8).kind_name == "gemv_simple"       # N % 4 != 0
    assert ql.plan_linear(64, 5, 16, 8).kind_name == "gemm_simple"
    for M, N, K in [(1, 896, 896), (4, 3584, 18944), (16, 18944, 3584)]:
        a, b = ql.plan_linear(M, N, K), ql.plan_linear(M, N, K)
        assert bytes(a) == bytes(b)
        assert a.split >= 1 and a.grid_x == -(-N // 256) * a.split
        G = K // 128
        assert a.split <= G
        # activations are prepared inside the kernel; scratch holds split-K partial sums only
        part = a.split * M * N * 4 if a.split > 1 else 0
        assert a.scratch_bytes == (part + 255) // 256 * 256


def test_plan_rejects_bad_dims(ql):
    with pytest.raises(ql.QlError) as e:
        ql.plan_linear(0, 8, 8, 8)
    assert e.value.name == "QL_E_DIMS"
    with pytest.raises(ql.QlError) as e:
        ql.plan_linear(1, 8, 8, 0)
    assert e.value.name == "QL_E_GROUP"


def test_batch_plan_sums_scratch(ql):
    ds = [ql.make_desc(0, None, 0, 896, n, 128) for n in (896, 128, 128)]
    total = ql.plan_batch(ds, 1)
    assert total == sum((ql.plan_linear(1, n, 896).scratch_bytes + 255) // 256 * 256
                        for n in (896, 128, 128))
    with pytest.raises(ql.QlError):
        ql.plan_batch([ds[0]] * 9, 1)


def test_null_handles_are_errors_not_crashes(ql):
    L = ql.lib()
    assert L.ql_sync(None) == -10
    assert L.ql_destroy(None) == -10
    assert L.ql_arena_release(None) == -10
    assert L.ql_graph_destroy(None) == -10
    assert L.ql_arena_size(None) == 0
    assert b"null" in L.ql_last_error()


def test_attention_plans(ql):
    """ql_plan_attention (host only): each GPU attention case's heads per run and key splits, as
    the GPU test asserts them before its launch, including 128 splits and the workspace cap."""
    from tests.test_gpu_attn import CASES

    for M, H, KV, D, past, max_t, hpr, nsplit, label in CASES:
        plan = ql.plan_attention(max_t, M, H, KV, D, past)
        assert (plan.heads_per_run, plan.nsplit) == (hpr, nsplit), label
        assert plan.workgroups >= 1 and plan.keys_per_split * plan.nsplit >= past + M
    with pytest.raises(ql.QlError):
        ql.plan_attention(8192, 2, 28, 4, 128, 8191)      # past + M beyond the cache
    with pytest.raises(ql.QlError):
        ql.plan_attention(64, 1, 6, 4, 64, 0)             # H not a multiple of KV
