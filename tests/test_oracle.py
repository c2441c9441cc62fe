"""Pins the C oracle (oracle/gptq_oracle.c) before it is trusted as the parity checker.

Each oracle function is checked against something that does not share its code: the reference's
own GPTQ known-answer test, IEEE-754 conversions done by hardware/numpy, numpy float64 matmul, the
documented planGemvSplit table, and hand-derived cases. CPU only.
"""
import json
import os
import struct

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _bits_to_f32(bits):
    return np.array(bits, dtype=np.uint32).view(np.float32)


# ---------------------------------------------------------------- f32 <-> f16 (a3, a6)

def test_f16_encode_golden_cases(orc):
    for case in json.load(open(os.path.join(GOLDEN, "f16_cases.json"))):
        f = struct.unpack("<f", struct.pack("<I", case["f32_bits"]))[0]
        got = orc.lib().orc_f32_to_f16_bits(f)
        assert got == case["f16_bits"], (hex(case["f32_bits"]), hex(got), case["note"])


def test_f16_encode_exhaustive_vs_hardware_rne(orc):
    """All 2^32 f32 patterns against the F16C conversion (IEEE RNE). The only differences
    allowed are the reference's documented ones: (2^-25, 2^-24) flushed to +-0 (buffer.ts:73)
    and every NaN encoded as 0x7e00 (buffer.ts:61)."""
    total, quirk, nan, other = orc.f16_exhaustive_check()
    assert other == 0
    assert quirk == 2 * (2 ** 23 - 1)          # exponent field 102, mantissa != 0, both signs
    # F16C keeps the sign and the top 9 payload bits and sets the quiet bit, so it also yields
    # 0x7e00 for +NaN with mantissa in [1, 2^13) or [2^22, 2^22 + 2^13): 2^14 - 1 patterns
    assert nan == 2 * (2 ** 23 - 1) - (2 ** 14 - 1)
    assert total == quirk + nan


def test_f16_encode_vs_numpy_sample(orc):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    got = orc.f32_to_f16_bits(f)
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    finite = ~np.isnan(f)
    exp = (bits >> 23) & 0xFF
    quirk = (exp == 102) & ((bits & 0x7FFFFF) != 0)
    assert np.array_equal(got[finite & ~quirk], want[finite & ~quirk])
    assert np.all(got[~finite] == 0x7E00)


def test_f16_decode_exhaustive(orc):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_bits_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.all(np.isnan(got[nan]))


# ---------------------------------------------------------------- dequantizeGptqInt4 (a2)

def _kat():
    d = json.load(open(os.path.join(GOLDEN, "gptq_kat.json")))
    qweight = np.array(d["qweight_u32"], dtype=np.uint32)
    qzeros = np.array(d["qzeros_u32"], dtype=np.uint32)
    scales = _bits_to_f32(d["scales_f32_bits"])
    want = _bits_to_f32(d["want_f32_bits"]).reshape(d["out_features"], d["in_features"])
    return d, qweight, qzeros, scales, want


def test_dequant_reference_kat(orc):
    d, qweight, qzeros, scales, want = _kat()
    rc, W = orc.dequantize_gptq_int4(qweight, qzeros, scales, d["in_features"],
                                     d["out_features"], d["group_size"])
    assert rc == 0
    ok, max_abs, _ = orc.check_tolerance(W, want, 1e-6, 1e-6)   # weights.ts:125
    assert ok and max_abs == 0.0
    assert np.array_equal(W.view(np.uint32), want.view(np.uint32))


def test_dequant_reference_kat_symmetric_fallback(orc):
    d, qweight, _, scales, want = _kat()
    rc, W = orc.dequantize_gptq_int4(qweight, None, scales, d["in_features"], d["out_features"],
                                     d["group_size"])
    assert rc == 0
    assert np.array_equal(W.view(np.uint32), want.view(np.uint32))   # weights.ts:127-136


def _numpy_dequant(qweight, qzeros, scales, K, N, group):
    """Independent vectorised formulation of the GPTQ layout (quant.ts:1-14)."""
    k = np.arange(K)
    q = (qweight[k // 8, :] >> (4 * (k % 8)).astype(np.uint32)[:, None]) & 15   # [K, N]
    g = k // group
    n = np.arange(N)
    if qzeros is None:
        z = np.full((K, N), 8, dtype=np.int64)
    else:
        z = ((qzeros[g][:, n // 8] >> (4 * (n % 8)).astype(np.uint32)[None, :]) & 15) + 1
    w = (q.astype(np.int64) - z.astype(np.int64)).astype(np.float64) * scales[g, :].astype(np.float64)
    return w.astype(np.float32).T.copy()


@pytest.mark.parametrize("K,N,group", [(16, 5, 8), (20, 13, 8), (136, 12, 8), (256, 40, 128),
                                       (384, 24, 64), (130, 9, 16)])
def test_dequant_brute_force(orc, K, N, group):
    rng = np.random.default_rng(K * 1000 + N)
    P, G, NC = (K + 7) // 8, (K + group - 1) // group, (N + 7) // 8
    qweight = rng.integers(0, 1 << 32, size=(P, N), dtype=np.uint64).astype(np.uint32)
    qzeros = rng.integers(0, 1 << 32, size=(G, NC), dtype=np.uint64).astype(np.uint32)
    scales = (rng.standard_normal((G, N)) * 0.01).astype(np.float32)
    for qz in (qzeros, None):
        rc, W = orc.dequantize_gptq_int4(qweight, qz, scales, K, N, group)
        assert rc == 0
        assert np.array_equal(W.view(np.uint32), _numpy_dequant(qweight, qz, scales, K, N, group).view(np.uint32))


def test_dequant_invariants(orc):
    """qwen-format.ts:112-123, :159-163: stored nibble 7 everywhere -> zero 8; |w| <= 8*max s."""
    rng = np.random.default_rng(5)
    K, N, group = 512, 64, 128
    qweight = rng.integers(0, 1 << 32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
    qzeros = np.full((K // group, N // 8), 0x77777777, dtype=np.uint32)
    # fp16-valued scales (as stored in the checkpoint): (q - 8) * s is then exact in f32
    scales = (np.abs(rng.standard_normal((K // group, N))) * 0.01).astype(np.float16).astype(np.float32)
    _, W = orc.dequantize_gptq_int4(qweight, qzeros, scales, K, N, group)
    _, Ws = orc.dequantize_gptq_int4(qweight, None, scales, K, N, group)
    assert np.array_equal(W, Ws)
    assert np.abs(W).max() <= 8 * scales.max()
    # every nibble value appears; W / s recovers q - 8 exactly
    k = np.arange(K)
    q = (qweight[k // 8, :] >> (4 * (k % 8)).astype(np.uint32)[:, None]) & 15
    ratio = W.T / scales[k // group, :]
    assert np.array_equal(ratio, q.astype(np.float32) - 8)


def test_dequant_zero_sixteen(orc):
    """Stored nibble 15 -> zero 16 (computed in int, not nibble-wrapped)."""
    qweight = np.full((1, 8), 0xFFFFFFFF, dtype=np.uint32)   # q = 15
    qzeros = np.full((1, 1), 0xFFFFFFFF, dtype=np.uint32)    # z = 16
    scales = np.ones((1, 8), dtype=np.float32)
    _, W = orc.dequantize_gptq_int4(qweight, qzeros, scales, 8, 8, 8)
    assert np.all(W == -1.0)


@pytest.mark.parametrize("kw,code", [
    (dict(bits=3), "bits"), (dict(group=0), "group"), (dict(K=0), "dims"), (dict(N=-1), "dims"),
    (dict(qw_short=True), "qweight_short"), (dict(sc_short=True), "scales_short"),
    (dict(qz_short=True), "qzeros_short"), (dict(group=12, K=24), "group_pack"),
    (dict(bits=3, group=0), "bits"), (dict(group=12, qw_short=True, K=24), "qweight_short"),
])
def test_dequant_error_classes(orc, kw, code):
    """quant.ts:46-79: same failure class, checked in the same order."""
    K, N, group = kw.get("K", 16), kw.get("N", 8), kw.get("group", 8)
    P = (max(K, 1) + 7) // 8
    G = (max(K, 1) + max(group, 1) - 1) // max(group, 1)
    qw = np.zeros(P * max(N, 1) - (1 if kw.get("qw_short") else 0), dtype=np.uint32)
    qz = np.zeros(G * 1 * 4 - (1 if kw.get("qz_short") else 0), dtype=np.uint8)
    sc = np.zeros(G * max(N, 1) - (1 if kw.get("sc_short") else 0), dtype=np.float32)
    rc, _ = orc.dequantize_gptq_int4(qw, qz, sc, K, N, group, kw.get("bits", 4))
    assert orc.ERRORS[rc] == code


def test_dequant_f16_is_encode_of_dequant(orc):
    """The fp16 arena the loader uploads = f32ToF16Bits(dequantizeGptqInt4(...)), including
    f16-subnormal scales (about 0.5 % of |N(0,1)|*0.01)."""
    rng = np.random.default_rng(7)
    K, N, group = 256, 48, 128
    qweight = rng.integers(0, 1 << 32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
    qzeros = rng.integers(0, 1 << 32, size=(K // group, N // 8), dtype=np.uint64).astype(np.uint32)
    s = np.abs(rng.standard_normal((K // group, N))).astype(np.float32) * 0.01
    s[0, :8] = np.float32(2.0 ** -20)   # subnormal in f16
    s[1, :4] = np.float32(2.0 ** -24)
    sf16 = s.astype(np.float16).view(np.uint16)
    got = orc.dequantize_gptq_int4_f16(qweight, qzeros, sf16, K, N, group)
    _, W = orc.dequantize_gptq_int4(qweight, qzeros, orc.f16_bits_to_f32(sf16), K, N, group)
    assert np.array_equal(got, orc.f32_to_f16_bits(W))
    # products of f16 values by small integers are never inside the (2^-25, 2^-24) flush range
    assert np.array_equal(got, W.astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------- gemmNTRef (a13)

def test_gemm_nt_vs_float64(orc):
    rng = np.random.default_rng(11)
    for M, N, K in [(1, 53, 42), (3, 64, 896), (5, 7, 1)]:
        A = rng.standard_normal((M, K)).astype(np.float32)
        W = rng.standard_normal((N, K)).astype(np.float32)
        b = rng.standard_normal(N).astype(np.float32)
        for bias in (None, b):
            C = orc.gemm_nt(A, W, bias)
            ref = A.astype(np.float64) @ W.astype(np.float64).T
            if bias is not None:
                ref = ref + bias.astype(np.float64)
            ref32 = ref.astype(np.float32)
            ulp = np.spacing(np.abs(ref32))
            assert np.all(np.abs(C - ref32) <= ulp)


def test_gemm_nt_hand_case(orc):
    A = np.array([[1, 2, 3]], dtype=np.float32)
    W = np.array([[1, 0, -1], [0.5, 0.25, 0.125]], dtype=np.float32)
    C = orc.gemm_nt(A, W, np.array([10, 0], dtype=np.float32))
    assert C.tolist() == [[8.0, 1.375]]


def test_gemm_nt_accumulates_in_double(orc):
    """1e8 + 1 - 1e8 in f32 loses the 1; the reference's JS-number accumulator keeps it."""
    A = np.array([[1e8, 1.0, -1e8]], dtype=np.float32)
    W = np.ones((1, 3), dtype=np.float32)
    assert orc.gemm_nt(A, W)[0, 0] == 1.0


def test_gptq_linear_equals_dequant_then_gemm(orc):
    rng = np.random.default_rng(13)
    K, N, M, group = 256, 40, 3, 128
    qweight = rng.integers(0, 1 << 32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
    qzeros = rng.integers(0, 1 << 32, size=(K // group, N // 8), dtype=np.uint64).astype(np.uint32)
    sf16 = (np.abs(rng.standard_normal((K // group, N))) * 0.01).astype(np.float16).view(np.uint16)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    _, W = orc.dequantize_gptq_int4(qweight, qzeros, orc.f16_bits_to_f32(sf16), K, N, group)
    for qz in (qzeros, None):
        _, W = orc.dequantize_gptq_int4(qweight, qz, orc.f16_bits_to_f32(sf16), K, N, group)
        y = orc.gptq_linear(qweight, qz, sf16, x, bias, group)
        assert np.array_equal(y, orc.gemm_nt(x, W, bias))


@pytest.mark.parametrize("K,N,M,threads", [(256, 40, 3, 1), (1000, 72, 5, 3), (896, 130, 16, 8)])
def test_gptq_linear_cols_bit_identical(orc, K, N, M, threads):
    """The threaded column-subset form returns gptq_linear's bits for any column order,
    repeated columns, ragged K (K % 8 != 0) and a remainder of fewer than 4 columns."""
    rng = np.random.default_rng(K + N)
    group = 128 if K % 128 == 0 else 8
    P, G = (K + 7) // 8, (K + group - 1) // group
    qweight = rng.integers(0, 1 << 32, size=(P, N), dtype=np.uint64).astype(np.uint32)
    qzeros = rng.integers(0, 1 << 32, size=(G, (N + 7) // 8), dtype=np.uint64).astype(np.uint32)
    sf16 = (np.abs(rng.standard_normal((G, N))) * 0.01).astype(np.float16).view(np.uint16)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    cols = np.concatenate([rng.permutation(N)[: N - 3], [0, N - 1, 0]]).astype(np.int32)
    for qz, b in ((qzeros, bias), (None, None)):
        full = orc.gptq_linear(qweight, qz, sf16, x, b, group)
        part = orc.gptq_linear_cols(qweight, qz, sf16, x, cols, b, group, threads=threads)
        assert np.array_equal(part.view(np.uint32), full[:, cols].view(np.uint32))
    with pytest.raises(ValueError):
        orc.gptq_linear_cols(qweight, qzeros, sf16, x, [N], None, group)
    # fp16 weights: gemmNTRef over the uploaded fp16 arena, bit for bit
    if K % 8 == 0:
        W16 = orc.f16_bits_to_f32(orc.dequantize_gptq_int4_f16(qweight, qzeros, sf16, K, N, group))
        part = orc.gptq_linear_cols(qweight, qzeros, sf16, x, cols, bias, group, threads=threads, w_f16=True)
        assert np.array_equal(part.view(np.uint32), orc.gemm_nt(x, W16, bias)[:, cols].view(np.uint32))


# ---------------------------------------------------------------- planGemvSplit (a7)

def test_plan_gemv_split_documented_table(orc):
    """src/model/qwen.ts:54-59 (Qwen2.5-0.5B schedule)."""
    assert orc.plan_gemv_split(1, 896) == 64      # k/v_proj
    assert orc.plan_gemv_split(4, 896) == 64      # q/o_proj
    assert orc.plan_gemv_split(4, 4864) == 64     # down_proj
    assert orc.plan_gemv_split(19, 896) == 16     # gate/up
    assert orc.plan_gemv_split(594, 896) == 1     # lm_head
    # 7B schedule under the same policy
    assert orc.plan_gemv_split(74, 3584) == 8
    assert orc.plan_gemv_split(14, 18944) == 32
    assert orc.plan_gemv_split(14, 3584) == 32


def test_plan_gemv_split_edge_cases(orc):
    assert orc.plan_gemv_split(256, 8) == 1
    assert orc.plan_gemv_split(1, 24) == 1        # 24/8 = 3 odd; 16, 32, 64 do not divide
    assert orc.plan_gemv_split(1, 48) == 8        # 48/8 = 6 even; 48/16 = 3 odd; 32, 64 do not divide
    assert orc.plan_gemv_split(300, 896) == 1
    assert orc.plan_gemv_split(16, 896) == 16     # 16*16 = 256 reaches the target exactly


# ---------------------------------------------------------------- checkTolerance, makeRng (a14)

def test_check_tolerance_hand_cases(orc):
    got = np.array([1.0, 2.0], dtype=np.float32)
    ref = np.array([1.0, 2.1], dtype=np.float32)
    ok, ma, mr = orc.check_tolerance(got, ref, 0.0, 0.05)
    assert ok and abs(ma - 0.1) < 1e-6 and abs(mr - 0.1 / 2.1) < 1e-6
    ok, _, _ = orc.check_tolerance(got, ref, 0.0, 0.04)
    assert not ok
    ok, _, mr = orc.check_tolerance(np.array([1e-6], np.float32), np.array([0.0], np.float32),
                                    1e-5, 0.0)
    assert ok and mr > 1e20       # near-zero reference: rel error explodes, atol passes
    with pytest.raises(ValueError):
        orc.check_tolerance(got, ref[:1], 0, 0)


def test_rng_golden(orc):
    d = json.load(open(os.path.join(GOLDEN, "rng.json")))
    for key, seed in [("seed_1", 1), ("seed_0", 0), ("seed_0x9ef0", 0x9EF0), ("seed_0x5e11", 0x5E11)]:
        r = orc.Rng(seed)
        assert [r.step() for _ in d[key]] == d[key]
    r = orc.Rng(1)
    assert r() == 270369 / 2 ** 32


def _xorshift_py(seed, n):
    """makeRng in Python ints (cpu-ref.ts:57-67), independent of the C oracle."""
    s = (seed & 0xFFFFFFFF) or 1
    out = []
    for _ in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out.append(s)
    return out


def test_random_f32_closed_form(orc):
    """randomF32 (cpu-ref.ts:50-54): f32(s/2^32 * 2 - 1) = f32((s - 2^31) / 2^31); the double is
    exact, numpy rounds it to f32 (RNE) independently; values lie in [-1, 1)."""
    for seed in (0x9EF0, 0x5E11, 1):
        got = orc.Rng(seed).random_f32(4096)
        want = np.array([(s - 2 ** 31) / 2 ** 31 for s in _xorshift_py(seed, 4096)], np.float64).astype(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        assert got.min() >= -1.0 and got.max() < 1.0
    # a value that needs rounding: s = 2^31 + 1 gives 2^-31, exact; s = 1 gives -1 + 2^-31 -> -1 in f32
    assert np.float32((1 - 2 ** 31) / 2 ** 31) == np.float32(-1.0)


def test_make_normal_box_muller(orc):
    """makeNormal (init.ts:36-52): values in pairs (cos first, then the kept sin), zero draws
    skipped; against a float64 numpy Box-Muller over the Python-int stream to 1e-15 relative
    (libm vs V8 transcendental last-ulp differences stay within that), and N(0,1) moments."""
    seed, n = 0x1234, 20000
    nrm = orc.Normal(seed)
    got = np.array([nrm() for _ in range(n)])
    u = np.array(_xorshift_py(seed, n), np.float64) / 2 ** 32      # no zero draws for this seed
    assert np.all(u > 0)
    uu, vv = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(uu))
    want = np.empty(n)
    want[0::2] = r * np.cos(2 * np.pi * vv)
    want[1::2] = r * np.sin(2 * np.pi * vv)
    assert np.allclose(got, want, rtol=1e-15, atol=1e-15)
    assert abs(got.mean()) < 0.03 and abs(got.std() - 1) < 0.02


def _attention_torch(q, kc, vc, H, KV, D, past):
    """Textbook causal attention in float64 (torch.softmax), kv head h // (H // KV) repeated per
    query head: an independent route to the same numbers."""
    import torch
    M = q.shape[0]
    T = past + M
    Q = torch.from_numpy(q.astype(np.float64)).reshape(M, H, D).transpose(0, 1)           # [H, M, D]
    Kt = torch.from_numpy(kc[:T].astype(np.float64)).reshape(T, KV, D).transpose(0, 1)    # [KV, T, D]
    Vt = torch.from_numpy(vc[:T].astype(np.float64)).reshape(T, KV, D).transpose(0, 1)
    Kt = Kt.repeat_interleave(H // KV, dim=0)
    Vt = Vt.repeat_interleave(H // KV, dim=0)
    S = Q @ Kt.transpose(1, 2) / np.sqrt(D)
    pos = past + torch.arange(M).unsqueeze(1)
    S = S.masked_fill(torch.arange(T).unsqueeze(0) > pos, float("-inf"))
    return (torch.softmax(S, dim=-1) @ Vt).transpose(0, 1).numpy()                        # [M, H, D]


@pytest.mark.parametrize("M,H,KV,D,past", [(1, 14, 2, 64, 0), (1, 14, 2, 64, 127), (5, 4, 2, 48, 9),
                                           (3, 8, 8, 16, 30), (1, 28, 4, 128, 300)])
def test_attention_oracle_vs_textbook(orc, M, H, KV, D, past):
    """The attention oracle against softmax(QK^T / sqrt(D)) V in float64 with a causal mask
    and grouped kv heads (a swapped head mapping h % KV, a missing scale or an off-by-one in the
    visible range all fail this)."""
    rng = np.random.default_rng(M * 1000 + past)
    T = past + M
    q = rng.standard_normal((M, H, D)).astype(np.float32)
    kc = rng.standard_normal((T, KV * D)).astype(np.float32)
    vc = rng.standard_normal((T, KV * D)).astype(np.float32)
    got = orc.attention_gqa_cache(q, kc, vc, H, KV, D, past)
    ref = _attention_torch(q, kc, vc, H, KV, D, past)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6), np.abs(got - ref).max()


def test_attention_oracle_special_cases(orc):
    """One visible key: the output is that key's value, exactly. Equal keys: uniform weights, the
    mean of the values."""
    rng = np.random.default_rng(7)
    H, KV, D = 4, 2, 32
    q = rng.standard_normal((1, H, D)).astype(np.float32)
    kc = rng.standard_normal((1, KV * D)).astype(np.float32)
    vc = rng.standard_normal((1, KV * D)).astype(np.float32)
    got = orc.attention_gqa_cache(q, kc, vc, H, KV, D, 0)
    for h in range(H):
        kvh = h // (H // KV)
        assert np.array_equal(got[0, h], vc[0, kvh * D:(kvh + 1) * D])
    T = 9
    kc = np.tile(rng.standard_normal((1, KV * D)).astype(np.float32), (T, 1))
    vc = rng.standard_normal((T, KV * D)).astype(np.float32)
    got = orc.attention_gqa_cache(q, kc, vc, H, KV, D, T - 1)
    for h in range(H):
        kvh = h // (H // KV)
        assert np.allclose(got[0, h], vc[:, kvh * D:(kvh + 1) * D].astype(np.float64).mean(0), atol=1e-6)


def test_rmsnorm_oracle_vs_textbook(orc):
    """rmsNormRef restated, against x / sqrt(mean(x^2) + eps) * w in float64 (numpy), with and
    without the residual add; a constant row c gives c / sqrt(c^2 + eps) * w."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((5, 896)).astype(np.float32)
    d = rng.standard_normal((5, 896)).astype(np.float32)
    w = rng.standard_normal(896).astype(np.float32)
    for dd in (None, d):
        s, y = orc.add_rmsnorm(x, w, 1e-6, dd)
        s64 = x.astype(np.float64) + (0 if dd is None else dd.astype(np.float64))
        assert np.array_equal(s, (x + d) if dd is not None else x)
        ref = s.astype(np.float64) / np.sqrt((s.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * w
        assert np.allclose(y, ref, rtol=2e-7, atol=1e-7)
        assert np.allclose(s, s64, rtol=1e-7)
    c = np.full((1, 64), 3.0, np.float32)
    _, y = orc.add_rmsnorm(c, np.ones(64, np.float32), 1e-6)
    assert np.allclose(y, 3.0 / np.sqrt(9.0 + 1e-6), rtol=1e-7)


def test_silu_mul_oracle_vs_expit(orc):
    """siluMulRef restated, against scipy's logistic function: g * expit(g) * u; silu(0) = 0."""
    from scipy.special import expit
    rng = np.random.default_rng(12)
    g = (rng.standard_normal(4097) * 6).astype(np.float32)
    u = rng.standard_normal(4097).astype(np.float32)
    got = orc.silu_mul(g, u)
    ref = g.astype(np.float64) * expit(g.astype(np.float64)) * u
    assert np.allclose(got, ref, rtol=2e-7, atol=1e-30)
    assert orc.silu_mul(np.zeros(3, np.float32), np.ones(3, np.float32)).tolist() == [0.0, 0.0, 0.0]
