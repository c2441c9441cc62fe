"""GPU tests of the host mirror: load a synthetic Qwen-shaped GPTQ checkpoint through
load_qwen_weights (qwen-loader.ts) and run QwenGpt.gemm-style dispatch, checked against the
oracle. The checks restate the reference's loader exactness test (tests/infer/qwen-infer.ts:33-57:
the uploaded fp16 weights equal f16(CPU dequant), first 4096 elements of L0 q/k/o/gate/up/down)."""
import json
import os

import numpy as np
import pytest

from webllm_amd import gptq, synth
from webllm_amd import qlinear as ql

from .checkpoint import TINY, write_checkpoint as _checkpoint

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def loaded(ctx, tmp_path_factory):
    path = str(tmp_path_factory.mktemp("ckpt") / "model.safetensors")
    kept = _checkpoint(path, TINY)
    model = gptq.QuantLinearModel(ctx, 64 << 20)
    progress = []
    res = gptq.load_qwen_weights(model, path, TINY, on_progress=lambda *a: progress.append(a),
                                 keep_layer=0)
    return model, res, kept, progress


def test_loader_result_and_progress(loaded):
    model, res, kept, progress = loaded
    assert res.tensor_count == 2 + TINY.n_layer * (2 + 7 + 3)
    assert res.gpu_bytes == model.weight_bytes > 0
    assert [p[0] for p in progress] == list(range(1, TINY.n_layer + 1))
    assert set(res.layer) == {k for k, _ in gptq._PROJ}


def test_loader_exactness_fp16_first_4096(loaded, orc, ctx):
    """qwen-infer.ts:33-57 restated: uploaded fp16 == f16(CPU dequant), first 4096 elements."""
    model, res, kept, _ = loaded
    pool = gptq.ActivationArena(ctx, 16 << 20)
    for key in ("qW", "kW", "oW", "gateW", "upW", "downW"):
        t, _ = kept[(0, key)]
        out = pool.alloc((t.N, t.K), "f16")
        model.unpack_f16(f"L0.{key}", out)
        got = out.read().view(np.uint16).reshape(-1)[:4096]
        want = orc.dequantize_gptq_int4_f16(t.qweight, t.qzeros, t.scales, t.K, t.N, 128).reshape(-1)[:4096]
        assert np.array_equal(got, want), key
        # keep_layer returns the exact fp32 dequant (quant.ts output)
        _, W = orc.dequantize_gptq_int4(t.qweight, t.qzeros, orc.f16_bits_to_f32(t.scales), t.K, t.N, 128)
        assert np.array_equal(res.layer[key].view(np.uint32), W.view(np.uint32)), key
        pool.reset()


def test_gemm_dispatch_matches_oracle(loaded, orc, ctx):
    model, _, kept, _ = loaded
    pool = gptq.ActivationArena(ctx, 32 << 20)
    for M in (1, 3, 64):
        for key in ("qW", "vW", "downW"):
            t, b = kept[(1, key)]
            x = synth.activations(M, t.K, seed=0x77, key=(M,))
            A = pool.alloc((M, t.K))
            C = pool.alloc((M, t.N))
            A.write(x)
            model.gemm(A, f"L1.{key}", C, f"L1.{key[0]}B" if b is not None else None, M, t.N, t.K)
            y = C.read()
            if M <= 16:
                ref = orc.gptq_linear(t.qweight, t.qzeros, t.scales, x, b)
                ok, ma, _ = orc.check_tolerance(y, ref, 1e-5, 1e-4)
            else:
                W16 = orc.f16_bits_to_f32(orc.dequantize_gptq_int4_f16(t.qweight, t.qzeros, t.scales, t.K, t.N, 128))
                ref = orc.gemm_nt(orc.f16_bits_to_f32(orc.f32_to_f16_bits(x)), W16, b)
                ok, ma, _ = orc.check_tolerance(y, ref, 1e-5, 2e-3)
            assert ok, (M, key, ma)
            pool.reset()


def test_gemm_lm_head_over_embed(loaded, orc, ctx):
    """gemm(lnf, 'embed', logits, null, M, V, C) (qwen.ts:488-489): the tied fp16 embedding as the
    lm_head weight, f32 in and out, at the GEMV bar; M = 6 takes two passes over the weights."""
    model, _, kept, _ = loaded
    emb = kept["embed"]
    V, C = emb.shape
    pool = gptq.ActivationArena(ctx, 8 << 20)
    for M in (1, 6):
        x = synth.activations(M, C, seed=0x79, key=(M,))
        A, L = pool.alloc((M, C)), pool.alloc((M, V))
        A.write(x)
        model.gemm(A, "embed", L, None, M, V, C)
        ok, ma, _ = orc.check_tolerance(L.read(), orc.gemm_nt(x, emb.astype(np.float32)), 1e-5, 1e-4)
        assert ok, (M, ma)
        with pytest.raises(ValueError, match="embed"):
            model.gemm(A, "embed", L, None, M, V - 1, C)
        pool.reset()


def test_gemm_batch_qkv(loaded, orc, ctx):
    model, _, kept, _ = loaded
    pool = gptq.ActivationArena(ctx, 8 << 20)
    x = synth.activations(2, TINY.n_embd, seed=0x78)
    A = pool.alloc((2, TINY.n_embd))
    A.write(x)
    outs = [pool.alloc((2, kept[(0, k)][0].N)) for k in ("qW", "kW", "vW")]
    model.gemm_batch(A, ["L0.qW", "L0.kW", "L0.vW"], outs, 2)
    for k, C in zip(("qW", "kW", "vW"), outs):
        t, b = kept[(0, k)]
        ok, ma, _ = orc.check_tolerance(C.read(), orc.gptq_linear(t.qweight, t.qzeros, t.scales, x, b), 1e-5, 1e-4)
        assert ok, (k, ma)


def test_gemm_errors(loaded, ctx):
    model, _, _, _ = loaded
    pool = gptq.ActivationArena(ctx, 1 << 20)
    A, C = pool.alloc((1, 256)), pool.alloc((1, 256))
    with pytest.raises(ValueError, match="missing int4 weight"):
        model.gemm(A, "L9.qW", C, None, 1, 256, 256)
    with pytest.raises(ValueError, match="missing f32 weight"):
        model.gemm(A, "L0.oW", C, "L0.oB", 1, 256, 256)
    with pytest.raises(ValueError):
        model.gemm(A, "L0.oW", C, None, 1, 128, 256)


def test_loader_rejects_wrong_shapes(ctx, tmp_path):
    path = str(tmp_path / "bad.safetensors")
    _checkpoint(path, TINY)
    model = gptq.QuantLinearModel(ctx, 64 << 20)
    bigger = gptq.QwenConfig(512, 16, 2, 4, 2, 256, 768)     # intermediate differs
    with pytest.raises(ValueError, match="shape"):
        gptq.load_qwen_weights(model, path, bigger)
    with pytest.raises(ValueError, match="embed_tokens"):
        gptq.load_qwen_weights(gptq.QuantLinearModel(ctx, 64 << 20), path,
                               gptq.QwenConfig(1000, 16, 2, 4, 2, 256, 640))


def test_loader_url_embed_rows_and_zero_counts(ctx, tmp_path):
    """loadQwenWeights options: url (file://), keepEmbedRows -> embedRows (qwen-loader.ts:134-135,
    :175), and the stored-zero counts of the format probe (qwen-format.ts:112-123)."""
    path = tmp_path / "model.safetensors"
    kept = _checkpoint(str(path), TINY)
    model = gptq.QuantLinearModel(ctx, 64 << 20)
    res = gptq.load_qwen_weights(model, url=path.as_uri(), config=TINY,
                                 keep_embed_rows={"start": 100, "rows": 4})
    assert np.array_equal(res.embed_rows, kept["embed"][100:104].astype(np.float32).reshape(-1))
    want = np.zeros(16, np.int64)
    for (i, key), (t, _) in ((k, v) for k, v in kept.items() if k != "embed"):
        nib = (t.qzeros[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
        want += np.bincount(nib.reshape(t.qzeros.shape[0], -1)[:, :t.N].reshape(-1), minlength=16)
    assert res.stored_zeros == {v: int(c) for v, c in enumerate(want) if c}
    assert res.layer is None and res.file_bytes == os.path.getsize(path)
    model.release()


def test_loader_rejects_act_order_checkpoint(ctx, tmp_path):
    """A desc_act=true checkpoint (permuted g_idx) would load and compute wrong outputs with
    kernels that assume g = k / group: the loader throws (qwen-format.ts:125-130)."""
    path = str(tmp_path / "model.safetensors")
    _checkpoint(path, TINY, act_order=(1, "downW"))
    model = gptq.QuantLinearModel(ctx, 64 << 20)
    with pytest.raises(ValueError, match="not the identity"):
        gptq.load_qwen_weights(model, path, TINY)
    model.release()


def test_dequantize_gptq_int4_any_f32_scales(ctx, orc):
    """Scales that fp16 cannot represent, subnormal products, overflow to inf and NaN scales,
    as any Float32Array may hold (quant.ts:22-23): bit-identical to the oracle's dequant."""
    rng = np.random.default_rng(0x5CA1)
    K, N, group = 256, 40, 64
    qw = rng.integers(0, 1 << 32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
    qz = rng.integers(0, 1 << 32, size=(K // group, N // 8), dtype=np.uint64).astype(np.uint32)
    sc = (rng.standard_normal((K // group, N)) * 0.01).astype(np.float32)
    sc[0, :8] = np.float32(1e-44)               # products in the f32 subnormal range
    sc[1, :8] = np.float32(3e38)                # products overflow to +-inf
    sc[2, 0] = np.float32("nan")
    sc[3, :8] = -sc[3, :8]
    for qzeros in (qz, None):
        rc, want = orc.dequantize_gptq_int4(qw, qzeros, sc, K, N, group)
        assert rc == 0
        got = gptq.dequantize_gptq_int4(ctx, qw.tobytes(), None if qzeros is None else qzeros.tobytes(),
                                        sc, K, N, group)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequantize_gptq_int4_reference_kat(ctx):
    """quant.ts through the GPU drop-in on the reference's own KAT (weights.ts:62-137), with its
    f32 scales 0.01*(g+1)*(o+1) (not fp16 values): bit-identical to the KAT's expected weights,
    and the symmetric fallback (qzeros null -> zero 8) gives the same values here because the KAT
    stores zero 7."""
    d = json.load(open(os.path.join(GOLDEN, "gptq_kat.json")))
    qw = np.array(d["qweight_u32"], np.uint32).tobytes()
    qz = np.array(d["qzeros_u32"], np.uint32).tobytes()
    sc = np.array(d["scales_f32_bits"], np.uint32).view(np.float32)
    want = np.array(d["want_f32_bits"], np.uint32)
    got = gptq.dequantize_gptq_int4(ctx, qw, qz, sc, 16, 5, 8)
    assert np.array_equal(got.view(np.uint32).reshape(-1), want)
    got_sym = gptq.dequantize_gptq_int4(ctx, qw, None, sc, 16, 5, 8)
    assert np.array_equal(got_sym.view(np.uint32).reshape(-1), want)
    # fp16-valued scales (what a checkpoint holds) give the closed form on those scales
    s16 = sc.astype(np.float16).astype(np.float32)
    q = [[(o * 7 + i * 3) & 15 for i in range(16)] for o in range(5)]
    want16 = np.array([[(q[o][i] - 8) * s16[(i // 8) * 5 + o] for i in range(16)] for o in range(5)],
                      dtype=np.float32)
    got16 = gptq.dequantize_gptq_int4(ctx, qw, qz, s16, 16, 5, 8)
    assert np.array_equal(got16.view(np.uint32), want16.view(np.uint32))
    for kw, code in [(dict(bits=3), "QL_E_BITS"), (dict(group_size=0), "QL_E_GROUP"),
                     (dict(in_features=0), "QL_E_DIMS"), (dict(group_size=12), "QL_E_GROUP_PACK")]:
        args = dict(in_features=16, out_features=5, group_size=8)
        args.update(kw)
        with pytest.raises(ql.QlError) as e:
            gptq.dequantize_gptq_int4(ctx, qw, qz, s16, **args)
        assert e.value.name == code
    with pytest.raises(ql.QlError) as e:
        gptq.dequantize_gptq_int4(ctx, qw[:-4], qz, s16, 16, 5, 8)
    assert e.value.name == "QL_E_QWEIGHT_SHORT"
