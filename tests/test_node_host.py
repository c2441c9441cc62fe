"""The Node host (webllm_amd/js over the Node-API addon): the reference's own host language.

CPU: the addon loads under Node and exports the binding of every C-ABI entry point the host
needs; its plans and validation codes equal the Python binding's. GPU: loadQwenWeights on a
synthetic checkpoint, QuantLinearModel.gemm / gemmBatch / unpackF16 and dequantizeGptqInt4 from
JavaScript, checked against the C oracle with the same bars as the Python-host tests."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from webllm_amd import gptq, synth
from webllm_amd import qlinear as ql

from .checkpoint import TINY, post_norm_weight, write_checkpoint

NODE = shutil.which("node")
HERE = os.path.dirname(os.path.abspath(__file__))
SCRIPT = os.path.join(HERE, "js", "node_host_check.js")
ADDON = os.path.join(os.path.dirname(HERE), "webllm_amd", "lib", "qlinear_napi.node")

needs_node = pytest.mark.skipif(NODE is None, reason="node not installed")

# the N-API exports and the C-ABI entry points each one forwards to
BINDING = {
    "create": "ql_create", "destroy": "ql_destroy", "deviceInfo": "ql_device_info",
    "lastError": "ql_last_error", "arenaReserve": "ql_arena_reserve",
    "arenaRelease": "ql_arena_release", "arenaSize": "ql_arena_size",
    "arenaWrite": "ql_arena_write", "arenaRead": "ql_arena_read", "gptqSizes": "ql_gptq_sizes",
    "validate": "ql_gptq_validate", "planLinear": "ql_plan_linear", "planBatch": "ql_plan_batch",
    "unpack": "ql_unpack_f16", "unpackBatch": "ql_unpack_f16_batch", "linear": "ql_linear", "linearBatch": "ql_linear_batch",
    "sync": "ql_sync", "timerStart": "ql_timer_start", "timerStop": "ql_timer_stop",
    "graphBegin": "ql_graph_begin", "graphEnd": "ql_graph_end", "graphLaunch": "ql_graph_launch",
    "graphDestroy": "ql_graph_destroy", "seqCreate": "ql_seq_create", "seqRun": "ql_seq_run",
    "seqStatus": "ql_seq_status", "seqInfo": "ql_seq_get_info", "seqDestroy": "ql_seq_destroy",
    "gemvF16w": "ql_gemv_f16w", "embedF16": "ql_embed_f16", "kvStore": "ql_kv_store", "attention": "ql_attention_decode",
    "addRmsNorm": "ql_add_rmsnorm", "siluMul": "ql_silu_mul",
}


def _node(mode, d, timeout):
    r = subprocess.run([NODE, SCRIPT, mode, str(d)], capture_output=True, text=True,
                       timeout=timeout)
    assert r.returncode == 0, r.stderr[-4000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


def _js_config(c):
    return {"vocabSize": c.vocab_size, "blockSize": c.block_size, "nLayer": c.n_layer,
            "nHead": c.n_head, "nKvHead": c.n_kv_head, "nEmbd": c.n_embd,
            "intermediate": c.intermediate}


@needs_node
def test_addon_exports_and_host_logic(tmp_path):
    assert os.path.exists(ADDON), "run __graft_entry__.build() first"
    kept = write_checkpoint(str(tmp_path / "model.safetensors"), TINY)
    write_checkpoint(str(tmp_path / "act_order.safetensors"), TINY, act_order=(1, "gateW"))
    res = _node("abi", tmp_path, 120)
    pr = res["probes"]
    assert pr["gIdxOk"] is None
    assert "is not the identity map i/128" in pr["gIdxActOrder"]
    rows = np.fromfile(tmp_path / "rows.f32", dtype=np.float32)
    assert np.array_equal(rows, kept["embed"][5:8].astype(np.float32).reshape(-1))
    t, _ = kept[(0, "kW")]
    nib = (t.qzeros[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
    assert pr["zerosK"] == np.bincount(nib.reshape(-1)[: t.qzeros.shape[0] * t.N], minlength=16).tolist()
    assert pr["urls"] == ["/tmp/a b/model.safetensors", "rel/model.safetensors"]
    assert "only a local path" in pr["badUrl"]
    assert res["exports"] == sorted(BINDING)
    declared = set(ql.header_functions())
    assert set(BINDING.values()) <= declared
    for p in res["plans"]:
        want = ql.plan_linear(p["M"], p["N"], p["K"], 128)
        assert p["kind"] == want.kind_name and p["split"] == want.split
        assert p["gridX"] == want.grid_x and p["scratchBytes"] == want.scratch_bytes
        assert p["refSplit"] == want.ref_split
    assert res["validate"] == {"ok": 0, "bits": -1, "group": -2, "dims": -3, "pack": -7}
    assert tuple(res["sizes"].values()) == ql.gptq_sizes(896, 4864, 128)
    assert res["tensors"] == 2 + TINY.n_layer * (2 + 7 * 4 + 3)
    assert res["embedShape"] == [TINY.vocab_size, TINY.n_embd]
    assert "too short" in res["badParse"]


@needs_node
@pytest.mark.gpu
def test_node_host_matches_oracle(tmp_path, orc):
    kept = write_checkpoint(str(tmp_path / "model.safetensors"), TINY)
    write_checkpoint(str(tmp_path / "act_order.safetensors"), TINY, act_order=(1, "downW"))
    shapes = gptq.qwen_linear_shapes(TINY)
    cases = {"config": _js_config(TINY), "gemm": [], "batch": []}
    refs = {}
    for i, (key, M, f16) in enumerate([("qW", 1, False), ("gateW", 1, False), ("downW", 3, False),
                                       ("upW", 16, False), ("kW", 64, False), ("oW", 70, True)]):
        K, N = shapes[key]
        t, b = kept[(0, key)]
        x = synth.activations(M, K, seed=0x40DE, key=(i,))
        if f16:
            x = x.astype(np.float16).astype(np.float32)
            x.astype(np.float16).tofile(tmp_path / f"x{i}")
        else:
            x.tofile(tmp_path / f"x{i}")
        bias = f"L0.{key[0]}B" if b is not None else None
        cases["gemm"].append({"weight": f"L0.{key}", "M": M, "N": N, "K": K, "bias": bias,
                              "f16": f16, "x": f"x{i}", "out": f"y{i}.f32"})
        refs[f"y{i}.f32"] = (orc.gptq_linear(t.qweight, t.qzeros, t.scales, x, b), M >= 17)
    emb = kept["embed"]                      # the tied lm_head over the fp16 embedding (qwen.ts:488-489)
    for j, M in enumerate((1, 5)):
        x = synth.activations(M, TINY.n_embd, seed=0x40E0, key=(M,))
        x.tofile(tmp_path / f"xe{j}")
        cases["gemm"].append({"weight": "embed", "M": M, "N": TINY.vocab_size, "K": TINY.n_embd, "bias": None,
                              "f16": False, "x": f"xe{j}", "out": f"ye{j}.f32"})
        refs[f"ye{j}.f32"] = (orc.gemm_nt(x, emb.astype(np.float32)), False)
    xb = synth.activations(2, TINY.n_embd, seed=0x40DF)
    xb.tofile(tmp_path / "xb")
    names = ["qW", "kW", "vW"]
    cases["batch"].append({"weights": [f"L1.{k}" for k in names], "M": 2, "K": TINY.n_embd,
                           "N": [shapes[k][1] for k in names], "x": "xb",
                           "outs": [f"b{k}.f32" for k in names]})
    for k in names:
        t, b = kept[(1, k)]
        refs[f"b{k}.f32"] = (orc.gptq_linear(t.qweight, t.qzeros, t.scales, xb, b), False)
    seq_names = ["qW", "oW", "gateW", "downW"]
    xs = synth.activations(1, TINY.n_embd, seed=0x40E0)
    xs.tofile(tmp_path / "xs")
    cases["seq"] = {"weights": [f"L0.{k}" for k in seq_names], "M": 1, "x": "xs",
                    "outs": [f"s{k}.f32" for k in seq_names]}
    fz = ["qW", "kW", "vW", "oW", "gateW", "upW", "downW"]
    xf = synth.activations(1, TINY.n_embd, seed=0x40E7)
    xf.tofile(tmp_path / "xf")
    cases["fused"] = {"x": "xf", "M": 1, "eps": 1e-6, "outs": [f"f{k}.f32" for k in fz]}
    K, N = shapes["gateW"]
    cases["unpack"] = {"weight": "L1.gateW", "N": N, "K": K, "out": "u.f16"}
    ua = ["gateW", "downW", "kW"]
    cases["unpackAll"] = {"weights": [f"L0.{k}" for k in ua], "N": [shapes[k][1] for k in ua],
                          "K": [shapes[k][0] for k in ua], "outs": [f"ua_{k}.f16" for k in ua]}
    cases["dequant"] = {"prefix": "model.layers.1.mlp.down_proj", "K": shapes["downW"][0],
                        "N": shapes["downW"][1], "out": "w.f32"}
    rng_s = np.random.default_rng(0x40E6)
    dK, dN, dG = 256, 48, 64
    d_qw = rng_s.integers(0, 1 << 32, size=(dK // 8, dN), dtype=np.uint64).astype(np.uint32)
    d_qz = rng_s.integers(0, 1 << 32, size=(dK // dG, dN // 8), dtype=np.uint64).astype(np.uint32)
    d_sc = (rng_s.standard_normal((dK // dG, dN)) * 0.01).astype(np.float32)
    d_sc[0, :8], d_sc[1, :8] = np.float32(1e-44), np.float32(3e38)
    for name, arr in (("dq_qw", d_qw), ("dq_qz", d_qz), ("dq_sc", d_sc)):
        arr.tofile(tmp_path / name)
    cases["dequantF32"] = {"qweight": "dq_qw", "qzeros": "dq_qz", "scales": "dq_sc", "K": dK, "N": dN,
                           "group": dG, "out": "w32.f32"}
    # residual add + RMSNorm over the loaded L0.inNorm (ones in the checkpoint), SiLU-mul, and
    # three decode steps of the KV cache on layer 1
    ex, er = synth.activations(2, TINY.n_embd, seed=0x40E1), synth.activations(2, TINY.n_embd, seed=0x40E2)
    eg, eu = synth.activations(1, 2 * TINY.intermediate, seed=0x40E3), synth.activations(1, 2 * TINY.intermediate, seed=0x40E4)
    for name, arr in (("el_x", ex), ("el_r", er), ("el_g", eg), ("el_u", eu)):
        arr.tofile(tmp_path / name)
    cases["elem"] = {"M": 2, "C": TINY.n_embd, "n": 2 * TINY.intermediate, "x": "el_x", "r": "el_r",
                     "g": "el_g", "u": "el_u"}
    es, ey = orc.add_rmsnorm(ex, np.ones(TINY.n_embd, np.float32), 1e-6, er)
    refs["el_y.f32"] = (ey, False)
    refs["el_o.f32"] = (orc.silu_mul(eg, eu), False)
    H, KVH = TINY.n_head, TINY.n_kv_head
    D = TINY.n_embd // H
    rng = np.random.default_rng(0x40E5)
    kk, vv = [], []
    cases["kvSteps"] = 3
    for t in range(3):
        k, v = (rng.standard_normal((1, KVH * D)).astype(np.float32) for _ in range(2))
        qv = rng.standard_normal((1, H * D)).astype(np.float32)
        for name, arr in (("kv_k", k), ("kv_v", v), ("kv_q", qv)):
            arr.tofile(tmp_path / f"{name}{t}")
        kk.append(k)
        vv.append(v)
        refs[f"kv_o{t}.f32"] = (orc.attention_gqa_cache(qv.reshape(1, H, D), np.concatenate(kk), np.concatenate(vv),
                                                        H, KVH, D, t).reshape(1, H * D), False)
    (tmp_path / "cases.json").write_text(json.dumps(cases))

    print(f"node host: {len(cases['gemm'])} gemm cases, 1 batch", flush=True)
    res = _node("gpu", tmp_path, 300)

    assert np.array_equal(np.fromfile(tmp_path / "el_s.f32", dtype=np.float32).reshape(es.shape), es)
    assert res["tensorCount"] == 2 + TINY.n_layer * (2 + 7 + 3)
    assert res["progress"] == list(range(1, TINY.n_layer + 1))
    for out, (ref, gemm) in refs.items():
        got = np.fromfile(tmp_path / out, dtype=np.float32).reshape(ref.shape)
        # decode GEMV: |d| <= 1e-5 + 1e-4|ref|; MFMA f16 GEMM (M >= 17): 2e-3 normwise
        if gemm:
            err = np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)
            assert err <= 2e-3, (out, err)
        else:
            ok, max_abs, max_rel = orc.check_tolerance(got, ref, 1e-5, 1e-4)
            assert ok, (out, max_abs, max_rel)
    t, _ = kept[(1, "gateW")]
    u = np.fromfile(tmp_path / "u.f16", dtype=np.uint16).reshape(t.N, t.K)
    assert np.array_equal(u, orc.dequantize_gptq_int4_f16(t.qweight, t.qzeros, t.scales, t.K, t.N, 128))
    for k in ("gateW", "downW", "kW"):
        t, _ = kept[(0, k)]
        u = np.fromfile(tmp_path / f"ua_{k}.f16", dtype=np.uint16).reshape(t.N, t.K)
        assert np.array_equal(u, orc.dequantize_gptq_int4_f16(t.qweight, t.qzeros, t.scales, t.K, t.N, 128)), k
    for out, (t, _) in (("w.f32", kept[(1, "downW")]), ("kept_qW.f32", kept[(0, "qW")])):
        _, W = orc.dequantize_gptq_int4(t.qweight, t.qzeros, orc.f16_bits_to_f32(t.scales), t.K,
                                        t.N, 128)
        got = np.fromfile(tmp_path / out, dtype=np.float32).reshape(t.N, t.K)
        assert np.array_equal(got.view(np.uint32), W.view(np.uint32)), out
    # the JavaScript-built sequence: each linear against the oracle on the input it consumed
    assert res["seqInfo"]["passes"] == 4 and res["seqInfo"]["linears"] == 4
    x_in = xs
    for k in seq_names:
        t, b = kept[(0, k)]
        y = np.fromfile(tmp_path / f"s{k}.f32", dtype=np.float32).reshape(1, t.N)
        ref = orc.gptq_linear(t.qweight, t.qzeros, t.scales, x_in, b)
        atol = 1e-5 * max(1.0, float(np.sqrt(np.mean(x_in.astype(np.float64) ** 2))))
        ok, max_abs, _ = orc.check_tolerance(y, ref, atol, 1e-4)
        assert ok, f"seq {k}: maxAbs {max_abs:.3e}"
        x_in = y
    # the JavaScript-built fused layer: each linear against the oracle's composition on the inputs
    # the GPU used (rmsNormRef / siluMulRef, gemmNTRef, vec_add)
    assert res["fusedInfo"]["passes"] == 4 and res["fusedInfo"]["linears"] == 7
    assert res["fusedInfo"]["kernel"] == 0          # QL_SEQ_TILES
    assert res["fusedBoth"] and "QL_E_INVALID" in res["fusedBoth"]
    ys = {k: np.fromfile(tmp_path / f"f{k}.f32", dtype=np.float32).reshape(1, -1) for k in fz}
    ln1, ln2 = np.ones(TINY.n_embd, np.float32), post_norm_weight(TINY, 0)
    n1 = orc.add_rmsnorm(xf, ln1, 1e-6)[1]
    n2 = orc.add_rmsnorm(ys["oW"], ln2, 1e-6)[1]
    plan = {"qW": (n1, None), "kW": (n1, None), "vW": (n1, None), "oW": (ys["qW"], xf),
            "gateW": (n2, None), "upW": (n2, None),
            "downW": (orc.silu_mul(ys["gateW"], ys["upW"]), ys["oW"])}
    for k in fz:
        t, b = kept[(0, k)]
        x_in, res_in = plan[k]
        ref = orc.gptq_linear(t.qweight, t.qzeros, t.scales, x_in, b)
        if res_in is not None:
            ref = ref + res_in
        atol = 1e-5 * max(1.0, float(np.sqrt(np.mean(x_in.astype(np.float64) ** 2))))
        ok, max_abs, _ = orc.check_tolerance(ys[k], ref, atol, 1e-4)
        assert ok, f"fused {k}: maxAbs {max_abs:.3e}"
    got = np.fromfile(tmp_path / "w32.f32", dtype=np.float32).reshape(dN, dK)
    _, want = orc.dequantize_gptq_int4(d_qw, d_qz, d_sc, dK, dN, dG)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert res["isPromise"]
    assert np.array_equal(np.fromfile(tmp_path / "embed_rows.f32", dtype=np.float32),
                          kept["embed"][100:104].astype(np.float32).reshape(-1))
    want_z = np.zeros(16, np.int64)
    for key, (t, _) in ((k, v) for k, v in kept.items() if k != "embed"):
        nib = (t.qzeros[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
        want_z += np.bincount(nib.reshape(t.qzeros.shape[0], -1)[:, :t.N].reshape(-1), minlength=16)
    assert res["storedZeros"] == {str(v): int(c) for v, c in enumerate(want_z) if c}
    assert "model.layers.1.mlp.down_proj.g_idx" in res["actOrder"]
    e = res["errors"]
    assert "missing int4 weight: L9.qW" in e["missingWeight"]
    assert "called with N=" in e["wrongShape"]
    assert "missing f32 weight: L0.oB" in e["missingBias"]
    assert "already exists" in e["duplicate"]
    assert "QL_E_BITS" in e["bits"]
    assert "share one arena" in e["rmsnormArena"] and "share one arena" in e["rmsnormSumArena"]
    assert "share one arena" in e["attendArena"]
