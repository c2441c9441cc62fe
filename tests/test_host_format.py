"""Safetensors format boundary of the host mirror (webllm_amd/gptq.py), CPU only.
Restates the reference's testWeightsFormat file (tests/qwen/weights.ts:7-41, :44-60) and the
parser's error checks (src/weights/safetensors.ts:84-124)."""
import json
import struct

import numpy as np
import pytest

from webllm_amd import gptq


def _reference_test_file() -> bytes:
    """weights.ts:7-41: F32 bias [1,-2,0.5], F16 [1,-0.5], BF16 [1,-2]."""
    bias = np.array([1, -2, 0.5], dtype=np.float32).tobytes()
    half = bytes([0x00, 0x3C, 0x00, 0xB8])
    bfloat = bytes([0x80, 0x3F, 0x00, 0xC0])
    tensors = [("bias", "F32", [3], bias), ("half", "F16", [2], half), ("bfloat", "BF16", [2], bfloat)]
    header = {"__metadata__": {"format": "test"}}
    off = 0
    for n, d, s, b in tensors:
        header[n] = {"dtype": d, "shape": s, "data_offsets": [off, off + len(b)]}
        off += len(b)
    hb = json.dumps(header).encode()
    return struct.pack("<II", len(hb), 0) + hb + b"".join(t[3] for t in tensors)


def test_reference_weights_format_file():
    f = gptq.parse_safetensors(_reference_test_file())
    gptq.expect_tensor(f, "bias", "F32", [3])
    gptq.expect_tensor(f, "half", "F16", [2])
    gptq.expect_tensor(f, "bfloat", "BF16", [2])
    assert gptq.read_tensor_f32(f, "bias").tolist() == [1.0, -2.0, 0.5]
    assert gptq.read_tensor_f32(f, "half").tolist() == [1.0, -0.5]
    assert gptq.read_tensor_f32(f, "bfloat").tolist() == [1.0, -2.0]
    assert bytes(gptq.read_tensor_bytes(f, "half")) == bytes([0x00, 0x3C, 0x00, 0xB8])


def test_parser_errors():
    good = _reference_test_file()
    with pytest.raises(ValueError, match="too short"):
        gptq.parse_safetensors(good[:7])
    with pytest.raises(ValueError, match="4 GiB"):
        gptq.parse_safetensors(good[:4] + struct.pack("<I", 1) + good[8:])
    with pytest.raises(ValueError, match="header length"):
        gptq.parse_safetensors(struct.pack("<II", 10 ** 6, 0) + good[8:])
    with pytest.raises(ValueError, match="JSON"):
        gptq.parse_safetensors(struct.pack("<II", 3, 0) + b"{x}")
    hb = json.dumps({"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 64]}}).encode()
    with pytest.raises(ValueError, match="out of range"):
        gptq.parse_safetensors(struct.pack("<II", len(hb), 0) + hb + bytes(16))
    hb = json.dumps({"t": {"dtype": "F32", "shape": [4], "data_offsets": [8, 4]}}).encode()
    with pytest.raises(ValueError, match="data_offsets"):
        gptq.parse_safetensors(struct.pack("<II", len(hb), 0) + hb + bytes(16))
    f = gptq.parse_safetensors(good)
    with pytest.raises(ValueError, match="missing tensor"):
        gptq.require_tensor(f, "nope")
    with pytest.raises(ValueError, match="dtype"):
        gptq.expect_tensor(f, "bias", "F16", [3])
    with pytest.raises(ValueError, match="shape"):
        gptq.expect_tensor(f, "bias", "F32", [4])
    with pytest.raises(ValueError):
        gptq.dtype_byte_size("F8")


def test_writer_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    a = rng.integers(0, 1 << 32, size=(4, 8), dtype=np.uint64).astype(np.uint32)
    s = rng.standard_normal((2, 8)).astype(np.float16)
    p = tmp_path / "m.safetensors"
    gptq.write_safetensors(str(p), {"w.qweight": ("I32", a.shape, a.tobytes()),
                                    "w.scales": ("F16", s.shape, s.tobytes())})
    f = gptq.open_safetensors(str(p))
    assert np.array_equal(np.frombuffer(gptq.read_tensor_bytes(f, "w.qweight"), np.uint32).reshape(4, 8), a)
    assert np.array_equal(gptq.read_tensor_f32(f, "w.scales").reshape(2, 8), s.astype(np.float32))


def test_qwen_config():
    c = gptq.QWEN25_05B
    assert gptq.qwen_head_dim(c) == 64 and gptq.qwen_kv_dim(c) == 128
    shapes = gptq.qwen_linear_shapes(c)
    assert shapes["kW"] == (896, 128) and shapes["downW"] == (4864, 896)
    with pytest.raises(ValueError):
        gptq.qwen_head_dim(gptq.QwenConfig(10, 8, 1, 3, 1, 8, 16))


def test_loader_format_probes(tmp_path):
    """qwen-format.ts:112-130 restated on synthetic checkpoints: g_idx must be the identity i/128
    (an act-order checkpoint is rejected, a missing g_idx accepted); stored-zero nibbles are
    counted per value; readF16Rows (qwen-loader.ts:70-93) decodes embed rows exactly."""
    from .checkpoint import TINY, write_checkpoint
    p = str(tmp_path / "model.safetensors")
    kept = write_checkpoint(p, TINY)
    f = gptq.open_safetensors(p)
    shapes = gptq.qwen_linear_shapes(TINY)
    for i in range(TINY.n_layer):
        for key, proj in gptq._PROJ:
            gptq.check_g_idx(f, f"model.layers.{i}.{proj}", shapes[key][0], 128)
    t, _ = kept[(0, "qW")]
    counts = gptq.stored_zero_counts(gptq.read_tensor_bytes(f, "model.layers.0.self_attn.q_proj.qzeros"),
                                     t.qzeros.shape[0], t.N)
    assert counts[7] == t.qzeros.shape[0] * t.N and counts.sum() == counts[7]
    t, _ = kept[(0, "kW")]                       # random stored zeros
    counts = gptq.stored_zero_counts(gptq.read_tensor_bytes(f, "model.layers.0.self_attn.k_proj.qzeros"),
                                     t.qzeros.shape[0], t.N)
    nib = [(int(w) >> (4 * (n % 8))) & 15 for g in range(t.qzeros.shape[0]) for n, w in
           ((n, t.qzeros[g, n // 8]) for n in range(t.N))]
    assert counts.tolist() == np.bincount(nib, minlength=16).tolist()
    rows = gptq.read_f16_rows(f, "model.embed_tokens.weight", 5, 3, TINY.n_embd)
    assert np.array_equal(rows, kept["embed"][5:8].astype(np.float32).reshape(-1))
    with pytest.raises(ValueError, match="outside"):
        gptq.read_f16_rows(f, "model.embed_tokens.weight", TINY.vocab_size - 1, 2, TINY.n_embd)
    p2 = str(tmp_path / "act_order.safetensors")
    write_checkpoint(p2, TINY, act_order=(1, "gateW"))
    f2 = gptq.open_safetensors(p2)
    gptq.check_g_idx(f2, "model.layers.1.mlp.up_proj", TINY.n_embd, 128)
    with pytest.raises(ValueError, match="not the identity"):
        gptq.check_g_idx(f2, "model.layers.1.mlp.gate_proj", TINY.n_embd, 128)
    p3 = str(tmp_path / "no_g_idx.safetensors")
    write_checkpoint(p3, TINY, no_g_idx=True)
    gptq.check_g_idx(gptq.open_safetensors(p3), "model.layers.0.mlp.gate_proj", TINY.n_embd, 128)


def test_url_to_path():
    assert gptq.url_to_path("file:///tmp/a%20b/model.safetensors") == "/tmp/a b/model.safetensors"
    assert gptq.url_to_path("models/x/model.safetensors") == "models/x/model.safetensors"
    assert gptq.url_to_path("/abs/model.safetensors") == "/abs/model.safetensors"
    with pytest.raises(ValueError, match="local path"):
        gptq.url_to_path("https://huggingface.co/x/model.safetensors")
