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
