"""Host-side mirror of the reference's GPTQ loader and linear dispatch, over libqlinear.

Same names, argument meaning and error behaviour as the reference's TypeScript surface
(paths relative to the intplusplus/webllm checkout), with the int4 work moved to the GPU:

  parse_safetensors / require_tensor /      src/weights/safetensors.ts:84-124, :155-161, :201-222
  expect_tensor / read_tensor_bytes /
  dtype_byte_size / f16_bits_to_f32
  dequantize_gptq_int4                      src/weights/quant.ts:42-118 (exact, on the GPU)
  QuantLinearModel.upload_gptq_linear       src/model/qwen.ts:246-293 uploadLayer / uploadF16, but
                                            the packed tensors are uploaded as they are
  QuantLinearModel.gemm                     src/model/qwen.ts:568-618 QwenGpt.gemm
  load_qwen_weights                         src/weights/qwen-loader.ts:102-177 loadQwenWeights
  read_f16_rows                             src/weights/qwen-loader.ts:70-93 readF16Rows
  check_g_idx / stored_zero_counts          src/tests/qwen/qwen-format.ts:112-130 (format probes)
  QwenConfig / QWEN25_05B / qwen_kv_dim     src/model/qwen-config.ts:1-54

Tensors are slices of device arenas (`Tensor{arena, offset, length, shape}`, buffer.ts:12-18);
errors are raised as ValueError (reference: `throw new Error(msg)`) or qlinear.QlError.
"""
from __future__ import annotations

import json
import mmap
import os
import struct
from dataclasses import dataclass, field

import numpy as np

from . import qlinear as ql

# ------------------------------------------------------------------ config (qwen-config.ts)


@dataclass(frozen=True)
class QwenConfig:
    vocab_size: int
    block_size: int
    n_layer: int
    n_head: int
    n_kv_head: int
    n_embd: int
    intermediate: int
    rms_eps: float = 1e-6
    rope_theta: float = 1000000.0


QWEN25_05B = QwenConfig(vocab_size=151936, block_size=128, n_layer=24, n_head=14, n_kv_head=2,
                        n_embd=896, intermediate=4864)


def qwen_head_dim(c: QwenConfig) -> int:
    if c.n_embd % c.n_head:
        raise ValueError(f"nEmbd({c.n_embd}) must be divisible by nHead({c.n_head})")
    return c.n_embd // c.n_head


def qwen_kv_dim(c: QwenConfig) -> int:
    return qwen_head_dim(c) * c.n_kv_head


# ------------------------------------------------------------------ safetensors (safetensors.ts)

_DTYPE_SIZE = {"F64": 8, "I64": 8, "F32": 4, "I32": 4, "F16": 2, "BF16": 2, "I16": 2, "I8": 1,
               "U8": 1, "BOOL": 1}


def dtype_byte_size(dtype: str) -> int:
    if dtype not in _DTYPE_SIZE:
        raise ValueError(f"unknown safetensors dtype: {dtype}")
    return _DTYPE_SIZE[dtype]


@dataclass
class SafetensorEntry:
    dtype: str
    shape: list
    data_offsets: tuple


@dataclass
class SafetensorFile:
    buffer: memoryview          # the whole file (memory-mapped when loaded from a path)
    data_start: int
    header: dict = field(default_factory=dict)


def parse_safetensors_header(header_bytes: bytes) -> dict:
    try:
        parsed = json.loads(bytes(header_bytes).decode("utf-8"))
    except Exception as e:  # noqa: BLE001 - message mirrors the reference's
        raise ValueError(f"safetensors: header JSON parse failed: {e}") from None
    if not isinstance(parsed, dict):
        raise ValueError("safetensors: header is not a JSON object")
    header = {}
    for name, raw in parsed.items():
        if name == "__metadata__":
            continue
        if not isinstance(raw, dict):
            raise ValueError(f"safetensors: {name} entry is invalid")
        if not isinstance(raw.get("dtype"), str):
            raise ValueError(f"safetensors: {name} has no dtype")
        if not isinstance(raw.get("shape"), list):
            raise ValueError(f"safetensors: {name} has no shape")
        offs = raw.get("data_offsets")
        if not isinstance(offs, list) or len(offs) != 2:
            raise ValueError(f"safetensors: {name} data_offsets invalid")
        start, end = (float(v) for v in offs)
        if not (np.isfinite(start) and np.isfinite(end)) or start < 0 or end < start:
            raise ValueError(f"safetensors: {name} data_offsets values invalid")
        header[name] = SafetensorEntry(raw["dtype"], [int(v) for v in raw["shape"]],
                                       (int(start), int(end)))
    return header


def parse_safetensors(buffer) -> SafetensorFile:
    """safetensors.ts:84-110: u64 LE header length (upper 4 bytes must be 0), JSON header, data."""
    buf = memoryview(buffer).cast("B")
    if buf.nbytes < 8:
        raise ValueError("safetensors: buffer too short")
    header_len, upper = struct.unpack_from("<II", buf, 0)
    if upper != 0:
        raise ValueError("safetensors: header length above 4 GiB is not supported")
    data_start = 8 + header_len
    if header_len <= 0 or data_start > buf.nbytes:
        raise ValueError(f"safetensors: invalid header length headerLen={header_len} "
                         f"bufferSize={buf.nbytes}")
    header = parse_safetensors_header(buf[8:data_start])
    for name, e in header.items():
        if data_start + e.data_offsets[1] > buf.nbytes:
            raise ValueError(f"safetensors: {name} data out of range end={e.data_offsets[1]}")
    return SafetensorFile(buf, data_start, header)


def tensor_count(e: SafetensorEntry) -> int:
    n = 1
    for d in e.shape:
        n *= d
    return n


def require_tensor(f: SafetensorFile, name: str) -> SafetensorEntry:
    e = f.header.get(name)
    if e is None:
        raise ValueError(f"safetensors: missing tensor {name}")
    return e


def expect_tensor(f: SafetensorFile, name: str, dtype: str, shape) -> SafetensorEntry:
    e = require_tensor(f, name)
    if e.dtype != dtype:
        raise ValueError(f"safetensors: {name} dtype={e.dtype}, expected {dtype}")
    if list(e.shape) != list(shape):
        raise ValueError(f"safetensors: {name} shape={e.shape}, expected {list(shape)}")
    return e


def read_tensor_bytes(f: SafetensorFile, name: str) -> memoryview:
    """The tensor's raw bytes (a view, not a copy: uploads read straight from the mapping)."""
    e = require_tensor(f, name)
    start = f.data_start + e.data_offsets[0]
    return f.buffer[start:start + tensor_count(e) * dtype_byte_size(e.dtype)]


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """safetensors.ts:144-152: exact binary16 decode (every f16 value is an f32 value)."""
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def read_tensor_f32(f: SafetensorFile, name: str) -> np.ndarray:
    """safetensors.ts:164-198 for F32/F16/BF16/U8/I8."""
    e = require_tensor(f, name)
    raw = np.frombuffer(read_tensor_bytes(f, name), dtype=np.uint8)
    if e.dtype == "F32":
        return raw.view("<f4").astype(np.float32)
    if e.dtype == "F16":
        return f16_bits_to_f32(raw.view("<u2"))
    if e.dtype == "BF16":
        return (raw.view("<u2").astype(np.uint32) << 16).view(np.float32)
    if e.dtype == "U8":
        return raw.astype(np.float32)
    if e.dtype == "I8":
        return raw.view(np.int8).astype(np.float32)
    raise ValueError(f"readTensorF32: unsupported dtype {e.dtype} ({name})")


# ------------------------------------------------------------------ tensors and the model


@dataclass
class Tensor:
    """A slice of a device arena (buffer.ts:12-18: buffer, offset, length, shape)."""
    arena: ql.Arena
    offset: int
    length: int                  # elements
    shape: tuple
    dtype: str = "f32"
    pool: "ActivationArena | None" = None

    def read(self) -> np.ndarray:
        dt = {"f32": np.float32, "f16": np.float16, "u8": np.uint8, "u32": np.uint32}[self.dtype]
        return self.arena.read(self.offset, self.shape, dt)

    def write(self, data: np.ndarray):
        self.arena.write(self.offset, np.ascontiguousarray(data))


class ActivationArena:
    """Bump allocator of tensors inside one device arena; reset() per forward (arena.ts:35-59)."""

    def __init__(self, ctx: ql.Context, nbytes: int):
        self.arena = ctx.arena(nbytes)
        self.layout = ql.ArenaLayout()

    def alloc(self, shape, dtype: str = "f32") -> Tensor:
        n = int(np.prod(shape))
        size = n * {"f16": 2, "u8": 1}.get(dtype, 4)
        off = self.layout.take(size)
        if self.layout.used > self.arena.size:
            raise ValueError(f"activation arena exhausted ({self.layout.used} > {self.arena.size})")
        return Tensor(self.arena, off, n, tuple(shape), dtype, self)

    def scratch_offset(self, nbytes: int) -> int:
        """Split-K scratch at the tail of the arena, clear of every live tensor (the reference
        takes the partial-sum buffer from its activation arena too, qwen.ts:583)."""
        if nbytes == 0:
            return 0
        off = (self.arena.size - nbytes) // 256 * 256
        if off < self.layout.used:
            raise ValueError(f"activation arena too small for {nbytes} bytes of split-K scratch")
        return off

    def reset(self):
        self.layout = ql.ArenaLayout()


class KvCache:
    """Per-layer fp32 K and V caches [block_size, n_kv_head * D] in one device arena, and the
    decode attention over them: QwenGpt's kCache/vCache (qwen.ts:140-141, :200-205), kv store
    (qwen.ts:427-428) and attention_gqa_cache dispatch (qwen.ts:429-440). Stream order replaces
    the reference's pass breaks. The caller keeps the context length (the reference's cacheLen,
    qwen.ts:142, :490) and passes it as pos0 / past_len."""

    def __init__(self, ctx: ql.Context, config: QwenConfig):
        self.ctx = ctx
        self.config = config
        self.D = qwen_head_dim(config)
        self.row_len = qwen_kv_dim(config)
        self.region = -(-config.block_size * self.row_len * 4 // 256) * 256
        self.arena = ctx.arena(2 * config.n_layer * self.region)

    def offsets(self, layer: int):
        if not 0 <= layer < self.config.n_layer:
            raise ValueError(f"layer {layer} out of range")
        base = 2 * layer * self.region
        return base, base + self.region

    def store(self, layer: int, k: Tensor, v: Tensor, rows: int, pos0: int):
        """cache[pos0 + r] = k[r] / v[r] for r < rows (after RoPE on k, as the reference)."""
        if k.length < rows * self.row_len or v.length < rows * self.row_len:
            raise ValueError("kv store: k/v tensors smaller than [rows, n_kv_head * D]")
        ko, vo = self.offsets(layer)
        for t, off in ((k, ko), (v, vo)):
            self.ctx.kv_store(t.arena, t.offset, self.arena, off, self.config.block_size, rows,
                              self.row_len, pos0)

    def attend(self, layer: int, q: Tensor, out: Tensor, M: int, past_len: int):
        """out [M, n_head * D] = causal GQA attention of q's M rows at positions past_len + m."""
        c = self.config
        if q.length < M * c.n_head * self.D or out.length < M * c.n_head * self.D:
            raise ValueError("attention: q/out smaller than [M, n_head * D]")
        if q.arena is not out.arena:
            raise ValueError("attention: q and out must live in the same activation arena")
        ko, vo = self.offsets(layer)
        self.ctx.attention_decode(q.arena, q.offset, self.arena, ko, vo, c.block_size, M, c.n_head,
                                  c.n_kv_head, self.D, past_len, out.offset)

    def release(self):
        self.arena.release()


@dataclass
class _Linear:
    desc: ql.GptqDesc
    K: int
    N: int


class QuantLinearModel:
    """Weight side of QwenGpt with GPTQ weights kept packed in one device arena.

    Weights are addressed by name ("L{i}.qW" ...), as in the reference (qwen.ts:134, :633-638)."""

    def __init__(self, ctx: ql.Context, weight_capacity: int, scratch_capacity: int = 64 << 20):
        self.ctx = ctx
        self.weights = ctx.arena(weight_capacity)
        self.layout = ql.ArenaLayout()
        self.linears: dict[str, _Linear] = {}
        self.f32: dict[str, Tensor] = {}
        self.f16: dict[str, Tensor] = {}
        self.scratch = ctx.arena(scratch_capacity)

    @property
    def weight_bytes(self) -> int:
        return self.layout.used

    def _place(self, data) -> int:
        buf = np.frombuffer(data, dtype=np.uint8) if not isinstance(data, np.ndarray) else \
            np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        off = self.layout.take(buf.nbytes)
        if self.layout.used > self.weights.size:
            raise ValueError(f"weight arena exhausted ({self.layout.used} > {self.weights.size})")
        self.weights.write(off, buf)
        return off

    def upload_gptq_linear(self, name: str, qweight, qzeros, scales_f16, in_features: int,
                           out_features: int, group_size: int = 128, bias=None):
        """One GPTQ int4 linear, packed: qweight I32 [in/8, out], qzeros I32 [in/g, out/8] or
        None (zero 8), scales F16 [in/g, out] (raw bytes), bias F32 [out] or None."""
        if name in self.linears:
            raise ValueError(f"weight already exists: {name}")
        qw = self._place(qweight)
        qz = None if qzeros is None else self._place(qzeros)
        sc = self._place(scales_f16)
        b = None if bias is None else self._place(np.ascontiguousarray(bias, dtype=np.float32))
        desc = ql.make_desc(qw, qz, sc, in_features, out_features, group_size, b)
        self.ctx.check(desc, self.weights)      # quant.ts:44-79 validation, on the arena
        self.linears[name] = _Linear(desc, in_features, out_features)

    def upload_f32(self, name: str, data):
        if name in self.f32:
            raise ValueError(f"weight already exists: {name}")
        data = np.ascontiguousarray(data, dtype=np.float32)
        off = self._place(data)
        self.f32[name] = Tensor(self.weights, off, data.size, data.shape, "f32")

    def upload_f16_bits(self, name: str, bits, shape):
        if name in self.f16:
            raise ValueError(f"weight already exists: {name}")
        off = self._place(bits)
        self.f16[name] = Tensor(self.weights, off, int(np.prod(shape)), tuple(shape), "f16")

    def release(self):
        """Frees the weight arena (the reference's QwenGpt.destroy of its weight buffers)."""
        self.weights.release()

    def linear(self, name: str) -> _Linear:
        lin = self.linears.get(name)
        if lin is None:
            raise ValueError(f"missing int4 weight: {name}")
        return lin

    def gemm(self, A: Tensor, weight: str, C: Tensor, bias: str | None, M: int, N: int, K: int):
        """C[M,N] = A[M,K] @ W^T (+ bias) — qwen.ts:568-618. A is f32 (decode) or f16; C is f32.
        The bias is the linear's own (upload_gptq_linear(bias=...)); passing another name raises,
        as a missing weight does in the reference (qwen.ts:640-645)."""
        if weight in self.f16 and weight not in self.linears:
            return self._gemm_f16(A, weight, C, bias, M, N, K)
        lin = self.linear(weight)
        if (lin.K, lin.N) != (K, N):
            raise ValueError(f"gemm: {weight} is [{lin.N},{lin.K}], called with N={N} K={K}")
        if bias is not None and lin.desc.bias_off == ql.QL_NONE:
            raise ValueError(f"missing f32 weight: {bias}")
        desc = lin.desc
        if bias is None and desc.bias_off != ql.QL_NONE:
            desc = ql.make_desc(desc.qweight_off, None if desc.qzeros_off == ql.QL_NONE else
                                desc.qzeros_off, desc.scales_off, K, N, desc.group)
        if A.arena is not C.arena:
            raise ValueError("gemm: A and C must live in the same activation arena")
        if A.length < M * K or C.length < M * N:
            raise ValueError("gemm: tensor too small for [M,K] / [M,N]")
        if A.pool is None or A.pool is not C.pool:
            raise ValueError("gemm: A and C must come from one ActivationArena")
        plan = ql.plan_linear(M, N, K, desc.group)
        scratch = A.pool.scratch_offset(plan.scratch_bytes)
        self.ctx.linear(desc, self.weights, A.arena, A.offset,
                        ql.DTYPE_F32 if A.dtype == "f32" else ql.DTYPE_F16, M, C.offset, scratch)

    def embed(self, tokens: Tensor, out: Tensor, M: int, weight: str = "embed"):
        """out[M, C] = the fp16 table's rows tokens[0..M) as f32: the forward's first dispatch
        (embedding_f16.wgsl, qwen.ts:391-392). Token ids >= vocab give zero rows."""
        w = self.f16.get(weight)
        if w is None:
            raise ValueError(f"missing f16 weight: {weight}")
        vocab, C = w.shape
        if tokens.dtype != "u32" or tokens.length < M:
            raise ValueError("embed: tokens must be a u32 tensor of at least M ids")
        if out.dtype != "f32" or out.length < M * C or out.arena is not tokens.arena:
            raise ValueError("embed: out must be an f32 [M, C] tensor in the tokens' arena")
        self.ctx.embed_f16(self.weights, w.offset, vocab, C, tokens.arena, tokens.offset, M, out.offset)

    def rmsnorm(self, x: Tensor, weight: str, y: Tensor, M: int, C: int, eps: float,
                residual: Tensor | None = None, sum_out: Tensor | None = None):
        """y = rmsnorm(x (+ residual)) * weight (rmsnorm.wgsl, qwen.ts:403-404, :456-457); with
        `residual` the add of vec_add.wgsl (qwen.ts:475-476) runs in the same launch and the sum
        goes to `sum_out` (the next residual stream) when given."""
        w = self.f32.get(weight)
        if w is None:
            raise ValueError(f"missing f32 weight: {weight}")
        if w.length != C:
            raise ValueError(f"rmsnorm: {weight} has {w.length} values, C={C}")
        ts = [t for t in (x, y, residual, sum_out) if t is not None]
        if any(t.arena is not x.arena for t in ts) or any(t.length < M * C for t in ts):
            raise ValueError("rmsnorm: tensors must be [M, C] in one activation arena")
        self.ctx.add_rmsnorm(x.arena, x.offset, None if residual is None else residual.offset, self.weights,
                             w.offset, eps, M, C, y.offset, None if sum_out is None else sum_out.offset)

    def silu_mul(self, gate: Tensor, up: Tensor, out: Tensor, n: int):
        """out = silu(gate) * up (silu_mul.wgsl, qwen.ts:468-469)."""
        ts = (gate, up, out)
        if any(t.arena is not gate.arena for t in ts) or any(t.length < n for t in ts):
            raise ValueError("silu_mul: tensors must hold n values in one activation arena")
        self.ctx.silu_mul(gate.arena, gate.offset, up.offset, n, out.offset)

    def _gemm_f16(self, A: Tensor, weight: str, C: Tensor, bias: str | None, M: int, N: int, K: int):
        """C[M,N] = A[M,K] @ W^T (+ bias) over an fp16 weight [N,K] (the tied lm_head `embed`,
        qwen.ts:488-489 with gemm_gemv_f16.wgsl semantics): f32 A and C, fp32 accumulation."""
        w = self.f16[weight]
        if w.shape != (N, K):
            raise ValueError(f"gemm: {weight} is {list(w.shape)}, called with N={N} K={K}")
        b = None
        if bias is not None:
            t = self.f32.get(bias)
            if t is None:
                raise ValueError(f"missing f32 weight: {bias}")
            if t.length != N:
                raise ValueError(f"gemm: bias {bias} has {t.length} values, N={N}")
            b = t.offset
        if A.dtype != "f32" or C.dtype != "f32":
            raise ValueError("gemm over fp16 weights takes f32 A and C")
        if A.arena is not C.arena:
            raise ValueError("gemm: A and C must live in the same activation arena")
        if A.length < M * K or C.length < M * N:
            raise ValueError("gemm: tensor too small for [M,K] / [M,N]")
        self.ctx.gemv_f16w(self.weights, w.offset, b, A.arena, A.offset, M, N, K, C.offset)

    def gemm_batch(self, A: Tensor, weights: list, Cs: list, M: int):
        """Several linears on one input in one launch (q/k/v, gate/up; qwen.ts:411-413, :464-465)."""
        lins = [self.linear(w) for w in weights]
        descs = [l.desc for l in lins]
        if A.pool is None or any(c.pool is not A.pool for c in Cs):
            raise ValueError("gemm_batch: A and every C must come from one ActivationArena")
        scratch = A.pool.scratch_offset(ql.plan_batch(descs, M))
        self.ctx.linear_batch(descs, self.weights, A.arena, [A.offset] * len(lins),
                              ql.DTYPE_F32 if A.dtype == "f32" else ql.DTYPE_F16, M,
                              [c.offset for c in Cs], scratch)

    def unpack_f16(self, name: str, out: Tensor):
        """fp16 [N,K] copy of an int4 weight, bit-identical to the reference's uploaded buffer."""
        lin = self.linear(name)
        if out.length < lin.N * lin.K or out.dtype != "f16":
            raise ValueError("unpack_f16: output must be an f16 tensor of N*K elements")
        self.ctx.unpack_f16(lin.desc, self.weights, out.arena, out.offset)

    def dequantize(self, name: str) -> np.ndarray:
        """fp32 [N,K] = dequantizeGptqInt4 of the stored tensors (computed on the GPU)."""
        lin = self.linear(name)
        tmp = self.ctx.arena(lin.N * lin.K * 4)
        try:
            self.ctx.unpack_f32(lin.desc, self.weights, tmp, 0)
            return tmp.read(0, (lin.N, lin.K), np.float32)
        finally:
            tmp.release()


def dequantize_gptq_int4(ctx: ql.Context, qweight, qzeros, scales, in_features: int,
                         out_features: int, group_size: int = 128, bits: int = 4) -> np.ndarray:
    """quant.ts:42-118 with the same inputs (raw I32 bytes, any f32 scales — GptqInt4Params.scales
    is a Float32Array, quant.ts:22-23) and the same output (fp32 [out, in]), computed on the GPU
    (ql_unpack_f32_ex with f32 scales: bit-identical for every f32 scale)."""
    sc = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
    qw = np.frombuffer(bytes(qweight), dtype=np.uint8)
    qz = None if qzeros is None else np.frombuffer(bytes(qzeros), dtype=np.uint8)
    # quant.ts:46-79 order: bits, group, dims, qweight bytes, scales count, qzeros bytes, group % 8
    shape_rc = ql.validate(ql.make_desc(0, None, 0, in_features, out_features, group_size, None,
                                        bits), 1 << 62)
    if shape_rc in (-1, -2, -3):
        raise ql.QlError(shape_rc, ql.lib().ql_last_error().decode())
    need_qw, need_qz, need_sc = ql.gptq_sizes(in_features, out_features, group_size)
    if qw.nbytes < need_qw:
        raise ql.QlError(-4, f"GPTQ: qweight needs {need_qw} bytes, got {qw.nbytes}")
    if sc.size < need_sc // 2:
        raise ql.QlError(-5, f"GPTQ: scales need {need_sc // 2} values, got {sc.size}")
    if qz is not None and qz.nbytes < need_qz:
        raise ql.QlError(-6, f"GPTQ: qzeros need {need_qz} bytes, got {qz.nbytes}")
    if shape_rc == -7:
        raise ql.QlError(-7, f"GPTQ: group size {group_size} must be a multiple of 8")
    lay = ql.ArenaLayout()
    o_qw = lay.take(need_qw)
    o_qz = None if qz is None else lay.take(need_qz)
    o_sc = lay.take(2 * need_sc)                  # f32 scales
    desc = ql.make_desc(o_qw, o_qz, o_sc, in_features, out_features, group_size, None, bits)
    w = ctx.arena(lay.used + 256)
    out = ctx.arena(max(in_features * out_features * 4, 16))
    try:
        w.write(o_qw, qw[:need_qw])
        if qz is not None:
            w.write(o_qz, qz[:need_qz])
        w.write(o_sc, sc[:need_sc // 2])
        ctx.unpack_f32(desc, w, out, 0, ql.DTYPE_F32)
        return out.read(0, (out_features, in_features), np.float32)
    finally:
        w.release()
        out.release()


# ------------------------------------------------------------------ loader (qwen-loader.ts)

_PROJ = [("qW", "self_attn.q_proj"), ("kW", "self_attn.k_proj"), ("vW", "self_attn.v_proj"),
         ("oW", "self_attn.o_proj"), ("gateW", "mlp.gate_proj"), ("upW", "mlp.up_proj"),
         ("downW", "mlp.down_proj")]
_BIASED = {"qW", "kW", "vW"}


QWEN_LOCAL_DIR = "models/qwen2.5-0.5b-int4/"     # qwen-loader.ts:27 (public/models layout)


@dataclass
class QwenLoadResult:
    gpu_bytes: int
    tensor_count: int
    file_bytes: int
    layer: dict | None = None
    embed_rows: np.ndarray | None = None      # keep_embed_rows: fp32 [rows * C]
    # stored qzeros nibbles over every GPTQ linear: {nibble: count}; {7: n} for the symmetric
    # 4-bit checkpoints tests/qwen/qwen-format.ts:112-123 expects (zero 8 stored as 7)
    stored_zeros: dict = field(default_factory=dict)


def url_to_path(url: str) -> str:
    """A local file path or a file:// URL (the reference fetches `url`, qwen-loader.ts:113-115;
    this host reads local files only: there is no network)."""
    from urllib.parse import unquote, urlparse
    u = urlparse(url)
    if u.scheme == "file":
        return unquote(u.path)
    if u.scheme in ("", ) or (len(u.scheme) == 1 and url[1:3] in (":\\", ":/")):
        return url
    raise ValueError(f"qwen-loader: cannot load {url}: only a local path or a file:// URL")


def read_f16_rows(f: SafetensorFile, name: str, row_start: int, row_count: int,
                  row_length: int) -> np.ndarray:
    """readF16Rows (qwen-loader.ts:70-93): rows [row_start, row_start + row_count) of a 2-D F16
    tensor, decoded to fp32 (flat)."""
    e = require_tensor(f, name)
    if e.dtype != "F16":
        raise ValueError(f"qwen-loader: {name} expected F16, got {e.dtype}")
    if len(e.shape) != 2 or e.shape[0] * row_length != e.shape[0] * e.shape[1]:
        raise ValueError(f"qwen-loader: {name} shape {e.shape} does not match rowLength={row_length}")
    if row_start < 0 or row_count < 0 or row_start + row_count > e.shape[0]:
        raise ValueError(f"qwen-loader: rows [{row_start}, {row_start + row_count}) outside {name} "
                         f"[{e.shape[0]}, {e.shape[1]}]")
    start = f.data_start + e.data_offsets[0] + row_start * row_length * 2
    raw = np.frombuffer(f.buffer[start:start + row_count * row_length * 2], dtype="<u2")
    return f16_bits_to_f32(raw)


def check_g_idx(f: SafetensorFile, prefix: str, in_features: int, group_size: int):
    """desc_act=false: g_idx, when present, must be the identity map i // group
    (tests/qwen/qwen-format.ts:125-130); the fused kernels assume it, so any other order
    (an act-order checkpoint) is rejected instead of loaded wrong."""
    name = f"{prefix}.g_idx"
    if name not in f.header:
        return
    e = expect_tensor(f, name, "I32", [in_features])
    g = np.frombuffer(read_tensor_bytes(f, name), dtype="<i4")
    want = np.arange(in_features, dtype=np.int64) // group_size
    bad = np.nonzero(g != want)[0]
    if bad.size:
        i = int(bad[0])
        raise ValueError(f"qwen-loader: {name}[{i}] = {int(g[i])} is not the identity map i/{group_size} "
                         f"(desc_act checkpoints are not supported)")
    del e


def stored_zero_counts(qzeros, groups: int, out_features: int) -> np.ndarray:
    """Counts of each stored qzeros nibble (0..15) over the real columns of a linear
    (qwen-format.ts:112-123 collects the same set)."""
    nc = (out_features + 7) // 8
    w = np.frombuffer(qzeros, dtype="<u4")[:groups * nc].reshape(groups, nc)
    nib = (w[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
    return np.bincount(nib.reshape(groups, nc * 8)[:, :out_features].reshape(-1), minlength=16)


def qwen_linear_shapes(c: QwenConfig) -> dict:
    C, HI, I = c.n_embd, qwen_kv_dim(c), c.intermediate
    return {"qW": (C, C), "kW": (C, HI), "vW": (C, HI), "oW": (C, C), "gateW": (C, I),
            "upW": (C, I), "downW": (I, C)}


def open_safetensors(path: str) -> SafetensorFile:
    fh = open(path, "rb")
    mm = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
    fh.close()
    return parse_safetensors(mm)


def load_qwen_weights(model: QuantLinearModel, path: str | None = None, config: QwenConfig = QWEN25_05B,
                      on_progress=None, keep_layer: int | None = None,
                      group_size: int = 128, url: str | None = None,
                      keep_embed_rows: tuple | dict | None = None) -> QwenLoadResult:
    """loadQwenWeights (qwen-loader.ts:102-177): embed (F16, tied lm_head), final norm, then per
    layer the 7 GPTQ linears, q/k/v biases and the two norms. The int4 tensors go to the GPU
    packed — no CPU dequant — after the shape checks the reference's format probe makes
    (tests/qwen/qwen-format.ts:72-80) and its g_idx identity check (:125-130); the stored-zero
    nibbles are counted into the result (:112-123).

    The file is `url` (a path or file:// URL, default QWEN_LOCAL_DIR + "model.safetensors", as
    qwen-loader.ts:113) or `path`, memory-mapped. keep_layer returns that layer's fp32 weights;
    keep_embed_rows = (start, rows) or {"start", "rows"} returns those embed rows in fp32
    (qwen-loader.ts:134-135)."""
    if path is None:
        path = url_to_path(url if url is not None else QWEN_LOCAL_DIR + "model.safetensors")
    f = open_safetensors(path)
    count = 0
    C = config.n_embd
    emb = require_tensor(f, "model.embed_tokens.weight")
    if emb.shape != [config.vocab_size, C]:
        raise ValueError(f"qwen-loader: embed_tokens shape {emb.shape}, expected "
                         f"[{config.vocab_size},{C}]")
    if emb.dtype != "F16":
        raise ValueError(f"qwen-loader: model.embed_tokens.weight expected F16, got {emb.dtype}")
    model.upload_f16_bits("embed", read_tensor_bytes(f, "model.embed_tokens.weight"),
                          (config.vocab_size, C))
    count += 1
    embed_rows = None
    if keep_embed_rows is not None:
        start, rows = ((keep_embed_rows["start"], keep_embed_rows["rows"])
                       if isinstance(keep_embed_rows, dict) else keep_embed_rows)
        embed_rows = read_f16_rows(f, "model.embed_tokens.weight", start, rows, C)
    model.upload_f32("finalNorm", read_tensor_f32(f, "model.norm.weight"))
    count += 1
    shapes = qwen_linear_shapes(config)
    kept = None
    zeros = np.zeros(16, dtype=np.int64)
    for i in range(config.n_layer):
        p = f"model.layers.{i}"
        model.upload_f32(f"L{i}.inNorm", read_tensor_f32(f, f"{p}.input_layernorm.weight"))
        model.upload_f32(f"L{i}.postNorm", read_tensor_f32(f, f"{p}.post_attention_layernorm.weight"))
        count += 2
        layer = {}
        for key, proj in _PROJ:
            K, N = shapes[key]
            pre = f"{p}.{proj}"
            P, G, NC = (K + 7) // 8, (K + group_size - 1) // group_size, (N + 7) // 8
            expect_tensor(f, f"{pre}.qweight", "I32", [P, N])
            expect_tensor(f, f"{pre}.qzeros", "I32", [G, NC])
            expect_tensor(f, f"{pre}.scales", "F16", [G, N])
            check_g_idx(f, pre, K, group_size)
            zeros += stored_zero_counts(read_tensor_bytes(f, f"{pre}.qzeros"), G, N)
            bias = read_tensor_f32(f, f"{pre}.bias") if key in _BIASED else None
            model.upload_gptq_linear(f"L{i}.{key}", read_tensor_bytes(f, f"{pre}.qweight"),
                                     read_tensor_bytes(f, f"{pre}.qzeros"),
                                     read_tensor_bytes(f, f"{pre}.scales"), K, N, group_size, bias)
            count += 1 + (1 if bias is not None else 0)
            if keep_layer == i:
                layer[key] = model.dequantize(f"L{i}.{key}")
        if keep_layer == i:
            kept = layer
        if on_progress:
            on_progress(i + 1, config.n_layer, f"layer {i + 1}/{config.n_layer}")
    return QwenLoadResult(model.weight_bytes, count, f.buffer.nbytes, kept, embed_rows,
                          {int(v): int(c) for v, c in enumerate(zeros) if c})


def write_safetensors(path: str, tensors: dict, metadata: dict | None = None):
    """Minimal writer (the reference's test builder, tests/qwen/weights.ts:7-41): name ->
    (dtype, shape, bytes). Used to produce synthetic checkpoints offline."""
    header = {"__metadata__": metadata or {"format": "pt"}}
    off = 0
    for name, (dtype, shape, data) in tensors.items():
        n = len(data)
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + n]}
        off += n
    hb = json.dumps(header).encode()
    with open(path, "wb") as fh:
        fh.write(struct.pack("<Q", len(hb)))
        fh.write(hb)
        for _, (_, _, data) in tensors.items():
            fh.write(bytes(data))
    return os.path.getsize(path)
