"""ctypes binding of libqlinear.so (include/qlinear.h).

Thin, typed wrapper: contexts, arenas, GPTQ descriptors, plans, linears, timers and graphs.
Status codes become `QlError` exceptions carrying the library's message, the way the reference
throws `Error(msg)` on bad shapes (src/weights/quant.ts:46-79). There is no fallback: if the
shared library is missing, importing this module raises.
"""
from __future__ import annotations

import ctypes
import os
import re
import weakref
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libqlinear.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "qlinear.h")

SEQ_TILES, SEQ_STRIPS, SEQ_PREFILL, SEQ_STRIP_PASSES, SEQ_PREFILL_PASSES = 0, 1, 2, 3, 4   # ql_seq_info.kernel
QL_NONE = (1 << 64) - 1
NOALLOC_SCRATCH_BYTES = 8 << 20   # QL_NOALLOC_SCRATCH_BYTES
DTYPE_F32 = 0
DTYPE_F16 = 1
KIND_NAMES = {1: "gemv_mfma", 2: "gemv_simple", 3: "gemm_mfma", 4: "gemm_simple"}

ERROR_NAMES = {
    -1: "QL_E_BITS", -2: "QL_E_GROUP", -3: "QL_E_DIMS", -4: "QL_E_QWEIGHT_SHORT",
    -5: "QL_E_SCALES_SHORT", -6: "QL_E_QZEROS_SHORT", -7: "QL_E_GROUP_PACK",
    -10: "QL_E_INVALID", -11: "QL_E_RANGE", -12: "QL_E_ALIGN", -13: "QL_E_HIP",
    -14: "QL_E_STATE",
}


class QlError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {message}")
        self.code = code
        self.name = ERROR_NAMES.get(code, str(code))


class GptqDesc(ctypes.Structure):
    _fields_ = [("qweight_off", ctypes.c_uint64), ("qzeros_off", ctypes.c_uint64),
                ("scales_off", ctypes.c_uint64), ("bias_off", ctypes.c_uint64),
                ("K", ctypes.c_int32), ("N", ctypes.c_int32), ("group", ctypes.c_int32),
                ("bits", ctypes.c_int32)]


class SeqFuse(ctypes.Structure):
    """Elementwise work folded into one linear of a fused sequence (ql_seq_fuse): RMSNorm of x
    (norm weight in the weights arena), silu(x) * x2, and a residual added to y; offsets of
    another linear's output make that linear a producer."""
    _fields_ = [("norm_w_off", ctypes.c_uint64), ("x2_off", ctypes.c_uint64),
                ("res_off", ctypes.c_uint64), ("norm_eps", ctypes.c_float),
                ("reserved", ctypes.c_int32)]


def make_fuse(norm_w_off: int | None = None, norm_eps: float = 1e-6, x2_off: int | None = None,
              res_off: int | None = None) -> SeqFuse:
    return SeqFuse(QL_NONE if norm_w_off is None else norm_w_off, QL_NONE if x2_off is None else x2_off,
                   QL_NONE if res_off is None else res_off, norm_eps, 0)


class Plan(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("split", ctypes.c_int32), ("waves", ctypes.c_int32),
                ("grid_x", ctypes.c_int32), ("grid_y", ctypes.c_int32), ("block", ctypes.c_int32),
                ("scratch_bytes", ctypes.c_uint64), ("ref_split", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]

    @property
    def kind_name(self) -> str:
        return KIND_NAMES.get(self.kind, "?")


class SeqInfo(ctypes.Structure):
    _fields_ = [("linears", ctypes.c_int32), ("passes", ctypes.c_int32), ("tiles", ctypes.c_int32),
                ("reduces", ctypes.c_int32), ("grid", ctypes.c_int32), ("max_split", ctypes.c_int32),
                ("lds_bytes", ctypes.c_uint64), ("device_bytes", ctypes.c_uint64),
                ("total_units", ctypes.c_uint64), ("busiest_units", ctypes.c_uint64),
                ("kernel", ctypes.c_int32), ("split", ctypes.c_int32), ("stream", ctypes.c_int32),
                ("variant", ctypes.c_int32), ("launches", ctypes.c_int32)]

    def as_dict(self) -> dict:
        return {f: getattr(self, f) for f, _ in self._fields_}

    @property
    def balance(self) -> float:
        """Block-groups of the busiest workgroup over the mean (1.0 = perfectly even)."""
        return self.busiest_units * self.grid / max(1, self.total_units)


class AttnInfo(ctypes.Structure):
    """The launch shape ql_attention_decode picks (ql_attn_info)."""
    _fields_ = [("heads_per_run", ctypes.c_int32), ("nsplit", ctypes.c_int32),
                ("workgroups", ctypes.c_int32), ("keys_per_split", ctypes.c_int32)]


_lib = None


def header_functions() -> list[str]:
    """Names of every function declared in include/qlinear.h."""
    text = open(HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ql_\w+)\s*\(", text, flags=re.M)


def lib():
    """Loads libqlinear.so; raises if it is missing (no fallback path exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"libqlinear.so not built at {LIB_PATH}: run __graft_entry__.build()")
    L = ctypes.CDLL(LIB_PATH)
    P, I, U64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint64
    pp = ctypes.POINTER(ctypes.c_void_p)
    sig = {
        "ql_create": (I, [I, pp]),
        "ql_destroy": (I, [P]),
        "ql_last_error": (ctypes.c_char_p, []),
        "ql_device_info": (I, [P, ctypes.c_char_p, I, ctypes.POINTER(I), ctypes.POINTER(U64)]),
        "ql_arena_reserve": (I, [P, U64, pp]),
        "ql_arena_release": (I, [P]),
        "ql_arena_size": (U64, [P]),
        "ql_arena_device_ptr": (U64, [P]),
        "ql_arena_write": (I, [P, U64, P, U64]),
        "ql_arena_read": (I, [P, U64, P, U64]),
        "ql_arena_copy": (I, [P, P, U64, P, U64, U64]),
        "ql_gptq_sizes": (I, [I, I, I, ctypes.POINTER(U64), ctypes.POINTER(U64),
                              ctypes.POINTER(U64)]),
        "ql_gptq_validate": (I, [ctypes.POINTER(GptqDesc), U64]),
        "ql_gptq_check": (I, [ctypes.POINTER(GptqDesc), P]),
        "ql_unpack_f16": (I, [P, ctypes.POINTER(GptqDesc), P, P, U64]),
        "ql_unpack_f32": (I, [P, ctypes.POINTER(GptqDesc), P, P, U64]),
        "ql_unpack_f32_ex": (I, [P, ctypes.POINTER(GptqDesc), P, I, P, U64]),
        "ql_unpack_f16_batch": (I, [P, I, ctypes.POINTER(GptqDesc), P, P, ctypes.POINTER(U64)]),
        "ql_plan_linear": (I, [I, I, I, I, ctypes.POINTER(Plan)]),
        "ql_gemv_f16w": (I, [P, P, U64, U64, P, U64, I, I, I, U64]),
        "ql_kv_store": (I, [P, P, U64, P, U64, I, I, I, I]),
        "ql_embed_f16": (I, [P, P, U64, I, I, P, U64, I, U64]),
        "ql_add_rmsnorm": (I, [P, P, U64, U64, P, U64, ctypes.c_float, I, I, U64, U64]),
        "ql_silu_mul": (I, [P, P, U64, U64, ctypes.c_int64, U64]),
        "ql_attention_decode": (I, [P, P, U64, P, U64, U64, I, I, I, I, I, I, U64]),
        "ql_plan_attention": (I, [I, I, I, I, I, I, ctypes.POINTER(AttnInfo)]),
        "ql_linear": (I, [P, ctypes.POINTER(GptqDesc), P, P, U64, I, I, U64, U64]),
        "ql_linear_noalloc": (I, [P, ctypes.POINTER(GptqDesc), P, P, U64, I, I, U64]),
        "ql_plan_batch": (I, [I, ctypes.POINTER(GptqDesc), I, ctypes.POINTER(U64)]),
        "ql_linear_batch": (I, [P, I, ctypes.POINTER(GptqDesc), P, P, ctypes.POINTER(U64), I, I,
                                ctypes.POINTER(U64), U64]),
        "ql_sync": (I, [P]),
        "ql_timer_start": (I, [P]),
        "ql_timer_stop": (I, [P, ctypes.POINTER(ctypes.c_float)]),
        "ql_graph_begin": (I, [P]),
        "ql_graph_end": (I, [P, pp]),
        "ql_graph_launch": (I, [P, P]),
        "ql_graph_destroy": (I, [P]),
        "ql_plan_seq": (I, [I, ctypes.POINTER(GptqDesc), I, ctypes.POINTER(U64), I,
                            ctypes.POINTER(U64), I, ctypes.POINTER(SeqInfo)]),
        "ql_seq_create": (I, [P, I, ctypes.POINTER(GptqDesc), P, P, ctypes.POINTER(U64), I, I,
                              ctypes.POINTER(U64), pp]),
        "ql_plan_seq_fused": (I, [I, ctypes.POINTER(GptqDesc), I, ctypes.POINTER(U64), I,
                                  ctypes.POINTER(U64), ctypes.POINTER(SeqFuse), I, ctypes.POINTER(SeqInfo)]),
        "ql_seq_create_fused": (I, [P, I, ctypes.POINTER(GptqDesc), P, P, ctypes.POINTER(U64), I, I,
                                    ctypes.POINTER(U64), ctypes.POINTER(SeqFuse), pp]),
        "ql_seq_get_info": (I, [P, ctypes.POINTER(SeqInfo)]),
        "ql_seq_run": (I, [P, P]),
        "ql_seq_status": (I, [P, P]),
        "ql_seq_set_spin_limit": (I, [P, ctypes.c_uint32]),
        "ql_seq_destroy": (I, [P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(rc: int):
    if rc != 0:
        raise QlError(rc, lib().ql_last_error().decode(errors="replace"))


def gptq_sizes(K: int, N: int, group: int = 128) -> tuple[int, int, int]:
    a, b, c = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    _check(lib().ql_gptq_sizes(K, N, group, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)))
    return a.value, b.value, c.value


def plan_linear(M: int, N: int, K: int, group: int = 128) -> Plan:
    p = Plan()
    _check(lib().ql_plan_linear(M, N, K, group, ctypes.byref(p)))
    return p


def plan_attention(max_t: int, M: int, n_head: int, n_kv_head: int, D: int, past_len: int) -> AttnInfo:
    """The launch shape of ql_attention_decode for these dimensions (host only)."""
    info = AttnInfo()
    _check(lib().ql_plan_attention(max_t, M, n_head, n_kv_head, D, past_len, ctypes.byref(info)))
    return info


def plan_batch(descs: list[GptqDesc], M: int) -> int:
    arr = (GptqDesc * len(descs))(*descs)
    out = ctypes.c_uint64()
    _check(lib().ql_plan_batch(len(descs), arr, M, ctypes.byref(out)))
    return out.value


def plan_seq(descs: list[GptqDesc], M: int, x_offs, y_offs, grid: int,
             x_dtype: int = DTYPE_F32, fuse: list[SeqFuse] | None = None) -> SeqInfo:
    """Validation and plan figures of a linear sequence for `grid` workgroups (host only)."""
    n = len(descs)
    info = SeqInfo()
    if fuse is None:
        _check(lib().ql_plan_seq(n, (GptqDesc * n)(*descs), M, (ctypes.c_uint64 * n)(*x_offs), x_dtype,
                                 (ctypes.c_uint64 * n)(*y_offs), grid, ctypes.byref(info)))
    else:
        if len(fuse) != n:
            raise ValueError(f"fuse has {len(fuse)} entries for {n} linears")
        _check(lib().ql_plan_seq_fused(n, (GptqDesc * n)(*descs), M, (ctypes.c_uint64 * n)(*x_offs), x_dtype,
                                       (ctypes.c_uint64 * n)(*y_offs), (SeqFuse * n)(*fuse), grid,
                                       ctypes.byref(info)))
    return info


def validate(desc: GptqDesc, arena_bytes: int) -> int:
    """Host-only validation (quant.ts:44-79 classes); returns the status code, does not raise."""
    return lib().ql_gptq_validate(ctypes.byref(desc), arena_bytes)


def make_desc(qweight_off: int, qzeros_off: int | None, scales_off: int, K: int, N: int,
              group: int = 128, bias_off: int | None = None, bits: int = 4) -> GptqDesc:
    return GptqDesc(qweight_off, QL_NONE if qzeros_off is None else qzeros_off, scales_off,
                    QL_NONE if bias_off is None else bias_off, K, N, group, bits)


class Arena:
    """One device allocation addressed by byte offset (src/gpu/arena.ts:17-59 intent)."""

    def __init__(self, ctx: "Context", nbytes: int):
        h = ctypes.c_void_p()
        _check(lib().ql_arena_reserve(ctx.handle, nbytes, ctypes.byref(h)))
        self.ctx = ctx
        self.handle = h
        self.size = nbytes
        ctx._owned.add(self)

    def write(self, off: int, data: np.ndarray | bytes):
        buf = np.ascontiguousarray(np.frombuffer(data, dtype=np.uint8) if isinstance(data, bytes)
                                   else data)
        _check(lib().ql_arena_write(self.handle, off, buf.ctypes.data, buf.nbytes))

    def read(self, off: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        _check(lib().ql_arena_read(self.handle, off, out.ctypes.data, out.nbytes))
        return out

    @property
    def device_ptr(self) -> int:
        return lib().ql_arena_device_ptr(self.handle)

    def release(self):
        if self.handle:
            _check(lib().ql_arena_release(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class Graph:
    def __init__(self, ctx: "Context", handle):
        self.ctx = ctx
        self.handle = handle
        ctx._owned.add(self)

    def launch(self):
        _check(lib().ql_graph_launch(self.ctx.handle, self.handle))

    def destroy(self):
        if self.handle:
            _check(lib().ql_graph_destroy(self.handle))
            self.handle = None


class Seq:
    """Decode linears run as one persistent launch; linear i consumes linear j's output when
    x_offs[i] == y_offs[j] (src/gpu/pipeline.ts:71-116 CommandBatch with passBreak)."""

    def __init__(self, ctx: "Context", descs: list[GptqDesc], weights: Arena, act: Arena, x_offs,
                 x_dtype: int, M: int, y_offs, fuse: list[SeqFuse] | None = None):
        n = len(descs)
        h = ctypes.c_void_p()
        if fuse is None:
            _check(lib().ql_seq_create(ctx.handle, n, (GptqDesc * n)(*descs), weights.handle,
                                       act.handle, (ctypes.c_uint64 * n)(*x_offs), x_dtype, M,
                                       (ctypes.c_uint64 * n)(*y_offs), ctypes.byref(h)))
        else:
            if len(fuse) != n:
                raise ValueError(f"fuse has {len(fuse)} entries for {n} linears")
            _check(lib().ql_seq_create_fused(ctx.handle, n, (GptqDesc * n)(*descs), weights.handle,
                                             act.handle, (ctypes.c_uint64 * n)(*x_offs), x_dtype, M,
                                             (ctypes.c_uint64 * n)(*y_offs), (SeqFuse * n)(*fuse),
                                             ctypes.byref(h)))
        self.ctx = ctx
        self.handle = h
        ctx._owned.add(self)

    @property
    def info(self) -> SeqInfo:
        out = SeqInfo()
        _check(lib().ql_seq_get_info(self.handle, ctypes.byref(out)))
        return out

    def run(self):
        _check(lib().ql_seq_run(self.ctx.handle, self.handle))

    def status(self):
        """Waits for the stream; raises QlError(QL_E_STATE) if a run was aborted."""
        _check(lib().ql_seq_status(self.ctx.handle, self.handle))

    def set_spin_limit(self, polls: int):
        _check(lib().ql_seq_set_spin_limit(self.handle, polls))

    def destroy(self):
        if self.handle:
            _check(lib().ql_seq_destroy(self.handle))
            self.handle = None


class Context:
    """One device, one HIP stream (src/gpu/device.ts:40-98 initGpu)."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        _check(lib().ql_create(device, ctypes.byref(h)))
        self.handle = h
        self._owned = weakref.WeakSet()    # arenas and graphs, released before the context

    def info(self) -> dict:
        name = ctypes.create_string_buffer(256)
        cus = ctypes.c_int32()
        hbm = ctypes.c_uint64()
        _check(lib().ql_device_info(self.handle, name, 256, ctypes.byref(cus), ctypes.byref(hbm)))
        return {"name": name.value.decode(), "cu_count": cus.value, "hbm_bytes": hbm.value}

    def arena(self, nbytes: int) -> Arena:
        return Arena(self, nbytes)

    def copy(self, dst: Arena, dst_off: int, src: Arena, src_off: int, nbytes: int):
        _check(lib().ql_arena_copy(self.handle, dst.handle, dst_off, src.handle, src_off, nbytes))

    def check(self, desc: GptqDesc, weights: Arena):
        _check(lib().ql_gptq_check(ctypes.byref(desc), weights.handle))

    def unpack_f16(self, desc: GptqDesc, weights: Arena, out: Arena, out_off: int):
        _check(lib().ql_unpack_f16(self.handle, ctypes.byref(desc), weights.handle, out.handle,
                                   out_off))

    def unpack_f16_batch(self, descs, weights: Arena, out: Arena, out_offs):
        n = len(descs)
        arr = (GptqDesc * n)(*descs)
        offs = (ctypes.c_uint64 * n)(*out_offs)
        _check(lib().ql_unpack_f16_batch(self.handle, n, arr, weights.handle, out.handle, offs))

    def gemv_f16w(self, weights: Arena, w_off: int, bias_off, act: Arena, x_off: int, M: int, N: int,
                  K: int, y_off: int):
        """y[M,N] = x[M,K] . W^T (+ bias) for fp16 W [N,K] (the tied lm_head, qwen.ts:488-489)."""
        _check(lib().ql_gemv_f16w(self.handle, weights.handle, w_off,
                                  QL_NONE if bias_off is None else bias_off, act.handle, x_off, M, N,
                                  K, y_off))

    def embed_f16(self, weights: Arena, embed_off: int, vocab: int, D: int, act: Arena, tokens_off: int,
                  rows: int, out_off: int):
        """out[r, :] = f32(embed[tokens[r], :]) (embedding_f16.wgsl; qwen.ts:392); token ids >= vocab
        give zero rows."""
        _check(lib().ql_embed_f16(self.handle, weights.handle, embed_off, vocab, D, act.handle, tokens_off,
                                  rows, out_off))

    def kv_store(self, act: Arena, src_off: int, cache: Arena, cache_off: int, max_t: int, rows: int,
                 row_len: int, pos0: int):
        """cache[pos0 + r, :] = src[r, :] (misc/kv_store.wgsl; qwen.ts:427-428)."""
        _check(lib().ql_kv_store(self.handle, act.handle, src_off, cache.handle, cache_off, max_t, rows,
                                 row_len, pos0))

    def attention_decode(self, act: Arena, q_off: int, cache: Arena, k_off: int, v_off: int, max_t: int,
                         M: int, n_head: int, n_kv_head: int, D: int, past_len: int, out_off: int):
        """Causal GQA attention of M new query rows over the KV cache (attention_gqa_cache.wgsl)."""
        _check(lib().ql_attention_decode(self.handle, act.handle, q_off, cache.handle, k_off, v_off,
                                         max_t, M, n_head, n_kv_head, D, past_len, out_off))

    def add_rmsnorm(self, act: Arena, x_off: int, d_off, weights: Arena, w_off: int, eps: float, M: int,
                    C: int, y_off: int, sum_off=None):
        """y = rmsnorm(x (+ d)) * w, the sum stored at sum_off (vec_add + rmsnorm.wgsl in one launch)."""
        _check(lib().ql_add_rmsnorm(self.handle, act.handle, x_off, QL_NONE if d_off is None else d_off,
                                    weights.handle, w_off, eps, M, C,
                                    QL_NONE if sum_off is None else sum_off, y_off))

    def silu_mul(self, act: Arena, gate_off: int, up_off: int, n: int, y_off: int):
        """y = silu(gate) * up (activation/silu_mul.wgsl)."""
        _check(lib().ql_silu_mul(self.handle, act.handle, gate_off, up_off, n, y_off))

    def unpack_f32(self, desc: GptqDesc, weights: Arena, out: Arena, out_off: int,
                   scales_dtype: int = DTYPE_F16):
        """fp32 [N,K] dequant; scales_dtype DTYPE_F32 reads f32 scales at desc.scales_off."""
        _check(lib().ql_unpack_f32_ex(self.handle, ctypes.byref(desc), weights.handle, scales_dtype,
                                      out.handle, out_off))

    def linear(self, desc: GptqDesc, weights: Arena, act: Arena, x_off: int, x_dtype: int, M: int,
               y_off: int, scratch_off: int = 0):
        _check(lib().ql_linear(self.handle, ctypes.byref(desc), weights.handle, act.handle, x_off,
                               x_dtype, M, y_off, scratch_off))

    def linear_noalloc(self, desc: GptqDesc, weights: Arena, act: Arena, x_off: int, x_dtype: int,
                       M: int, y_off: int):
        """ql_linear without a scratch argument: split-K partials in the library's static
        per-GPU array (NOALLOC_SCRATCH_BYTES); calls overlapping on one GPU race."""
        _check(lib().ql_linear_noalloc(self.handle, ctypes.byref(desc), weights.handle, act.handle,
                                       x_off, x_dtype, M, y_off))

    def linear_batch(self, descs: list[GptqDesc], weights: Arena, act: Arena, x_offs, x_dtype: int,
                     M: int, y_offs, scratch_off: int = 0):
        n = len(descs)
        arr = (GptqDesc * n)(*descs)
        xo = (ctypes.c_uint64 * n)(*x_offs)
        yo = (ctypes.c_uint64 * n)(*y_offs)
        _check(lib().ql_linear_batch(self.handle, n, arr, weights.handle, act.handle, xo, x_dtype,
                                     M, yo, scratch_off))

    def seq(self, descs: list[GptqDesc], weights: Arena, act: Arena, x_offs, x_dtype: int, M: int,
            y_offs, fuse: list[SeqFuse] | None = None) -> Seq:
        return Seq(self, descs, weights, act, x_offs, x_dtype, M, y_offs, fuse)

    def sync(self):
        _check(lib().ql_sync(self.handle))

    def timer_start(self):
        _check(lib().ql_timer_start(self.handle))

    def timer_stop(self) -> float:
        ms = ctypes.c_float()
        _check(lib().ql_timer_stop(self.handle, ctypes.byref(ms)))
        return ms.value

    def graph_begin(self):
        _check(lib().ql_graph_begin(self.handle))

    def graph_end(self) -> Graph:
        h = ctypes.c_void_p()
        _check(lib().ql_graph_end(self.handle, ctypes.byref(h)))
        return Graph(self, h)

    def destroy(self):
        if self.handle:
            for obj in list(self._owned):
                if isinstance(obj, (Graph, Seq)):
                    obj.destroy()
            for obj in list(self._owned):
                if isinstance(obj, Arena):
                    obj.release()
            _check(lib().ql_destroy(self.handle))
            self.handle = None


@dataclass
class ArenaLayout:
    """Bump allocator over byte offsets, 256-byte aligned (src/gpu/buffer.ts:3 ALIGN=256)."""
    used: int = 0

    def take(self, nbytes: int, align: int = 256) -> int:
        off = (self.used + align - 1) // align * align
        self.used = off + nbytes
        return off
