"""ctypes bindings for the C oracle (oracle/gptq_oracle.c) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module,
and only as the checker. The product path (webllm_amd) never imports it.

The oracle restates the reference CPU path (intplusplus/webllm):
  dequantizeGptqInt4      src/weights/quant.ts:42-118
  f32ToF16Bits            src/gpu/buffer.ts:57-100
  f16BitsToF32            src/weights/safetensors.ts:144-152
  gemmNTRef               src/reference/qwen-ref.ts:126-145 (gptq_linear; gptq_linear_cols is the
                          same per output, on a column subset and several threads)
  planGemvSplit           src/model/qwen.ts:61-74
  checkTolerance/makeRng  src/reference/cpu-ref.ts:27-67 (with randomF32)
  makeNormal              src/model/init.ts:36-52
  rmsNormRef (+ vec_add)  src/reference/qwen-ref.ts:12-28, src/gpu/kernels/misc/vec_add.wgsl
  siluMulRef              src/reference/qwen-ref.ts:114-121
  attentionGqaRef         src/reference/qwen-ref.ts:65-111 (over a KV cache, with the positions of
                          src/gpu/kernels/attention/attention_gqa_cache.wgsl)
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "liboracle.so")
_lib = None

ERRORS = {
    0: "ok",
    -1: "bits",
    -2: "group",
    -3: "dims",
    -4: "qweight_short",
    -5: "scales_short",
    -6: "qzeros_short",
    -7: "group_pack",
}


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        L.orc_f32_to_f16_bits.restype = ctypes.c_uint16
        L.orc_f32_to_f16_bits.argtypes = [ctypes.c_float]
        L.orc_f16_bits_to_f32.restype = ctypes.c_float
        L.orc_f16_bits_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16_array.argtypes = [P, P, ctypes.c_size_t]
        L.orc_f16_to_f32_array.argtypes = [P, P, ctypes.c_size_t]
        L.orc_f16_exhaustive_check.argtypes = [P]
        L.orc_dequant_gptq_int4.restype = ctypes.c_int
        L.orc_dequant_gptq_int4.argtypes = [P, ctypes.c_size_t, P, ctypes.c_size_t, P,
                                            ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_int, P]
        L.orc_dequant_gptq_int4_f16.restype = ctypes.c_int
        L.orc_dequant_gptq_int4_f16.argtypes = [P, ctypes.c_size_t, P, ctypes.c_size_t, P,
                                                ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                                ctypes.c_int, P]
        L.orc_gemm_nt.argtypes = [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P]
        L.orc_gptq_linear.restype = ctypes.c_int
        L.orc_gptq_linear.argtypes = [P, P, P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, P]
        L.orc_gptq_linear_cols.restype = ctypes.c_int
        L.orc_gptq_linear_cols.argtypes = [P, P, P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P]
        L.orc_plan_gemv_split.restype = ctypes.c_int
        L.orc_plan_gemv_split.argtypes = [ctypes.c_int, ctypes.c_int]
        L.orc_add_rmsnorm.restype = None
        L.orc_add_rmsnorm.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_double, P, P]
        L.orc_silu_mul.restype = None
        L.orc_silu_mul.argtypes = [P, P, ctypes.c_size_t, P]
        L.orc_attention_gqa_cache.restype = ctypes.c_int
        L.orc_attention_gqa_cache.argtypes = [P, P, P] + [ctypes.c_int] * 5 + [P]
        L.orc_check_tolerance.restype = ctypes.c_int
        L.orc_check_tolerance.argtypes = [P, P, ctypes.c_size_t, ctypes.c_double, ctypes.c_double,
                                          ctypes.POINTER(ctypes.c_double),
                                          ctypes.POINTER(ctypes.c_double)]
        L.orc_rng_step.restype = ctypes.c_uint32
        L.orc_rng_step.argtypes = [ctypes.POINTER(ctypes.c_uint32)]
        L.orc_rng_next.restype = ctypes.c_double
        L.orc_rng_next.argtypes = [ctypes.POINTER(ctypes.c_uint32)]
        L.orc_rng_seed.argtypes = [ctypes.POINTER(ctypes.c_uint32), ctypes.c_uint32]
        L.orc_random_f32.restype = None
        L.orc_random_f32.argtypes = [ctypes.POINTER(ctypes.c_uint32), ctypes.c_size_t, P]
        L.orc_normal_next.restype = ctypes.c_double
        L.orc_normal_next.argtypes = [ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_double),
                                      ctypes.POINTER(ctypes.c_int)]
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out


def f16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().orc_f16_to_f32_array(_ptr(b), _ptr(out), b.size)
    return out


def f16_exhaustive_check() -> list:
    counts = np.zeros(4, dtype=np.uint64)
    lib().orc_f16_exhaustive_check(_ptr(counts))
    return [int(c) for c in counts]


def dequantize_gptq_int4(qweight: bytes | np.ndarray, qzeros, scales: np.ndarray,
                         in_features: int, out_features: int, group_size: int = 128,
                         bits: int = 4):
    """Returns (rc, W[out,in] float32). rc < 0 is the quant.ts error class (ERRORS)."""
    qw = np.frombuffer(bytes(qweight), dtype=np.uint8) if not isinstance(qweight, np.ndarray) \
        else np.ascontiguousarray(qweight).view(np.uint8).reshape(-1)
    qz = None
    if qzeros is not None:
        qz = np.frombuffer(bytes(qzeros), dtype=np.uint8) if not isinstance(qzeros, np.ndarray) \
            else np.ascontiguousarray(qzeros).view(np.uint8).reshape(-1)
    sc = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
    n_out = max(in_features, 0) * max(out_features, 0)
    out = np.zeros(max(n_out, 1), dtype=np.float32)
    rc = lib().orc_dequant_gptq_int4(_ptr(qw), qw.size, _ptr(qz), 0 if qz is None else qz.size,
                                     _ptr(sc), sc.size, in_features, out_features, group_size,
                                     bits, _ptr(out))
    if rc != 0:
        return rc, None
    return rc, out[:n_out].reshape(out_features, in_features)


def dequantize_gptq_int4_f16(qweight: np.ndarray, qzeros, scales_f16: np.ndarray, K: int,
                             N: int, group: int = 128) -> np.ndarray:
    """fp16 [N,K] bits as the reference loader uploads them (dequant, then f32ToF16Bits)."""
    qw = np.ascontiguousarray(qweight, dtype=np.uint32)
    qz = None if qzeros is None else np.ascontiguousarray(qzeros, dtype=np.uint32)
    sc = np.ascontiguousarray(scales_f16).view(np.uint16)
    out = np.empty((N, K), dtype=np.uint16)
    rc = lib().orc_dequant_gptq_int4_f16(_ptr(qw), qw.nbytes, _ptr(qz),
                                         0 if qz is None else qz.nbytes, _ptr(sc), sc.size, K, N,
                                         group, _ptr(out))
    if rc != 0:
        raise ValueError(f"oracle dequant failed: {ERRORS.get(rc, rc)}")
    return out


def gemm_nt(A: np.ndarray, W: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    A = np.ascontiguousarray(A, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.float32)
    M, K = A.shape
    N = W.shape[0]
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    C = np.empty((M, N), dtype=np.float32)
    lib().orc_gemm_nt(_ptr(A), _ptr(W), M, N, K, _ptr(b), _ptr(C))
    return C


def gptq_linear(qweight, qzeros, scales_f16, x, bias=None, group: int = 128) -> np.ndarray:
    """y[M,N] = gemmNTRef(x, dequantizeGptqInt4(...)) (+bias), double accumulation."""
    qw = np.ascontiguousarray(qweight, dtype=np.uint32)
    qz = None if qzeros is None else np.ascontiguousarray(qzeros, dtype=np.uint32)
    sc = np.ascontiguousarray(scales_f16).view(np.uint16)
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    N = qw.shape[1]
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    y = np.empty((M, N), dtype=np.float32)
    rc = lib().orc_gptq_linear(_ptr(qw), _ptr(qz), _ptr(sc), _ptr(b), _ptr(x), M, K, N, group,
                               _ptr(y))
    if rc != 0:
        raise ValueError("oracle gptq_linear: bad arguments")
    return y


def default_threads() -> int:
    """Oracle threads: the host's cores, at most 16 (a GPU box's CPU share)."""
    return max(1, min(16, os.cpu_count() or 1))


def gptq_linear_cols(qweight, qzeros, scales_f16, x, cols, bias=None, group: int = 128,
                     threads: int | None = None, w_f16: bool = False) -> np.ndarray:
    """gptq_linear for the output columns `cols` only: y[M, len(cols)], every value
    bit-identical to gptq_linear(...)[:, cols]; the columns are shared among threads.
    w_f16: the weights rounded to fp16 first (the GEMM path's operand: gemm_nt over
    dequantize_gptq_int4_f16)."""
    qw = np.ascontiguousarray(qweight, dtype=np.uint32)
    qz = None if qzeros is None else np.ascontiguousarray(qzeros, dtype=np.uint32)
    sc = np.ascontiguousarray(scales_f16).view(np.uint16)
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    N = qw.shape[1]
    c = np.ascontiguousarray(cols, dtype=np.int32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    y = np.empty((M, c.size), dtype=np.float32)
    rc = lib().orc_gptq_linear_cols(_ptr(qw), _ptr(qz), _ptr(sc), _ptr(b), _ptr(x), M, K, N, group,
                                    _ptr(c), c.size, threads or default_threads(), int(w_f16), _ptr(y))
    if rc != 0:
        raise ValueError("oracle gptq_linear_cols: bad arguments")
    return y


def add_rmsnorm(x: np.ndarray, w: np.ndarray, eps: float, d: np.ndarray | None = None):
    """(s, y): s = x + d (or x), y = rmsNormRef(s, w, eps) over the rows of [M, C]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, C = x.shape
    dd = None if d is None else np.ascontiguousarray(d, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    s = np.empty_like(x)
    y = np.empty_like(x)
    lib().orc_add_rmsnorm(_ptr(x), _ptr(dd), _ptr(w), M, C, eps, _ptr(s), _ptr(y))
    return s, y


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(gate, dtype=np.float32).reshape(-1)
    u = np.ascontiguousarray(up, dtype=np.float32).reshape(-1)
    out = np.empty_like(g)
    lib().orc_silu_mul(_ptr(g), _ptr(u), g.size, _ptr(out))
    return out.reshape(np.shape(gate))


def attention_gqa_cache(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, H: int, KV: int, D: int,
                        past: int) -> np.ndarray:
    """Causal GQA attention of q [M, H, D] over caches [>= past + M, KV * D] (attentionGqaRef)."""
    q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1, H, D)
    kc = np.ascontiguousarray(kc, dtype=np.float32).reshape(-1)
    vc = np.ascontiguousarray(vc, dtype=np.float32).reshape(-1)
    M = q.shape[0]
    if kc.size < (past + M) * KV * D or vc.size < (past + M) * KV * D:
        raise ValueError("oracle attention: cache shorter than past + M rows")
    out = np.empty((M, H, D), dtype=np.float32)
    if lib().orc_attention_gqa_cache(_ptr(q), _ptr(kc), _ptr(vc), M, H, KV, D, past, _ptr(out)) != 0:
        raise ValueError("oracle attention: bad dimensions")
    return out


def plan_gemv_split(wg_n: int, K: int) -> int:
    return lib().orc_plan_gemv_split(wg_n, K)


def check_tolerance(got: np.ndarray, ref: np.ndarray, atol: float, rtol: float):
    got = np.ascontiguousarray(got, dtype=np.float32).reshape(-1)
    ref = np.ascontiguousarray(ref, dtype=np.float32).reshape(-1)
    if got.size != ref.size:
        raise ValueError(f"checkTolerance: length mismatch got={got.size} ref={ref.size}")
    ma = ctypes.c_double()
    mr = ctypes.c_double()
    ok = lib().orc_check_tolerance(_ptr(got), _ptr(ref), got.size, atol, rtol, ctypes.byref(ma),
                                   ctypes.byref(mr))
    return bool(ok), ma.value, mr.value


class Rng:
    """makeRng (cpu-ref.ts:57-67)."""

    def __init__(self, seed: int):
        self.state = ctypes.c_uint32()
        lib().orc_rng_seed(ctypes.byref(self.state), seed & 0xFFFFFFFF)

    def step(self) -> int:
        return lib().orc_rng_step(ctypes.byref(self.state))

    def __call__(self) -> float:
        return lib().orc_rng_next(ctypes.byref(self.state))

    def random_f32(self, n: int) -> np.ndarray:
        """randomF32(n, rng) (cpu-ref.ts:50-54): n values f32(rng() * 2 - 1) in [-1, 1)."""
        out = np.empty(n, dtype=np.float32)
        lib().orc_random_f32(ctypes.byref(self.state), n, _ptr(out))
        return out


class Normal:
    """makeNormal(rng) (model/init.ts:36-52): Box-Muller pairs over a makeRng stream."""

    def __init__(self, seed: int):
        self.rng = Rng(seed)
        self.spare = ctypes.c_double()
        self.has = ctypes.c_int(0)

    def __call__(self) -> float:
        return lib().orc_normal_next(ctypes.byref(self.rng.state), ctypes.byref(self.spare),
                                     ctypes.byref(self.has))
