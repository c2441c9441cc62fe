"""Synthetic GPTQ int4 linears and activations for the benchmark configurations.

No checkpoints are available offline, so weights are random with the real layouts
(src/weights/quant.ts:6-12): qweight int32 [K/8, N] of uniform random nibbles, qzeros int32
[K/128, N/8] all 0x77777777 (stored 7 -> zero 8, the value tests/qwen/qwen-format.ts:112-123
observes in the real checkpoint), scales fp16 [K/128, N] = f16(|N(0,1)| * 0.01), activations
fp32 ~ N(0,1). Each tensor has its own numpy PCG64 stream derived from (seed, layer, proj), so
the same bytes can be regenerated for the CPU baseline.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

# Qwen2.5-0.5B (src/model/qwen-config.ts:44-54): C=896, intermediate 4864, kv dim 128, 24 layers
QWEN05_C, QWEN05_I, QWEN05_KV, QWEN05_LAYERS = 896, 4864, 128, 24
# Qwen2.5-7B-shaped linears used for the cache-exceeding roofline: C=3584, I=18944, 28 layers
QWEN7_C, QWEN7_I, QWEN7_LAYERS = 3584, 18944, 28

PROJ_05B = [("q", QWEN05_C, QWEN05_C), ("k", QWEN05_C, QWEN05_KV), ("v", QWEN05_C, QWEN05_KV),
            ("o", QWEN05_C, QWEN05_C), ("gate", QWEN05_C, QWEN05_I), ("up", QWEN05_C, QWEN05_I),
            ("down", QWEN05_I, QWEN05_C)]
# 7B config as BASELINE states it: q,o 3584->3584, gate,up 3584->18944, down 18944->3584
PROJ_7B = [("q", QWEN7_C, QWEN7_C), ("o", QWEN7_C, QWEN7_C), ("gate", QWEN7_C, QWEN7_I),
           ("up", QWEN7_C, QWEN7_I), ("down", QWEN7_I, QWEN7_C)]


@dataclass
class GptqTensors:
    K: int
    N: int
    group: int
    qweight: np.ndarray      # uint32 [ceil(K/8), N]
    qzeros: np.ndarray       # uint32 [ceil(K/group), ceil(N/8)]
    scales: np.ndarray       # uint16 fp16 bits [ceil(K/group), N]

    @property
    def nbytes(self) -> int:
        return self.qweight.nbytes + self.qzeros.nbytes + self.scales.nbytes


def _stream(seed: int, *keys: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, *keys])))


def gptq_linear(K: int, N: int, group: int = 128, seed: int = 0x9EF0, key: tuple = (),
                stored_zero: int | None = 7, scale_mult: float = 0.01) -> GptqTensors:
    """Random GPTQ int4 linear. stored_zero=None draws random stored zeros (0..15)."""
    rng = _stream(seed, *key)
    P = (K + 7) // 8
    G = (K + group - 1) // group
    NC = (N + 7) // 8
    qweight = rng.integers(0, 1 << 32, size=(P, N), dtype=np.uint32)
    if K % 8:
        # nibbles past K are never read by the reference (quant.ts:110); keep them random
        pass
    if stored_zero is None:
        nib = rng.integers(0, 16, size=(G, NC * 8), dtype=np.uint32)
        qzeros = np.zeros((G, NC), dtype=np.uint32)
        for i in range(8):
            qzeros |= nib[:, i::8] << np.uint32(4 * i)
    else:
        word = 0
        for i in range(8):
            word |= (stored_zero & 15) << (4 * i)
        qzeros = np.full((G, NC), word, dtype=np.uint32)
    scales = (np.abs(rng.standard_normal((G, N), dtype=np.float32)) * np.float32(scale_mult))
    scales = scales.astype(np.float16).view(np.uint16)
    return GptqTensors(K, N, group, qweight, qzeros, scales)


def activations(M: int, K: int, seed: int = 0x9EF1, key: tuple = (), dtype=np.float32) -> np.ndarray:
    rng = _stream(seed, *key)
    x = rng.standard_normal((M, K), dtype=np.float32)
    return x.astype(dtype) if dtype != np.float32 else x


def model_linears(shape: str) -> list[tuple[int, str, int, int]]:
    """(layer, proj, K, N) for every linear of a decode step, in execution order."""
    if shape == "0.5b":
        return [(l, p, k, n) for l in range(QWEN05_LAYERS) for (p, k, n) in PROJ_05B]
    if shape == "7b":
        return [(l, p, k, n) for l in range(QWEN7_LAYERS) for (p, k, n) in PROJ_7B]
    raise ValueError(shape)


PROJ_INDEX = {"q": 0, "k": 1, "v": 2, "o": 3, "gate": 4, "up": 5, "down": 6}
