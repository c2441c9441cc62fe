"""Writes the small golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

Every expected value here comes from a closed form or IEEE-754 semantics, computed with plain
Python/numpy — not from the oracle under test:
  gptq_kat.json   the reference's own GPTQ known-answer test, tests/qwen/weights.ts:62-137 of
                  intplusplus/webllm (inF=16, outF=5, group 8, q[o][i]=(o*7+i*3)&15,
                  scale=0.01(g+1)(o+1) as f32, stored zero 7 -> (q-8)*scale)
  f16_cases.json  f32 -> f16 encodings fixed by IEEE binary16 round-to-nearest-even, plus the
                  reference encoder's flush of (2^-25, 2^-24) to zero (src/gpu/buffer.ts:73)
  rng.json        xorshift32 (13,17,5) outputs (src/reference/cpu-ref.ts:57-67); the first value
                  from state 1 is Marsaglia's published 270369
"""
import json
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def kat():
    inF, outF, group = 16, 5, 8
    q = [[(o * 7 + i * 3) & 0x0F for i in range(inF)] for o in range(outF)]
    scales = np.zeros((inF // group) * outF, dtype=np.float32)
    for g in range(inF // group):
        for o in range(outF):
            scales[g * outF + o] = 0.01 * (g + 1) * (o + 1)
    qweight = []
    for p in range(inF // 8):
        for o in range(outF):
            w = 0
            for k in range(8):
                w |= (q[o][p * 8 + k] & 0x0F) << (4 * k)
            qweight.append(w)
    zero_cols = (outF + 7) // 8
    stored = 7
    zw = 0
    for k in range(8):
        zw |= stored << (4 * k)
    qzeros = [zw] * ((inF // group) * zero_cols)
    want = np.zeros(outF * inF, dtype=np.float32)
    for o in range(outF):
        for i in range(inF):
            g = i // group
            want[o * inF + i] = (q[o][i] - (stored + 1)) * float(scales[g * outF + o])
    return {
        "source": "intplusplus/webllm src/tests/qwen/weights.ts:62-137",
        "in_features": inF, "out_features": outF, "group_size": group,
        "qweight_u32": qweight, "qzeros_u32": qzeros,
        "scales_f32_bits": [f32_bits(float(s)) for s in scales],
        "want_f32_bits": [f32_bits(float(v)) for v in want],
    }


def f16_cases():
    # (f32 bits, expected f16 bits, note). IEEE RNE except where noted.
    cases = [
        (0x3F800000, 0x3C00, "1.0"),
        (0xBF000000, 0xB800, "-0.5"),
        (0x477FE000, 0x7BFF, "65504 max finite"),
        (0x477FEFFF, 0x7BFF, "just below the overflow tie"),
        (0x477FF000, 0x7C00, "65520 ties to even -> Inf"),
        (0x7F800000, 0x7C00, "+Inf"),
        (0xFF800000, 0xFC00, "-Inf"),
        (0x7FC00000, 0x7E00, "NaN -> 0x7e00"),
        (0xFFC00001, 0x7E00, "negative NaN with payload -> 0x7e00 (buffer.ts:61)"),
        (0x3F801000, 0x3C00, "1 + 2^-11 ties to even (down)"),
        (0x3F803000, 0x3C02, "1 + 3*2^-11 ties to even (up)"),
        (0x3F801001, 0x3C01, "just above the tie rounds up"),
        (0x38800000, 0x0400, "2^-14 smallest normal"),
        (0x387FC000, 0x03FF, "largest subnormal"),
        (0x33800000, 0x0001, "2^-24 smallest subnormal"),
        (0x33000000, 0x0000, "2^-25 ties to even -> 0"),
        (0x33400000, 0x0000, "1.5*2^-25: IEEE gives 0x0001; buffer.ts:73 flushes to 0"),
        (0xB3400000, 0x8000, "-1.5*2^-25: flushed to -0"),
        (0x33C00000, 0x0002, "1.5*2^-24 ties to even -> 2"),
        (0x00000001, 0x0000, "f32 subnormal -> 0"),
        (0x80000000, 0x8000, "-0"),
        (0x3C23D70A, 0x211F, "0.01"),
    ]
    # cross-check the IEEE entries against numpy (the flush entries differ on purpose)
    for bits, want, note in cases:
        if "flush" in note or "NaN" in note:
            continue
        got = int(np.array([struct.unpack("<f", struct.pack("<I", bits))[0]],
                           dtype=np.float32).astype(np.float16).view(np.uint16)[0])
        assert got == want, (hex(bits), hex(got), hex(want), note)
    return [{"f32_bits": b, "f16_bits": w, "note": n} for b, w, n in cases]


def rng():
    def run(seed, n):
        s = (seed & 0xFFFFFFFF) or 1
        out = []
        for _ in range(n):
            s ^= (s << 13) & 0xFFFFFFFF
            s ^= s >> 17
            s ^= (s << 5) & 0xFFFFFFFF
            out.append(s)
        return out
    first = run(1, 1)[0]
    assert first == 270369, first
    return {"seed_1": run(1, 4), "seed_0": run(0, 4), "seed_0x9ef0": run(0x9EF0, 16),
            "seed_0x5e11": run(0x5E11, 16)}


def main():
    with open(os.path.join(HERE, "gptq_kat.json"), "w") as f:
        json.dump(kat(), f, indent=1)
    with open(os.path.join(HERE, "f16_cases.json"), "w") as f:
        json.dump(f16_cases(), f, indent=1)
    with open(os.path.join(HERE, "rng.json"), "w") as f:
        json.dump(rng(), f, indent=1)


if __name__ == "__main__":
    main()
