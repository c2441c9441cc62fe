"""The Node CPU baseline (oracle/js/gptq_ref.js, the reference CPU path restated for Node) that
bench.py times beside the GPU: its f32ToF16Bits against the C oracle's restatement of
src/gpu/buffer.ts:57-104 on random and edge bit patterns, and its dequant + matvec outputs and
timing record (variants (i), (ii) and the fp16 unpack) on small linears against the oracle."""
import json
import os
import shutil
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

NODE = shutil.which("node")
pytestmark = pytest.mark.skipif(NODE is None, reason="node not on PATH")


def test_js_f32_to_f16_matches_oracle(orc):
    rng = np.random.default_rng(0xF16)
    bits = list(rng.integers(0, 1 << 32, size=20000, dtype=np.uint64).astype(np.uint32))
    # edges: zero, the smallest/largest normals and subnormals, the overflow and rounding ties,
    # values just below 2^-24 (the reference's flush to zero), infinities and NaNs
    for f in (0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 65536.0, 2.0 ** -14, 2.0 ** -24,
              2.0 ** -25, 1.5 * 2.0 ** -25, 0.99999994 * 2.0 ** -24, 2.0 ** -24 * 1.5, 1.0009765625,
              1.00048828125, 1.00146484375, np.inf, -np.inf, np.nan):
        bits.append(int(np.array(f, dtype=np.float32).view(np.uint32)))
    r = subprocess.run([NODE, os.path.join(ROOT, "oracle", "js", "gptq_ref.js"), "--f16-selftest"],
                       input=json.dumps([int(b) for b in bits]), capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    got = np.array(json.loads(r.stdout), dtype=np.uint16)
    want = orc.f32_to_f16_bits(np.array(bits, dtype=np.uint32).view(np.float32))
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(bits[i]), hex(got[i]), hex(want[i])) for i in bad[:5]]


def test_node_run_matches_oracle(orc):
    import bench
    from webllm_amd import synth
    items = []
    for i, (K, N, M) in enumerate([(896, 128, 1), (256, 520, 3), (1024, 64, 2)]):
        t = synth.gptq_linear(K, N, 128, seed=0xCB, key=(i,), stored_zero=None if i == 1 else 7)
        items.append((t, synth.activations(M, K, seed=0xCC, key=(i,))))
    res, ys = bench.node_run(items, 0.05, {"fused_reps": 2, "f16_reps": 1})
    for key in ("dequant_ms", "matvec_ms", "matvec_median_ms", "fused_ms", "f16_ms", "reps", "macs"):
        assert res[key] is not None and res[key] >= 0, key
    assert res["reps"] >= 3 and res["macs"] == sum(t.K * t.N * x.shape[0] for t, x in items)
    refs = [orc.gptq_linear(t.qweight, t.qzeros, t.scales, x) for t, x in items]
    for y, ref in zip(ys, refs):
        assert y.shape == ref.shape
        np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-6)
    ok, worst = bench.gpu_cpu_check(refs, ys, [x for _, x in items])
    assert ok and worst < 1e-2
