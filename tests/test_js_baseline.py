"""The Node CPU baseline (oracle/js/gptq_ref.js) computes exactly what the C oracle computes:
same dequant (quant.ts) and the same double-accumulated matvec (gemmNTRef), so outputs are
bit-identical. CPU only; skipped where Node is absent."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from webllm_amd import synth

NODE = shutil.which("node")
JS = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "js",
                  "gptq_ref.js")


@pytest.mark.skipif(NODE is None, reason="node not installed")
def test_js_port_bit_identical_to_c_oracle(orc, tmp_path):
    cases = [(256, 64, 2, 7), (896, 128, 1, None), (20, 13, 1, None)]
    meta = {"linears": []}
    tensors = []
    for i, (K, N, M, zero) in enumerate(cases):
        group = 128 if K % 128 == 0 else 8
        t = synth.gptq_linear(K, N, group, seed=0x15, key=(i,), stored_zero=zero)
        x = synth.activations(M, K, seed=0x16, key=(i,))
        t.qweight.tofile(tmp_path / f"qw{i}"); t.qzeros.tofile(tmp_path / f"qz{i}")
        t.scales.tofile(tmp_path / f"sc{i}"); x.tofile(tmp_path / f"x{i}")
        meta["linears"].append({"K": K, "N": N, "M": M, "group": group, "qweight": f"qw{i}",
                                "qzeros": f"qz{i}", "scales": f"sc{i}", "x": f"x{i}"})
        tensors.append((t, x, group))
    (tmp_path / "meta.json").write_text(json.dumps(meta))
    r = subprocess.run([NODE, JS, str(tmp_path), "0"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["linears"] == 3 and res["threads"] == 1
    for i, (t, x, group) in enumerate(tensors):
        y_js = np.fromfile(tmp_path / f"y_{i}.f32", dtype=np.float32)
        y_c = orc.gptq_linear(t.qweight, t.qzeros, t.scales, x, None, group).reshape(-1)
        assert np.array_equal(y_js.view(np.uint32), y_c.view(np.uint32)), i
