"""SHA-256 digests of the synthetic benchmark inputs, so a run can show it
used the same bytes: the GPU steps in bench.py and the Node CPU baseline read these exact tensors.

    python tests/golden/make_digests.py        # rewrites tests/golden/input_digests.json

Generators (webllm_amd/synth.py, numpy PCG64 streams keyed by (seed, layer, proj)):
  config 1  gate 896->4864: synth.gptq_linear(896, 4864, 128, seed=0x9EF0), x = synth.activations(1, 896, seed=0x9EF1)
  config 2  bench.Model("0.5b", seed=0x9EF0): linear (layer, proj) = synth.gptq_linear(K, N, 128,
            seed=0x9EF0, key=(layer, PROJ_INDEX[proj])); inputs of bench.SeqStep(M, chained=False):
            synth.activations(M, K, seed=0x5EED, key=(0, 0, M)) for the first linear, key
            (layer + 1, i, M) for linear i of each layer otherwise
  config 4  bench.Model("7b", seed=0x7B): the same with the 7B shapes (28 layers x q, o, gate, up, down)
Each weights digest covers qweight, qzeros and scales of every linear in execution order.
"""
import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from webllm_amd import synth  # noqa: E402

OUT = os.path.join(HERE, "input_digests.json")
PROJS = {"0.5b": [p for p, _, _ in synth.PROJ_05B], "7b": [p for p, _, _ in synth.PROJ_7B]}


def weights_digest(shape: str, seed: int, layers=None) -> str:
    h = hashlib.sha256()
    for (layer, proj, K, N) in synth.model_linears(shape):
        if layers is not None and layer not in layers:
            continue
        t = synth.gptq_linear(K, N, 128, seed=seed, key=(layer, synth.PROJ_INDEX[proj]))
        h.update(t.qweight.tobytes())
        h.update(t.qzeros.tobytes())
        h.update(t.scales.tobytes())
    return h.hexdigest()


def step_inputs_digest(shape: str, M: int, seed: int = 0x5EED) -> str:
    """The external inputs of bench.SeqStep(model, M, chained=False), from the list SeqStep itself
    writes (bench.step_inputs), in its order."""
    import bench
    h = hashlib.sha256()
    for _, K, key in bench.step_inputs(shape, M, chained=False):
        h.update(synth.activations(M, K, seed=seed, key=key).tobytes())
    return h.hexdigest()


def config1_digests() -> dict:
    t = synth.gptq_linear(896, 4864, 128, seed=0x9EF0)
    x = synth.activations(1, 896, seed=0x9EF1)
    return {"qweight": hashlib.sha256(t.qweight.tobytes()).hexdigest(),
            "qzeros": hashlib.sha256(t.qzeros.tobytes()).hexdigest(),
            "scales": hashlib.sha256(t.scales.tobytes()).hexdigest(),
            "x": hashlib.sha256(x.tobytes()).hexdigest()}


def all_digests() -> dict:
    return {
        "config1_gate": config1_digests(),
        "config2_weights": weights_digest("0.5b", 0x9EF0),
        "config2_inputs_m1": step_inputs_digest("0.5b", 1),
        "config2_inputs_m16": step_inputs_digest("0.5b", 16),
        "config4_weights_layer0": weights_digest("7b", 0x7B, layers={0}),
        "config4_weights": weights_digest("7b", 0x7B),
        "config4_inputs_m1": step_inputs_digest("7b", 1),
    }


if __name__ == "__main__":
    d = all_digests()
    with open(OUT, "w") as f:
        json.dump(d, f, indent=1)
        f.write("\n")
    print(json.dumps(d, indent=1))
