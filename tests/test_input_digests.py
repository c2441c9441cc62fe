"""The synthetic benchmark inputs are the bytes their recorded SHA-256 digests name
(tests/golden/input_digests.json, written by tests/golden/make_digests.py): config 1, the whole
0.5B step (weights and the M = 1 and 16 inputs), and layer 0 of the 7B step. CPU only."""
import json
import os

from tests.golden import make_digests as md

D = json.load(open(md.OUT))


def test_config1_digests():
    assert md.config1_digests() == D["config1_gate"]


def test_config2_digests():
    assert md.weights_digest("0.5b", 0x9EF0) == D["config2_weights"]
    assert md.step_inputs_digest("0.5b", 1) == D["config2_inputs_m1"]
    assert md.step_inputs_digest("0.5b", 16) == D["config2_inputs_m16"]


def test_config4_layer0_digest():
    assert md.weights_digest("7b", 0x7B, layers={0}) == D["config4_weights_layer0"]
    assert os.path.getsize(md.OUT) < 4096
