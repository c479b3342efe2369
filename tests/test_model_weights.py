"""The converter's model-weights format (scripts/convert_qwen36.py:222-327):
the repository's restatement of its writer (tests/golden/model_weights_recipe.py)
reproduces the bytes the converter itself wrote for a two-layer mini model
(the SHA-256 in tests/golden/model_weights_mini.sha256) and its tensor table
(tests/golden/model_weights_mini.json).  The device tests load that file
through nmoe_hip_load_model_weights."""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import model_weights_recipe as R  # noqa: E402


def test_writer_reproduces_the_converter(tmp_path):
    path = str(tmp_path / "model_weights.bin")
    table = R.write_model_weights(path)
    digest, size = open(os.path.join(HERE, "golden", "model_weights_mini.sha256")).read().split()
    assert os.path.getsize(path) == int(size)
    assert R.sha256(path) == digest
    manifest = json.load(open(os.path.join(HERE, "golden", "model_weights_mini.json")))
    assert manifest["tensors"] == table
    assert manifest["num_tensors"] == len(table) == 39
    # the converter leaves the routed experts (packed separately) and the vision tower out
    assert not any(".mlp.experts." in n or "visual" in n for n in table)
    assert table["model.layers.0.linear_attn.A_log"]["dtype"] == "F32"
    assert all(v["offset"] % 64 == 0 for v in table.values())
