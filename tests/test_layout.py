"""layout.json validation (nmoe_hip_validate_layout): the converter's schema
(scripts/convert_qwen36.py:341-360; fixtures tests/golden/layout_q4.json and
layout_q2.json hold its output format for q4 and q2) and the richer schema
src/expert_io.m:230-320 reads are accepted; any mismatch with the fixed pack
layout is rejected.  Host code only: no GPU needed."""
import copy
import json
import os

import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def nh():
    import nmoe_hip
    return nmoe_hip


def _load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def _check(nh, tmp_path, doc, text=None):
    p = tmp_path / "layout.json"
    p.write_text(text if text is not None else json.dumps(doc))
    return nh.validate_layout(str(p))


@pytest.mark.parametrize("name,bits", [("layout_q4.json", 4), ("layout_q2.json", 2)])
def test_converter_schema_accepted(nh, name, bits):
    rc, b, nl, msg = nh.validate_layout(os.path.join(GOLDEN, name))
    assert (rc, b, nl) == (0, bits, 40), msg


def test_rich_schema_accepted(nh, tmp_path):
    """bits/quant, dtype, shape and logical_shape as expert_io.m expects them."""
    d = _load("layout_q4.json")
    d["quant"] = "Q4"
    rows = {"gate": 512, "up": 512, "down": 2048}
    cols = {"gate": 2048, "up": 2048, "down": 512}
    for c in d["components"]:
        m, kind = c["name"].split("_proj.")
        packed = cols[m] // 8 if kind == "weight" else cols[m] // 64
        c.update(dtype="U32" if kind == "weight" else "u16", shape=[rows[m], packed], logical_shape=[rows[m], cols[m]])
    assert _check(nh, tmp_path, d)[:3] == (0, 4, 40)
    del d["expert_size"], d["num_layers"]
    assert _check(nh, tmp_path, d)[:3] == (0, 4, 0)


def _mut(d, f):
    d = copy.deepcopy(d)
    f(d)
    return d


REJECT = {
    "offset": lambda d: d["components"][4].update(offset=d["components"][4]["offset"] + 4),
    "size": lambda d: d["components"][8].update(size=32767),
    "order": lambda d: d["components"].__setitem__(slice(0, 2), [d["components"][1], d["components"][0]]),
    "missing": lambda d: d["components"].pop(),
    "name": lambda d: d["components"][3].update(name="up.weight"),
    "expert_size": lambda d: d.update(expert_size=1769473),
    "bits_disagree": lambda d: d.update(bits=2),
    "bad_quant": lambda d: d.update(quant="q8"),
    "num_experts": lambda d: d.update(num_experts=128),
    "num_layers": lambda d: d.update(num_layers=0),
    "no_bits": lambda d: d.pop("expert_size"),
    "dtype": lambda d: d["components"][0].update(dtype="u16"),
    "shape": lambda d: d["components"][6].update(shape=[2048, 32]),
    "offset_type": lambda d: d["components"][2].update(offset="557056"),
    "not_object": lambda d: d["components"].__setitem__(5, [1, 2]),
}


@pytest.mark.parametrize("case", sorted(REJECT))
def test_mismatches_rejected(nh, tmp_path, case):
    rc, _, _, msg = _check(nh, tmp_path, _mut(_load("layout_q4.json"), REJECT[case]))
    assert rc == nh.EINVAL and msg, case


@pytest.mark.parametrize("text", ["", "{", "[1, 2]", '{"expert_size": 983040,}', '{"a": 1} x', "nul"])
def test_bad_json_rejected(nh, tmp_path, text):
    assert _check(nh, tmp_path, None, text=text)[0] == nh.EINVAL


def test_missing_file(nh, tmp_path):
    assert nh.validate_layout(str(tmp_path / "nope.json"))[0] == nh.ENOENT
