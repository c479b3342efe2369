"""The library's plain-C host code (host/json.c, layout.c, weights.c,
pack_io.c) and the CPU oracle built with AddressSanitizer and
UndefinedBehaviorSanitizer (tests/host_sanitize.c, the device side replaced
by host-memory stand-ins), then run on hostile inputs: truncated, oversized,
deeply nested and non-finite JSON (-nan, 1e400, hex and inf forms), layout
and model-weights manifests whose offsets, sizes, shapes and types are
wrong, short layer files, and the oracle's routing, norm and dequant on
NaN/inf values.  Every run must end with no sanitizer report, and the
inputs the parser must refuse are refused.  (The reference builds its host
code with -Wall -Wextra only, Makefile:7.)"""
import json
import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PKG = os.path.join(ROOT, "nano-metal-moe-qwen36_amd")
sys.path.insert(0, os.path.join(HERE, "golden"))

SOURCES = [os.path.join(HERE, "host_sanitize.c")] + [os.path.join(PKG, "host", f) for f in
                                                     ("json.c", "layout.c", "weights.c", "pack_io.c")] + \
          [os.path.join(ROOT, "oracle", "nmoe_oracle.c")]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    out = str(tmp_path_factory.mktemp("san") / "host_sanitize")
    cmd = ["gcc", "-std=gnu11", "-g", "-O1", "-fno-omit-frame-pointer", "-Wall", "-Wextra", "-Werror",
           "-fsanitize=address,undefined", "-fsanitize=float-cast-overflow", "-fno-sanitize-recover=all",
           "-I" + os.path.join(ROOT, "include")] + SOURCES + ["-lm", "-o", out]
    subprocess.run(cmd, check=True)
    return out


def run(harness, *args):
    r = subprocess.run([harness, *map(str, args)], capture_output=True, text=True, env=ENV, timeout=120)
    report = "AddressSanitizer" in r.stderr or "runtime error" in r.stderr or "LeakSanitizer" in r.stderr
    assert r.returncode == 0 and not report, f"{args}: exit {r.returncode}\n{r.stderr[-3000:]}"
    line = [l for l in r.stdout.splitlines() if l.startswith("rc=")]
    return int(line[-1][3:])


JSON_BAD = [
    b"", b" ", b"{", b"[", b"-", b"1e", b"{\"a\"", b"{\"a\":", b"{\"a\": [1, 2", b"\"abc", b"\"abc\\", b"\"\\u12",
    b"{\"a\": \"x\\u\"", b"[1, 2,", b"[1 2]", b"{\"a\" 1}", b"{1: 2}", b"tru", b"nul", b"[true, fals]",
    b"-nan", b"nan", b"NaN", b"inf", b"-inf", b"Infinity", b"0x10", b"1e400", b"-1e400", b"[1e999]",
    b"{\"offset\": -nan}", b"1" * 80, b"[" * 40 + b"]" * 40, b"{\"a\":" * 40 + b"1" + b"}" * 40,
    b"[" * 100000, b"{\"a\": 1} x", bytes(range(256)),
]
JSON_GOOD = [
    b"0", b"-0", b"[]", b"{}", b"1.5e-400", b"[1.0e15, 9.1e15, -3]", b"\"\\u00e9\\n\\t\"", b"[" * 32 + b"]" * 32,
    b"{\"a\": [1, 2, {\"b\": -1e3, \"c\": null, \"d\": true}]}", b"[" + b",".join([b"1"] * 100000) + b"]",
    b"\"" + b"x" * 200000 + b"\"",
]


def test_json_reader_hostile_inputs(harness, tmp_path):
    for i, doc in enumerate(JSON_BAD + JSON_GOOD):
        p = tmp_path / f"j{i}.json"
        p.write_bytes(doc)
        rc = run(harness, "json", p)
        want = 0 if doc in JSON_GOOD else -1
        assert rc == want, (doc[:60], rc)


def _layout(bits=4):
    return json.load(open(os.path.join(HERE, "golden", f"layout_q{bits}.json")))


def test_layout_validator_hostile_inputs(harness, tmp_path):
    good = _layout(4)
    cases = []
    cases.append((json.dumps(good), 0))
    for mutate in (
        lambda d: d["components"].pop(),
        lambda d: d["components"][3].update(offset=-1),
        lambda d: d["components"][3].update(offset=1e300),
        lambda d: d["components"][3].update(size="big"),
        lambda d: d["components"][0].pop("name"),
        lambda d: d["components"][0].update(name=7),
        lambda d: d["components"][1].update(shape=[512]),
        lambda d: d["components"][1].update(shape="512x32"),
        lambda d: d["components"][1].update(dtype=["u16"]),
        lambda d: d.update(expert_size=983040),
        lambda d: d.update(num_layers=0),
        lambda d: d.update(num_layers=65),
        lambda d: d.update(num_experts=128),
        lambda d: d.update(bits="q44444444444444444444"),
        lambda d: d.update(components={}),
        lambda d: d.update(components=[1, 2, 3, 4, 5, 6, 7, 8, 9]),
    ):
        d = json.loads(json.dumps(good))
        mutate(d)
        cases.append((json.dumps(d), -22))
    cases.append((json.dumps(good)[:-5], -22))  # truncated
    cases.append((json.dumps(good).replace("1769472", "-nan"), -22))
    cases.append((json.dumps(good).replace("1769472", "1e400"), -22))
    cases.append((" " * (2 << 20) + json.dumps(good), -22))  # larger than the validator reads
    for i, (text, want) in enumerate(cases):
        p = tmp_path / f"layout{i}.json"
        p.write_text(text)
        assert run(harness, "layout", p) == want, (i, text[:120])
    assert run(harness, "layout", tmp_path / "missing.json") == -2


def test_model_weights_hostile_manifests(harness, tmp_path):
    import model_weights_recipe as R
    bin_path = str(tmp_path / "model_weights.bin")
    R.write_model_weights(bin_path)
    good = json.load(open(os.path.join(HERE, "golden", "model_weights_mini.json")))
    size = os.path.getsize(bin_path)
    base = tmp_path / "mw.json"
    base.write_text(json.dumps(good))
    assert run(harness, "weights", bin_path, base, 2) == 0
    name = "model.layers.1.mlp.gate.weight"
    cases = []
    # an offset past the file is EIO; one a manifest number cannot hold (above 9e15, negative, a string
    # type) leaves the tensor out, so it is missing (ENOENT)
    for upd, want in (({"offset": size}, -5), ({"offset": 2 ** 52}, -5), ({"offset": 2 ** 53 - 1}, -2),
                      ({"offset": 1e300}, -2), ({"size": 7}, -22), ({"dtype": "F32"}, -22), ({"dtype": 5}, -2),
                      ({"offset": -64}, -2)):
        d = json.loads(json.dumps(good))
        d["tensors"][name].update(upd)
        cases.append((json.dumps(d), want))
    d = json.loads(json.dumps(good))
    d["config"]["rms_norm_eps"] = -1.0
    cases.append((json.dumps(d), -22))
    d = json.loads(json.dumps(good))
    del d["tensors"][name]
    cases.append((json.dumps(d), -2))
    cases.append((json.dumps(good).replace("1e-06", "-nan"), -22))
    cases.append((json.dumps(good)[: len(json.dumps(good)) // 2], -22))
    cases.append(("{" * 30 + "}" * 30, -22))
    cases.append(("[]", -22))
    for i, (text, want) in enumerate(cases):
        p = tmp_path / f"mw{i}.json"
        p.write_text(text)
        assert run(harness, "weights", bin_path, p, 2) == want, (i, text[:100])
    # a short weights file: every tensor lies beyond its end
    short = tmp_path / "short.bin"
    short.write_bytes(open(bin_path, "rb").read(4096))
    assert run(harness, "weights", short, base, 2) == -5


def test_layer_files_and_expert_dir(harness, tmp_path):
    """Layer files (q2, the smaller format: a full-size read under the
    sanitizer costs seconds of page faults) and an expert directory."""
    esz = 983040
    good = tmp_path / "layer_00.bin"
    with open(good, "wb") as f:
        f.truncate(256 * esz)
    short = tmp_path / "short.bin"
    with open(short, "wb") as f:
        f.truncate(256 * esz - 1)
    assert run(harness, "layer", short, 2) == -5
    assert run(harness, "layer", good, 3) == -22
    assert run(harness, "layer", tmp_path / "none.bin", 2) == -2
    d = tmp_path / "experts"
    d.mkdir()
    lay = _layout(2)
    lay["num_layers"] = 1
    (d / "layout.json").write_text(json.dumps(lay))
    assert run(harness, "expdir", d, 1) == -2  # layer_00.bin missing
    os.link(good, d / "layer_00.bin")
    assert run(harness, "expdir", d, 2) == -22  # beyond num_layers
    assert run(harness, "expdir", d, 1) == 0


def test_oracle_on_non_finite_values(harness):
    assert run(harness, "oracle") == 0
