"""The C boundary as compiled code: include/nmoe_hip.h builds as C11, C++17
and Objective-C with warnings as errors, a C client links libnmoe_hip.so and
gets the documented answers from every call that needs no GPU, the header's
struct layouts equal the ctypes binding's, and every ctypes signature
matches the header's parameter types (read from clang's AST of the header).
The -m gpu test runs one decode step from the prebuilt C client (built by
__graft_entry__.build(), not on the GPU box) and checks it against the
oracle."""
import ctypes as C
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import nmoe_hip as nh
from conftest import ROOT, assert_close

INC = os.path.join(ROOT, "include")
SRC = os.path.join(ROOT, "tests", "abi_client.c")
LIBDIR = os.path.dirname(nh.LIB_PATH)
CLANG = "/opt/rocm/llvm/bin/clang"
PREBUILT = os.path.join(LIBDIR, "_build", "abi_client")
WARN = ["-Wall", "-Wextra", "-Werror"]


def _link(out):
    return ["-o", out, "-x", "none", nh.LIB_PATH, f"-Wl,-rpath,{LIBDIR}"]


@pytest.fixture(scope="module")
def clients(tmp_path_factory):
    d = tmp_path_factory.mktemp("abi")
    c_bin, cpp_bin = str(d / "client_c"), str(d / "client_cpp")
    subprocess.run(["gcc", "-std=c11", "-pedantic", *WARN, f"-I{INC}", SRC, *_link(c_bin)], check=True)
    subprocess.run(["g++", "-x", "c++", "-std=c++17", *WARN, f"-I{INC}", SRC, *_link(cpp_bin)], check=True)
    return c_bin, cpp_bin


def test_header_is_objective_c_compatible():
    """The reference's callers are Objective-C (src/runtime.m:3198-3201,
    3544-3547): the header and the client parse as Objective-C."""
    if not os.path.exists(CLANG):
        pytest.skip("no clang in this image")
    for src in (os.path.join(INC, "nmoe_hip.h"), SRC):
        subprocess.run([CLANG, "-x", "objective-c", "-fsyntax-only", *WARN, f"-I{INC}", src], check=True)


@pytest.mark.parametrize("which", [0, 1], ids=["c", "cpp"])
def test_client_cpu_answers(clients, which):
    r = subprocess.run([clients[which], "cpu", os.path.join(ROOT, "tests", "golden")], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failed" in r.stdout


def test_struct_layouts_match_binding(clients):
    out = subprocess.run([clients[0], "layout"], capture_output=True, text=True, check=True).stdout.split("\n")
    got = {line.split()[0]: [int(v) for v in line.split()[1:]] for line in out if line.strip()}
    R, Q, S = nh.Router, nh.QTensor, nh.SharedExpert
    assert got["router"] == [C.sizeof(R)] + [getattr(R, f).offset for f in
                                            ("kind", "num_experts", "w_bf16", "w_q4", "scales", "biases")]
    assert got["qtensor"] == [C.sizeof(Q)] + [getattr(Q, f).offset for f in ("w", "scales", "biases")]
    assert got["shared"] == [C.sizeof(S)] + [getattr(S, f).offset for f in ("gate", "up", "down", "score")]
    M = nh.MoeBlock
    assert got["block"] == [C.sizeof(M)] + [getattr(M, f).offset for f in
                                           ("router", "has_shared", "shared", "post_norm", "next_norm", "add_one",
                                            "eps")]


def _kind(ctype_name):
    """A C parameter type as the ctypes category it needs."""
    t = ctype_name.replace("const ", "").strip()
    if "*" in t or t.endswith("]"):
        return "ptr"
    # size_t and uint64_t are the same 64-bit unsigned type on this ABI (as
    # ctypes' c_size_t and c_uint64 are)
    return {"int": "int", "float": "float", "size_t": "u64", "uint64_t": "u64", "uint32_t": "u32",
            "uint16_t": "u16", "void": "void"}[t]


def _ckind(ct):
    if ct is None:
        return "void"
    if ct in (C.c_void_p, C.c_char_p) or (isinstance(ct, type) and issubclass(ct, C._Pointer)):
        return "ptr"
    return {C.c_int: "int", C.c_float: "float", C.c_size_t: "u64", C.c_uint64: "u64", C.c_uint32: "u32",
            C.c_uint16: "u16"}[ct]


def test_binding_signatures_match_header():
    if not os.path.exists(CLANG):
        pytest.skip("no clang in this image")
    ast = json.loads(subprocess.run([CLANG, "-x", "c", "-fsyntax-only", "-Xclang", "-ast-dump=json",
                                     os.path.join(INC, "nmoe_hip.h")], capture_output=True, text=True,
                                    check=True).stdout)
    decls = {}
    for node in ast.get("inner", []):
        if node.get("kind") == "FunctionDecl" and node.get("name", "").startswith("nmoe_"):
            qt = node["type"]["qualType"]
            ret = qt.split("(")[0].strip()
            params = [p["type"]["qualType"] for p in node.get("inner", []) if p.get("kind") == "ParmVarDecl"]
            decls[node["name"]] = (_kind(ret), [_kind(p) for p in params])
    assert set(decls) == set(nh._SIGS)
    for name, (res, args) in nh._SIGS.items():
        want_ret, want_args = decls[name]
        assert _ckind(res) == want_ret, name
        assert [_ckind(a) for a in args] == want_args, name


@pytest.mark.gpu
def test_client_runs_a_layer_on_device(tmp_path):
    """One q4 top-8 decode step driven from C (synthetic layer, router and x
    of seed 0, zero h_mid): routing bit-exact with the oracle, output within
    max-abs 2e-3 / rel-L2 1e-3; and a 3-layer stack from C, its one-launch
    and per-layer forms bit for bit equal."""
    from oracle import binding as B
    assert os.path.exists(PREBUILT), "build first: python -c 'import __graft_entry__ as g; g.build()'"
    out = tmp_path / "step.bin"
    r = subprocess.run([PREBUILT, "gpu", str(out)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "stack: one launch equals one launch per layer: yes" in r.stdout
    raw = np.fromfile(out, np.uint8)
    idx, w, got = raw[:32].view(np.uint32), raw[32:64].view(np.float32), raw[64:].view(np.float32)
    W = B.syn_bf16(256 * 2048, 0, 0, 16, 0.02).reshape(256, 2048)
    x = B.bf16_to_f32(B.syn_bf16(2048, 0, 0, 17, 1.0))
    oi, ow, _ = B.route(B.router_logits_bf16(W, x), 8)
    np.testing.assert_array_equal(idx, oi)
    np.testing.assert_array_equal(w.view(np.uint32), ow.view(np.uint32))
    esz = B.EXPERT_SIZE[4]
    pack = np.zeros(256 * esz, np.uint8)
    for e in oi:
        pack[int(e) * esz:(int(e) + 1) * esz] = B.syn_expert(4, 0, 0, int(e), 0.02)
    want = B.moe_experts(pack, 4, x[None], 8, oi[None], ow[None], np.zeros((1, 2048), np.float32))[0]
    assert_close(got, want, what="C client step")
