"""The CPU baseline routines bench.py times (oracle/cpu_step.c), on the CPU:
the per-token form with given logits (the batched-decode and prefill
configs) against the oracle's routing and expert path, the 40-layer-stack
form against the same decode step applied layer by layer, and, where the
reference's src/math.m was compiled into oracle/_ref, the reference build
against the restatement bit for bit."""
import ctypes as C

import numpy as np
import pytest

from conftest import assert_close
from oracle import binding as B


@pytest.fixture(scope="module")
def layers():
    esz = B.EXPERT_SIZE[2]
    out = []
    for l in range(2):
        p = np.empty(256 * esz, np.uint8)
        for e in range(256):
            p[e * esz:(e + 1) * esz] = B.syn_expert(2, 7, l, e, 0.05)
        out.append(p)
    return out


def _tokens(ntok, seed):
    rng = np.random.default_rng(seed)
    lg = rng.random((ntok, 256), dtype=np.float32)
    x = rng.standard_normal((ntok, 2048)).astype(np.float32)
    h = rng.standard_normal((ntok, 2048)).astype(np.float32)
    return lg, x, h


@pytest.mark.parametrize("k", [8, 6])
def test_tokens_bench_matches_oracle(layers, k):
    """The last token's output equals the oracle's route + experts + combine
    on the same logits (routing decided by math.m's softmax / top-k)."""
    ntok = 3
    lg, x, h = _tokens(ntok, 11 + k)
    out = np.zeros(2048, np.float32)
    sec = B.oracle().orc_cpu_tokens_bench_port(layers[0].ctypes.data, 2, lg.ctypes.data, x.ctypes.data,
                                               h.ctypes.data, ntok, k, 1, out.ctypes.data)
    assert sec > 0
    idx, w, n = B.route(lg[-1], k)
    want = B.moe_experts(layers[0], 2, x[-1:], k, idx[None], w[None], h[-1:])[0]
    assert_close(out, want, what="tokens bench, last token")


def test_stack_bench_is_the_layer_loop(layers):
    """h after nl layers (pack and router l % npacks) equals the decode step
    applied layer by layer to x = RMSNorm(h)."""
    nl, k, eps = 3, 8, 1e-6
    routers = [B.syn_bf16(256 * 2048, 7, l, 16, 0.02) for l in range(2)]
    h0 = np.random.default_rng(5).standard_normal((1, 2048)).astype(np.float32)
    pp = (C.c_void_p * 2)(*[p.ctypes.data for p in layers])
    rp = (C.c_void_p * 2)(*[r.ctypes.data for r in routers])
    got = np.zeros(2048, np.float32)
    B.oracle().orc_cpu_stack_bench_port(pp, rp, 2, nl, 2, h0.ctypes.data, 1, k, eps, 1, got.ctypes.data)
    h = h0[0].copy()
    o = B.oracle()
    for l in range(nl):
        x = np.zeros(2048, np.float32)
        o.orc_rms_norm(h.ctypes.data, None, x.ctypes.data, 2048, eps, 0)
        out = np.zeros(2048, np.float32)
        idx, w = np.zeros(8, np.uint32), np.zeros(8, np.float32)
        o.orc_cpu_step_port(layers[l % 2].ctypes.data, 2, routers[l % 2].ctypes.data, x.ctypes.data, k, h.ctypes.data,
                            out.ctypes.data, idx.ctypes.data, w.ctypes.data)
        h = out
    np.testing.assert_array_equal(got.view(np.uint32), h.view(np.uint32))


def test_reference_build_equals_port(layers):
    """oracle/_ref's build (the reference's own math.m) gives the same bits
    as the restatement in every baseline routine."""
    ref = B.ref_step()
    if ref is None:
        pytest.skip("oracle/_ref was not built (no reference sources)")
    o = B.oracle()
    ntok, k = 2, 8
    lg, x, h = _tokens(ntok, 3)
    a, b = np.zeros(2048, np.float32), np.zeros(2048, np.float32)
    o.orc_cpu_tokens_bench_port(layers[1].ctypes.data, 2, lg.ctypes.data, x.ctypes.data, h.ctypes.data, ntok, k, 1,
                                a.ctypes.data)
    ref.orc_cpu_tokens_bench_ref(layers[1].ctypes.data, 2, lg.ctypes.data, x.ctypes.data, h.ctypes.data, ntok, k, 1,
                                 b.ctypes.data)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    routers = [B.syn_bf16(256 * 2048, 7, l, 16, 0.02) for l in range(2)]
    pp = (C.c_void_p * 2)(*[p.ctypes.data for p in layers])
    rp = (C.c_void_p * 2)(*[r.ctypes.data for r in routers])
    o.orc_cpu_stack_bench_port(pp, rp, 2, 2, 2, h.ctypes.data, 1, k, 1e-6, 1, a.ctypes.data)
    ref.orc_cpu_stack_bench_ref(pp, rp, 2, 2, 2, h.ctypes.data, 1, k, 1e-6, 1, b.ctypes.data)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
