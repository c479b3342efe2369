"""nmoe_moe_layer_static (the per-layer call that allocates nothing, its
scratch a fixed device array) against nmoe_moe_layer, through the C ABI:
two calls in a row, the second with fewer tokens, each compared with the
context entry point on the same inputs -- routing bit-exact, outputs within
max-abs 2e-3 / rel-L2 1e-3 (here they are the same kernels, so also equal)."""
import os
import subprocess
import sys

import numpy as np
import pytest

from conftest import assert_close
from oracle import binding as B

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nh():
    import nmoe_hip
    return nmoe_hip


@pytest.mark.parametrize("bits,router", [(4, "bf16"), (2, "q4")])
def test_static_layer_matches_context_layer(nh, bits, router):
    rng = np.random.default_rng(90 + bits)
    seed, layer, k = 61, 5, 8 if bits == 4 else 6
    with nh.Context(0, max_tokens=16) as ctx:
        ctx.synth_layer(layer, bits, seed, 0.02 if bits == 4 else 0.05)
        pack = ctx.layer_pack_ptr(layer)
        if router == "bf16":
            W = B.syn_bf16(256 * 2048, seed, layer, 16, 0.02).reshape(256, 2048)
            r = ctx.router_bf16(ctx.to_device(W))
        else:
            wq = rng.integers(0, 2**32, size=(256, 256), dtype=np.uint64).astype(np.uint32)
            sq = B.f32_to_bf16((rng.standard_normal((256, 32)) * 0.01).astype(np.float32))
            bq = B.f32_to_bf16((rng.standard_normal((256, 32)) * 0.02).astype(np.float32))
            r = ctx.router_q4(ctx.to_device(wq), ctx.to_device(sq), ctx.to_device(bq))
        for ntok in (5, 1, 3):  # each call after the first is smaller than the one before it or than the first
            print(f"[no-alloc] q{bits} {router} router ntok={ntok}", flush=True)
            x = rng.standard_normal((ntok, 2048)).astype(np.float32)
            h = rng.standard_normal((ntok, 2048)).astype(np.float32)
            sh = rng.standard_normal((ntok, 2048)).astype(np.float32)
            g = rng.standard_normal(ntok).astype(np.float32)
            dx, dh, dsh, dg = ctx.to_device(x), ctx.to_device(h), ctx.to_device(sh), ctx.to_device(g)
            outs = {}
            for path in ("context", "static"):
                out, idx, w = ctx.alloc(ntok * 8192), ctx.alloc(ntok * 32), ctx.alloc(ntok * 32)
                if path == "context":
                    ctx._check(ctx.moe_layer(layer, r, dx, nh.F32, ntok, k, dh, out, idx, w, None, dsh, dg))
                else:
                    rc = nh.moe_layer_static(pack, bits, r, dx, nh.F32, ntok, k, dh, out, idx, w, dsh, dg,
                                             stream=ctx.stream)
                    assert rc == nh.OK, rc
                ctx.sync()
                outs[path] = (out.download(np.float32, (ntok, 2048)), idx.download(np.uint32, (ntok, 8)),
                              w.download(np.float32, (ntok, 8)))
            assert ctx.device_status() == nh.OK
            (oc, ic, wc), (os_, is_, ws) = outs["context"], outs["static"]
            np.testing.assert_array_equal(is_, ic)
            np.testing.assert_array_equal(ws.view(np.uint32), wc.view(np.uint32))
            assert_close(os_, oc, what=f"static vs context ntok={ntok}")
            np.testing.assert_array_equal(os_.view(np.uint32), oc.view(np.uint32))


def test_static_layer_rejects_bad_arguments(nh):
    with nh.Context(0, max_tokens=4) as ctx:
        ctx.synth_layer(0, 4, 1, 0.02)
        pack = ctx.layer_pack_ptr(0)
        W = ctx.to_device(B.syn_bf16(256 * 2048, 1, 0, 16, 0.02))
        r = ctx.router_bf16(W)
        x, h, out = ctx.alloc(17 * 8192), ctx.alloc(17 * 8192), ctx.alloc(17 * 8192)
        mx = nh.STATIC_MAX_TOKENS
        assert nh.moe_layer_static(pack, 4, r, x, nh.F32, mx + 1, 8, h, out) == nh.EINVAL  # beyond the scratch
        assert nh.moe_layer_static(pack, 4, r, x, nh.F32, 0, 8, h, out) == nh.EINVAL
        assert nh.moe_layer_static(pack, 4, r, x, nh.F32, 1, 9, h, out) == nh.EINVAL
        assert nh.moe_layer_static(pack, 3, r, x, nh.F32, 1, 8, h, out) == nh.EINVAL
        assert nh.moe_layer_static(None, 4, r, x, nh.F32, 1, 8, h, out) == nh.EINVAL
        assert nh.moe_layer_static(pack, 4, r, x, nh.F32, 1, 8, None, out) == nh.EINVAL
        assert nh.moe_layer_static(pack, 4, r, x, nh.F32, 1, 8, h, out, shared_out=h) == nh.EINVAL
        r_bad = nh.Context.router_bf16(W, num_experts=128)
        assert nh.moe_layer_static(pack, 4, r_bad, x, nh.F32, 1, 8, h, out) == nh.EINVAL


@pytest.mark.parametrize("bits,router,k", [(4, "bf16", 8), (2, "q4", 6)])
def test_static_layer_first_call_under_graph_capture(bits, router, k):
    """The first call on the device made inside hipStreamBeginCapture (global
    mode) captures one kernel node and nothing else; four replays with new
    inputs, an eager call, and two more replays each equal nmoe_moe_layer bit
    for bit (each replay takes a new epoch on the device, so no replay can
    accept the previous one's exchange words).  A fresh process, so that the
    call under capture is the first on the device."""
    client = os.path.join(os.path.dirname(os.path.abspath(__file__)), "static_capture_client.py")
    print(f"[no-alloc] capture client q{bits} {router} k={k}", flush=True)
    r = subprocess.run([sys.executable, "-u", client, str(bits), router, str(k)], capture_output=True, text=True,
                       timeout=110)
    print(r.stdout[-4000:], r.stderr[-4000:], flush=True)
    assert r.returncode == 0, f"capture client exited {r.returncode}"
    assert "[static-capture] ok" in r.stdout
