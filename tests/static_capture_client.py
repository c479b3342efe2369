"""A fresh process whose FIRST nmoe_moe_layer_static call on the device is
made while the stream is being captured into a HIP graph (global capture
mode: any call that is illegal during capture fails the capture).  The graph
is then replayed several times with new inputs written into the captured
buffers, and each replay is compared bit for bit with nmoe_moe_layer on the
same inputs.  Run by tests/test_zz_no_alloc.py; prints one line per step and
exits non-zero on the first mismatch.

usage: python static_capture_client.py BITS ROUTER(bf16|q4) K
"""
import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "nano-metal-moe-qwen36_amd"))

import nmoe_hip as nh  # noqa: E402
from oracle import binding as B  # noqa: E402

HIP_CAPTURE_GLOBAL = 0
HIP_GRAPH_NODE_KERNEL = 0


def hip():
    nh.lib()  # loads the HIP runtime libnmoe_hip.so links against; the same instance is returned below
    h = C.CDLL("libamdhip64.so.7")
    P, I = C.c_void_p, C.c_int
    sigs = {
        "hipStreamBeginCapture": [P, I],
        "hipStreamEndCapture": [P, C.POINTER(P)],
        "hipGraphInstantiate": [C.POINTER(P), P, P, C.c_char_p, C.c_size_t],
        "hipGraphLaunch": [P, P],
        "hipGraphGetNodes": [P, P, C.POINTER(C.c_size_t)],
        "hipGraphNodeGetType": [P, C.POINTER(I)],
        "hipGraphExecDestroy": [P],
        "hipGraphDestroy": [P],
    }
    for name, args in sigs.items():
        fn = getattr(h, name)
        fn.restype, fn.argtypes = I, args
    return h


def say(msg):
    print(f"[static-capture] {msg}", flush=True)


def main():
    bits, router_kind, k = int(sys.argv[1]), sys.argv[2], int(sys.argv[3])
    hp = hip()
    rng = np.random.default_rng(300 + bits)
    seed, layer = 17, 3
    with nh.Context(0, max_tokens=4) as ctx:
        ctx.synth_layer(layer, bits, seed, 0.02 if bits == 4 else 0.05)
        pack = ctx.layer_pack_ptr(layer)
        if router_kind == "bf16":
            W = B.syn_bf16(256 * 2048, seed, layer, 16, 0.02).reshape(256, 2048)
            r = ctx.router_bf16(ctx.to_device(W))
        else:
            wq = rng.integers(0, 2**32, size=(256, 256), dtype=np.uint64).astype(np.uint32)
            sq = B.f32_to_bf16((rng.standard_normal((256, 32)) * 0.01).astype(np.float32))
            bq = B.f32_to_bf16((rng.standard_normal((256, 32)) * 0.02).astype(np.float32))
            r = ctx.router_q4(ctx.to_device(wq), ctx.to_device(sq), ctx.to_device(bq))
        # the captured call's buffers: new inputs are written into them before each replay
        dx, dh, dsh, dg = ctx.alloc(8192), ctx.alloc(8192), ctx.alloc(8192), ctx.alloc(4)
        out, idx, w = ctx.alloc(8192), ctx.alloc(32), ctx.alloc(32)
        ref_out, ref_idx, ref_w = ctx.alloc(8192), ctx.alloc(32), ctx.alloc(32)
        stream = ctx.stream

        say(f"q{bits} {router_kind} router k={k}: first static call under capture")
        graph = C.c_void_p()
        assert hp.hipStreamBeginCapture(stream, HIP_CAPTURE_GLOBAL) == 0
        rc = nh.moe_layer_static(pack, bits, r, dx, nh.F32, 1, k, dh, out, idx, w, dsh, dg, stream=stream)
        ec = hp.hipStreamEndCapture(stream, C.byref(graph))
        assert rc == nh.OK, f"static call under capture returned {rc}"
        assert ec == 0, f"hipStreamEndCapture: {ec} (a call inside the capture was illegal)"
        n = C.c_size_t(0)
        assert hp.hipGraphGetNodes(graph, None, C.byref(n)) == 0
        nodes = (C.c_void_p * n.value)()
        assert hp.hipGraphGetNodes(graph, nodes, C.byref(n)) == 0
        kinds = []
        for i in range(n.value):
            t = C.c_int(-1)
            assert hp.hipGraphNodeGetType(nodes[i], C.byref(t)) == 0
            kinds.append(t.value)
        assert kinds == [HIP_GRAPH_NODE_KERNEL], f"captured nodes {kinds}: one kernel launch and nothing else"
        exe = C.c_void_p()
        assert hp.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0

        def compare(tag):
            ctx._check(ctx.moe_layer(layer, r, dx, nh.F32, 1, k, dh, ref_out, ref_idx, ref_w, None, dsh, dg))
            ctx.sync()
            assert ctx.device_status() == nh.OK
            got = (out.download(np.float32, 2048), idx.download(np.uint32, 8), w.download(np.float32, 8))
            want = (ref_out.download(np.float32, 2048), ref_idx.download(np.uint32, 8), ref_w.download(np.float32, 8))
            assert np.all(np.isfinite(got[0])), f"{tag}: non-finite output (an expired wait)"
            np.testing.assert_array_equal(got[1], want[1], err_msg=f"{tag}: experts")
            np.testing.assert_array_equal(got[2].view(np.uint32), want[2].view(np.uint32), err_msg=f"{tag}: weights")
            np.testing.assert_array_equal(got[0].view(np.uint32), want[0].view(np.uint32), err_msg=f"{tag}: out")
            say(f"{tag}: experts {list(map(int, got[1][:k]))} equal to nmoe_moe_layer, bit for bit")

        def new_inputs():
            dx.upload(rng.standard_normal(2048).astype(np.float32))
            dh.upload(rng.standard_normal(2048).astype(np.float32))
            dsh.upload(rng.standard_normal(2048).astype(np.float32))
            dg.upload(rng.standard_normal(1).astype(np.float32))
            out.upload(np.full(2048, np.nan, np.float32))

        for rep in range(4):
            new_inputs()
            assert hp.hipGraphLaunch(exe, stream) == 0
            ctx.sync()
            compare(f"replay {rep}")
        # an eager call (the first outside capture: it checks the die placement), then the graph again
        new_inputs()
        rc = nh.moe_layer_static(pack, bits, r, dx, nh.F32, 1, k, dh, out, idx, w, dsh, dg, stream=stream)
        assert rc == nh.OK, rc
        ctx.sync()
        compare("eager call after the replays")
        for rep in range(2):
            new_inputs()
            assert hp.hipGraphLaunch(exe, stream) == 0
            ctx.sync()
            compare(f"replay {4 + rep} after the eager call")
        assert hp.hipGraphExecDestroy(exe) == 0
        assert hp.hipGraphDestroy(graph) == 0
    say("ok")


if __name__ == "__main__":
    main()
