"""The context's entry points captured into HIP graphs and replayed, as a
serving loop would: nmoe_moe_experts_from_logits (the grouped path, with
gate/up and down in one launch and in two, and with two pass lanes) and
nmoe_moe_layer (the fused single-token launch).  Capture is global-mode, so
any call illegal under capture fails it; every captured node must be a
kernel (no memset or copy nodes).  Each replay runs on new inputs written
into the captured buffers, with eager calls of the same entry point in
between, and must equal the eager call on the same inputs bit for bit
(routing, weights and outputs): the launches keep no state that a replay
would repeat (epochs, counters and schedule words are counted or cleared on
the device)."""
import ctypes as C

import numpy as np
import pytest

from oracle import binding as B
from static_capture_client import HIP_CAPTURE_GLOBAL, HIP_GRAPH_NODE_KERNEL, hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nh():
    import nmoe_hip
    return nmoe_hip


class Graph:
    """One capture of fn() on the context's stream, instantiated."""

    def __init__(self, hp, stream, fn):
        self.hp, self.stream = hp, stream
        self.graph, self.exe = C.c_void_p(), C.c_void_p()
        assert hp.hipStreamBeginCapture(stream, HIP_CAPTURE_GLOBAL) == 0
        rc = fn()
        ec = hp.hipStreamEndCapture(stream, C.byref(self.graph))
        assert rc == 0, f"call under capture returned {rc}"
        assert ec == 0, f"hipStreamEndCapture: {ec} (a call inside the capture was illegal)"
        n = C.c_size_t(0)
        assert hp.hipGraphGetNodes(self.graph, None, C.byref(n)) == 0
        nodes = (C.c_void_p * n.value)()
        assert hp.hipGraphGetNodes(self.graph, nodes, C.byref(n)) == 0
        self.kinds = []
        for i in range(n.value):
            t = C.c_int(-1)
            assert hp.hipGraphNodeGetType(nodes[i], C.byref(t)) == 0
            self.kinds.append(t.value)
        assert self.kinds and all(t == HIP_GRAPH_NODE_KERNEL for t in self.kinds), f"captured nodes {self.kinds}"
        assert hp.hipGraphInstantiate(C.byref(self.exe), self.graph, None, None, 0) == 0

    def launch(self):
        assert self.hp.hipGraphLaunch(self.exe, self.stream) == 0

    def close(self):
        assert self.hp.hipGraphExecDestroy(self.exe) == 0
        assert self.hp.hipGraphDestroy(self.graph) == 0


def _same(got, want, what):
    for g, w, name in zip(got, want, ("idx", "w", "out")):
        np.testing.assert_array_equal(g.view(np.uint32), w.view(np.uint32), err_msg=f"{what}: {name}")


@pytest.mark.parametrize("bits,ntok,one", [(4, 64, True), (4, 64, False), (2, 64, True), (4, 1200, True)])
def test_grouped_from_logits_graph_replays(nh, bits, ntok, one):
    """64 tokens: one pass lane (gate/up and down in one launch, or in two);
    1200 tokens: two pass lanes and 8 dispatch slices (two launches)."""
    hp = hip()
    k, layer = 8, 6
    rng = np.random.default_rng(900 + bits + ntok)
    with nh.Context(0, max_tokens=ntok) as ctx:
        if one and not ctx.set_grouped_one_launch(True):
            pytest.skip("the one-launch form needs the round-robin die placement")
        if not one:
            ctx.set_grouped_one_launch(False)
        ctx.synth_layer(layer, bits, 23, 0.02 if bits == 4 else 0.05)
        d_lg, d_x, d_h = ctx.alloc(ntok * 1024), ctx.alloc(ntok * 4096), ctx.alloc(ntok * 8192)
        g_out, g_idx, g_w = ctx.alloc(ntok * 8192), ctx.alloc(ntok * 32), ctx.alloc(ntok * 32)
        e_out, e_idx, e_w = ctx.alloc(ntok * 8192), ctx.alloc(ntok * 32), ctx.alloc(ntok * 32)
        s = ctx.stream

        def call(out, idx, w):
            return ctx.experts_from_logits(layer, d_lg, d_x, nh.BF16, ntok, k, d_h, out, idx, w, stream=s)

        def new_inputs():
            d_lg.upload(rng.random((ntok, 256), dtype=np.float32))
            d_x.upload(B.f32_to_bf16(rng.standard_normal((ntok, 2048)).astype(np.float32)))
            d_h.upload(rng.standard_normal((ntok, 2048)).astype(np.float32))
            g_out.upload(np.full(ntok * 2048, np.nan, np.float32))

        def read(out, idx, w):
            return (idx.download(np.uint32, (ntok, 8)), w.download(np.float32, (ntok, 8)),
                    out.download(np.float32, (ntok, 2048)))

        new_inputs()
        ctx._check(call(e_out, e_idx, e_w))  # an eager call first, then the capture
        ctx.sync()
        g = Graph(hp, s, lambda: call(g_out, g_idx, g_w))
        print(f"[graph] q{bits} ntok={ntok} one={one}: {len(g.kinds)} kernel nodes", flush=True)
        try:
            for rep in range(5):
                new_inputs()
                g.launch()
                if rep % 2 == 1:  # eager work of the program between replays
                    ctx._check(call(e_out, e_idx, e_w))
                ctx.sync()
                assert ctx.device_status() == nh.OK
                got = read(g_out, g_idx, g_w)
                ctx._check(call(e_out, e_idx, e_w))
                ctx.sync()
                _same(got, read(e_out, e_idx, e_w), f"replay {rep}")
                assert np.isfinite(got[2]).all()
        finally:
            g.close()
            ctx.set_grouped_one_launch(True)


@pytest.mark.parametrize("bits", [4, 2])
def test_fused_layer_graph_replays(nh, bits):
    """nmoe_moe_layer (one token: the fused launch, routing from the bf16
    router) captured once and replayed with new x and h; each launch takes a
    new epoch on the device, so no replay can accept the words of the one
    before."""
    hp = hip()
    k, layer, seed = 8, 3, 31
    rng = np.random.default_rng(40 + bits)
    with nh.Context(0, max_tokens=4) as ctx:
        ctx.synth_layer(layer, bits, seed, 0.02 if bits == 4 else 0.05)
        W = B.syn_bf16(256 * 2048, seed, layer, 16, 0.02).reshape(256, 2048)
        r = ctx.router_bf16(ctx.to_device(W))
        dx, dh = ctx.alloc(8192), ctx.alloc(8192)
        g_out, g_idx, g_w = ctx.alloc(8192), ctx.alloc(32), ctx.alloc(32)
        e_out, e_idx, e_w = ctx.alloc(8192), ctx.alloc(32), ctx.alloc(32)
        s = ctx.stream

        def call(out, idx, w):
            return ctx.moe_layer(layer, r, dx, nh.F32, 1, k, dh, out, idx, w, stream=s)

        def read(out, idx, w):
            return idx.download(np.uint32, 8), w.download(np.float32, 8), out.download(np.float32, 2048)

        g = Graph(hp, s, lambda: call(g_out, g_idx, g_w))
        try:
            for rep in range(6):
                dx.upload(rng.standard_normal(2048).astype(np.float32))
                dh.upload(rng.standard_normal(2048).astype(np.float32))
                g_out.upload(np.full(2048, np.nan, np.float32))
                g.launch()
                if rep % 2 == 0:
                    ctx._check(call(e_out, e_idx, e_w))
                ctx.sync()
                assert ctx.device_status() == nh.OK
                got = read(g_out, g_idx, g_w)
                ctx._check(call(e_out, e_idx, e_w))
                ctx.sync()
                _same(got, read(e_out, e_idx, e_w), f"q{bits} replay {rep}")
        finally:
            g.close()
