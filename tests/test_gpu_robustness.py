"""The failure path of the persistent kernels, forced from the host.

A fused decode launch needs all 256 of its blocks resident at once; when
one is not, the others' bounded waits give up.  The host forces exactly
that outcome without starving the device: NMOE_HIP_OPT_SKEW_EPOCH moves one
block's launch epoch ahead, so no other block ever sees its words (and it
sees none of theirs), and NMOE_HIP_OPT_SPIN_LIMIT shortens every wait to a
few thousand polls.  Every kernel still runs to its end; the test checks
that the launch reports ETIMEDOUT, that everything it wrote is NaN (no
result from words that never arrived passes for a valid one), and that the
next launch after nmoe_hip_check_device_status is correct again (the
reference's rule that every error path still signals its waiters,
src/runtime.m:2944-2959)."""
import numpy as np
import pytest

from conftest import assert_close
from oracle import binding as B

pytestmark = pytest.mark.gpu

SPIN = 4096  # poll rounds: a few ms per wait instead of about a second


@pytest.fixture(scope="module")
def nh():
    import nmoe_hip
    return nmoe_hip


def _layer_setup(ctx, nh, bits=4, seed=5, layer=3):
    ctx.synth_layer(layer, bits, seed, 0.02)
    W = B.syn_bf16(256 * 2048, seed, layer, 16, 0.02).reshape(256, 2048)
    x = B.bf16_to_f32(B.syn_bf16(2048, seed, layer, 17, 1.0))
    rng = np.random.default_rng(seed)
    h = rng.standard_normal(2048).astype(np.float32)
    idx, w, _ = B.route(B.router_logits_bf16(W, x), 8)
    pack = np.zeros(256 * B.EXPERT_SIZE[bits], np.uint8)
    esz = B.EXPERT_SIZE[bits]
    for e in idx:
        pack[int(e) * esz:(int(e) + 1) * esz] = B.syn_expert(bits, seed, layer, int(e), 0.02)
    want = B.moe_experts(pack, bits, x[None], 8, idx[None], w[None], h[None])[0]
    return dict(W=ctx.to_device(W), x=ctx.to_device(x), h=ctx.to_device(h), idx=idx, w=w, want=want, layer=layer)


def _run(ctx, nh, s, out, di, dw):
    return ctx.moe_layer(s["layer"], ctx.router_bf16(s["W"]), s["x"], nh.F32, 1, 8, s["h"], out, di, dw)


def test_expired_wait_poisons_output_and_recovers(nh):
    with nh.Context(0, max_tokens=4) as ctx:
        s = _layer_setup(ctx, nh)
        out, di, dw = ctx.alloc(2048 * 4), ctx.alloc(32), ctx.alloc(32)
        ctx._check(ctx.set_option(nh.OPT_SPIN_LIMIT, SPIN))
        # a clean launch first
        ctx._check(_run(ctx, nh, s, out, di, dw))
        assert ctx.device_status() == nh.OK
        good = out.download(np.float32, 2048)
        assert_close(good, s["want"], what="before")
        for block in (0, 37, 255):
            print(f"[robust] skewed block {block}", flush=True)
            ctx._check(ctx.set_option(nh.OPT_SKEW_EPOCH, block))
            assert _run(ctx, nh, s, out, di, dw) == nh.OK  # asynchronous: the failure shows at the check
            got = out.download(np.float32, 2048)
            assert np.isnan(got).all(), f"block {block}: {np.count_nonzero(~np.isnan(got))} rows not poisoned"
            assert np.isnan(dw.download(np.float32, 8)).all()
            assert ctx.device_status() == nh.ETIMEDOUT
            assert ctx.device_status() == nh.OK  # the check cleared and realigned
            ctx._check(_run(ctx, nh, s, out, di, dw))
            assert ctx.device_status() == nh.OK
            again = out.download(np.float32, 2048)
            np.testing.assert_array_equal(again.view(np.uint32), good.view(np.uint32))
            np.testing.assert_array_equal(di.download(np.uint32, 8), s["idx"])
        ctx._check(ctx.set_option(nh.OPT_SPIN_LIMIT, 0))


def test_block_expired_wait_poisons_and_recovers(nh):
    """The whole-block form (nmoe_moe_block with the shared expert and the
    next layer's norm): its waits span the shared expert's activations and
    down rows, the combine and the norm's partial sums.  A skewed block --
    a combining block, another block of its chunk, an idle group's block
    (k = 6) -- makes the launch report ETIMEDOUT with out, next_x and the
    weights all NaN, and the next launch gives the clean bits again."""
    with nh.Context(0, max_tokens=4) as ctx:
        seed, layer, k = 31, 5, 6
        ctx.synth_layer(layer, 4, seed, 0.02)
        W = ctx.to_device(B.syn_bf16(256 * 2048, seed, layer, 16, 0.02))
        se = B.syn_shared_expert(13)
        dev = {n: tuple(ctx.to_device(np.ascontiguousarray(a)) for a in se[n]) for n in se}
        blk = nh.MoeBlock()
        blk.router = ctx.router_bf16(W)
        blk.has_shared = 1
        blk.shared = nh.Context.shared_expert_desc(dev["gate"], dev["up"], dev["down"], dev["score"])
        blk.eps = 1e-6
        h = (np.random.default_rng(seed).standard_normal(2048) * 1.5).astype(np.float32)
        dh, out, nx, di, dw = ctx.to_device(h), ctx.alloc(8192), ctx.alloc(8192), ctx.alloc(32), ctx.alloc(32)
        run = lambda: ctx.moe_block(layer, blk, dh, k, out, nx, di, dw)
        ctx._check(ctx.set_option(nh.OPT_SPIN_LIMIT, SPIN))
        try:
            ctx._check(run())
            assert ctx.device_status() == nh.OK
            good = out.download(np.float32, 2048), nx.download(np.float32, 2048), di.download(np.uint32, 8)
            assert np.isfinite(good[0]).all() and np.isfinite(good[1]).all()
            for block in (0, 8 * 5 + 3, 8 * 9 + 7):  # combining (group 0), routed (group 3), idle (group 7)
                print(f"[robust] block form, skewed block {block}", flush=True)
                ctx._check(ctx.set_option(nh.OPT_SKEW_EPOCH, block))
                assert run() == nh.OK
                assert np.isnan(out.download(np.float32, 2048)).all(), f"block {block}: out not poisoned"
                assert np.isnan(nx.download(np.float32, 2048)).all(), f"block {block}: next_x not poisoned"
                assert np.isnan(dw.download(np.float32, 8)[:k]).all()
                assert ctx.device_status() == nh.ETIMEDOUT
                assert ctx.device_status() == nh.OK
                ctx._check(run())
                assert ctx.device_status() == nh.OK
                again = out.download(np.float32, 2048), nx.download(np.float32, 2048), di.download(np.uint32, 8)
                for a, b in zip(again, good):
                    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
        finally:
            ctx.set_option(nh.OPT_SPIN_LIMIT, 0)


def test_sync_check_returns_etimedout(nh):
    """With NMOE_HIP_OPT_SYNC_CHECK the layer call itself reports the
    expired wait, and the stack reports it once, after its last layer; the
    stack's poisoned layers feed NaN forward (no layer after the failure
    produces numbers)."""
    with nh.Context(0, max_tokens=4) as ctx:
        s = _layer_setup(ctx, nh)
        out, di, dw = ctx.alloc(2048 * 4), ctx.alloc(32), ctx.alloc(32)
        ctx._check(ctx.set_option(nh.OPT_SPIN_LIMIT, SPIN))
        ctx._check(ctx.set_option(nh.OPT_SYNC_CHECK, 1))
        ctx._check(_run(ctx, nh, s, out, di, dw))
        ctx._check(ctx.set_option(nh.OPT_SKEW_EPOCH, 100))
        assert _run(ctx, nh, s, out, di, dw) == nh.ETIMEDOUT
        assert np.isnan(out.download(np.float32, 2048)).all()
        ctx._check(_run(ctx, nh, s, out, di, dw))  # realigned by the failed call's check
        assert_close(out.download(np.float32, 2048), s["want"], what="after sync-check recovery")
        # the stack: three layers over the same pack, failure from the first
        nl = 3
        rng = np.random.default_rng(9)
        h0 = rng.standard_normal(2048).astype(np.float32)
        h_seq = ctx.alloc((nl + 1) * 2048 * 4)
        h_seq.upload(h0)
        r = ctx.router_bf16(s["W"])
        ctx._check(ctx.set_option(nh.OPT_SKEW_EPOCH, 200))
        assert ctx.moe_stack([s["layer"]] * nl, [r] * nl, 8, 1e-6, h_seq) == nh.ETIMEDOUT
        hs = h_seq.download(np.float32, (nl + 1, 2048))
        np.testing.assert_array_equal(hs[0], h0)
        assert np.isnan(hs[1:]).all()
        ctx._check(ctx.moe_stack([s["layer"]] * nl, [r] * nl, 8, 1e-6, h_seq))
        hs = h_seq.download(np.float32, (nl + 1, 2048))
        assert np.isfinite(hs).all()
        ctx._check(ctx.set_option(nh.OPT_SYNC_CHECK, 0))
        ctx._check(ctx.set_option(nh.OPT_SPIN_LIMIT, 0))


def test_grouped_one_launch_wrong_tile_count_poisons_and_recovers(nh):
    """The one-launch grouped form: a down tile checks that its expert's
    gate/up tiles are all counted, each from this block's die.  With the
    count of expert rank 0 started at an impossible value
    (NMOE_HIP_OPT_SKEW_TILES), its down tiles find it wrong: the call's
    outputs are NaN and the status reports ETIMEDOUT; the next call is the
    same bits as the two-launch form's."""
    rng = np.random.default_rng(77)
    ntok, k, layer, bits = 64, 8, 4, 4
    with nh.Context(0, max_tokens=ntok) as ctx:
        if not ctx.set_grouped_one_launch(True):
            pytest.skip("the one-launch form needs the round-robin die placement")
        ctx.synth_layer(layer, bits, 11, 0.02)
        idx = np.zeros((ntok, 8), np.uint32)
        for t in range(ntok):
            idx[t, :k] = rng.choice(256, k, replace=False)
        idx[:40, 0] = 7  # rank 0: expert 7 with 40 entries
        w = rng.dirichlet(np.ones(k), size=ntok).astype(np.float32)
        x = rng.standard_normal((ntok, 2048)).astype(np.float32)
        h = rng.standard_normal((ntok, 2048)).astype(np.float32)
        d = [ctx.to_device(a) for a in (x, idx, w, h)]
        out = ctx.alloc(ntok * 2048 * 4)

        def run():
            ctx._check(ctx.experts(bits, layer, d[0], nh.F32, ntok, k, d[1], d[2], d[3], out))
            return out.download(np.float32, (ntok, 2048))

        ctx.set_grouped_one_launch(False)
        want = run()
        assert ctx.device_status() == nh.OK
        ctx.set_grouped_one_launch(True)
        np.testing.assert_array_equal(run().view(np.uint32), want.view(np.uint32))
        assert ctx.device_status() == nh.OK
        ctx._check(ctx.set_option(nh.OPT_SKEW_TILES, 0))
        bad = run()
        assert ctx.device_status() == nh.ETIMEDOUT
        assert np.isnan(bad).all()
        np.testing.assert_array_equal(run().view(np.uint32), want.view(np.uint32))
        assert ctx.device_status() == nh.OK
        assert ctx.set_option(nh.OPT_SKEW_TILES, 256) == nh.EINVAL


def test_grouped_routed_after_aborted_launch(nh):
    """The routed preparation tags each entry with its launch's epoch, a
    device counter that one block advances per launch.  After a launch that
    is aborted (here its one-launch GEMM, through NMOE_HIP_OPT_SKEW_TILES:
    NaN outputs, ETIMEDOUT), the recovery moves the counter past any epoch
    that launch's entries can carry; the calls after it, each with new
    logits, give the same routing and outputs as the two-launch form on a
    context that never failed."""
    rng = np.random.default_rng(78)
    ntok, k, layer, bits = 64, 8, 5, 4
    calls = [(rng.random((ntok, 256), dtype=np.float32), rng.standard_normal((ntok, 2048)).astype(np.float32),
              rng.standard_normal((ntok, 2048)).astype(np.float32)) for _ in range(4)]

    def run_all(ctx, skew_before):
        ctx.synth_layer(layer, bits, 12, 0.02)
        out, idx, w = ctx.alloc(ntok * 8192), ctx.alloc(ntok * 32), ctx.alloc(ntok * 32)
        res = []
        for i, (lg, x, h) in enumerate(calls):
            if i == skew_before:
                ctx._check(ctx.set_option(nh.OPT_SKEW_TILES, 0))
                d = [ctx.to_device(a) for a in (lg, x, h)]
                ctx._check(ctx.experts_from_logits(layer, d[0], d[1], nh.F32, ntok, k, d[2], out, idx, w))
                assert ctx.device_status() == nh.ETIMEDOUT
                assert np.isnan(out.download(np.float32, (ntok, 2048))).all()
            d = [ctx.to_device(a) for a in (lg, x, h)]
            ctx._check(ctx.experts_from_logits(layer, d[0], d[1], nh.F32, ntok, k, d[2], out, idx, w))
            assert ctx.device_status() == nh.OK
            res.append((idx.download(np.uint32, (ntok, 8)), w.download(np.float32, (ntok, 8)),
                        out.download(np.float32, (ntok, 2048))))
        return res

    with nh.Context(0, max_tokens=ntok) as ctx:
        ctx.set_grouped_one_launch(False)
        want = run_all(ctx, -1)
    with nh.Context(0, max_tokens=ntok) as ctx:
        if not ctx.set_grouped_one_launch(True):
            pytest.skip("the one-launch form needs the round-robin die placement")
        got = run_all(ctx, 1)
    for i, (g, e) in enumerate(zip(got, want)):
        for a, b, name in zip(g, e, ("idx", "w", "out")):
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg=f"call {i}: {name}")


def test_option_arguments_validated(nh):
    with nh.Context(0, max_tokens=4) as ctx:
        assert ctx.set_option(nh.OPT_SPIN_LIMIT, -1) == nh.EINVAL
        assert ctx.set_option(nh.OPT_SPIN_LIMIT, (1 << 26) + 1) == nh.EINVAL
        assert ctx.set_option(nh.OPT_SKEW_EPOCH, 256) == nh.EINVAL
        assert ctx.set_option(nh.OPT_SKEW_EPOCH, -1) == nh.EINVAL
        assert ctx.set_option(99, 0) == nh.EINVAL


def test_repeated_launches_bit_identical(nh):
    """Every launch form, run 100 times on the same inputs, gives the same
    bits each time: the fused single-token layer, the grouped 64-token
    layer, the layer loop in both forms (one launch per token, one per layer)
    and the block form with its shared expert and next-layer norm.  A late
    or lost word in the inter-block exchanges, or an epoch counter that
    does not reset between launches, would show here as a changed bit."""
    with nh.Context(0, max_tokens=64) as ctx:
        seed, k, nl, ni = 5, 8, 4, 8
        for l in range(nl):
            ctx.synth_layer(l, 4, seed, 0.02)
        R = ctx.alloc(nl * 256 * 4096)
        for l in range(nl):
            ctx.synth_bf16(R, 256 * 2048, seed, l, 16, 0.02, offset=l * 256 * 4096)
        rts = [ctx.router_bf16(R.ptr + l * 256 * 4096) for l in range(nl)]
        X, hb = ctx.alloc(64 * 4096), ctx.alloc(64 * 4096)
        ctx.synth_bf16(X, 64 * 2048, seed, 0, 17, 1.0)
        ctx.synth_bf16(hb, 64 * 2048, seed, 0, 18, 1.0)
        h = (hb.download(np.uint16, (64, 2048)).astype(np.uint32) << 16).view(np.float32)
        H = ctx.to_device(h)
        o1, i1, w1 = ctx.alloc(ni * 8192), ctx.alloc(ni * 32), ctx.alloc(ni * 32)
        og, ig, wg = ctx.alloc(64 * 8192), ctx.alloc(64 * 32), ctx.alloc(64 * 32)
        row = (nl + 1) * 8192
        HS, IS, WS = ctx.alloc(ni * row), ctx.alloc(ni * nl * 32), ctx.alloc(ni * nl * 32)
        se = B.syn_shared_expert(13)
        dev = {n: tuple(ctx.to_device(np.ascontiguousarray(a)) for a in se[n]) for n in se}
        blk = nh.MoeBlock()
        blk.router, blk.has_shared, blk.eps = rts[1], 1, 1e-6
        blk.shared = nh.Context.shared_expert_desc(dev["gate"], dev["up"], dev["down"], dev["score"])
        nrm = ctx.to_device(B.f32_to_bf16((np.random.default_rng(seed).standard_normal(2048) * 0.1).astype(np.float32)))
        blk.post_norm, blk.next_norm, blk.add_one = nrm.ptr, nrm.ptr, 1
        ob, nb, ib, wb = ctx.alloc(ni * 8192), ctx.alloc(ni * 8192), ctx.alloc(ni * 32), ctx.alloc(ni * 32)

        def c1():
            for i in range(ni):
                ctx._check(ctx.moe_layer(i % nl, rts[i % nl], X.ptr + i * 4096, nh.BF16, 1, k, H.ptr + i * 8192,
                                         o1.ptr + i * 8192, i1.ptr + i * 32, w1.ptr + i * 32))
            return o1, i1, w1

        def grouped():
            ctx._check(ctx.moe_layer(2, rts[2], X, nh.BF16, 64, k, H, og, ig, wg))
            return og, ig, wg

        def stack(loop):
            ctx._check(ctx.set_option(nh.OPT_STACK_LOOP, loop))
            for t in range(ni):
                HS.upload(h[t], offset=t * row)
            for t in range(ni):
                ctx._check(ctx.moe_stack(list(range(nl)), rts, k, 1e-6, HS.ptr + t * row, IS.ptr + t * nl * 32,
                                         WS.ptr + t * nl * 32))
            return HS, IS, WS

        def block():
            for i in range(ni):
                ctx._check(ctx.moe_block(1, blk, H.ptr + i * 8192, k, ob.ptr + i * 8192, nb.ptr + i * 8192,
                                         ib.ptr + i * 32, wb.ptr + i * 32))
            return ob, nb, ib, wb

        forms = {"fused layer": c1, "grouped layer": grouped, "stack, one launch per token": lambda: stack(1),
                 "stack, one launch per layer": lambda: stack(0), "block": block}
        try:
            for name, f in forms.items():
                first = [b.download(np.uint32, b.nbytes // 4) for b in f()]
                assert ctx.device_status() == nh.OK
                assert all(np.isfinite(a.view(np.float32)).all() for a in first), name
                print(f"[robust] repeated launches: {name}", flush=True)
                for r in range(100):
                    got = [b.download(np.uint32, b.nbytes // 4) for b in f()]
                    for j, (a, b) in enumerate(zip(got, first)):
                        assert np.array_equal(a, b), f"{name}: repeat {r}, output {j} changed in {int((a != b).sum())} words"
                assert ctx.device_status() == nh.OK
        finally:
            ctx.set_option(nh.OPT_STACK_LOOP, 1)
