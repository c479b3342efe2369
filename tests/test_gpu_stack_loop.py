"""nmoe_moe_stack's persistent form: all layers of one token in one launch
(the layer loop of NMOEProcessToken, src/runtime.m:3732-3777, restricted to
the MoE tails, with the next layer's input RMSNorm, runtime.m:2893-2900).

Checked against the oracle layer by layer (teacher-forced: routing
bit-exact, outputs within max-abs 2e-3 / rel-L2 1e-3), and against the
one-launch-per-layer form bit for bit (hidden states, routing, weights):
bf16 and q4 routers, q4 and q2 packs, top-8 and top-6 (two idle groups),
more layers than one launch holds, and a forced bounded-wait expiry with
its recovery."""
import numpy as np
import pytest

from conftest import assert_close
from oracle import binding as B

pytestmark = pytest.mark.gpu

SIGMA = {4: 0.02, 2: 0.05}
SPIN = 4096


@pytest.fixture(scope="module")
def nh():
    import nmoe_hip
    return nmoe_hip


@pytest.fixture(scope="module")
def ctx(nh):
    c = nh.Context(0, max_tokens=8)
    yield c
    c.close()


def _routers(ctx, kind, layers, seed):
    """(device routers, host weights) for each layer."""
    rng = np.random.default_rng(seed)
    dev, host = [], []
    for layer in layers:
        if kind == "bf16":
            W = B.syn_bf16(256 * 2048, seed, layer, 16, 0.02).reshape(256, 2048)
            dev.append(ctx.router_bf16(ctx.to_device(W)))
            host.append({"w": W})
        else:
            wq = rng.integers(0, 2**32, size=(256, 256), dtype=np.uint64).astype(np.uint32)
            sq = B.f32_to_bf16((rng.standard_normal((256, 32)) * 0.01).astype(np.float32))
            bq = B.f32_to_bf16((rng.standard_normal((256, 32)) * 0.02).astype(np.float32))
            dev.append(ctx.router_q4(ctx.to_device(wq), ctx.to_device(sq), ctx.to_device(bq)))
            host.append({"q4": (wq, sq, bq)})
    return dev, host


def _pack(bits, seed, layer, experts):
    """Host layer with only `experts` generated (the others never read)."""
    esz = B.EXPERT_SIZE[bits]
    pack = np.zeros(B.EXPERTS * esz, np.uint8)
    for e in sorted(set(int(v) for v in experts)):
        pack[e * esz:(e + 1) * esz] = B.syn_expert(bits, seed, layer, e, SIGMA[bits])
    return pack


def _run(ctx, nh, loop, layers, routers, k, h0):
    nl = len(layers)
    ctx._check(ctx.set_option(nh.OPT_STACK_LOOP, int(loop)))
    hs, idx_s, w_s = ctx.alloc((nl + 1) * 8192), ctx.alloc(nl * 32), ctx.alloc(nl * 32)
    hs.upload(h0)
    rc = ctx.moe_stack(layers, routers, k, 1e-6, hs, idx_s, w_s)
    ctx.sync()
    out = (hs.download(np.float32, (nl + 1, 2048)), idx_s.download(np.uint32, (nl, 8)),
           w_s.download(np.float32, (nl, 8)))
    ctx._check(ctx.set_option(nh.OPT_STACK_LOOP, 1))
    return rc, out


def _same(a, b):
    np.testing.assert_array_equal(a[0].view(np.uint32), b[0].view(np.uint32), err_msg="hidden states")
    np.testing.assert_array_equal(a[1], b[1], err_msg="routing")
    np.testing.assert_array_equal(a[2].view(np.uint32), b[2].view(np.uint32), err_msg="weights")


@pytest.mark.parametrize("bits,kind,k", [(4, "bf16", 8), (4, "q4", 8), (2, "bf16", 6), (2, "q4", 8), (4, "bf16", 6)])
def test_stack_loop_against_oracle_and_per_layer(ctx, nh, bits, kind, k):
    seed, nl = 41 + bits, 5
    layers = [20 + 6 * (bits == 2) + i for i in range(nl)]
    print(f"[stack-loop] q{bits} {kind} router k={k}", flush=True)
    for layer in layers:
        ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    routers, host = _routers(ctx, kind, layers, seed)
    h0 = B.bf16_to_f32(B.syn_bf16(2048, seed, 99, 18, 1.0))
    rc, got = _run(ctx, nh, True, layers, routers, k, h0)
    assert rc == nh.OK and ctx.device_status() == nh.OK
    rc, per_layer = _run(ctx, nh, False, layers, routers, k, h0)
    assert rc == nh.OK and ctx.device_status() == nh.OK
    _same(got, per_layer)
    H, I, Wt = got
    np.testing.assert_array_equal(H[0], h0)
    for l in (0, nl - 1):  # teacher-forced on the GPU's own input
        pack = _pack(bits, seed, layers[l], I[l][:k])
        want, oi, ow, _, _ = B.moe_block(pack, bits, host[l], H[l], k)
        np.testing.assert_array_equal(I[l][:k], oi[:k], err_msg=f"layer {l}")
        np.testing.assert_array_equal(Wt[l].view(np.uint32), ow.view(np.uint32), err_msg=f"layer {l}")
        assert_close(H[l + 1], want, what=f"layer {l}")


def test_stack_loop_more_layers_than_one_launch(ctx, nh):
    """70 layer entries over 5 resident packs: two launches (64 + 6)."""
    bits, seed, k = 4, 53, 8
    res = [30 + i for i in range(5)]
    for layer in res:
        ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    routers5, _ = _routers(ctx, "bf16", res, seed)
    layers = [res[i % 5] for i in range(70)]
    routers = [routers5[i % 5] for i in range(70)]
    h0 = B.bf16_to_f32(B.syn_bf16(2048, seed, 98, 18, 1.0))
    rc, got = _run(ctx, nh, True, layers, routers, k, h0)
    assert rc == nh.OK and ctx.device_status() == nh.OK
    rc, per_layer = _run(ctx, nh, False, layers, routers, k, h0)
    assert rc == nh.OK and ctx.device_status() == nh.OK
    _same(got, per_layer)
    assert np.isfinite(got[0]).all()


def test_stack_loop_expired_wait_poisons_and_recovers(ctx, nh):
    """One block's epoch forced a launch ahead (from the host): the stack's
    bounded waits give up, the status reports it, every hidden state the
    launch writes is NaN, and after nmoe_hip_check_device_status the next
    stack is correct again."""
    bits, seed, k, nl = 4, 59, 8, 3
    layers = [40 + i for i in range(nl)]
    for layer in layers:
        ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    routers, _ = _routers(ctx, "bf16", layers, seed)
    h0 = B.bf16_to_f32(B.syn_bf16(2048, seed, 97, 18, 1.0))
    rc, ref = _run(ctx, nh, False, layers, routers, k, h0)
    assert rc == nh.OK and ctx.device_status() == nh.OK
    ctx._check(ctx.set_option(nh.OPT_SPIN_LIMIT, SPIN))
    try:
        for block in (0, 131):
            ctx._check(ctx.set_option(nh.OPT_SKEW_EPOCH, block))
            rc, bad = _run(ctx, nh, True, layers, routers, k, h0)
            assert rc == nh.OK  # asynchronous: the failure shows in the status and the data
            assert ctx.device_status() == nh.ETIMEDOUT
            assert np.isnan(bad[0][1:]).all(), f"block {block}: a hidden state escaped the poisoning"
            assert (bad[1] < 256).all()
            rc, again = _run(ctx, nh, True, layers, routers, k, h0)
            assert rc == nh.OK and ctx.device_status() == nh.OK
            _same(again, ref)
    finally:
        ctx._check(ctx.set_option(nh.OPT_SPIN_LIMIT, 0))


@pytest.mark.parametrize("nl,xcd_local", [(1, 1), (4, 0)])
def test_stack_loop_one_layer_and_without_die_local_words(ctx, nh, nl, xcd_local):
    """A one-layer stack (no gather, no prefetch), and the loop with every
    exchange word device-coherent (NMOE_HIP_OPT_XCD_LOCAL off, as on a device
    whose blocks are not dealt round-robin over its dies): both bit for bit
    the one-launch-per-layer form."""
    bits, seed, k = 4, 61, 8
    layers = [44 + i for i in range(nl)]
    for layer in layers:
        ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    routers, host = _routers(ctx, "bf16", layers, seed)
    h0 = B.bf16_to_f32(B.syn_bf16(2048, seed, 96, 18, 1.0))
    if xcd_local == 0:
        ctx._check(ctx.set_option(nh.OPT_XCD_LOCAL, 0))
    try:
        rc, got = _run(ctx, nh, True, layers, routers, k, h0)
        assert rc == nh.OK and ctx.device_status() == nh.OK
        rc, per_layer = _run(ctx, nh, False, layers, routers, k, h0)
        assert rc == nh.OK and ctx.device_status() == nh.OK
    finally:
        ctx.set_option(nh.OPT_XCD_LOCAL, 1)  # back on where the device's placement allows it
    _same(got, per_layer)
    H, I, Wt = got
    pack = _pack(bits, seed, layers[-1], I[-1][:k])
    want, oi, ow, _, _ = B.moe_block(pack, bits, host[-1], H[-2], k)
    np.testing.assert_array_equal(I[-1], oi)
    assert_close(H[-1], want, what="last layer")
