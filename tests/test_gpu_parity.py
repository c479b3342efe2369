"""GPU parity: libnmoe_hip.so's kernels, called through the C ABI, against the
CPU oracle and the reference math.m golden vectors.

Bars: routing indices, probabilities, dequantised weights and generator
bytes bit-exact; floating-point outputs within max-abs 2e-3 and relative L2
1e-3 (tests/conftest.py MAX_ABS / REL_L2)."""
import os

import numpy as np
import pytest

from conftest import assert_close
from oracle import binding as B

pytestmark = pytest.mark.gpu

SIGMA = {4: 0.02, 2: 0.05}


@pytest.fixture(scope="module")
def nh():
    import nmoe_hip
    return nmoe_hip


@pytest.fixture(scope="module")
def ctx(nh):
    c = nh.Context(0, max_tokens=64)
    yield c
    c.close()


def oracle_experts_threaded(pack, bits, x, k, idx, w, h, chunk=64):
    """The oracle's experts (B.moe_experts) over chunks of tokens on host
    threads: the C call releases the interpreter lock and keeps its state on
    its own stack and heap, once the first chunk, run alone, has built the
    exp table that it fills at first use."""
    from concurrent.futures import ThreadPoolExecutor

    def part(t0):
        sl = slice(t0, t0 + chunk)
        return B.moe_experts(pack, bits, x[sl], k, idx[sl], w[sl], h[sl])

    first = part(0)
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        rest = list(ex.map(part, range(chunk, x.shape[0], chunk)))
    return np.concatenate([first] + rest)


def host_pack(bits, seed, layer, experts):
    """Zero-filled host layer with only `experts` generated (pages of the
    untouched experts are never allocated)."""
    esz = B.EXPERT_SIZE[bits]
    pack = np.zeros(B.EXPERTS * esz, np.uint8)
    for e in sorted(set(int(v) for v in experts)):
        pack[e * esz:(e + 1) * esz] = B.syn_expert(bits, seed, layer, e, SIGMA[bits])
    return pack


def test_argument_validation(ctx, nh):
    x = ctx.alloc(2048 * 4)
    idx = ctx.alloc(8 * 4)
    w = ctx.alloc(8 * 4)
    h = ctx.alloc(2048 * 4)
    out = ctx.alloc(2048 * 4)
    ctx.synth_layer(3, 4, 1, 0.02)
    for k in (0, 9, -1):
        assert ctx.experts(4, 3, x, nh.F32, 1, k, idx, w, h, out) == nh.EINVAL
    assert ctx.experts(4, 4, x, nh.F32, 1, 8, idx, w, h, out) == nh.ENOENT  # layer not resident
    assert ctx.experts(2, 3, x, nh.F32, 1, 8, idx, w, h, out) == nh.EINVAL  # q4 layer called as q2
    assert ctx.experts(4, 3, x.ptr + 4, nh.F32, 1, 8, idx, w, h, out) == nh.EINVAL  # misaligned x
    assert ctx.experts(4, 3, x, nh.F32, 65, 8, idx, w, h, out) == nh.EINVAL  # ntok > max_tokens
    assert ctx.experts(4, 3, None, nh.F32, 1, 8, idx, w, h, out) == nh.EINVAL
    assert ctx.experts(4, 3, x, nh.F32, 1, 8, idx, w, h, out, shared_out=h) == nh.EINVAL
    r = ctx.router_bf16(None)
    assert ctx.route(r, x, nh.BF16, 1, 8, idx, w) == nh.EINVAL
    assert ctx.topk(x, 1, 256, 9, idx, w) == nh.EINVAL
    bad = np.zeros(100, np.uint8)
    with pytest.raises(nh.NmoeError):
        ctx.upload_layer(5, 4, bad)
    ctx.sync()


@pytest.mark.parametrize("bits", [4, 2])
def test_device_generator_matches_oracle(ctx, bits):
    layer = 7 if bits == 4 else 8
    ctx.synth_layer(layer, bits, 1234, SIGMA[bits])
    ctx.sync()
    for e in (0, 1, 77, 255):
        got = ctx.download_expert(layer, e, bits)
        want = B.syn_expert(bits, 1234, layer, e, SIGMA[bits])
        np.testing.assert_array_equal(got, want, err_msg=f"expert {e}")
    buf = ctx.alloc(4096 * 2)
    ctx.synth_bf16(buf, 4096, 99, 3, 17, 1.0)
    np.testing.assert_array_equal(buf.download(np.uint16, 4096), B.syn_bf16(4096, 99, 3, 17, 1.0))


@pytest.mark.parametrize("bits", [4, 2])
def test_dequant_probe_bit_exact(ctx, golden, bits):
    wg, sg, bg = golden[f"q{bits}_packed"], golden[f"q{bits}_scales"], golden[f"q{bits}_biases"]
    rows = wg.shape[0]
    dw, ds, db = ctx.to_device(wg), ctx.to_device(sg), ctx.to_device(bg)
    out = ctx.alloc(rows * 2048 * 4)
    ctx._check(ctx.dequant_rows(bits, dw, ds, db, rows, 2048, out))
    got = out.download(np.float32, (rows, 2048))
    np.testing.assert_array_equal(got.view(np.uint32), golden[f"q{bits}_dequant"].view(np.uint32))


def test_topk_matches_math_m_golden(ctx, golden):
    L = golden["route_logits"]
    n = L.shape[0]
    lg = ctx.to_device(L)
    idx = ctx.alloc(n * 8 * 4)
    w = ctx.alloc(n * 8 * 4)
    probs = ctx.alloc(n * 256 * 4)
    for k in range(1, 9):
        ctx._check(ctx.topk(lg, n, 256, k, idx, w, probs))
        gi = idx.download(np.uint32, (n, 8))
        gw = w.download(np.float32, (n, 8))
        gp = probs.download(np.float32, (n, 256))
        np.testing.assert_array_equal(gp.view(np.uint32), golden["route_probs"].view(np.uint32))
        for c in np.nonzero(golden["route_k"] == k)[0]:
            np.testing.assert_array_equal(gi[c], golden["route_idx"][c], err_msg=f"case {c}")
            np.testing.assert_array_equal(gw[c].view(np.uint32), golden["route_w"][c].view(np.uint32),
                                          err_msg=f"case {c}")


def test_topk_fewer_experts_than_k(ctx, golden):
    lg = ctx.to_device(golden["small_logits"])
    idx, w, probs = ctx.alloc(32), ctx.alloc(32), ctx.alloc(32)
    ctx._check(ctx.topk(lg, 1, 5, 8, idx, w, probs))
    np.testing.assert_array_equal(idx.download(np.uint32, 8), golden["small_idx"])
    np.testing.assert_array_equal(w.download(np.float32, 8).view(np.uint32), golden["small_w"].view(np.uint32))
    np.testing.assert_array_equal(probs.download(np.float32, 5).view(np.uint32),
                                  golden["small_probs"].view(np.uint32))


def test_topk_random_against_oracle(ctx):
    """Many tokens, spreads from narrow to > 100 (slow exact-sum path), ties."""
    rng = np.random.default_rng(21)
    ntok = 64
    L = (rng.standard_normal((ntok, 256)) * rng.choice([0.05, 1, 4, 30, 120], size=(ntok, 1))).astype(np.float32)
    L[::5, 100:110] = L[::5, 100:101]  # exact ties
    L[1::7, :] = np.round(L[1::7, :], 1)  # many coarse ties
    lg = ctx.to_device(L)
    idx, w, probs = ctx.alloc(ntok * 32), ctx.alloc(ntok * 32), ctx.alloc(ntok * 1024)
    for k in (1, 6, 8):
        ctx._check(ctx.topk(lg, ntok, 256, k, idx, w, probs))
        gi, gw, gp = idx.download(np.uint32, (ntok, 8)), w.download(np.float32, (ntok, 8)), probs.download(np.float32, (ntok, 256))
        for t in range(ntok):
            oi, ow, on, op = B.route(L[t], k, want_probs=True)
            np.testing.assert_array_equal(gp[t].view(np.uint32), op.view(np.uint32), err_msg=f"t={t}")
            np.testing.assert_array_equal(gi[t], oi, err_msg=f"t={t} k={k}")
            np.testing.assert_array_equal(gw[t].view(np.uint32), ow.view(np.uint32), err_msg=f"t={t} k={k}")


def test_router_logits_bit_exact(ctx, nh):
    rng = np.random.default_rng(22)
    ntok = 5
    W = B.syn_bf16(256 * 2048, 3, 0, 16, 0.02).reshape(256, 2048)
    xb = B.f32_to_bf16(rng.standard_normal((ntok, 2048)).astype(np.float32))
    xf = B.bf16_to_f32(xb) * np.float32(1.37)  # not bf16-representable: exercises the fp32 path
    dW = ctx.to_device(W)
    lg = ctx.alloc(ntok * 256 * 4)
    r = ctx.router_bf16(dW)
    for xarr, dt in ((xb, nh.BF16), (xf, nh.F32)):
        dx = ctx.to_device(xarr)
        ctx._check(ctx.router_logits(r, dx, dt, ntok, lg))
        got = lg.download(np.float32, (ntok, 256))
        xw = B.bf16_to_f32(xarr) if dt == nh.BF16 else xarr
        for t in range(ntok):
            want = B.router_logits_bf16(W, xw[t])
            np.testing.assert_array_equal(got[t].view(np.uint32), want.view(np.uint32))
    # the reference model's q4 router (kernels.metal:472-513 semantics)
    wq = rng.integers(0, 2**32, size=(256, 256), dtype=np.uint64).astype(np.uint32)
    sq = B.f32_to_bf16((rng.standard_normal((256, 32)) * 0.01).astype(np.float32))
    bq = B.f32_to_bf16((-8 * B.bf16_to_f32(sq)).astype(np.float32))
    rq = ctx.router_q4(ctx.to_device(wq), ctx.to_device(sq), ctx.to_device(bq))
    dx = ctx.to_device(xf)
    ctx._check(ctx.router_logits(rq, dx, nh.F32, ntok, lg))
    got = lg.download(np.float32, (ntok, 256))
    for t in range(ntok):
        want = np.zeros(256, np.float32)
        B.oracle().orc_router_logits_q4(wq.ctypes.data, sq.ctypes.data, bq.ctypes.data, xf[t].ctypes.data, 256, 2048,
                                        want.ctypes.data)
        np.testing.assert_array_equal(got[t].view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("ntok,k", [(1, 8), (1, 1), (3, 6), (4, 8)])
def test_experts_against_oracle(ctx, nh, bits, ntok, k):
    rng = np.random.default_rng(100 * bits + 10 * ntok + k)
    seed, layer = 5, 10 + bits
    ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    idx = np.zeros((ntok, 8), np.uint32)
    for t in range(ntok):
        idx[t, :k] = rng.choice(256, k, replace=False)
    w = np.zeros((ntok, 8), np.float32)
    w[:, :k] = rng.dirichlet(np.ones(k), size=ntok).astype(np.float32)
    xb = B.f32_to_bf16(rng.standard_normal((ntok, 2048)).astype(np.float32))
    x = B.bf16_to_f32(xb).reshape(ntok, 2048)
    h = rng.standard_normal((ntok, 2048)).astype(np.float32)
    pack = host_pack(bits, seed, layer, idx[:, :k].ravel())
    want = B.moe_experts(pack, bits, x, k, idx, w, h)
    d_idx, d_w, d_h, out = ctx.to_device(idx), ctx.to_device(w), ctx.to_device(h), ctx.alloc(ntok * 2048 * 4)
    for fused in (True, False):
        ctx.set_fused(fused)
        for arr, dt in ((xb, nh.BF16), (x, nh.F32)):
            ctx._check(ctx.experts(bits, layer, ctx.to_device(arr), dt, ntok, k, d_idx, d_w, d_h, out))
            got = out.download(np.float32, (ntok, 2048))
            assert_close(got, want, what=f"q{bits} ntok={ntok} k={k} dt={dt} fused={fused}")
    ctx.set_fused(True)
    assert ctx.device_status() == nh.OK
    # shared-expert term, updated in place on the residual (out aliases h_mid)
    sh = rng.standard_normal((ntok, 2048)).astype(np.float32)
    g = rng.standard_normal(ntok).astype(np.float32)
    want_sh = B.moe_experts(pack, bits, x, k, idx, w, h, shared_out=sh, shared_gate_raw=g)
    d_res = ctx.to_device(h)
    ctx._check(ctx.experts(bits, layer, ctx.to_device(x), nh.F32, ntok, k, d_idx, d_w, d_res, d_res,
                           shared_out=ctx.to_device(sh), shared_gate_raw=ctx.to_device(g)))
    assert_close(d_res.download(np.float32, (ntok, 2048)), want_sh, what="shared + in place")


@pytest.mark.parametrize("name,bits,k", [("step_q4_k8", 4, 8), ("step_q2_k8", 2, 8), ("step_q2_k6", 2, 6)])
def test_layer_matches_math_m_golden(ctx, nh, golden, name, bits, k):
    """The whole per-layer call on the config inputs (seed 0, layer 0) against
    the decode step computed by the reference's own math.m."""
    seed, layer = 0, 20 + bits
    # the generator keys on the layer number: layer 0's selected experts, held in slot `layer`
    ctx.upload_layer(layer, bits, host_pack(bits, seed, 0, golden[f"{name}_idx"][:k]))
    router = ctx.alloc(256 * 2048 * 2)
    ctx.synth_bf16(router, 256 * 2048, seed, 0, 16, 0.02)
    x = ctx.alloc(2048 * 2)
    ctx.synth_bf16(x, 2048, seed, 0, 17, 1.0)
    hb = ctx.alloc(2048 * 2)
    ctx.synth_bf16(hb, 2048, seed, 0, 18, 1.0)
    h = ctx.to_device(B.bf16_to_f32(hb.download(np.uint16, 2048)))
    for fused in (True, False):
        ctx.set_fused(fused)
        out, idx, w, lg = ctx.alloc(2048 * 4), ctx.alloc(32), ctx.alloc(32), ctx.alloc(1024)
        ctx._check(ctx.moe_layer(layer, ctx.router_bf16(router), x, nh.BF16, 1, k, h, out, idx, w, lg))
        np.testing.assert_array_equal(lg.download(np.float32, 256).view(np.uint32),
                                      golden[f"{name}_logits"].view(np.uint32))
        np.testing.assert_array_equal(idx.download(np.uint32, 8), golden[f"{name}_idx"])
        np.testing.assert_array_equal(w.download(np.float32, 8).view(np.uint32), golden[f"{name}_w"].view(np.uint32))
        assert_close(out.download(np.float32, 2048), golden[f"{name}_out"], what=f"{name} fused={fused}")
    ctx.set_fused(True)
    assert ctx.device_status() == nh.OK


@pytest.mark.parametrize("bits,ntok", [(4, 6), (2, 6), (4, 24), (2, 24)])
def test_layer_multi_token_against_oracle(ctx, nh, bits, ntok):
    """Several tokens through nmoe_moe_layer: 6 tokens take the per-token
    kernels, 24 the router launch and then the routing inside the grouped
    path's first launch."""
    rng = np.random.default_rng(7 + bits + ntok)
    seed, layer, k = 11, 30 + bits, 8
    ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    W = B.syn_bf16(256 * 2048, seed, layer, 16, 0.02).reshape(256, 2048)
    xb = B.f32_to_bf16(rng.standard_normal((ntok, 2048)).astype(np.float32))
    x = B.bf16_to_f32(xb).reshape(ntok, 2048)
    h = rng.standard_normal((ntok, 2048)).astype(np.float32)
    idx_o = np.zeros((ntok, 8), np.uint32)
    w_o = np.zeros((ntok, 8), np.float32)
    for t in range(ntok):
        idx_o[t], w_o[t], _ = B.route(B.router_logits_bf16(W, x[t]), k)
    want = B.moe_experts(host_pack(bits, seed, layer, idx_o[:, :k].ravel()), bits, x, k, idx_o, w_o, h)
    out, idx, w = ctx.alloc(ntok * 2048 * 4), ctx.alloc(ntok * 32), ctx.alloc(ntok * 32)
    ctx._check(ctx.moe_layer(layer, ctx.router_bf16(ctx.to_device(W)), ctx.to_device(xb), nh.BF16, ntok, k,
                             ctx.to_device(h), out, idx, w))
    np.testing.assert_array_equal(idx.download(np.uint32, (ntok, 8)), idx_o)
    np.testing.assert_array_equal(w.download(np.float32, (ntok, 8)).view(np.uint32), w_o.view(np.uint32))
    assert_close(out.download(np.float32, (ntok, 2048)), want, what=f"layer q{bits}")


@pytest.mark.parametrize("bits", [4, 2])
def test_fused_repeated_launches(ctx, nh, bits):
    """Many back-to-back persistent launches over several layers and inputs:
    the grid barrier counters must reset between launches, and every step
    must match the oracle (routing bit-exact)."""
    rng = np.random.default_rng(40 + bits)
    seed, k, nl, steps = 3, 8, 4, 64
    layers = [40 + 4 * (bits == 2) + i for i in range(nl)]
    for i, layer in enumerate(layers):
        ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    W = [B.syn_bf16(256 * 2048, seed, layer, 16, 0.02).reshape(256, 2048) for layer in layers]
    dW = [ctx.to_device(w) for w in W]
    xb = B.f32_to_bf16(rng.standard_normal((steps, 2048)).astype(np.float32))
    h = rng.standard_normal((steps, 2048)).astype(np.float32)
    dx, dh = ctx.to_device(xb), ctx.to_device(h)
    out, idx, w = ctx.alloc(steps * 8192), ctx.alloc(steps * 32), ctx.alloc(steps * 32)
    for i in range(steps):
        ctx._check(ctx.moe_layer(layers[i % nl], ctx.router_bf16(dW[i % nl]), dx.ptr + i * 4096, nh.BF16, 1, k,
                                 dh.ptr + i * 8192, out.ptr + i * 8192, idx.ptr + i * 32, w.ptr + i * 32))
    assert ctx.device_status() == nh.OK
    go, gi, gw = out.download(np.float32, (steps, 2048)), idx.download(np.uint32, (steps, 8)), w.download(np.float32, (steps, 8))
    x = B.bf16_to_f32(xb).reshape(steps, 2048)
    for i in range(0, steps, 9):
        l = i % nl
        oi, ow, _ = B.route(B.router_logits_bf16(W[l], x[i]), k)
        np.testing.assert_array_equal(gi[i], oi)
        np.testing.assert_array_equal(gw[i].view(np.uint32), ow.view(np.uint32))
        want = B.moe_experts(host_pack(bits, seed, layers[l], oi[:k]), bits, x[i:i + 1], k, oi[None], ow[None], h[i:i + 1])
        assert_close(go[i], want[0], what=f"step {i}")


def _oracle_layer_rmsnorm(pack, bits, W, h_in, k, eps=1e-6):
    h_out = np.zeros(2048, np.float32)
    idx = np.zeros(8, np.uint32)
    w = np.zeros(8, np.float32)
    x = np.zeros(2048, np.float32)
    rc = B.oracle().orc_moe_layer_rmsnorm(pack.ctypes.data, bits, np.ascontiguousarray(W).ctypes.data,
                                          np.ascontiguousarray(h_in, np.float32).ctypes.data, eps, k,
                                          h_out.ctypes.data, idx.ctypes.data, w.ctypes.data, x.ctypes.data)
    assert rc == 0
    return h_out, idx, w, x


@pytest.mark.parametrize("bits", [4, 2])
def test_stack_teacher_forced(ctx, nh, bits):
    """The routed-expert stack of one token: every layer's routing bit-exact
    and its output within tolerance, each layer checked on the GPU's own input
    (RMSNorm in front of every layer, math.m:34-65)."""
    seed, k, nl = 17, 8, 6
    layers = [50 + 6 * (bits == 2) + i for i in range(nl)]
    for layer in layers:
        ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    W = [B.syn_bf16(256 * 2048, seed, layer, 16, 0.02).reshape(256, 2048) for layer in layers]
    dW = [ctx.to_device(w) for w in W]
    h0 = B.bf16_to_f32(B.syn_bf16(2048, seed, 99, 18, 1.0))
    hs = ctx.alloc((nl + 1) * 8192)
    hs.upload(h0)
    idx_s, w_s = ctx.alloc(nl * 32), ctx.alloc(nl * 32)
    ctx._check(ctx.moe_stack(layers, [ctx.router_bf16(d) for d in dW], k, 1e-6, hs, idx_s, w_s))
    assert ctx.device_status() == nh.OK
    H = hs.download(np.float32, (nl + 1, 2048))
    I, Wt = idx_s.download(np.uint32, (nl, 8)), w_s.download(np.float32, (nl, 8))
    np.testing.assert_array_equal(H[0], h0)
    for l in range(nl):
        x = np.zeros(2048, np.float32)
        B.oracle().orc_rms_norm(H[l].ctypes.data, None, x.ctypes.data, 2048, 1e-6, 0)
        oi, ow, _ = B.route(B.router_logits_bf16(W[l], x), k)
        pack = host_pack(bits, seed, layers[l], oi[:k])
        h_out, oi2, ow2, _ = _oracle_layer_rmsnorm(pack, bits, W[l], H[l], k)
        np.testing.assert_array_equal(oi2, oi)
        np.testing.assert_array_equal(I[l], oi, err_msg=f"layer {l}")
        np.testing.assert_array_equal(Wt[l].view(np.uint32), ow.view(np.uint32), err_msg=f"layer {l}")
        assert_close(H[l + 1], h_out, what=f"layer {l}")


def test_rmsnorm_midpoint_takes_exact_path(ctx, nh):
    """h_i = 1 + 2^-12 for all i: the mean square 1 + 2^-11 + 2^-24 is exactly
    a float rounding midpoint, which the double-double fast test rejects, so
    the sequential x87 replay must produce math.m's float."""
    bits, seed, k, layer = 4, 23, 8, 60
    ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    W = B.syn_bf16(256 * 2048, seed, layer, 16, 0.02).reshape(256, 2048)
    dW = ctx.to_device(W)
    for h in (np.full(2048, 1 + 2 ** -12, np.float32),
              np.concatenate([np.full(2047, 1 + 2 ** -12), [1.5]]).astype(np.float32)):
        x = np.zeros(2048, np.float32)
        B.oracle().orc_rms_norm(h.ctypes.data, None, x.ctypes.data, 2048, 1e-6, 0)
        oi, ow, _ = B.route(B.router_logits_bf16(W, x), k)
        dh, dout, di, dw, dl = ctx.to_device(h), ctx.alloc(8192), ctx.alloc(32), ctx.alloc(32), ctx.alloc(1024)
        ctx._check(ctx.moe_layer_rmsnorm(layer, ctx.router_bf16(dW), dh, 1e-6, k, dout, di, dw, dl))
        np.testing.assert_array_equal(dl.download(np.float32, 256).view(np.uint32),
                                      B.router_logits_bf16(W, x).view(np.uint32))
        np.testing.assert_array_equal(di.download(np.uint32, 8), oi)
        h_out, _, _, _ = _oracle_layer_rmsnorm(host_pack(bits, seed, layer, oi[:k]), bits, W, h, k)
        assert_close(dout.download(np.float32, 2048), h_out, what="midpoint rms")


def test_fused_wide_logit_spread(ctx, nh):
    """Logits spread over ~100 (x scaled by 40): many softmax terms fall below
    2^-32, so the fused kernel replays the long double sum sequentially."""
    rng = np.random.default_rng(77)
    bits, seed, k, layer = 4, 31, 8, 61
    ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    W = B.syn_bf16(256 * 2048, seed, layer, 16, 0.02).reshape(256, 2048)
    x = (rng.standard_normal(2048) * 40).astype(np.float32)
    h = rng.standard_normal(2048).astype(np.float32)
    lg = B.router_logits_bf16(W, x)
    assert (np.exp(lg.astype(np.float64) - lg.max()) < 2.0 ** -32).any()
    oi, ow, _ = B.route(lg, k)
    want = B.moe_experts(host_pack(bits, seed, layer, oi[:k]), bits, x[None], k, oi[None], ow[None], h[None])[0]
    out, di, dw = ctx.alloc(8192), ctx.alloc(32), ctx.alloc(32)
    ctx._check(ctx.moe_layer(layer, ctx.router_bf16(ctx.to_device(W)), ctx.to_device(x), nh.F32, 1, k,
                             ctx.to_device(h), out, di, dw))
    np.testing.assert_array_equal(di.download(np.uint32, 8), oi)
    np.testing.assert_array_equal(dw.download(np.float32, 8).view(np.uint32), ow.view(np.uint32))
    # x is scaled by 40, so outputs reach ~1e5: the absolute bound scales with them
    scale = max(1.0, float(np.abs(want).max()) / 10.0)
    assert_close(out.download(np.float32, 2048), want, max_abs=2e-3 * scale, what="wide spread")


def _tie_router(k):
    """Router rows and x whose logits put a probability tie on the top-k
    boundary between two entries with different logits: k-1 experts at logit
    2^-10, expert 200 at 2^-11 and expert 3 at 2^-11 - 2^-30 (everything else
    -1).  exp() of the two boundary arguments rounds to the same float, so
    the k largest logits hold 200 while math.m's top-k takes 3 (lower index
    among equal probabilities)."""
    W = np.zeros((256, 2048), np.float32)
    W[:, 0] = -1.0
    top = [50 + 10 * i for i in range(k - 1)]
    W[top, 0] = 2.0 ** -10
    W[200, 0] = 2.0 ** -11
    W[3, 0] = 2.0 ** -11
    W[3, 1] = -(2.0 ** -10)
    x = np.zeros(2048, np.float32)
    x[0], x[1] = 1.0, 2.0 ** -20
    Wb = B.f32_to_bf16(W.ravel()).reshape(256, 2048)
    return Wb, x, top


@pytest.mark.gpu
@pytest.mark.parametrize("bits,k", [(4, 8), (2, 6)])
def test_fused_probability_tie_at_boundary(ctx, nh, bits, k):
    """The fused kernel starts streaming the k largest logits' experts before
    the softmax; a probability tie across the boundary must still give
    math.m's selection, slot order and weights, with the right expert's
    weights in the combine."""
    seed, layer = 41, 62
    Wb, x, top = _tie_router(k)
    lg = B.router_logits_bf16(Wb, x)
    assert lg[200] > lg[3]
    oi, ow, _ = B.route(lg, k)
    assert 3 in oi[:k] and 200 not in oi[:k]  # the construction holds
    assert sorted(np.argsort(-lg, kind="stable")[:k].tolist()) == sorted(top + [200])
    ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    rng = np.random.default_rng(5)
    h = rng.standard_normal(2048).astype(np.float32)
    want = B.moe_experts(host_pack(bits, seed, layer, oi[:k]), bits, x[None], k, oi[None], ow[None], h[None])[0]
    out, di, dw = ctx.alloc(8192), ctx.alloc(32), ctx.alloc(32)
    ctx._check(ctx.moe_layer(layer, ctx.router_bf16(ctx.to_device(Wb)), ctx.to_device(x), nh.F32, 1, k,
                             ctx.to_device(h), out, di, dw))
    np.testing.assert_array_equal(di.download(np.uint32, 8)[:k], oi[:k])
    np.testing.assert_array_equal(dw.download(np.float32, 8)[:k].view(np.uint32), ow[:k].view(np.uint32))
    assert_close(out.download(np.float32, 2048), want, what="tie at boundary")


def _near_tie_router(k):
    """Router rows and x whose logits put two entries a few ulps apart on the
    top-k boundary, the higher one at the higher index: k-1 experts at logit
    1, expert 3 at 0.5 and expert 200 at 0.5 + 2^-22 (everything else -1).
    The two agree in their top 24 key bits, so a selection on those bits
    prefers the lower entry 3, while their probabilities differ and math.m's
    top-k takes 200."""
    W = np.zeros((256, 2048), np.float32)
    W[:, 0] = -1.0
    top = [50 + 10 * i for i in range(k - 1)]
    W[top, 0] = 1.0
    W[3, 0] = 0.5
    W[200, 0] = 0.5
    W[200, 1] = 0.25
    x = np.zeros(2048, np.float32)
    x[0], x[1] = 1.0, 2.0 ** -20
    Wb = B.f32_to_bf16(W.ravel()).reshape(256, 2048)
    return Wb, x, top


@pytest.mark.gpu
@pytest.mark.parametrize("bits,k", [(4, 8), (2, 6)])
def test_fused_near_tie_candidate_corrected(ctx, nh, bits, k):
    """The fused kernel's early candidates compare logits on their top 24
    key bits; when that picks the wrong one of two near-equal boundary
    logits, the exact routing must re-point the group to math.m's expert,
    with math.m's slot order, weights and output."""
    seed, layer = 43, 61
    Wb, x, top = _near_tie_router(k)
    lg = B.router_logits_bf16(Wb, x)
    key = lambda f: int(np.float32(f).view(np.uint32)) | 0x80000000  # positive logits
    assert lg[200] > lg[3] and key(lg[200]) >> 8 == key(lg[3]) >> 8  # the construction holds
    oi, ow, _ = B.route(lg, k)
    assert 200 in oi[:k] and 3 not in oi[:k]
    ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    rng = np.random.default_rng(6)
    h = rng.standard_normal(2048).astype(np.float32)
    want = B.moe_experts(host_pack(bits, seed, layer, oi[:k]), bits, x[None], k, oi[None], ow[None], h[None])[0]
    out, di, dw = ctx.alloc(8192), ctx.alloc(32), ctx.alloc(32)
    ctx._check(ctx.moe_layer(layer, ctx.router_bf16(ctx.to_device(Wb)), ctx.to_device(x), nh.F32, 1, k,
                             ctx.to_device(h), out, di, dw))
    np.testing.assert_array_equal(di.download(np.uint32, 8)[:k], oi[:k])
    np.testing.assert_array_equal(dw.download(np.float32, 8)[:k].view(np.uint32), ow[:k].view(np.uint32))
    assert_close(out.download(np.float32, 2048), want, what="near tie at boundary")


@pytest.mark.gpu
def test_xcd_placement_and_die_local_exchange(ctx, nh):
    """MI355X deals a launch's blocks round-robin over its 8 dies (checked at
    create), so the die-local exchange is available; with it on or off the
    fused step gives identical results, equal to the oracle's routing."""
    bits, seed, k, layer = 4, 52, 8, 63
    ctx.set_xcd_local(True)  # raises where the placement check failed
    ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    rng = np.random.default_rng(9)
    W = B.syn_bf16(256 * 2048, seed, layer, 16, 0.02).reshape(256, 2048)
    x = rng.standard_normal(2048).astype(np.float32)
    h = rng.standard_normal(2048).astype(np.float32)
    oi, ow, _ = B.route(B.router_logits_bf16(W, x), k)
    want = B.moe_experts(host_pack(bits, seed, layer, oi[:k]), bits, x[None], k, oi[None], ow[None], h[None])[0]
    rt, xd, hd = ctx.router_bf16(ctx.to_device(W)), ctx.to_device(x), ctx.to_device(h)
    outs = []
    try:
        for on in (True, False, True):
            ctx.set_xcd_local(on)
            out, di, dw = ctx.alloc(8192), ctx.alloc(32), ctx.alloc(32)
            for _ in range(3):
                ctx._check(ctx.moe_layer(layer, rt, xd, nh.F32, 1, k, hd, out, di, dw))
            assert ctx.device_status() == 0
            np.testing.assert_array_equal(di.download(np.uint32, 8), oi)
            outs.append(out.download(np.float32, 2048))
    finally:
        ctx.set_xcd_local(True)
    np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    np.testing.assert_array_equal(outs[0].view(np.uint32), outs[2].view(np.uint32))
    assert_close(outs[0], want, what="die-local exchange")


# ---------------------------------------------------------------- grouped path

def zipf_idx(rng, ntok, k, alpha=1.1):
    """Per token, k distinct experts drawn without replacement with
    p_e ~ rank_e^-alpha over a seeded permutation (Gumbel-top-k)."""
    order = rng.permutation(256)
    logp = np.empty(256)
    logp[order] = -alpha * np.log(np.arange(1, 257))
    g = logp[None, :] + rng.gumbel(size=(ntok, 256))
    idx = np.zeros((ntok, 8), np.uint32)
    idx[:, :k] = np.argsort(-g, axis=1, kind="stable")[:, :k]
    return idx


@pytest.fixture(scope="module")
def big(nh):
    c = nh.Context(0, max_tokens=2048)
    yield c
    c.close()


@pytest.mark.parametrize("ntok,k,kind", [(1, 8, "uniform"), (64, 8, "zipf"), (2048, 8, "uniform"), (33, 6, "zipf"),
                                         (100, 3, "uniform"), (64, 8, "invalid")])
def test_dispatch_matches_oracle(big, ntok, k, kind):
    """a14: the stable counting sort of (t, s) entries by expert is bit-exact
    with the oracle's (numpy's stable argsort); entries outside the layer
    are left out."""
    rng = np.random.default_rng(ntok * 10 + k)
    if kind == "zipf":
        idx = zipf_idx(rng, ntok, k)
    else:
        idx = np.zeros((ntok, 8), np.uint32)
        idx[:, :k] = rng.integers(0, 256, size=(ntok, k))
    if kind == "invalid":
        idx[rng.integers(0, ntok, 20), rng.integers(0, k, 20)] = 300 + rng.integers(0, 50, 20)
    flat = idx[:, :k].reshape(-1)
    valid = flat < 256
    perm = big.alloc(ntok * k * 4)
    offs = big.alloc(257 * 4)
    big._check(big.dispatch(big.to_device(idx), ntok, k, perm, offs))
    got_p = perm.download(np.uint32, ntok * k)
    got_o = offs.download(np.uint32, 257)
    if kind != "invalid":
        want_p, want_o = B.dispatch(idx, ntok, k, 8)
    else:
        keys = np.where(valid, flat, 256)
        want_p = np.argsort(keys, kind="stable")[:valid.sum()].astype(np.uint32)
        want_o = np.concatenate([[0], np.cumsum(np.bincount(flat[valid], minlength=256))]).astype(np.uint32)
    np.testing.assert_array_equal(got_o, want_o)
    np.testing.assert_array_equal(got_p[:int(want_o[256])], want_p)


def test_dispatch_long_slices(nh):
    """10,000 tokens x 8 = 80,000 entries: 64 dispatch blocks of 1,250
    entries, so each slice spans five 256-entry chunks (four read up front,
    the fifth read in the scatter, ragged), with Zipf routing and some
    entries outside the layer."""
    c = nh.Context(0, max_tokens=10000)
    try:
        rng = np.random.default_rng(5000)
        ntok, k = 10000, 8
        idx = zipf_idx(rng, ntok, k)
        idx[rng.integers(0, ntok, 50), rng.integers(0, k, 50)] = 256 + rng.integers(0, 100, 50)
        flat = idx[:, :k].reshape(-1)
        valid = flat < 256
        perm, offs = c.alloc(ntok * k * 4), c.alloc(257 * 4)
        c._check(c.dispatch(c.to_device(idx), ntok, k, perm, offs))
        got_p, got_o = perm.download(np.uint32, ntok * k), offs.download(np.uint32, 257)
        keys = np.where(valid, flat, 256)
        want_p = np.argsort(keys, kind="stable")[:valid.sum()].astype(np.uint32)
        want_o = np.concatenate([[0], np.cumsum(np.bincount(flat[valid], minlength=256))]).astype(np.uint32)
        np.testing.assert_array_equal(got_o, want_o)
        np.testing.assert_array_equal(got_p[:int(want_o[256])], want_p)
        assert c.device_status() == nh.OK
    finally:
        c.close()


def gemm_forms(big):
    """The grouped path's GEMM forms the device runs: gate/up and down in one
    launch (which needs the round-robin die placement checked at create) and
    in two."""
    forms = [(name, one) for name, one in (("one launch", True), ("two launches", False))
             if big.set_grouped_one_launch(one)]
    big.set_grouped_one_launch(True)
    return forms


def run_forms(big, fn):
    """fn() under each GEMM form; the outputs (arrays) must be the same bits
    in every form (each output element takes the same arithmetic whatever
    the tile it falls in).  Returns the first form's."""
    outs = []
    try:
        for name, one in gemm_forms(big):
            big.set_grouped_one_launch(one)
            outs.append((name, fn()))
    finally:
        big.set_grouped_one_launch(True)
    for name, o in outs[1:]:
        for a, b in zip(outs[0][1], o):
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg=f"{outs[0][0]} vs {name}")
    return outs[0][1]


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("ntok,k,xkind,ikind", [(8, 8, "bf16", "uniform"), (64, 8, "bf16", "zipf"),
                                               (64, 6, "f32", "zipf"), (40, 8, "f32", "uniform")])
def test_grouped_experts_against_oracle(big, nh, bits, ntok, k, xkind, ikind):
    """a15: the grouped matrix-core path (dispatch, gate/up + SwiGLU, down,
    slot-order combine) against the oracle, and against the per-token
    kernels, with shared-expert term and an invalid slot."""
    rng = np.random.default_rng(1000 * bits + ntok + k)
    seed, layer = 21, 40 + bits
    big.synth_layer(layer, bits, seed, SIGMA[bits])
    idx = zipf_idx(rng, ntok, k) if ikind == "zipf" else np.zeros((ntok, 8), np.uint32)
    if ikind == "uniform":
        for t in range(ntok):
            idx[t, :k] = rng.choice(256, k, replace=False)
    w = np.zeros((ntok, 8), np.float32)
    w[:, :k] = rng.dirichlet(np.ones(k), size=ntok).astype(np.float32)
    idx[3, 1] = 999  # invalid slot: weight 0 (runtime.m:2977-2981)
    w_eff = w.copy()
    w_eff[3, 1] = 0.0
    idx_eff = idx.copy()
    idx_eff[3, 1] = idx[3, 0]
    xf = rng.standard_normal((ntok, 2048)).astype(np.float32)
    if xkind == "bf16":
        xb = B.f32_to_bf16(xf)
        x, xdev, dt = B.bf16_to_f32(xb).reshape(ntok, 2048), xb, nh.BF16
    else:
        x, xdev, dt = xf, xf, nh.F32
    h = rng.standard_normal((ntok, 2048)).astype(np.float32)
    sh = rng.standard_normal((ntok, 2048)).astype(np.float32)
    gr = rng.standard_normal(ntok).astype(np.float32)
    pack = host_pack(bits, seed, layer, idx_eff[:, :k].ravel())
    want = B.moe_experts(pack, bits, x, k, idx_eff, w_eff, h, sh, gr)
    d = [big.to_device(a) for a in (xdev, idx, w, h, sh, gr)]

    def run():
        out = big.alloc(ntok * 2048 * 4)
        big._check(big.experts(bits, layer, d[0], dt, ntok, k, d[1], d[2], d[3], out, d[4], d[5]))
        return (out.download(np.float32, (ntok, 2048)),)

    outs = {}
    try:
        big.set_grouped_min_tokens(1)
        outs["grouped"] = run_forms(big, run)[0]
        big.set_grouped_min_tokens(1 << 20)
        outs["per-token"] = run()[0]
    finally:
        big.set_grouped_min_tokens(8)
    assert big.device_status() == nh.OK
    for path, got in outs.items():
        assert_close(got, want, what=f"{path} q{bits} ntok={ntok} k={k} x={xkind}")


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("xkind", ["bf16", "f32"])
def test_grouped_small_and_big_forms(big, nh, bits, xkind):
    """Experts of at most 16 entries take the small form (one 16-entry pass,
    two groups a ring step), larger ones the 64-entry passes, in the same
    launch: experts of exactly 16, 17, 64, 65 and 1 entries, every token's
    output against the oracle."""
    rng = np.random.default_rng(700 + 10 * bits + (xkind == "f32"))
    seed, layer, ntok, k = 29, 45 + bits, 80, 8
    big.synth_layer(layer, bits, seed, SIGMA[bits])
    want_n = {5: 16, 6: 17, 7: 64, 8: 65, 9: 1}
    idx = np.zeros((ntok, 8), np.uint32)
    rest = np.array([e for e in range(256) if e not in want_n])
    for t in range(ntok):
        idx[t, :k] = rng.choice(rest, k, replace=False)
    slot = 0
    for e, cnt in want_n.items():  # expert e replaces one slot of cnt distinct tokens
        for t in rng.choice(ntok, cnt, replace=False):
            idx[t, slot] = e
        slot += 1
    counts = np.bincount(idx[:, :k].ravel(), minlength=256)
    for e, cnt in want_n.items():
        assert counts[e] == cnt
    w = rng.dirichlet(np.ones(k), size=ntok).astype(np.float32)
    xf = rng.standard_normal((ntok, 2048)).astype(np.float32)
    if xkind == "bf16":
        xb = B.f32_to_bf16(xf)
        x, xdev, dt = B.bf16_to_f32(xb).reshape(ntok, 2048), xb, nh.BF16
    else:
        x, xdev, dt = xf, xf, nh.F32
    h = rng.standard_normal((ntok, 2048)).astype(np.float32)
    d = [big.to_device(a) for a in (xdev, idx, w, h)]

    def run():
        out = big.alloc(ntok * 2048 * 4)
        big._check(big.experts(bits, layer, d[0], dt, ntok, k, d[1], d[2], d[3], out))
        return (out.download(np.float32, (ntok, 2048)),)

    got = run_forms(big, run)[0]
    assert big.device_status() == nh.OK
    pack = host_pack(bits, seed, layer, idx[:, :k].ravel())
    want = B.moe_experts(pack, bits, x, k, idx, w, h)
    assert_close(got, want, what=f"small/big forms q{bits} x={xkind}")


@pytest.mark.parametrize("bits", [4, 2])
def test_grouped_on_uploaded_layer_and_reupload(big, nh, bits):
    """The grouped GEMMs read the layer's stripe-major copy, written on the
    device after every upload: a layer uploaded from the host, then the
    same layer uploaded again with other experts (and then synthesised on
    the device over it), each time every token against the oracle on the
    pack just written, never on the one before."""
    rng = np.random.default_rng(810 + bits)
    layer, ntok, k = 50 + bits, 24, 8
    idx = np.zeros((ntok, 8), np.uint32)
    for t in range(ntok):
        idx[t, :k] = rng.choice(256, k, replace=False)
    w = rng.dirichlet(np.ones(k), size=ntok).astype(np.float32)
    x = rng.standard_normal((ntok, 2048)).astype(np.float32)
    h = rng.standard_normal((ntok, 2048)).astype(np.float32)
    d = [big.to_device(a) for a in (x, idx, w, h)]

    def run():
        out = big.alloc(ntok * 2048 * 4)
        big._check(big.experts(bits, layer, d[0], nh.F32, ntok, k, d[1], d[2], d[3], out))
        return (out.download(np.float32, (ntok, 2048)),)

    try:
        big.set_grouped_min_tokens(1)
        for step, seed in enumerate((33, 34, None)):
            if seed is None:  # synthesised on the device over the uploaded layer
                seed = 35
                big.synth_layer(layer, bits, seed, SIGMA[bits])
                pack = host_pack(bits, seed, layer, idx[:, :k].ravel())
            else:
                pack = host_pack(bits, seed, layer, idx[:, :k].ravel())
                big.upload_layer(layer, bits, pack)
            got = run_forms(big, run)[0]
            assert big.device_status() == nh.OK
            want = B.moe_experts(pack, bits, x, k, idx, w, h)
            assert_close(got, want, what=f"q{bits} layer written {step + 1} times (seed {seed})")
            del pack
    finally:
        big.set_grouped_min_tokens(8)


def test_grouped_layer_changes_code_width(big, nh):
    """A layer written as q4, then as q2, then as q4 again: each write of
    another width allocates the pack and its stripe-major copy anew, and the
    grouped path reads the copy of the width just written (every token
    against the oracle)."""
    rng = np.random.default_rng(830)
    layer, ntok, k = 54, 20, 8
    idx = np.zeros((ntok, 8), np.uint32)
    for t in range(ntok):
        idx[t, :k] = rng.choice(256, k, replace=False)
    w = rng.dirichlet(np.ones(k), size=ntok).astype(np.float32)
    x = rng.standard_normal((ntok, 2048)).astype(np.float32)
    h = rng.standard_normal((ntok, 2048)).astype(np.float32)
    d = [big.to_device(a) for a in (x, idx, w, h)]
    try:
        big.set_grouped_min_tokens(1)
        for bits, seed in ((4, 41), (2, 42), (4, 43)):
            big.synth_layer(layer, bits, seed, SIGMA[bits])
            out = big.alloc(ntok * 2048 * 4)
            big._check(big.experts(bits, layer, d[0], nh.F32, ntok, k, d[1], d[2], d[3], out))
            assert big.device_status() == nh.OK
            pack = host_pack(bits, seed, layer, idx[:, :k].ravel())
            want = B.moe_experts(pack, bits, x, k, idx, w, h)
            assert_close(out.download(np.float32, (ntok, 2048)), want, what=f"layer as q{bits} (seed {seed})")
            del pack
    finally:
        big.set_grouped_min_tokens(8)


@pytest.mark.parametrize("bits", [4, 2])
def test_prefill_2048_every_token(big, nh, bits):
    """C5 shape: 2048 tokens, uniform-random logits -> device top-8 ->
    grouped experts; routing bit-exact for all 2048 tokens; the outputs of
    all 2048 tokens against the oracle (on host threads) and against the
    per-token kernels on the same routing."""
    rng = np.random.default_rng(2048 + bits)
    seed, layer, ntok, k = 33, 50 + bits, 2048, 8
    big.synth_layer(layer, bits, seed, SIGMA[bits])
    logits = rng.random((ntok, 256), dtype=np.float32)
    xb = B.f32_to_bf16(rng.standard_normal((ntok, 2048)).astype(np.float32))
    x = B.bf16_to_f32(xb).reshape(ntok, 2048)
    h = rng.standard_normal((ntok, 2048)).astype(np.float32)
    d_lg, d_x, d_h = big.to_device(logits), big.to_device(xb), big.to_device(h)

    def run():
        d_idx, d_w, out = big.alloc(ntok * 32), big.alloc(ntok * 32), big.alloc(ntok * 2048 * 4)
        big._check(big.topk(d_lg, ntok, 256, k, d_idx, d_w))
        big._check(big.experts(bits, layer, d_x, nh.BF16, ntok, k, d_idx, d_w, d_h, out))
        return d_idx.download(np.uint32, (ntok, 8)), d_w.download(np.float32, (ntok, 8)), \
            out.download(np.float32, (ntok, 2048))

    idx, w, full = run_forms(big, run)
    for t in range(ntok):  # every token's routing
        oi, ow, _ = B.route(logits[t], k)
        np.testing.assert_array_equal(idx[t], oi, err_msg=f"t={t}")
        np.testing.assert_array_equal(w[t].view(np.uint32), ow.view(np.uint32), err_msg=f"t={t}")
    assert big.device_status() == nh.OK
    print(f"[prefill] q{bits}: 2048 tokens through the oracle", flush=True)
    pack = host_pack(bits, seed, layer, idx[:, :k].ravel())
    want = oracle_experts_threaded(pack, bits, x, k, idx, w, h)
    del pack
    for t0 in range(0, ntok, 256):  # every token, in blocks that name the first failing one
        assert_close(full[t0:t0 + 256], want[t0:t0 + 256], what=f"prefill q{bits} tokens {t0}..{t0 + 255}")
    print(f"[prefill] q{bits}: 2048 tokens through the per-token kernels", flush=True)
    d_idx, d_w, out = big.to_device(idx), big.to_device(w), big.alloc(ntok * 2048 * 4)
    try:
        big.set_grouped_min_tokens(ntok + 1)
        big._check(big.experts(bits, layer, d_x, nh.BF16, ntok, k, d_idx, d_w, d_h, out))
    finally:
        big.set_grouped_min_tokens(8)
    assert big.device_status() == nh.OK
    per_token = out.download(np.float32, (ntok, 2048))
    for t0 in range(0, ntok, 256):  # every token, in blocks that name the first failing one
        assert_close(full[t0:t0 + 256], per_token[t0:t0 + 256], what=f"prefill q{bits} tokens {t0}..{t0 + 255}")


@pytest.mark.parametrize("bits,ntok,k,xkind,lkind", [
    (4, 64, 8, "bf16", "zipf"),      # C4's shape: one dispatch block
    (2, 2048, 8, "bf16", "uniform"),  # C5's shape: 64 dispatch blocks
    (4, 300, 6, "f32", "zipf"),       # 8 dispatch blocks, k = 6
    (2, 8, 1, "f32", "uniform"),      # the grouped threshold, k = 1
    (4, 5, 8, "bf16", "uniform"),     # below it: the top-k launch and the per-token kernels
])
def test_experts_from_logits_equals_topk_then_experts(big, nh, bits, ntok, k, xkind, lkind):
    """nmoe_moe_experts_from_logits (the routing inside the grouped path's
    first launch) against nmoe_moe_topk then nmoe_moe_experts on the same
    inputs: idx, w and out bit for bit, and every token's routing against the
    oracle's math.m routing; two calls in a row (the routing counter starts
    from 0 for the second), the second on other logits."""
    rng = np.random.default_rng(5000 + 100 * bits + ntok + k)
    seed, layer = 41, 20 + bits
    big.synth_layer(layer, bits, seed, SIGMA[bits])
    for call in range(2):
        print(f"[from-logits] q{bits} ntok={ntok} k={k} x={xkind} {lkind} call {call}", flush=True)
        if lkind == "zipf":
            order = rng.permutation(256)
            logp = np.empty(256)
            logp[order] = -1.1 * np.log(np.arange(1, 257))
            logits = (logp[None, :] + rng.gumbel(size=(ntok, 256))).astype(np.float32)
        else:
            logits = rng.random((ntok, 256), dtype=np.float32)
        xf = rng.standard_normal((ntok, 2048)).astype(np.float32)
        xdev, dt = (B.f32_to_bf16(xf), nh.BF16) if xkind == "bf16" else (xf, nh.F32)
        h = rng.standard_normal((ntok, 2048)).astype(np.float32)
        d_lg, d_x, d_h = big.to_device(logits), big.to_device(xdev), big.to_device(h)
        res = {}
        for path in ("from_logits", "topk_then_experts"):
            idx, w, out = big.alloc(ntok * 32), big.alloc(ntok * 32), big.alloc(ntok * 2048 * 4)
            if path == "from_logits":
                big._check(big.experts_from_logits(layer, d_lg, d_x, dt, ntok, k, d_h, out, idx, w))
            else:
                big._check(big.topk(d_lg, ntok, 256, k, idx, w))
                big._check(big.experts(bits, layer, d_x, dt, ntok, k, idx, w, d_h, out))
            res[path] = (idx.download(np.uint32, (ntok, 8)), w.download(np.float32, (ntok, 8)),
                         out.download(np.float32, (ntok, 2048)))
        assert big.device_status() == nh.OK
        (ia, wa, oa), (ib, wb, ob) = res["from_logits"], res["topk_then_experts"]
        np.testing.assert_array_equal(ia, ib)
        np.testing.assert_array_equal(wa.view(np.uint32), wb.view(np.uint32))
        np.testing.assert_array_equal(oa.view(np.uint32), ob.view(np.uint32))
        for t in range(ntok):
            oi, ow, _ = B.route(logits[t], k)
            np.testing.assert_array_equal(ia[t], oi, err_msg=f"t={t}")
            np.testing.assert_array_equal(wa[t].view(np.uint32), ow.view(np.uint32), err_msg=f"t={t}")


@pytest.mark.parametrize("offset", [4, 8, 12])
def test_experts_from_logits_logits_4_byte_aligned(big, nh, offset):
    """Logits 4-byte aligned but not 16-byte aligned (the entry point takes
    them): the routing wavefronts read them a lane a word instead of by
    16-byte direct loads, with the same bits as the topk launch."""
    rng = np.random.default_rng(6100 + offset)
    ntok, k, bits, layer = 64, 8, 4, 27
    big.synth_layer(layer, bits, 43, SIGMA[bits])
    logits = rng.random((ntok, 256), dtype=np.float32)
    x = B.f32_to_bf16(rng.standard_normal((ntok, 2048)).astype(np.float32))
    h = rng.standard_normal((ntok, 2048)).astype(np.float32)
    d_lg = big.alloc(ntok * 1024 + 16)
    d_lg.upload(logits, offset)
    d_x, d_h = big.to_device(x), big.to_device(h)
    res = []
    for use_offset in (True, False):
        idx, w, out = big.alloc(ntok * 32), big.alloc(ntok * 32), big.alloc(ntok * 2048 * 4)
        if use_offset:
            big._check(big.experts_from_logits(layer, d_lg.ptr + offset, d_x, nh.BF16, ntok, k, d_h, out, idx, w))
        else:
            d_al = big.to_device(logits)
            big._check(big.topk(d_al, ntok, 256, k, idx, w))
            big._check(big.experts(bits, layer, d_x, nh.BF16, ntok, k, idx, w, d_h, out))
        res.append((idx.download(np.uint32, (ntok, 8)), w.download(np.float32, (ntok, 8)),
                    out.download(np.float32, (ntok, 2048))))
    assert big.device_status() == nh.OK
    for a, b_, name in zip(res[0], res[1], ("idx", "w", "out")):
        np.testing.assert_array_equal(a.view(np.uint32), b_.view(np.uint32), err_msg=name)


def test_experts_from_logits_slices_past_four_chunks(nh):
    """8,448 tokens x 8 = 67,584 entries: 64 dispatch slices of 1,056, so
    each slice's last chunk is read after the first four (the tagged entries
    polled again there).  Bit for bit against nmoe_moe_topk then
    nmoe_moe_experts (whose dispatch reads idx), and a sample of tokens'
    routing against the oracle's."""
    rng = np.random.default_rng(6200)
    ntok, k, bits, layer = 8448, 8, 2, 3
    with nh.Context(0, max_tokens=ntok) as ctx:
        ctx.synth_layer(layer, bits, 47, SIGMA[bits])
        logits = rng.random((ntok, 256), dtype=np.float32)
        x = B.f32_to_bf16(rng.standard_normal((ntok, 2048)).astype(np.float32))
        h = rng.standard_normal((ntok, 2048)).astype(np.float32)
        d_lg, d_x, d_h = ctx.to_device(logits), ctx.to_device(x), ctx.to_device(h)
        res = []
        for path in ("from_logits", "topk_then_experts"):
            print(f"[from-logits] {ntok} tokens: {path}", flush=True)
            idx, w, out = ctx.alloc(ntok * 32), ctx.alloc(ntok * 32), ctx.alloc(ntok * 2048 * 4)
            if path == "from_logits":
                ctx._check(ctx.experts_from_logits(layer, d_lg, d_x, nh.BF16, ntok, k, d_h, out, idx, w))
            else:
                ctx._check(ctx.topk(d_lg, ntok, 256, k, idx, w))
                ctx._check(ctx.experts(bits, layer, d_x, nh.BF16, ntok, k, idx, w, d_h, out))
            res.append((idx.download(np.uint32, (ntok, 8)), w.download(np.float32, (ntok, 8)),
                        out.download(np.float32, (ntok, 2048))))
        assert ctx.device_status() == nh.OK
    for a, b_, name in zip(res[0], res[1], ("idx", "w", "out")):
        np.testing.assert_array_equal(a.view(np.uint32), b_.view(np.uint32), err_msg=name)
    for t in rng.choice(ntok, 32, replace=False):
        oi, ow, _ = B.route(logits[t], k)
        np.testing.assert_array_equal(res[0][0][t], oi, err_msg=f"t={t}")
        np.testing.assert_array_equal(res[0][1][t].view(np.uint32), ow.view(np.uint32), err_msg=f"t={t}")


def test_experts_from_logits_rejects(big, nh):
    big.synth_layer(25, 4, 1, 0.02)
    lg, x, h, out = big.alloc(64 * 1024), big.alloc(64 * 4096), big.alloc(64 * 8192), big.alloc(64 * 8192)
    idx, w = big.alloc(64 * 32), big.alloc(64 * 32)
    assert big.experts_from_logits(25, None, x, nh.BF16, 64, 8, h, out, idx, w) == nh.EINVAL
    assert big.experts_from_logits(25, lg, x, nh.BF16, 64, 8, h, out, None, w) == nh.EINVAL
    assert big.experts_from_logits(25, lg, x, nh.BF16, 64, 9, h, out, idx, w) == nh.EINVAL
    assert big.experts_from_logits(25, lg, x, nh.BF16, 4096, 8, h, out, idx, w) == nh.EINVAL
    assert big.experts_from_logits(26, lg, x, nh.BF16, 64, 8, h, out, idx, w) == nh.ENOENT


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("xkind", ["bf16", "f32"])
def test_grouped_zipf_1200_sampled(big, nh, bits, xkind):
    """1200 tokens x 8 entries with Zipf routing: several hundred entries on
    the hottest experts (many 64-entry passes, every row-block count in the
    last one) and a handful on the tail; outputs on 40 sampled tokens (token
    3 with an invalid slot among them) against the oracle."""
    rng = np.random.default_rng(128 + 10 * bits + (xkind == "f32"))
    seed, layer, ntok, k = 37, 56 + bits, 1200, 8
    big.synth_layer(layer, bits, seed, SIGMA[bits])
    idx = zipf_idx(rng, ntok, k)
    counts = np.bincount(idx[:, :k].ravel(), minlength=256)
    assert counts.max() > 256
    w = rng.dirichlet(np.ones(k), size=ntok).astype(np.float32)
    idx[3, 1] = 999
    w_eff = w.copy()
    w_eff[3, 1] = 0.0
    idx_eff = idx.copy()
    idx_eff[3, 1] = idx[3, 0]
    xf = rng.standard_normal((ntok, 2048)).astype(np.float32)
    if xkind == "bf16":
        xb = B.f32_to_bf16(xf)
        x, xdev, dt = B.bf16_to_f32(xb).reshape(ntok, 2048), xb, nh.BF16
    else:
        x, xdev, dt = xf, xf, nh.F32
    h = rng.standard_normal((ntok, 2048)).astype(np.float32)
    d = [big.to_device(a) for a in (xdev, idx, w, h)]

    def run():
        out = big.alloc(ntok * 2048 * 4)
        big._check(big.experts(bits, layer, d[0], dt, ntok, k, d[1], d[2], d[3], out))
        return (out.download(np.float32, (ntok, 2048)),)

    full = run_forms(big, run)[0]
    assert big.device_status() == nh.OK
    sample = np.concatenate([[3], rng.choice(np.arange(4, ntok), 39, replace=False)])
    got = full[sample]
    pack = host_pack(bits, seed, layer, idx_eff[sample, :k].ravel())
    want = B.moe_experts(pack, bits, x[sample], k, idx_eff[sample], w_eff[sample], h[sample])
    assert_close(got, want, what=f"zipf 1200 q{bits} x={xkind}")


@pytest.mark.parametrize("xdt,ntok", [("f32", 1), ("bf16", 1), ("f32", 5), ("bf16", 6)])
def test_shared_expert_against_oracle(ctx, nh, xdt, ntok):
    """nmoe_moe_shared_expert (kernels.metal:421-469, 510-513, 1520-1537)
    against the oracle: shared_out and the gate score within tolerance."""
    se = B.syn_shared_expert(11)
    dev = {n: tuple(ctx.to_device(np.ascontiguousarray(a)) for a in se[n]) for n in se}
    desc = nh.Context.shared_expert_desc(dev["gate"], dev["up"], dev["down"], dev["score"])
    rng = np.random.default_rng(ntok)
    x = rng.standard_normal((ntok, 2048)).astype(np.float32)
    if xdt == "bf16":
        xb = B.f32_to_bf16(x)
        x, dx, dt = B.bf16_to_f32(xb), ctx.to_device(xb), nh.BF16
    else:
        dx, dt = ctx.to_device(x), nh.F32
    so, gr = ctx.alloc(ntok * 8192), ctx.alloc(ntok * 4)
    ctx._check(ctx.shared_expert(desc, dx, dt, ntok, so, gr))
    want_so, want_g = B.shared_expert(se, x)
    assert_close(so.download(np.float32, (ntok, 2048)), want_so, what="shared_out")
    assert_close(gr.download(np.float32, ntok), want_g, what="shared_gate_raw")


def test_shared_expert_then_layer(ctx, nh):
    """The reference's whole layer tail: the shared expert's outputs feed the
    routed combine, out = h_mid + sum_s w_s y_s + sigmoid(g) * shared_out."""
    seed, bits, k, layer, ntok = 23, 4, 8, 44, 2
    ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    se = B.syn_shared_expert(12)
    dev = {n: tuple(ctx.to_device(np.ascontiguousarray(a)) for a in se[n]) for n in se}
    desc = nh.Context.shared_expert_desc(dev["gate"], dev["up"], dev["down"], dev["score"])
    rng = np.random.default_rng(3)
    x = rng.standard_normal((ntok, 2048)).astype(np.float32)
    h = rng.standard_normal((ntok, 2048)).astype(np.float32)
    idx = np.array([[3, 9, 27, 81, 100, 200, 250, 7], [5, 6, 7, 8, 9, 10, 11, 12]], np.uint32)
    w = np.full((ntok, 8), 0.125, np.float32)
    dx, dh = ctx.to_device(x), ctx.to_device(h)
    so, gr, out = ctx.alloc(ntok * 8192), ctx.alloc(ntok * 4), ctx.alloc(ntok * 8192)
    ctx._check(ctx.shared_expert(desc, dx, nh.F32, ntok, so, gr))
    ctx._check(ctx.experts(bits, layer, dx, nh.F32, ntok, k, ctx.to_device(idx), ctx.to_device(w), dh, out,
                           shared_out=so, shared_gate_raw=gr))
    want_so, want_g = B.shared_expert(se, x)
    pack = host_pack(bits, seed, layer, idx.ravel())
    want = B.moe_experts(pack, bits, x, k, idx, w, h, shared_out=want_so, shared_gate_raw=want_g)
    assert_close(out.download(np.float32, (ntok, 2048)), want, what="layer with the shared expert")


def test_load_expert_dir(nh, tmp_path):
    """nmoe_hip_load_expert_dir: layout.json validated (the converter's
    schema), layer_00.bin made resident byte for byte; a truncated layer file
    is refused with the reference's size check (runtime.m:2444-2451)."""
    import shutil
    import os
    d = tmp_path / "packed_experts_2bit"
    d.mkdir()
    shutil.copy(os.path.join(os.path.dirname(__file__), "golden", "layout_q2.json"), d / "layout.json")
    pack = B.syn_layer(2, 31, 0, SIGMA[2])
    pack.tofile(d / "layer_00.bin")
    c = nh.Context(0, max_tokens=1)
    try:
        assert c.load_expert_dir(str(d), nlayers=1) == (2, 1)
        for e in (0, 129, 255):
            np.testing.assert_array_equal(c.download_expert(0, e, 2), B.syn_expert(2, 31, 0, e, SIGMA[2]))
        with open(d / "layer_00.bin", "r+b") as f:
            f.truncate(pack.nbytes - 1)
        with pytest.raises(nh.NmoeError):
            c.load_expert_dir(str(d), nlayers=1)
        with pytest.raises(nh.NmoeError):  # layout.json says 40 layers; only layer_00.bin exists
            c.load_expert_dir(str(d))
    finally:
        c.close()


@pytest.mark.parametrize("bits", [4, 2])
def test_fused_layer_with_q4_router(ctx, nh, bits):
    """One token through nmoe_moe_layer with the model's q4 router: the fused
    launch (router row per block, kernels.metal:472-513 semantics) routes
    bit-exactly like the oracle and like the multi-launch kernels, and its
    output is within tolerance."""
    rng = np.random.default_rng(40 + bits)
    seed, k, layer = 41, 8, 30 + bits
    ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    wq = rng.integers(0, 2**32, size=(256, 256), dtype=np.uint64).astype(np.uint32)
    sq = B.f32_to_bf16((rng.standard_normal((256, 32)) * 0.01).astype(np.float32))
    bq = B.f32_to_bf16((-8 * B.bf16_to_f32(sq)).astype(np.float32))
    rq = ctx.router_q4(ctx.to_device(wq), ctx.to_device(sq), ctx.to_device(bq))
    x = rng.standard_normal(2048).astype(np.float32)
    h = rng.standard_normal(2048).astype(np.float32)
    dx, dh = ctx.to_device(x), ctx.to_device(h)
    lg_want = np.zeros(256, np.float32)
    B.oracle().orc_router_logits_q4(wq.ctypes.data, sq.ctypes.data, bq.ctypes.data, x.ctypes.data, 256, 2048,
                                    lg_want.ctypes.data)
    oi, ow, _ = B.route(lg_want, k)
    want = B.moe_experts(host_pack(bits, seed, layer, oi[:k]), bits, x[None], k, oi[None], ow[None], h[None])[0]
    for fused in (True, False):
        ctx.set_fused(fused)
        out, idx, w, lg = ctx.alloc(8192), ctx.alloc(32), ctx.alloc(32), ctx.alloc(1024)
        ctx._check(ctx.moe_layer(layer, rq, dx, nh.F32, 1, k, dh, out, idx, w, lg))
        assert ctx.device_status() == nh.OK
        np.testing.assert_array_equal(lg.download(np.float32, 256).view(np.uint32), lg_want.view(np.uint32))
        np.testing.assert_array_equal(idx.download(np.uint32, 8), oi, err_msg=f"fused={fused}")
        np.testing.assert_array_equal(w.download(np.float32, 8).view(np.uint32), ow.view(np.uint32))
        assert_close(out.download(np.float32, 2048), want, what=f"q4 router fused={fused}")
    ctx.set_fused(True)


def test_router_q4_scaled_one_hot_on_device(ctx, nh):
    """The q4 router kernel on x = v e_j: each logit is the reference's
    per-element form fma(q, fl(s v), fl(b v)) rounded once
    (kernels.metal:500-508), computed here from the closed form, not from
    the oracle; scales and biases independent, so a swapped pair, a wrong
    group or a wrong nibble fails."""
    rng = np.random.default_rng(55)
    wq = rng.integers(0, 2**32, size=(256, 256), dtype=np.uint64).astype(np.uint32)
    sq = B.f32_to_bf16((rng.standard_normal((256, 32)) * 0.02).astype(np.float32))
    bq = B.f32_to_bf16((rng.standard_normal((256, 32)) * 0.05).astype(np.float32))
    q = ((wq[:, :, None] >> (np.arange(8, dtype=np.uint32) * 4)) & 15).reshape(256, 2048)
    rq = ctx.router_q4(ctx.to_device(wq), ctx.to_device(sq), ctx.to_device(bq))
    cols = [0, 9, 63, 64, 777, 1546, 2047]
    vals = [np.float32(1.37), np.float32(-0.7133), np.float32(123.456)]
    X = np.zeros((len(cols) * len(vals), 2048), np.float32)
    want = np.zeros((X.shape[0], 256), np.float32)
    s32, b32 = B.bf16_to_f32(sq), B.bf16_to_f32(bq)
    for i, (j, v) in enumerate((j, v) for j in cols for v in vals):
        X[i, j] = v
        sv, bv = s32[:, j // 64] * v, b32[:, j // 64] * v
        want[i] = (q[:, j].astype(np.float64) * sv.astype(np.float64) + bv.astype(np.float64)).astype(np.float32)
    ntok = X.shape[0]
    lg = ctx.alloc(ntok * 1024)
    ctx._check(ctx.router_logits(rq, ctx.to_device(X), nh.F32, ntok, lg))
    got = lg.download(np.float32, (ntok, 256))
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bits", [4, 2])
def test_fused_q4_router_with_rmsnorm(ctx, nh, bits):
    """nmoe_moe_layer_rmsnorm with the model's q4 router: the fused
    <q4 router, in-kernel RMSNorm> variant maps the normalised x onto its
    router columns correctly -- routing bit-exact and output within
    tolerance against the oracle's whole block (orc_moe_block); then a
    two-layer stack of such layers, teacher-forced."""
    rng = np.random.default_rng(70 + bits)
    seed, k = 43, 8
    layers = [34 + 2 * (bits == 2), 35 + 2 * (bits == 2)]
    for layer in layers:
        ctx.synth_layer(layer, bits, seed, SIGMA[bits])
    R = []
    for _ in layers:
        wq = rng.integers(0, 2**32, size=(256, 256), dtype=np.uint64).astype(np.uint32)
        sq = B.f32_to_bf16((rng.standard_normal((256, 32)) * 0.01).astype(np.float32))
        bq = B.f32_to_bf16((rng.standard_normal((256, 32)) * 0.02).astype(np.float32))
        R.append((wq, sq, bq))
    dR = [ctx.router_q4(ctx.to_device(a), ctx.to_device(b_), ctx.to_device(c)) for a, b_, c in R]
    h0 = rng.standard_normal(2048).astype(np.float32) * np.float32(3.0)
    dh, dout = ctx.to_device(h0), ctx.alloc(8192)
    idx, w = ctx.alloc(32), ctx.alloc(32)
    ctx._check(ctx.moe_layer_rmsnorm(layers[0], dR[0], dh, 1e-6, k, dout, idx, w))
    assert ctx.device_status() == nh.OK
    full = B.syn_layer(bits, seed, layers[0], SIGMA[bits])
    want, oi, ow, _, _ = B.moe_block(full, bits, {"q4": R[0]}, h0, k)
    np.testing.assert_array_equal(idx.download(np.uint32, 8), oi)
    np.testing.assert_array_equal(w.download(np.float32, 8).view(np.uint32), ow.view(np.uint32))
    assert_close(dout.download(np.float32, 2048), want, what=f"q{bits} q4-router rmsnorm layer")
    hs = ctx.alloc(3 * 8192)
    hs.upload(h0)
    idx_s, w_s = ctx.alloc(64), ctx.alloc(64)
    ctx._check(ctx.moe_stack(layers, dR, k, 1e-6, hs, idx_s, w_s))
    assert ctx.device_status() == nh.OK
    H = hs.download(np.float32, (3, 2048))
    I, Wt = idx_s.download(np.uint32, (2, 8)), w_s.download(np.float32, (2, 8))
    for l in range(2):
        pack = full if l == 0 else B.syn_layer(bits, seed, layers[1], SIGMA[bits])
        want, oi, ow, _, _ = B.moe_block(pack, bits, {"q4": R[l]}, H[l], k)
        np.testing.assert_array_equal(I[l], oi, err_msg=f"layer {l}")
        np.testing.assert_array_equal(Wt[l].view(np.uint32), ow.view(np.uint32), err_msg=f"layer {l}")
        assert_close(H[l + 1], want, what=f"q{bits} q4-router stack layer {l}")


@pytest.mark.parametrize("bits", [4, 2])
def test_converter_packs_on_device(ctx, nh, bits):
    """The writer side of the format, end to end.  (a) The converter's own
    quantised rows (tests/golden/converter_golden.npz, from
    scripts/convert_qwen36.py:147-211) dequantised by the device probe equal
    math.m's dequant (math.m:206-234) bit for bit.  (b) Experts quantised the
    converter's way (orc_quantize_rows, pinned to the converter's outputs)
    and laid out at its offsets (convert_qwen36.py:38-64, 402-406), uploaded
    unchanged, run through the expert path within tolerance of the oracle."""
    import os
    cg = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "converter_golden.npz"))
    o = B.oracle()
    for name, cols in (("gu", 2048), ("dn", 512)):
        packed, sc, bi = (cg[f"{name}_q{bits}_{t}"] for t in ("packed", "scales", "biases"))
        rows = packed.shape[0]
        out = ctx.alloc(rows * cols * 4)
        ctx._check(ctx.dequant_rows(bits, ctx.to_device(packed), ctx.to_device(sc), ctx.to_device(bi), rows, cols, out))
        got = out.download(np.float32, (rows, cols))
        for r in range(rows):
            want = np.zeros(cols, np.float32)
            o.orc_dequant_row(np.ascontiguousarray(packed[r]).ctypes.data, np.ascontiguousarray(sc[r]).ctypes.data,
                              np.ascontiguousarray(bi[r]).ctypes.data, want.ctypes.data, cols, bits)
            np.testing.assert_array_equal(got[r].view(np.uint32), want.view(np.uint32), err_msg=f"{name} row {r}")
    # (b) a layer of converter-quantised experts
    rng = np.random.default_rng(300 + bits)
    layer, k = 46 + bits, 8
    experts = [3, 77, 140, 255, 0, 9, 200, 31]
    esz = B.EXPERT_SIZE[bits]
    off = np.zeros(9, np.uint64)
    o.orc_expert_offsets(bits, off.ctypes.data)
    pack = np.zeros(256 * esz, np.uint8)
    for e in experts:
        base = e * esz
        for i, (r_, c_) in enumerate(((512, 2048), (512, 2048), (2048, 512))):
            w = B.f32_to_bf16((rng.standard_normal((r_, c_)) * 0.02).astype(np.float32))
            pk, s_, b_ = B.quantize_rows(w, bits)
            for j, arr in enumerate((pk, s_, b_)):
                raw = arr.view(np.uint8).ravel()
                o0 = base + int(off[3 * i + j])
                pack[o0:o0 + raw.size] = raw
    ctx.upload_layer(layer, bits, pack)
    x = B.f32_to_bf16(rng.standard_normal((1, 2048)).astype(np.float32))
    h = rng.standard_normal((1, 2048)).astype(np.float32)
    idx = np.array([experts], np.uint32)
    w = rng.dirichlet(np.ones(k), size=1).astype(np.float32)
    want = B.moe_experts(pack, bits, B.bf16_to_f32(x).reshape(1, 2048), k, idx, w, h)
    out = ctx.alloc(8192)
    ctx._check(ctx.experts(bits, layer, ctx.to_device(x), nh.BF16, 1, k, ctx.to_device(idx), ctx.to_device(w),
                           ctx.to_device(h), out))
    assert ctx.device_status() == nh.OK
    assert_close(out.download(np.float32, (1, 2048)), want, what=f"converter-quantised q{bits} layer")


def _mini_weights(tmp_path):
    import json
    import shutil
    import sys
    import os
    gold = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    sys.path.insert(0, gold)
    import model_weights_recipe as R
    bin_path, json_path = str(tmp_path / "model_weights.bin"), str(tmp_path / "model_weights.json")
    R.write_model_weights(bin_path)
    shutil.copyfile(os.path.join(gold, "model_weights_mini.json"), json_path)
    return R, bin_path, json_path


@pytest.mark.parametrize("bits,k", [(4, 8), (2, 6)])
def test_moe_block_from_model_weights(ctx, nh, tmp_path, bits, k):
    """The model's per-layer MoE half in one launch (nmoe_moe_block)
    with the tensors nmoe_hip_load_model_weights made resident from a
    converter-format model_weights.bin: weighted post-attention RMSNorm, q4
    router, shared expert, experts, combine and the next layer's weighted
    input norm, against the whole-block oracle (orc_moe_block, the
    reference's order runtime.m:3144-3201, 2908-2999, 2893-2900): routing
    bit-exact, out and next_x within tolerance; the in-place form (out over
    h_mid) gives the same bits."""
    R, bin_path, json_path = _mini_weights(tmp_path)
    assert ctx.load_model_weights(bin_path, json_path, 2) == 2
    rng = np.random.default_rng(500 + bits)
    seed = 71
    for l in range(2):
        layer = 60 + l
        ctx.synth_layer(layer, bits, seed, SIGMA[bits])
        blk = ctx.layer_block(l)
        assert blk.has_shared == 1 and blk.add_one == 1 and abs(blk.eps - 1e-6) < 1e-12
        assert (blk.next_norm is None) == (l == 1)
        h = (rng.standard_normal(2048) * 2.0).astype(np.float32)
        dh, out, nx, di, dw = ctx.to_device(h), ctx.alloc(8192), ctx.alloc(8192), ctx.alloc(32), ctx.alloc(32)
        ctx._check(ctx.moe_block(layer, blk, dh, k, out, nx, di, dw))
        assert ctx.device_status() == nh.OK
        got_out, got_nx = out.download(np.float32, 2048), nx.download(np.float32, 2048)
        gi, gw = di.download(np.uint32, 8), dw.download(np.float32, 8)
        host = R.layer_host(l)
        next_norm = R.layer_host(l + 1)["input_norm"] if l == 0 else None
        pack = host_pack(bits, seed, layer, gi[:k])
        want, oi, ow, _, want_nx = B.moe_block(pack, bits, {"q4": host["router"]}, h, k, post_norm=host["post_norm"],
                                               add_one=1, shared=host["shared"], next_norm=next_norm, want_next=True)
        np.testing.assert_array_equal(gi, oi, err_msg=f"layer {l}")
        np.testing.assert_array_equal(gw.view(np.uint32), ow.view(np.uint32), err_msg=f"layer {l}")
        assert_close(got_out, want, what=f"block q{bits} layer {l} out")
        assert_close(got_nx, want_nx, what=f"block q{bits} layer {l} next_x")
        # in place: out over h_mid
        ctx._check(ctx.moe_block(layer, blk, dh, k, dh, nx))
        np.testing.assert_array_equal(dh.download(np.float32, 2048).view(np.uint32), got_out.view(np.uint32))


def test_moe_block_coherent_words_and_2_byte_scales(ctx, nh):
    """The block form with every exchange word device-coherent
    (NMOE_HIP_OPT_XCD_LOCAL off) gives the same bits as the die-local form,
    and both match orc_moe_block; the shared expert's scales and biases sit
    at 2-byte (not 16-byte) aligned addresses, the alignment the entry point
    accepts for them, and the bf16 router is used."""
    seed, layer, k = 77, 63, 8
    ctx.synth_layer(layer, 4, seed, SIGMA[4])
    W = B.syn_bf16(256 * 2048, seed, layer, 16, 0.02).reshape(256, 2048)
    se = B.syn_shared_expert(14)
    keep = []

    def odd(a):  # a device copy at an address 2 bytes past a 256-byte boundary
        a = np.ascontiguousarray(a)
        buf = ctx.alloc(a.nbytes + 256)
        keep.append(buf)
        buf.upload(a, offset=2)
        return buf.ptr + 2

    dev = {n: (ctx.to_device(np.ascontiguousarray(se[n][0])), odd(se[n][1]), odd(se[n][2])) for n in se}
    rng = np.random.default_rng(seed)
    post = B.f32_to_bf16((rng.standard_normal(2048) * 0.1).astype(np.float32))
    nxt = B.f32_to_bf16((rng.standard_normal(2048) * 0.1).astype(np.float32))
    blk = nh.MoeBlock()
    blk.router = ctx.router_bf16(ctx.to_device(W))
    blk.has_shared = 1
    blk.shared = nh.Context.shared_expert_desc(dev["gate"], dev["up"], dev["down"], dev["score"])
    blk.post_norm, blk.next_norm = ctx.to_device(post).ptr, ctx.to_device(nxt).ptr
    blk.add_one, blk.eps = 1, 1e-6
    h = (rng.standard_normal(2048) * 1.5).astype(np.float32)
    dh = ctx.to_device(h)
    got = []
    for xl in (1, 0):
        out, nx, di, dw = ctx.alloc(8192), ctx.alloc(8192), ctx.alloc(32), ctx.alloc(32)
        ctx._check(ctx.set_option(nh.OPT_XCD_LOCAL, xl))
        try:
            ctx._check(ctx.moe_block(layer, blk, dh, k, out, nx, di, dw))
            assert ctx.device_status() == nh.OK
        finally:
            ctx.set_option(nh.OPT_XCD_LOCAL, 1)  # back on where the device's placement allows it
        got.append((out.download(np.float32, 2048), nx.download(np.float32, 2048), di.download(np.uint32, 8),
                    dw.download(np.float32, 8)))
    for a, b in zip(got[0], got[1]):
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    out, nx, gi, gw = got[0]
    pack = host_pack(4, seed, layer, gi[:k])
    want, oi, ow, _, want_nx = B.moe_block(pack, 4, {"w": W}, h, k, post_norm=post, add_one=1, shared=se,
                                           next_norm=nxt, want_next=True)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gw.view(np.uint32), ow.view(np.uint32))
    assert_close(out, want, what="block out")
    assert_close(nx, want_nx, what="block next_x")


def test_moe_block_plain_equals_layer_rmsnorm(ctx, nh):
    """With unit norms, no shared expert and no next norm the block is the
    layer with its input RMSNorm: the same bits as nmoe_moe_layer_rmsnorm."""
    seed, layer, k = 73, 62, 8
    ctx.synth_layer(layer, 4, seed, 0.02)
    W = ctx.to_device(B.syn_bf16(256 * 2048, seed, layer, 16, 0.02))
    blk = nh.MoeBlock()
    blk.router = ctx.router_bf16(W)
    blk.eps = 1e-6
    h = (np.random.default_rng(5).standard_normal(2048) * 1.5).astype(np.float32)
    dh, o1, o2 = ctx.to_device(h), ctx.alloc(8192), ctx.alloc(8192)
    ctx._check(ctx.moe_block(layer, blk, dh, k, o1))
    ctx._check(ctx.moe_layer_rmsnorm(layer, ctx.router_bf16(W), dh, 1e-6, k, o2))
    assert ctx.device_status() == nh.OK
    np.testing.assert_array_equal(o1.download(np.float32, 2048).view(np.uint32),
                                  o2.download(np.float32, 2048).view(np.uint32))


def test_load_model_weights_rejects(ctx, nh, tmp_path):
    """Missing layers, a wrong dtype, a truncated file and broken JSON are
    refused with the reference's categories (runtime.m:2278-2297)."""
    import json
    R, bin_path, json_path = _mini_weights(tmp_path)
    lib = nh.lib()
    n = __import__("ctypes").c_int(0)
    # config.num_hidden_layers is 40, the file holds 2
    assert lib.nmoe_hip_load_model_weights(ctx.h, bin_path.encode(), json_path.encode(), 0, None) == nh.ENOENT
    assert "model.layers.2." in ctx.last_error()
    m = json.load(open(json_path))
    m["tensors"]["model.layers.1.mlp.gate.scales"]["dtype"] = "F32"
    bad = str(tmp_path / "bad.json")
    json.dump(m, open(bad, "w"))
    assert lib.nmoe_hip_load_model_weights(ctx.h, bin_path.encode(), bad.encode(), 2, None) == nh.EINVAL
    with open(bad, "w") as f:
        f.write("{\"tensors\": {")
    assert lib.nmoe_hip_load_model_weights(ctx.h, bin_path.encode(), bad.encode(), 2, None) == nh.EINVAL
    short = str(tmp_path / "short.bin")
    with open(bin_path, "rb") as f, open(short, "wb") as g:
        g.write(f.read(1 << 20))
    assert lib.nmoe_hip_load_model_weights(ctx.h, short.encode(), json_path.encode(), 2, None) == nh.EIO
    del n
