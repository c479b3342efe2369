"""Pins the CPU oracle with what the mathematics fixes: closed forms,
invariants, brute force on small inputs, independent float64 computations
and known SplitMix64 outputs.  Each check is chosen so that a plausible slip
(dropped term, wrong index or shift, transposed operand) fails it."""
import ctypes
import math

import numpy as np

from oracle import binding as B

LIBM = ctypes.CDLL("libm.so.6")
LIBM.expf.restype = ctypes.c_float
LIBM.expf.argtypes = [ctypes.c_float]


def test_expf_restatement_matches_libm_sampled():
    """The restated glibc expf equals the host libm on a strided sweep of all
    non-positive floats (the full 2^31 sweep found 0 mismatches)."""
    o = B.oracle()
    bits = np.arange(0x80000000, 0xFF800001, 9973, dtype=np.uint64).astype(np.uint32)
    xs = bits.view(np.float32)
    for x in xs[:: max(1, xs.size // 40000)]:
        a = o.orc_expf_restated(float(x))
        b = LIBM.expf(float(x))
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), float(x)


def test_expf_restatement_close_to_float64_exp():
    o = B.oracle()
    for x in np.linspace(-103, 0, 5001, dtype=np.float32):
        got = o.orc_expf_restated(float(x))
        want = math.exp(float(x))
        assert abs(got - want) <= 0.51 * np.spacing(np.float32(want)) + 1e-45


def test_softmax_topk_invariants():
    rng = np.random.default_rng(1)
    for _ in range(300):
        lg = (rng.standard_normal(256) * rng.choice([0.3, 1, 5])).astype(np.float32)
        k = int(rng.integers(1, 9))
        idx, w, n, probs = B.route(lg, k, want_probs=True)
        assert n == k
        sel = idx[:k].astype(int)
        assert len(set(sel)) == k
        # descending probability, ties by lower index
        for a, b in zip(sel[:-1], sel[1:]):
            assert probs[a] > probs[b] or (probs[a] == probs[b] and a < b)
        # every unselected expert is not better than the last selected
        last = sel[-1]
        for e in range(256):
            if e not in sel:
                assert probs[e] < probs[last] or (probs[e] == probs[last] and e > last)
        assert abs(float(w[:k].astype(np.float64).sum()) - 1.0) <= 1e-6
        assert np.all(idx[k:] == 0) and np.all(w[k:] == 0)
        # float64 softmax agrees to float precision
        ref = np.exp(lg.astype(np.float64) - lg.max())
        ref /= ref.sum()
        np.testing.assert_allclose(probs, ref, rtol=2e-6, atol=1e-12)


def test_route_closed_forms():
    # k = 1 gives weight exactly 1
    idx, w, n = B.route(np.linspace(-1, 1, 256, dtype=np.float32), 1)
    assert n == 1 and idx[0] == 255 and w[0] == np.float32(1.0)
    # equal logits: uniform probabilities, the k lowest indices, weights 1/k
    idx, w, n, probs = B.route(np.full(256, 0.25, np.float32), 8, want_probs=True)
    assert list(idx) == list(range(8))
    assert np.all(probs == np.float32(1.0) / np.float32(256.0))
    assert np.all(w == np.float32(1.0 / 8))
    # bad k is rejected
    assert B.oracle().orc_route(np.zeros(256, np.float32).ctypes.data, 256, 0, np.zeros(8, np.uint32).ctypes.data,
                                np.zeros(8, np.float32).ctypes.data, None) == -1


def test_dequant_one_hot_and_integer_dot():
    """x = e_j makes the matvec return column j of the dequantised matrix
    exactly; scale 1 / bias 0 turns it into an exact integer dot product."""
    o = B.oracle()
    rng = np.random.default_rng(2)
    for bits in (4, 2):
        vpw = 32 // bits
        rows, cols = 16, 2048
        packed = rng.integers(0, 2**32, size=(rows, cols // vpw), dtype=np.uint64).astype(np.uint32)
        sc = B.f32_to_bf16((rng.standard_normal((rows, cols // 64)) * 0.02).astype(np.float32))
        bi = B.f32_to_bf16((rng.standard_normal((rows, cols // 64)) * 0.1).astype(np.float32))
        deq = np.zeros((rows, cols), np.float32)
        for r in range(rows):
            o.orc_dequant_row(packed[r].ctypes.data, sc[r].ctypes.data, bi[r].ctypes.data, deq[r].ctypes.data, cols, bits)
        # independent unpack: field v of word w is column w*vpw + v
        q = ((packed[:, :, None] >> (np.arange(vpw, dtype=np.uint32) * bits)) & ((1 << bits) - 1)).reshape(rows, cols)
        want = q.astype(np.float32) * np.repeat(B.bf16_to_f32(sc), 64, axis=1) + np.repeat(B.bf16_to_f32(bi), 64, axis=1)
        np.testing.assert_array_equal(deq, want)
        for j in (0, 1, 63, 64, 777, 2047):
            x = np.zeros(cols, np.float32)
            x[j] = 1.0
            y = np.zeros(rows, np.float32)
            o.orc_dequant_matvec(packed.ctypes.data, sc.ctypes.data, bi.ctypes.data, x.ctypes.data, y.ctypes.data,
                                 rows, cols, bits)
            np.testing.assert_array_equal(y, deq[:, j])
        one = np.full_like(sc, B.f32_to_bf16(np.float32([1.0]))[0])
        zero = np.zeros_like(bi)
        xi = rng.integers(-50, 50, cols).astype(np.float32)
        y = np.zeros(rows, np.float32)
        o.orc_dequant_matvec(packed.ctypes.data, one.ctypes.data, zero.ctypes.data, xi.ctypes.data, y.ctypes.data,
                             rows, cols, bits)
        np.testing.assert_array_equal(y.astype(np.int64), q.astype(np.int64) @ xi.astype(np.int64))


def test_router_logits_mirror_equals_float64_dot():
    rng = np.random.default_rng(3)
    w = B.f32_to_bf16((rng.standard_normal((256, 2048)) * 0.02).astype(np.float32))
    x = rng.standard_normal(2048).astype(np.float32)
    got = B.router_logits_bf16(w, x)
    want = B.bf16_to_f32(w).astype(np.float64) @ x.astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)
    # a transposed / shifted operand would be far off
    assert np.abs(got - np.roll(want, 1)).max() > 1e-2


def test_expert_and_combine_against_float64():
    rng = np.random.default_rng(4)
    for bits, sigma in ((4, 0.02), (2, 0.05)):
        ex = B.syn_expert(bits, 9, 1, 5, sigma)
        o9 = {4: (0, 524288, 557056, 589824, 1114112, 1146880, 1179648, 1703936, 1736704),
              2: (0, 262144, 294912, 327680, 589824, 622592, 655360, 917504, 950272)}[bits]

        def dense(i, rows, cols):
            vpw = 32 // bits
            w = ex[o9[3 * i]:o9[3 * i + 1]].view(np.uint32).reshape(rows, cols // vpw)
            s = B.bf16_to_f32(ex[o9[3 * i + 1]:o9[3 * i + 2]].view(np.uint16).reshape(rows, cols // 64))
            b = B.bf16_to_f32(ex[o9[3 * i + 2]:o9[3 * i + 2] + rows * cols // 64 * 2].view(np.uint16).reshape(rows, cols // 64))
            q = ((w[:, :, None] >> (np.arange(vpw, dtype=np.uint32) * bits)) & ((1 << bits) - 1)).reshape(rows, cols)
            return q * np.repeat(s, 64, 1).astype(np.float64) + np.repeat(b, 64, 1)

        G, U, D = dense(0, 512, 2048), dense(1, 512, 2048), dense(2, 2048, 512)
        x = B.bf16_to_f32(B.f32_to_bf16(rng.standard_normal(2048).astype(np.float32)))
        act = np.zeros(512, np.float32)
        B.oracle().orc_expert_gate_up(ex.ctypes.data, bits, x.ctypes.data, act.ctypes.data)
        g, u = G @ x, U @ x
        want_act = g / (1 + np.exp(-g)) * u
        np.testing.assert_allclose(act, want_act, rtol=1e-4, atol=1e-4)
        y = np.zeros(2048, np.float32)
        B.oracle().orc_expert_down(ex.ctypes.data, bits, act.ctypes.data, y.ctypes.data)
        np.testing.assert_allclose(y, D @ act.astype(np.float64), rtol=1e-4, atol=1e-4)


def test_shared_expert_against_float64_and_one_hot():
    """The shared expert (gate/up -> SwiGLU -> down, plus the score row)
    against float64 dense algebra on the dequantised tensors, and the score
    row with one-hot x equal to that row's dequantised column exactly."""
    se = B.syn_shared_expert(5)

    def dense(t, rows, cols):
        w, s, b = t
        q = ((w.reshape(rows, cols // 8)[:, :, None] >> (np.arange(8, dtype=np.uint32) * 4)) & 15).reshape(rows, cols)
        return q * np.repeat(B.bf16_to_f32(s.reshape(rows, cols // 64)), 64, 1).astype(np.float64) + \
            np.repeat(B.bf16_to_f32(b.reshape(rows, cols // 64)), 64, 1)

    G, U, D, S = dense(se["gate"], 512, 2048), dense(se["up"], 512, 2048), dense(se["down"], 2048, 512), \
        dense(se["score"], 1, 2048)
    rng = np.random.default_rng(6)
    x = rng.standard_normal((2, 2048)).astype(np.float32)
    out, g = B.shared_expert(se, x)
    for t in range(2):
        gg, uu = G @ x[t], U @ x[t]
        act = gg / (1 + np.exp(-gg)) * uu
        np.testing.assert_allclose(out[t], D @ act, rtol=1e-4, atol=2e-4)
        np.testing.assert_allclose(g[t], (S @ x[t])[0], rtol=1e-4, atol=1e-4)
    for j in (0, 777, 2047):
        e = np.zeros(2048, np.float32)
        e[j] = 1.0
        _, gj = B.shared_expert(se, e)
        assert gj[0] == np.float32(S[0, j])


def test_combine_formula():
    rng = np.random.default_rng(6)
    h = rng.standard_normal(2048).astype(np.float32)
    y = rng.standard_normal((8, 2048)).astype(np.float32)
    w = rng.uniform(size=8).astype(np.float32)
    sh = rng.standard_normal(2048).astype(np.float32)
    g = np.float32([0.7])
    out = np.zeros(2048, np.float32)
    B.oracle().orc_combine(h.ctypes.data, y.ctypes.data, w.ctypes.data, 8, sh.ctypes.data, g.ctypes.data,
                           out.ctypes.data, 2048)
    want = h + (w[:, None].astype(np.float64) * y).sum(0) + sh / (1 + math.exp(-0.7))
    np.testing.assert_allclose(out, want, atol=1e-5)
    out2 = np.zeros(2048, np.float32)
    B.oracle().orc_combine(h.ctypes.data, y.ctypes.data, w.ctypes.data, 3, None, None, out2.ctypes.data, 2048)
    np.testing.assert_allclose(out2, h + (w[:3, None].astype(np.float64) * y[:3]).sum(0), atol=1e-5)


def test_dispatch_is_stable_sort():
    rng = np.random.default_rng(7)
    for ntok, k in ((1, 8), (64, 8), (2048, 8), (33, 6)):
        idx = np.zeros((ntok, 8), np.uint32)
        idx[:, :k] = rng.integers(0, 256, size=(ntok, k))
        perm, offsets = B.dispatch(idx, ntok, k, 8)
        flat = idx[:, :k].reshape(-1)
        want = np.argsort(flat, kind="stable")
        np.testing.assert_array_equal(perm, want)
        np.testing.assert_array_equal(offsets, np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=256))]))


def test_splitmix64_known_values():
    """orc_syn_rand64(0, i) is the canonical SplitMix64 sequence from state 0."""
    o = B.oracle()
    assert o.orc_syn_rand64(0, 0) == 0xE220A8397B1DCDAF
    assert o.orc_syn_rand64(0, 1) == 0x6E789E6AA1B965F4
    assert o.orc_syn_rand64(0, 2) == 0x06C45D188009454F


def test_generator_distribution_and_layout():
    o = B.oracle()
    st = o.orc_syn_stream(123, 4, 5, 1)
    z = np.array([o.orc_syn_normal(st, i) for i in range(200000)], np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.var() - 1.0) < 0.01 and z.min() >= -6 and z.max() <= 6
    for bits, sigma in ((4, 0.02), (2, 0.05)):
        ex = B.syn_expert(bits, 1, 2, 3, sigma)
        assert ex.size == B.EXPERT_SIZE[bits]
        o9 = {4: (524288, 557056), 2: (262144, 294912)}[bits]
        s = B.bf16_to_f32(ex[o9[0]:o9[1]].view(np.uint16))
        b = B.bf16_to_f32(ex[o9[1]:o9[1] + 32768].view(np.uint16))
        assert abs(s.std() - sigma) < 0.05 * sigma
        if bits == 4:
            np.testing.assert_array_equal(b, -8.0 * s)  # exact: power of two
        else:
            np.testing.assert_array_equal(b, B.bf16_to_f32(B.f32_to_bf16((np.float32(-1.5) * s).astype(np.float32))))
        vpw = 32 // bits
        w = ex[:o9[0]].view(np.uint32)
        q = ((w[:, None] >> (np.arange(vpw, dtype=np.uint32) * bits)) & ((1 << bits) - 1)).ravel()
        counts = np.bincount(q, minlength=1 << bits) / q.size
        assert np.all(np.abs(counts - 1.0 / (1 << bits)) < 0.01)


def test_pack_layout_closed_form():
    """Offsets/sizes follow from the dims: gate/up [512][2048], down [2048][512],
    group 64, bf16 scales and biases (convert_qwen36.py:38-64)."""
    for bits in (4, 2):
        vpw = 32 // bits
        sizes = [512 * 2048 // vpw * 4, 512 * 32 * 2, 512 * 32 * 2] * 2 + [2048 * 512 // vpw * 4, 2048 * 8 * 2, 2048 * 8 * 2]
        offs = np.concatenate([[0], np.cumsum(sizes)])
        assert offs[-1] == B.EXPERT_SIZE[bits] == B.oracle().orc_expert_size(bits)
        arr = (ctypes.c_size_t * 9)()
        B.oracle().orc_expert_offsets(bits, arr)
        assert list(arr) == list(offs[:9])


def _q4_router_case(seed):
    """A q4 router with scales and biases drawn independently (a swapped
    scale/bias, a wrong group or nibble then shows), and its dense float64
    dequantisation."""
    rng = np.random.default_rng(seed)
    wq = rng.integers(0, 2**32, size=(256, 256), dtype=np.uint64).astype(np.uint32)
    sq = B.f32_to_bf16((rng.standard_normal((256, 32)) * 0.02).astype(np.float32))
    bq = B.f32_to_bf16((rng.standard_normal((256, 32)) * 0.05).astype(np.float32))
    q = ((wq[:, :, None] >> (np.arange(8, dtype=np.uint32) * 4)) & 15).reshape(256, 2048)
    dense = q * np.repeat(B.bf16_to_f32(sq), 64, 1).astype(np.float64) + np.repeat(B.bf16_to_f32(bq), 64, 1)
    return rng, wq, sq, bq, q, dense


def _q4_logits(wq, sq, bq, x):
    out = np.zeros(256, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    B.oracle().orc_router_logits_q4(wq.ctypes.data, sq.ctypes.data, bq.ctypes.data, x.ctypes.data, 256, 2048,
                                    out.ctypes.data)
    return out


def test_router_q4_against_float64_dot():
    """orc_router_logits_q4 (kernels.metal:472-513) against a float64 dot of
    the dequantised router: within a bound of 64 fp32 roundings of the
    largest partial sum, far from a shifted row."""
    rng, wq, sq, bq, q, dense = _q4_router_case(31)
    for _ in range(3):
        x = rng.standard_normal(2048).astype(np.float32)
        got = _q4_logits(wq, sq, bq, x)
        want = dense @ x.astype(np.float64)
        bound = 64 * 2.0**-24 * np.abs(dense * x.astype(np.float64)).sum(1)
        assert np.all(np.abs(got - want) <= bound)
        assert np.abs(got - np.roll(want, 1)).max() > 1.0


def test_router_q4_scaled_one_hot_closed_form():
    """x = v e_j leaves one term: the logit of row e is exactly the
    reference's per-element form fma(q, fl(s v), fl(b v)) rounded once
    (kernels.metal:500-508), with q the nibble j % 8 of word j / 8 and s, b
    the scale and bias of group j / 64.  The same value through the other
    association, fl(fl(q s + b) v), differs on most rows, so the test tells
    the two forms apart."""
    from fractions import Fraction
    _, wq, sq, bq, q, _ = _q4_router_case(32)
    s32, b32 = B.bf16_to_f32(sq), B.bf16_to_f32(bq)
    differs = 0
    for j in (0, 7, 8, 63, 64, 1000, 1543, 2047):
        for v in (np.float32(1.37), np.float32(-0.7133), np.float32(3.1e-3), np.float32(123.456)):
            x = np.zeros(2048, np.float32)
            x[j] = v
            got = _q4_logits(wq, sq, bq, x)
            g = j // 64
            sv = s32[:, g] * v  # fp32 products, correctly rounded
            bv = b32[:, g] * v
            qj = q[:, j].astype(np.float64)
            exact = qj * sv.astype(np.float64) + bv.astype(np.float64)
            for e in (0, 77, 255):  # the sum is exact in double, so one rounding to fp32 is the fma
                assert Fraction(float(exact[e])) == Fraction(int(q[e, j])) * Fraction(float(sv[e])) + \
                    Fraction(float(bv[e]))
            want = exact.astype(np.float32)
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=f"j={j} v={v}")
            other = ((q[:, j].astype(np.float32) * s32[:, g] + b32[:, g]) * v).astype(np.float32)
            differs += int(np.count_nonzero(other.view(np.uint32) != want.view(np.uint32)))
    assert differs > 100
