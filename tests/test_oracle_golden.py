"""The CPU oracle against the reference's own math.m (golden vectors and, when
it is built, oracle/_ref live).  Bit-exact: same operations, same order."""
import numpy as np
import pytest

from oracle import binding as B


def test_route_matches_math_m_golden(golden):
    o = B.oracle()
    for i in range(golden["route_logits"].shape[0]):
        lg = golden["route_logits"][i]
        k = int(golden["route_k"][i])
        idx, w, n, probs = B.route(lg, k, want_probs=True)
        assert n == golden["route_n"][i]
        np.testing.assert_array_equal(probs.view(np.uint32), golden["route_probs"][i].view(np.uint32), err_msg=f"case {i}")
        np.testing.assert_array_equal(idx, golden["route_idx"][i], err_msg=f"case {i}")
        np.testing.assert_array_equal(w.view(np.uint32), golden["route_w"][i].view(np.uint32), err_msg=f"case {i}")
    del o


def test_route_fewer_experts_than_k(golden):
    idx, w, n, probs = B.route(golden["small_logits"], 8, want_probs=True)
    assert n == int(golden["small_n"]) == 5
    np.testing.assert_array_equal(idx, golden["small_idx"])
    np.testing.assert_array_equal(w.view(np.uint32), golden["small_w"].view(np.uint32))


def test_rms_norm_matches_math_m_golden(golden):
    o = B.oracle()
    X = golden["rms_x"]
    for i in range(X.shape[0]):
        y = np.zeros(B.HIDDEN, np.float32)
        o.orc_rms_norm(X[i].ctypes.data, None, y.ctypes.data, B.HIDDEN, 1e-6, 0)
        np.testing.assert_array_equal(y.view(np.uint32), golden["rms_y"][i].view(np.uint32))
    y = np.zeros(B.HIDDEN, np.float32)
    wt = golden["rms_weight"]
    o.orc_rms_norm(X[0].ctypes.data, wt.ctypes.data, y.ctypes.data, B.HIDDEN, 1e-6, 1)
    np.testing.assert_array_equal(y.view(np.uint32), golden["rms_y_weighted"].view(np.uint32))


def test_activations_match_math_m_golden(golden):
    o = B.oracle()
    g, u = golden["act_gate"], golden["act_up"]
    sw = np.zeros_like(g)
    o.orc_swiglu(g.ctypes.data, u.ctypes.data, sw.ctypes.data, g.size)
    np.testing.assert_array_equal(sw.view(np.uint32), golden["act_swiglu"].view(np.uint32))
    sig = np.array([o.orc_sigmoid(float(v)) for v in g], np.float32)
    np.testing.assert_array_equal(sig.view(np.uint32), golden["act_sigmoid"].view(np.uint32))


@pytest.mark.parametrize("bits", [4, 2])
def test_unpack_dequant_matvec_match_math_m_golden(golden, bits):
    o = B.oracle()
    wg, sg, bg = golden[f"q{bits}_packed"], golden[f"q{bits}_scales"], golden[f"q{bits}_biases"]
    rows = wg.shape[0]
    for r in range(rows):
        unp = np.zeros(2048, np.uint16)
        o.orc_unpack_row(wg[r].ctypes.data, unp.ctypes.data, 2048, bits)
        np.testing.assert_array_equal(unp, golden[f"q{bits}_unpacked"][r])
        deq = np.zeros(2048, np.float32)
        o.orc_dequant_row(wg[r].ctypes.data, sg[r].ctypes.data, bg[r].ctypes.data, deq.ctypes.data, 2048, bits)
        np.testing.assert_array_equal(deq.view(np.uint32), golden[f"q{bits}_dequant"][r].view(np.uint32))
    mv = np.zeros(rows, np.float32)
    x = golden[f"q{bits}_x"]
    o.orc_dequant_matvec(wg.ctypes.data, sg.ctypes.data, bg.ctypes.data, x.ctypes.data, mv.ctypes.data, rows, 2048, bits)
    np.testing.assert_array_equal(mv.view(np.uint32), golden[f"q{bits}_matvec"].view(np.uint32))


@pytest.mark.parametrize("name,bits,k,sigma", [("step_q4_k8", 4, 8, 0.02), ("step_q2_k8", 2, 8, 0.05),
                                               ("step_q2_k6", 2, 6, 0.05)])
def test_decode_step_matches_math_m_golden(golden, name, bits, k, sigma):
    """One token through a synthetic layer: routing and expert math from
    math.m in the fixture, from the restatement here; only the 8 selected
    experts are generated."""
    seed, layer = 0, 0
    router = B.syn_bf16(B.EXPERTS * B.HIDDEN, seed, layer, 16, 0.02).reshape(B.EXPERTS, B.HIDDEN)
    x = B.bf16_to_f32(B.syn_bf16(B.HIDDEN, seed, layer, 17, 1.0))
    h_mid = B.bf16_to_f32(B.syn_bf16(B.HIDDEN, seed, layer, 18, 1.0))
    logits = B.router_logits_bf16(router, x)
    np.testing.assert_array_equal(logits.view(np.uint32), golden[f"{name}_logits"].view(np.uint32))
    idx, w, n = B.route(logits, k)
    np.testing.assert_array_equal(idx, golden[f"{name}_idx"])
    np.testing.assert_array_equal(w.view(np.uint32), golden[f"{name}_w"].view(np.uint32))
    esz = B.EXPERT_SIZE[bits]
    pack = np.zeros(B.EXPERTS * esz, np.uint8)
    for s in range(n):
        e = int(idx[s])
        pack[e * esz:(e + 1) * esz] = B.syn_expert(bits, seed, layer, e, sigma)
    out = B.moe_experts(pack, bits, x[None], k, idx[None], w[None], h_mid[None])
    np.testing.assert_array_equal(out[0].view(np.uint32), golden[f"{name}_out"].view(np.uint32))


def test_oracle_against_live_ref_when_built():
    """oracle/_ref (math.m compiled here) vs the restatement on fresh inputs."""
    ref = B.ref_math()
    if ref is None:
        pytest.skip("oracle/_ref not built (needs the reference sources)")
    rng = np.random.default_rng(5)
    for trial in range(200):
        lg = (rng.standard_normal(256) * rng.choice([0.5, 1, 4, 16, 40])).astype(np.float32)
        k = int(rng.integers(1, 9))
        v = lg.copy()
        ref.nmoe_cpu_softmax(v.ctypes.data, 256)
        idx = np.zeros(8, np.uint64)
        val = np.zeros(8, np.float32)
        got = ref.nmoe_cpu_topk(v.ctypes.data, 256, k, idx.ctypes.data, val.ctypes.data)
        ref.nmoe_cpu_renormalize(val.ctypes.data, got)
        oi, ow, on, op = B.route(lg, k, want_probs=True)
        assert on == got
        np.testing.assert_array_equal(op.view(np.uint32), v.view(np.uint32))
        np.testing.assert_array_equal(oi[:got], idx[:got].astype(np.uint32))
        np.testing.assert_array_equal(ow[:got].view(np.uint32), val[:got].view(np.uint32))


def test_f32_to_bf16_matches_math_m_golden(golden):
    """orc_f32_to_bf16 (math.m:14-19) on raw bit patterns against the compiled
    reference: ties to even, carries into the exponent and the sign bit,
    subnormals, the finite values that round to Inf, NaN payloads."""
    bits_in, want = golden["f2bf_in"], golden["f2bf_out"]
    got = np.zeros(bits_in.size, np.uint16)
    B.oracle().orc_f32_to_bf16_bits(bits_in.ctypes.data, got.ctypes.data, bits_in.size)
    np.testing.assert_array_equal(got, want)
    # the vectorised copy the tests use to build bf16 data
    np.testing.assert_array_equal(B.f32_to_bf16(bits_in.view(np.float32)), want)
    # the crafted half covers both tie directions and the exponent carry
    assert want[3] == 0x3F80 and want[4] == 0x3F82 and want[8] == 0x4000
