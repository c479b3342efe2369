"""The writer side of the expert-pack format: the oracle's restatement of
scripts/convert_qwen36.py:147-211 (quantise + pack) against the converter's
own outputs (tests/golden/converter_golden.npz, written by
make_converter_golden.py where the reference is present), and what the
mathematics fixes about them."""
import os

import numpy as np
import pytest

from oracle import binding as B

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "converter_golden.npz")


@pytest.fixture(scope="module")
def cg():
    return np.load(GOLDEN)


@pytest.mark.parametrize("name", ["gu", "dn"])
@pytest.mark.parametrize("bits", [4, 2])
def test_quantiser_matches_converter(cg, name, bits):
    rows = cg[f"{name}_q{bits}_rows"]
    packed, scales, biases = B.quantize_rows(rows, bits)
    np.testing.assert_array_equal(packed, cg[f"{name}_q{bits}_packed"])
    np.testing.assert_array_equal(scales, cg[f"{name}_q{bits}_scales"])
    np.testing.assert_array_equal(biases, cg[f"{name}_q{bits}_biases"])


@pytest.mark.parametrize("bits", [4, 2])
def test_converter_packing_is_math_m_bit_order(cg, bits):
    """The converter's packer and math.m's unpack (math.m:191-204) agree on
    the bit order: unpacking the converter's words gives back its codes."""
    codes, words = cg[f"pack{bits}_codes"], cg[f"pack{bits}_words"]
    o = B.oracle()
    for r in range(codes.shape[0]):
        out = np.zeros(256, np.uint16)
        o.orc_unpack_row(np.ascontiguousarray(words[r]).ctypes.data, out.ctypes.data, 256, bits)
        np.testing.assert_array_equal(out, codes[r])


def _codes(packed, bits, cols):
    vpw = 32 // bits
    return ((packed[:, :, None] >> (np.arange(vpw, dtype=np.uint32) * bits)) & ((1 << bits) - 1)).reshape(-1, cols)


def test_converter_ties_round_to_even_and_zero_range(cg):
    """Crafted rows: a group with min 0 and max 15 has scale exactly 1, so
    each code is rint(x) with .5 going to the even neighbour; a constant
    group (zero range) gets scale 0 and code 0 (the safe scale of 1 is used
    for the division only); the same for q2 with max 3."""
    rows = B.bf16_to_f32(cg["gu_q4_rows"])
    q = _codes(cg["gu_q4_packed"], 4, 2048)
    np.testing.assert_array_equal(q[1], np.rint(rows[1]).astype(np.int64))
    assert set(q[1][:64][2:17].tolist()) >= {0, 2, 4, 6, 8, 10, 12, 14}  # 0.5 -> 0, 2.5 -> 2, ...
    np.testing.assert_array_equal(q[0], 0)
    assert np.all(cg["gu_q4_scales"][0] == 0)
    np.testing.assert_array_equal(B.bf16_to_f32(cg["gu_q4_biases"][0]), rows[0][::64])
    rows2 = B.bf16_to_f32(cg["gu_q2_rows"])
    q2 = _codes(cg["gu_q2_packed"], 2, 2048)
    np.testing.assert_array_equal(q2[2], np.rint(rows2[2]).astype(np.int64))


@pytest.mark.parametrize("name,cols", [("gu", 2048), ("dn", 512)])
@pytest.mark.parametrize("bits", [4, 2])
def test_converter_round_trip_error_bound(cg, name, cols, bits):
    """Dequantising the converter's output (math.m:206-234) gives back each
    finite input to within half a quantisation step plus the bf16 rounding
    of the stored scale and minimum."""
    rows = B.bf16_to_f32(cg[f"{name}_q{bits}_rows"]).astype(np.float64)
    packed, sc, bi = cg[f"{name}_q{bits}_packed"], cg[f"{name}_q{bits}_scales"], cg[f"{name}_q{bits}_biases"]
    o = B.oracle()
    qmax = 15.0 if bits == 4 else 3.0
    g = rows.reshape(rows.shape[0], -1, 64)
    s_exact = (g.max(2) - g.min(2)) / qmax
    for r in range(rows.shape[0]):
        deq = np.zeros(cols, np.float32)
        o.orc_dequant_row(np.ascontiguousarray(packed[r]).ctypes.data, np.ascontiguousarray(sc[r]).ctypes.data,
                          np.ascontiguousarray(bi[r]).ctypes.data, deq.ctypes.data, cols, bits)
        s_b = B.bf16_to_f32(sc[r]).astype(np.float64)
        m_b = B.bf16_to_f32(bi[r]).astype(np.float64)
        bound = 0.5 * s_exact[r] * 1.0001 + qmax * np.abs(s_b - s_exact[r]) + np.abs(m_b - g[r].min(1))
        err = np.abs(deq.astype(np.float64).reshape(-1, 64) - g[r])
        assert np.all(err <= bound[:, None] + 1e-45), (name, bits, r, float((err - bound[:, None]).max()))
