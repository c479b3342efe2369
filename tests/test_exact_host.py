"""The library's bit-exact routing arithmetic (csrc/nmoe_exact.h), built for
the host, against libm expf and native x87 `long double` running sums -- the
operations math.m:67-93 and math.m:34-65 perform on the reference's host."""
import ctypes
import math
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBM = ctypes.CDLL("libm.so.6")
LIBM.expf.restype = ctypes.c_float
LIBM.expf.argtypes = [ctypes.c_float]
LIBM.exp2l.restype = ctypes.c_longdouble
LIBM.exp2l.argtypes = [ctypes.c_longdouble]


@pytest.fixture(scope="module")
def h(tmp_path_factory):
    d = tmp_path_factory.mktemp("exact")
    so = str(d / "libexact.so")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fPIC", "-shared", "-std=gnu11",
                    "-I", os.path.join(ROOT, "nano-metal-moe-qwen36_amd", "csrc"),
                    os.path.join(ROOT, "tests", "exact_harness.c"), "-o", so, "-lm"], check=True)
    lib = ctypes.CDLL(so)
    P = ctypes.c_void_p
    lib.h_tab.restype, lib.h_tab.argtypes = ctypes.c_uint64, [ctypes.c_int]
    lib.h_expf.restype, lib.h_expf.argtypes = ctypes.c_float, [ctypes.c_float]
    for n in ("h_x87_sum", "h_native_sum", "h_native_mean_sq"):
        getattr(lib, n).restype = ctypes.c_float
        getattr(lib, n).argtypes = [P, ctypes.c_int]
    lib.h_x87_mean_sq.restype, lib.h_x87_mean_sq.argtypes = ctypes.c_float, [P, ctypes.c_int, ctypes.c_int]
    lib.h_fixed_sum.restype, lib.h_fixed_sum.argtypes = ctypes.c_int, [P, ctypes.c_int, P]
    lib.h_u64e_to_f32.restype, lib.h_u64e_to_f32.argtypes = ctypes.c_float, [ctypes.c_uint64, ctypes.c_int]
    lib.h_sqrtf.restype, lib.h_sqrtf.argtypes = ctypes.c_float, [ctypes.c_float]
    lib.h_tree_mean_sq.restype, lib.h_tree_mean_sq.argtypes = ctypes.c_float, [P]
    return lib


def test_exp2_table_entries(h):
    for i in range(32):
        d = np.float64(LIBM.exp2l(i / 32.0))
        want = int(d.view(np.uint64)) - (i << 47)
        assert h.h_tab(i) == want, i


def test_expf_matches_libm(h):
    bits = np.arange(0x80000000, 0xFF800001, 104729, dtype=np.uint64).astype(np.uint32)
    for x in bits.view(np.float32):
        a, b = h.h_expf(float(x)), LIBM.expf(float(x))
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), float(x)
    for x in (0.0, -0.0, float("-inf"), -87.5, -103.9, -104.0, -200.0):
        assert np.float32(h.h_expf(x)).view(np.uint32) == np.float32(LIBM.expf(x)).view(np.uint32)


def test_expf_matches_libm_densely(h):
    """Every 61st bit pattern of the whole float line (both signs: the
    softmax's arguments are <= 0, NaN or -inf; the rest covers overflow), and
    every bit pattern from -88 to -104, where e_expf.c's special-case block
    begins, against libm expf."""
    h.h_expf_mismatches.restype = ctypes.c_long
    h.h_expf_mismatches.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
    assert h.h_expf_mismatches(0, 0xFFFFFFFF, 61) == 0
    lo, hi = int(np.float32(-88.0).view(np.uint32)), int(np.float32(-104.0).view(np.uint32))
    assert h.h_expf_mismatches(lo, hi + 1, 1) == 0
    for x in (float("nan"), float("inf"), 88.72283935546875, 88.7228469848632812, -103.97207641601562):
        a, b = np.float32(h.h_expf(x)), np.float32(LIBM.expf(x))
        assert (np.isnan(a) and np.isnan(b)) or a.view(np.uint32) == b.view(np.uint32), x


def test_x87_emulation_matches_long_double(h):
    rng = np.random.default_rng(11)
    for trial in range(400):
        n = int(rng.integers(1, 300))
        scale = rng.choice([1e-12, 1e-6, 1.0, 1e3])
        v = np.abs(rng.standard_normal(n) * scale).astype(np.float32)
        if trial % 3 == 0:  # terms spanning > 64 binades force rounding in the running sum
            v = (np.exp(rng.uniform(-60, 0, n)) * rng.uniform(0.5, 1, n)).astype(np.float32)
        if trial % 7 == 0:
            v[rng.integers(0, n)] = 0.0
        a = h.h_x87_sum(v.ctypes.data, n)
        b = h.h_native_sum(v.ctypes.data, n)
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), trial


def test_x87_mean_square_matches_long_double(h):
    rng = np.random.default_rng(12)
    for trial in range(60):
        v = (rng.standard_normal(2048) * rng.choice([1e-3, 1.0, 50.0])).astype(np.float32)
        a = h.h_x87_mean_sq(v.ctypes.data, 2048, 11)
        b = h.h_native_mean_sq(v.ctypes.data, 2048)
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), trial


def test_tree_mean_square_fast_path(h):
    """The device norm's double tree sum: wherever it takes its fast path
    the float equals math.m's long double mean square bit for bit; at float
    rounding midpoints it declines (the x87 replay takes over)."""
    rng = np.random.default_rng(15)
    taken = 0
    for trial in range(400):
        scale = rng.choice([1e-18, 1e-3, 1.0, 50.0, 1e15])
        v = (rng.standard_normal(2048) * scale).astype(np.float32)
        if trial % 4 == 1:  # wide dynamic range within one vector
            v *= (np.float32(2.0) ** rng.integers(-40, 40, 2048)).astype(np.float32)
        if trial % 4 == 2:  # few large terms
            v[rng.integers(0, 2048, 5)] = np.float32(1e4)
        m = h.h_tree_mean_sq(v.ctypes.data)
        want = h.h_native_mean_sq(v.ctypes.data, 2048)
        if m >= 0.0:
            taken += 1
            assert np.float32(m).view(np.uint32) == np.float32(want).view(np.uint32), trial
    assert taken >= 300  # declines: means outside the normal float range
    # exact midpoints of two floats: mean 1 + 2^-11 + 2^-24 (h = 1 + 2^-12)
    for v in (np.full(2048, 1 + 2 ** -12, np.float32), np.full(2048, 2 * (1 + 2 ** -12), np.float32)):
        assert h.h_tree_mean_sq(v.ctypes.data) == -1.0
    z = np.zeros(2048, np.float32)
    assert h.h_tree_mean_sq(z.ctypes.data) == 0.0
    tiny = np.full(2048, 1e-30, np.float32)  # mean square below the normal range
    assert h.h_tree_mean_sq(tiny.ctypes.data) == -1.0


def test_fixed_point_fast_path(h):
    """Terms >= 2^-32 (in [0,1]): the integer sum equals the exact sum, and
    math.m's long double running sum is exact there too."""
    rng = np.random.default_rng(13)
    out = np.zeros(1, np.float32)
    for trial in range(300):
        lg = (rng.standard_normal(256) * rng.choice([0.5, 1.0, 3.0])).astype(np.float32)
        e = np.array([LIBM.expf(float(x)) for x in (lg - lg.max())], np.float32)
        if e[e > 0].min() < 2.0 ** -32:
            continue
        assert h.h_fixed_sum(e.ctypes.data, 256, out.ctypes.data) == 1
        b = h.h_native_sum(e.ctypes.data, 256)
        assert out[0].view(np.uint32) == np.float32(b).view(np.uint32)
    tiny = np.array([1.0, 2.0 ** -33], np.float32)
    assert h.h_fixed_sum(tiny.ctypes.data, 2, out.ctypes.data) == 0


def test_u64_to_float_rounding(h):
    rng = np.random.default_rng(14)
    for _ in range(2000):
        m = int(rng.integers(1, 2**63, dtype=np.uint64))
        e = int(rng.integers(-80, 40))
        got = h.h_u64e_to_f32(m, e)
        # float(int) is correctly rounded in Python; scaling by 2^e is exact here
        want = np.float32(math.ldexp(float(m), e)) if m < 2**53 else np.float32(m * 2.0 ** e)
        if m >= 2**53:
            # exact reference via fractions
            from fractions import Fraction
            want = np.float32(float(Fraction(m) * Fraction(2) ** e))  # double rounding free: check below
            # float(Fraction) rounds once to double; then to float32 may double-round, so compare by bounds
            lo, hi = np.nextafter(np.float32(got), np.float32(-np.inf)), np.nextafter(np.float32(got), np.float32(np.inf))
            exact = Fraction(m) * Fraction(2) ** e
            assert abs(Fraction(float(got)) - exact) <= abs(Fraction(float(lo)) - exact)
            assert abs(Fraction(float(got)) - exact) <= abs(Fraction(float(hi)) - exact)
        else:
            assert np.float32(got) == want


def test_sqrtf_correctly_rounded(h):
    """nmoe_sqrtf_rn == libm sqrtf (IEEE correctly rounded) on a sweep of
    positive normal floats, including the neighbours of exact squares."""
    LIBM.sqrtf.restype, LIBM.sqrtf.argtypes = ctypes.c_float, [ctypes.c_float]
    bits = np.arange(0x00800000, 0x7f800000, 7919, dtype=np.uint64).astype(np.uint32)
    vals = list(bits.view(np.float32))
    for r in (1.0, 1.5, 3.0, 1.0031055, 7.25):
        sq = np.float32(np.float32(r) * np.float32(r))
        vals += [sq, np.nextafter(sq, np.float32(0)), np.nextafter(sq, np.float32(np.inf))]
    for v in vals:
        a, b = h.h_sqrtf(float(v)), LIBM.sqrtf(float(v))
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), float(v)
