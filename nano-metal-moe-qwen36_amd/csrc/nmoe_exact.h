/*
 * nmoe_exact.h -- bit-exact restatements of the host arithmetic the
 * reference's CPU router depends on, usable on the GPU and on the host.
 *
 * The reference routes on the host (runtime.m:1498-1511) with math.m's
 * softmax (math.m:67-93): glibc expf, an x87 `long double` running sum,
 * float conversions.  Top-k (math.m:95-132) breaks ties by lower index, so
 * two different logits whose probabilities round to the same float are
 * ordered by index: reproducing the selected indices bit-exactly needs the
 * probabilities bit-exactly.  This header provides:
 *
 *   nmoe_expf_glibc      glibc's expf (sysdeps/ieee754/flt-32/e_expf.c, the
 *                        ARM optimized-routines method: x*32/ln2 = k + r,
 *                        2^(k/32) from a 32-entry table, cubic in r, all in
 *                        double) with every multiply-add fused, which is the
 *                        variant x86-64 glibc selects on FMA hosts.
 *   nmoe_x87_*           80-bit extended addition with round-to-nearest-even
 *                        on a 64-bit significand (positive operands only), to
 *                        replay math.m's `long double` running sums exactly.
 *   nmoe_u64_to_f32_rne  correctly rounded integer -> float conversion.
 *
 * Compiles as C (gcc, for host-side pinning tests) and as HIP device code.
 * Must be compiled without FP contraction (-ffp-contract=off): every fused
 * operation below is written with fma().
 */
#ifndef NMOE_EXACT_H
#define NMOE_EXACT_H

#include <stdint.h>

#if defined(__HIPCC__)
#define NMOE_HD __host__ __device__ __forceinline__
#else
#include <math.h>
#include <string.h>
#define NMOE_HD static inline
#endif

NMOE_HD uint64_t nmoe_dbl_bits(double d) {
#if defined(__HIPCC__)
    return (uint64_t)__builtin_bit_cast(unsigned long long, d);
#else
    uint64_t u;
    memcpy(&u, &d, 8);
    return u;
#endif
}

NMOE_HD double nmoe_bits_dbl(uint64_t u) {
#if defined(__HIPCC__)
    return __builtin_bit_cast(double, (unsigned long long)u);
#else
    double d;
    memcpy(&d, &u, 8);
    return d;
#endif
}

NMOE_HD uint32_t nmoe_flt_bits(float f) {
#if defined(__HIPCC__)
    return __builtin_bit_cast(uint32_t, f);
#else
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
#endif
}

NMOE_HD float nmoe_bits_flt(uint32_t u) {
#if defined(__HIPCC__)
    return __builtin_bit_cast(float, u);
#else
    float f;
    memcpy(&f, &u, 4);
    return f;
#endif
}

NMOE_HD int nmoe_clz64(uint64_t v) {
#if defined(__HIPCC__)
    return v == 0 ? 64 : __builtin_clzll(v);
#else
    return v == 0 ? 64 : __builtin_clzll(v);
#endif
}

/* Entry i is 2^(i/32) rounded to double with i<<47 subtracted, so that adding
 * k<<47 to entry k%32 yields the bits of 2^(k/32) (a host test recomputes
 * every entry from exp2l). */
#define NMOE_EXP2_TAB32                                                                           \
    {                                                                                             \
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
            0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
            0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
            0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
            0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
            0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
            0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
            0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull  \
    }

/* glibc expf, FMA variant.  tab = NMOE_EXP2_TAB32 (constant memory on the
 * device).  Special cases follow e_expf.c: -inf -> 0, NaN/inf propagate,
 * overflow -> inf, x < log(2^-150) -> 0.  Branch-free: the main path runs
 * for every x (its table index is in range for any input) and the special
 * cases are selected afterwards -- the same result as e_expf.c's early
 * returns, which apply only where |x| >= 88 (or x is not finite) and there
 * give exactly these values. */
NMOE_HD float nmoe_expf_glibc(float x, const uint64_t *tab) {
    const double invln2n = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    double xd = (double)x;
    double kd = fma(invln2n, xd, shift);
    uint64_t ki = nmoe_dbl_bits(kd);
    kd -= shift;
    double r = fma(invln2n, xd, -kd);
    uint64_t t = tab[ki % 32] + (ki << 47);
    double s = nmoe_bits_dbl(t);
    double z = fma(c0, r, c1);
    double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    float res = (float)y;
    res = x > 0x1.62e42ep6f ? nmoe_bits_flt(0x7f800000u) : res; /* overflow (and +inf) */
    res = x < -0x1.9fe368p6f ? 0.0f : res;                       /* underflow (and -inf) */
    return x != x ? x + x : res;                                 /* NaN */
}

/* ---------------------------------------------------------------------
 * x87 extended precision (64-bit significand), positive values only.
 * value = m * 2^e, m normalised (bit 63 set) unless the value is zero.
 * ------------------------------------------------------------------- */
typedef struct {
    uint64_t m;
    int32_t e;
} nmoe_x87;

NMOE_HD nmoe_x87 nmoe_x87_zero(void) {
    nmoe_x87 z;
    z.m = 0;
    z.e = 0;
    return z;
}

NMOE_HD nmoe_x87 nmoe_x87_norm(uint64_t mant, int32_t exp2) {
    nmoe_x87 v;
    if (mant == 0) return nmoe_x87_zero();
    int lz = nmoe_clz64(mant);
    v.m = mant << lz;
    v.e = exp2 - lz;
    return v;
}

/* |f| as an extended value (exact). */
NMOE_HD nmoe_x87 nmoe_x87_from_float(float f) {
    uint32_t b = nmoe_flt_bits(f) & 0x7fffffffu;
    uint32_t ex = b >> 23;
    uint64_t mant = b & 0x7fffffu;
    if (ex == 0) return nmoe_x87_norm(mant, -149);
    return nmoe_x87_norm(mant | 0x800000u, (int32_t)ex - 150);
}

/* f*f as an extended value (exact: at most 48 significant bits). */
NMOE_HD nmoe_x87 nmoe_x87_square(float f) {
    nmoe_x87 a = nmoe_x87_from_float(f);
    if (a.m == 0) return a;
    uint64_t top = a.m >> 40; /* 24 significant bits */
    return nmoe_x87_norm(top * top, 2 * (a.e + 40));
}

/* a + b rounded to nearest-even on 64 bits; a, b >= 0. */
NMOE_HD nmoe_x87 nmoe_x87_add(nmoe_x87 a, nmoe_x87 b) {
    if (a.m == 0) return b;
    if (b.m == 0) return a;
    if (a.e < b.e) {
        nmoe_x87 t = a;
        a = b;
        b = t;
    }
    uint32_t d = (uint32_t)(a.e - b.e);
    /* 128-bit fixed point in units of 2^(a.e - 64): a = (a.m : 0). */
    uint64_t bh, bl, sticky = 0;
    if (d == 0) {
        bh = b.m;
        bl = 0;
    } else if (d < 64) {
        bh = b.m >> d;
        bl = b.m << (64 - d);
    } else if (d == 64) {
        bh = 0;
        bl = b.m;
    } else if (d < 128) {
        bh = 0;
        bl = b.m >> (d - 64);
        sticky = (b.m << (128 - d)) != 0;
    } else {
        bh = 0;
        bl = 0;
        sticky = 1;
    }
    uint64_t h = a.m + bh;
    uint64_t carry = h < a.m;
    uint64_t l = bl;
    int32_t e = a.e;
    if (carry) {
        sticky |= l & 1u;
        l = (l >> 1) | (h << 63);
        h = (h >> 1) | (1ull << 63);
        e += 1;
    }
    uint64_t guard = l >> 63;
    uint64_t rest = ((l << 1) != 0) | sticky;
    if (guard && (rest || (h & 1u))) {
        h += 1;
        if (h == 0) {
            h = 1ull << 63;
            e += 1;
        }
    }
    nmoe_x87 r;
    r.m = h;
    r.e = e;
    return r;
}

/* Round a non-negative 64-bit-significand value m*2^e to float (nearest
 * even).  Results below FLT_MIN are not handled (callers' values are >= 1
 * or squares of normal floats). */
NMOE_HD float nmoe_u64e_to_f32_rne(uint64_t m, int32_t e) {
    if (m == 0) return 0.0f;
    int lz = nmoe_clz64(m);
    m <<= lz;
    e -= lz;
    uint64_t t = m >> 40;
    uint64_t rem = m & ((1ull << 40) - 1);
    const uint64_t half = 1ull << 39;
    if (rem > half || (rem == half && (t & 1u))) {
        t += 1;
        if (t == (1ull << 24)) {
            t >>= 1;
            e += 1;
        }
    }
    int32_t bexp = e + 40 + 23 + 127;
    if (bexp >= 255) return nmoe_bits_flt(0x7f800000u);
    if (bexp <= 0) return 0.0f;
    return nmoe_bits_flt(((uint32_t)bexp << 23) | ((uint32_t)t & 0x7fffffu));
}

NMOE_HD float nmoe_x87_to_float(nmoe_x87 a) { return nmoe_u64e_to_f32_rne(a.m, a.e); }

/* u * 2^-55 rounded to float. */
NMOE_HD float nmoe_u64_scaled_to_f32_rne(uint64_t u) { return nmoe_u64e_to_f32_rne(u, -55); }

/* The softmax terms exp(l - max) lie in [0, 1].  When every nonzero term is
 * at least 2^-32 it is an integer multiple of 2^-55, and 256 such terms sum
 * below 2^63: math.m's running long double sum is then exact, equal to this
 * integer sum.  Returns 0 and leaves *out untouched if the term is too small. */
NMOE_HD int nmoe_softmax_term_fixed(float e, uint64_t *out) {
    const uint32_t b = nmoe_flt_bits(e);
    const uint32_t ex = b >> 23;
    const int fits = ex >= 127u - 32u && ex <= 127u;
    const uint64_t mant = (uint64_t)((b & 0x7fffffu) | 0x800000u);
    /* e = mant * 2^(ex-150); times 2^55 -> mant << (ex - 95) (branch-free:
     * the shift count is clamped into range where the term does not fit) */
    const uint64_t v = mant << (fits ? ex - 95u : 0u);
    if (b == 0 || fits) *out = b == 0 ? 0 : v;
    return b == 0 || fits;
}

/* Correctly rounded single-precision square root of v >= 0 (normal range),
 * as sqrtf: an estimate r from double precision, then the exact test against
 * the squares of the neighbouring rounding midpoints (a midpoint has 25
 * significant bits, so its square is exact in double; v never equals one,
 * having only 24). */
NMOE_HD float nmoe_sqrtf_rn(float v) {
    if (!(v > 0.0f)) return v == 0.0f ? v : nmoe_bits_flt(0x7fc00000u);
    double vd = (double)v;
    float r = (float)sqrt(vd);
    uint32_t rb = nmoe_flt_bits(r);
    double up = ((double)r + (double)nmoe_bits_flt(rb + 1u)) * 0.5;
    if (vd > up * up) return nmoe_bits_flt(rb + 1u);
    double dn = ((double)r + (double)nmoe_bits_flt(rb - 1u)) * 0.5;
    if (vd < dn * dn) return nmoe_bits_flt(rb - 1u);
    return r;
}

/* math.m:46-52's mean square of 2048 floats as a float, from S, their
 * squares (each exact in double) summed in double as a binary tree of
 * depth at most 11.  Summing non-negative terms, a tree of depth d is
 * within (1 + 2^-53)^d - 1 < 11.001 * 2^-53 relative of the exact sum;
 * math.m's x87 long double running sum is within 2047 * 2^-64 < 2^-53 of
 * it, and dividing by 2048 is exact in both.  So when no float rounding
 * midpoint lies within 2^-48 (= 32 * 2^-53) relative of S / 2048, math.m's
 * mean rounds to the float S / 2048 rounds to.  Returns that float, or -1
 * when the caller must replay the x87 sum (a near-midpoint, or a mean
 * outside the normal float range). */
NMOE_HD float nmoe_mean_sq_from_sum(double S) {
    const double m = S * (1.0 / 2048.0); /* exact */
    if (m == 0.0) return 0.0f;           /* every square, hence every term, is 0 */
    const float f = (float)m;
    const uint32_t fb = nmoe_flt_bits(f);
    if (fb < 0x00800000u || fb >= 0x7f000000u) return -1.0f;
    const double up = ((double)f + (double)nmoe_bits_flt(fb + 1u)) * 0.5;
    const double dn = ((double)f + (double)nmoe_bits_flt(fb - 1u)) * 0.5;
    const double margin = m * 0x1p-48;
    return (up - m) > margin && (m - dn) > margin ? f : -1.0f;
}

#endif
