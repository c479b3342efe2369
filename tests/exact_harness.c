/* Host build of the library's device-side exact arithmetic
 * (nano-metal-moe-qwen36_amd/csrc/nmoe_exact.h) so CPU tests can pin it
 * against libm expf and native x87 long double sums.  Compiled by
 * tests/test_exact_host.py with gcc -O2 -ffp-contract=off. */
#include <math.h>
#include <stdint.h>

#include "nmoe_exact.h"

static const uint64_t tab[32] = NMOE_EXP2_TAB32;

uint64_t h_tab(int i) { return tab[i]; }
float h_expf(float x) { return nmoe_expf_glibc(x, tab); }

/* The bit patterns start, start + stride, ... below end (as floats) where
 * the restatement and libm expf differ; returns their count. */
long h_expf_mismatches(uint32_t start, uint32_t end, uint32_t stride) {
    long bad = 0;
    for (uint64_t u = start; u < end; u += stride) {
        union { uint32_t u; float f; } a, r, w;
        a.u = (uint32_t)u;
        r.f = nmoe_expf_glibc(a.f, tab);
        w.f = expf(a.f);
        if (r.u != w.u && !(r.f != r.f && w.f != w.f)) bad++;
    }
    return bad;
}

float h_x87_sum(const float *v, int n) {
    nmoe_x87 acc = nmoe_x87_zero();
    for (int i = 0; i < n; i++) acc = nmoe_x87_add(acc, nmoe_x87_from_float(v[i]));
    return nmoe_x87_to_float(acc);
}

float h_native_sum(const float *v, int n) {
    long double acc = 0.0L;
    for (int i = 0; i < n; i++) acc += v[i];
    return (float)acc;
}

/* returns 1 and the float of the exact sum when every term qualifies */
int h_fixed_sum(const float *v, int n, float *out) {
    uint64_t s = 0;
    for (int i = 0; i < n; i++) {
        uint64_t f;
        if (!nmoe_softmax_term_fixed(v[i], &f)) return 0;
        s += f;
    }
    *out = nmoe_u64_scaled_to_f32_rne(s);
    return 1;
}

float h_x87_mean_sq(const float *v, int n, int log2n) {
    nmoe_x87 acc = nmoe_x87_zero();
    for (int i = 0; i < n; i++) acc = nmoe_x87_add(acc, nmoe_x87_square(v[i]));
    acc.e -= log2n;
    return nmoe_x87_to_float(acc);
}

float h_native_mean_sq(const float *v, int n) {
    long double acc = 0.0L;
    for (int i = 0; i < n; i++) {
        long double x = v[i];
        acc += x * x;
    }
    return (float)(acc / (long double)n);
}

/* nmoe_block_rms_exact's double tree over 2048 values, in its order:
 * 8 per thread pairwise, then rows of 16 threads (DPP xor 1, xor 2, half
 * mirror, mirror), the 4 rows of a wavefront, the 4 wavefronts; then
 * nmoe_mean_sq_from_sum (-1: the x87 replay is needed) */
float h_tree_mean_sq(const float *v) {
    double t[256], w[4];
    for (int i = 0; i < 256; i++) {
        double q[8];
        for (int k = 0; k < 8; k++) q[k] = (double)v[8 * i + k] * (double)v[8 * i + k];
        t[i] = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
    }
    for (int wv = 0; wv < 4; wv++) {
        double r[4];
        for (int row = 0; row < 4; row++) {
            double a[16];
            for (int i = 0; i < 16; i++) a[i] = t[64 * wv + 16 * row + i];
            double b[16];
            for (int i = 0; i < 16; i++) b[i] = a[i] + a[i ^ 1];
            for (int i = 0; i < 16; i++) a[i] = b[i] + b[i ^ 2];
            for (int i = 0; i < 16; i++) b[i] = a[i] + a[(i & 8) | (7 - (i & 7))];
            for (int i = 0; i < 16; i++) a[i] = b[i] + b[15 - i];
            r[row] = a[0];
        }
        w[wv] = (r[0] + r[1]) + (r[2] + r[3]);
    }
    return nmoe_mean_sq_from_sum((w[0] + w[1]) + (w[2] + w[3]));
}

float h_u64e_to_f32(uint64_t m, int e) { return nmoe_u64e_to_f32_rne(m, e); }

float h_sqrtf(float v) { return nmoe_sqrtf_rn(v); }
