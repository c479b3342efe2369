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

float h_u64e_to_f32(uint64_t m, int e) { return nmoe_u64e_to_f32_rne(m, e); }

float h_sqrtf(float v) { return nmoe_sqrtf_rn(v); }
