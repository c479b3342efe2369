/*
 * ref_harness.c -- array entry points around the reference's own math.m
 * routines, linked into oracle/_ref/libnmoe_math_ref.so.
 *
 * TEST INFRASTRUCTURE ONLY (tests/golden/make_golden.py).  A float handed
 * through Python's ctypes passes through a double, which quiets signalling
 * NaNs; these entry points take raw bit patterns instead, so the reference's
 * conversion (src/math.m:14-19) sees every input exactly.
 */
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include "nmoe/math.h"

void orc_ref_f32_to_bf16_bits(const uint32_t *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float f;
        memcpy(&f, &in[i], sizeof(f));
        out[i] = nmoe_f32_to_bf16(f);
    }
}
