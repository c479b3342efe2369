/*
 * nmoe_oracle.c -- CPU oracle for the routed-expert MoE path.
 *
 * TEST INFRASTRUCTURE ONLY (see nmoe_oracle.h).  Compiled with
 * -O2 -ffp-contract=off; `long double` is the x86-64 80-bit type, as in the
 * reference's math.m on the host that runs this oracle.
 */
#include "nmoe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- math.m */

/* math.m:7-12 */
float orc_bf16_to_f32(uint16_t v) {
    uint32_t bits = ((uint32_t)v) << 16;
    float out;
    memcpy(&out, &bits, sizeof(out));
    return out;
}

/* math.m:14-19: round-to-nearest-even on the upper half (no NaN special case). */
uint16_t orc_f32_to_bf16(float v) {
    uint32_t bits;
    memcpy(&bits, &v, sizeof(bits));
    uint32_t r = bits + 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)(r >> 16);
}

/* orc_f32_to_bf16 over raw bit patterns (every NaN payload reaches it as is). */
void orc_f32_to_bf16_bits(const uint32_t *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float f;
        memcpy(&f, &in[i], sizeof(f));
        out[i] = orc_f32_to_bf16(f);
    }
}

void orc_bf16_to_f32_array(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_bf16_to_f32(in[i]);
}

/* math.m:21-28: branch on sign so exp never overflows. */
float orc_sigmoid(float x) {
    if (x >= 0.0f) {
        float z = expf(-x);
        return 1.0f / (1.0f + z);
    }
    float z = expf(x);
    return z / (1.0f + z);
}

/* math.m:30-32 */
float orc_silu(float x) { return x * orc_sigmoid(x); }

/* math.m:34-65: long double sum of squares, rms = sqrtf(mean + eps). */
void orc_rms_norm(const float *input, const uint16_t *weight_bf16, float *output, size_t count, float eps,
                  int add_one) {
    if (input == NULL || output == NULL || count == 0) return;
    long double acc = 0.0L;
    for (size_t i = 0; i < count; i++) {
        long double v = input[i];
        acc += v * v;
    }
    float rms = sqrtf((float)(acc / (long double)count) + eps);
    if (rms == 0.0f) rms = 1.0f;
    for (size_t i = 0; i < count; i++) {
        float wt = 1.0f;
        if (weight_bf16 != NULL) {
            wt = orc_bf16_to_f32(weight_bf16[i]);
            if (add_one) wt += 1.0f;
        }
        output[i] = (input[i] / rms) * wt;
    }
}

/* math.m:67-93: max, expf(v - max), long double sum, scale by 1/(float)sum;
 * a zero sum gives the uniform distribution. */
void orc_softmax(float *values, size_t count) {
    if (values == NULL || count == 0) return;
    float maxv = values[0];
    for (size_t i = 1; i < count; i++)
        if (values[i] > maxv) maxv = values[i];
    long double total = 0.0L;
    for (size_t i = 0; i < count; i++) {
        values[i] = expf(values[i] - maxv);
        total += values[i];
    }
    if (total == 0.0L) {
        float u = 1.0f / (float)count;
        for (size_t i = 0; i < count; i++) values[i] = u;
        return;
    }
    float inv = 1.0f / (float)total;
    for (size_t i = 0; i < count; i++) values[i] *= inv;
}

/* math.m:95-132: k passes of an arg-max over the untaken entries; a strictly
 * greater value wins, an equal value wins only with a lower index. */
size_t orc_topk(const float *values, size_t count, size_t k, uint32_t *indices, float *selected_values) {
    if (values == NULL || count == 0 || indices == NULL || k == 0) return 0;
    if (k > count) k = count;
    uint8_t *taken = calloc(count, 1);
    if (taken == NULL) return 0;
    size_t n = 0;
    while (n < k) {
        size_t bi = 0;
        float bv = -INFINITY;
        for (size_t i = 0; i < count; i++) {
            if (taken[i]) continue;
            float v = values[i];
            if (v > bv || (v == bv && i < bi)) {
                bv = v;
                bi = i;
            }
        }
        taken[bi] = 1;
        indices[n] = (uint32_t)bi;
        if (selected_values != NULL) selected_values[n] = bv;
        n++;
    }
    free(taken);
    return n;
}

/* math.m:134-153: fp32 sequential sum, multiply by 1/sum; zero sum -> 1/k. */
void orc_renormalize(float *values, size_t count) {
    if (values == NULL || count == 0) return;
    float s = 0.0f;
    for (size_t i = 0; i < count; i++) s += values[i];
    if (s == 0.0f) {
        float u = 1.0f / (float)count;
        for (size_t i = 0; i < count; i++) values[i] = u;
        return;
    }
    float inv = 1.0f / s;
    for (size_t i = 0; i < count; i++) values[i] *= inv;
}

/* math.m:155-162 */
void orc_swiglu(const float *gate, const float *up, float *output, size_t count) {
    for (size_t i = 0; i < count; i++) output[i] = orc_silu(gate[i]) * up[i];
}

/* math.m:191-204: field v of word w is column w*vpw + v. */
void orc_unpack_row(const uint32_t *packed_row, uint16_t *output, size_t in_dim, int quant_bits) {
    size_t vpw = (size_t)(32 / quant_bits);
    uint32_t mask = quant_bits == 2 ? 0x3u : 0xFu;
    for (size_t w = 0; w < in_dim / vpw; w++)
        for (size_t v = 0; v < vpw; v++)
            output[w * vpw + v] = (uint16_t)((packed_row[w] >> (v * (size_t)quant_bits)) & mask);
}

/* math.m:206-234: w = q*scale + bias per group of 64 columns. */
void orc_dequant_row(const uint32_t *packed_row, const uint16_t *scales_row, const uint16_t *biases_row,
                     float *output, size_t in_dim, int quant_bits) {
    size_t vpw = (size_t)(32 / quant_bits);
    size_t groups = in_dim / ORC_GROUP;
    size_t wpg = ORC_GROUP / vpw;
    uint32_t mask = quant_bits == 2 ? 0x3u : 0xFu;
    for (size_t g = 0; g < groups; g++) {
        float s = orc_bf16_to_f32(scales_row[g]);
        float b = orc_bf16_to_f32(biases_row[g]);
        for (size_t w = 0; w < wpg; w++) {
            uint32_t word = packed_row[g * wpg + w];
            for (size_t v = 0; v < vpw; v++) {
                uint32_t q = (word >> (v * (size_t)quant_bits)) & mask;
                output[g * ORC_GROUP + w * vpw + v] = (float)q * s + b;
            }
        }
    }
}

/* math.m:236-274: one fp32 accumulator per row, columns in order. */
void orc_dequant_matvec(const uint32_t *packed, const uint16_t *scales, const uint16_t *biases,
                        const float *input, float *output, size_t out_dim, size_t in_dim, int quant_bits) {
    size_t vpw = (size_t)(32 / quant_bits);
    size_t pcols = in_dim / vpw;
    size_t groups = in_dim / ORC_GROUP;
    size_t wpg = ORC_GROUP / vpw;
    uint32_t mask = quant_bits == 2 ? 0x3u : 0xFu;
    for (size_t r = 0; r < out_dim; r++) {
        const uint32_t *pr = packed + r * pcols;
        const uint16_t *sr = scales + r * groups;
        const uint16_t *br = biases + r * groups;
        float acc = 0.0f;
        for (size_t g = 0; g < groups; g++) {
            float s = orc_bf16_to_f32(sr[g]);
            float b = orc_bf16_to_f32(br[g]);
            for (size_t w = 0; w < wpg; w++) {
                uint32_t word = pr[g * wpg + w];
                for (size_t v = 0; v < vpw; v++) {
                    uint32_t q = (word >> (v * (size_t)quant_bits)) & mask;
                    acc += ((float)q * s + b) * input[g * ORC_GROUP + w * vpw + v];
                }
            }
        }
        output[r] = acc;
    }
}

/* ------------------------------------------------------- the writer side */

/* scripts/convert_qwen36.py:167-211 (quantize_rows_bf16 / _2bit with
 * pack_4bit / pack_2bit): per group of 64 columns of a bf16 row, min and max
 * in fp32, scale = (max - min) / 15 (q4) or / 3 (q2) in fp32, a zero scale
 * replaced by 1 for the division only, q = rint((x - min) / scale) (ties to
 * even, the default rounding mode) clipped to the code range, column 8w + v
 * (16w + v for q2) in field v of word w; scale and min stored as bf16 by the
 * math.m:14-19 rule (the converter's f32_to_bf16, :151-155).  Inputs are
 * finite. */
void orc_quantize_rows(const uint16_t *rows_bf16, int rows, int in_dim, int bits, uint32_t *packed,
                       uint16_t *scales, uint16_t *biases) {
    const int vpw = 32 / bits, groups = in_dim / ORC_GROUP;
    const float qmax = bits == 4 ? 15.0f : 3.0f;
    for (int r = 0; r < rows; r++) {
        const uint16_t *row = rows_bf16 + (size_t)r * in_dim;
        uint32_t *pr = packed + (size_t)r * (in_dim / vpw);
        memset(pr, 0, sizeof(uint32_t) * (size_t)(in_dim / vpw));
        for (int g = 0; g < groups; g++) {
            float mn = orc_bf16_to_f32(row[g * ORC_GROUP]), mx = mn;
            for (int i = 1; i < ORC_GROUP; i++) {
                const float v = orc_bf16_to_f32(row[g * ORC_GROUP + i]);
                if (v < mn) mn = v;
                if (v > mx) mx = v;
            }
            const float scale = (mx - mn) / qmax;
            const float safe = scale == 0.0f ? 1.0f : scale;
            for (int i = 0; i < ORC_GROUP; i++) {
                const int c = g * ORC_GROUP + i;
                float q = rintf((orc_bf16_to_f32(row[c]) - mn) / safe);
                q = q < 0.0f ? 0.0f : q > qmax ? qmax : q;
                pr[c / vpw] |= (uint32_t)q << (bits * (c % vpw));
            }
            scales[(size_t)r * groups + g] = orc_f32_to_bf16(scale);
            biases[(size_t)r * groups + g] = orc_f32_to_bf16(mn);
        }
    }
}

/* ------------------------------------------------------------- routing */

/* runtime.m:1498-1511 with the slot padding of kernels.metal:1767-1775. */
int orc_route(const float *logits, int num_experts, int k, uint32_t *idx8, float *w8, float *probs) {
    if (k < 1 || k > ORC_MAX_K || num_experts < 1) return -1;
    float *p = malloc(sizeof(float) * (size_t)num_experts);
    if (p == NULL) return -1;
    memcpy(p, logits, sizeof(float) * (size_t)num_experts);
    orc_softmax(p, (size_t)num_experts);
    uint32_t idx[ORC_MAX_K] = {0};
    float val[ORC_MAX_K] = {0};
    size_t n = orc_topk(p, (size_t)num_experts, (size_t)k, idx, val);
    orc_renormalize(val, n);
    for (int i = 0; i < ORC_MAX_K; i++) {
        idx8[i] = (size_t)i < n ? idx[i] : 0u;
        w8[i] = (size_t)i < n ? val[i] : 0.0f;
    }
    if (probs != NULL) memcpy(probs, p, sizeof(float) * (size_t)num_experts);
    free(p);
    return (int)n;
}

/* ------------------------------------------------- glibc expf restatement */

static uint64_t orc_asu64(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static double orc_asdbl(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
static uint32_t orc_asu32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* 2^(i/32) rounded to double, minus i<<47 so that adding k<<47 rebuilds
 * 2^(k/32); computed from exp2l at first use. */
static uint64_t orc_exp2_tab[32];
static int orc_exp2_tab_ready;

static void orc_exp2_tab_init(void) {
    for (int i = 0; i < 32; i++) {
        double d = (double)exp2l((long double)i / 32.0L);
        orc_exp2_tab[i] = orc_asu64(d) - ((uint64_t)i << 47);
    }
    orc_exp2_tab_ready = 1;
}

float orc_expf_restated(float x) {
    if (!orc_exp2_tab_ready) orc_exp2_tab_init();
    const double invln2n = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    uint32_t abstop = (orc_asu32(x) >> 20) & 0x7ff;
    if (abstop >= ((orc_asu32(88.0f) >> 20) & 0x7ff)) {
        if (orc_asu32(x) == orc_asu32(-INFINITY)) return 0.0f;
        if (abstop >= ((orc_asu32(INFINITY) >> 20) & 0x7ff)) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    double xd = (double)x;
    double kd = fma(invln2n, xd, shift);
    uint64_t ki = orc_asu64(kd);
    kd -= shift;
    double r = fma(invln2n, xd, -kd);
    uint64_t t = orc_exp2_tab[ki % 32] + (ki << 47);
    double s = orc_asdbl(t);
    double z = fma(c0, r, c1);
    double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return (float)y;
}

/* ------------------------------------------------------- router logits */

/* Balanced pairwise tree over the 64 lane partials in lane order:
 * (p0+p1)+(p2+p3), ..., the combination the GPU's DPP reduction performs. */
static float orc_tree64(float p[64]) {
    for (int n = 64; n > 1; n >>= 1)
        for (int i = 0; i < n / 2; i++) p[i] = p[2 * i] + p[2 * i + 1];
    return p[0];
}

void orc_router_logits_bf16(const uint16_t *w, const float *x, int num_experts, int hidden, float *out) {
    int chunks = hidden / 8;
    for (int e = 0; e < num_experts; e++) {
        const uint16_t *row = w + (size_t)e * (size_t)hidden;
        float p[64];
        for (int l = 0; l < 64; l++) {
            float acc = 0.0f;
            for (int c = l; c < chunks; c += 64)
                for (int j = 0; j < 8; j++) acc = fmaf(orc_bf16_to_f32(row[c * 8 + j]), x[c * 8 + j], acc);
            p[l] = acc;
        }
        out[e] = orc_tree64(p);
    }
}

/* The reference model's q4 router, metal/kernels.metal:472-513: per column
 * acc += fma(q, scale * x, bias * x) (kernels.metal:500-508: both products
 * rounded, then the fma, then the add), the words of a row lane-strided; the
 * reference's simd_sum order is the closed Metal compiler's, so the lanes
 * here are the GPU kernel's 64 and their partials meet in its tree. */
void orc_router_logits_q4(const uint32_t *w, const uint16_t *scales, const uint16_t *biases, const float *x,
                          int num_experts, int hidden, float *out) {
    int words = hidden / 8;
    int groups = hidden / ORC_GROUP;
    for (int e = 0; e < num_experts; e++) {
        const uint32_t *row = w + (size_t)e * (size_t)words;
        float p[64];
        for (int l = 0; l < 64; l++) {
            float acc = 0.0f;
            for (int c = l; c < words; c += 64) {
                int g = c / 8;
                float s = orc_bf16_to_f32(scales[(size_t)e * groups + g]);
                float b = orc_bf16_to_f32(biases[(size_t)e * groups + g]);
                for (int j = 0; j < 8; j++) {
                    float q = (float)((row[c] >> (4 * j)) & 0xFu);
                    float sx = s * x[c * 8 + j], bx = b * x[c * 8 + j];
                    acc = acc + fmaf(q, sx, bx);
                }
            }
            p[l] = acc;
        }
        out[e] = orc_tree64(p);
    }
}

/* ------------------------------------------------------ expert packs */

/* expert_io.m:90-99 */
size_t orc_expert_size(int bits) { return bits == 4 ? 1769472u : bits == 2 ? 983040u : 0u; }

/* runtime.m:2240-2252 (== convert_qwen36.py:38-64) */
void orc_expert_offsets(int bits, size_t off9[9]) {
    static const size_t q4[9] = {0, 524288, 557056, 589824, 1114112, 1146880, 1179648, 1703936, 1736704};
    static const size_t q2[9] = {0, 262144, 294912, 327680, 589824, 622592, 655360, 917504, 950272};
    memcpy(off9, bits == 2 ? q2 : q4, sizeof(q4));
}

void orc_expert_gate_up(const uint8_t *expert, int bits, const float *x, float *act512) {
    size_t off[9];
    orc_expert_offsets(bits, off);
    float gate[ORC_INTER], up[ORC_INTER];
    orc_dequant_matvec((const uint32_t *)(expert + off[0]), (const uint16_t *)(expert + off[1]),
                       (const uint16_t *)(expert + off[2]), x, gate, ORC_INTER, ORC_HIDDEN, bits);
    orc_dequant_matvec((const uint32_t *)(expert + off[3]), (const uint16_t *)(expert + off[4]),
                       (const uint16_t *)(expert + off[5]), x, up, ORC_INTER, ORC_HIDDEN, bits);
    orc_swiglu(gate, up, act512, ORC_INTER);
}

void orc_expert_down(const uint8_t *expert, int bits, const float *act512, float *y2048) {
    size_t off[9];
    orc_expert_offsets(bits, off);
    orc_dequant_matvec((const uint32_t *)(expert + off[6]), (const uint16_t *)(expert + off[7]),
                       (const uint16_t *)(expert + off[8]), act512, y2048, ORC_HIDDEN, ORC_INTER, bits);
}

/* The shared expert of one token: metal/kernels.metal:421-469 (rows 0-511:
 * SiLU(gate.x) * (up.x)) and 510-513 (row 768: the gate score), whose rows
 * use the router's per-element form (orc_router_logits_q4), and 1520-1537
 * (the shared down) as a math.m:236-274 dequant matvec (q4). */
void orc_shared_expert(const uint32_t *gw, const uint16_t *gs, const uint16_t *gb, const uint32_t *uw,
                       const uint16_t *us, const uint16_t *ub, const uint32_t *dw, const uint16_t *ds,
                       const uint16_t *db, const uint32_t *sw, const uint16_t *ss, const uint16_t *sb, const float *x,
                       float *shared_out, float *shared_gate_raw) {
    float gate[ORC_INTER], up[ORC_INTER], act[ORC_INTER];
    orc_router_logits_q4(gw, gs, gb, x, ORC_INTER, ORC_HIDDEN, gate);
    orc_router_logits_q4(uw, us, ub, x, ORC_INTER, ORC_HIDDEN, up);
    orc_swiglu(gate, up, act, ORC_INTER);
    orc_dequant_matvec(dw, ds, db, act, shared_out, ORC_HIDDEN, ORC_INTER, 4);
    orc_router_logits_q4(sw, ss, sb, x, 1, ORC_HIDDEN, shared_gate_raw);
}

/* kernels.metal:1394-1423 (and the fused tail at 1539-1541). */
void orc_combine(const float *h_mid, const float *y, const float *w, int k, const float *shared_out,
                 const float *shared_gate_raw, float *out, int hidden) {
    float sg = shared_out != NULL && shared_gate_raw != NULL ? orc_sigmoid(shared_gate_raw[0]) : 0.0f;
    for (int r = 0; r < hidden; r++) {
        float moe = 0.0f;
        for (int s = 0; s < k; s++) moe += w[s] * y[(size_t)s * hidden + r];
        float sh = shared_out != NULL && shared_gate_raw != NULL ? sg * shared_out[r] : 0.0f;
        out[r] = h_mid[r] + moe + sh;
    }
}

int orc_moe_experts(const uint8_t *layer_pack, int bits, const float *x, int ntok, int k, const uint32_t *idx,
                    const float *w, const float *h_mid, const float *shared_out, const float *shared_gate_raw,
                    float *out, float *act) {
    if (k < 1 || k > ORC_MAX_K) return -1;
    size_t esz = orc_expert_size(bits);
    float *y = malloc(sizeof(float) * ORC_MAX_K * ORC_HIDDEN);
    float a[ORC_INTER];
    if (y == NULL) return -1;
    for (int t = 0; t < ntok; t++) {
        float wk[ORC_MAX_K];
        for (int s = 0; s < k; s++) {
            uint32_t e = idx[(size_t)t * ORC_MAX_K + s];
            const uint8_t *ex = layer_pack + (size_t)e * esz;
            orc_expert_gate_up(ex, bits, x + (size_t)t * ORC_HIDDEN, a);
            if (act != NULL) memcpy(act + ((size_t)t * ORC_MAX_K + s) * ORC_INTER, a, sizeof(a));
            orc_expert_down(ex, bits, a, y + (size_t)s * ORC_HIDDEN);
            wk[s] = w[(size_t)t * ORC_MAX_K + s];
        }
        orc_combine(h_mid + (size_t)t * ORC_HIDDEN, y, wk, k, shared_out ? shared_out + (size_t)t * ORC_HIDDEN : NULL,
                    shared_gate_raw ? shared_gate_raw + t : NULL, out + (size_t)t * ORC_HIDDEN, ORC_HIDDEN);
    }
    free(y);
    return 0;
}

int orc_moe_step_bf16router(const uint8_t *layer_pack, int bits, const uint16_t *router_w, const float *x,
                            int ntok, int k, const float *h_mid, const float *shared_out,
                            const float *shared_gate_raw, float *out, uint32_t *idx, float *w, float *logits,
                            float *act) {
    if (k < 1 || k > ORC_MAX_K) return -1;
    float lg[ORC_EXPERTS];
    for (int t = 0; t < ntok; t++) {
        orc_router_logits_bf16(router_w, x + (size_t)t * ORC_HIDDEN, ORC_EXPERTS, ORC_HIDDEN, lg);
        if (logits != NULL) memcpy(logits + (size_t)t * ORC_EXPERTS, lg, sizeof(lg));
        if (orc_route(lg, ORC_EXPERTS, k, idx + (size_t)t * ORC_MAX_K, w + (size_t)t * ORC_MAX_K, NULL) < 0)
            return -1;
    }
    return orc_moe_experts(layer_pack, bits, x, ntok, k, idx, w, h_mid, shared_out, shared_gate_raw, out, act);
}

int orc_moe_layer_rmsnorm(const uint8_t *layer_pack, int bits, const uint16_t *router_w, const float *h_in, float eps,
                          int k, float *h_out, uint32_t *idx8, float *w8, float *x_out) {
    float x[ORC_HIDDEN], lg[ORC_EXPERTS];
    uint32_t idx[ORC_MAX_K];
    float w[ORC_MAX_K];
    orc_rms_norm(h_in, NULL, x, ORC_HIDDEN, eps, 0);
    if (x_out != NULL) memcpy(x_out, x, sizeof(x));
    orc_router_logits_bf16(router_w, x, ORC_EXPERTS, ORC_HIDDEN, lg);
    if (orc_route(lg, ORC_EXPERTS, k, idx, w, NULL) < 0) return -1;
    if (idx8 != NULL) memcpy(idx8, idx, sizeof(idx));
    if (w8 != NULL) memcpy(w8, w, sizeof(w));
    return orc_moe_experts(layer_pack, bits, x, 1, k, idx, w, h_in, NULL, NULL, h_out, NULL);
}

/* One token through one layer's MoE block, in the reference's order
 * (src/runtime.m:3144-3201 then NMOEPipelinedExpertTail :2908-2999):
 *   x      = RMSNorm(h_mid, post_norm, add_one)      (runtime.m:3148-3150, math.m:34-65)
 *   logits = router . x  (bf16 router, or the model's q4 router kernels.metal:472-513)
 *   route  = softmax -> top-k -> renormalise         (runtime.m:1498-1511)
 *   shared = Wsd . (SiLU(Wsg x) * (Wsu x)), g = Wss . x  (kernels.metal:421-469, 510-513, 1520-1537)
 *   out    = h_mid + sum_s w_s y_s + sigmoid(g) shared   (kernels.metal:1539-1541)
 *   next_x = RMSNorm(out, next_norm, add_one)        (runtime.m:2893-2900)
 * post_norm NULL: unit weight; shared (nullable): 12 pointers gate w/s/b,
 * up w/s/b, down w/s/b, score w/s/b; next_norm / next_x nullable (no next
 * norm when next_x is NULL).  idx8/w8/x_out nullable. */
int orc_moe_block(const uint8_t *layer_pack, int bits, int router_kind, const uint16_t *router_bf16,
                  const uint32_t *rq_w, const uint16_t *rq_s, const uint16_t *rq_b, const void *const *shared,
                  const uint16_t *post_norm, int add_one, const float *h_mid, float eps, int k, float *out,
                  const uint16_t *next_norm, float *next_x, uint32_t *idx8, float *w8, float *x_out) {
    float x[ORC_HIDDEN], lg[ORC_EXPERTS], so[ORC_HIDDEN], g = 0.0f;
    uint32_t idx[ORC_MAX_K];
    float w[ORC_MAX_K];
    orc_rms_norm(h_mid, post_norm, x, ORC_HIDDEN, eps, post_norm != NULL ? add_one : 0);
    if (x_out != NULL) memcpy(x_out, x, sizeof(x));
    if (router_kind == 0)
        orc_router_logits_bf16(router_bf16, x, ORC_EXPERTS, ORC_HIDDEN, lg);
    else
        orc_router_logits_q4(rq_w, rq_s, rq_b, x, ORC_EXPERTS, ORC_HIDDEN, lg);
    if (orc_route(lg, ORC_EXPERTS, k, idx, w, NULL) < 0) return -1;
    if (idx8 != NULL) memcpy(idx8, idx, sizeof(idx));
    if (w8 != NULL) memcpy(w8, w, sizeof(w));
    if (shared != NULL)
        orc_shared_expert(shared[0], shared[1], shared[2], shared[3], shared[4], shared[5], shared[6], shared[7],
                          shared[8], shared[9], shared[10], shared[11], x, so, &g);
    int rc = orc_moe_experts(layer_pack, bits, x, 1, k, idx, w, h_mid, shared != NULL ? so : NULL,
                             shared != NULL ? &g : NULL, out, NULL);
    if (rc == 0 && next_x != NULL) orc_rms_norm(out, next_norm, next_x, ORC_HIDDEN, eps, next_norm != NULL ? add_one : 0);
    return rc;
}

/* ------------------------------------------------------------ dispatch */

void orc_dispatch(const uint32_t *idx, int ntok, int k, int stride, int num_experts, uint32_t *perm,
                  uint32_t *offsets) {
    memset(offsets, 0, sizeof(uint32_t) * (size_t)(num_experts + 1));
    for (int t = 0; t < ntok; t++)
        for (int s = 0; s < k; s++) offsets[idx[(size_t)t * stride + s] + 1]++;
    for (int e = 0; e < num_experts; e++) offsets[e + 1] += offsets[e];
    uint32_t *cursor = malloc(sizeof(uint32_t) * (size_t)num_experts);
    memcpy(cursor, offsets, sizeof(uint32_t) * (size_t)num_experts);
    for (int t = 0; t < ntok; t++)
        for (int s = 0; s < k; s++) perm[cursor[idx[(size_t)t * stride + s]]++] = (uint32_t)(t * k + s);
    free(cursor);
}

/* ----------------------------------------------------------- generator */

#define ORC_GOLDEN 0x9E3779B97F4A7C15ull

uint64_t orc_syn_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t orc_syn_stream(uint64_t seed, uint32_t layer, uint32_t expert, uint32_t tag) {
    uint64_t s = orc_syn_mix64(seed + ORC_GOLDEN);
    return orc_syn_mix64(s ^ (((uint64_t)layer << 40) | ((uint64_t)expert << 16) | (uint64_t)tag));
}

uint64_t orc_syn_rand64(uint64_t stream, uint64_t i) { return orc_syn_mix64(stream + (i + 1) * ORC_GOLDEN); }

/* Irwin-Hall(12) normal: twelve 16-bit uniforms (u + 1/2)/65536, sum - 6. */
float orc_syn_normal(uint64_t stream, uint64_t i) {
    uint32_t sum = 0;
    for (uint64_t j = 0; j < 3; j++) {
        uint64_t r = orc_syn_rand64(stream, 3 * i + j);
        sum += (uint32_t)(r & 0xFFFF) + (uint32_t)((r >> 16) & 0xFFFF) + (uint32_t)((r >> 32) & 0xFFFF) +
               (uint32_t)(r >> 48);
    }
    return (float)(sum + 6u) * (1.0f / 65536.0f) - 6.0f;
}

void orc_syn_expert(uint8_t *dst, int bits, uint64_t seed, uint32_t layer, uint32_t expert, float sigma) {
    size_t off[9];
    orc_expert_offsets(bits, off);
    for (int m = 0; m < 3; m++) {
        uint32_t *wds = (uint32_t *)(dst + off[3 * m]);
        uint16_t *sc = (uint16_t *)(dst + off[3 * m + 1]);
        uint16_t *bi = (uint16_t *)(dst + off[3 * m + 2]);
        size_t nwords = (off[3 * m + 1] - off[3 * m]) / 4;
        size_t ngroups = (off[3 * m + 2] - off[3 * m + 1]) / 2;
        uint64_t sw = orc_syn_stream(seed, layer, expert, (uint32_t)(2 * m));
        uint64_t ss = orc_syn_stream(seed, layer, expert, (uint32_t)(2 * m + 1));
        for (size_t j = 0; j < nwords; j++) {
            uint64_t r = orc_syn_rand64(sw, j >> 1);
            wds[j] = (j & 1) ? (uint32_t)(r >> 32) : (uint32_t)r;
        }
        for (size_t g = 0; g < ngroups; g++) {
            uint16_t s16 = orc_f32_to_bf16(orc_syn_normal(ss, g) * sigma);
            float s = orc_bf16_to_f32(s16);
            sc[g] = s16;
            bi[g] = orc_f32_to_bf16(bits == 4 ? -8.0f * s : -1.5f * s);
        }
    }
}

void orc_syn_layer(uint8_t *dst, int bits, uint64_t seed, uint32_t layer, float sigma) {
    size_t esz = orc_expert_size(bits);
    for (uint32_t e = 0; e < ORC_EXPERTS; e++) orc_syn_expert(dst + (size_t)e * esz, bits, seed, layer, e, sigma);
}

void orc_syn_bf16_normal(uint16_t *dst, size_t n, uint64_t seed, uint32_t layer, uint32_t tag, float sigma) {
    uint64_t s = orc_syn_stream(seed, layer, 0xFFFFu, tag);
    for (size_t i = 0; i < n; i++) dst[i] = orc_f32_to_bf16(orc_syn_normal(s, i) * sigma);
}
