/*
 * cpu_step.c -- the reference's CPU decode step, timed for the CPU baseline.
 *
 * TEST / BASELINE INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg calls it,
 * nothing in libnmoe_hip.so does.
 *
 * One token through one routed-expert layer, the way the reference's CPU
 * routines do it, single-threaded:
 *   router logits  : bf16 router x fp32 input, one sequential fp32
 *                    accumulator per row (the math.m:257-272 loop shape; the
 *                    reference has no CPU bf16 router, so this is glue)
 *   routing        : softmax -> top-k -> renormalise (math.m:67-153,
 *                    orchestrated as runtime.m:1498-1511)
 *   per expert     : gate and up dequant matvecs (math.m:236-274), SwiGLU
 *                    (math.m:155-162), down dequant matvec
 *   combine        : kernels.metal:1394-1423 transcribed
 *
 * Built twice: against this oracle (liboracle.so, "port") and, with
 * ORC_CPU_STEP_USE_REF, against the reference's own src/math.m compiled as C
 * (oracle/_ref/libnmoe_cpu_step_ref.so, "reference").
 */
#define _POSIX_C_SOURCE 199309L
#include "nmoe_oracle.h"

#include <stdlib.h>
#include <string.h>
#include <time.h>

#ifdef ORC_CPU_STEP_USE_REF
#include "nmoe/math.h"
#define STEP_SOFTMAX(v, n) nmoe_cpu_softmax((v), (n))
#define STEP_RENORM(v, n) nmoe_cpu_renormalize((v), (n))
#define STEP_SWIGLU(g, u, o, n) nmoe_cpu_swiglu((g), (u), (o), (n))
#define STEP_MATVEC nmoe_cpu_dequant_matvec
static size_t step_topk(const float *v, size_t n, size_t k, uint32_t *idx, float *val) {
    size_t tmp[ORC_MAX_K];
    size_t got = nmoe_cpu_topk(v, n, k, tmp, val);
    for (size_t i = 0; i < got; i++) idx[i] = (uint32_t)tmp[i];
    return got;
}
#define STEP_NAME(x) x##_ref
#else
#define STEP_SOFTMAX(v, n) orc_softmax((v), (n))
#define STEP_RENORM(v, n) orc_renormalize((v), (n))
#define STEP_SWIGLU(g, u, o, n) orc_swiglu((g), (u), (o), (n))
#define STEP_MATVEC orc_dequant_matvec
static size_t step_topk(const float *v, size_t n, size_t k, uint32_t *idx, float *val) {
    return orc_topk(v, n, k, idx, val);
}
#define STEP_NAME(x) x##_port
#endif

/* One decode step for one token.  Returns the number of selected experts. */
int STEP_NAME(orc_cpu_step)(const uint8_t *layer_pack, int bits, const uint16_t *router_w, const float *x, int k,
                            const float *h_mid, float *out, uint32_t *idx8, float *w8) {
    float logits[ORC_EXPERTS];
    for (int e = 0; e < ORC_EXPERTS; e++) {
        const uint16_t *row = router_w + (size_t)e * ORC_HIDDEN;
        float acc = 0.0f;
        for (int j = 0; j < ORC_HIDDEN; j++) acc += orc_bf16_to_f32(row[j]) * x[j];
        logits[e] = acc;
    }
    STEP_SOFTMAX(logits, ORC_EXPERTS);
    uint32_t idx[ORC_MAX_K] = {0};
    float val[ORC_MAX_K] = {0};
    size_t n = step_topk(logits, ORC_EXPERTS, (size_t)k, idx, val);
    STEP_RENORM(val, n);

    size_t off[9];
    orc_expert_offsets(bits, off);
    size_t esz = orc_expert_size(bits);
    static float y[ORC_MAX_K][ORC_HIDDEN];
    float gate[ORC_INTER], up[ORC_INTER], act[ORC_INTER];
    for (size_t s = 0; s < n; s++) {
        const uint8_t *ex = layer_pack + (size_t)idx[s] * esz;
        STEP_MATVEC((const uint32_t *)(ex + off[0]), (const uint16_t *)(ex + off[1]), (const uint16_t *)(ex + off[2]),
                    x, gate, ORC_INTER, ORC_HIDDEN, bits);
        STEP_MATVEC((const uint32_t *)(ex + off[3]), (const uint16_t *)(ex + off[4]), (const uint16_t *)(ex + off[5]),
                    x, up, ORC_INTER, ORC_HIDDEN, bits);
        STEP_SWIGLU(gate, up, act, ORC_INTER);
        STEP_MATVEC((const uint32_t *)(ex + off[6]), (const uint16_t *)(ex + off[7]), (const uint16_t *)(ex + off[8]),
                    act, y[s], ORC_HIDDEN, ORC_INTER, bits);
    }
    orc_combine(h_mid, &y[0][0], val, (int)n, NULL, NULL, out, ORC_HIDDEN);
    for (int i = 0; i < ORC_MAX_K; i++) {
        idx8[i] = (size_t)i < n ? idx[i] : 0u;
        w8[i] = (size_t)i < n ? val[i] : 0.0f;
    }
    return (int)n;
}

static double step_now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* Times `steps` decode steps per repeat over `nlayers` resident layer packs
 * (step i uses layer i % nlayers and input i % ninputs) and returns the
 * median seconds per step over `repeats` repeats (CLOCK_MONOTONIC, as
 * runtime.m:2139-2143). */
double STEP_NAME(orc_cpu_step_bench)(const uint8_t *const *layer_packs, const uint16_t *const *routers, int nlayers,
                                     int bits, const float *x, const float *h_mid, int ninputs, int k, int steps,
                                     int repeats, float *out_last) {
    double times[64];
    if (repeats > 64) repeats = 64;
    float out[ORC_HIDDEN];
    uint32_t idx[ORC_MAX_K];
    float w[ORC_MAX_K];
    for (int r = 0; r < repeats; r++) {
        double t0 = step_now();
        for (int i = 0; i < steps; i++) {
            int l = i % nlayers, t = i % ninputs;
            STEP_NAME(orc_cpu_step)(layer_packs[l], bits, routers[l], x + (size_t)t * ORC_HIDDEN,
                                    k, h_mid + (size_t)t * ORC_HIDDEN, out, idx, w);
        }
        times[r] = (step_now() - t0) / (double)steps;
    }
    for (int i = 1; i < repeats; i++)
        for (int j = i; j > 0 && times[j] < times[j - 1]; j--) {
            double tmp = times[j];
            times[j] = times[j - 1];
            times[j - 1] = tmp;
        }
    if (out_last != NULL) memcpy(out_last, out, sizeof(out));
    return times[repeats / 2];
}
