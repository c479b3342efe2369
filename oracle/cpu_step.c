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
#define STEP_RMSNORM(in, o, n, eps) nmoe_cpu_rms_norm((in), NULL, (o), (n), (eps), 0)
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
#define STEP_RMSNORM(in, o, n, eps) orc_rms_norm((in), NULL, (o), (n), (eps), 0)
static size_t step_topk(const float *v, size_t n, size_t k, uint32_t *idx, float *val) {
    return orc_topk(v, n, k, idx, val);
}
#define STEP_NAME(x) x##_port
#endif

/* The expert half of one token: routing from its logits (softmax, top-k,
 * renormalise; `logits` is overwritten with the probabilities), the
 * selected experts, the combine.  Returns the number of selected experts. */
static int STEP_NAME(step_experts)(const uint8_t *layer_pack, int bits, float *logits, const float *x, int k,
                                   const float *h_mid, float *out, uint32_t *idx8, float *w8) {
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
    return STEP_NAME(step_experts)(layer_pack, bits, logits, x, k, h_mid, out, idx8, w8);
}

static double STEP_NAME(median)(double *times, int n) {
    for (int i = 1; i < n; i++)
        for (int j = i; j > 0 && times[j] < times[j - 1]; j--) {
            double tmp = times[j];
            times[j] = times[j - 1];
            times[j - 1] = tmp;
        }
    return times[n / 2];
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
    if (out_last != NULL) memcpy(out_last, out, sizeof(out));
    return STEP_NAME(median)(times, repeats);
}

/* Tokens with given router logits (the batched-decode and prefill configs,
 * whose logits are inputs), one token at a time as the reference's prompt
 * loop runs them (runtime.m:3814-3818): logits [ntok][256], x and h_mid
 * [ntok][2048] fp32, one layer pack.  Returns the median seconds per token
 * over `repeats` passes over all ntok tokens. */
double STEP_NAME(orc_cpu_tokens_bench)(const uint8_t *layer_pack, int bits, const float *logits, const float *x,
                                       const float *h_mid, int ntok, int k, int repeats, float *out_last) {
    double times[64];
    if (repeats > 64) repeats = 64;
    float lg[ORC_EXPERTS], out[ORC_HIDDEN];
    uint32_t idx[ORC_MAX_K];
    float w[ORC_MAX_K];
    for (int r = 0; r < repeats; r++) {
        double t0 = step_now();
        for (int t = 0; t < ntok; t++) {
            memcpy(lg, logits + (size_t)t * ORC_EXPERTS, sizeof(lg));
            STEP_NAME(step_experts)(layer_pack, bits, lg, x + (size_t)t * ORC_HIDDEN, k,
                                    h_mid + (size_t)t * ORC_HIDDEN, out, idx, w);
        }
        times[r] = (step_now() - t0) / (double)ntok;
    }
    if (out_last != NULL) memcpy(out_last, out, sizeof(out));
    return STEP_NAME(median)(times, repeats);
}

/* The routed-expert stack of one decode token (the layer loop of
 * runtime.m:3732-3777 restricted to the MoE tails): for l < nl,
 * x = RMSNorm(h) (math.m:34-65, unit weight), h = h + MoE_l(x), with layer
 * l taking pack and router l % npacks.  h0 [ntok][2048].  Returns the
 * median seconds per token over `repeats` passes over all ntok tokens;
 * h_last receives the last token's final h. */
double STEP_NAME(orc_cpu_stack_bench)(const uint8_t *const *layer_packs, const uint16_t *const *routers, int npacks,
                                      int nl, int bits, const float *h0, int ntok, int k, float eps, int repeats,
                                      float *h_last) {
    double times[64];
    if (repeats > 64) repeats = 64;
    float h[ORC_HIDDEN], x[ORC_HIDDEN], out[ORC_HIDDEN];
    uint32_t idx[ORC_MAX_K];
    float w[ORC_MAX_K];
    for (int r = 0; r < repeats; r++) {
        double t0 = step_now();
        for (int t = 0; t < ntok; t++) {
            memcpy(h, h0 + (size_t)t * ORC_HIDDEN, sizeof(h));
            for (int l = 0; l < nl; l++) {
                STEP_RMSNORM(h, x, ORC_HIDDEN, eps);
                STEP_NAME(orc_cpu_step)(layer_packs[l % npacks], bits, routers[l % npacks], x, k, h, out, idx, w);
                memcpy(h, out, sizeof(h));
            }
        }
        times[r] = (step_now() - t0) / (double)ntok;
    }
    if (h_last != NULL) memcpy(h_last, h, sizeof(h));
    return STEP_NAME(median)(times, repeats);
}
