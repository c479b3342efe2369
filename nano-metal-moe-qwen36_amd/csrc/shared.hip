/*
 * shared.hip -- the shared expert of a Qwen3.6 MoE layer on gfx950.
 *
 * The reference evaluates it in two kernels:
 *   - nmoe_route_shared_q4 (metal/kernels.metal:384-514): rows 0-511 give
 *     the shared activation SiLU(gate.x) * (up.x), rows 512-767 the router
 *     logits, row 768 the shared-expert gate score;
 *   - the shared down inside nmoe_expert_down_combine_q4 (:1520-1537).
 * Here the shared expert has its own two launches; the router logits stay
 * with the router kernels.  Weights are the model's q4 tensors as stored
 * (w = q*scale + bias, math.m:206-234), each row reduced by one wavefront.
 */
#include "nmoe_device.h"

/* Wavefront w of block b reduces row 4b + w of gate and of up (rows
 * 0..511); block 128 wavefront 0 reduces the score row.  Lane L owns the
 * words L, L+64, L+128, L+192 of a 256-word row (columns 8 word .. +7) and
 * accumulates acc + fma(q, s*x, b*x) per column, the reference's form for
 * these rows (kernels.metal:444-460, 500-508); lanes combined by the pairwise
 * tree.  The row's codes and scales stay in registers over the block's
 * tokens. */
template <typename XT>
__global__ void __launch_bounds__(256) nmoe_shared_gateup_kernel(
    const uint32_t *__restrict__ gw, const uint16_t *__restrict__ gs, const uint16_t *__restrict__ gb,
    const uint32_t *__restrict__ uw, const uint16_t *__restrict__ us, const uint16_t *__restrict__ ub,
    const uint32_t *__restrict__ sw, const uint16_t *__restrict__ ss, const uint16_t *__restrict__ sb,
    const XT *__restrict__ x, int ntok, int tok_per_block, float *__restrict__ act, float *__restrict__ graw) {
    constexpr int WPR = NMOE_HIDDEN / 8, GPR = NMOE_HIDDEN / NMOE_GROUP;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = 4 * blockIdx.x + wave;
    const bool score = row >= NMOE_INTER;
    if (score && row != NMOE_INTER) return;
    const uint32_t *w0 = score ? sw : gw + (size_t)row * WPR;
    const uint16_t *s0 = score ? ss : gs + (size_t)row * GPR, *b0 = score ? sb : gb + (size_t)row * GPR;
    uint32_t wa[4], wb[4];
    float sa[4], ba[4], sbv[4], bbv[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int c = lane + 64 * j;
        wa[j] = w0[c];
        sa[j] = nmoe_bf16f(s0[c / 8]);
        ba[j] = nmoe_bf16f(b0[c / 8]);
        if (!score) {
            wb[j] = uw[(size_t)row * WPR + c];
            sbv[j] = nmoe_bf16f(us[(size_t)row * GPR + c / 8]);
            bbv[j] = nmoe_bf16f(ub[(size_t)row * GPR + c / 8]);
        }
    }
    const int t0 = blockIdx.y * tok_per_block, t1 = min(ntok, t0 + tok_per_block);
    for (int t = t0; t < t1; t++) {
        const XT *xt = x + (size_t)t * NMOE_HIDDEN;
        float ga = 0.0f, ua = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float xv[8];
            nmoe_load_cols<XT>(xt, (lane + 64 * j) * 8, 8, xv);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                ga = nmoe_router_q4_term(ga, (wa[j] >> (4 * i)) & 0xFu, sa[j], ba[j], xv[i]);
                if (!score) ua = nmoe_router_q4_term(ua, (wb[j] >> (4 * i)) & 0xFu, sbv[j], bbv[j], xv[i]);
            }
        }
        ga = nmoe_wave_sum_tree(ga);
        if (score) {
            if (lane == 0) graw[t] = ga;
        } else {
            ua = nmoe_wave_sum_tree(ua);
            if (lane == 0) act[(size_t)t * NMOE_INTER + row] = nmoe_silu_dev(ga) * ua;
        }
    }
}

/* Wavefront w of block b reduces row 4b + w (of 2048) of the shared down
 * against act: lane L owns word L of the 64-word row (columns 8L..8L+7) and
 * accumulates fma(q, s, b) * x per column, the reference's form for this
 * matrix (kernels.metal:1533), as one fma. */
__global__ void __launch_bounds__(256) nmoe_shared_down_kernel(const uint32_t *__restrict__ dw,
                                                               const uint16_t *__restrict__ ds,
                                                               const uint16_t *__restrict__ db,
                                                               const float *__restrict__ act, int ntok,
                                                               int tok_per_block, float *__restrict__ out) {
    constexpr int WPR = NMOE_INTER / 8, GPR = NMOE_INTER / NMOE_GROUP;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = 4 * blockIdx.x + wave;
    const uint32_t wv = dw[(size_t)row * WPR + lane];
    const float s = nmoe_bf16f(ds[(size_t)row * GPR + lane / 8]), b = nmoe_bf16f(db[(size_t)row * GPR + lane / 8]);
    const int t0 = blockIdx.y * tok_per_block, t1 = min(ntok, t0 + tok_per_block);
    for (int t = t0; t < t1; t++) {
        float xv[8];
        nmoe_load_cols<float>(act + (size_t)t * NMOE_INTER, 8 * lane, 8, xv);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) acc = __builtin_fmaf(__builtin_fmaf((float)((wv >> (4 * i)) & 0xFu), s, b), xv[i], acc);
        acc = nmoe_wave_sum_tree(acc);
        if (lane == 0) out[(size_t)t * NMOE_HIDDEN + row] = acc;
    }
}

int nmoe_check_x(nmoe_hip_ctx *ctx, const void *x, int x_dtype, int ntok);

static bool nmoe_qtensor_ok(const nmoe_hip_qtensor &q) {
    return q.w != NULL && q.scales != NULL && q.biases != NULL && nmoe_aligned(q.w, 4) && nmoe_aligned(q.scales, 2) &&
           nmoe_aligned(q.biases, 2);
}

extern "C" int nmoe_moe_shared_expert(nmoe_hip_ctx *ctx, const nmoe_hip_shared_expert *se, const void *x,
                                      int x_dtype, int ntok, float *shared_out, float *shared_gate_raw,
                                      void *stream) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (se == NULL || !nmoe_qtensor_ok(se->gate) || !nmoe_qtensor_ok(se->up) || !nmoe_qtensor_ok(se->down) ||
        !nmoe_qtensor_ok(se->score))
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "shared expert: NULL or misaligned tensor (w 4 B, scales/biases 2 B)");
    int rc = nmoe_check_x(ctx, x, x_dtype, ntok);
    if (rc != NMOE_HIP_OK) return rc;
    if (shared_out == NULL || shared_gate_raw == NULL || !nmoe_aligned(shared_out, 16))
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "shared_out (16-byte aligned) and shared_gate_raw are required");
    const int tpb = ntok <= 4 ? ntok : 4;
    const dim3 ggu(NMOE_INTER / 4 + 1, (ntok + tpb - 1) / tpb), gdn(NMOE_HIDDEN / 4, (ntok + tpb - 1) / tpb);
    hipStream_t s = nmoe_stream_of(ctx, stream);
    if (x_dtype == NMOE_HIP_BF16)
        hipLaunchKernelGGL(nmoe_shared_gateup_kernel<uint16_t>, ggu, dim3(256), 0, s, se->gate.w, se->gate.scales,
                           se->gate.biases, se->up.w, se->up.scales, se->up.biases, se->score.w, se->score.scales,
                           se->score.biases, (const uint16_t *)x, ntok, tpb, ctx->s_act, shared_gate_raw);
    else
        hipLaunchKernelGGL(nmoe_shared_gateup_kernel<float>, ggu, dim3(256), 0, s, se->gate.w, se->gate.scales,
                           se->gate.biases, se->up.w, se->up.scales, se->up.biases, se->score.w, se->score.scales,
                           se->score.biases, (const float *)x, ntok, tpb, ctx->s_act, shared_gate_raw);
    hipLaunchKernelGGL(nmoe_shared_down_kernel, gdn, dim3(256), 0, s, se->down.w, se->down.scales, se->down.biases,
                       (const float *)ctx->s_act, ntok, tpb, shared_out);
    NMOE_HIP_TRY(ctx, hipGetLastError());
    return NMOE_HIP_OK;
}
