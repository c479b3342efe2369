/*
 * experts.hip -- routed-expert gate/up + SwiGLU and down + weighted combine
 * for q4 / q2 packs resident in HBM (the multi-launch decode path).
 *
 * Reference: metal/kernels.metal:562-640 (nmoe_expert_gate_up_q4_batched:
 * per expert row, SiLU(gate.x) * (up.x)), 642-714 / 1456-1542 (down and the
 * fused weighted combine), 1394-1454 (weighted sum into the residual);
 * q2 runs as separate dequant matvecs (kernels.metal:192-238, 303-319).
 * Expert bases are `layer_pack + idx[slot] * expert_size`, as in the
 * reference's all-resident variant (kernels.metal:716-856).
 *
 * MI355X mapping.  Every lane loads exactly 16 bytes (4 packed words) of a
 * row per step, so a wavefront covers 1 KB:
 *   q4 gate/up row = 256 words -> 64 lanes per row (32 columns per lane)
 *   q2 gate/up row = 128 words -> 32 lanes per row (64 columns per lane)
 *   q4 down row    =  64 words -> 16 lanes per row (4 rows per wavefront)
 *   q2 down row    =  32 words ->  8 lanes per row (8 rows per wavefront)
 * A lane's columns always sit inside one 64-column quantisation group, so
 * its partial dot product is  scale * sum(q * x) + bias * sum(x)  with one
 * scale/bias pair; sum(x) over the lane's columns is computed once and reused
 * for every row.  Nibbles/crumbs are expanded with byte masks and
 * v_cvt_f32_ubyte{0..3}; accumulation is fp32.
 */
#include <string.h>

#include "nmoe_device.h"

/* ----------------------------------------------------------- gate/up */

#define NMOE_GU_ROWS_PER_WAVE 4
#define NMOE_GU_WAVES 4
#define NMOE_GU_ROWS_PER_BLOCK (NMOE_GU_ROWS_PER_WAVE * NMOE_GU_WAVES)

/* grid (512/16, k, ntok), 256 threads.  act[t][s][row] = SiLU(g)*u. */
template <int BITS, typename XT>
__global__ void __launch_bounds__(256) nmoe_gateup_kernel(const uint8_t *__restrict__ pack, const XT *__restrict__ x,
                                                          const uint32_t *__restrict__ idx, float *__restrict__ act) {
    using Q = nmoe_q<BITS>;
    using L = nmoe_layout<BITS>;
    constexpr int RPS = NMOE_WAVE / Q::LPR_G;           /* rows per wave step: 1 (q4) / 2 (q2) */
    constexpr int STEPS = NMOE_GU_ROWS_PER_WAVE / RPS;
    const int t = blockIdx.z, s = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int sub = lane / Q::LPR_G, l = lane % Q::LPR_G;
    uint32_t e = idx[(size_t)t * NMOE_MAX_K + s];
    e = e < NMOE_EXPERTS ? e : 0u; /* invalid slot: never read outside the pack */
    const uint8_t *ex = pack + (size_t)e * L::expert_size;
    const int row0 = blockIdx.x * NMOE_GU_ROWS_PER_BLOCK + wave * NMOE_GU_ROWS_PER_WAVE + sub;

    uint4 gw[STEPS], uw[STEPS];
    uint32_t gs[STEPS], gb[STEPS], us[STEPS], ub[STEPS];
    const int grp = l * Q::CPL / NMOE_GROUP;
#pragma unroll
    for (int i = 0; i < STEPS; i++) {
        int row = row0 + i * RPS;
        gw[i] = ((const uint4 *)(ex + L::gate_w))[(size_t)row * (Q::WPR_G / 4) + l];
        uw[i] = ((const uint4 *)(ex + L::up_w))[(size_t)row * (Q::WPR_G / 4) + l];
        gs[i] = ((const uint16_t *)(ex + L::gate_s))[row * Q::GPR_G + grp];
        gb[i] = ((const uint16_t *)(ex + L::gate_b))[row * Q::GPR_G + grp];
        us[i] = ((const uint16_t *)(ex + L::up_s))[row * Q::GPR_G + grp];
        ub[i] = ((const uint16_t *)(ex + L::up_b))[row * Q::GPR_G + grp];
    }
    float xs[Q::CPL];
    nmoe_load_cols<XT>(x + (size_t)t * NMOE_HIDDEN, l * Q::CPL, Q::CPL, xs);
    float xsum = 0.0f;
#pragma unroll
    for (int c = 0; c < Q::CPL; c++) xsum += xs[c];

#pragma unroll
    for (int i = 0; i < STEPS; i++) {
        float g = __builtin_fmaf(nmoe_bf16f(gs[i]), nmoe_dot16<BITS>(gw[i], xs), nmoe_bf16f(gb[i]) * xsum);
        float u = __builtin_fmaf(nmoe_bf16f(us[i]), nmoe_dot16<BITS>(uw[i], xs), nmoe_bf16f(ub[i]) * xsum);
        g = nmoe_lanes_sum<Q::LPR_G>(g);
        u = nmoe_lanes_sum<Q::LPR_G>(u);
        if (l == 0) act[((size_t)t * NMOE_MAX_K + s) * NMOE_INTER + row0 + i * RPS] = nmoe_silu_dev(g) * u;
    }
}

/* -------------------------------------------------------- down+combine */

#define NMOE_DC_WAVES 4

/* LDS position of act column `col` so that the LPR_D lanes of a row read
 * consecutive 16-byte chunks (conflict-free ds_read_b128). */
template <int BITS>
__device__ __forceinline__ int nmoe_act_swz(int col) {
    using Q = nmoe_q<BITS>;
    return (((col % Q::CPL) >> 2) * Q::LPR_D + col / Q::CPL) * 4 + (col & 3);
}

/* grid (2048 / rows_per_block, ntok), 256 threads.
 * out[t][r] = h_mid[t][r] + sum_s w[t][s] * y_s[r] (+ sigmoid(g_t) * shared[t][r]). */
template <int BITS>
__global__ void __launch_bounds__(256) nmoe_down_combine_kernel(
    const uint8_t *__restrict__ pack, int k, const uint32_t *__restrict__ idx, const float *__restrict__ wts,
    const float *__restrict__ act, const float *h_mid, const float *__restrict__ shared_out,
    const float *__restrict__ shared_gate_raw, float *out) {
    using Q = nmoe_q<BITS>;
    using L = nmoe_layout<BITS>;
    constexpr int RPW = NMOE_WAVE / Q::LPR_D;            /* rows per wavefront: 4 (q4) / 8 (q2) */
    constexpr int RPB = RPW * NMOE_DC_WAVES;
    __shared__ float4 act_s[NMOE_MAX_K * NMOE_INTER / 4];
    __shared__ float asum_s[NMOE_MAX_K][Q::LPR_D];
    const int t = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int sub = lane / Q::LPR_D, l = lane % Q::LPR_D;
    const int row = blockIdx.x * RPB + wave * RPW + sub;

    /* issue the weight loads for all slots first */
    uint4 dw[NMOE_MAX_K];
    uint32_t ds[NMOE_MAX_K], db[NMOE_MAX_K];
    float wk[NMOE_MAX_K];
    const int grp = l * Q::CPL / NMOE_GROUP;
#pragma unroll
    for (int s = 0; s < NMOE_MAX_K; s++) {
        if (s < k) {
            uint32_t e = idx[(size_t)t * NMOE_MAX_K + s];
            /* an index outside the layer is an invalid slot: weight 0, as for
             * a failed expert read in the reference (runtime.m:2977-2981) */
            wk[s] = e < NMOE_EXPERTS ? wts[(size_t)t * NMOE_MAX_K + s] : 0.0f;
            e = e < NMOE_EXPERTS ? e : 0u;
            const uint8_t *ex = pack + (size_t)e * L::expert_size;
            dw[s] = ((const uint4 *)(ex + L::down_w))[(size_t)row * (Q::WPR_D / 4) + l];
            ds[s] = ((const uint16_t *)(ex + L::down_s))[row * Q::GPR_D + grp];
            db[s] = ((const uint16_t *)(ex + L::down_b))[row * Q::GPR_D + grp];
        }
    }
    /* stage this token's activations, swizzled */
    const float4 *a4 = (const float4 *)(act + (size_t)t * NMOE_MAX_K * NMOE_INTER);
    for (int f = threadIdx.x; f < k * (NMOE_INTER / 4); f += blockDim.x) {
        int s = f / (NMOE_INTER / 4), col = (f % (NMOE_INTER / 4)) * 4;
        act_s[s * (NMOE_INTER / 4) + (nmoe_act_swz<BITS>(col) >> 2)] = a4[f];
    }
    __syncthreads();
    for (int p = threadIdx.x; p < k * Q::LPR_D; p += blockDim.x) {
        int s = p / Q::LPR_D, ll = p % Q::LPR_D;
        float a = 0.0f;
        for (int c = 0; c < Q::CPL / 4; c++) {
            float4 v = act_s[s * (NMOE_INTER / 4) + c * Q::LPR_D + ll];
            a += (v.x + v.y) + (v.z + v.w);
        }
        asum_s[s][ll] = a;
    }
    __syncthreads();

    float moe = 0.0f;
#pragma unroll
    for (int s = 0; s < NMOE_MAX_K; s++) {
        if (s < k) {
            float xs[Q::CPL];
#pragma unroll
            for (int c = 0; c < Q::CPL / 4; c++) {
                float4 v = act_s[s * (NMOE_INTER / 4) + c * Q::LPR_D + l];
                xs[4 * c] = v.x; xs[4 * c + 1] = v.y; xs[4 * c + 2] = v.z; xs[4 * c + 3] = v.w;
            }
            float y = __builtin_fmaf(nmoe_bf16f(ds[s]), nmoe_dot16<BITS>(dw[s], xs), nmoe_bf16f(db[s]) * asum_s[s][l]);
            y = nmoe_dpp_group_sum<Q::LPR_D>(y);
            moe += wk[s] * y;
        }
    }
    if (l == 0) {
        size_t o = (size_t)t * NMOE_HIDDEN + row;
        float r = h_mid[o] + moe;
        if (shared_out != NULL) r = r + nmoe_sigmoid_dev(shared_gate_raw[t]) * shared_out[o];
        out[o] = r;
    }
}

/* ------------------------------------------------------- entry points */

int nmoe_check_x(nmoe_hip_ctx *ctx, const void *x, int x_dtype, int ntok);
int nmoe_check_router(nmoe_hip_ctx *ctx, const nmoe_hip_router *r);

static int nmoe_check_experts(nmoe_hip_ctx *ctx, int layer, int bits, const void *x, int x_dtype, int ntok, int k,
                              const uint32_t *idx, const float *w, const float *h_mid, const float *shared_out,
                              const float *shared_gate_raw, const float *out, const uint8_t **pack) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (k < 1 || k > NMOE_MAX_K) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "k=%d outside 1..8", k);
    int rc = nmoe_check_x(ctx, x, x_dtype, ntok);
    if (rc != NMOE_HIP_OK) return rc;
    if (idx == NULL || w == NULL || h_mid == NULL || out == NULL)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "NULL idx/w/h_mid/out");
    if (!nmoe_aligned(h_mid, 4) || !nmoe_aligned(out, 4) || !nmoe_aligned(idx, 4) || !nmoe_aligned(w, 4))
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "misaligned idx/w/h_mid/out");
    if ((shared_out == NULL) != (shared_gate_raw == NULL))
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "shared_out and shared_gate_raw must both be set or both NULL");
    if (layer < 0 || layer >= NMOE_HIP_MAX_LAYERS || ctx->packs[layer].dev == NULL)
        return nmoe_fail(ctx, NMOE_HIP_ENOENT, "layer %d has no resident pack", layer);
    if (ctx->packs[layer].bits != bits)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "layer %d is q%d, called as q%d", layer, ctx->packs[layer].bits, bits);
    *pack = (const uint8_t *)ctx->packs[layer].dev;
    return NMOE_HIP_OK;
}

extern "C" int nmoe_grouped_experts(nmoe_hip_ctx *ctx, int bits, const uint8_t *pack, const void *x, int x_dtype,
                                    int ntok, int k, const uint32_t *idx, const float *w, const float *h_mid,
                                    const float *shared_out, const float *shared_gate_raw, float *out,
                                    hipStream_t s);
extern "C" int nmoe_grouped_dispatch(nmoe_hip_ctx *ctx, const uint32_t *idx, int ntok, int k, uint32_t *perm,
                                     uint32_t *offsets, hipStream_t s);

extern "C" int nmoe_moe_dispatch(nmoe_hip_ctx *ctx, const uint32_t *idx, int ntok, int k, uint32_t *perm,
                                 uint32_t *offsets, void *stream) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (k < 1 || k > NMOE_MAX_K) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "k=%d outside 1..8", k);
    if (ntok < 1 || ntok > ctx->max_tokens)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "ntok=%d outside 1..%d", ntok, ctx->max_tokens);
    if (idx == NULL || perm == NULL || offsets == NULL) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "NULL idx/perm/offsets");
    if (!nmoe_aligned(idx, 4) || !nmoe_aligned(perm, 4) || !nmoe_aligned(offsets, 4))
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "misaligned idx/perm/offsets");
    return nmoe_grouped_dispatch(ctx, idx, ntok, k, perm, offsets, nmoe_stream_of(ctx, stream));
}

/* The per-token expert kernels (gate/up + SwiGLU into act [ntok][8][512],
 * then down + combine), arguments already checked. */
template <int BITS>
static hipError_t nmoe_launch_experts_act(const uint8_t *pack, const void *x, int x_dtype, int ntok, int k,
                                          const uint32_t *idx, const float *w, const float *h_mid,
                                          const float *shared_out, const float *shared_gate_raw, float *out,
                                          float *act, hipStream_t s) {
    using Q = nmoe_q<BITS>;
    dim3 g1(NMOE_INTER / NMOE_GU_ROWS_PER_BLOCK, k, ntok);
    if (x_dtype == NMOE_HIP_BF16)
        hipLaunchKernelGGL((nmoe_gateup_kernel<BITS, uint16_t>), g1, dim3(256), 0, s, pack, (const uint16_t *)x, idx,
                           act);
    else
        hipLaunchKernelGGL((nmoe_gateup_kernel<BITS, float>), g1, dim3(256), 0, s, pack, (const float *)x, idx, act);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    constexpr int RPB = (NMOE_WAVE / Q::LPR_D) * NMOE_DC_WAVES;
    dim3 g2(NMOE_HIDDEN / RPB, ntok);
    hipLaunchKernelGGL((nmoe_down_combine_kernel<BITS>), g2, dim3(256), 0, s, pack, k, idx, w, act, h_mid, shared_out,
                       shared_gate_raw, out);
    return hipGetLastError();
}

extern "C" hipError_t nmoe_experts_launch(int bits, const uint8_t *pack, const void *x, int x_dtype, int ntok, int k,
                                         const uint32_t *idx, const float *w, const float *h_mid,
                                         const float *shared_out, const float *shared_gate_raw, float *out,
                                         float *act, hipStream_t s) {
    return bits == 4 ? nmoe_launch_experts_act<4>(pack, x, x_dtype, ntok, k, idx, w, h_mid, shared_out,
                                                   shared_gate_raw, out, act, s)
                     : nmoe_launch_experts_act<2>(pack, x, x_dtype, ntok, k, idx, w, h_mid, shared_out,
                                                   shared_gate_raw, out, act, s);
}

template <int BITS>
static int nmoe_launch_experts(nmoe_hip_ctx *ctx, const uint8_t *pack, const void *x, int x_dtype, int ntok, int k,
                               const uint32_t *idx, const float *w, const float *h_mid, const float *shared_out,
                               const float *shared_gate_raw, float *out, hipStream_t s) {
    NMOE_HIP_TRY(ctx, nmoe_launch_experts_act<BITS>(pack, x, x_dtype, ntok, k, idx, w, h_mid, shared_out,
                                                    shared_gate_raw, out, ctx->act, s));
    return NMOE_HIP_OK;
}

extern "C" int nmoe_fused_decode(nmoe_hip_ctx *ctx, int bits, int route, const void *x, int xmode, float eps, int k,
                                 const nmoe_hip_router *router, const uint32_t *idx_in, const float *w_in,
                                 const float *h_mid, const float *shared_out, const float *shared_gate_raw, float *out,
                                 uint32_t *idx_out, float *w_out, float *logits_out, const uint8_t *pack,
                                 hipStream_t s);

/* The layer's pack (checked resident, of BITS), by the token count: the
 * fused single-token launch, the grouped GEMMs (on the stripe-major copy)
 * or the per-token kernels. */
template <int BITS>
static int nmoe_experts_dispatch(nmoe_hip_ctx *ctx, int layer, const void *x, int x_dtype, int ntok, int k,
                                 const uint32_t *idx, const float *w, const float *h_mid, const float *shared_out,
                                 const float *shared_gate_raw, float *out, hipStream_t s) {
    const uint8_t *pack = (const uint8_t *)ctx->packs[layer].dev;
    if (ntok == 1 && ctx->fused_blocks > 0 && ctx->use_fused)
        return nmoe_fused_decode(ctx, BITS, 0, x, x_dtype, 0.0f, k, NULL, idx, w, h_mid, shared_out, shared_gate_raw,
                                 out, NULL, NULL, NULL, pack, s);
    if (ntok >= ctx->grouped_min_tokens)
        return nmoe_grouped_experts(ctx, BITS, (const uint8_t *)ctx->packs[layer].stripes, x, x_dtype, ntok, k, idx,
                                    w, h_mid, shared_out, shared_gate_raw, out, s);
    return nmoe_launch_experts<BITS>(ctx, pack, x, x_dtype, ntok, k, idx, w, h_mid, shared_out, shared_gate_raw, out, s);
}

extern "C" int nmoe_moe_experts_q4(nmoe_hip_ctx *ctx, int layer, const void *x, int x_dtype, int ntok, int k,
                                   const uint32_t *idx, const float *w, const float *h_mid, const float *shared_out,
                                   const float *shared_gate_raw, float *out, void *stream) {
    const uint8_t *pack = NULL;
    int rc = nmoe_check_experts(ctx, layer, 4, x, x_dtype, ntok, k, idx, w, h_mid, shared_out, shared_gate_raw, out,
                                &pack);
    if (rc != NMOE_HIP_OK) return rc;
    rc = nmoe_experts_dispatch<4>(ctx, layer, x, x_dtype, ntok, k, idx, w, h_mid, shared_out, shared_gate_raw, out,
                                  nmoe_stream_of(ctx, stream));
    return rc != NMOE_HIP_OK ? rc : nmoe_sync_check(ctx, stream);
}

extern "C" int nmoe_moe_experts_q2(nmoe_hip_ctx *ctx, int layer, const void *x, int x_dtype, int ntok, int k,
                                   const uint32_t *idx, const float *w, const float *h_mid, const float *shared_out,
                                   const float *shared_gate_raw, float *out, void *stream) {
    const uint8_t *pack = NULL;
    int rc = nmoe_check_experts(ctx, layer, 2, x, x_dtype, ntok, k, idx, w, h_mid, shared_out, shared_gate_raw, out,
                                &pack);
    if (rc != NMOE_HIP_OK) return rc;
    rc = nmoe_experts_dispatch<2>(ctx, layer, x, x_dtype, ntok, k, idx, w, h_mid, shared_out, shared_gate_raw, out,
                                  nmoe_stream_of(ctx, stream));
    return rc != NMOE_HIP_OK ? rc : nmoe_sync_check(ctx, stream);
}

extern "C" int nmoe_grouped_experts_routed(nmoe_hip_ctx *ctx, int bits, const uint8_t *pack, const float *logits,
                                           const void *x, int x_dtype, int ntok, int k, uint32_t *idx, float *w,
                                           const float *h_mid, const float *shared_out, const float *shared_gate_raw,
                                           float *out, hipStream_t s);
extern "C" hipError_t nmoe_topk_launch(const float *logits, int ntok, int num_experts, int k, uint32_t *idx, float *w,
                                      float *probs, hipStream_t s);
extern "C" hipError_t nmoe_router_logits_launch(const nmoe_hip_router *router, const void *x, int x_dtype, int ntok,
                                               float *logits, hipStream_t s);

/* Routing from the given logits and the routed experts in one call: from
 * grouped_min_tokens tokens on, the routing runs inside the grouped path's
 * preparation launch (no launch of its own); below, the top-k launch and
 * the per-token kernels. */
static int nmoe_experts_from_logits_run(nmoe_hip_ctx *ctx, int layer, const float *logits, const void *x,
                                        int x_dtype, int ntok, int k, const float *h_mid, const float *shared_out,
                                        const float *shared_gate_raw, float *out, uint32_t *idx, float *w,
                                        hipStream_t s) {
    const int bits = ctx->packs[layer].bits;
    if (ntok >= ctx->grouped_min_tokens)
        return nmoe_grouped_experts_routed(ctx, bits, (const uint8_t *)ctx->packs[layer].stripes, logits, x, x_dtype,
                                           ntok, k, idx, w, h_mid, shared_out, shared_gate_raw, out, s);
    NMOE_HIP_TRY(ctx, nmoe_topk_launch(logits, ntok, NMOE_EXPERTS, k, idx, w, NULL, s));
    return bits == 4 ? nmoe_experts_dispatch<4>(ctx, layer, x, x_dtype, ntok, k, idx, w, h_mid, shared_out,
                                                shared_gate_raw, out, s)
                     : nmoe_experts_dispatch<2>(ctx, layer, x, x_dtype, ntok, k, idx, w, h_mid, shared_out,
                                                shared_gate_raw, out, s);
}

extern "C" int nmoe_moe_experts_from_logits(nmoe_hip_ctx *ctx, int layer, const float *logits, const void *x,
                                            int x_dtype, int ntok, int k, const float *h_mid, const float *shared_out,
                                            const float *shared_gate_raw, float *out, uint32_t *idx, float *w,
                                            void *stream) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (layer < 0 || layer >= NMOE_HIP_MAX_LAYERS || ctx->packs[layer].dev == NULL)
        return nmoe_fail(ctx, NMOE_HIP_ENOENT, "layer %d has no resident pack", layer);
    const uint8_t *pack = NULL;
    if (logits == NULL || !nmoe_aligned(logits, 4)) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "logits NULL or misaligned");
    int rc = nmoe_check_experts(ctx, layer, ctx->packs[layer].bits, x, x_dtype, ntok, k, idx, w, h_mid, shared_out,
                                shared_gate_raw, out, &pack);
    if (rc != NMOE_HIP_OK) return rc;
    rc = nmoe_experts_from_logits_run(ctx, layer, logits, x, x_dtype, ntok, k, h_mid, shared_out, shared_gate_raw, out,
                                      idx, w, nmoe_stream_of(ctx, stream));
    return rc != NMOE_HIP_OK ? rc : nmoe_sync_check(ctx, stream);
}

extern "C" int nmoe_moe_layer(nmoe_hip_ctx *ctx, int layer, const nmoe_hip_router *router, const void *x, int x_dtype,
                              int ntok, int k, const float *h_mid, const float *shared_out,
                              const float *shared_gate_raw, float *out, uint32_t *idx, float *w, float *logits,
                              void *stream) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (layer < 0 || layer >= NMOE_HIP_MAX_LAYERS || ctx->packs[layer].dev == NULL)
        return nmoe_fail(ctx, NMOE_HIP_ENOENT, "layer %d has no resident pack", layer);
    int rc = nmoe_check_router(ctx, router);
    if (rc != NMOE_HIP_OK) return rc;
    if (router->num_experts != NMOE_EXPERTS)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "a layer pack holds 256 experts; router has %d", router->num_experts);
    rc = nmoe_check_x(ctx, x, x_dtype, ntok);
    if (rc != NMOE_HIP_OK) return rc;
    if (k < 1 || k > NMOE_MAX_K) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "k=%d outside 1..8", k);
    if (h_mid == NULL || out == NULL) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "NULL h_mid/out");
    if ((shared_out == NULL) != (shared_gate_raw == NULL))
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "shared_out and shared_gate_raw must both be set or both NULL");
    if (ntok == 1 && ctx->fused_blocks > 0 && ctx->use_fused) {
        rc = nmoe_fused_decode(ctx, ctx->packs[layer].bits, 1, x, x_dtype, 0.0f, k, router, NULL, NULL, h_mid,
                               shared_out, shared_gate_raw, out, idx, w, logits,
                               (const uint8_t *)ctx->packs[layer].dev, nmoe_stream_of(ctx, stream));
        return rc != NMOE_HIP_OK ? rc : nmoe_sync_check(ctx, stream);
    }
    uint32_t *ri = idx != NULL ? idx : ctx->idx;
    float *rw = w != NULL ? w : ctx->w;
    if (ntok >= ctx->grouped_min_tokens) { /* the router launch, then routing and experts from its logits */
        const uint8_t *pack = NULL;
        float *lg = logits != NULL ? logits : ctx->logits;
        rc = nmoe_check_experts(ctx, layer, ctx->packs[layer].bits, x, x_dtype, ntok, k, ri, rw, h_mid, shared_out,
                                shared_gate_raw, out, &pack);
        if (rc != NMOE_HIP_OK) return rc;
        NMOE_HIP_TRY(ctx, nmoe_router_logits_launch(router, x, x_dtype, ntok, lg, nmoe_stream_of(ctx, stream)));
        rc = nmoe_experts_from_logits_run(ctx, layer, lg, x, x_dtype, ntok, k, h_mid, shared_out, shared_gate_raw, out,
                                          ri, rw, nmoe_stream_of(ctx, stream));
        return rc != NMOE_HIP_OK ? rc : nmoe_sync_check(ctx, stream);
    }
    rc = nmoe_moe_route(ctx, router, x, x_dtype, ntok, k, ri, rw, logits, stream);
    if (rc != NMOE_HIP_OK) return rc;
    if (ctx->packs[layer].bits == 4)
        return nmoe_moe_experts_q4(ctx, layer, x, x_dtype, ntok, k, ri, rw, h_mid, shared_out, shared_gate_raw, out,
                                   stream);
    return nmoe_moe_experts_q2(ctx, layer, x, x_dtype, ntok, k, ri, rw, h_mid, shared_out, shared_gate_raw, out,
                               stream);
}

/* nmoe_moe_layer_rmsnorm without the NMOE_HIP_OPT_SYNC_CHECK wait (the
 * stack checks once, after its last layer). */
extern "C" int nmoe_layer_rmsnorm_launch(nmoe_hip_ctx *ctx, int layer, const nmoe_hip_router *router,
                                         const float *h_in, float eps, int k, float *h_out, uint32_t *idx, float *w,
                                         float *logits, void *stream) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (layer < 0 || layer >= NMOE_HIP_MAX_LAYERS || ctx->packs[layer].dev == NULL)
        return nmoe_fail(ctx, NMOE_HIP_ENOENT, "layer %d has no resident pack", layer);
    int rc = nmoe_check_router(ctx, router);
    if (rc != NMOE_HIP_OK) return rc;
    if (router->num_experts != NMOE_EXPERTS)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "nmoe_moe_layer_rmsnorm needs a router of 256 experts");
    if (k < 1 || k > NMOE_MAX_K) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "k=%d outside 1..8", k);
    if (h_in == NULL || h_out == NULL || !nmoe_aligned(h_in, 16) || !nmoe_aligned(h_out, 4))
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "h_in (16-byte aligned) and h_out are required");
    if (h_in == h_out) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "h_out must not alias h_in");
    if (ctx->fused_blocks == 0)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "the device cannot hold the 256-block fused grid");
    return nmoe_fused_decode(ctx, ctx->packs[layer].bits, 1, h_in, 2 /* XNORM */, eps, k, router, NULL, NULL,
                             h_in, NULL, NULL, h_out, idx, w, logits, (const uint8_t *)ctx->packs[layer].dev,
                             nmoe_stream_of(ctx, stream));
}

extern "C" int nmoe_fused_stack(nmoe_hip_ctx *ctx, int bits, int q4r, int nl, const uint8_t *const *packs,
                                const nmoe_hip_router *routers, float *h_seq, float eps, int k, uint32_t *idx_seq,
                                float *w_seq, hipStream_t s);

/* nmoe_moe_stack as persistent launches, each running up to 64 of the
 * token's layers.  Checks every layer as nmoe_layer_rmsnorm_launch does
 * (so both forms reject the same calls); returns 1, having launched
 * nothing, when the layers do not share one bit width and one router kind
 * or the option is off. */
extern "C" int nmoe_stack_loop_launch(nmoe_hip_ctx *ctx, int nlayers, const int *layers,
                                      const nmoe_hip_router *routers, int k, float eps, float *h_seq,
                                      uint32_t *idx_seq, float *w_seq, void *stream) {
    constexpr int CHUNK = 64;
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (!ctx->stack_loop || ctx->fused_blocks == 0) return 1;
    int bits = 0, q4r = 0;
    for (int l = 0; l < nlayers; l++) {
        const int layer = layers[l];
        if (layer < 0 || layer >= NMOE_HIP_MAX_LAYERS || ctx->packs[layer].dev == NULL)
            return nmoe_fail(ctx, NMOE_HIP_ENOENT, "layer %d has no resident pack", layer);
        const int rc = nmoe_check_router(ctx, &routers[l]);
        if (rc != NMOE_HIP_OK) return rc;
        if (routers[l].num_experts != NMOE_EXPERTS)
            return nmoe_fail(ctx, NMOE_HIP_EINVAL, "nmoe_moe_layer_rmsnorm needs a router of 256 experts");
        const int q = routers[l].kind == NMOE_HIP_ROUTER_Q4;
        if (l == 0) {
            bits = ctx->packs[layer].bits;
            q4r = q;
        } else if (ctx->packs[layer].bits != bits || q != q4r) {
            return 1;
        }
    }
    if (k < 1 || k > NMOE_MAX_K) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "k=%d outside 1..8", k);
    if (!nmoe_aligned(h_seq, 16)) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "h_in (16-byte aligned) and h_out are required");
    const uint8_t *packs[CHUNK];
    for (int c = 0; c < nlayers; c += CHUNK) {
        const int n = nlayers - c < CHUNK ? nlayers - c : CHUNK;
        for (int l = 0; l < n; l++) packs[l] = (const uint8_t *)ctx->packs[layers[c + l]].dev;
        const int rc = nmoe_fused_stack(ctx, bits, q4r, n, packs, routers + c, h_seq + (size_t)c * NMOE_HIDDEN, eps, k,
                                        idx_seq != NULL ? idx_seq + (size_t)c * NMOE_MAX_K : NULL,
                                        w_seq != NULL ? w_seq + (size_t)c * NMOE_MAX_K : NULL,
                                        nmoe_stream_of(ctx, stream));
        if (rc != NMOE_HIP_OK) return rc;
    }
    return NMOE_HIP_OK;
}

extern "C" int nmoe_moe_layer_rmsnorm(nmoe_hip_ctx *ctx, int layer, const nmoe_hip_router *router,
                                      const float *h_in, float eps, int k, float *h_out, uint32_t *idx, float *w,
                                      float *logits, void *stream) {
    const int rc = nmoe_layer_rmsnorm_launch(ctx, layer, router, h_in, eps, k, h_out, idx, w, logits, stream);
    return rc != NMOE_HIP_OK ? rc : nmoe_sync_check(ctx, stream);
}

extern "C" int nmoe_fused_block(nmoe_hip_ctx *ctx, int bits, const nmoe_hip_router *router, const float *h_mid,
                                float eps, int k, const nmoe_block_ext *blk, float *out, uint32_t *idx_out,
                                float *w_out, float *logits_out, const uint8_t *pack, hipStream_t s);

static bool nmoe_qtensor_set(const nmoe_hip_qtensor &q) {
    return q.w != NULL && q.scales != NULL && q.biases != NULL && nmoe_aligned(q.w, 16) && nmoe_aligned(q.scales, 2) &&
           nmoe_aligned(q.biases, 2);
}

extern "C" int nmoe_moe_block(nmoe_hip_ctx *ctx, int layer, const nmoe_hip_moe_block *blk, const float *h_mid, int k,
                              float *out, float *next_x, uint32_t *idx, float *w, float *logits, void *stream) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (blk == NULL) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "NULL block descriptor");
    if (layer < 0 || layer >= NMOE_HIP_MAX_LAYERS || ctx->packs[layer].dev == NULL)
        return nmoe_fail(ctx, NMOE_HIP_ENOENT, "layer %d has no resident pack", layer);
    int rc = nmoe_check_router(ctx, &blk->router);
    if (rc != NMOE_HIP_OK) return rc;
    if (blk->router.num_experts != NMOE_EXPERTS)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "a layer pack holds 256 experts; router has %d", blk->router.num_experts);
    if (k < 1 || k > NMOE_MAX_K) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "k=%d outside 1..8", k);
    if (h_mid == NULL || out == NULL || !nmoe_aligned(h_mid, 16) || !nmoe_aligned(out, 4) ||
        (next_x != NULL && !nmoe_aligned(next_x, 4)))
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "h_mid (16-byte aligned) and out are required");
    if (blk->has_shared && !(nmoe_qtensor_set(blk->shared.gate) && nmoe_qtensor_set(blk->shared.up) &&
                             nmoe_qtensor_set(blk->shared.down) && nmoe_qtensor_set(blk->shared.score)))
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "shared expert: NULL or misaligned tensor (w 16 B, scales/biases 2 B)");
    if ((blk->post_norm != NULL && !nmoe_aligned(blk->post_norm, 2)) ||
        (blk->next_norm != NULL && !nmoe_aligned(blk->next_norm, 2)))
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "misaligned norm weight");
    if (!(blk->eps >= 0.0f)) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "eps must be >= 0");
    if (ctx->fused_blocks == 0)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "the device cannot hold the 256-block fused grid");
    nmoe_block_ext ext;
    memset(&ext, 0, sizeof(ext));
    ext.norm_w = blk->post_norm;
    ext.next_w = blk->next_norm;
    ext.add_one = blk->add_one != 0;
    ext.next_x = next_x;
    if (blk->has_shared) ext.sh = blk->shared;
    rc = nmoe_fused_block(ctx, ctx->packs[layer].bits, &blk->router, h_mid, blk->eps, k, &ext, out, idx, w, logits,
                          (const uint8_t *)ctx->packs[layer].dev, nmoe_stream_of(ctx, stream));
    return rc != NMOE_HIP_OK ? rc : nmoe_sync_check(ctx, stream);
}
