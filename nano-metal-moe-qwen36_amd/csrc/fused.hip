/*
 * fused.hip -- the whole batch-1 routed-MoE step in one persistent launch.
 *
 * Reference: the per-layer MoE tail NMOEPipelinedExpertTail
 * (src/runtime.m:2908-2999) runs router logits on the GPU
 * (kernels.metal:472-513), routes on the host (runtime.m:1498-1511, math.m),
 * preads the K selected experts, then runs gate/up + SwiGLU
 * (kernels.metal:562-640) and down + weighted combine (kernels.metal:
 * 1456-1542) -- three host/device crossings per layer.  Here the layer pack
 * is resident in HBM and the step is one cooperative kernel of 256 blocks x
 * 4 wavefronts with two grid barriers:
 *
 *   R  router: wave 0 of block b computes logit b (1 MB bf16 router read
 *      once across the grid), writes it to global scratch.      -- barrier 1
 *   T  every block routes the token itself from the 256 logits (bit-exact
 *      math.m softmax / top-k / renormalise in one wavefront), so no second
 *      barrier is needed to publish the routing.
 *   P  every wavefront issues all of its weight loads at once: its gate/up
 *      rows (K x 512 rows spread over the grid's 1024 wavefronts) AND the
 *      down rows it will need after the next barrier (block b owns output
 *      rows 8b..8b+7 of all K experts), so the down stream overlaps the
 *      gate/up stream: ~14 MB in flight in one wave of requests.
 *   G  gate/up dot products + SwiGLU -> act[K][512] in global scratch.
 *                                                             -- barrier 2
 *   D  down dot products from the prefetched registers against act, then
 *      out = h_mid + sum_s w_s y_s (+ sigmoid(g) shared), slot order.
 *
 * Without routing (routing given), R and T are skipped and there is one
 * barrier.  The grid is launched cooperatively, so all 256 blocks are
 * co-resident; every wait is bounded (nmoe_grid_barrier).
 */
#include "nmoe_device.h"

#pragma clang fp contract(off)

static __constant__ uint64_t nmoe_fused_exp2_tab[32] = NMOE_EXP2_TAB32;

#define NMOE_FUSED_BLOCKS 256
#define NMOE_FUSED_WAVES 4
#define NMOE_FUSED_MAXS 4 /* weight-load steps per wavefront and phase */
#define NMOE_FUSED_OUT_ROWS (NMOE_HIDDEN / NMOE_FUSED_BLOCKS) /* 8 output rows per block */

struct nmoe_fused_args {
    const uint8_t *pack;
    const uint16_t *router_w; /* bf16 [256][2048] (ROUTE) */
    const void *x;            /* [2048] fp32 or bf16 */
    int k;
    const uint32_t *idx_in; /* [8] (!ROUTE) */
    const float *w_in;      /* [8] (!ROUTE) */
    const float *h_mid;
    const float *shared_out;
    const float *shared_gate_raw;
    float *out;
    uint32_t *idx_out; /* nullable (ROUTE) */
    float *w_out;      /* nullable (ROUTE) */
    float *logits;     /* [256] global scratch / output (ROUTE) */
    float *act;        /* [8][512] global scratch */
    uint32_t *sync;
};

template <int BITS, bool ROUTE, typename XT>
__global__ void __launch_bounds__(256) nmoe_fused_decode_kernel(nmoe_fused_args a) {
    using Q = nmoe_q<BITS>;
    using L = nmoe_layout<BITS>;
    constexpr int RPS = NMOE_WAVE / Q::LPR_G; /* gate/up rows per wave step: 1 (q4) / 2 (q2) */
    constexpr int RPW_D = NMOE_WAVE / Q::LPR_D; /* down rows per wave step: 4 (q4) / 8 (q2) */
    constexpr int DSTEPS_PER_EXPERT = NMOE_FUSED_OUT_ROWS / RPW_D; /* 2 (q4) / 1 (q2) */
    __shared__ float route_scratch[NMOE_EXPERTS];
    __shared__ uint32_t s_idx[NMOE_MAX_K];
    __shared__ float s_w[NMOE_MAX_K];
    __shared__ float s_y[NMOE_MAX_K][NMOE_FUSED_OUT_ROWS];

    const int nb = gridDim.x;
    const int b = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int k = a.k;
    const XT *x = (const XT *)a.x;
    uint32_t phase_target = 0;

    if (ROUTE) {
        /* ---- R: router rows, one per block (wave 0) */
        if (wave == 0) {
            for (int e = b; e < NMOE_EXPERTS; e += nb) {
                const uint4 *row = (const uint4 *)(a.router_w + (size_t)e * NMOE_HIDDEN);
                uint4 wv[4];
                float xs[32];
#pragma unroll
                for (int j = 0; j < 4; j++) wv[j] = row[lane + 64 * j];
#pragma unroll
                for (int j = 0; j < 4; j++) nmoe_load_cols<XT>(x, (lane + 64 * j) * 8, 8, xs + 8 * j);
                float logit = nmoe_router_row_bf16(wv, xs);
                if (lane == 0) a.logits[e] = logit;
            }
        }
        phase_target += (uint32_t)nb;
        nmoe_grid_barrier(a.sync, phase_target);
        /* ---- T: route the token in every block */
        if (wave == 0) {
            uint32_t si[NMOE_MAX_K];
            float sw[NMOE_MAX_K];
            nmoe_wave_route(a.logits, NMOE_EXPERTS, k, route_scratch, nmoe_fused_exp2_tab, si, sw, NULL);
            if (lane < NMOE_MAX_K) {
                uint32_t vi = 0;
                float vw = 0.0f;
#pragma unroll
                for (int s = 0; s < NMOE_MAX_K; s++)
                    if (s == lane) {
                        vi = si[s];
                        vw = sw[s];
                    }
                s_idx[lane] = vi;
                s_w[lane] = vw;
                if (b == 0 && a.idx_out != NULL) a.idx_out[lane] = vi;
                if (b == 0 && a.w_out != NULL) a.w_out[lane] = vw;
            }
        }
    } else {
        if (threadIdx.x < NMOE_MAX_K) {
            uint32_t e = threadIdx.x < (unsigned)k ? a.idx_in[threadIdx.x] : 0u;
            float wv = threadIdx.x < (unsigned)k ? a.w_in[threadIdx.x] : 0.0f;
            /* an index outside the layer is an invalid slot: weight 0
             * (failed expert reads get weight 0, runtime.m:2977-2981) */
            s_w[threadIdx.x] = e < NMOE_EXPERTS ? wv : 0.0f;
            s_idx[threadIdx.x] = e < NMOE_EXPERTS ? e : 0u;
        }
    }
    __syncthreads();

    /* ---- P: issue every weight load of this wavefront */
    const int nw = nb * NMOE_FUSED_WAVES;
    const int gw = b * NMOE_FUSED_WAVES + wave;
    const int g_units = k * (NMOE_INTER / RPS);
    const int gsub = lane / Q::LPR_G, gl = lane % Q::LPR_G;
    const int ggrp = gl * Q::CPL / NMOE_GROUP;
    uint4 gwv[NMOE_FUSED_MAXS], uwv[NMOE_FUSED_MAXS];
    uint32_t gsb[NMOE_FUSED_MAXS], usb[NMOE_FUSED_MAXS]; /* scale | bias << 16 */
#pragma unroll
    for (int i = 0; i < NMOE_FUSED_MAXS; i++) {
        int u = gw + nw * i;
        if (u < g_units) {
            int s = u / (NMOE_INTER / RPS);
            int row = (u % (NMOE_INTER / RPS)) * RPS + gsub;
            const uint8_t *ex = a.pack + (size_t)s_idx[s] * L::expert_size;
            gwv[i] = ((const uint4 *)(ex + L::gate_w))[(size_t)row * (Q::WPR_G / 4) + gl];
            uwv[i] = ((const uint4 *)(ex + L::up_w))[(size_t)row * (Q::WPR_G / 4) + gl];
            const uint16_t *gs = (const uint16_t *)(ex + L::gate_s) + row * Q::GPR_G + ggrp;
            const uint16_t *us = (const uint16_t *)(ex + L::up_s) + row * Q::GPR_G + ggrp;
            gsb[i] = (uint32_t)gs[0] | ((uint32_t)gs[NMOE_INTER * Q::GPR_G] << 16);
            usb[i] = (uint32_t)us[0] | ((uint32_t)us[NMOE_INTER * Q::GPR_G] << 16);
        }
    }
    const int d_units = k * DSTEPS_PER_EXPERT;
    const int dsub = lane / Q::LPR_D, dl = lane % Q::LPR_D;
    const int dgrp = dl * Q::CPL / NMOE_GROUP;
    uint4 dwv[NMOE_FUSED_MAXS];
    uint32_t dsb[NMOE_FUSED_MAXS];
#pragma unroll
    for (int i = 0; i < NMOE_FUSED_MAXS; i++) {
        int v = wave + NMOE_FUSED_WAVES * i;
        if (v < d_units) {
            int s = v / DSTEPS_PER_EXPERT;
            int row = b * NMOE_FUSED_OUT_ROWS + (v % DSTEPS_PER_EXPERT) * RPW_D + dsub;
            const uint8_t *ex = a.pack + (size_t)s_idx[s] * L::expert_size;
            dwv[i] = ((const uint4 *)(ex + L::down_w))[(size_t)row * (Q::WPR_D / 4) + dl];
            const uint16_t *ds = (const uint16_t *)(ex + L::down_s) + row * Q::GPR_D + dgrp;
            dsb[i] = (uint32_t)ds[0] | ((uint32_t)ds[NMOE_HIDDEN * Q::GPR_D] << 16);
        }
    }

    /* ---- G: gate/up + SwiGLU */
    {
        float xs[Q::CPL];
        nmoe_load_cols<XT>(x, gl * Q::CPL, Q::CPL, xs);
        float xsum = 0.0f;
#pragma unroll
        for (int c = 0; c < Q::CPL; c++) xsum += xs[c];
#pragma unroll
        for (int i = 0; i < NMOE_FUSED_MAXS; i++) {
            int u = gw + nw * i;
            if (u < g_units) { /* uniform across the wavefront */
                int s = u / (NMOE_INTER / RPS);
                int row = (u % (NMOE_INTER / RPS)) * RPS + gsub;
                float g = __builtin_fmaf(nmoe_bf16f(gsb[i] & 0xffffu), nmoe_dot16<BITS>(gwv[i], xs),
                                         nmoe_bf16f(gsb[i] >> 16) * xsum);
                float up = __builtin_fmaf(nmoe_bf16f(usb[i] & 0xffffu), nmoe_dot16<BITS>(uwv[i], xs),
                                          nmoe_bf16f(usb[i] >> 16) * xsum);
                g = nmoe_lanes_sum<Q::LPR_G>(g);
                up = nmoe_lanes_sum<Q::LPR_G>(up);
                if (gl == 0) a.act[s * NMOE_INTER + row] = nmoe_silu_dev(g) * up;
            }
        }
    }
    phase_target += (uint32_t)nb;
    nmoe_grid_barrier(a.sync, phase_target);

    /* ---- D: down + combine */
#pragma unroll
    for (int i = 0; i < NMOE_FUSED_MAXS; i++) {
        int v = wave + NMOE_FUSED_WAVES * i;
        if (v < d_units) {
            int s = v / DSTEPS_PER_EXPERT;
            int rloc = (v % DSTEPS_PER_EXPERT) * RPW_D + dsub;
            float as[Q::CPL];
            const float4 *a4 = (const float4 *)(a.act + s * NMOE_INTER + dl * Q::CPL);
#pragma unroll
            for (int c = 0; c < Q::CPL / 4; c++) {
                float4 t = a4[c];
                as[4 * c] = t.x;
                as[4 * c + 1] = t.y;
                as[4 * c + 2] = t.z;
                as[4 * c + 3] = t.w;
            }
            float asum = 0.0f;
#pragma unroll
            for (int c = 0; c < Q::CPL; c++) asum += as[c];
            float y = __builtin_fmaf(nmoe_bf16f(dsb[i] & 0xffffu), nmoe_dot16<BITS>(dwv[i], as),
                                     nmoe_bf16f(dsb[i] >> 16) * asum);
            y = nmoe_dpp_group_sum<Q::LPR_D>(y);
            if (dl == 0) s_y[s][rloc] = y;
        }
    }
    __syncthreads();
    if (threadIdx.x < NMOE_FUSED_OUT_ROWS) {
        int row = b * NMOE_FUSED_OUT_ROWS + threadIdx.x;
        float moe = 0.0f;
        for (int s = 0; s < k; s++) moe += s_w[s] * s_y[s][threadIdx.x];
        float r = a.h_mid[row] + moe;
        if (a.shared_out != NULL) r = r + nmoe_sigmoid_dev(a.shared_gate_raw[0]) * a.shared_out[row];
        a.out[row] = r;
    }
    nmoe_grid_exit(a.sync, (uint32_t)nb);
}

/* ----------------------------------------------------------- launching */

template <int BITS, bool ROUTE, typename XT>
static hipError_t nmoe_fused_launch(const nmoe_fused_args &args, hipStream_t s) {
    nmoe_fused_args a = args;
    void *kargs[] = {&a};
    return hipLaunchCooperativeKernel((const void *)nmoe_fused_decode_kernel<BITS, ROUTE, XT>,
                                      dim3(NMOE_FUSED_BLOCKS), dim3(256), kargs, 0, s);
}

template <int BITS, bool ROUTE, typename XT>
static int nmoe_fused_fits(int num_cus) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, nmoe_fused_decode_kernel<BITS, ROUTE, XT>, 256, 0) !=
        hipSuccess)
        return 0;
    return per_cu * num_cus >= NMOE_FUSED_BLOCKS;
}

extern "C" int nmoe_decode_init(nmoe_hip_ctx *ctx) {
    int coop = 0;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, ctx->device) != hipSuccess) coop = 0;
    int ok = coop && nmoe_fused_fits<4, true, uint16_t>(ctx->num_cus) && nmoe_fused_fits<4, true, float>(ctx->num_cus) &&
             nmoe_fused_fits<2, true, uint16_t>(ctx->num_cus) && nmoe_fused_fits<2, true, float>(ctx->num_cus) &&
             nmoe_fused_fits<4, false, uint16_t>(ctx->num_cus) && nmoe_fused_fits<4, false, float>(ctx->num_cus) &&
             nmoe_fused_fits<2, false, uint16_t>(ctx->num_cus) && nmoe_fused_fits<2, false, float>(ctx->num_cus);
    ctx->fused_blocks = ok ? NMOE_FUSED_BLOCKS : 0;
    return NMOE_HIP_OK;
}

/* One token; routing computed (route != 0) or given (idx_in / w_in). */
int nmoe_fused_decode(nmoe_hip_ctx *ctx, int bits, int route, const void *x, int x_dtype, int k,
                      const uint16_t *router_w, const uint32_t *idx_in, const float *w_in, const float *h_mid,
                      const float *shared_out, const float *shared_gate_raw, float *out, uint32_t *idx_out,
                      float *w_out, float *logits, const uint8_t *pack, hipStream_t s) {
    nmoe_fused_args a;
    a.pack = pack;
    a.router_w = router_w;
    a.x = x;
    a.k = k;
    a.idx_in = idx_in;
    a.w_in = w_in;
    a.h_mid = h_mid;
    a.shared_out = shared_out;
    a.shared_gate_raw = shared_gate_raw;
    a.out = out;
    a.idx_out = idx_out;
    a.w_out = w_out;
    a.logits = logits != NULL ? logits : ctx->logits;
    a.act = ctx->act;
    a.sync = ctx->sync;
    bool bf = x_dtype == NMOE_HIP_BF16;
    hipError_t e;
    if (bits == 4) {
        if (route)
            e = bf ? nmoe_fused_launch<4, true, uint16_t>(a, s) : nmoe_fused_launch<4, true, float>(a, s);
        else
            e = bf ? nmoe_fused_launch<4, false, uint16_t>(a, s) : nmoe_fused_launch<4, false, float>(a, s);
    } else {
        if (route)
            e = bf ? nmoe_fused_launch<2, true, uint16_t>(a, s) : nmoe_fused_launch<2, true, float>(a, s);
        else
            e = bf ? nmoe_fused_launch<2, false, uint16_t>(a, s) : nmoe_fused_launch<2, false, float>(a, s);
    }
    if (e != hipSuccess) return nmoe_hip_check(ctx, e, "hipLaunchCooperativeKernel(fused decode)");
    return NMOE_HIP_OK;
}
