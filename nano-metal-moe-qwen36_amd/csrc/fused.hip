/*
 * fused.hip -- the whole batch-1 routed-MoE step in one launch.
 *
 * Reference: the per-layer MoE tail NMOEPipelinedExpertTail
 * (src/runtime.m:2908-2999) computes router logits on the GPU
 * (kernels.metal:472-513), routes on the host (runtime.m:1498-1511, math.m),
 * preads the K selected experts, then runs gate/up + SwiGLU
 * (kernels.metal:562-640), down + weighted combine (kernels.metal:1456-1542)
 * and the next layer's input RMSNorm (runtime.m:2893-2900) -- three
 * host/device crossings per layer.  Here the layer pack is resident in HBM
 * and the step is one launch of 256 blocks x 4 wavefronts.
 *
 * Blocks form 8 groups of 32 (group g = block % 8, j = block / 8); group g
 * streams expert slot g.
 *
 *   N  (stack variant) every block derives x = RMSNorm(h) itself, bit-exact
 *      with math.m:34-65.
 *   R  block b computes router row b in its first wavefront: the 1 MB
 *      router is read once per step (one 4 KB row per block).
 *   T  every block waits for all 256 logits and routes the token (bit-exact
 *      math.m softmax / top-k / renormalise in one wavefront).
 *   P  block j of group g issues all weight loads of slot g at once: gate/up
 *      rows 16j..16j+15 and down rows 64j..64j+63 (~55 KB per block, the
 *      whole 14 MB of expert weights in flight across the grid).
 *   G  gate/up dot products + SwiGLU -> act[g][512].
 *   D  block j waits for act[g], computes y_g = down_g . act[g] for rows
 *      64j..64j+63 -> ypart[g].
 *   C  block j of group 0 waits for the K partials of its rows and combines
 *      out = h_mid + sum_s w_s y_s (+ sigmoid(g) * shared) in slot order.
 *
 * Values cross blocks as 64-bit (epoch, value) words written and read with
 * one device-coherent (sc1) access each; a consumer polls the words it needs
 * until all carry this launch's epoch.  That merges "wait" and "fetch" into
 * one memory round trip: no barrier counter, no same-address atomics, no
 * L2-wide cache maintenance.  The epoch is the launch count, kept per block
 * (each block increments its own word once per launch, so all agree).  A
 * group's barrier-free hand-offs also mean idle groups (K < 8) simply exit.
 * Every wait is bounded.
 */
#include "nmoe_device.h"

#pragma clang fp contract(off)

static __constant__ uint64_t nmoe_fused_exp2_tab[32] = NMOE_EXP2_TAB32;

#define NMOE_FUSED_BLOCKS 256
#define NMOE_FUSED_GROUPS 8
#define NMOE_FUSED_GROUP_BLOCKS (NMOE_FUSED_BLOCKS / NMOE_FUSED_GROUPS) /* 32 */
#define NMOE_FUSED_CHUNK (NMOE_HIDDEN / NMOE_FUSED_GROUP_BLOCKS)         /* 64 output rows per block */
#define NMOE_FUSED_GU_ROWS (NMOE_INTER / NMOE_FUSED_GROUP_BLOCKS)        /* 16 gate/up rows per block */

/* sync words: per-block launch epochs, 64 bytes apart */
#define NMOE_SYNC_EPOCH(b) (64 + 16 * (b))

/* exchange scratch layout (64-bit tagged words) */
/* Words that many blocks poll sit 64 bytes apart (SP words): polling a
 * densely packed word array from every block serialises on its few cache
 * lines (measured: the last of 256 packed words is seen ~2.6 us after it is
 * written by 256 polling blocks, ~1.2 us when the words are 64 B apart). */
#define NMOE_XCH_SP 8
#define NMOE_XCH_LOGITS 0
#define NMOE_XCH_ACT (NMOE_XCH_SP * NMOE_EXPERTS)
#define NMOE_XCH_YPART (NMOE_XCH_ACT + NMOE_XCH_SP * NMOE_FUSED_GROUPS * NMOE_INTER)
#define NMOE_XCH_WORDS (NMOE_XCH_YPART + NMOE_FUSED_GROUPS * NMOE_HIDDEN)

/* x sources: XF32 / XBF16 = activations given; XNORM = x is RMSNorm(h). */
#define NMOE_XF32 0
#define NMOE_XBF16 1
#define NMOE_XNORM 2

struct nmoe_fused_args {
    const uint8_t *pack;
    const uint16_t *router_w; /* bf16 [256][2048] (routing) */
    const void *x;            /* [2048]: fp32 x, bf16 x, or fp32 h (XNORM) */
    float eps;                /* XNORM */
    int k;
    const uint32_t *idx_in; /* [8] (routing given) */
    const float *w_in;
    const float *h_mid; /* residual in */
    const float *shared_out;
    const float *shared_gate_raw;
    float *out; /* residual out (may alias h_mid unless XNORM) */
    uint32_t *idx_out;
    float *w_out;
    float *logits_out;
    uint64_t *xch;
    uint32_t *sync;
};

/* Polls n tagged words until all carry `epoch` (bounded); returns the
 * values.  Each lane polls its own words. */
template <int N>
__device__ __forceinline__ void nmoe_poll(const uint64_t *const p[N], uint32_t epoch, float v[N], uint32_t *status) {
    /* a word, once seen with this epoch, is not loaded again: after the
     * first round only the stragglers' words are re-polled, which keeps the
     * polling traffic off the memory channels the late writers need */
    uint32_t need = (1u << N) - 1u, spins = 0;
    for (;;) {
        uint64_t w[N];
#pragma unroll
        for (int i = 0; i < N; i++) /* all loads of a round in flight together */
            if (need & (1u << i)) w[i] = nmoe_ld_tagged(p[i]);
#pragma unroll
        for (int i = 0; i < N; i++)
            if ((need & (1u << i)) && nmoe_tag_is(w[i], epoch)) {
                v[i] = nmoe_tag_val(w[i]);
                need &= ~(1u << i);
            }
        if (need == 0) return;
        __builtin_amdgcn_s_sleep(1);
        if (++spins > NMOE_SPIN_LIMIT) {
            __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
    }
}

/* The lane's n activations at columns c0.. (fp32, bf16, or normalised h).
 * Normalised: math.m:63 computes (input / rms) * 1.0f.  With rinv the double
 * reciprocal of rms, (float)(h * rinv) is that correctly rounded quotient:
 * its error before the final rounding is below 2^-51 relative, while a
 * quotient of two floats never lies within 2^-49 of a float rounding
 * midpoint (nor exactly on one). */
template <int XMODE>
__device__ __forceinline__ void nmoe_x_cols(const void *x, int c0, int n, double rinv, float *out) {
    if (XMODE == NMOE_XBF16) {
        nmoe_load_cols<uint16_t>((const uint16_t *)x, c0, n, out);
    } else {
        nmoe_load_cols<float>((const float *)x, c0, n, out);
        if (XMODE == NMOE_XNORM)
            for (int i = 0; i < n; i++) out[i] = (float)((double)out[i] * rinv);
    }
}

/* LDS slot of act element e.  Lane dl of a down row reads float4 chunks
 * dl*N .. dl*N+N-1 (N = CPL/4); chunk c of lane dl is stored at position
 * (c + dl + dl/8) mod N of its lane's span, so the lanes of one LDS pass
 * (8 or 16 consecutive dl, one chunk each) hit distinct banks. */
template <int N>
__device__ __forceinline__ int nmoe_act_slot(int e) {
    const int f = e >> 2, dl = f / N, c = f % N;
    return 4 * (dl * N + ((c + dl + (dl >> 3)) & (N - 1))) + (e & 3);
}

template <int BITS, bool ROUTE, int XMODE>
__global__ void __launch_bounds__(256) nmoe_fused_decode_kernel(nmoe_fused_args a) {
    using Q = nmoe_q<BITS>;
    using L = nmoe_layout<BITS>;
    constexpr int RPS = NMOE_WAVE / Q::LPR_G;   /* gate/up rows per wave step: 1 (q4) / 2 (q2) */
    constexpr int GSTEPS = 4 / RPS;             /* 4 gate/up rows per wavefront */
    constexpr int RPW_D = NMOE_WAVE / Q::LPR_D; /* down rows per wave step: 4 (q4) / 8 (q2) */
    constexpr int DSTEPS = 16 / RPW_D;          /* 16 down rows per wavefront */
    __shared__ uint64_t s_tab[32];
    __shared__ float s_lg[NMOE_EXPERTS];
    __shared__ float s_scratch[NMOE_EXPERTS];
    __shared__ float s_act[NMOE_INTER];
    __shared__ float s_y[NMOE_FUSED_CHUNK];
    __shared__ uint32_t s_idx[NMOE_MAX_K];
    __shared__ float s_w[NMOE_MAX_K];
    __shared__ double s_dd[8];
    __shared__ float s_f[1];
    __shared__ uint32_t s_epoch;
    __shared__ float s_h[XMODE == NMOE_XNORM ? NMOE_HIDDEN : 1];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = blockIdx.x % NMOE_FUSED_GROUPS, j = blockIdx.x / NMOE_FUSED_GROUPS;
    const int k = a.k;
    uint32_t *status = a.sync + NMOE_SYNC_STATUS;
    uint64_t *xlg = a.xch + NMOE_XCH_LOGITS;
    uint64_t *xact = a.xch + NMOE_XCH_ACT + NMOE_XCH_SP * g * NMOE_INTER;
    uint64_t *ypart = a.xch + NMOE_XCH_YPART;

    /* Independent loads go out first and unconditionally (loads retire in
     * order, so a later wait on one of them must not cover the big ones):
     * the launch epoch, the exp2 table entry, the residual row this thread
     * may combine; then this block's router row and its x columns. */
    uint32_t *ep = a.sync + NMOE_SYNC_EPOCH(blockIdx.x);
    const uint32_t ep_old = nmoe_ld_u32_dev(ep);
    const uint64_t tab_v = nmoe_fused_exp2_tab[tid & 31];
    const int crow = j * NMOE_FUSED_CHUNK + (tid & (NMOE_FUSED_CHUNK - 1));
    const float hm = a.h_mid[crow];
    const float sh = a.shared_out != NULL ? a.shared_out[crow] : 0.0f;
    uint4 wv[4];
    float xs_r[32];
    if (ROUTE && wave == 0) {
        const uint4 *row = (const uint4 *)(a.router_w + (size_t)blockIdx.x * NMOE_HIDDEN);
#pragma unroll
        for (int q = 0; q < 4; q++) wv[q] = row[lane + 64 * q];
        if (XMODE != NMOE_XNORM)
#pragma unroll
            for (int q = 0; q < 4; q++) nmoe_x_cols<XMODE>(a.x, (lane + 64 * q) * 8, 8, 1.0, xs_r + 8 * q);
    }
    if (tid < 32) s_tab[tid] = tab_v;
    if (tid == 0) {
        __hip_atomic_store(ep, ep_old + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_epoch = ep_old + 1u;
    }
    double rinv = 1.0;
    if (XMODE == NMOE_XNORM) rinv = 1.0 / (double)nmoe_block_rms_exact((const float *)a.x, a.eps, s_h, s_dd, s_f);
    __syncthreads();
    const uint32_t epoch = s_epoch;

    if (ROUTE) {
        /* ---- R + T in the first wavefront: router row blockIdx.x, then wait
         * for all 256 logits and route */
        if (wave == 0) {
            if (XMODE == NMOE_XNORM)
#pragma unroll
                for (int q = 0; q < 4; q++) nmoe_x_cols<XMODE>(a.x, (lane + 64 * q) * 8, 8, rinv, xs_r + 8 * q);
            float logit = nmoe_router_row_bf16(wv, xs_r);
            if (lane == 0) nmoe_st_tagged(xlg + NMOE_XCH_SP * blockIdx.x, epoch, logit);
            const uint64_t *pl[4] = {xlg + NMOE_XCH_SP * lane, xlg + NMOE_XCH_SP * (lane + 64),
                                     xlg + NMOE_XCH_SP * (lane + 128), xlg + NMOE_XCH_SP * (lane + 192)};
            float lv[4];
            nmoe_poll<4>(pl, epoch, lv, status);
#pragma unroll
            for (int q = 0; q < 4; q++) s_lg[lane + 64 * q] = lv[q];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            uint32_t si[NMOE_MAX_K];
            float sw[NMOE_MAX_K];
            nmoe_wave_route(s_lg, NMOE_EXPERTS, k, s_scratch, s_tab, si, sw, NULL);
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
                if (blockIdx.x == 0 && a.idx_out != NULL) a.idx_out[lane] = vi;
                if (blockIdx.x == 0 && a.w_out != NULL) a.w_out[lane] = vw;
            }
            if (blockIdx.x == 0 && a.logits_out != NULL)
#pragma unroll
                for (int q = 0; q < 4; q++) a.logits_out[lane + 64 * q] = s_lg[lane + 64 * q];
        }
    } else {
        if (tid < NMOE_MAX_K) {
            uint32_t e = tid < k ? a.idx_in[tid] : 0u;
            float wv = tid < k ? a.w_in[tid] : 0.0f;
            /* an index outside the layer is an invalid slot: weight 0, as
             * for a failed expert read (runtime.m:2977-2981) */
            s_w[tid] = e < NMOE_EXPERTS ? wv : 0.0f;
            s_idx[tid] = e < NMOE_EXPERTS ? e : 0u;
        }
    }
    __syncthreads();
    if (g >= k) return; /* group g streams expert slot g */
    const uint8_t *ex = a.pack + (size_t)s_idx[g] * L::expert_size;

    /* ---- P: issue all weight loads of this wavefront */
    const int gsub = lane / Q::LPR_G, gl = lane % Q::LPR_G, ggrp = gl * Q::CPL / NMOE_GROUP;
    const int dsub = lane / Q::LPR_D, dl = lane % Q::LPR_D, dgrp = dl * Q::CPL / NMOE_GROUP;
    const int grow0 = j * NMOE_FUSED_GU_ROWS + 4 * wave + gsub;
    const int drow0 = j * NMOE_FUSED_CHUNK + 16 * wave + dsub;
    /* x first: loads retire in order, so G can start while down rows stream */
    float xs[Q::CPL];
    nmoe_x_cols<XMODE>(a.x, gl * Q::CPL, Q::CPL, rinv, xs);
    uint4 gwv[GSTEPS], uwv[GSTEPS], dwv[DSTEPS];
    uint32_t gsb[GSTEPS], usb[GSTEPS], dsb[DSTEPS]; /* scale | bias << 16 */
#pragma unroll
    for (int i = 0; i < GSTEPS; i++) {
        int row = grow0 + i * RPS;
        gwv[i] = ((const uint4 *)(ex + L::gate_w))[(size_t)row * (Q::WPR_G / 4) + gl];
        uwv[i] = ((const uint4 *)(ex + L::up_w))[(size_t)row * (Q::WPR_G / 4) + gl];
        const uint16_t *gs = (const uint16_t *)(ex + L::gate_s) + row * Q::GPR_G + ggrp;
        const uint16_t *us = (const uint16_t *)(ex + L::up_s) + row * Q::GPR_G + ggrp;
        gsb[i] = (uint32_t)gs[0] | ((uint32_t)gs[NMOE_INTER * Q::GPR_G] << 16);
        usb[i] = (uint32_t)us[0] | ((uint32_t)us[NMOE_INTER * Q::GPR_G] << 16);
    }
#pragma unroll
    for (int i = 0; i < DSTEPS; i++) {
        int row = drow0 + i * RPW_D;
        dwv[i] = ((const uint4 *)(ex + L::down_w))[(size_t)row * (Q::WPR_D / 4) + dl];
        const uint16_t *ds = (const uint16_t *)(ex + L::down_s) + row * Q::GPR_D + dgrp;
        dsb[i] = (uint32_t)ds[0] | ((uint32_t)ds[NMOE_HIDDEN * Q::GPR_D] << 16);
    }
    /* keep every weight load above in one burst: no compute hoisted into it */
    __builtin_amdgcn_sched_barrier(0);
    /* ---- G: gate/up + SwiGLU -> act[g] */
    {
        float xsum = 0.0f;
#pragma unroll
        for (int c = 0; c < Q::CPL; c++) xsum += xs[c];
#pragma unroll
        for (int i = 0; i < GSTEPS; i++) {
            float gv = __builtin_fmaf(nmoe_bf16f(gsb[i] & 0xffffu), nmoe_dot16<BITS>(gwv[i], xs),
                                      nmoe_bf16f(gsb[i] >> 16) * xsum);
            float uv = __builtin_fmaf(nmoe_bf16f(usb[i] & 0xffffu), nmoe_dot16<BITS>(uwv[i], xs),
                                      nmoe_bf16f(usb[i] >> 16) * xsum);
            gv = nmoe_lanes_sum<Q::LPR_G>(gv);
            uv = nmoe_lanes_sum<Q::LPR_G>(uv);
            if (gl == 0) nmoe_st_tagged(xact + NMOE_XCH_SP * (grow0 + i * RPS), epoch, nmoe_silu_dev(gv) * uv);
        }
    }

    /* ---- D: wait for act[g], then y_g for rows 64j..64j+63 */
    {
        const uint64_t *pa[2] = {xact + NMOE_XCH_SP * tid, xact + NMOE_XCH_SP * (tid + 256)};
        float av[2];
        nmoe_poll<2>(pa, epoch, av, status);
        s_act[nmoe_act_slot<Q::CPL / 4>(tid)] = av[0];
        s_act[nmoe_act_slot<Q::CPL / 4>(tid + 256)] = av[1];
    }
    __syncthreads();
    /* this lane's CPL act columns, read once (conflict-free: swizzled) */
    float as[Q::CPL];
#pragma unroll
    for (int c = 0; c < Q::CPL / 4; c++) {
        float4 t = ((const float4 *)s_act)[nmoe_act_slot<Q::CPL / 4>(4 * (dl * (Q::CPL / 4) + c)) / 4];
        as[4 * c] = t.x;
        as[4 * c + 1] = t.y;
        as[4 * c + 2] = t.z;
        as[4 * c + 3] = t.w;
    }
    float asum = 0.0f;
#pragma unroll
    for (int c = 0; c < Q::CPL; c++) asum += as[c];
#pragma unroll
    for (int i = 0; i < DSTEPS; i++) {
        float y = __builtin_fmaf(nmoe_bf16f(dsb[i] & 0xffffu), nmoe_dot16<BITS>(dwv[i], as),
                                 nmoe_bf16f(dsb[i] >> 16) * asum);
        y = nmoe_dpp_group_sum<Q::LPR_D>(y);
        if (dl == 0) s_y[16 * wave + dsub + i * RPW_D] = y;
    }
    __syncthreads();
    const int row = j * NMOE_FUSED_CHUNK + tid;
    if (g != 0) {
        if (tid < NMOE_FUSED_CHUNK) nmoe_st_tagged(ypart + g * NMOE_HIDDEN + row, epoch, s_y[tid]);
        return;
    }

    /* ---- C: block j of group 0 combines rows 64j..64j+63 over the K slots */
    if (tid < NMOE_FUSED_CHUNK) {
        /* one polling round loads all K-1 partials at once */
        float ys[NMOE_MAX_K];
        ys[0] = s_y[tid];
        uint32_t need = 0, spins = 0;
#pragma unroll
        for (int s = 1; s < NMOE_MAX_K; s++) {
            ys[s] = 0.0f;
            if (s < k) need |= 1u << s;
        }
        for (;;) {
            uint64_t w[NMOE_MAX_K];
#pragma unroll
            for (int s = 1; s < NMOE_MAX_K; s++)
                if (need & (1u << s)) w[s] = nmoe_ld_tagged(ypart + s * NMOE_HIDDEN + row);
#pragma unroll
            for (int s = 1; s < NMOE_MAX_K; s++)
                if ((need & (1u << s)) && nmoe_tag_is(w[s], epoch)) {
                    ys[s] = nmoe_tag_val(w[s]);
                    need &= ~(1u << s);
                }
            if (need == 0) break;
            __builtin_amdgcn_s_sleep(1);
            if (++spins > NMOE_SPIN_LIMIT) {
                __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
        float moe = 0.0f;
#pragma unroll
        for (int s = 0; s < NMOE_MAX_K; s++)
            if (s < k) moe += s_w[s] * ys[s];
        float r = hm + moe;
        if (a.shared_out != NULL) r = r + nmoe_sigmoid_dev(a.shared_gate_raw[0]) * sh;
        a.out[row] = r;
    }
}

/* ----------------------------------------------------------- launching */

template <int BITS, bool ROUTE, int XMODE>
static hipError_t nmoe_fused_launch(const nmoe_fused_args &args, hipStream_t s) {
    hipLaunchKernelGGL((nmoe_fused_decode_kernel<BITS, ROUTE, XMODE>), dim3(NMOE_FUSED_BLOCKS), dim3(256), 0, s, args);
    return hipGetLastError();
}

template <int BITS, bool ROUTE, int XMODE>
static int nmoe_fused_fits(int num_cus) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, nmoe_fused_decode_kernel<BITS, ROUTE, XMODE>, 256, 0) !=
        hipSuccess)
        return 0;
    return per_cu >= 1 && per_cu * num_cus >= NMOE_FUSED_BLOCKS;
}

/* The fused path needs all 256 blocks resident at once (its group barriers
 * wait on each other); decided here from the occupancy of every variant. */
extern "C" int nmoe_decode_init(nmoe_hip_ctx *ctx) {
    int n = ctx->num_cus;
    int ok = nmoe_fused_fits<4, true, NMOE_XBF16>(n) && nmoe_fused_fits<4, true, NMOE_XF32>(n) &&
             nmoe_fused_fits<4, true, NMOE_XNORM>(n) && nmoe_fused_fits<2, true, NMOE_XBF16>(n) &&
             nmoe_fused_fits<2, true, NMOE_XF32>(n) && nmoe_fused_fits<2, true, NMOE_XNORM>(n) &&
             nmoe_fused_fits<4, false, NMOE_XBF16>(n) && nmoe_fused_fits<4, false, NMOE_XF32>(n) &&
             nmoe_fused_fits<2, false, NMOE_XBF16>(n) && nmoe_fused_fits<2, false, NMOE_XF32>(n);
    ctx->fused_blocks = ok ? NMOE_FUSED_BLOCKS : 0;
    ctx->xch_bytes = (size_t)NMOE_XCH_WORDS * sizeof(uint64_t);
    if (hipMalloc((void **)&ctx->xch, ctx->xch_bytes) != hipSuccess) return NMOE_HIP_ENOMEM;
    if (hipMemset(ctx->xch, 0, ctx->xch_bytes) != hipSuccess) return NMOE_HIP_EHIP;
    return NMOE_HIP_OK;
}

/* One token.  route != 0: routing computed from router_w; else given by
 * idx_in / w_in.  xmode: NMOE_XF32 / NMOE_XBF16 / NMOE_XNORM. */
extern "C" int nmoe_fused_decode(nmoe_hip_ctx *ctx, int bits, int route, const void *x, int xmode, float eps, int k,
                                 const uint16_t *router_w, const uint32_t *idx_in, const float *w_in,
                                 const float *h_mid, const float *shared_out, const float *shared_gate_raw, float *out,
                                 uint32_t *idx_out, float *w_out, float *logits_out, const uint8_t *pack,
                                 hipStream_t s) {
    nmoe_fused_args a;
    a.pack = pack;
    a.router_w = router_w;
    a.x = x;
    a.eps = eps;
    a.k = k;
    a.idx_in = idx_in;
    a.w_in = w_in;
    a.h_mid = h_mid;
    a.shared_out = shared_out;
    a.shared_gate_raw = shared_gate_raw;
    a.out = out;
    a.idx_out = idx_out;
    a.w_out = w_out;
    a.logits_out = logits_out;
    a.xch = ctx->xch;
    a.sync = ctx->sync;
    hipError_t e = hipErrorInvalidValue;
    if (bits == 4) {
        if (route) {
            if (xmode == NMOE_XBF16) e = nmoe_fused_launch<4, true, NMOE_XBF16>(a, s);
            else if (xmode == NMOE_XF32) e = nmoe_fused_launch<4, true, NMOE_XF32>(a, s);
            else e = nmoe_fused_launch<4, true, NMOE_XNORM>(a, s);
        } else {
            e = xmode == NMOE_XBF16 ? nmoe_fused_launch<4, false, NMOE_XBF16>(a, s)
                                    : nmoe_fused_launch<4, false, NMOE_XF32>(a, s);
        }
    } else {
        if (route) {
            if (xmode == NMOE_XBF16) e = nmoe_fused_launch<2, true, NMOE_XBF16>(a, s);
            else if (xmode == NMOE_XF32) e = nmoe_fused_launch<2, true, NMOE_XF32>(a, s);
            else e = nmoe_fused_launch<2, true, NMOE_XNORM>(a, s);
        } else {
            e = xmode == NMOE_XBF16 ? nmoe_fused_launch<2, false, NMOE_XBF16>(a, s)
                                    : nmoe_fused_launch<2, false, NMOE_XF32>(a, s);
        }
    }
    if (e != hipSuccess) return nmoe_hip_check(ctx, e, "fused decode launch");
    return NMOE_HIP_OK;
}
