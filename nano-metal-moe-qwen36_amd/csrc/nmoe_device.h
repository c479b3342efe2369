/*
 * nmoe_device.h -- device building blocks shared by the decode kernels:
 * DPP reductions, q4/q2 row dot products, the router row, bit-exact routing
 * of one token by one wavefront, the tagged words the persistent kernels
 * exchange and the exact RMSNorm.  Header-only (every .hip file is its own
 * code object).
 */
#ifndef NMOE_DEVICE_H
#define NMOE_DEVICE_H

#include "nmoe_hip_internal.h"

/* ---------------------------------------------------------------- DPP */

/* DPP controls (gfx9): quad_perm [1,0,3,2] = lane^1, [2,3,0,1] = lane^2,
 * row_half_mirror = 7-i within 8 lanes, row_mirror = 15-i within 16 lanes. */
#define NMOE_DPP_XOR1 0xB1
#define NMOE_DPP_XOR2 0x4E
#define NMOE_DPP_HALF_MIRROR 0x141
#define NMOE_DPP_MIRROR 0x140

template <int CTRL>
__device__ __forceinline__ uint32_t nmoe_dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ float nmoe_dpp_f(float v) {
    return __uint_as_float(nmoe_dpp_u<CTRL>(__float_as_uint(v)));
}

__device__ __forceinline__ float nmoe_readlane_f(float v, int lane) {
    return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), lane));
}

/* Sum over aligned groups of W lanes (W = 4, 8, 16), every lane of a group
 * receiving its group's sum.  The combination is the balanced pairwise tree
 * over the group's lanes in order: (l0+l1)+(l2+l3), then quads, then octets. */
template <int W>
__device__ __forceinline__ float nmoe_dpp_group_sum(float v) {
    v = v + nmoe_dpp_f<NMOE_DPP_XOR1>(v);
    v = v + nmoe_dpp_f<NMOE_DPP_XOR2>(v);
    if (W >= 8) v = v + nmoe_dpp_f<NMOE_DPP_HALF_MIRROR>(v);
    if (W >= 16) v = v + nmoe_dpp_f<NMOE_DPP_MIRROR>(v);
    return v;
}

/* Wave sum as the balanced pairwise tree over lanes 0..63 in order
 * (rows of 16 by DPP, then (r0 + r1) + (r2 + r3)); uniform result. */
__device__ __forceinline__ float nmoe_wave_sum_tree(float v) {
    v = nmoe_dpp_group_sum<16>(v);
    float r0 = nmoe_readlane_f(v, 0), r1 = nmoe_readlane_f(v, 16);
    float r2 = nmoe_readlane_f(v, 32), r3 = nmoe_readlane_f(v, 48);
    return (r0 + r1) + (r2 + r3);
}

/* Sum over each half wave (lanes 0-31, 32-63), same tree shape. */
__device__ __forceinline__ float nmoe_half_sum_tree(float v) {
    v = nmoe_dpp_group_sum<16>(v);
    float r0 = nmoe_readlane_f(v, 0), r1 = nmoe_readlane_f(v, 16);
    float r2 = nmoe_readlane_f(v, 32), r3 = nmoe_readlane_f(v, 48);
    return (threadIdx.x & 32) ? (r2 + r3) : (r0 + r1);
}

/* Group sum for W in {8, 16, 32, 64} lanes (every lane of a group gets it). */
template <int W>
__device__ __forceinline__ float nmoe_lanes_sum(float v) {
    if (W == 64) return nmoe_wave_sum_tree(v);
    if (W == 32) return nmoe_half_sum_tree(v);
    return nmoe_dpp_group_sum<W>(v);
}

__device__ __forceinline__ float nmoe_wave_max_f(float v) {
    v = fmaxf(v, nmoe_dpp_f<NMOE_DPP_XOR1>(v));
    v = fmaxf(v, nmoe_dpp_f<NMOE_DPP_XOR2>(v));
    v = fmaxf(v, nmoe_dpp_f<NMOE_DPP_HALF_MIRROR>(v));
    v = fmaxf(v, nmoe_dpp_f<NMOE_DPP_MIRROR>(v));
    return fmaxf(fmaxf(nmoe_readlane_f(v, 0), nmoe_readlane_f(v, 16)),
                 fmaxf(nmoe_readlane_f(v, 32), nmoe_readlane_f(v, 48)));
}

__device__ __forceinline__ float nmoe_wave_min_f(float v) {
    v = fminf(v, nmoe_dpp_f<NMOE_DPP_XOR1>(v));
    v = fminf(v, nmoe_dpp_f<NMOE_DPP_XOR2>(v));
    v = fminf(v, nmoe_dpp_f<NMOE_DPP_HALF_MIRROR>(v));
    v = fminf(v, nmoe_dpp_f<NMOE_DPP_MIRROR>(v));
    return fminf(fminf(nmoe_readlane_f(v, 0), nmoe_readlane_f(v, 16)),
                 fminf(nmoe_readlane_f(v, 32), nmoe_readlane_f(v, 48)));
}

__device__ __forceinline__ uint32_t nmoe_wave_max_u32(uint32_t v) {
    v = max(v, nmoe_dpp_u<NMOE_DPP_XOR1>(v));
    v = max(v, nmoe_dpp_u<NMOE_DPP_XOR2>(v));
    v = max(v, nmoe_dpp_u<NMOE_DPP_HALF_MIRROR>(v));
    v = max(v, nmoe_dpp_u<NMOE_DPP_MIRROR>(v));
    uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return max(max(r0, r1), max(r2, r3));
}

/* Inclusive prefix sum over the wavefront's 64 lanes by DPP: row_shr 1, 2,
 * 4, 8 scan each row of 16 lanes (a lane with no source adds 0), then
 * row_bcast:15 adds each even row's total to the row after it and
 * row_bcast:31 the first two rows' total to the last two (gfx9 controls). */
__device__ __forceinline__ uint32_t nmoe_wave_incl_scan_u32(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false); /* row_shr:1 */
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false); /* row_shr:2 */
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false); /* row_shr:4 */
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false); /* row_shr:8 */
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false); /* row_bcast:15, rows 1, 3 */
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false); /* row_bcast:31, rows 2, 3 */
    return v;
}

template <int CTRL>
__device__ __forceinline__ uint64_t nmoe_dpp_u64(uint64_t v) {
    return ((uint64_t)nmoe_dpp_u<CTRL>((uint32_t)(v >> 32)) << 32) | nmoe_dpp_u<CTRL>((uint32_t)v);
}

__device__ __forceinline__ uint64_t nmoe_readlane_u64(uint64_t v, int lane) {
    uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
    uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t nmoe_wave_sum_u64(uint64_t v) {
    v += nmoe_dpp_u64<NMOE_DPP_XOR1>(v);
    v += nmoe_dpp_u64<NMOE_DPP_XOR2>(v);
    v += nmoe_dpp_u64<NMOE_DPP_HALF_MIRROR>(v);
    v += nmoe_dpp_u64<NMOE_DPP_MIRROR>(v);
    return (nmoe_readlane_u64(v, 0) + nmoe_readlane_u64(v, 16)) + (nmoe_readlane_u64(v, 32) + nmoe_readlane_u64(v, 48));
}

/* ------------------------------------------------------- q4 / q2 rows */

template <int BITS>
struct nmoe_q {
    static constexpr int VPW = 32 / BITS;            /* values per word */
    static constexpr int CPL = 4 * VPW;              /* columns per lane (one 16-byte load) */
    static constexpr int LPR_G = NMOE_HIDDEN / CPL;  /* lanes per gate/up row: 64 / 32 */
    static constexpr int LPR_D = NMOE_INTER / CPL;   /* lanes per down row: 16 / 8 */
    static constexpr int WPR_G = NMOE_HIDDEN / VPW;  /* words per gate/up row */
    static constexpr int WPR_D = NMOE_INTER / VPW;   /* words per down row */
    static constexpr int GPR_G = NMOE_HIDDEN / NMOE_GROUP;
    static constexpr int GPR_D = NMOE_INTER / NMOE_GROUP;
};

/* sum_j q_j * x_j over the 16 bytes `q` (column order of the pack). */
template <int BITS>
__device__ __forceinline__ float nmoe_dot16(uint4 q, const float *xs);

template <>
__device__ __forceinline__ float nmoe_dot16<4>(uint4 q, const float *xs) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t lo = w[i] & 0x0F0F0F0Fu;
        uint32_t hi = (w[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            a0 = __builtin_fmaf((float)((lo >> (8 * j)) & 0xFFu), xs[8 * i + 2 * j], a0);
            a1 = __builtin_fmaf((float)((hi >> (8 * j)) & 0xFFu), xs[8 * i + 2 * j + 1], a1);
        }
    }
    return a0 + a1;
}

/* The 32 q4 codes of `q` as floats, in the element order nmoe_dot16<4>
 * uses, and the same dot product over such floats: nmoe_dot_f4(w, xs) with
 * nmoe_unpack_q4(q, w) equals nmoe_dot16<4>(q, xs) bit for bit. */
__device__ __forceinline__ void nmoe_unpack_q4(uint4 q, float *w) {
    const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t lo = u[i] & 0x0F0F0F0Fu, hi = (u[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            w[8 * i + 2 * j] = (float)((lo >> (8 * j)) & 0xFFu);
            w[8 * i + 2 * j + 1] = (float)((hi >> (8 * j)) & 0xFFu);
        }
    }
}
__device__ __forceinline__ float nmoe_dot_f4(const float *w, const float *xs) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            a0 = __builtin_fmaf(w[8 * i + 2 * j], xs[8 * i + 2 * j], a0);
            a1 = __builtin_fmaf(w[8 * i + 2 * j + 1], xs[8 * i + 2 * j + 1], a1);
        }
    }
    return a0 + a1;
}

template <>
__device__ __forceinline__ float nmoe_dot16<2>(uint4 q, const float *xs) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int m = 0; m < 4; m++) {
            uint32_t p = (w[i] >> (2 * m)) & 0x03030303u;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float v = (float)((p >> (8 * j)) & 0xFFu);
                if (m & 1)
                    a1 = __builtin_fmaf(v, xs[16 * i + 4 * j + m], a1);
                else
                    a0 = __builtin_fmaf(v, xs[16 * i + 4 * j + m], a0);
            }
        }
    }
    return a0 + a1;
}

__device__ __forceinline__ float nmoe_sigmoid_dev(float x) {
    /* math.m:21-28 form: exp of a non-positive argument only */
    if (x >= 0.0f) {
        float z = __expf(-x);
        return 1.0f / (1.0f + z);
    }
    float z = __expf(x);
    return z / (1.0f + z);
}

__device__ __forceinline__ float nmoe_silu_dev(float x) { return x * nmoe_sigmoid_dev(x); }

__device__ __forceinline__ void nmoe_unpack_bf16x8(uint4 v, float out[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        out[2 * i] = __uint_as_float(w[i] << 16);
        out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

/* n consecutive activations starting at column c0, as fp32. */
template <typename XT>
__device__ __forceinline__ void nmoe_load_cols(const XT *x, int c0, int n, float *out);

template <>
__device__ __forceinline__ void nmoe_load_cols<float>(const float *x, int c0, int n, float *out) {
    for (int c = 0; c < n; c += 4) {
        float4 v = *(const float4 *)(x + c0 + c);
        out[c] = v.x;
        out[c + 1] = v.y;
        out[c + 2] = v.z;
        out[c + 3] = v.w;
    }
}

template <>
__device__ __forceinline__ void nmoe_load_cols<uint16_t>(const uint16_t *x, int c0, int n, float *out) {
    for (int c = 0; c < n; c += 8) nmoe_unpack_bf16x8(*(const uint4 *)(x + c0 + c), out + c);
}

/* ------------------------------------------------------------ router */

/* Router logit of one bf16 row against x, by one wavefront: lane L owns the
 * 16-byte chunks L, L+64, L+128, L+192 (8 columns each) and accumulates them
 * in order with fma; the lane partials are combined by the balanced pairwise
 * tree (nmoe_wave_sum_tree).  xs holds the lane's 32 columns of x in the
 * same chunk order.  Uniform result. */
__device__ __forceinline__ float nmoe_router_row_bf16(const uint4 wv[4], const float xs[32]) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        float wf[8];
        nmoe_unpack_bf16x8(wv[j], wf);
#pragma unroll
        for (int i = 0; i < 8; i++) acc = __builtin_fmaf(wf[i], xs[8 * j + i], acc);
    }
    return nmoe_wave_sum_tree(acc);
}

/* One element of the q4 router's dot product in the reference's per-element
 * form (metal/kernels.metal:500-508): acc + fma(q, scale*x, bias*x), both
 * products rounded to fp32 before the fma and the fma rounded before the add. */
__device__ __forceinline__ float nmoe_router_q4_term(float acc, uint32_t q, float s, float b, float x) {
#pragma clang fp contract(off)
    const float sx = s * x, bx = b * x;
    return acc + __builtin_fmaf((float)q, sx, bx);
}

/* Router logit of one q4 row (the model's router, metal/kernels.metal:472-513)
 * by one wavefront: lane L owns the words L, L+64, L+128, L+192 (columns
 * 8 word .. +7) and their groups' raw bf16 scale and bias, and accumulates
 * its columns in order with nmoe_router_q4_term; the lane partials are
 * combined by the pairwise tree.  The multi-launch q4 router kernel uses the
 * same order, so both paths give the same logits. */
__device__ __forceinline__ float nmoe_router_row_q4(const uint32_t wq[4], const uint16_t s[4], const uint16_t b[4],
                                                    const float xs[32]) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float sf = nmoe_bf16f(s[j]), bf = nmoe_bf16f(b[j]);
#pragma unroll
        for (int i = 0; i < 8; i++) acc = nmoe_router_q4_term(acc, (wq[j] >> (4 * i)) & 0xFu, sf, bf, xs[8 * j + i]);
    }
    return nmoe_wave_sum_tree(acc);
}

/* ------------------------------------------------------------ routing */

/* Softmax probabilities of one token (math.m:67-93 bit for bit), entry
 * lane + 64 j in p[j] (0 for entries >= num_experts).  l: the lane's four
 * logits; scratch: 256 floats of LDS for the sequential exact-sum path;
 * tab: the exp2 table. */
__device__ __forceinline__ void nmoe_wave_softmax(const float l_in[4], int num_experts, float *scratch,
                                                  const uint64_t *tab, float p[4]) {
    const int lane = threadIdx.x & 63;
    float l[4];
#pragma unroll
    for (int j = 0; j < 4; j++) l[j] = lane + 64 * j < num_experts ? l_in[j] : -__builtin_inff();
    /* the maximum (order-free for finite logits; zeros of either sign give
     * the same exp arguments' results) */
    float m = nmoe_wave_max_f(fmaxf(fmaxf(l[0], l[1]), fmaxf(l[2], l[3])));

    float e[4];
    uint64_t fx = 0;
    int ok = 1;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        int i = lane + 64 * j;
        e[j] = i < num_experts ? nmoe_expf_glibc(l[j] - m, tab) : 0.0f;
        uint64_t f = 0;
        ok &= nmoe_softmax_term_fixed(e[j], &f);
        fx += f;
    }
    float total;
    if (__ballot(!ok) == 0) {
        /* every term is a multiple of 2^-55 and the sum stays below 2^63:
         * math.m's long double running sum was exact and equals this sum */
        total = nmoe_u64_scaled_to_f32_rne(nmoe_wave_sum_u64(fx));
    } else {
        /* replay the long double running sum in index order in lane 0 */
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int i = lane + 64 * j;
            if (i < num_experts) scratch[i] = e[j];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        float t = 0.0f;
        if (lane == 0) {
            nmoe_x87 acc = nmoe_x87_zero();
            for (int i = 0; i < num_experts; i++) acc = nmoe_x87_add(acc, nmoe_x87_from_float(scratch[i]));
            t = nmoe_x87_to_float(acc);
        }
        total = nmoe_readlane_f(t, 0);
        __builtin_amdgcn_wave_barrier();
    }
    float inv = total == 0.0f ? 0.0f : 1.0f / total;
#pragma unroll
    for (int j = 0; j < 4; j++)
        p[j] = lane + 64 * j < num_experts ? (total == 0.0f ? 1.0f / (float)num_experts : e[j] * inv) : 0.0f;
}

/* Order-preserving key of a float: a > b <=> key(a) > key(b) (-0 < +0);
 * never 0, so 0 can mark an absent or taken entry. */
__device__ __forceinline__ uint32_t nmoe_fkey(float f) {
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* The n (<= NMOE_MAX_K) largest of the wavefront's 256 keys (key[j] of
 * lane L belongs to entry L + 64 j; 0 = absent), in decreasing key order,
 * ties to the lower entry -- the selection rule of math.m:95-132.  Per
 * round: the wave maximum, then the lowest entry holding it from the
 * compare masks (lowest j with a hit, then its lowest lane); keys all below
 * 2^30 take the shorter rounds of the first branch.  Consumes key;
 * uniform results, slots >= n zero; hook(s, entry) runs after round s. */
struct nmoe_no_round_hook {
    __device__ void operator()(int, uint32_t) const {}
};

template <typename Hook = nmoe_no_round_hook>
__device__ __forceinline__ void nmoe_wave_top_keys(uint32_t key[4], int n, uint32_t sel[NMOE_MAX_K],
                                                   uint32_t selkey[NMOE_MAX_K], Hook hook = Hook()) {
    const int lane = threadIdx.x & 63;
    if (__ballot((key[0] | key[1] | key[2] | key[3]) >= (1u << 30)) == 0) {
        /* Every key below 2^30 (probability keys are, unless NaN): the
         * slot j goes into two free low bits as 3 - j, so a lane's keys are
         * distinct and a tie between slots goes to the lower one (the lower
         * entry, as entry = lane + 64 j); kept sorted, a round is one wave
         * maximum of the lanes' first keys and one ballot for the lowest
         * lane holding it.  The same selection as the rounds below. */
        uint32_t kk[4];
#pragma unroll
        for (int j = 0; j < 4; j++) kk[j] = key[j] == 0u ? 0u : (key[j] << 2) | (uint32_t)(3 - j);
        auto ce = [](uint32_t &a, uint32_t &b) {
            const uint32_t hi = max(a, b), lo = min(a, b);
            a = hi;
            b = lo;
        };
        ce(kk[0], kk[1]);
        ce(kk[2], kk[3]);
        ce(kk[0], kk[2]);
        ce(kk[1], kk[3]);
        ce(kk[1], kk[2]);
#pragma unroll
        for (int s = 0; s < NMOE_MAX_K; s++) {
            sel[s] = 0;
            selkey[s] = 0;
            if (s < n) {
                const uint32_t best = nmoe_wave_max_u32(kk[0]);
                const uint64_t m = __ballot(kk[0] == best);
                const uint32_t l0 = (uint32_t)__ffsll((unsigned long long)m) - 1u;
                const uint32_t win = l0 + 64u * (3u - (best & 3u));
                if ((uint32_t)lane == l0) {
                    kk[0] = kk[1];
                    kk[1] = kk[2];
                    kk[2] = kk[3];
                    kk[3] = 0u;
                }
                sel[s] = win;
                selkey[s] = best >> 2;
                hook(s, win);
            }
        }
        return;
    }
#pragma unroll
    for (int s = 0; s < NMOE_MAX_K; s++) {
        sel[s] = 0;
        selkey[s] = 0;
        if (s < n) {
            const uint32_t best = nmoe_wave_max_u32(max(max(key[0], key[1]), max(key[2], key[3])));
            const uint64_t m0 = __ballot(key[0] == best), m1 = __ballot(key[1] == best);
            const uint64_t m2 = __ballot(key[2] == best), m3 = __ballot(key[3] == best);
            /* branch-free: find-first-set of each mask (0 = none) */
            const int f0 = __ffsll((unsigned long long)m0), f1 = __ffsll((unsigned long long)m1);
            const int f2 = __ffsll((unsigned long long)m2), f3 = __ffsll((unsigned long long)m3);
            const uint32_t win = f0 ? f0 - 1 : f1 ? 63 + f1 : f2 ? 127 + f2 : 191 + f3;
            const bool here = (uint32_t)lane == (win & 63u);
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (here && (win >> 6) == (uint32_t)j) key[j] = 0u; /* taken */
            sel[s] = win;
            selkey[s] = best;
            hook(s, win); /* e.g. publish each selection as soon as it is made */
        }
    }
}

/* math.m:134-153: weights = selected probabilities / their sum, summed in
 * slot order (1/n each when the sum is 0). */
__device__ __forceinline__ void nmoe_renormalize(const float sel_v[NMOE_MAX_K], int n, float sel_w[NMOE_MAX_K]) {
    float sum = 0.0f;
#pragma unroll
    for (int s = 0; s < NMOE_MAX_K; s++)
        if (s < n) sum += sel_v[s];
    float rinv = sum == 0.0f ? 1.0f / (float)n : 1.0f / sum;
#pragma unroll
    for (int s = 0; s < NMOE_MAX_K; s++) sel_w[s] = s < n ? (sum == 0.0f ? rinv : sel_v[s] * rinv) : 0.0f;
}

/* Routes one token with a full wavefront (math.m:67-153 bit for bit).
 * lg: the token's logits (any memory); scratch: 256 floats of LDS for the
 * sequential exact-sum path; tab: the exp2 table (LDS or constant memory).
 * On return every lane holds sel_i / sel_w (slots >= n zero); probs, if not
 * NULL, receives the probabilities.  Returns n = min(k, E). */
__device__ __forceinline__ int nmoe_wave_route(const float *lg, int num_experts, int k, float *scratch,
                                               const uint64_t *tab, uint32_t sel_i[NMOE_MAX_K],
                                               float sel_w[NMOE_MAX_K], float *probs) {
    const int lane = threadIdx.x & 63;
    float l[4], p[4];
#pragma unroll
    for (int j = 0; j < 4; j++) l[j] = lane + 64 * j < num_experts ? lg[lane + 64 * j] : 0.0f;
    nmoe_wave_softmax(l, num_experts, scratch, tab, p);
    if (probs != NULL) {
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (lane + 64 * j < num_experts) probs[lane + 64 * j] = p[j];
    }
    /* probabilities are >= 0, so their bits order like the values; +1 keeps
     * 0 free for absent entries */
    const int n = min(k, num_experts);
    uint32_t key[4], selkey[NMOE_MAX_K];
#pragma unroll
    for (int j = 0; j < 4; j++) key[j] = lane + 64 * j < num_experts ? __float_as_uint(p[j]) + 1u : 0u;
    nmoe_wave_top_keys(key, n, sel_i, selkey);
    float sel_v[NMOE_MAX_K];
#pragma unroll
    for (int s = 0; s < NMOE_MAX_K; s++) sel_v[s] = s < n ? __uint_as_float(selkey[s] - 1u) : 0.0f;
    nmoe_renormalize(sel_v, n, sel_w);
    return n;
}

/* --------------------------------------------- exchange across blocks */

/* Device-coherent loads/stores of values exchanged between blocks of one
 * launch: agent-scope relaxed atomics (global_load/store ... sc1), so no
 * L2-wide writeback or invalidate is needed; ordering comes from s_waitcnt
 * before the counter update that publishes them.
 *
 * Every such pointer is cast to the global address space first.  Through a
 * generic pointer the access is a flat instruction, which may reach LDS as
 * far as the compiler knows: in a kernel that also loads LDS directly from
 * memory (global_load_lds), it then waits for all of those loads (and with
 * them every other load in flight) before each exchange access. */
typedef __attribute__((address_space(1))) uint32_t nmoe_g32;
typedef __attribute__((address_space(1))) uint64_t nmoe_g64;
typedef __attribute__((address_space(1))) uint8_t nmoe_gu8;
__device__ __forceinline__ void nmoe_st_dev(float *p, float v) {
    __hip_atomic_store((nmoe_g32 *)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float nmoe_ld_dev(const float *p) {
    return __uint_as_float(__hip_atomic_load((nmoe_g32 *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ uint32_t nmoe_ld_u32_dev(uint32_t *p) {
    return __hip_atomic_load((nmoe_g32 *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t nmoe_add_u32_dev(uint32_t *p, uint32_t v) {
    return __hip_atomic_fetch_add((nmoe_g32 *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Accelerator die (XCC) the calling wave runs on. */
__device__ __forceinline__ uint32_t nmoe_xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(v));
    return v;
}

/* Values exchanged between the blocks of one launch travel as 64-bit words
 * (launch epoch << 32 | float bits), written and read whole with one
 * device-coherent access: a consumer polls the data itself until every word
 * carries the current epoch, so no separate counter round trip is needed. */
__device__ __forceinline__ void nmoe_st_tagged(uint64_t *p, uint32_t epoch, float v) {
    __hip_atomic_store((nmoe_g64 *)p, ((uint64_t)epoch << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t nmoe_ld_tagged(const uint64_t *p) {
    return __hip_atomic_load((nmoe_g64 *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool nmoe_tag_is(uint64_t w, uint32_t epoch) { return (uint32_t)(w >> 32) == epoch; }
__device__ __forceinline__ float nmoe_tag_val(uint64_t w) { return __uint_as_float((uint32_t)w); }

/* Bounded spin so that a grid whose blocks are not all resident still ends:
 * the waiting block gives up after this many unsuccessful poll rounds (the
 * default; NMOE_HIP_OPT_SPIN_LIMIT changes it), records the failure in the
 * status word and carries on (the host then reports ETIMEDOUT). */
#define NMOE_SPIN_LIMIT (1u << 20)

/* ------------------------------------------------------------ RMSNorm */

template <int CTRL>
__device__ __forceinline__ double nmoe_dpp_d(double v) {
    uint64_t u = __builtin_bit_cast(uint64_t, v);
    u = ((uint64_t)nmoe_dpp_u<CTRL>((uint32_t)(u >> 32)) << 32) | nmoe_dpp_u<CTRL>((uint32_t)u);
    return __builtin_bit_cast(double, u);
}

__device__ __forceinline__ double nmoe_readlane_d(double v, int lane) {
    uint64_t u = __builtin_bit_cast(uint64_t, v);
    uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
    uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

/* The sum of v * v over a wavefront, one v per lane: exact squares (a
 * float times a float fits a double), added as a tree of depth 6 (4 DPP
 * levels within each row of 16 lanes, then rows (0 + 16) + (32 + 48)).
 * Uniform.  Every lane must be active. */
__device__ __forceinline__ double nmoe_wave_sq_tree(float v) {
    double sq = (double)v * (double)v;
    sq = sq + nmoe_dpp_d<NMOE_DPP_XOR1>(sq);
    sq = sq + nmoe_dpp_d<NMOE_DPP_XOR2>(sq);
    sq = sq + nmoe_dpp_d<NMOE_DPP_HALF_MIRROR>(sq);
    sq = sq + nmoe_dpp_d<NMOE_DPP_MIRROR>(sq);
    return (nmoe_readlane_d(sq, 0) + nmoe_readlane_d(sq, 16)) + (nmoe_readlane_d(sq, 32) + nmoe_readlane_d(sq, 48));
}

/* The sum of 32 doubles held by lanes 0..31 (the other lanes hold 0), a
 * tree of depth 5 in a fixed order.  Uniform.  Every lane must be active.
 * 32 partials from nmoe_wave_sq_tree make a tree of depth 11 over 2048
 * squares, the depth nmoe_mean_sq_from_sum allows for. */
__device__ __forceinline__ double nmoe_sum32_tree(double ps) {
    ps = ps + nmoe_dpp_d<NMOE_DPP_XOR1>(ps);
    ps = ps + nmoe_dpp_d<NMOE_DPP_XOR2>(ps);
    ps = ps + nmoe_dpp_d<NMOE_DPP_HALF_MIRROR>(ps);
    ps = ps + nmoe_dpp_d<NMOE_DPP_MIRROR>(ps);
    return nmoe_readlane_d(ps, 0) + nmoe_readlane_d(ps, 16);
}

/* rms of math.m:34-65 (unit weight) over the 2048 fp32 values h, by a whole
 * block of 256 or more threads (threads 0..255 hold the data, the rest
 * only take part in the barriers); uniform result.  math.m sums the squares
 * in an x87 `long double` (64-bit significand) running sum.  The block sums
 * the squares in double as a tree of depth 11 (3 levels in a thread, 4 DPP
 * levels in a row of 16 lanes, 2 over the rows, 2 over the 4 wavefronts),
 * a short dependency chain; nmoe_mean_sq_from_sum turns that into math.m's
 * float wherever no rounding midpoint is near, and otherwise (a near-tie,
 * or tiny values) lane 0 replays the x87 running sum in index order.
 * lds_h: 2048 floats of LDS, lds_dd: 8 doubles, lds_f: 1 float.  vals
 * (nullable) receives the thread's 8 values h[8 tid ..] (0 beyond 2048). */
__device__ float nmoe_block_rms_exact(const float *h, float eps, float *lds_h, double *lds_dd, float *lds_f,
                                      float *vals = nullptr) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float4 *h4 = (const float4 *)h;
    const bool holds = tid < NMOE_HIDDEN / 8;
    float4 v0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), v1 = v0;
    if (holds) {
        v0 = h4[2 * tid];
        v1 = h4[2 * tid + 1];
    }
    float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    if (vals != nullptr)
#pragma unroll
        for (int i = 0; i < 8; i++) vals[i] = vv[i];
    double q[8];
#pragma unroll
    for (int i = 0; i < 8; i++) q[i] = (double)vv[i] * (double)vv[i]; /* exact: 48 significant bits */
    double s = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
    /* with every lane active (reading other lanes from inside a
     * lane-divergent branch would read undefined values); each step adds
     * the same two sums in both lanes of a pair, so a row's 16 lanes end
     * with equal values */
    s = s + nmoe_dpp_d<NMOE_DPP_XOR1>(s);
    s = s + nmoe_dpp_d<NMOE_DPP_XOR2>(s);
    s = s + nmoe_dpp_d<NMOE_DPP_HALF_MIRROR>(s);
    s = s + nmoe_dpp_d<NMOE_DPP_MIRROR>(s);
    const double ws = (nmoe_readlane_d(s, 0) + nmoe_readlane_d(s, 16)) + (nmoe_readlane_d(s, 32) + nmoe_readlane_d(s, 48));
    if (lane == 0 && holds) lds_dd[wave] = ws;
    __syncthreads();
    if (tid == 0) lds_f[0] = nmoe_mean_sq_from_sum((lds_dd[0] + lds_dd[1]) + (lds_dd[2] + lds_dd[3]));
    __syncthreads();
    float mean = lds_f[0];
    if (mean < 0.0f) {
        /* near a rounding midpoint: replay the x87 running sum */
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (holds) lds_h[8 * tid + i] = vv[i];
        __syncthreads();
        if (tid == 0) {
            nmoe_x87 acc = nmoe_x87_zero();
            for (int i = 0; i < NMOE_HIDDEN; i++) acc = nmoe_x87_add(acc, nmoe_x87_square(lds_h[i]));
            acc.e -= 11; /* / 2048, exact */
            lds_f[0] = nmoe_x87_to_float(acc);
        }
        __syncthreads();
        mean = lds_f[0];
    }
    float rms = nmoe_sqrtf_rn(mean + eps); /* sqrtf((float)mean + eps) */
    return rms == 0.0f ? 1.0f : rms;
}

#endif
