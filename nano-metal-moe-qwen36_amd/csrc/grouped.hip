/*
 * grouped.hip -- the routed experts of many tokens as grouped GEMMs on the
 * matrix cores (batched decode, prefill).
 *
 * Reference: the runtime runs its MoE tail once per token
 * (src/runtime.m:3816 loops tokens over NMOEPipelinedExpertTail,
 * runtime.m:2908-2999), so every token re-reads its experts.  Here the
 * (token, slot) pairs are first permuted into per-expert groups (a stable
 * counting sort), and each expert's weights are read once for all of its
 * tokens:
 *
 *   D1/D2  dispatch: per-block expert histograms, then offsets[257] and the
 *          stable permutation perm[] of the entries q = t*k + s (ties by t,
 *          then s).  Entries whose index is outside the layer are left out.
 *   X      per token: x in the matrix-core operand order (bf16; fp32 input
 *          also gets a low plane x - bf16(x)) and its 32 group sums.
 *   G      per (expert, 64 gate/up rows): Act = SwiGLU(X_e Wg^T, X_e Wu^T)
 *          for all of the expert's rows, as hi + lo bf16 planes, and the
 *          8 group sums of each act row.
 *   Dn     per (expert, 64 down rows): Y_e = Act_e Wd^T -> Y[q][2048].
 *   C      per token: out = h_mid + sum_s w_s y_s in slot order
 *          (kernels.metal:1394-1423) (+ sigmoid(g) * shared).
 *
 * Exactness on the matrix cores.  The dequantised weight is q*scale + bias
 * per group of 64 (math.m:206-234).  A bf16 weight would round q*scale, so
 * the cores multiply the integer codes instead, exactly: the code q is fed
 * as the bf16 value 128 + q (bit pattern 0x4300 | q, one and-or per two
 * codes), and
 *     sum_k w_k x_k = sum_g s_g P_g + sum_g (b_g - 128 s_g) xs_g,
 *     P_g = sum_{k in g} (128 + q_k) x_k,   xs_g = sum_{k in g} x_k,
 * with P_g from v_mfma_f32_16x16x32_bf16 (bf16 products are exact in fp32),
 * the s_g scaling applied per group in fp32, and the second sum from
 * v_mfma_f32_16x16x4_f32 over the 32 (gate/up) or 8 (down) groups.  x is
 * bf16 (exact) or a hi + lo bf16 pair; act is a hi + lo pair (16
 * significant bits).  So the only rounding beyond fp32 accumulation is
 * act's 2^-17.
 *
 * Operand order: an MFMA lane owns 8 consecutive k of a 32-deep slice; the
 * sum over k does not care which k a lane owns, so each lane owns the 16 k
 * of one word (q2) or two words (q4) of a row and the two slices split
 * them in the order that makes the code unpacking cheapest; x and act are
 * stored in that order (nmoe_kperm).
 */
#include "nmoe_device.h"

#pragma clang fp contract(off)

typedef __attribute__((ext_vector_type(8))) __bf16 nmoe_bf16x8;
typedef __attribute__((ext_vector_type(4))) float nmoe_f32x4;

#define NMOE_DISPATCH_BLOCKS 16
#define NMOE_GU_TILE 64   /* gate/up rows per block (one down-K group) */
#define NMOE_DN_TILE 64   /* down rows per block */
#define NMOE_MCHUNK 64    /* expert rows per pass (four 16-row MFMA blocks) */

/* k offset (within a lane's 16-k span) of operand element `slot`
 * (slot = 8 * slice + 2 * dword + half). */
template <int BITS>
__host__ __device__ constexpr int nmoe_kperm(int slot) {
    return BITS == 4 ? 8 * (slot >> 3) + ((slot >> 1) & 3) + 4 * (slot & 1)
                     : 4 * (slot >> 3) + ((slot >> 1) & 3) + 8 * (slot & 1);
}

template <int BITS>
__device__ __forceinline__ int nmoe_kperm_inv(int off) {
#pragma unroll
    for (int slot = 0; slot < 16; slot++)
        if (nmoe_kperm<BITS>(slot) == off) return slot;
    return 0;
}

/* The codes of one lane's 16-k span as two MFMA operands of bf16(128 + q):
 * q4: words w0 (k 0..7), w1 (k 8..15); q2: word w0 (k 0..15). */
template <int BITS>
__device__ __forceinline__ void nmoe_codes_bf16(uint32_t w0, uint32_t w1, uint4 &b0, uint4 &b1) {
    if (BITS == 4) {
        b0.x = (w0 & 0x000F000Fu) | 0x43004300u;
        b0.y = ((w0 >> 4) & 0x000F000Fu) | 0x43004300u;
        b0.z = ((w0 >> 8) & 0x000F000Fu) | 0x43004300u;
        b0.w = ((w0 >> 12) & 0x000F000Fu) | 0x43004300u;
        b1.x = (w1 & 0x000F000Fu) | 0x43004300u;
        b1.y = ((w1 >> 4) & 0x000F000Fu) | 0x43004300u;
        b1.z = ((w1 >> 8) & 0x000F000Fu) | 0x43004300u;
        b1.w = ((w1 >> 12) & 0x000F000Fu) | 0x43004300u;
    } else {
        b0.x = (w0 & 0x00030003u) | 0x43004300u;
        b0.y = ((w0 >> 2) & 0x00030003u) | 0x43004300u;
        b0.z = ((w0 >> 4) & 0x00030003u) | 0x43004300u;
        b0.w = ((w0 >> 6) & 0x00030003u) | 0x43004300u;
        b1.x = ((w0 >> 8) & 0x00030003u) | 0x43004300u;
        b1.y = ((w0 >> 10) & 0x00030003u) | 0x43004300u;
        b1.z = ((w0 >> 12) & 0x00030003u) | 0x43004300u;
        b1.w = ((w0 >> 14) & 0x00030003u) | 0x43004300u;
    }
}

__device__ __forceinline__ nmoe_bf16x8 nmoe_as_bf16x8(uint4 v) { return __builtin_bit_cast(nmoe_bf16x8, v); }

__device__ __forceinline__ nmoe_f32x4 nmoe_mfma16(uint4 a, uint4 b, nmoe_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(nmoe_as_bf16x8(a), nmoe_as_bf16x8(b), c, 0, 0, 0);
}

/* bf16 of an fp32 value, round to nearest even (finite inputs). */
__device__ __forceinline__ uint32_t nmoe_bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

/* ------------------------------------------------------------ dispatch */

__device__ __forceinline__ uint32_t nmoe_entry_expert(const uint32_t *idx, int q, int k) {
    const uint32_t e = idx[(size_t)(q / k) * NMOE_MAX_K + (q % k)];
    return e < NMOE_EXPERTS ? e : (uint32_t)NMOE_EXPERTS; /* 256: left out */
}

/* D1: counts[b][257] = expert histogram of entry slice b. */
__global__ void __launch_bounds__(256) nmoe_dispatch_count_kernel(const uint32_t *idx, int ntok, int k,
                                                                   uint32_t *counts) {
    __shared__ uint32_t h[NMOE_EXPERTS + 1];
    const int tid = threadIdx.x, b = blockIdx.x, n = ntok * k;
    const int per = (n + NMOE_DISPATCH_BLOCKS - 1) / NMOE_DISPATCH_BLOCKS;
    for (int i = tid; i <= NMOE_EXPERTS; i += 256) h[i] = 0;
    __syncthreads();
    const int q1 = min(n, (b + 1) * per);
    for (int q = b * per + tid; q < q1; q += 256) atomicAdd(&h[nmoe_entry_expert(idx, q, k)], 1u);
    __syncthreads();
    for (int i = tid; i <= NMOE_EXPERTS; i += 256) counts[b * (NMOE_EXPERTS + 1) + i] = h[i];
}

/* D2: offsets (block 0 writes them) and the stable permutation of slice b:
 * chunks of 256 entries in order; within a chunk the rank of an entry is
 * its rank among the equal-expert lanes of its wavefront (a 9-bit
 * multi-split by ballots) plus the counts of the earlier wavefronts. */
__global__ void __launch_bounds__(256) nmoe_dispatch_scatter_kernel(const uint32_t *idx, int ntok, int k,
                                                                     const uint32_t *counts, uint32_t *perm,
                                                                     uint32_t *offsets) {
    __shared__ uint32_t s_base[NMOE_EXPERTS];
    __shared__ uint32_t s_scan[256];
    __shared__ uint32_t s_wc[4][NMOE_EXPERTS + 1];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, b = blockIdx.x, n = ntok * k;
    const int per = (n + NMOE_DISPATCH_BLOCKS - 1) / NMOE_DISPATCH_BLOCKS;
    /* thread e: total of expert e and its count in the slices before b */
    uint32_t total = 0, before = 0;
    for (int bb = 0; bb < NMOE_DISPATCH_BLOCKS; bb++) {
        const uint32_t c = counts[bb * (NMOE_EXPERTS + 1) + tid];
        total += c;
        before += bb < b ? c : 0u;
    }
    /* exclusive scan of total over the 256 experts (Hillis-Steele in LDS) */
    s_scan[tid] = total;
    __syncthreads();
    for (int d = 1; d < 256; d <<= 1) {
        const uint32_t v = tid >= d ? s_scan[tid - d] : 0u;
        __syncthreads();
        s_scan[tid] += v;
        __syncthreads();
    }
    const uint32_t off = s_scan[tid] - total;
    if (b == 0) {
        offsets[tid] = off;
        if (tid == 255) offsets[NMOE_EXPERTS] = s_scan[255];
    }
    s_base[tid] = off + before;
    for (int i = tid; i < 4 * (NMOE_EXPERTS + 1); i += 256) (&s_wc[0][0])[i] = 0;
    __syncthreads();
    const int q0 = b * per, q1 = min(n, (b + 1) * per);
    for (int c0 = q0; c0 < q1; c0 += 256) {
        const int q = c0 + tid;
        const uint32_t e = q < q1 ? nmoe_entry_expert(idx, q, k) : (uint32_t)NMOE_EXPERTS;
        uint64_t peers = ~0ull;
#pragma unroll
        for (int bit = 0; bit < 9; bit++) {
            const uint64_t m = __ballot((e >> bit) & 1u);
            peers &= ((e >> bit) & 1u) ? m : ~m;
        }
        const uint32_t rank = (uint32_t)__builtin_popcountll(peers & ((1ull << lane) - 1ull));
        if (rank == 0) s_wc[wave][e] = (uint32_t)__builtin_popcountll(peers);
        __syncthreads();
        if (e < NMOE_EXPERTS) {
            uint32_t pos = s_base[e] + rank;
            for (int w = 0; w < wave; w++) pos += s_wc[w][e];
            perm[pos] = (uint32_t)q;
        }
        __syncthreads();
        s_base[tid] += s_wc[0][tid] + s_wc[1][tid] + s_wc[2][tid] + s_wc[3][tid];
        s_wc[0][tid] = s_wc[1][tid] = s_wc[2][tid] = s_wc[3][tid] = 0;
        if (tid == 0) s_wc[0][NMOE_EXPERTS] = s_wc[1][NMOE_EXPERTS] = s_wc[2][NMOE_EXPERTS] = s_wc[3][NMOE_EXPERTS] = 0;
        __syncthreads();
    }
}

/* ------------------------------------------------------------ X prep */

/* xp[t][16 span + slot] = x[t][16 span + kperm(slot)] as bf16 (hi plane; the
 * lo plane x - hi when x is fp32), xs[t][g] = sum of the 64 values of group
 * g (hi + lo, in a fixed order). */
template <int BITS, typename XT>
__global__ void __launch_bounds__(256) nmoe_grouped_xprep_kernel(const XT *x, uint16_t *xhi, uint16_t *xlo,
                                                                  float *xs) {
    const int t = blockIdx.x, tid = threadIdx.x; /* 8 elements per thread: half a span */
    const int span = tid >> 1, half = tid & 1;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int slot = 8 * half + i;
        const int c = 16 * span + nmoe_kperm<BITS>(slot);
        if (sizeof(XT) == 2)
            v[i] = nmoe_bf16f(((const uint16_t *)x)[(size_t)t * NMOE_HIDDEN + c]);
        else
            v[i] = ((const float *)x)[(size_t)t * NMOE_HIDDEN + c];
    }
    uint32_t hi[8];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        hi[i] = nmoe_bf16_rne(v[i]);
        const float lo = v[i] - nmoe_bf16f(hi[i]);
        sum += nmoe_bf16f(hi[i]) + nmoe_bf16f(nmoe_bf16_rne(lo));
        if (xlo != NULL) xlo[(size_t)t * NMOE_HIDDEN + 16 * span + 8 * half + i] = (uint16_t)nmoe_bf16_rne(lo);
    }
    uint4 pk;
    pk.x = hi[0] | (hi[1] << 16);
    pk.y = hi[2] | (hi[3] << 16);
    pk.z = hi[4] | (hi[5] << 16);
    pk.w = hi[6] | (hi[7] << 16);
    ((uint4 *)(xhi + (size_t)t * NMOE_HIDDEN))[2 * span + half] = pk;
    /* group sums: a group is 64 columns = 4 spans = 8 threads (consecutive) */
    sum = sum + nmoe_dpp_f<NMOE_DPP_XOR1>(sum);
    sum = sum + nmoe_dpp_f<NMOE_DPP_XOR2>(sum);
    sum = sum + nmoe_dpp_f<NMOE_DPP_HALF_MIRROR>(sum);
    if ((tid & 7) == 0) xs[(size_t)t * (NMOE_HIDDEN / NMOE_GROUP) + (tid >> 3)] = sum;
}

/* ------------------------------------------------------------ gate/up */

/* Expert blockIdx.x, gate/up rows 64 * blockIdx.y .. +63: act rows of all the
 * expert's entries.  Wave w owns rows 16w..16w+15 of the tile for gate and
 * up alike, so a lane holds gate and up of the same (entry, row). */
template <int BITS, int XPL>
__global__ void __launch_bounds__(256) nmoe_grouped_gateup_kernel(const uint8_t *pack, const uint16_t *xhi,
                                                                   const uint16_t *xlo, const float *xs,
                                                                   const uint32_t *perm, const uint32_t *offsets,
                                                                   int k, uint16_t *ahi, uint16_t *alo, float *as) {
    using Q = nmoe_q<BITS>;
    using L = nmoe_layout<BITS>;
    constexpr int G = NMOE_HIDDEN / NMOE_GROUP; /* 32 groups */
    __shared__ float s_sc[2][NMOE_GU_TILE][G];  /* scale */
    __shared__ float s_cc[2][NMOE_GU_TILE][G];  /* bias - 128 scale */
    __shared__ float s_as[4][NMOE_MCHUNK];
    const int e = blockIdx.x, nt = blockIdx.y;
    const uint32_t p0 = offsets[e], n = offsets[e + 1] - p0;
    if (n == 0) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, kb = lane >> 4;
    const uint8_t *ex = pack + (size_t)e * L::expert_size;
    for (int i = tid; i < 2 * NMOE_GU_TILE * G; i += 256) {
        const int mat = i / (NMOE_GU_TILE * G), rr = (i / G) % NMOE_GU_TILE, g = i % G;
        const size_t so = mat == 0 ? L::gate_s : L::up_s;
        const size_t sb = mat == 0 ? L::gate_b : L::up_b;
        const int row = nt * NMOE_GU_TILE + rr;
        const float s = nmoe_bf16f(((const uint16_t *)(ex + so))[row * G + g]);
        const float b = nmoe_bf16f(((const uint16_t *)(ex + sb))[row * G + g]);
        s_sc[mat][rr][g] = s;
        s_cc[mat][rr][g] = b - 128.0f * s; /* exact: both have 8 significant bits */
    }
    __syncthreads();
    const int rt = wave * 16 + col;           /* row within the tile */
    const int r = nt * NMOE_GU_TILE + rt;      /* gate/up row */
    const uint32_t *gw = (const uint32_t *)(ex + L::gate_w) + (size_t)r * Q::WPR_G;
    const uint32_t *uw = (const uint32_t *)(ex + L::up_w) + (size_t)r * Q::WPR_G;

    for (uint32_t m0 = 0; m0 < n; m0 += NMOE_MCHUNK) {
        /* A rows: entry m0 + 16 mb + col; output rows: 16 mb + 4 kb + i */
        const uint16_t *xa[4], *xla[4];
        const float *xsa[4];
#pragma unroll
        for (int mb = 0; mb < 4; mb++) {
            const uint32_t m = m0 + 16 * mb + col;
            const uint32_t t = m < n ? perm[p0 + m] / (uint32_t)k : perm[p0] / (uint32_t)k;
            xa[mb] = xhi + (size_t)t * NMOE_HIDDEN + 16 * kb;
            xla[mb] = XPL == 2 ? xlo + (size_t)t * NMOE_HIDDEN + 16 * kb : NULL;
            xsa[mb] = xs + (size_t)t * G;
        }
        const int nb = (int)min((n - m0 + 15) / 16, 4u);
        nmoe_f32x4 acc[2][4];
        /* sum_g (b_g - 128 s_g) xs_g on the fp32 cores: A lane = (entry col, group 4tq + kb),
         * B lane = (row col, group 4tq + kb) */
#pragma unroll
        for (int mb = 0; mb < 4; mb++) {
            acc[0][mb] = nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            acc[1][mb] = nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if (mb < nb) {
#pragma unroll
                for (int tq = 0; tq < G / 4; tq++) {
                    const float a = xsa[mb][4 * tq + kb];
                    acc[0][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, s_cc[0][rt][4 * tq + kb], acc[0][mb], 0, 0, 0);
                    acc[1][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, s_cc[1][rt][4 * tq + kb], acc[1][mb], 0, 0, 0);
                }
            }
        }
        for (int g = 0; g < G; g++) {
            uint32_t g0, g1 = 0, u0, u1 = 0;
            if (BITS == 4) {
                const uint2 gv = *(const uint2 *)(gw + 8 * g + 2 * kb);
                const uint2 uv = *(const uint2 *)(uw + 8 * g + 2 * kb);
                g0 = gv.x, g1 = gv.y, u0 = uv.x, u1 = uv.y;
            } else {
                g0 = gw[4 * g + kb];
                u0 = uw[4 * g + kb];
            }
            uint4 bg0, bg1, bu0, bu1;
            nmoe_codes_bf16<BITS>(g0, g1, bg0, bg1);
            nmoe_codes_bf16<BITS>(u0, u1, bu0, bu1);
            /* the lane's column is the same row for every group: its scales */
            const float sg = s_sc[0][rt][g], su = s_sc[1][rt][g];
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                if (mb < nb) {
                    const uint4 *pa = (const uint4 *)(xa[mb] + 64 * g);
                    const uint4 a0 = pa[0], a1 = pa[1];
                    nmoe_f32x4 pg = nmoe_mfma16(a0, bg0, nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f});
                    pg = nmoe_mfma16(a1, bg1, pg);
                    nmoe_f32x4 pu = nmoe_mfma16(a0, bu0, nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f});
                    pu = nmoe_mfma16(a1, bu1, pu);
                    if (XPL == 2) {
                        const uint4 *pl = (const uint4 *)(xla[mb] + 64 * g);
                        const uint4 l0 = pl[0], l1 = pl[1];
                        pg = nmoe_mfma16(l0, bg0, pg);
                        pg = nmoe_mfma16(l1, bg1, pg);
                        pu = nmoe_mfma16(l0, bu0, pu);
                        pu = nmoe_mfma16(l1, bu1, pu);
                    }
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        acc[0][mb][i] = __builtin_fmaf(sg, pg[i], acc[0][mb][i]);
                        acc[1][mb][i] = __builtin_fmaf(su, pu[i], acc[1][mb][i]);
                    }
                }
            }
        }
        /* epilogue: act = SiLU(gate) * up as hi + lo bf16, in the down
         * kernel's operand order; group sums of act rows over this tile */
        const int span = (nt * NMOE_GU_TILE + wave * 16) / 16;
        const int slot = nmoe_kperm_inv<BITS>(col);
#pragma unroll
        for (int mb = 0; mb < 4; mb++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t m = m0 + 16 * mb + 4 * kb + i;
                const float a = nmoe_silu_dev(acc[0][mb][i]) * acc[1][mb][i];
                const uint32_t h = nmoe_bf16_rne(a);
                const uint32_t l = nmoe_bf16_rne(a - nmoe_bf16f(h));
                float part = nmoe_bf16f(h) + nmoe_bf16f(l);
                if (mb < nb && m < n) {
                    const size_t o = (size_t)(p0 + m) * NMOE_INTER + 16 * span + slot;
                    ahi[o] = (uint16_t)h;
                    alo[o] = (uint16_t)l;
                }
                part = nmoe_dpp_group_sum<16>(part); /* the 16 rows of this wave */
                if (col == 0) s_as[wave][16 * mb + 4 * kb + i] = part;
            }
        }
        __syncthreads();
        if (tid < NMOE_MCHUNK) {
            const uint32_t m = m0 + tid;
            if (m < n)
                as[(size_t)(p0 + m) * (NMOE_INTER / NMOE_GROUP) + nt] =
                    (s_as[0][tid] + s_as[1][tid]) + (s_as[2][tid] + s_as[3][tid]);
        }
        __syncthreads();
    }
}

/* ------------------------------------------------------------ down */

/* Expert blockIdx.x, down rows 64 * blockIdx.y .. +63: y[q][row] for all the
 * expert's entries q. */
template <int BITS>
__global__ void __launch_bounds__(256) nmoe_grouped_down_kernel(const uint8_t *pack, const uint16_t *ahi,
                                                                 const uint16_t *alo, const float *as,
                                                                 const uint32_t *perm, const uint32_t *offsets,
                                                                 float *y) {
    using Q = nmoe_q<BITS>;
    using L = nmoe_layout<BITS>;
    constexpr int G = NMOE_INTER / NMOE_GROUP; /* 8 groups */
    const int e = blockIdx.x, nt = blockIdx.y;
    const uint32_t p0 = offsets[e], n = offsets[e + 1] - p0;
    if (n == 0) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, kb = lane >> 4;
    const uint8_t *ex = pack + (size_t)e * L::expert_size;
    const int r = nt * NMOE_DN_TILE + wave * 16 + col;
    const uint32_t *dw = (const uint32_t *)(ex + L::down_w) + (size_t)r * Q::WPR_D;
    float sc[G], cc[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        sc[g] = nmoe_bf16f(((const uint16_t *)(ex + L::down_s))[r * G + g]);
        cc[g] = nmoe_bf16f(((const uint16_t *)(ex + L::down_b))[r * G + g]) - 128.0f * sc[g];
    }
    for (uint32_t m0 = 0; m0 < n; m0 += NMOE_MCHUNK) {
        const int nb = (int)min((n - m0 + 15) / 16, 4u);
        const uint16_t *ah[4], *al[4];
        const float *asa[4];
#pragma unroll
        for (int mb = 0; mb < 4; mb++) {
            const uint32_t m = min(m0 + 16 * mb + col, n - 1);
            ah[mb] = ahi + (size_t)(p0 + m) * NMOE_INTER + 16 * kb;
            al[mb] = alo + (size_t)(p0 + m) * NMOE_INTER + 16 * kb;
            asa[mb] = as + (size_t)(p0 + m) * G;
        }
        nmoe_f32x4 acc[4];
#pragma unroll
        for (int mb = 0; mb < 4; mb++) {
            acc[mb] = nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if (mb < nb) {
#pragma unroll
                for (int tq = 0; tq < G / 4; tq++) {
                    const float c = tq == 0 ? (kb == 0 ? cc[0] : kb == 1 ? cc[1] : kb == 2 ? cc[2] : cc[3])
                                            : (kb == 0 ? cc[4] : kb == 1 ? cc[5] : kb == 2 ? cc[6] : cc[7]);
                    acc[mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(asa[mb][4 * tq + kb], c, acc[mb], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            uint32_t w0, w1 = 0;
            if (BITS == 4) {
                const uint2 v = *(const uint2 *)(dw + 8 * g + 2 * kb);
                w0 = v.x, w1 = v.y;
            } else {
                w0 = dw[4 * g + kb];
            }
            uint4 b0, b1;
            nmoe_codes_bf16<BITS>(w0, w1, b0, b1);
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                if (mb < nb) {
                    const uint4 *ph = (const uint4 *)(ah[mb] + 64 * g);
                    const uint4 *pl = (const uint4 *)(al[mb] + 64 * g);
                    nmoe_f32x4 p = nmoe_mfma16(ph[0], b0, nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f});
                    p = nmoe_mfma16(ph[1], b1, p);
                    p = nmoe_mfma16(pl[0], b0, p);
                    p = nmoe_mfma16(pl[1], b1, p);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[mb][i] = __builtin_fmaf(sc[g], p[i], acc[mb][i]);
                }
            }
        }
#pragma unroll
        for (int mb = 0; mb < 4; mb++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t m = m0 + 16 * mb + 4 * kb + i;
                if (mb < nb && m < n) y[(size_t)perm[p0 + m] * NMOE_HIDDEN + r] = acc[mb][i];
            }
        }
    }
}

/* ------------------------------------------------------------ combine */

/* out[t] = h_mid[t] + sum_{s<k} w[t][s] y[t*k+s] in slot order
 * (kernels.metal:1394-1423) (+ sigmoid(g) * shared_out); a slot whose index
 * is outside the layer contributes nothing (runtime.m:2977-2981). */
__global__ void __launch_bounds__(256) nmoe_grouped_combine_kernel(const float *y, const uint32_t *idx,
                                                                    const float *w, int k, const float *h_mid,
                                                                    const float *shared_out,
                                                                    const float *shared_gate_raw, float *out) {
    const int t = blockIdx.y, r = blockIdx.x * 256 + threadIdx.x;
    float moe = 0.0f;
    for (int s = 0; s < k; s++) {
        const size_t q = (size_t)t * k + s;
        if (idx[(size_t)t * NMOE_MAX_K + s] < NMOE_EXPERTS) moe += w[(size_t)t * NMOE_MAX_K + s] * y[q * NMOE_HIDDEN + r];
    }
    float o = h_mid[(size_t)t * NMOE_HIDDEN + r] + moe;
    if (shared_out != NULL) o = o + nmoe_sigmoid_dev(shared_gate_raw[t]) * shared_out[(size_t)t * NMOE_HIDDEN + r];
    out[(size_t)t * NMOE_HIDDEN + r] = o;
}

/* ------------------------------------------------------------ host */

extern "C" int nmoe_grouped_init(nmoe_hip_ctx *ctx) {
    const size_t mt = (size_t)ctx->max_tokens, rows = mt * NMOE_MAX_K;
    ctx->grouped_min_tokens = 8;
    if (hipMalloc((void **)&ctx->g_counts, NMOE_DISPATCH_BLOCKS * (NMOE_EXPERTS + 1) * sizeof(uint32_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_perm, rows * sizeof(uint32_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_offsets, (NMOE_EXPERTS + 1) * sizeof(uint32_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_xhi, mt * NMOE_HIDDEN * sizeof(uint16_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_xlo, mt * NMOE_HIDDEN * sizeof(uint16_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_xs, mt * (NMOE_HIDDEN / NMOE_GROUP) * sizeof(float)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_ahi, rows * NMOE_INTER * sizeof(uint16_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_alo, rows * NMOE_INTER * sizeof(uint16_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_as, rows * (NMOE_INTER / NMOE_GROUP) * sizeof(float)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_y, rows * NMOE_HIDDEN * sizeof(float)) != hipSuccess)
        return NMOE_HIP_ENOMEM;
    return NMOE_HIP_OK;
}

extern "C" void nmoe_grouped_free(nmoe_hip_ctx *ctx) {
    void *p[] = {ctx->g_counts, ctx->g_perm, ctx->g_offsets, ctx->g_xhi, ctx->g_xlo,
                 ctx->g_xs,     ctx->g_ahi,  ctx->g_alo,     ctx->g_as,  ctx->g_y};
    for (void *q : p)
        if (q != NULL) (void)hipFree(q);
}

/* D1 + D2 into perm / offsets (any device buffers of T*k and 257 words). */
extern "C" int nmoe_grouped_dispatch(nmoe_hip_ctx *ctx, const uint32_t *idx, int ntok, int k, uint32_t *perm,
                                     uint32_t *offsets, hipStream_t s) {
    hipLaunchKernelGGL(nmoe_dispatch_count_kernel, dim3(NMOE_DISPATCH_BLOCKS), dim3(256), 0, s, idx, ntok, k,
                       ctx->g_counts);
    hipLaunchKernelGGL(nmoe_dispatch_scatter_kernel, dim3(NMOE_DISPATCH_BLOCKS), dim3(256), 0, s, idx, ntok, k,
                       (const uint32_t *)ctx->g_counts, perm, offsets);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? NMOE_HIP_OK : nmoe_hip_check(ctx, e, "dispatch launch");
}

template <int BITS>
static int nmoe_grouped_run(nmoe_hip_ctx *ctx, const uint8_t *pack, const void *x, int x_dtype, int ntok, int k,
                            const uint32_t *idx, const float *w, const float *h_mid, const float *shared_out,
                            const float *shared_gate_raw, float *out, hipStream_t s) {
    int rc = nmoe_grouped_dispatch(ctx, idx, ntok, k, ctx->g_perm, ctx->g_offsets, s);
    if (rc != NMOE_HIP_OK) return rc;
    const bool bf = x_dtype == NMOE_HIP_BF16;
    if (bf)
        hipLaunchKernelGGL((nmoe_grouped_xprep_kernel<BITS, uint16_t>), dim3(ntok), dim3(256), 0, s,
                           (const uint16_t *)x, ctx->g_xhi, (uint16_t *)NULL, ctx->g_xs);
    else
        hipLaunchKernelGGL((nmoe_grouped_xprep_kernel<BITS, float>), dim3(ntok), dim3(256), 0, s, (const float *)x,
                           ctx->g_xhi, ctx->g_xlo, ctx->g_xs);
    const dim3 ggu(NMOE_EXPERTS, NMOE_INTER / NMOE_GU_TILE), gdn(NMOE_EXPERTS, NMOE_HIDDEN / NMOE_DN_TILE);
    if (bf)
        hipLaunchKernelGGL((nmoe_grouped_gateup_kernel<BITS, 1>), ggu, dim3(256), 0, s, pack,
                           (const uint16_t *)ctx->g_xhi, (const uint16_t *)ctx->g_xlo, (const float *)ctx->g_xs,
                           (const uint32_t *)ctx->g_perm, (const uint32_t *)ctx->g_offsets, k, ctx->g_ahi,
                           ctx->g_alo, ctx->g_as);
    else
        hipLaunchKernelGGL((nmoe_grouped_gateup_kernel<BITS, 2>), ggu, dim3(256), 0, s, pack,
                           (const uint16_t *)ctx->g_xhi, (const uint16_t *)ctx->g_xlo, (const float *)ctx->g_xs,
                           (const uint32_t *)ctx->g_perm, (const uint32_t *)ctx->g_offsets, k, ctx->g_ahi,
                           ctx->g_alo, ctx->g_as);
    hipLaunchKernelGGL((nmoe_grouped_down_kernel<BITS>), gdn, dim3(256), 0, s, pack, (const uint16_t *)ctx->g_ahi,
                       (const uint16_t *)ctx->g_alo, (const float *)ctx->g_as, (const uint32_t *)ctx->g_perm,
                       (const uint32_t *)ctx->g_offsets, ctx->g_y);
    hipLaunchKernelGGL(nmoe_grouped_combine_kernel, dim3(NMOE_HIDDEN / 256, ntok), dim3(256), 0, s,
                       (const float *)ctx->g_y, idx, w, k, h_mid, shared_out, shared_gate_raw, out);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? NMOE_HIP_OK : nmoe_hip_check(ctx, e, "grouped expert launch");
}

extern "C" int nmoe_grouped_experts(nmoe_hip_ctx *ctx, int bits, const uint8_t *pack, const void *x, int x_dtype,
                                    int ntok, int k, const uint32_t *idx, const float *w, const float *h_mid,
                                    const float *shared_out, const float *shared_gate_raw, float *out,
                                    hipStream_t s) {
    if (bits == 4)
        return nmoe_grouped_run<4>(ctx, pack, x, x_dtype, ntok, k, idx, w, h_mid, shared_out, shared_gate_raw, out,
                                   s);
    return nmoe_grouped_run<2>(ctx, pack, x, x_dtype, ntok, k, idx, w, h_mid, shared_out, shared_gate_raw, out, s);
}
