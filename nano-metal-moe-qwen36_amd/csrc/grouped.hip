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
    /* 0x43004300 in a VGPR: (x & mask) | c is then one v_and_or_b32 with
     * the mask in an SGPR (a VOP3 of gfx9 takes no literal) */
    uint32_t c;
    asm("v_mov_b32 %0, 0x43004300" : "=v"(c));
    if (BITS == 4) {
        b0.x = (w0 & 0x000F000Fu) | c;
        b0.y = ((w0 >> 4) & 0x000F000Fu) | c;
        b0.z = ((w0 >> 8) & 0x000F000Fu) | c;
        b0.w = ((w0 >> 12) & 0x000F000Fu) | c;
        b1.x = (w1 & 0x000F000Fu) | c;
        b1.y = ((w1 >> 4) & 0x000F000Fu) | c;
        b1.z = ((w1 >> 8) & 0x000F000Fu) | c;
        b1.w = ((w1 >> 12) & 0x000F000Fu) | c;
    } else {
        b0.x = (w0 & 0x00030003u) | c;
        b0.y = ((w0 >> 2) & 0x00030003u) | c;
        b0.z = ((w0 >> 4) & 0x00030003u) | c;
        b0.w = ((w0 >> 6) & 0x00030003u) | c;
        b1.x = ((w0 >> 8) & 0x00030003u) | c;
        b1.y = ((w0 >> 10) & 0x00030003u) | c;
        b1.z = ((w0 >> 12) & 0x00030003u) | c;
        b1.w = ((w0 >> 14) & 0x00030003u) | c;
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

/* ------------------------------------------------------------ stage ring */

/* Both GEMMs stream one 64-deep K group per step through a ring of
 * NMOE_NS LDS stages, filled by direct global->LDS loads
 * (global_load_lds_dwordx4: lane l of a wavefront writes bytes 16l..16l+15
 * of the instruction's 1 KB), so a group is requested NMOE_NS - 1 steps
 * before it is multiplied.  A stage holds
 *   - the A rows of the group: PL planes of 64 rows x 64 bf16 (128 B); the
 *     16-byte chunk c of row r sits at slot c ^ ((r >> 1) & 7), so the 16
 *     rows of one ds_read_b128 pass cover all 64 banks;
 *   - the codes of the tile's weight rows for the group: rows of 32 B (q4,
 *     whose two 16-byte halves swap on rows with bit 3 set, making the
 *     ds_read_b64 of 16 rows x 2 lanes conflict-free) or 16 B (q2).
 * Each stage is a __shared__ variable of its own: the compiler then tells
 * the stages' direct loads apart and a read of one stage does not wait for
 * the loads still in flight into the others. */
#define NMOE_NS 4

typedef __attribute__((address_space(3))) void nmoe_lds_void;

template <int PL, int CW>
struct nmoe_stage {
    uint4 a[PL][NMOE_MCHUNK * 8];
    uint32_t b[CW];
};

/* Instruction j (rows 8j..8j+7) of one A plane: src_row is this lane's row
 * (8j + lane / 8) pointer at the group's first column. */
__device__ __forceinline__ void nmoe_stage_rows(uint4 *plane, const uint16_t *src_row, int j, int lane) {
    const int r = 8 * j + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    __builtin_amdgcn_global_load_lds((const void *)(src_row + 8 * c), (nmoe_lds_void *)(plane + 64 * j), 16, 0, 0);
}

/* MFMA A operand (the lane's two 8-element chunks 2kb, 2kb+1) of row r. */
__device__ __forceinline__ void nmoe_stage_operand(const uint4 *plane, int r, int kb, uint4 &a0, uint4 &a1) {
    const int h = (r >> 1) & 7;
    a0 = plane[8 * r + ((2 * kb) ^ h)];
    a1 = plane[8 * r + ((2 * kb + 1) ^ h)];
}

/* Code instructions per wavefront and stage: one 1-KB instruction (16 B a
 * lane) for q4; two 256-byte instructions (4 B a lane) for q2, whose
 * stage is half the size, so every wavefront issues the same number of
 * loads and the ring waits are compile-time constants. */
template <int BITS>
struct nmoe_code_ins {
    static constexpr int PER_WAVE = BITS == 4 ? 1 : 2;
    static constexpr int BYTES = BITS == 4 ? 1024 : 256;
};

/* Instruction j of the codes of one group g: stage rows are weight rows
 * base + row * wpr words. */
template <int BITS>
__device__ __forceinline__ void nmoe_stage_codes(uint32_t *stage, const uint32_t *base, int wpr, int g, int j,
                                                 int lane) {
    if (BITS == 4) {
        /* rows 32j + lane / 2, half lane % 2 (swapped on rows with bit 3 set) */
        const int row = 32 * j + (lane >> 1);
        const int half = (lane & 1) ^ ((row >> 3) & 1);
        __builtin_amdgcn_global_load_lds((const void *)(base + (size_t)row * wpr + 8 * g + 4 * half),
                                         (nmoe_lds_void *)(stage + 256 * j), 16, 0, 0);
    } else {
        /* rows 16j + lane / 4, word lane % 4 */
        const int row = 16 * j + (lane >> 2);
        __builtin_amdgcn_global_load_lds((const void *)(base + (size_t)row * wpr + 4 * g + (lane & 3)),
                                         (nmoe_lds_void *)(stage + 64 * j), 4, 0, 0);
    }
}

/* The lane's code words of stage row r: q4 words 2kb, 2kb+1; q2 word kb. */
template <int BITS>
__device__ __forceinline__ void nmoe_stage_code_words(const uint32_t *stage, int r, int kb, uint32_t &w0,
                                                      uint32_t &w1) {
    if (BITS == 4) {
        /* written as an index XOR: the compiler then still knows which
         * stage the read belongs to */
        const uint2 *rowp = (const uint2 *)(stage + 8 * r);
        const uint2 v = rowp[kb ^ (2 * ((r >> 3) & 1))];
        w0 = v.x;
        w1 = v.y;
    } else {
        w0 = stage[4 * r + kb];
        w1 = 0;
    }
}

/* Ring barrier: this wavefront's loads of the stage about to be used are
 * complete (vmcnt <= N: only later stages still in flight) and its LDS
 * accesses are done (lgkmcnt 0), then all wavefronts meet.  A bare
 * s_barrier: the usual __syncthreads() fence would wait for every load in
 * flight, the later stages included. */
template <int N>
__device__ __forceinline__ void nmoe_ring_barrier() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
    asm volatile("s_barrier" ::: "memory");
}

/* The barrier before group g of G, for a wavefront that issues L loads per
 * group: groups g+1 and g+2 may still be in flight. */
template <int L, int G>
__device__ __forceinline__ void nmoe_ring_step_barrier(int g) {
    if (g + 2 < G)
        nmoe_ring_barrier<2 * L>();
    else if (g + 1 < G)
        nmoe_ring_barrier<L>();
    else
        nmoe_ring_barrier<0>();
}

/* Runs step(g, stage, issue_ahead) over the G groups: the loop body issues
 * group g + NS - 1 unconditionally (a load issued under a runtime condition
 * makes the compiler wait for every stage), the last NS - 1 steps issue
 * nothing. */
template <int G, typename Step>
__device__ __forceinline__ void nmoe_ring_run(Step step) {
    static_assert(G % NMOE_NS == 0, "whole ring turns");
    constexpr int MAIN = G - NMOE_NS; /* steps in the loop */
#pragma unroll 1
    for (int g = 0; g < MAIN; g += NMOE_NS) {
        step(g, 0, true);
        step(g + 1, 1, true);
        step(g + 2, 2, true);
        step(g + 3, 3, true);
    }
    step(MAIN, 0, true);
    step(MAIN + 1, 1, false);
    step(MAIN + 2, 2, false);
    step(MAIN + 3, 3, false);
}

template <int N>
__device__ __forceinline__ void nmoe_wait_vm() {
    /* s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt[3:0] | vmcnt[5:4] << 14,
     * expcnt and lgkmcnt left at their maxima) */
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

/* ------------------------------------------------------------ gate/up */

#define NMOE_GU_ROWS 128 /* gate rows (and up rows) per block: 16 per wavefront */

/* Expert blockIdx.x, gate and up rows 128 * blockIdx.y .. +127 (one pair of
 * down-K groups): act rows of all the expert's entries, 64 entries per
 * pass.  Eight wavefronts, two per SIMD; wavefront w owns gate and up rows
 * 16w..16w+15 of the tile as one MFMA column block each, over four 16-entry
 * row blocks, so a lane holds gate and up of the same (entry, row).
 *
 * y = sum_g s_g P_g + sum_g (b_g - 128 s_g) xs_g with P_g the MFMA product
 * of the group's A rows and the codes as bf16(128 + q); the second sum runs
 * first, on the fp32 matrix cores. */
template <int BITS, int XPL>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
nmoe_grouped_gateup_kernel(const uint8_t *pack, const uint16_t *xhi, const uint16_t *xlo, const float *xs,
                           const uint32_t *perm, const uint32_t *offsets, int k, uint16_t *ahi, uint16_t *alo,
                           float *as) {
    using Q = nmoe_q<BITS>;
    using L = nmoe_layout<BITS>;
    constexpr int G = NMOE_HIDDEN / NMOE_GROUP; /* 32 groups */
    constexpr int NT = NMOE_GU_ROWS;
    constexpr int WPG = BITS == 4 ? 8 : 4;
    using CI = nmoe_code_ins<BITS>;
    constexpr int CPM = NT * WPG * 4 / CI::BYTES; /* code instructions per matrix: 4 (q4) / 8 (q2) */
    __shared__ uint16_t s_sb[4][NT][G];         /* gate s, gate b, up s, up b */
    typedef nmoe_stage<XPL, 2 * NT * WPG> Stage;
    __shared__ Stage s_st0, s_st1, s_st2, s_st3;
    auto stage = [&](int st) -> Stage & { return st == 0 ? s_st0 : st == 1 ? s_st1 : st == 2 ? s_st2 : s_st3; };
    __shared__ uint32_t s_tok[NMOE_MCHUNK];
    __shared__ float s_as[8][NMOE_MCHUNK];
    const int e = blockIdx.x, nt = blockIdx.y;
    const uint32_t p0 = offsets[e], n = offsets[e + 1] - p0;
    if (n == 0) return;
    const int tid = threadIdx.x, lane = tid & 63, col = lane & 15, kb = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint8_t *ex = pack + (size_t)e * L::expert_size;
    for (int i = tid; i < 4 * NT * G / 8; i += 512) {
        const int arr = i / (NT * G / 8), j = i % (NT * G / 8);
        const uint32_t so = arr == 0 ? L::gate_s : arr == 1 ? L::gate_b : arr == 2 ? L::up_s : L::up_b;
        ((uint4 *)&s_sb[arr][0][0])[j] = ((const uint4 *)(ex + so + (size_t)nt * NT * G * 2))[j];
    }
    const int rt = 16 * wave + col; /* this lane's tile row */
    /* this wavefront's code instructions CI::PER_WAVE * wave + i all fall in
     * matrix cmat (gate for wavefronts 0-3, up for 4-7) */
    const int cmat = wave >> 2;
    const uint32_t *cbase = (const uint32_t *)(ex + (cmat == 0 ? L::gate_w : L::up_w)) + (size_t)nt * NT * Q::WPR_G;

    for (uint32_t m0 = 0; m0 < n; m0 += NMOE_MCHUNK) {
        if (tid < NMOE_MCHUNK) s_tok[tid] = perm[p0 + min(m0 + tid, n - 1)] / (uint32_t)k;
        __syncthreads();
        const int nb = (int)min((n - m0 + 15) / 16, 4u);
        /* this lane's A row for instruction `wave`: entry 8 wave + lane / 8 */
        const uint32_t tsrc = s_tok[8 * wave + (lane >> 3)];
        const uint16_t *srow[XPL];
        srow[0] = xhi + (size_t)tsrc * NMOE_HIDDEN;
        if (XPL == 2) srow[XPL - 1] = xlo + (size_t)tsrc * NMOE_HIDDEN;
        auto issue = [&](int g, int st) {
#pragma unroll
            for (int pl = 0; pl < XPL; pl++) nmoe_stage_rows(stage(st).a[pl], srow[pl] + 64 * g, wave, lane);
#pragma unroll
            for (int i = 0; i < CI::PER_WAVE; i++)
                nmoe_stage_codes<BITS>(stage(st).b + cmat * NT * WPG, cbase, Q::WPR_G, g,
                                       (CI::PER_WAVE * wave + i) % CPM, lane);
        };
        nmoe_f32x4 acc[2][4];
        {
            /* all operand loads first (one memory round trip), then the MFMAs:
             * A lane = (entry col, group 4tq + kb), B lane = (row col, group 4tq + kb) */
            float xv[4][G / 4];
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                const float *xsr = xs + (size_t)s_tok[16 * mb + col] * G;
#pragma unroll
                for (int tq = 0; tq < G / 4; tq++) xv[mb][tq] = xsr[4 * tq + kb];
            }
#pragma unroll
            for (int mat = 0; mat < 2; mat++) {
                float cv[G / 4];
#pragma unroll
                for (int tq = 0; tq < G / 4; tq++) {
                    const float sc = nmoe_bf16f(s_sb[2 * mat][rt][4 * tq + kb]);
                    cv[tq] = nmoe_bf16f(s_sb[2 * mat + 1][rt][4 * tq + kb]) - 128.0f * sc;
                }
#pragma unroll
                for (int mb = 0; mb < 4; mb++) {
                    acc[mat][mb] = nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                    if (mb < nb)
#pragma unroll
                        for (int tq = 0; tq < G / 4; tq++)
                            acc[mat][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[mb][tq], cv[tq], acc[mat][mb], 0, 0, 0);
                }
            }
        }
        /* keep every operand load above out of the vmcnt ring below */
        nmoe_wait_vm<0>();
#pragma unroll
        for (int st = 0; st < NMOE_NS - 1; st++) issue(st, st);
        auto step = [&](int g, const int st, const bool ahead) {
            nmoe_ring_step_barrier<XPL + CI::PER_WAVE, G>(g);
            if (ahead) issue(g + NMOE_NS - 1, (st + NMOE_NS - 1) % NMOE_NS);
            uint4 bq[2][2];
            float sg[2];
#pragma unroll
            for (int mat = 0; mat < 2; mat++) {
                uint32_t w0, w1;
                /* kept apart: a read merged across the two matrices loses
                 * the stage it belongs to, and then waits for every stage */
                if (mat == 1) asm volatile("" ::: "memory");
                nmoe_stage_code_words<BITS>(stage(st).b + mat * NT * WPG, rt, kb, w0, w1);
                nmoe_codes_bf16<BITS>(w0, w1, bq[mat][0], bq[mat][1]);
                sg[mat] = nmoe_bf16f(s_sb[2 * mat][rt][g]);
            }
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                if (mb < nb) {
                    uint4 a[XPL][2];
#pragma unroll
                    for (int pl = 0; pl < XPL; pl++)
                        nmoe_stage_operand(stage(st).a[pl], 16 * mb + col, kb, a[pl][0], a[pl][1]);
#pragma unroll
                    for (int mat = 0; mat < 2; mat++) {
                        nmoe_f32x4 pp = nmoe_mfma16(a[0][0], bq[mat][0], nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f});
                        pp = nmoe_mfma16(a[0][1], bq[mat][1], pp);
                        if (XPL == 2) {
                            pp = nmoe_mfma16(a[XPL - 1][0], bq[mat][0], pp);
                            pp = nmoe_mfma16(a[XPL - 1][1], bq[mat][1], pp);
                        }
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[mat][mb][i] = __builtin_fmaf(sg[mat], pp[i], acc[mat][mb][i]);
                    }
                }
            }
        };
        nmoe_ring_run<G>(step);
        /* epilogue: act = SiLU(gate) * up as hi + lo bf16, in the down
         * kernel's operand order; group sums of act rows (a down group is
         * 64 act columns = wavefronts 0-3 or 4-7 of this tile) */
        {
            const int r = nt * NT + rt; /* act column */
            const int span = r >> 4;
            const int slot = nmoe_kperm_inv<BITS>(r & 15);
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t m = m0 + 16 * mb + 4 * kb + i;
                    const float av = nmoe_silu_dev(acc[0][mb][i]) * acc[1][mb][i];
                    const uint32_t h = nmoe_bf16_rne(av);
                    const uint32_t l = nmoe_bf16_rne(av - nmoe_bf16f(h));
                    float part = nmoe_bf16f(h) + nmoe_bf16f(l);
                    if (mb < nb && m < n) {
                        const size_t o = (size_t)(p0 + m) * NMOE_INTER + 16 * span + slot;
                        ahi[o] = (uint16_t)h;
                        alo[o] = (uint16_t)l;
                    }
                    part = nmoe_dpp_group_sum<16>(part); /* the 16 rows of this column block */
                    if (col == 0) s_as[wave][16 * mb + 4 * kb + i] = part;
                }
            }
        }
        __syncthreads();
        if (tid < 2 * NMOE_MCHUNK) {
            const int half = tid >> 6, row = tid & 63;
            const uint32_t m = m0 + row;
            if (m < n)
                as[(size_t)(p0 + m) * (NMOE_INTER / NMOE_GROUP) + 2 * nt + half] =
                    (s_as[4 * half][row] + s_as[4 * half + 1][row]) + (s_as[4 * half + 2][row] + s_as[4 * half + 3][row]);
        }
        __syncthreads();
    }
}

/* ------------------------------------------------------------ down */

#define NMOE_DN_ROWS 256 /* down rows per block: 32 per wavefront */

/* Expert blockIdx.x, down rows 256 * blockIdx.y .. +255: y[q][row] for all
 * the expert's entries q.  Eight wavefronts; wavefront w owns rows
 * 32w..32w+31 of the tile as two 16-row column blocks.  act enters as hi
 * and lo bf16 planes. */
template <int BITS>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
nmoe_grouped_down_kernel(const uint8_t *pack, const uint16_t *ahi, const uint16_t *alo, const float *as,
                         const uint32_t *perm, const uint32_t *offsets, float *y) {
    using Q = nmoe_q<BITS>;
    using L = nmoe_layout<BITS>;
    constexpr int G = NMOE_INTER / NMOE_GROUP; /* 8 groups */
    constexpr int WPG = BITS == 4 ? 8 : 4;
    using CI = nmoe_code_ins<BITS>;
    __shared__ uint16_t s_sb[2][NMOE_DN_ROWS][G];
    typedef nmoe_stage<2, NMOE_DN_ROWS * WPG> Stage;
    __shared__ Stage s_st0, s_st1, s_st2, s_st3;
    auto stage = [&](int st) -> Stage & { return st == 0 ? s_st0 : st == 1 ? s_st1 : st == 2 ? s_st2 : s_st3; };
    __shared__ uint32_t s_q[NMOE_MCHUNK]; /* the chunk's output slots */
    const int e = blockIdx.x, nt = blockIdx.y;
    const uint32_t p0 = offsets[e], n = offsets[e + 1] - p0;
    if (n == 0) return;
    const int tid = threadIdx.x, lane = tid & 63, col = lane & 15, kb = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint8_t *ex = pack + (size_t)e * L::expert_size;
    for (int i = tid; i < 2 * NMOE_DN_ROWS * G / 8; i += 512) {
        const int arr = i / (NMOE_DN_ROWS * G / 8), j = i % (NMOE_DN_ROWS * G / 8);
        ((uint4 *)&s_sb[arr][0][0])[j] =
            ((const uint4 *)(ex + (arr == 0 ? L::down_s : L::down_b) + (size_t)nt * NMOE_DN_ROWS * G * 2))[j];
    }
    const int rt0 = 32 * wave + col; /* tile row of column block nb: rt0 + 16 nb */
    const uint32_t *cbase = (const uint32_t *)(ex + L::down_w) + (size_t)nt * NMOE_DN_ROWS * Q::WPR_D;
    __syncthreads();
    for (uint32_t m0 = 0; m0 < n; m0 += NMOE_MCHUNK) {
        const int nb = (int)min((n - m0 + 15) / 16, 4u);
        if (tid < NMOE_MCHUNK) s_q[tid] = perm[p0 + min(m0 + tid, n - 1)]; /* visible after the first ring barrier */
        /* this lane's A row for instruction `wave`: act row p0 + m0 + 8 wave + lane / 8 */
        const uint32_t msrc = min(m0 + 8 * wave + (lane >> 3), n - 1);
        const uint16_t *srow[2] = {ahi + (size_t)(p0 + msrc) * NMOE_INTER, alo + (size_t)(p0 + msrc) * NMOE_INTER};
        auto issue = [&](int g, int st) {
#pragma unroll
            for (int pl = 0; pl < 2; pl++) nmoe_stage_rows(stage(st).a[pl], srow[pl] + 64 * g, wave, lane);
#pragma unroll
            for (int i = 0; i < CI::PER_WAVE; i++)
                nmoe_stage_codes<BITS>(stage(st).b, cbase, Q::WPR_D, g, CI::PER_WAVE * wave + i, lane);
        };
        nmoe_f32x4 acc[2][4];
        {
            float av[4][G / 4];
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                const float *asr = as + (size_t)(p0 + min(m0 + 16 * mb + col, n - 1)) * G;
#pragma unroll
                for (int tq = 0; tq < G / 4; tq++) av[mb][tq] = asr[4 * tq + kb];
            }
#pragma unroll
            for (int nb2 = 0; nb2 < 2; nb2++) {
                const int rr = rt0 + 16 * nb2;
                float cv[G / 4];
#pragma unroll
                for (int tq = 0; tq < G / 4; tq++) {
                    const float sc = nmoe_bf16f(s_sb[0][rr][4 * tq + kb]);
                    cv[tq] = nmoe_bf16f(s_sb[1][rr][4 * tq + kb]) - 128.0f * sc;
                }
#pragma unroll
                for (int mb = 0; mb < 4; mb++) {
                    acc[nb2][mb] = nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                    if (mb < nb)
#pragma unroll
                        for (int tq = 0; tq < G / 4; tq++)
                            acc[nb2][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mb][tq], cv[tq], acc[nb2][mb], 0, 0, 0);
                }
            }
        }
        nmoe_wait_vm<0>();
#pragma unroll
        for (int st = 0; st < NMOE_NS - 1; st++) issue(st, st);
        auto step = [&](int g, const int st, const bool ahead) {
            nmoe_ring_step_barrier<2 + CI::PER_WAVE, G>(g);
            if (ahead) issue(g + NMOE_NS - 1, (st + NMOE_NS - 1) % NMOE_NS);
            uint4 bq[2][2];
            float sg[2];
#pragma unroll
            for (int nb2 = 0; nb2 < 2; nb2++) {
                uint32_t w0, w1;
                nmoe_stage_code_words<BITS>(stage(st).b, rt0 + 16 * nb2, kb, w0, w1);
                nmoe_codes_bf16<BITS>(w0, w1, bq[nb2][0], bq[nb2][1]);
                sg[nb2] = nmoe_bf16f(s_sb[0][rt0 + 16 * nb2][g]);
            }
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                if (mb < nb) {
                    uint4 h0, h1, l0, l1;
                    nmoe_stage_operand(stage(st).a[0], 16 * mb + col, kb, h0, h1);
                    nmoe_stage_operand(stage(st).a[1], 16 * mb + col, kb, l0, l1);
#pragma unroll
                    for (int nb2 = 0; nb2 < 2; nb2++) {
                        nmoe_f32x4 pp = nmoe_mfma16(h0, bq[nb2][0], nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f});
                        pp = nmoe_mfma16(h1, bq[nb2][1], pp);
                        pp = nmoe_mfma16(l0, bq[nb2][0], pp);
                        pp = nmoe_mfma16(l1, bq[nb2][1], pp);
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[nb2][mb][i] = __builtin_fmaf(sg[nb2], pp[i], acc[nb2][mb][i]);
                    }
                }
            }
        };
        nmoe_ring_run<G>(step);
#pragma unroll
        for (int nb2 = 0; nb2 < 2; nb2++) {
            const int r = nt * NMOE_DN_ROWS + rt0 + 16 * nb2;
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t m = m0 + 16 * mb + 4 * kb + i;
                    if (mb < nb && m < n) y[(size_t)s_q[m - m0] * NMOE_HIDDEN + r] = acc[nb2][mb][i];
                }
            }
        }
        __syncthreads(); /* the stage ring and s_q are reused by the next chunk */
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
    const dim3 ggu(NMOE_EXPERTS, NMOE_INTER / NMOE_GU_ROWS), gdn(NMOE_EXPERTS, NMOE_HIDDEN / NMOE_DN_ROWS);
    if (bf)
        hipLaunchKernelGGL((nmoe_grouped_gateup_kernel<BITS, 1>), ggu, dim3(512), 0, s, pack,
                           (const uint16_t *)ctx->g_xhi, (const uint16_t *)ctx->g_xlo, (const float *)ctx->g_xs,
                           (const uint32_t *)ctx->g_perm, (const uint32_t *)ctx->g_offsets, k, ctx->g_ahi,
                           ctx->g_alo, ctx->g_as);
    else
        hipLaunchKernelGGL((nmoe_grouped_gateup_kernel<BITS, 2>), ggu, dim3(512), 0, s, pack,
                           (const uint16_t *)ctx->g_xhi, (const uint16_t *)ctx->g_xlo, (const float *)ctx->g_xs,
                           (const uint32_t *)ctx->g_perm, (const uint32_t *)ctx->g_offsets, k, ctx->g_ahi,
                           ctx->g_alo, ctx->g_as);
    hipLaunchKernelGGL((nmoe_grouped_down_kernel<BITS>), gdn, dim3(512), 0, s, pack, (const uint16_t *)ctx->g_ahi,
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
