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

/* A rows of one 64-deep group reach LDS by direct global->LDS loads
 * (global_load_lds_dwordx4: lane l of a wavefront writes bytes 16l..16l+15
 * of the instruction's 1 KB), into a ring of NMOE_NS stages, so a group's
 * rows are requested NMOE_NS - 1 groups before they are multiplied.  A
 * stage row is 64 bf16 = 8 chunks of 16 bytes; chunk c of row r sits at
 * slot c ^ (r & 7), so the 16 rows one MFMA operand read touches spread
 * over the banks.  The codes of the weight rows go through a register ring
 * of the same depth. */
#define NMOE_NS 4

typedef __attribute__((address_space(3))) void nmoe_lds_void;

/* One ring stage: the activation rows of a group (PL planes of 64 rows x
 * 64 bf16) and the codes of the tile's weight rows for that group.  Each
 * stage is a __shared__ variable of its own: the compiler then tells the
 * stages' direct loads apart and a read of one stage does not wait for
 * the loads still in flight into the others. */
template <int PL, int CW>
struct nmoe_stage {
    uint4 a[PL][NMOE_MCHUNK * 8];
    uint32_t b[CW];
};

/* Issue the direct loads of one stage: `nins` 1-KB instructions per
 * wavefront; instruction j of plane pl covers stage rows 8j..8j+7. */
__device__ __forceinline__ void nmoe_stage_rows(uint4 *stage, const uint16_t *src_row0, const uint16_t *src_row1,
                                                int j0, int lane) {
    /* rows 8 j0 + (lane >> 3) and 8 (j0 + 1) + (lane >> 3): source row
     * pointers already include the group's column offset */
    const int slot = lane & 7;
    const int r0 = 8 * j0 + (lane >> 3), r1 = r0 + 8;
    const int c0 = slot ^ (r0 & 7), c1 = slot ^ (r1 & 7);
    __builtin_amdgcn_global_load_lds((const void *)(src_row0 + 8 * c0), (nmoe_lds_void *)(stage + 64 * j0), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void *)(src_row1 + 8 * c1), (nmoe_lds_void *)(stage + 64 * (j0 + 1)), 16, 0, 0);
}

/* MFMA A operand (two slices) of stage row r, lane k-block kb. */
__device__ __forceinline__ void nmoe_stage_operand(const uint4 *stage, int r, int kb, uint4 &a0, uint4 &a1) {
    a0 = stage[8 * r + ((2 * kb) ^ (r & 7))];
    a1 = stage[8 * r + ((2 * kb + 1) ^ (r & 7))];
}

/* Direct loads of one group's codes of `rows` weight rows (starting at
 * global row pointer base + row * wpr words, group g) into a stage of
 * [rows][wpg] words; wpg = 8 (q4) or 4 (q2) words = 32 / 16 bytes per row.
 * Instruction j of this wavefront covers 1 KB of the stage. */
template <int BITS>
__device__ __forceinline__ void nmoe_stage_codes(uint32_t *stage, const uint32_t *base, int wpr, int g, int j,
                                                 int lane) {
    constexpr int WPG = BITS == 4 ? 8 : 4;
    const int byte = 1024 * j + 16 * lane;
    const int row = byte / (4 * WPG), w = (byte % (4 * WPG)) / 4;
    __builtin_amdgcn_global_load_lds((const void *)(base + (size_t)row * wpr + WPG * g + w),
                                     (nmoe_lds_void *)(stage + 256 * j), 16, 0, 0);
}

/* The lane's code words of stage row r: q4 words 2kb, 2kb+1; q2 word kb. */
template <int BITS>
__device__ __forceinline__ void nmoe_stage_code_words(const uint32_t *stage, int r, int kb, uint32_t &w0,
                                                      uint32_t &w1) {
    if (BITS == 4) {
        const uint2 v = *(const uint2 *)(stage + 8 * r + 2 * kb);
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

template <int N>
__device__ __forceinline__ void nmoe_wait_vm() {
    /* s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt[3:0] | vmcnt[5:4] << 14,
     * expcnt and lgkmcnt left at their maxima) */
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

/* Expert blockIdx.x, gate/up rows 128 * blockIdx.y .. +127 (both
 * matrices): act rows of all the expert's entries.  Wave w owns gate and up
 * rows 32w..32w+31 of the tile as two 16-row MFMA column blocks each, over
 * four 16-row blocks of entries: a lane holds gate and up of the same
 * (entry, row). */
template <int BITS, int XPL>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
nmoe_grouped_gateup_kernel(const uint8_t *pack, const uint16_t *xhi, const uint16_t *xlo, const float *xs,
                           const uint32_t *perm, const uint32_t *offsets, int k, uint16_t *ahi, uint16_t *alo,
                           float *as) {
    using Q = nmoe_q<BITS>;
    using L = nmoe_layout<BITS>;
    constexpr int G = NMOE_HIDDEN / NMOE_GROUP; /* 32 groups */
    constexpr int NT = 2 * NMOE_GU_TILE;        /* 128 rows per matrix per block */
    constexpr int WPG = BITS == 4 ? 8 : 4;      /* code words per row per group */
    constexpr int BI = 2 * NT * WPG * 4 / 1024 / 4; /* code instructions per wavefront per stage: 2 (q4) / 1 (q2) */
    constexpr int LPG = 2 * XPL + BI;           /* loads per group per wavefront */
    __shared__ uint16_t s_sb[4][NT][G];         /* gate s, gate b, up s, up b */
    typedef nmoe_stage<XPL, 2 * NT * WPG> Stage;
    __shared__ Stage s_st0, s_st1, s_st2, s_st3;
    auto stage = [&](int st) -> Stage & { return st == 0 ? s_st0 : st == 1 ? s_st1 : st == 2 ? s_st2 : s_st3; };
    __shared__ uint32_t s_tok[NMOE_MCHUNK];
    __shared__ float s_as[4][NMOE_MCHUNK];
    const int e = blockIdx.x, nt = blockIdx.y;
    const uint32_t p0 = offsets[e], n = offsets[e + 1] - p0;
    if (n == 0) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, kb = lane >> 4;
    const uint8_t *ex = pack + (size_t)e * L::expert_size;
    for (int i = tid; i < 4 * NT * G / 8; i += 256) {
        const int arr = i / (NT * G / 8), j = i % (NT * G / 8);
        const uint32_t so = arr == 0 ? L::gate_s : arr == 1 ? L::gate_b : arr == 2 ? L::up_s : L::up_b;
        ((uint4 *)&s_sb[arr][0][0])[j] = ((const uint4 *)(ex + so + (size_t)nt * NT * G * 2))[j];
    }
    const int rt0 = 32 * wave + col; /* tile row of column block nb2: rt0 + 16 nb2 */
    const uint32_t *wbase[2] = {(const uint32_t *)(ex + L::gate_w) + (size_t)nt * NT * Q::WPR_G,
                                (const uint32_t *)(ex + L::up_w) + (size_t)nt * NT * Q::WPR_G};

    for (uint32_t m0 = 0; m0 < n; m0 += NMOE_MCHUNK) {
        if (tid < NMOE_MCHUNK) s_tok[tid] = perm[p0 + min(m0 + tid, n - 1)] / (uint32_t)k;
        __syncthreads();
        const int nb = (int)min((n - m0 + 15) / 16, 4u);
        /* this lane's two stage rows (instructions 2w, 2w+1) */
        const uint16_t *srow[XPL][2];
#pragma unroll
        for (int jj = 0; jj < 2; jj++) {
            const uint32_t t = s_tok[8 * (2 * wave + jj) + (lane >> 3)];
            srow[0][jj] = xhi + (size_t)t * NMOE_HIDDEN;
            if (XPL == 2) srow[XPL - 1][jj] = xlo + (size_t)t * NMOE_HIDDEN;
        }
        auto issue = [&](int g, int st) {
#pragma unroll
            for (int pl = 0; pl < XPL; pl++)
                nmoe_stage_rows(stage(st).a[pl], srow[pl][0] + 64 * g, srow[pl][1] + 64 * g, 2 * wave, lane);
            /* codes: 2 matrices x NT rows x WPG words = 8 (q4) / 4 (q2) KB */
#pragma unroll
            for (int i = 0; i < BI; i++) {
                const int j = BI * wave + i;                 /* 0 .. 4 BI - 1 */
                const int mat = j / (2 * BI), jm = j % (2 * BI); /* instruction within the matrix */
                nmoe_stage_codes<BITS>(stage(st).b + mat * NT * WPG, wbase[mat], Q::WPR_G, g, jm, lane);
            }
        };
        /* sum_g (b_g - 128 s_g) xs_g on the fp32 cores: A lane = (entry col,
         * group 4tq + kb), B lane = (row col, group 4tq + kb) */
        nmoe_f32x4 acc[2][2][4];
        {
            /* all operand loads first (one memory round trip), then the MFMAs */
            float xv[4][G / 4];
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                const float *xsr = xs + (size_t)s_tok[16 * mb + col] * G;
#pragma unroll
                for (int tq = 0; tq < G / 4; tq++) xv[mb][tq] = xsr[4 * tq + kb];
            }
#pragma unroll
            for (int mat = 0; mat < 2; mat++)
#pragma unroll
                for (int nb2 = 0; nb2 < 2; nb2++) {
                    const int rr = rt0 + 16 * nb2;
                    float cv[G / 4];
#pragma unroll
                    for (int tq = 0; tq < G / 4; tq++) {
                        const float sc = nmoe_bf16f(s_sb[2 * mat][rr][4 * tq + kb]);
                        cv[tq] = nmoe_bf16f(s_sb[2 * mat + 1][rr][4 * tq + kb]) - 128.0f * sc;
                    }
#pragma unroll
                    for (int mb = 0; mb < 4; mb++) {
                        acc[mat][nb2][mb] = nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                        if (mb < nb)
#pragma unroll
                            for (int tq = 0; tq < G / 4; tq++)
                                acc[mat][nb2][mb] =
                                    __builtin_amdgcn_mfma_f32_16x16x4f32(xv[mb][tq], cv[tq], acc[mat][nb2][mb], 0, 0, 0);
                    }
                }
        }
        /* keep every operand load above out of the vmcnt ring below */
        nmoe_wait_vm<0>();
#pragma unroll
        for (int st = 0; st < NMOE_NS - 1; st++) issue(st, st);
        auto step = [&](int g, const int st) {
            /* group g's stage: groups g+1, g+2 may still be in flight */
            if (g + 2 < G)
                nmoe_ring_barrier<2 * LPG>();
            else if (g + 1 < G)
                nmoe_ring_barrier<LPG>();
            else
                nmoe_ring_barrier<0>();
            if (g + NMOE_NS - 1 < G) issue(g + NMOE_NS - 1, (st + NMOE_NS - 1) % NMOE_NS);
            uint4 bq[2][2][2];
            float sg[2][2];
#pragma unroll
            for (int mat = 0; mat < 2; mat++)
#pragma unroll
                for (int nb2 = 0; nb2 < 2; nb2++) {
                    uint32_t w0, w1;
                    /* kept apart: a read merged across the two matrices
                     * loses the stage it belongs to, and then waits for
                     * every stage's loads */
                    if (mat == 1 && nb2 == 0) asm volatile("" ::: "memory");
                    nmoe_stage_code_words<BITS>(stage(st).b + mat * NT * WPG, rt0 + 16 * nb2, kb, w0, w1);
                    nmoe_codes_bf16<BITS>(w0, w1, bq[mat][nb2][0], bq[mat][nb2][1]);
                    sg[mat][nb2] = nmoe_bf16f(s_sb[2 * mat][rt0 + 16 * nb2][g]);
                }
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                if (mb < nb) {
                    uint4 a[XPL][2];
#pragma unroll
                    for (int pl = 0; pl < XPL; pl++)
                        nmoe_stage_operand(stage(st).a[pl], 16 * mb + col, kb, a[pl][0], a[pl][1]);
#pragma unroll
                    for (int mat = 0; mat < 2; mat++)
#pragma unroll
                        for (int nb2 = 0; nb2 < 2; nb2++) {
                            nmoe_f32x4 pp = nmoe_mfma16(a[0][0], bq[mat][nb2][0], nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f});
                            pp = nmoe_mfma16(a[0][1], bq[mat][nb2][1], pp);
                            if (XPL == 2) {
                                pp = nmoe_mfma16(a[XPL - 1][0], bq[mat][nb2][0], pp);
                                pp = nmoe_mfma16(a[XPL - 1][1], bq[mat][nb2][1], pp);
                            }
#pragma unroll
                            for (int i = 0; i < 4; i++)
                                acc[mat][nb2][mb][i] = __builtin_fmaf(sg[mat][nb2], pp[i], acc[mat][nb2][mb][i]);
                        }
                }
            }
        };
#pragma unroll 1
        for (int g = 0; g < G; g += NMOE_NS) {
            step(g, 0);
            step(g + 1, 1);
            step(g + 2, 2);
            step(g + 3, 3);
        }
        /* epilogue: act = SiLU(gate) * up as hi + lo bf16, in the down
         * kernel's operand order; group sums of act rows (a down group is
         * 64 act columns = waves 0-1 or 2-3 of this tile) */
#pragma unroll
        for (int nb2 = 0; nb2 < 2; nb2++) {
            const int r = nt * NT + rt0 + 16 * nb2; /* act column */
            const int span = r >> 4;
            const int slot = nmoe_kperm_inv<BITS>(r & 15);
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t m = m0 + 16 * mb + 4 * kb + i;
                    const float av = nmoe_silu_dev(acc[0][nb2][mb][i]) * acc[1][nb2][mb][i];
                    const uint32_t h = nmoe_bf16_rne(av);
                    const uint32_t l = nmoe_bf16_rne(av - nmoe_bf16f(h));
                    float part = nmoe_bf16f(h) + nmoe_bf16f(l);
                    if (mb < nb && m < n) {
                        const size_t o = (size_t)(p0 + m) * NMOE_INTER + 16 * span + slot;
                        ahi[o] = (uint16_t)h;
                        alo[o] = (uint16_t)l;
                    }
                    part = nmoe_dpp_group_sum<16>(part); /* the 16 rows of this column block */
                    if (col == 0) {
                        if (nb2 == 0)
                            s_as[wave][16 * mb + 4 * kb + i] = part;
                        else
                            s_as[wave][16 * mb + 4 * kb + i] += part;
                    }
                }
            }
        }
        __syncthreads();
        if (tid < 2 * NMOE_MCHUNK) {
            const int half = tid >> 6, row = tid & 63;
            const uint32_t m = m0 + row;
            if (m < n)
                as[(size_t)(p0 + m) * (NMOE_INTER / NMOE_GROUP) + 2 * nt + half] =
                    s_as[2 * half][row] + s_as[2 * half + 1][row];
        }
        __syncthreads();
    }
}

/* ------------------------------------------------------------ down */

#define NMOE_DN_ROWS 256 /* down rows per block: 64 per wave */

/* Expert blockIdx.x, down rows 256 * blockIdx.y .. +255: y[q][row] for all
 * the expert's entries q.  Wave w owns rows 64w..64w+63 of the tile as four
 * 16-row column blocks. */
template <int BITS>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
nmoe_grouped_down_kernel(const uint8_t *pack, const uint16_t *ahi, const uint16_t *alo, const float *as,
                         const uint32_t *perm, const uint32_t *offsets, float *y) {
    using Q = nmoe_q<BITS>;
    using L = nmoe_layout<BITS>;
    constexpr int G = NMOE_INTER / NMOE_GROUP; /* 8 groups */
    constexpr int WPG = BITS == 4 ? 8 : 4;
    constexpr int BI = NMOE_DN_ROWS * WPG * 4 / 1024 / 4; /* code instructions per wavefront per stage: 2 / 1 */
    constexpr int LPG = 4 + BI;                /* loads per group per wavefront: 2 planes x 2 + codes */
    __shared__ uint16_t s_sb[2][NMOE_DN_ROWS][G];
    typedef nmoe_stage<2, NMOE_DN_ROWS * WPG> Stage;
    __shared__ Stage s_st0, s_st1, s_st2, s_st3;
    __shared__ uint32_t s_q[NMOE_MCHUNK]; /* the chunk's output slots */
    auto stage = [&](int st) -> Stage & { return st == 0 ? s_st0 : st == 1 ? s_st1 : st == 2 ? s_st2 : s_st3; };
    const int e = blockIdx.x, nt = blockIdx.y;
    const uint32_t p0 = offsets[e], n = offsets[e + 1] - p0;
    if (n == 0) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, kb = lane >> 4;
    const uint8_t *ex = pack + (size_t)e * L::expert_size;
    for (int i = tid; i < 2 * NMOE_DN_ROWS * G / 8; i += 256) {
        const int arr = i / (NMOE_DN_ROWS * G / 8), j = i % (NMOE_DN_ROWS * G / 8);
        ((uint4 *)&s_sb[arr][0][0])[j] =
            ((const uint4 *)(ex + (arr == 0 ? L::down_s : L::down_b) + (size_t)nt * NMOE_DN_ROWS * G * 2))[j];
    }
    const int rt0 = 64 * wave + col;
    const uint32_t *wbase = (const uint32_t *)(ex + L::down_w) + (size_t)nt * NMOE_DN_ROWS * Q::WPR_D;
    __syncthreads();
    for (uint32_t m0 = 0; m0 < n; m0 += NMOE_MCHUNK) {
        const int nb = (int)min((n - m0 + 15) / 16, 4u);
        if (tid < NMOE_MCHUNK) s_q[tid] = perm[p0 + min(m0 + tid, n - 1)]; /* visible after the first ring barrier */
        /* this lane's two stage rows: act rows p0 + m0 + 8 (2w + jj) + lane / 8 */
        const uint16_t *srow[2][2];
#pragma unroll
        for (int jj = 0; jj < 2; jj++) {
            const uint32_t m = min(m0 + 8 * (2 * wave + jj) + (lane >> 3), n - 1);
            srow[0][jj] = ahi + (size_t)(p0 + m) * NMOE_INTER;
            srow[1][jj] = alo + (size_t)(p0 + m) * NMOE_INTER;
        }
        auto issue = [&](int g, int st) {
#pragma unroll
            for (int pl = 0; pl < 2; pl++)
                nmoe_stage_rows(stage(st).a[pl], srow[pl][0] + 64 * g, srow[pl][1] + 64 * g, 2 * wave, lane);
#pragma unroll
            for (int i = 0; i < BI; i++) nmoe_stage_codes<BITS>(stage(st).b, wbase, Q::WPR_D, g, BI * wave + i, lane);
        };
        nmoe_f32x4 acc[4][4];
        {
            float av[4][G / 4];
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                const float *asr = as + (size_t)(p0 + min(m0 + 16 * mb + col, n - 1)) * G;
#pragma unroll
                for (int tq = 0; tq < G / 4; tq++) av[mb][tq] = asr[4 * tq + kb];
            }
#pragma unroll
            for (int nb4 = 0; nb4 < 4; nb4++) {
                const int rr = rt0 + 16 * nb4;
                float cv[G / 4];
#pragma unroll
                for (int tq = 0; tq < G / 4; tq++) {
                    const float sc = nmoe_bf16f(s_sb[0][rr][4 * tq + kb]);
                    cv[tq] = nmoe_bf16f(s_sb[1][rr][4 * tq + kb]) - 128.0f * sc;
                }
#pragma unroll
                for (int mb = 0; mb < 4; mb++) {
                    acc[nb4][mb] = nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                    if (mb < nb)
#pragma unroll
                        for (int tq = 0; tq < G / 4; tq++)
                            acc[nb4][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mb][tq], cv[tq], acc[nb4][mb], 0, 0, 0);
                }
            }
        }
        nmoe_wait_vm<0>();
#pragma unroll
        for (int st = 0; st < NMOE_NS - 1; st++) issue(st, st);
        auto step = [&](int g, const int st) {
            if (g + 2 < G)
                nmoe_ring_barrier<2 * LPG>();
            else if (g + 1 < G)
                nmoe_ring_barrier<LPG>();
            else
                nmoe_ring_barrier<0>();
            if (g + NMOE_NS - 1 < G) issue(g + NMOE_NS - 1, (st + NMOE_NS - 1) % NMOE_NS);
            uint4 bq[4][2];
            float sg[4];
#pragma unroll
            for (int nb4 = 0; nb4 < 4; nb4++) {
                uint32_t w0, w1;
                nmoe_stage_code_words<BITS>(stage(st).b, rt0 + 16 * nb4, kb, w0, w1);
                nmoe_codes_bf16<BITS>(w0, w1, bq[nb4][0], bq[nb4][1]);
                sg[nb4] = nmoe_bf16f(s_sb[0][rt0 + 16 * nb4][g]);
            }
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                if (mb < nb) {
                    uint4 h0, h1, l0, l1;
                    nmoe_stage_operand(stage(st).a[0], 16 * mb + col, kb, h0, h1);
                    nmoe_stage_operand(stage(st).a[1], 16 * mb + col, kb, l0, l1);
#pragma unroll
                    for (int nb4 = 0; nb4 < 4; nb4++) {
                        nmoe_f32x4 pp = nmoe_mfma16(h0, bq[nb4][0], nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f});
                        pp = nmoe_mfma16(h1, bq[nb4][1], pp);
                        pp = nmoe_mfma16(l0, bq[nb4][0], pp);
                        pp = nmoe_mfma16(l1, bq[nb4][1], pp);
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[nb4][mb][i] = __builtin_fmaf(sg[nb4], pp[i], acc[nb4][mb][i]);
                    }
                }
            }
        };
        step(0, 0);
        step(1, 1);
        step(2, 2);
        step(3, 3);
        step(4, 0);
        step(5, 1);
        step(6, 2);
        step(7, 3);
#pragma unroll
        for (int nb4 = 0; nb4 < 4; nb4++) {
            const int r = nt * NMOE_DN_ROWS + rt0 + 16 * nb4;
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t m = m0 + 16 * mb + 4 * kb + i;
                    if (mb < nb && m < n) y[(size_t)s_q[m - m0] * NMOE_HIDDEN + r] = acc[nb4][mb][i];
                }
            }
        }
        __syncthreads(); /* the stage ring is reused by the next chunk */
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
    const dim3 ggu(NMOE_EXPERTS, NMOE_INTER / (2 * NMOE_GU_TILE)), gdn(NMOE_EXPERTS, NMOE_HIDDEN / NMOE_DN_ROWS);
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
