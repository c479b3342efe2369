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
 *   prep   one launch: D1/D2 dispatch (per-slice expert histograms, then
 *          offsets[257], the stable permutation perm[] of the entries
 *          q = t*k + s (ties by t, then s; entries whose index is outside
 *          the layer are left out) and the experts ranked by work), and X
 *          per token: x in the matrix-core operand order (bf16; fp32 input
 *          also gets a low plane x - bf16(x)) and its 32 group sums.
 *   G      per (expert, 128 gate and 128 up rows): Act = SwiGLU(X_e Wg^T,
 *          X_e Wu^T) for all of the expert's rows, as hi + lo bf16 planes,
 *          and the 8 group sums of each act row.
 *   Dn     per (expert, 256 down rows): Y_e = Act_e Wd^T -> Y[q][2048].
 *   C      per token: out = h_mid + sum_s w_s y_s in slot order
 *          (kernels.metal:1394-1423) (+ sigmoid(g) * shared).
 * (Tile rows as built with four-wavefront blocks; NMOE_GROUPED_NW=8 doubles
 * them.)
 *
 * Exactness on the matrix cores.  The dequantised weight is q*scale + bias
 * per group of 64 (math.m:206-234).  A bf16 weight would round q*scale, so
 * the cores multiply the integer codes instead, exactly: the code q is fed
 * as the bf16 value 128 + q (bit pattern 0x4300 | q, one and-or per two
 * codes), and
 *     sum_k w_k x_k = sum_g s_g P_g + sum_g (b_g - 128 s_g) xs_g,
 *     P_g = sum_{k in g} (128 + q_k) x_k,   xs_g = sum_{k in g} x_k,
 * with P_g from v_mfma_f32_16x16x32_bf16 (bf16 products are exact in fp32),
 * the s_g scaling applied per group in fp32, and the second sum over the
 * 32 (gate/up) groups from the same bf16 MFMA (xs as three exact bf16
 * parts; b and s are bf16), over the 8 (down) groups from
 * v_mfma_f32_16x16x4_f32.  x is
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

/* Dispatch blocks: one up to 1,024 entries (its histogram never leaves
 * LDS), else a power of two up to 64 so that a slice is at most four
 * 256-entry chunks (the ones a block multi-splits at once) while the
 * entries fit (65,536 of them).  Each block reads the others' histogram
 * words 16 slices at a time: one round up to 16,384 entries. */
#define NMOE_DISPATCH_MAX 64
#define NMOE_DISPATCH_READ 16
__host__ __device__ constexpr int nmoe_dispatch_blocks(int n) {
    if (n <= 1024) return 1;
    int nd = 2;
    while (nd < NMOE_DISPATCH_MAX && nd * 1024 < n) nd *= 2;
    return nd;
}
#define NMOE_MCHUNK 64 /* expert rows (entries) per pass: four 16-row MFMA blocks */
/* Wavefronts per gate/up and down block: 8 (one block a CU) or 4 (two). */
#ifndef NMOE_GROUPED_NW
#define NMOE_GROUPED_NW 4
#endif
/* The small form: an expert of at most NMOE_SMALL_PASS entries (batched
 * decode leaves most experts with a few) runs one pass of one 16-row block
 * whose ring steps take NMOE_SMALL_GPS groups at a time, so each weight row
 * is read 64 B a step instead of 32 B and the A stage holds 16 rows, not
 * 64.  Built with four-wavefront blocks (one A load per wavefront a step). */
#define NMOE_SMALL_PASS 16
#define NMOE_SMALL_GPS 2
__host__ __device__ constexpr bool nmoe_small_form(int nw) { return nw == 4; }
/* Gate (and up) rows per block of NW wavefronts: 32 a wavefront for bf16 x
 * (one A plane), 16 for fp32 x (hi + lo planes). */
__host__ __device__ constexpr int nmoe_gu_rows(int xpl, int nw) { return nw * 32 / xpl; }

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

/* The same by the hardware conversion (v_cvt_pk_bf16_f32, round to nearest
 * even), one instruction. */
__device__ __forceinline__ uint32_t nmoe_bf16_cvt(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

/* A raw buffer resource over p: base in scalar registers, range 2 GB (the
 * offsets used stay far inside the allocation), untyped access. */
__device__ __forceinline__ __amdgpu_buffer_rsrc_t nmoe_buffer(void *p) {
    return __builtin_amdgcn_make_buffer_rsrc(p, (short)0, 0x7fffffff, 0x00020000);
}

/* An LDS address as the direct global->LDS loads take it. */
typedef __attribute__((address_space(3))) void nmoe_lds_void;

/* Phase timeline of the grouped launches (NMOE_TIMELINE builds; tl NULL
 * otherwise): block b's words tl[4b .. 4b+3] = the real-time clock at its
 * start, once its inputs are ready (a down tile of the one-launch form:
 * after its wait; a routing block: its first wavefront's token routed,
 * before its stores; the dispatch block: its slice routed; else its start) and at its
 * end, and what it ran: entries << 32 | kind << 28 | die << 24 | expert
 * rank (or block) << 8 | tile (kind 1 gate/up, 2 down; of the preparation
 * launch 3 routing, 4 dispatch, 5 x planes).  One lane stores, with a
 * vector store. */
#define NMOE_GTL_START 0
#define NMOE_GTL_READY 1
#define NMOE_GTL_END 2
#define NMOE_GTL_INFO 3
__device__ __forceinline__ void nmoe_gtl_put(uint64_t *tl, int w, uint64_t v) {
    if constexpr (NMOE_TIMELINE) {
        if (tl != nullptr) {
            uint64_t *p = tl + 4 * (size_t)blockIdx.x + w;
            asm volatile("global_store_dwordx2 %0, %1, off" ::"v"(p), "v"(v) : "memory");
        }
    }
}
__device__ __forceinline__ void nmoe_gtl_stamp(uint64_t *tl, int w) {
    if constexpr (NMOE_TIMELINE)
        if (tl != nullptr) nmoe_gtl_put(tl, w, __builtin_amdgcn_s_memrealtime());
}
/* start and ready at a block's entry, end and what it ran at its exit */
__device__ __forceinline__ void nmoe_gtl_begin(uint64_t *tl) {
    if constexpr (NMOE_TIMELINE) {
        if (tl != nullptr && threadIdx.x == 0) {
            const uint64_t t = __builtin_amdgcn_s_memrealtime();
            nmoe_gtl_put(tl, NMOE_GTL_START, t);
            nmoe_gtl_put(tl, NMOE_GTL_READY, t);
        }
    }
}
__device__ __forceinline__ void nmoe_gtl_end(uint64_t *tl, int kind, const uint4 *rank, int es, int nt, int pl,
                                             int nrows) {
    if constexpr (NMOE_TIMELINE) {
        if (tl != nullptr && threadIdx.x == 0) {
            nmoe_gtl_stamp(tl, NMOE_GTL_END);
            const uint4 rk = rank[es];
            const uint32_t p0 = min(rk.y, (uint32_t)nrows), n = min(rk.z, (uint32_t)nrows - p0);
            const uint32_t work = n > (uint32_t)(pl * NMOE_MCHUNK) ? n : 0u;
            nmoe_gtl_put(tl, NMOE_GTL_INFO,
                         ((uint64_t)work << 32) | ((uint64_t)kind << 28) | ((uint64_t)nmoe_xcc_id() << 24) |
                             ((uint64_t)es << 8) | (uint64_t)nt);
        }
    }
}

/* end and kind of a preparation block (thread 0) */
__device__ __forceinline__ void nmoe_gtl_prep_end(uint64_t *tl, int kind) {
    if constexpr (NMOE_TIMELINE) {
        if (tl != nullptr && threadIdx.x == 0) {
            nmoe_gtl_stamp(tl, NMOE_GTL_END);
            nmoe_gtl_put(tl, NMOE_GTL_INFO,
                         (1ull << 32) | ((uint64_t)kind << 28) | ((uint64_t)nmoe_xcc_id() << 24) |
                             ((uint64_t)blockIdx.x << 8));
        }
    }
}

/* ------------------------------------------------------------ dispatch */

/* Where the dispatch reads the expert of entry q (token q / k, slot
 * q % k): idx, or, when the routing runs in the same launch (ROUTED), the
 * entry's tagged word (launch epoch << 32 | expert), written by its routing
 * wavefront and polled (bounded) until it carries this launch's epoch: no
 * count of routed entries to wait for and no second read of idx. */
struct nmoe_entry_src {
    const uint32_t *idx;
    int k;
    const uint64_t *tags;
    uint32_t epoch;
    uint32_t *sync;
    uint32_t spin;
};

__device__ __forceinline__ uint32_t nmoe_clamp_expert(uint32_t e) {
    return e < NMOE_EXPERTS ? e : (uint32_t)NMOE_EXPERTS; /* 256: left out */
}

/* A tagged entry word of this launch: polls (bounded; an expired wait sets
 * the status word and the word read last is used) from a first read w. */
__device__ __forceinline__ uint32_t nmoe_entry_tagged(const nmoe_entry_src &s, int q, uint64_t w) {
    uint32_t spins = 0;
    while (!nmoe_tag_is(w, s.epoch)) {
        __builtin_amdgcn_s_sleep(1);
        w = nmoe_ld_tagged(s.tags + q);
        if (++spins > s.spin) {
            __hip_atomic_store((nmoe_g32 *)(s.sync + NMOE_SYNC_STATUS), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
    }
    return nmoe_clamp_expert((uint32_t)w);
}

template <bool ROUTED>
__device__ __forceinline__ uint32_t nmoe_entry_expert(const nmoe_entry_src &s, int q) {
    if constexpr (ROUTED) return nmoe_entry_tagged(s, q, nmoe_ld_tagged(s.tags + q));
    return nmoe_clamp_expert(s.idx[(size_t)(q / s.k) * NMOE_MAX_K + (q % s.k)]);
}

#define NMOE_DISPATCH_PRE 4 /* chunks of a slice whose entries are read up front */

/* This thread's entries of the first NMOE_DISPATCH_PRE chunks of slice b
 * (256 past the slice's end), all first reads in flight together; read once
 * for both phases. */
template <bool ROUTED>
__device__ __forceinline__ void nmoe_dispatch_entries(const nmoe_entry_src &s, int ntok, int b, int nd, uint32_t *ev) {
    const int n = ntok * s.k, per = (n + nd - 1) / nd, q1 = min(n, (b + 1) * per);
    if constexpr (ROUTED) {
        uint64_t w[NMOE_DISPATCH_PRE];
#pragma unroll
        for (int j = 0; j < NMOE_DISPATCH_PRE; j++) {
            const int q = b * per + 256 * j + (int)threadIdx.x;
            w[j] = q < q1 ? nmoe_ld_tagged(s.tags + q) : 0ull;
        }
#pragma unroll
        for (int j = 0; j < NMOE_DISPATCH_PRE; j++) {
            const int q = b * per + 256 * j + (int)threadIdx.x;
            ev[j] = q < q1 ? nmoe_entry_tagged(s, q, w[j]) : (uint32_t)NMOE_EXPERTS;
        }
    } else {
#pragma unroll
        for (int j = 0; j < NMOE_DISPATCH_PRE; j++) {
            const int q = b * per + 256 * j + (int)threadIdx.x;
            ev[j] = q < q1 ? nmoe_entry_expert<false>(s, q) : (uint32_t)NMOE_EXPERTS;
        }
    }
}

/* The scatter's LDS counts: per chunk of the first NMOE_DISPATCH_PRE and
 * wavefront, the entries of each expert (then their first places), and
 * the experts' work buckets.  Cleared by nmoe_dispatch_count. */
struct nmoe_scatter_lds {
    uint32_t wc[NMOE_DISPATCH_PRE][4][NMOE_EXPERTS + 1];
    uint32_t bk[64];
    uint32_t wbk[4][64]; /* each wavefront's experts of each work bucket */
};

/* D1: h = expert histogram of entry slice b of nd (in LDS). */
template <bool ROUTED>
__device__ __forceinline__ void nmoe_dispatch_count(const nmoe_entry_src &s, int ntok, uint32_t *h, int b, int nd,
                                                    const uint32_t *ev, nmoe_scatter_lds &sl) {
    const int tid = threadIdx.x, n = ntok * s.k;
    const int per = (n + nd - 1) / nd;
    for (int i = tid; i <= NMOE_EXPERTS; i += 256) h[i] = 0;
    for (int i = tid; i < (int)(sizeof(sl) / 4); i += 256) (&sl.wc[0][0][0])[i] = 0;
    __syncthreads();
    const int q1 = min(n, (b + 1) * per);
#pragma unroll
    for (int j = 0; j < NMOE_DISPATCH_PRE; j++)
        if (b * per + 256 * j + tid < q1) atomicAdd(&h[ev[j]], 1u);
    for (int q = b * per + 256 * NMOE_DISPATCH_PRE + tid; q < q1; q += 256)
        atomicAdd(&h[nmoe_entry_expert<ROUTED>(s, q)], 1u);
    __syncthreads();
}

/* The down tiles' order of the one-launch GEMM: order entry es (round
 * g = es / 8 of die d = es mod 8) goes to entry 8 j + d of a second list.
 * A die's large experts (more than NMOE_SMALL_PASS entries, its first nb
 * rounds) run the longest gate/up tiles, so their down tiles, taken first,
 * would hold their slots waiting; they now come after half of the die's
 * other experts whose gate/up tiles run in the first round of r1 experts
 * (rounds nb .. nb + h - 1 first, then 0 .. nb - 1, then the rest). */
__device__ __forceinline__ uint32_t nmoe_down_entry(uint32_t es, uint32_t nbig, uint32_t r1) {
    const uint32_t d = es & 7u, g = es >> 3, r = nbig >> 3, m = nbig & 7u;
    const uint32_t nb = r + (uint32_t)((r & 1u) ? d >= 8u - m : d < m); /* dealt as in the order */
    const uint32_t h = r1 > nb ? (r1 - nb) / 2u : 0u;
    const uint32_t j = g < nb ? h + g : g < nb + h ? g - nb : g;
    return 8u * j + d;
}

/* Rank of this lane among the wavefront's lanes of the same key e
 * (9 bits: the experts and 256, left out), and their count (a multi-split
 * by ballots). */
template <int NB = 9>
__device__ __forceinline__ uint32_t nmoe_multisplit9(uint32_t e, int lane, uint32_t &cnt) {
    uint64_t peers = ~0ull;
#pragma unroll
    for (int bit = 0; bit < NB; bit++) {
        const uint64_t m = __ballot((e >> bit) & 1u);
        peers &= ((e >> bit) & 1u) ? m : ~m;
    }
    cnt = (uint32_t)__builtin_popcountll(peers);
    return (uint32_t)__builtin_popcountll(peers & ((1ull << lane) - 1ull));
}

/* D2: offsets (block 0 writes them) and the stable permutation of slice b
 * (the slices' histograms from counts, or from h when there is one slice):
 * chunks of 256 entries in order; within a chunk the rank of an entry is
 * its rank among the equal-expert lanes of its wavefront (a 9-bit
 * multi-split by ballots) plus the counts of the earlier wavefronts. */
template <bool ROUTED, bool MULTI>
__device__ __forceinline__ void nmoe_dispatch_scatter(const nmoe_entry_src &src, int ntok, const uint64_t *counts,
                                                      const uint32_t *h, uint32_t *perm, uint32_t *offsets,
                                                      uint4 *rank, int b, int nd, const uint32_t *ev, uint32_t r1,
                                                      nmoe_scatter_lds &sl) {
    __shared__ uint32_t s_base[NMOE_EXPERTS];
    __shared__ uint32_t s_scan[4]; /* the wavefronts' totals */
    __shared__ uint32_t s_nbig;    /* the experts of more than one small pass */
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = ntok * src.k;
    const int per = (n + nd - 1) / nd, q0 = b * per, q1 = min(n, (b + 1) * per);
    /* thread e: total of expert e and its count in the slices before b,
     * from every slice's histogram word of expert e, tagged with the
     * launch's epoch: NMOE_DISPATCH_READ slices' loads in flight at once,
     * then the words still without the epoch read again in one round
     * (bounded) */
    uint32_t total = 0, before = 0;
    if constexpr (!MULTI) {
        total = h[tid];
    } else {
        uint32_t spins = 0;
        for (int b0 = 0; b0 < nd; b0 += NMOE_DISPATCH_READ) {
            uint64_t w[NMOE_DISPATCH_READ];
#pragma unroll
            for (int i = 0; i < NMOE_DISPATCH_READ; i++)
                w[i] = b0 + i < nd ? nmoe_ld_tagged(counts + (b0 + i) * NMOE_EXPERTS + tid) : (uint64_t)src.epoch << 32;
            for (;;) {
                bool seen = true;
#pragma unroll
                for (int i = 0; i < NMOE_DISPATCH_READ; i++) seen = seen && nmoe_tag_is(w[i], src.epoch);
                if (seen) break;
                if (++spins > src.spin) {
                    __hip_atomic_store((nmoe_g32 *)(src.sync + NMOE_SYNC_STATUS), 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
#pragma unroll
                for (int i = 0; i < NMOE_DISPATCH_READ; i++)
                    if (!nmoe_tag_is(w[i], src.epoch)) w[i] = nmoe_ld_tagged(counts + (b0 + i) * NMOE_EXPERTS + tid);
            }
#pragma unroll
            for (int i = 0; i < NMOE_DISPATCH_READ; i++) {
                const uint32_t c = b0 + i < nd ? (uint32_t)w[i] : 0u;
                total += c;
                before += b0 + i < b ? c : 0u;
            }
        }
        /* every slice read its entries, and with them every routing block
         * this launch's epoch, before it published its histogram: the next
         * launch takes the next epoch */
        if (b == 0 && tid == 0) nmoe_add_u32_dev(src.sync + NMOE_SYNC_PREP_EPOCH, 1u);
    }
    /* the experts by work, most first: bucket = 16-entry row blocks (63 and
     * more together), a counting sort over the buckets, the experts of one
     * bucket in index order (any order would do: the GEMM blocks' results
     * do not depend on it).  The
     * GEMM blocks take the experts in this order, so the longest tiles start
     * first and the launch's tail is short.  Entry es runs on die (es + c)
     * mod 8, so each round of eight is dealt back and forth (0..7, then
     * 7..0): dealt the same way every round, the same dies would take the
     * larger expert of every round and finish last. */
    const int bk = 63 - (int)min((total + 15u) / 16u, 63u);
    /* (block 0) the expert's place among its wavefront's experts of the same
     * bucket (a 6-bit multi-split), and each wavefront's count of them */
    uint32_t brk = 0u;
    if (b == 0) {
        uint32_t bcnt;
        brk = nmoe_multisplit9<6>((uint32_t)bk, lane, bcnt);
        if (brk == 0u) sl.wbk[wave][bk] = bcnt;
    }
    /* exclusive scan of total over the 256 experts: an inclusive scan within
     * each wavefront (DPP), then the earlier wavefronts' totals */
    const uint32_t inc = nmoe_wave_incl_scan_u32(total);
    if (lane == 63) s_scan[wave] = inc;
    /* the stable order within an expert is (chunk of 256, wavefront, lane):
     * the first NMOE_DISPATCH_PRE chunks (their entries in ev) at once,
     * each entry's rank among its wavefront's lanes of the same expert and
     * each (chunk, wavefront)'s count of every expert */
    uint32_t rk[NMOE_DISPATCH_PRE];
#pragma unroll
    for (int j = 0; j < NMOE_DISPATCH_PRE; j++) {
        rk[j] = 0u;
        if (q0 + 256 * j < q1) { /* (block-uniform) a chunk with entries */
            uint32_t cnt;
            rk[j] = nmoe_multisplit9<>(ev[j], lane, cnt);
            if (rk[j] == 0u) sl.wc[j][wave][ev[j]] = cnt;
        }
    }
    __syncthreads();
    uint32_t prior = 0;
    for (int w = 0; w < wave; w++) prior += s_scan[w];
    const uint32_t off = prior + inc - total;
    /* thread e: each (chunk, wavefront)'s first place for expert e, in
     * place of its count */
    uint32_t at = off + before;
#pragma unroll
    for (int j = 0; j < NMOE_DISPATCH_PRE; j++)
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t c = sl.wc[j][w][tid];
            sl.wc[j][w][tid] = at;
            at += c;
        }
    s_base[tid] = at; /* the chunks after those */
    if (b == 0) {
        offsets[tid] = off;
        if (tid == 255) offsets[NMOE_EXPERTS] = off + total;
        if (tid < 64) { /* exclusive scan of the 64 bucket sizes (one wavefront) */
            const uint32_t c = sl.wbk[0][tid] + sl.wbk[1][tid] + sl.wbk[2][tid] + sl.wbk[3][tid];
            const uint32_t binc = nmoe_wave_incl_scan_u32(c);
            sl.bk[tid] = binc - c;
            static_assert(NMOE_SMALL_PASS == 16, "bucket 62 holds the experts of one small pass");
            if (tid == 62) s_nbig = binc - c;
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NMOE_DISPATCH_PRE; j++) {
        const int q = q0 + 256 * j + tid;
        /* pos < n unless the wait for the slices' histograms gave up (then the counts of the
         * other slices may be stale and the launch reports it) */
        if (q < q1 && ev[j] < (uint32_t)NMOE_EXPERTS) {
            const uint32_t pos = sl.wc[j][wave][ev[j]] + rk[j];
            if (pos < (uint32_t)n) perm[pos] = (uint32_t)q;
        }
    }
    if (b == 0) {
        /* the order (its fourth word: the entry itself), and the same
         * entries in the down tiles' order after it */
        uint32_t pos = sl.bk[bk] + brk; /* the bucket's first place, the earlier wavefronts', this one's */
#pragma unroll
        for (int w = 0; w < 3; w++) pos += w < wave ? sl.wbk[w][bk] : 0u;
        const uint32_t round = pos >> 3;
        const uint32_t es = 8u * round + ((round & 1u) ? 7u - (pos & 7u) : (pos & 7u));
        const uint4 ent = make_uint4((uint32_t)tid, off, total, es);
        rank[es] = ent;
        rank[NMOE_EXPERTS + nmoe_down_entry(es, s_nbig, r1)] = ent;
    }
    /* slices of more than NMOE_DISPATCH_PRE chunks: the others one at a
     * time, counted in sl.wc[0] */
    for (int c0 = q0 + 256 * NMOE_DISPATCH_PRE; c0 < q1; c0 += 256) {
        __syncthreads(); /* sl.wc[0] and s_base are free */
#pragma unroll
        for (int w = 0; w < 4; w++) sl.wc[0][w][tid] = 0u;
        if (tid < 4) sl.wc[0][tid][NMOE_EXPERTS] = 0u;
        __syncthreads();
        const int q = c0 + tid;
        const uint32_t e = q < q1 ? nmoe_entry_expert<ROUTED>(src, q) : (uint32_t)NMOE_EXPERTS;
        uint32_t cnt;
        const uint32_t r = nmoe_multisplit9<>(e, lane, cnt);
        if (r == 0u) sl.wc[0][wave][e] = cnt;
        __syncthreads();
        if (q < q1 && e < (uint32_t)NMOE_EXPERTS) {
            uint32_t pos = s_base[e] + r;
            for (int w = 0; w < wave; w++) pos += sl.wc[0][w][e];
            if (pos < (uint32_t)n) perm[pos] = (uint32_t)q;
        }
        __syncthreads();
        s_base[tid] += sl.wc[0][0][tid] + sl.wc[0][1][tid] + sl.wc[0][2][tid] + sl.wc[0][3][tid];
    }
}

/* ------------------------------------------------------------ X prep */

/* xp[t][16 span + slot] = x[t][16 span + kperm(slot)] as bf16 (hi plane; the
 * lo plane x - hi when x is fp32); xs3[t][p][g] = part p of the sum of the 64
 * values of group g (hi + lo, in a fixed order) as three bf16 whose sum is
 * the fp32 sum exactly (8 + 8 + 8 significant bits), the matrix-core
 * operand of the correction. */
template <int BITS, typename XT>
__device__ __forceinline__ void nmoe_grouped_xprep(const XT *x, uint16_t *xhi, uint16_t *xlo, uint16_t *xs3, int t) {
    const int tid = threadIdx.x; /* 8 elements per thread: half a span */
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
    if ((tid & 7) == 0) {
        constexpr int G = NMOE_HIDDEN / NMOE_GROUP;
        const uint32_t h = nmoe_bf16_rne(sum);
        const float r = sum - nmoe_bf16f(h); /* exact */
        const uint32_t m = nmoe_bf16_rne(r);
        const uint32_t l = nmoe_bf16_rne(r - nmoe_bf16f(m)); /* exact: the last 8 bits */
        uint16_t *o = xs3 + (size_t)t * 3 * G + (tid >> 3);
        o[0] = (uint16_t)h;
        o[G] = (uint16_t)m;
        o[2 * G] = (uint16_t)l;
    }
}

static __constant__ uint64_t nmoe_grouped_exp2_tab[32] = NMOE_EXP2_TAB32;

/* The one-launch GEMM's schedule words (zeroed by the preparation launch):
 * done[256], per expert rank, counts the gate/up tiles whose act rows are
 * stored; each adds 1 + 2^(16 + its die). */
#define NMOE_SCHED_WORDS NMOE_EXPERTS

/* An expert's done word is touched only by the blocks of one die (its
 * gate/up and down tiles share a die): atomics performed in that die's L2
 * (workgroup scope: no write-through to memory) and loads that bypass the
 * L1 and are served by the L2 (sc0 sc1), a round trip through the die's L2
 * instead of memory. */
__device__ __forceinline__ uint32_t nmoe_add_u32_die(uint32_t *p, uint32_t v) {
    return __hip_atomic_fetch_add((nmoe_g32 *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ uint32_t nmoe_ld_u32_die(const uint32_t *p) {
    return __hip_atomic_load((nmoe_g32 *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

/* A down tile waits (thread 0, bounded) until the low 16 bits of its
 * expert's done word reach its n gate/up tiles, then checks the die bits:
 * every one of those tiles must have run on this block's die (their act
 * rows are in this die's L2, not yet in memory); otherwise, or when the
 * wait gives up, it sets the status word. */
__device__ __forceinline__ void nmoe_tile_done(uint32_t *cnt) { nmoe_add_u32_die(cnt, 1u + (1u << (16 + nmoe_xcc_id()))); }
__device__ __forceinline__ void nmoe_wait_tiles(uint32_t *cnt, uint32_t n, uint32_t *sync, uint32_t spin) {
    uint32_t spins = 0, v;
    while (((v = nmoe_ld_u32_die(cnt)) & 0xffffu) < n) {
        __builtin_amdgcn_s_sleep(1);
        if (++spins > spin) break;
    }
    if (v != n + (n << (16 + nmoe_xcc_id())))
        __hip_atomic_store((nmoe_g32 *)(sync + NMOE_SYNC_STATUS), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* One launch for the grouped path's preparation: blocks 0 .. nd-1 run the
 * dispatch (D1, then D2 once every slice's histogram is in), the blocks
 * after them prepare one token's x each (none when x is NULL).  With more
 * than one dispatch block, the nd blocks (the grid's first, so resident
 * together) meet at a counter in the sync words that grows by exactly 64
 * per launch (64 / nd from each block; bounded wait, an expired wait sets
 * the status word); a single block keeps its histogram in LDS.
 *
 * ROUTED: the routing is computed in the same launch from the token's
 * logits (math.m's softmax / top-k / renormalise, bit for bit, as
 * nmoe_moe_topk) by the nr = ceil(ntok / 4) blocks after the dispatch
 * blocks, one token a wavefront (so they are resident in the launch's
 * first round with the dispatch blocks that wait for them); the x blocks
 * come after them.  A wavefront writes idx / w of its token (the caller's
 * outputs) and each of its entries as a tagged word (epoch << 32 | expert,
 * one device-coherent store) in tags[]; a dispatch block polls the tagged
 * words of its slice (bounded) until each carries this launch's epoch.  The
 * epoch is the PREP_EPOCH sync word + 1, read by every routing and dispatch
 * block at its start; dispatch block 0 adds 1 to the word once every slice's
 * entries have been read (they were all written by then, so no block of
 * this launch can read the new value), and tagged words of earlier launches
 * carry earlier epochs, so none is taken for this launch's. */
template <int BITS, typename XT, bool ROUTED, bool MULTI>
__global__ void __launch_bounds__(256) nmoe_grouped_prep_kernel(const uint32_t *idx, int ntok, int k, int nd,
                                                                uint64_t *counts, uint32_t *perm, uint32_t *offsets,
                                                                uint4 *rank, uint32_t *sync, uint32_t spin,
                                                                const XT *x, uint16_t *xhi, uint16_t *xlo,
                                                                uint16_t *xs3, const float *logits, uint32_t *idx_out,
                                                                float *w_out, uint32_t *done, int skew,
                                                                uint64_t *tags, uint64_t *tl) {
    const int b = blockIdx.x;
    nmoe_gtl_begin(tl);
    /* this launch's epoch of the tagged entries and histogram words (read
     * at once by every block) */
    const uint32_t epoch = ROUTED || MULTI ? nmoe_ld_u32_dev(sync + NMOE_SYNC_PREP_EPOCH) + 1u : 0u;
    /* the one-launch GEMM's tile counts start from 0 (plain stores: the next
     * launch on the stream sees them); rank `skew` (a test of the failure
     * path) from a count no tiles can reach */
    if (done != NULL && b == 0)
        for (int i = threadIdx.x; i < NMOE_SCHED_WORDS; i += 256) done[i] = i == skew ? 0x8000u : 0u;
    const int nr = ROUTED ? (ntok + 3) / 4 : 0; /* routing blocks */
    if (ROUTED && b >= nd && b < nd + nr) {
        __shared__ float s_sm[4][NMOE_EXPERTS];
        __shared__ uint64_t s_tab[32];
        const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, t = 4 * (b - nd) + wave;
        /* the token's logits straight into LDS (one 1 KB direct load a
         * wavefront) and the exp table beside them, both in flight at once:
         * read from constant memory, each exp's table lookup was a memory
         * round trip of its own after the logits' */
        static_assert(NMOE_EXPERTS == 256, "a token's logits are one 1 KB direct load");
        if (t < ntok) { /* wavefront-uniform */
            if (((uintptr_t)logits & 15u) == 0u) {
                __builtin_amdgcn_global_load_lds((const void *)(logits + (size_t)t * NMOE_EXPERTS + 4 * lane),
                                                 (nmoe_lds_void *)&s_sm[wave][0], 16, 0, 0);
            } else { /* logits only 4-byte aligned: a lane a word */
#pragma unroll
                for (int q = 0; q < 4; q++) s_sm[wave][lane + 64 * q] = logits[(size_t)t * NMOE_EXPERTS + lane + 64 * q];
            }
        }
        if (threadIdx.x < 32) s_tab[threadIdx.x] = nmoe_grouped_exp2_tab[threadIdx.x];
        __builtin_amdgcn_s_waitcnt(0x0F70); /* vmcnt(0): the logits are in LDS */
        __syncthreads();
        if (t < ntok) {
            uint32_t si[NMOE_MAX_K];
            float sw[NMOE_MAX_K];
            /* (the logits are read into registers before s_sm[wave] serves as
             * the exact sum's scratch) */
            nmoe_wave_route(&s_sm[wave][0], NMOE_EXPERTS, k, s_sm[wave], s_tab, si, sw, NULL);
            if (threadIdx.x == 0) nmoe_gtl_stamp(tl, NMOE_GTL_READY);
            if (lane < NMOE_MAX_K) {
                uint32_t vi = 0;
                float vw = 0.0f;
#pragma unroll
                for (int q = 0; q < NMOE_MAX_K; q++)
                    if (q == lane) {
                        vi = si[q];
                        vw = sw[q];
                    }
                idx_out[(size_t)t * NMOE_MAX_K + lane] = vi;
                w_out[(size_t)t * NMOE_MAX_K + lane] = vw;
                if (lane < k)
                    __hip_atomic_store((nmoe_g64 *)&tags[(size_t)t * k + lane], ((uint64_t)epoch << 32) | vi,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        nmoe_gtl_prep_end(tl, 3);
        return;
    }
    if (b >= nd) {
        if (x != NULL) nmoe_grouped_xprep<BITS, XT>(x, xhi, xlo, xs3, b - nd - nr);
        nmoe_gtl_prep_end(tl, 5);
        return;
    }
    const nmoe_entry_src src = {idx, k, tags, epoch, sync, spin};
    uint32_t ev[NMOE_DISPATCH_PRE];
    nmoe_dispatch_entries<ROUTED>(src, ntok, b, nd, ev);
    if (ROUTED && threadIdx.x == 0) nmoe_gtl_stamp(tl, NMOE_GTL_READY);
    __shared__ uint32_t h[NMOE_EXPERTS + 1];
    __shared__ nmoe_scatter_lds s_scat;
    nmoe_dispatch_count<ROUTED>(src, ntok, h, b, nd, ev, s_scat);
    /* every entry of the one slice read: the next launch takes the next
     * epoch (with several slices, dispatch block 0 advances it once every
     * slice's histogram is in) */
    if (ROUTED && !MULTI && threadIdx.x == 0) nmoe_add_u32_dev(sync + NMOE_SYNC_PREP_EPOCH, 1u);
    if constexpr (MULTI)
        /* this slice's histogram for the other slices, each word tagged with
         * the launch's epoch (device-coherent stores): a reader takes a word
         * once it carries the epoch, so nothing waits for these stores and
         * no arrival is counted */
        for (int i = threadIdx.x; i < NMOE_EXPERTS; i += 256)
            __hip_atomic_store((nmoe_g64 *)&counts[b * NMOE_EXPERTS + i], ((uint64_t)epoch << 32) | h[i],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    /* experts whose gate/up tiles fill one die's first round: 32 CUs a
     * die, two four-wavefront blocks a CU (one of eight) */
    constexpr uint32_t R1 =
        (256u / NMOE_GROUPED_NW) / (uint32_t)(NMOE_INTER / nmoe_gu_rows(sizeof(XT) == 2 ? 1 : 2, NMOE_GROUPED_NW));
    nmoe_dispatch_scatter<ROUTED, MULTI>(src, ntok, counts, h, perm, offsets, rank, b, nd, ev, R1, s_scat);
    nmoe_gtl_prep_end(tl, 4);
}

/* ------------------------------------------------------------ stage ring */

/* Both GEMMs stream one 64-deep K group per step through a ring of NS LDS
 * stages (four where they fit the block's LDS share, else three), filled by
 * direct global->LDS loads (global_load_lds_dwordx4: lane l of a wavefront
 * writes bytes 16l..16l+15 of the instruction's 1 KB), so a group is
 * requested NS - 1 steps before it is multiplied.  A stage holds
 *   - the A rows of the group: PL planes of 64 rows x 64 bf16 (128 B); the
 *     16-byte chunk c of row r sits at slot c ^ ((r >> 1) & 7), so the 16
 *     rows of one ds_read_b128 pass cover all 64 banks;
 *   - the codes of the tile's weight rows for the group: q4 as rows of
 *     32 B whose two 16-byte halves swap on rows with bit 3 set (two lanes
 *     fetch a row's 32 bytes; the swap spreads the ds_read_b64 of 16 rows
 *     over more banks), q2 as rows of 16 B.
 * Each stage is a __shared__ variable of its own: the compiler then tells
 * the stages' direct loads apart and a read of one stage does not wait for
 * the loads still in flight into the others. */

template <int PL, int R, int CW>
struct nmoe_stage {
    uint4 a[PL][R * 8];
    uint32_t b[CW];
};

/* One stage buffer for both forms (the small form's stage where it is
 * built, else the big form's again). */
template <typename B, typename S>
union nmoe_stage_buf {
    B big;
    S small;
};

/* A direct load into LDS from a wavefront-uniform base plus a 32-bit
 * per-lane byte offset: the compiler can address it as a scalar base and a
 * vector offset, so the stages' per-group addresses cost no vector
 * registers (the group moves the scalar base). */
template <int SZ>
__device__ __forceinline__ void nmoe_dma(const void *ubase, uint32_t off, void *lds) {
    const void *src = (const void *)((const char *)ubase + off);
    if constexpr (SZ == 16)
        __builtin_amdgcn_global_load_lds(src, (nmoe_lds_void *)lds, 16, 0, 0);
    else
        __builtin_amdgcn_global_load_lds(src, (nmoe_lds_void *)lds, 4, 0, 0);
}

/* Instruction j (rows 8j..8j+7) of one A plane: ubase is the plane at the
 * group's first column (uniform), row_off this lane's row (8j + lane / 8)
 * in bytes. */
__device__ __forceinline__ void nmoe_stage_rows(uint4 *plane, const uint16_t *ubase, uint32_t row_off, int j, int lane) {
    const int r = 8 * j + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    nmoe_dma<16>(ubase, row_off + 16u * (uint32_t)c, plane + 64 * j);
}

/* MFMA A operand (the lane's two 8-element chunks 2kb, 2kb+1) of row r. */
__device__ __forceinline__ void nmoe_stage_operand(const uint4 *plane, int r, int kb, uint4 &a0, uint4 &a1) {
    const int h = (r >> 1) & 7;
    a0 = plane[8 * r + ((2 * kb) ^ h)];
    a1 = plane[8 * r + ((2 * kb + 1) ^ h)];
}

/* A stage holds GPS groups of each weight row: the row's GPS * 32 B (q4)
 * or GPS * 16 B (q2) of codes side by side, RB bytes a stage row.  Its
 * 16-byte parts are rotated by the row (part c of row r sits at c ^ swz(r))
 * so that the 16 rows a column block reads at once fall on distinct banks:
 * 32-byte rows swap halves on row bit 3, 64-byte rows rotate by row bits
 * 2-3. */
template <int BITS, int GPS>
struct nmoe_code_row {
    static constexpr int RB = GPS * (BITS == 4 ? 32 : 16); /* stage bytes a row */
    static constexpr int WPS = RB / 4;                      /* stage words a row */
    static constexpr int LPR = RB / 16;                     /* 16-byte parts a row */
    static_assert(LPR == 1 || LPR == 2 || LPR == 4, "a row is one, two or four 16-byte parts");
    __device__ static __forceinline__ int swz(int r) { return LPR == 4 ? (r >> 2) & 3 : LPR == 2 ? (r >> 3) & 1 : 0; }
};

/* The direct loads of one stage's codes (NR weight rows of RB bytes) over
 * the NW wavefronts of a block: 1-KB instructions (16 B a lane) where each
 * wavefront has at least 1 KB to load, else 256-byte ones (4 B a lane).
 * Every wavefront issues the same number, so the ring waits are
 * compile-time constants. */
template <int BITS, int NR, int NW, int GPS = 1>
struct nmoe_code_plan {
    static constexpr int BYTES = NR * nmoe_code_row<BITS, GPS>::RB;
    static constexpr bool WIDE = BYTES / NW >= 1024;
    static constexpr int INS_BYTES = WIDE ? 1024 : 256;
    static constexpr int PER_WAVE = BYTES / NW / INS_BYTES;
    static_assert(PER_WAVE >= 1 && PER_WAVE * INS_BYTES * NW == BYTES, "codes split evenly over the wavefronts");
    static_assert(WIDE || (BITS == 2 && GPS == 1), "only q2 rows of one group load in 4-byte lanes");
};

/* Words of group g from a row's first word: 8 (q4) or 4 (q2). */
template <int BITS>
__host__ __device__ constexpr int nmoe_gwords() { return BITS == 4 ? 8 : 4; }

/* The grouped GEMMs read a stripe-major copy of each layer's code
 * matrices (nmoe_pack_stripe): a matrix of rows of wpr words, groups of gw
 * words, is stored as stripes of NMOE_STRIPE rows, and within a stripe
 * group g of its rows side by side.  A ring step's codes (one or two
 * groups of a tile's 32..256 rows) are then runs of NMOE_STRIPE * gw words
 * (1-2 KB) instead of gw words a row, a row's length apart. */
#define NMOE_STRIPE 64
__host__ __device__ __forceinline__ uint32_t nmoe_stripe_word(uint32_t r, uint32_t g, uint32_t gw, uint32_t wpr) {
    return (r / NMOE_STRIPE) * NMOE_STRIPE * wpr + (g * NMOE_STRIPE + r % NMOE_STRIPE) * gw;
}

/* Instruction j of one stage's codes for rows row0 .. row0 + NR - 1 of a
 * stripe-major matrix at mbase, groups
 * GPS gs .. GPS gs + GPS - 1, in the stage layout above.  A 1-KB
 * instruction covers 64 / LPR rows, LPR lanes a row. */
template <int BITS, int NR, bool WIDE, int GPS = 1>
__device__ __forceinline__ void nmoe_stage_codes(uint32_t *stage, const uint32_t *mbase, int wpr, int row0, int gs,
                                                 int j, int lane) {
    using CR = nmoe_code_row<BITS, GPS>;
    constexpr uint32_t GW = nmoe_gwords<BITS>();
    const uint32_t *gbase = mbase + (size_t)(GPS * gs) * NMOE_STRIPE * GW; /* the step's first group (uniform) */
    if (WIDE) {
        const int row = (64 / CR::LPR) * j + lane / CR::LPR, part = (lane % CR::LPR) ^ CR::swz(row);
        const uint32_t u = (16u * part) / (4u * GW), w = ((16u * part) % (4u * GW)) / 4u; /* group of the step, word */
        nmoe_dma<16>(gbase, 4u * (nmoe_stripe_word((uint32_t)(row0 + row), u, GW, (uint32_t)wpr) + w),
                     stage + 256 * j);
    } else {
        /* q2, one group: rows 16j + lane / 4, word lane % 4 */
        const int row = 16 * j + (lane >> 2);
        nmoe_dma<4>(gbase, 4u * (nmoe_stripe_word((uint32_t)(row0 + row), 0u, GW, (uint32_t)wpr) + (lane & 3)),
                    stage + 64 * j);
    }
}

/* Byte offset, in a matrix's stage codes, of the lane's code words of
 * group u (of the stage's GPS) in stage row r: q4 words 2kb, 2kb+1; q2
 * word kb.  Computed once per lane, before the ring, and kept opaque: an
 * offset summed from its parts at every read becomes a chain of address
 * steps deep enough that the compiler no longer knows which stage the read
 * belongs to, and then makes it wait for every stage's loads. */
template <int BITS, int GPS = 1>
__device__ __forceinline__ uint32_t nmoe_code_off(int r, int u, int kb) {
    using CR = nmoe_code_row<BITS, GPS>;
    uint32_t off;
    if (BITS == 4) {
        const int c = 2 * u + (kb >> 1); /* the 16-byte part holding words 2kb, 2kb+1 of group u */
        off = (uint32_t)(CR::RB * r + 16 * (c ^ CR::swz(r)) + 8 * (kb & 1));
    } else {
        off = (uint32_t)(CR::RB * r + 16 * (u ^ CR::swz(r)) + 4 * kb);
    }
    asm("" : "+v"(off));
    return off;
}

/* The code words at byte offset off of a matrix's stage codes. */
template <int BITS>
__device__ __forceinline__ void nmoe_code_read(const uint32_t *codes, uint32_t off, uint32_t &w0, uint32_t &w1) {
    if (BITS == 4) {
        const uint2 v = *(const uint2 *)((const char *)codes + off);
        w0 = v.x;
        w1 = v.y;
    } else {
        w0 = *(const uint32_t *)((const char *)codes + off);
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

/* The barrier before group g of G in a ring of NS stages, for a wavefront
 * that issues L loads per group: groups g+1 .. g+NS-2 (those that exist)
 * may still be in flight.  (K: the groups allowed in flight, tried from
 * NS-2 down.) */
template <int L, int G, int NS, int K = NS - 2>
__device__ __forceinline__ void nmoe_ring_step_barrier(int g) {
    if constexpr (K == 0) {
        nmoe_ring_barrier<0>();
    } else {
        if (g + K < G)
            nmoe_ring_barrier<K * L>();
        else
            nmoe_ring_step_barrier<L, G, NS, K - 1>(g);
    }
}

template <int I, int NS, typename Step>
__device__ __forceinline__ void nmoe_ring_turn(Step &step, int g) {
    if constexpr (I < NS) {
        step(g + I, I, true);
        nmoe_ring_turn<I + 1, NS>(step, g);
    }
}

template <int G0, int G, int NS, int ISSUE, typename Step>
__device__ __forceinline__ void nmoe_ring_tail(Step &step) {
    if constexpr (G0 < G) {
        step(G0, G0 % NS, G0 < ISSUE);
        nmoe_ring_tail<G0 + 1, G, NS, ISSUE>(step);
    }
}

/* Runs step(g, stage, issue_ahead) over the G groups with NS stages: step g
 * issues group g + NS - 1 while it exists.  The loop's steps all issue,
 * unconditionally (a load issued under a runtime condition makes the
 * compiler wait for every stage); the remaining steps are unrolled with
 * their stage and issue flag known at compile time. */
template <int G, int NS, typename Step>
__device__ __forceinline__ void nmoe_ring_run(Step step) {
    constexpr int ISSUE = G - NS + 1;          /* steps that issue a later group */
    constexpr int MAIN = (ISSUE / NS) * NS;    /* steps in the loop, whole ring turns */
#pragma unroll 1
    for (int g = 0; g < MAIN; g += NS) nmoe_ring_turn<0, NS>(step, g);
    nmoe_ring_tail<MAIN, G, NS, ISSUE>(step);
}

/* Workgroup barrier over LDS only: waits for this wavefront's LDS accesses
 * (lgkmcnt 0) but not for its global stores, which __syncthreads() would. */
__device__ __forceinline__ void nmoe_lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F); /* vmcnt 63, expcnt 7, lgkmcnt 0 */
    asm volatile("s_barrier" ::: "memory");
}

template <int N>
__device__ __forceinline__ void nmoe_wait_vm() {
    /* s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt[3:0] | vmcnt[5:4] << 14,
     * expcnt and lgkmcnt left at their maxima) */
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

/* Block b of a 1-D grid of NMOE_EXPERTS * ntiles blocks -> (expert, tile).
 * Blocks b, b+8, b+16, ... land on the same die (blocks are dealt to the
 * eight dies in turn), so the tiles of one expert run side by side on one
 * die and share its activation rows in that die's L2. */
__device__ __forceinline__ void nmoe_die_tile(int b, int ntiles, int &e, int &nt) {
    e = 8 * (b / (8 * ntiles)) + (b & 7);
    nt = (b >> 3) % ntiles;
}

/* Entry es of the expert order (expert, first entry, entries), written by
 * the preparation launch and only read by the GEMM launches: one scalar
 * 16-byte load, through the constant address space, all four words needed
 * at once.  Read as a plain pointer, the compiler made it a vector load
 * where it could not prove the words unchanged in the launch (it then
 * waits in the CU's vector memory queue behind the stage loads of the
 * CU's other block) and split it into two dependent loads around the
 * empty-expert exit. */
__device__ __forceinline__ uint4 nmoe_rank_entry(const uint4 *rank, int es) {
    typedef uint32_t nmoe_v4u __attribute__((ext_vector_type(4)));
    typedef const __attribute__((address_space(4))) nmoe_v4u nmoe_const_v4u;
    const nmoe_v4u v = *(nmoe_const_v4u *)(uintptr_t)(rank + es);
    uint32_t x = v.x, y = v.y, z = v.z, w = v.w;
    asm volatile("" : "+s"(x), "+s"(y), "+s"(z), "+s"(w));
    return make_uint4(x, y, z, w);
}

/* SiLU for the grouped path (outputs are checked to a tolerance there):
 * the exp of a non-positive argument as in math.m:21-28, the reciprocal by
 * v_rcp_f32 instead of a full division. */
__device__ __forceinline__ float nmoe_silu_fast(float x) {
    const float z = __expf(-fabsf(x));
    const float r = __builtin_amdgcn_rcpf(1.0f + z);
    return x * (x >= 0.0f ? r : z * r);
}

/* ------------------------------------------------------------ gate/up */


/* Bytes of one gate/up stage with mch entries a pass and gps groups a step:
 * A rows (xpl planes x gps groups x mch rows x 128 B) and the codes of the
 * tile's gate and up rows. */
__host__ __device__ constexpr int nmoe_gu_stage(int bits, int xpl, int nw, int mch, int gps) {
    return xpl * gps * mch * 128 + 2 * nmoe_gu_rows(xpl, nw) * gps * (bits == 4 ? 32 : 16);
}
/* A stage buffer holds the stage of either form. */
__host__ __device__ constexpr int nmoe_gu_stage_max(int bits, int xpl, int nw) {
    return nmoe_small_form(nw) && nmoe_gu_stage(bits, xpl, nw, NMOE_SMALL_PASS, NMOE_SMALL_GPS) >
                                      nmoe_gu_stage(bits, xpl, nw, NMOE_MCHUNK, 1)
               ? nmoe_gu_stage(bits, xpl, nw, NMOE_SMALL_PASS, NMOE_SMALL_GPS)
               : nmoe_gu_stage(bits, xpl, nw, NMOE_MCHUNK, 1);
}
/* LDS bytes of a gate/up block with ns stages: the stages, the scales,
 * s_tok and s_as. */
__host__ __device__ constexpr int nmoe_gu_lds(int bits, int xpl, int nw, int ns) {
    return ns * nmoe_gu_stage_max(bits, xpl, nw) + 2 * nmoe_gu_rows(xpl, nw) * 64 + 4 * NMOE_MCHUNK * (1 + nw);
}
/* Stages: four where they fit the block's share of the CU's 160 KB (the
 * whole of it for eight wavefronts, half for four), else three. */
__host__ __device__ constexpr int nmoe_gu_stages(int bits, int xpl, int nw) {
    return nmoe_gu_lds(bits, xpl, nw, 4) <= (nw == 8 ? 160 : 80) * 1024 - 512 ? 4 : 3;
}


/* Expert e, gate and up rows NT * nt .. +NT-1: act rows of all the
 * expert's entries, 64 entries per pass (16 in one pass in the small
 * form).  NW wavefronts (eight: one block a CU; four: two blocks a CU, whose
 * set-up and epilogue then overlap the other's ring), two per SIMD either
 * way; wavefront w owns gate and up rows (NT/NW)w .. +NT/NW-1 of the tile as
 * NB 16-row MFMA column blocks each, over the pass's (up to four) 16-entry
 * row blocks, so a lane holds gate and up of the same (entry, row).
 *
 * y = sum_g s_g P_g + sum_g (b_g - 128 s_g) xs_g with P_g the MFMA product
 * of the group's A rows and the codes as bf16(128 + q); the second sum runs
 * first, as sum_g xs_g b_g - 128 sum_g xs_g s_g over the 32 groups: one bf16
 * MFMA (K = 32) per part of xs (three exact bf16 parts) and per operand (the
 * bf16 biases and scales as they are), fp32 accumulate. */
/* The LDS of a gate/up block.  The tile's gate and up scales chunk-major:
 * 16-byte chunk q (groups 8q..8q+7) of row r at [mat][q][r], so a ring
 * step's 16 rows of one group sit 16 bytes apart (distinct banks; row-major
 * rows 64 bytes apart put four rows on each bank).  The stage buffers hold
 * one stage of either form each, and every stage is a typed variable of its
 * own, so that the compiler tells the stages' direct loads apart. */
template <int BITS, int XPL, int NW>
struct nmoe_gu_lds_types {
    static constexpr int NT = nmoe_gu_rows(XPL, NW);
    typedef uint16_t Scales[2][NMOE_HIDDEN / NMOE_GROUP / 8][NT][8];
    typedef nmoe_stage<XPL, NMOE_MCHUNK, 2 * NT * nmoe_code_row<BITS, 1>::WPS> StageB;
    typedef nmoe_stage<XPL, NMOE_SMALL_GPS * NMOE_SMALL_PASS, 2 * NT * nmoe_code_row<BITS, NMOE_SMALL_GPS>::WPS>
        StageS;
    typedef nmoe_stage_buf<StageB, typename std::conditional<nmoe_small_form(NW), StageS, StageB>::type> StageU;
    static_assert(sizeof(StageU) == nmoe_gu_stage_max(BITS, XPL, NW), "stage buffer size");
};

/* Gate/up tile nt of the es-th expert by entries, pass lane pl, with NS
 * stages in the given LDS buffers (s_st3 is used only with NS = 4).  COUNT:
 * once the tile's act rows and group sums are stored (complete, in this
 * die's L2), the block counts itself in done[es] (nmoe_tile_done), which
 * the down tiles of the same launch wait for. */
template <int BITS, int XPL, int NW, int NS, bool COUNT>
__device__ __forceinline__ void nmoe_gu_tile(const uint8_t *pack, const uint16_t *xhi, const uint16_t *xlo,
                                             const uint16_t *xs3, const uint32_t *perm, const uint4 *rank, int k,
                                             int lanes, int nrows, uint16_t *ahi, uint16_t *alo, float *as, int es,
                                             int nt, int pl, typename nmoe_gu_lds_types<BITS, XPL, NW>::Scales &s_s,
                                             typename nmoe_gu_lds_types<BITS, XPL, NW>::StageU &s_st0,
                                             typename nmoe_gu_lds_types<BITS, XPL, NW>::StageU &s_st1,
                                             typename nmoe_gu_lds_types<BITS, XPL, NW>::StageU &s_st2,
                                             typename nmoe_gu_lds_types<BITS, XPL, NW>::StageU &s_st3,
                                             uint32_t (&s_tok)[NMOE_MCHUNK], float (&s_as)[NW][NMOE_MCHUNK],
                                             uint32_t *done) {
    using Q = nmoe_q<BITS>;
    using L = nmoe_layout<BITS>;
    constexpr int G = NMOE_HIDDEN / NMOE_GROUP; /* 32 groups */
    static_assert(G == 32, "the correction's operand layout assumes 8 groups per lane");
    static_assert(NW == 8 || NW == 4, "eight or four wavefronts");
    static_assert(NS == 3 || NS == 4, "three or four stages");
    constexpr int NT = nmoe_gu_rows(XPL, NW);
    constexpr int NB = NT / (16 * NW);          /* column blocks per wavefront and matrix */
    constexpr int NTH = 64 * NW;
    typedef typename nmoe_gu_lds_types<BITS, XPL, NW>::StageU StageU;
    /* (e, first entry, entries) of a dispatch whose histogram wait gave up can be
     * anything; the clamps keep every access inside the buffers */
    const uint4 rk = nmoe_rank_entry(rank, es);
    const int e = (int)min(rk.x, (uint32_t)(NMOE_EXPERTS - 1));
    const uint32_t p0 = min(rk.y, (uint32_t)nrows), n = min(rk.z, (uint32_t)nrows - p0);
    if (n <= (uint32_t)(pl * NMOE_MCHUNK)) return;
    const int tid = threadIdx.x, lane = tid & 63, col = lane & 15, kb = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint8_t *ex = pack + (size_t)e * L::expert_size;
    const int rt0 = (NT / NW) * wave + col; /* tile row of column block nb: rt0 + 16 nb */
    /* this wavefront's code instructions CP::PER_WAVE * wave + i all fall in
     * matrix cmat (gate for the first half of the wavefronts, up for the
     * second) */
    const int cmat = wave / (NW / 2);
    const uint32_t *cbase = (const uint32_t *)(ex + (cmat == 0 ? L::gate_w : L::up_w)); /* stripe-major */
    const uint16_t *bias[2] = {(const uint16_t *)(ex + L::gate_b) + (size_t)nt * NT * G,
                               (const uint16_t *)(ex + L::up_b) + (size_t)nt * NT * G};

    /* the passes of one form: MCH entries a pass, GPS groups a ring step */
    auto run = [&](auto mch_c, auto gps_c) {
    constexpr int MCH = decltype(mch_c)::value, GPS = decltype(gps_c)::value;
    constexpr int MB = MCH / 16;                /* row blocks per full pass */
    constexpr int AI = GPS * MCH / 8 / NW;      /* A instructions per plane and wavefront a step */
    static_assert(AI >= 1 && AI * NW * 8 == GPS * MCH, "A rows split evenly over the wavefronts");
    using CR = nmoe_code_row<BITS, GPS>;
    using CP = nmoe_code_plan<BITS, 2 * NT, NW, GPS>;
    constexpr int CPM = CP::BYTES / 2 / CP::INS_BYTES; /* code instructions per matrix */
    /* A rows of group u of a step at rows u MCH .. of each plane */
    typedef nmoe_stage<XPL, GPS * MCH, 2 * NT * CR::WPS> Stage;
    auto stage = [&](int st) -> Stage & {
        StageU &b = st == 0 ? s_st0 : st == 1 ? s_st1 : st == 2 ? s_st2 : s_st3;
        if constexpr (MCH == NMOE_MCHUNK) return b.big;
        else return b.small;
    };
    /* the lane's code-word offsets in a matrix's stage codes, per group of
     * a step and column block (the same in both matrices) */
    uint32_t coff[GPS][NB];
#pragma unroll
    for (int u = 0; u < GPS; u++)
#pragma unroll
        for (int b2 = 0; b2 < NB; b2++) coff[u][b2] = nmoe_code_off<BITS, GPS>(rt0 + 16 * b2, u, kb);

    for (uint32_t m0 = pl * MCH; m0 < n; m0 += lanes * MCH) {
        if (tid < MCH) s_tok[tid] = min(perm[p0 + min(m0 + tid, n - 1)], (uint32_t)nrows - 1u) / (uint32_t)k;
        nmoe_lds_barrier();
        /* this lane's A row for instruction j = wave + NW i (rows 8j .. 8j+7
         * of the stage plane: group j / (MCH / 8), entries 8 (j % (MCH / 8))
         * + lane / 8) */
        uint32_t row_off[AI];
#pragma unroll
        for (int i = 0; i < AI; i++)
            row_off[i] = s_tok[8 * ((wave + NW * i) % (MCH / 8)) + (lane >> 3)] * (uint32_t)(NMOE_HIDDEN * 2);
        const uint16_t *xpl[2] = {xhi, xlo};
        auto issue = [&](int gs, int st) {
#pragma unroll
            for (int pl = 0; pl < XPL; pl++)
#pragma unroll
                for (int i = 0; i < AI; i++) {
                    const int j = wave + NW * i;
                    nmoe_stage_rows(stage(st).a[pl], xpl[pl] + 64 * (GPS * gs + j / (MCH / 8)), row_off[i], j, lane);
                }
#pragma unroll
            for (int i = 0; i < CP::PER_WAVE; i++)
                nmoe_stage_codes<BITS, NT, CP::WIDE, GPS>(stage(st).b + cmat * NT * CR::WPS, cbase, Q::WPR_G,
                                                          nt * NT, gs, (CP::PER_WAVE * wave + i) % CPM, lane);
        };
        const int nb = (int)min((n - m0 + 15) / 16, (uint32_t)MB);
        nmoe_f32x4 acc[2][NB][MB];
        {
            /* The correction's operands go out first and the first ring
             * stages right after them: loads retire in order, so the
             * small loads then return without waiting for the stages,
             * and the correction's MFMAs run while the stages stream in.
             * A lane = (entry col, groups 8kb .. 8kb+7), B lane = (row
             * col, the same groups): a lane's eight groups are contiguous
             * (one 16-byte load per part of xs, one of the biases, one
             * LDS read of the scales). */
            constexpr int PER = 2 * NT * G / 8 / NTH;
            static_assert(PER * NTH == 2 * NT * G / 8, "scale chunks split evenly over the threads");
            /* the tile's scales straight into LDS, every pass (later
             * passes hit L2): wavefront w's q-th 1 KB at uint4 NTH q + 64w */
#pragma unroll
            for (int q = 0; q < PER; q++) {
                /* LDS chunk i = (mat, chunk, row) <- global chunk row * G/8 + chunk of the matrix */
                const int i = tid + NTH * q, mat = i / (NT * G / 8), j = i % (NT * G / 8);
                const int ch = j / NT, row = j % NT;
                const uint4 *src = (const uint4 *)(ex + (mat == 0 ? L::gate_s : L::up_s) + (size_t)nt * NT * G * 2) +
                                   row * (G / 8) + ch;
                __builtin_amdgcn_global_load_lds(
                    (const void *)src, (nmoe_lds_void *)((uint4 *)&s_s[0][0][0][0] + NTH * q + 64 * wave), 16, 0, 0);
            }
            uint4 xq[MB][3];
            uint4 bv[2][NB];
#pragma unroll
            for (int mb = 0; mb < MB; mb++)
#pragma unroll
                for (int p = 0; p < 3; p++)
                    xq[mb][p] = *(const uint4 *)(xs3 + ((size_t)s_tok[16 * mb + col] * 3 + p) * G + 8 * kb);
#pragma unroll
            for (int mat = 0; mat < 2; mat++)
#pragma unroll
                for (int b2 = 0; b2 < NB; b2++)
                    bv[mat][b2] = *(const uint4 *)(bias[mat] + (rt0 + 16 * b2) * G + 8 * kb);
#pragma unroll
            for (int st = 0; st < NS - 1; st++) issue(st, st);
            /* scales, xs and biases have landed once only the stages'
             * loads are in flight; then every wavefront's scales are in
             * LDS */
            nmoe_wait_vm<(NS - 1) * (XPL * AI + CP::PER_WAVE)>();
            nmoe_lds_barrier();
#pragma unroll
            for (int mat = 0; mat < 2; mat++)
#pragma unroll
                for (int b2 = 0; b2 < NB; b2++) {
                    const uint4 sv = *(const uint4 *)&s_s[mat][kb][rt0 + 16 * b2][0];
#pragma unroll
                    for (int mb = 0; mb < MB; mb++) {
                        nmoe_f32x4 a = nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                        if (mb < nb) {
                            nmoe_f32x4 t = nmoe_mfma16(xq[mb][0], sv, nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f});
                            t = nmoe_mfma16(xq[mb][1], sv, t);
                            t = nmoe_mfma16(xq[mb][2], sv, t);
                            a = nmoe_mfma16(xq[mb][0], bv[mat][b2], a);
                            a = nmoe_mfma16(xq[mb][1], bv[mat][b2], a);
                            a = nmoe_mfma16(xq[mb][2], bv[mat][b2], a);
#pragma unroll
                            for (int i = 0; i < 4; i++) a[i] = __builtin_fmaf(-128.0f, t[i], a[i]);
                        }
                        acc[mat][b2][mb] = a;
                    }
                }
        }
        auto step = [&](int gs, const int st, const bool ahead) {
            nmoe_ring_step_barrier<XPL * AI + CP::PER_WAVE, G / GPS, NS>(gs);
            if (ahead) issue(gs + NS - 1, (st + NS - 1) % NS);
            /* the step's scales: one bf16, or both groups' in one word */
            uint32_t sw[2][NB];
#pragma unroll
            for (int mat = 0; mat < 2; mat++)
#pragma unroll
                for (int b2 = 0; b2 < NB; b2++) {
                    const uint16_t *sp = &s_s[mat][(GPS * gs) >> 3][rt0 + 16 * b2][(GPS * gs) & 7];
                    sw[mat][b2] = GPS == 2 ? *(const uint32_t *)sp : (uint32_t)*sp;
                }
#pragma unroll
            for (int u = 0; u < GPS; u++) {
                uint4 bq[2][NB][2];
                float sg[2][NB];
#pragma unroll
                for (int mat = 0; mat < 2; mat++)
#pragma unroll
                    for (int b2 = 0; b2 < NB; b2++) {
                        uint32_t w0, w1;
                        /* kept apart: two reads merged into one instruction lose
                         * the stage they belong to, and then wait for every stage */
                        if (u + mat + b2 > 0) asm volatile("" ::: "memory");
                        nmoe_code_read<BITS>(stage(st).b + mat * NT * CR::WPS, coff[u][b2], w0, w1);
                        nmoe_codes_bf16<BITS>(w0, w1, bq[mat][b2][0], bq[mat][b2][1]);
                        sg[mat][b2] = nmoe_bf16f((uint16_t)(sw[mat][b2] >> (16 * u)));
                    }
#pragma unroll
                for (int mb = 0; mb < MB; mb++) {
                    if (mb < nb) {
                        uint4 a[XPL][2];
#pragma unroll
                        for (int pl = 0; pl < XPL; pl++)
                            nmoe_stage_operand(stage(st).a[pl], MCH * u + 16 * mb + col, kb, a[pl][0], a[pl][1]);
#pragma unroll
                        for (int mat = 0; mat < 2; mat++)
#pragma unroll
                            for (int b2 = 0; b2 < NB; b2++) {
                                nmoe_f32x4 pp =
                                    nmoe_mfma16(a[0][0], bq[mat][b2][0], nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f});
                                pp = nmoe_mfma16(a[0][1], bq[mat][b2][1], pp);
                                if (XPL == 2) {
                                    pp = nmoe_mfma16(a[XPL - 1][0], bq[mat][b2][0], pp);
                                    pp = nmoe_mfma16(a[XPL - 1][1], bq[mat][b2][1], pp);
                                }
#pragma unroll
                                for (int i = 0; i < 4; i++)
                                    acc[mat][b2][mb][i] = __builtin_fmaf(sg[mat][b2], pp[i], acc[mat][b2][mb][i]);
                            }
                    }
                }
            }
        };
        nmoe_ring_run<G / GPS, NS>(step);
        {
            /* epilogue: act = SiLU(gate) * up as hi + lo bf16, in the down
             * kernel's operand order; group sums of act rows (a down group
             * is 64 act columns, WPD wavefronts of this tile) */
            float part_sum[MB][4] = {};
            /* the act planes as buffers: a scalar base and a 32-bit lane
             * offset per store (no 64-bit address arithmetic) */
            const __amdgpu_buffer_rsrc_t rhi = nmoe_buffer(ahi), rlo = nmoe_buffer(alo);
            /* byte offset of this lane's act column in a row, per column block */
            uint32_t cb[NB];
#pragma unroll
            for (int b2 = 0; b2 < NB; b2++) {
                const int r = nt * NT + rt0 + 16 * b2; /* act column */
                cb[b2] = 2u * (uint32_t)(16 * (r >> 4) + nmoe_kperm_inv<BITS>(r & 15));
            }
#pragma unroll
            for (int mb = 0; mb < MB; mb++) {
                if (mb >= nb) continue;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t m = m0 + 16 * mb + 4 * kb + i;
                    /* the row's byte offset from the (uniform) plane base */
                    const uint32_t ro = (p0 + min(m, n - 1)) * (uint32_t)(NMOE_INTER * 2);
                    float part = 0.0f;
#pragma unroll
                    for (int b2 = 0; b2 < NB; b2++) {
                        const float av = nmoe_silu_fast(acc[0][b2][mb][i]) * acc[1][b2][mb][i];
                        const uint32_t h = nmoe_bf16_cvt(av);
                        const uint32_t l = nmoe_bf16_cvt(av - nmoe_bf16f(h));
                        part = part + (nmoe_bf16f(h) + nmoe_bf16f(l));
                        if (m < n) {
                            __builtin_amdgcn_raw_buffer_store_b16((uint16_t)h, rhi, ro + cb[b2], 0, 0);
                            __builtin_amdgcn_raw_buffer_store_b16((uint16_t)l, rlo, ro + cb[b2], 0, 0);
                        }
                    }
                    /* the wavefront's 2 NB x 16 act columns of this row */
                    part_sum[mb][i] = nmoe_dpp_group_sum<16>(part);
                }
            }
            if (col == 0)
#pragma unroll
                for (int mb = 0; mb < MB; mb++)
#pragma unroll
                    for (int i = 0; i < 4; i++) s_as[wave][16 * mb + 4 * kb + i] = part_sum[mb][i];
        }
        nmoe_lds_barrier();
        constexpr int DG = NT / 64;  /* down groups per tile */
        constexpr int WPD = NW / DG; /* wavefronts per down group */
        if (tid < DG * MCH) {
            const int dg = tid / MCH, row = tid % MCH;
            const uint32_t m = m0 + row;
            float t = s_as[WPD * dg][row];
#pragma unroll
            for (int q = 1; q < WPD; q++) t = t + s_as[WPD * dg + q][row];
            if (m < n) as[(size_t)(p0 + m) * (NMOE_INTER / NMOE_GROUP) + DG * nt + dg] = t;
        }
        nmoe_lds_barrier(); /* s_tok, s_as and the stages are reused by the next pass */
    }
    };
    /* block-uniform: the expert's entry count picks the form */
    if constexpr (nmoe_small_form(NW)) {
        if (n <= (uint32_t)NMOE_SMALL_PASS)
            run(std::integral_constant<int, NMOE_SMALL_PASS>{}, std::integral_constant<int, NMOE_SMALL_GPS>{});
        else
            run(std::integral_constant<int, NMOE_MCHUNK>{}, std::integral_constant<int, 1>{});
    } else {
        run(std::integral_constant<int, NMOE_MCHUNK>{}, std::integral_constant<int, 1>{});
    }
    if constexpr (COUNT) {
        /* every wavefront's act and group-sum stores complete (vmcnt 0: in
         * this die's L2), then the tile is counted */
        nmoe_wait_vm<0>();
        asm volatile("s_barrier" ::: "memory");
        if (threadIdx.x == 0) nmoe_tile_done(done + es);
    }
}

template <int BITS, int XPL, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
nmoe_grouped_gateup_kernel(const uint8_t *pack, const uint16_t *xhi, const uint16_t *xlo, const uint16_t *xs3,
                           const uint32_t *perm, const uint4 *rank, int k, int lanes, int nrows, uint16_t *ahi,
                           uint16_t *alo, float *as, uint64_t *tl) {
    nmoe_gtl_begin(tl);
    typedef nmoe_gu_lds_types<BITS, XPL, NW> T;
    __shared__ typename T::Scales s_s;
    __shared__ typename T::StageU s_st0, s_st1, s_st2, s_st3;
    __shared__ uint32_t s_tok[NMOE_MCHUNK];
    __shared__ float s_as[NW][NMOE_MCHUNK];
    /* pass lane pl of `lanes`: passes pl, pl + lanes, ... of tile (e, nt);
     * the tile's expert is the es-th by entries (most first), so the
     * longest tiles start first */
    constexpr int NTILE = NMOE_INTER / T::NT;
    const int pl = blockIdx.x / (NMOE_EXPERTS * NTILE);
    int es, nt;
    nmoe_die_tile(blockIdx.x % (NMOE_EXPERTS * NTILE), NTILE, es, nt);
    /* (five stages measured no faster than four) */
    nmoe_gu_tile<BITS, XPL, NW, nmoe_gu_stages(BITS, XPL, NW), false>(pack, xhi, xlo, xs3, perm, rank, k, lanes, nrows,
                                                                      ahi, alo, as, es, nt, pl, s_s, s_st0, s_st1,
                                                                      s_st2, s_st3, s_tok, s_as, NULL);
    nmoe_gtl_end(tl, 1, rank, es, nt, pl, nrows);
}

/* ------------------------------------------------------------ down */

/* Down rows per block of NW wavefronts: 64 a wavefront. */
__host__ __device__ constexpr int nmoe_dn_rows(int nw) { return nw * 64; }

/* Bytes of one down stage (act hi and lo rows, codes) of a tile of nt
 * rows with mch entries a pass and gps groups a step; a stage buffer holds
 * either form's. */
__host__ __device__ constexpr int nmoe_dn_stage(int bits, int nt, int mch, int gps) {
    return 2 * gps * mch * 128 + nt * gps * (bits == 4 ? 32 : 16);
}
__host__ __device__ constexpr int nmoe_dn_stage_max(int bits, int nw, int nt) {
    return nmoe_small_form(nw) && nmoe_dn_stage(bits, nt, NMOE_SMALL_PASS, NMOE_SMALL_GPS) >
                                      nmoe_dn_stage(bits, nt, NMOE_MCHUNK, 1)
               ? nmoe_dn_stage(bits, nt, NMOE_SMALL_PASS, NMOE_SMALL_GPS)
               : nmoe_dn_stage(bits, nt, NMOE_MCHUNK, 1);
}
/* LDS bytes of a down block with ns stages: the stages, the scales and
 * s_q. */
__host__ __device__ constexpr int nmoe_dn_lds(int bits, int nw, int nt, int ns) {
    return ns * nmoe_dn_stage_max(bits, nw, nt) + nt * 16 + 4 * NMOE_MCHUNK;
}
__host__ __device__ constexpr int nmoe_dn_stages(int bits, int nw) {
    return nmoe_dn_lds(bits, nw, nmoe_dn_rows(nw), 4) <= (nw == 8 ? 160 : 80) * 1024 - 512 ? 4 : 3;
}

/* The LDS of a down block of NT-row tiles (the scales of the tile, and
 * stage buffers as in the gate/up block). */
template <int BITS, int NW, int NT>
struct nmoe_dn_lds_types {
    typedef uint16_t Scales[NT][NMOE_INTER / NMOE_GROUP];
    typedef nmoe_stage<2, NMOE_MCHUNK, NT * nmoe_code_row<BITS, 1>::WPS> StageB;
    typedef nmoe_stage<2, NMOE_SMALL_GPS * NMOE_SMALL_PASS, NT * nmoe_code_row<BITS, NMOE_SMALL_GPS>::WPS> StageS;
    typedef nmoe_stage_buf<StageB, typename std::conditional<nmoe_small_form(NW), StageS, StageB>::type> StageU;
    static_assert(sizeof(StageU) == nmoe_dn_stage_max(BITS, NW, NT), "stage buffer size");
};

/* Down tile nt (NT rows) of the es-th expert by entries, pass lane pl:
 * y[q][row] for all the expert's entries q, 64 per pass (16 in one pass in
 * the small form), with NS stages in the given LDS buffers.  NW wavefronts
 * (as in the gate/up kernel); wavefront w owns rows (NT/NW)w .. +NT/NW-1 of
 * the tile as NB 16-row column blocks.  act enters as hi and lo bf16
 * planes.
 *
 * WAIT (the gate/up tiles run in the same launch): with its weight loads
 * in flight, a bounded wait until done[es] counts all gu_tiles gate/up
 * tiles of each pass lane that has work; those ran on this block's die (the
 * same block index mod 8; nmoe_wait_tiles checks it), so their act rows
 * are in this die's L2.  The act rows are then read through L1 as usual (no
 * block of this launch read them before they were complete: an act row is
 * 1 KB, whole cache lines), the group sums, whose 32-byte rows share cache
 * lines with other experts' rows, with loads that bypass L1. */
template <int BITS, int NW, int NT, int NS, bool WAIT>
__device__ __forceinline__ void nmoe_dn_tile(const uint8_t *pack, const uint16_t *ahi, const uint16_t *alo,
                                             const float *as, const uint32_t *perm, const uint4 *rank, int lanes,
                                             int nrows, float *y, int es, int nt, int pl,
                                             typename nmoe_dn_lds_types<BITS, NW, NT>::Scales &s_s,
                                             typename nmoe_dn_lds_types<BITS, NW, NT>::StageU &s_st0,
                                             typename nmoe_dn_lds_types<BITS, NW, NT>::StageU &s_st1,
                                             typename nmoe_dn_lds_types<BITS, NW, NT>::StageU &s_st2,
                                             typename nmoe_dn_lds_types<BITS, NW, NT>::StageU &s_st3,
                                             uint32_t (&s_q)[NMOE_MCHUNK], uint32_t *done, int gu_tiles,
                                             uint32_t *sync, uint32_t spin, uint64_t *tl) {
    using Q = nmoe_q<BITS>;
    using L = nmoe_layout<BITS>;
    constexpr int G = NMOE_INTER / NMOE_GROUP; /* 8 groups */
    static_assert(G == 8, "the correction's operand layout assumes 2 groups per lane");
    static_assert(NW == 8 || NW == 4, "eight or four wavefronts");
    static_assert(NS == 3 || NS == 4, "three or four stages");
    static_assert(NT % (16 * NW) == 0, "whole column blocks per wavefront");
    constexpr int NB = NT / (16 * NW);
    typedef typename nmoe_dn_lds_types<BITS, NW, NT>::StageU StageU;
    const uint4 rk = nmoe_rank_entry(rank, es); /* clamped as in the gate/up kernel */
    const int e = (int)min(rk.x, (uint32_t)(NMOE_EXPERTS - 1));
    const uint32_t p0 = min(rk.y, (uint32_t)nrows), n = min(rk.z, (uint32_t)nrows - p0);
    if (n <= (uint32_t)(pl * NMOE_MCHUNK)) return;
    static_assert(!WAIT || NS == 3, "the split prologue's waits are written for three stages");
    const int tid = threadIdx.x, lane = tid & 63, col = lane & 15, kb = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint8_t *ex = pack + (size_t)e * L::expert_size;
    const int rt0 = (NT / NW) * wave + col; /* tile row of column block nb: rt0 + 16 nb */
    const uint32_t *cbase = (const uint32_t *)(ex + L::down_w); /* stripe-major */
    const uint16_t *bias = (const uint16_t *)(ex + L::down_b) + (size_t)nt * NT * G;

    /* the passes of one form: MCH entries a pass, GPS groups a ring step */
    auto run = [&](auto mch_c, auto gps_c) {
    constexpr int MCH = decltype(mch_c)::value, GPS = decltype(gps_c)::value;
    constexpr int MB = MCH / 16;           /* row blocks per full pass */
    constexpr int AI = GPS * MCH / 8 / NW; /* A instructions per plane and wavefront a step */
    static_assert(AI >= 1 && AI * NW * 8 == GPS * MCH, "A rows split evenly over the wavefronts");
    using CR = nmoe_code_row<BITS, GPS>;
    using CP = nmoe_code_plan<BITS, NT, NW, GPS>;
    typedef nmoe_stage<2, GPS * MCH, NT * CR::WPS> Stage;
    auto stage = [&](int st) -> Stage & {
        StageU &b = st == 0 ? s_st0 : st == 1 ? s_st1 : st == 2 ? s_st2 : s_st3;
        if constexpr (MCH == NMOE_MCHUNK) return b.big;
        else return b.small;
    };
    /* the lane's code-word offsets in the stage codes (as in the gate/up kernel) */
    uint32_t coff[GPS][NB];
#pragma unroll
    for (int u = 0; u < GPS; u++)
#pragma unroll
        for (int b2 = 0; b2 < NB; b2++) coff[u][b2] = nmoe_code_off<BITS, GPS>(rt0 + 16 * b2, u, kb);
    for (uint32_t m0 = pl * MCH; m0 < n; m0 += lanes * MCH) {
        /* the chunk's output slots, stored to LDS after the stages are issued
         * (so that this load's wait does not hold them back) and visible
         * after the barrier below */
        const uint32_t qv = tid < MCH ? min(perm[p0 + min(m0 + tid, n - 1)], (uint32_t)nrows - 1u) : 0u;
        /* this lane's A row for instruction j = wave + NW i (group
         * j / (MCH / 8) of the step): act row p0 + m0 + 8 (j % (MCH / 8)) +
         * lane / 8 */
        uint32_t row_off[AI];
#pragma unroll
        for (int i = 0; i < AI; i++)
            row_off[i] = (p0 + min(m0 + 8 * ((wave + NW * i) % (MCH / 8)) + (lane >> 3), n - 1)) *
                         (uint32_t)(NMOE_INTER * 2);
        const uint16_t *apl[2] = {ahi, alo};
        /* a stage's act rows (2 AI loads) and its codes (CP::PER_WAVE loads) */
        auto issue_a = [&](int gs, int st) {
#pragma unroll
            for (int pl = 0; pl < 2; pl++)
#pragma unroll
                for (int i = 0; i < AI; i++) {
                    const int j = wave + NW * i;
                    nmoe_stage_rows(stage(st).a[pl], apl[pl] + 64 * (GPS * gs + j / (MCH / 8)), row_off[i], j, lane);
                }
        };
        auto issue_b = [&](int gs, int st) {
#pragma unroll
            for (int i = 0; i < CP::PER_WAVE; i++)
                nmoe_stage_codes<BITS, NT, CP::WIDE, GPS>(stage(st).b, cbase, Q::WPR_D, nt * NT, gs,
                                                          CP::PER_WAVE * wave + i, lane);
        };
        auto issue = [&](int gs, int st) {
            issue_a(gs, st);
            issue_b(gs, st);
        };
        const int nb = (int)min((n - m0 + 15) / 16, (uint32_t)MB);
        nmoe_f32x4 acc[NB][MB];
        {
            /* as in the gate/up kernel: the correction's operands
             * (scales straight into LDS, one 16-byte chunk a thread,
             * every pass), then the first ring stages, then a wait that
             * leaves only the stages in flight.
             * A lane = (entry col, groups 2kb + tq), B lane = (row col,
             * groups 2kb + tq) */
            static_assert(NT * G / 8 % 64 == 0 && NT * G / 8 <= 64 * NW, "at most one scale chunk per thread");
            if (NT * G / 8 == 64 * NW || tid < NT * G / 8) /* wavefront-uniform */
                __builtin_amdgcn_global_load_lds(
                    (const void *)((const uint4 *)(ex + L::down_s + (size_t)nt * NT * G * 2) + tid),
                    (nmoe_lds_void *)((uint4 *)&s_s[0][0] + 64 * wave), 16, 0, 0);
            float2 av[MB];
            uint32_t bv[NB];
            auto load_av = [&]() {
#pragma unroll
                for (int mb = 0; mb < MB; mb++) {
                    const float *ap = as + (size_t)(p0 + min(m0 + 16 * mb + col, n - 1)) * G + 2 * kb;
                    if constexpr (WAIT)
                        av[mb] = __builtin_bit_cast(float2, __hip_atomic_load((nmoe_g64 *)ap, __ATOMIC_RELAXED,
                                                                              __HIP_MEMORY_SCOPE_AGENT));
                    else
                        av[mb] = *(const float2 *)ap;
                }
            };
            if constexpr (WAIT) {
                /* the weights first (they do not wait for the gate/up
                 * tiles): biases and the first stages' codes; then, on the
                 * first pass, the wait for the expert's gate/up tiles (a
                 * barrier that leaves the loads in flight); then the act
                 * side: group sums and the first stages' act rows.  The wait
                 * below leaves only stage 1's act rows in flight, so stage 0
                 * is complete before the ring's first step. */
#pragma unroll
                for (int b2 = 0; b2 < NB; b2++) bv[b2] = *(const uint32_t *)(bias + (rt0 + 16 * b2) * G + 2 * kb);
#pragma unroll
                for (int st = 0; st < NS - 1; st++) issue_b(st, st);
                if (m0 == (uint32_t)(pl * MCH)) {
                    if (tid == 0) {
                        const uint32_t busy = min((uint32_t)lanes, (n + NMOE_MCHUNK - 1) / NMOE_MCHUNK);
                        /* the entry's fourth word: its place in the gate/up order */
                        nmoe_wait_tiles(done + (rk.w & (NMOE_EXPERTS - 1)), (uint32_t)gu_tiles * busy, sync, spin);
                        nmoe_gtl_stamp(tl, NMOE_GTL_READY);
                    }
                    nmoe_lds_barrier();
                }
                load_av();
#pragma unroll
                for (int st = 0; st < NS - 1; st++) issue_a(st, st);
                nmoe_wait_vm<(NS - 2) * 2 * AI>();
            } else {
                load_av();
#pragma unroll
                for (int b2 = 0; b2 < NB; b2++) bv[b2] = *(const uint32_t *)(bias + (rt0 + 16 * b2) * G + 2 * kb);
#pragma unroll
                for (int st = 0; st < NS - 1; st++) issue(st, st);
                nmoe_wait_vm<(NS - 1) * (2 * AI + CP::PER_WAVE)>();
            }
            if (tid < MCH) s_q[tid] = qv;
            nmoe_lds_barrier(); /* the scales and s_q */
            float cv[NB][G / 4];
#pragma unroll
            for (int b2 = 0; b2 < NB; b2++) {
                const uint32_t sw = *(const uint32_t *)&s_s[rt0 + 16 * b2][2 * kb];
                cv[b2][0] = __uint_as_float(bv[b2] << 16) - 128.0f * __uint_as_float(sw << 16);
                cv[b2][1] = __uint_as_float(bv[b2] & 0xffff0000u) - 128.0f * __uint_as_float(sw & 0xffff0000u);
#pragma unroll
                for (int mb = 0; mb < MB; mb++) acc[b2][mb] = nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
#pragma unroll
            for (int tq = 0; tq < G / 4; tq++)
#pragma unroll
                for (int mb = 0; mb < MB; mb++)
                    if (mb < nb)
#pragma unroll
                        for (int b2 = 0; b2 < NB; b2++)
                            acc[b2][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(tq == 0 ? av[mb].x : av[mb].y,
                                                                               cv[b2][tq], acc[b2][mb], 0, 0, 0);
        }
        auto step = [&](int gs, const int st, const bool ahead) {
            nmoe_ring_step_barrier<2 * AI + CP::PER_WAVE, G / GPS, NS>(gs);
            if (ahead) issue(gs + NS - 1, (st + NS - 1) % NS);
            /* the step's scales: one bf16, or both groups' in one word */
            uint32_t sw[NB];
#pragma unroll
            for (int b2 = 0; b2 < NB; b2++) {
                const uint16_t *sp = &s_s[rt0 + 16 * b2][GPS * gs];
                sw[b2] = GPS == 2 ? *(const uint32_t *)sp : (uint32_t)*sp;
            }
#pragma unroll
            for (int u = 0; u < GPS; u++) {
                uint4 bq[NB][2];
                float sg[NB];
#pragma unroll
                for (int b2 = 0; b2 < NB; b2++) {
                    uint32_t w0, w1;
                    /* kept apart, as in the gate/up kernel */
                    if (u + b2 > 0) asm volatile("" ::: "memory");
                    nmoe_code_read<BITS>(stage(st).b, coff[u][b2], w0, w1);
                    nmoe_codes_bf16<BITS>(w0, w1, bq[b2][0], bq[b2][1]);
                    sg[b2] = nmoe_bf16f((uint16_t)(sw[b2] >> (16 * u)));
                }
#pragma unroll
                for (int mb = 0; mb < MB; mb++) {
                    if (mb < nb) {
                        uint4 h0, h1, l0, l1;
                        nmoe_stage_operand(stage(st).a[0], MCH * u + 16 * mb + col, kb, h0, h1);
                        nmoe_stage_operand(stage(st).a[1], MCH * u + 16 * mb + col, kb, l0, l1);
#pragma unroll
                        for (int b2 = 0; b2 < NB; b2++) {
                            nmoe_f32x4 pp = nmoe_mfma16(h0, bq[b2][0], nmoe_f32x4{0.0f, 0.0f, 0.0f, 0.0f});
                            pp = nmoe_mfma16(h1, bq[b2][1], pp);
                            pp = nmoe_mfma16(l0, bq[b2][0], pp);
                            pp = nmoe_mfma16(l1, bq[b2][1], pp);
#pragma unroll
                            for (int i = 0; i < 4; i++)
                                acc[b2][mb][i] = __builtin_fmaf(sg[b2], pp[i], acc[b2][mb][i]);
                        }
                    }
                }
            }
        };
        nmoe_ring_run<G / GPS, NS>(step);
#pragma unroll
        for (int b2 = 0; b2 < NB; b2++) {
            const int r = nt * NT + rt0 + 16 * b2;
#pragma unroll
            for (int mb = 0; mb < MB; mb++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t m = m0 + 16 * mb + 4 * kb + i;
                    if (mb < nb && m < n) y[(size_t)s_q[m - m0] * NMOE_HIDDEN + r] = acc[b2][mb][i];
                }
            }
        }
        nmoe_lds_barrier(); /* the stages and s_q are reused by the next pass */
    }
    };
    /* block-uniform: the expert's entry count picks the form */
    if constexpr (nmoe_small_form(NW)) {
        if (n <= (uint32_t)NMOE_SMALL_PASS) {
            run(std::integral_constant<int, NMOE_SMALL_PASS>{}, std::integral_constant<int, NMOE_SMALL_GPS>{});
            return;
        }
    }
    run(std::integral_constant<int, NMOE_MCHUNK>{}, std::integral_constant<int, 1>{});
}

template <int BITS, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
nmoe_grouped_down_kernel(const uint8_t *pack, const uint16_t *ahi, const uint16_t *alo, const float *as,
                         const uint32_t *perm, const uint4 *rank, int lanes, int nrows, float *y, uint64_t *tl) {
    nmoe_gtl_begin(tl);
    constexpr int NT = nmoe_dn_rows(NW);
    typedef nmoe_dn_lds_types<BITS, NW, NT> T;
    __shared__ typename T::Scales s_s;
    __shared__ typename T::StageU s_st0, s_st1, s_st2, s_st3;
    __shared__ uint32_t s_q[NMOE_MCHUNK]; /* the chunk's output slots */
    /* pass lane and tile as in the gate/up kernel */
    constexpr int NTILE = NMOE_HIDDEN / NT;
    const int pl = blockIdx.x / (NMOE_EXPERTS * NTILE);
    int es, nt;
    nmoe_die_tile(blockIdx.x % (NMOE_EXPERTS * NTILE), NTILE, es, nt);
    nmoe_dn_tile<BITS, NW, NT, nmoe_dn_stages(BITS, NW), false>(pack, ahi, alo, as, perm, rank, lanes, nrows, y, es,
                                                                nt, pl, s_s, s_st0, s_st1, s_st2, s_st3, s_q, NULL, 0,
                                                                NULL, 0u, NULL);
    nmoe_gtl_end(tl, 2, rank, es, nt, pl, nrows);
}

/* ------------------------------------------------------------ gate/up + down in one launch */

/* Rows of a down tile when the down tiles share the launch with the gate/up
 * tiles: 32 a wavefront, so that a stage of either GEMM fits one stage
 * buffer and two blocks still share a CU. */
__host__ __device__ constexpr int nmoe_ffn_dn_rows(int nw) { return nw * 32; }
__host__ __device__ constexpr int nmoe_imax(int a, int b) { return a > b ? a : b; }
/* LDS bytes of the one-launch block with ns stages: stage buffers and
 * scales of either GEMM, s_tok (s_q) and s_as. */
__host__ __device__ constexpr int nmoe_ffn_lds(int bits, int xpl, int nw, int ns) {
    return ns * nmoe_imax(nmoe_gu_stage_max(bits, xpl, nw), nmoe_dn_stage_max(bits, nw, nmoe_ffn_dn_rows(nw))) +
           nmoe_imax(2 * nmoe_gu_rows(xpl, nw) * 64, nmoe_ffn_dn_rows(nw) * 16) + 4 * NMOE_MCHUNK * (1 + nw);
}
/* Three stages: the down tiles' split prologue waits for them (four-wavefront
 * blocks have no room for a fourth; eight-wavefront ones take three too). */
__host__ __device__ constexpr int nmoe_ffn_stages(int, int, int) { return 3; }

/* Gate/up and down of the grouped experts in one launch (one pass lane):
 * blocks 0 .. ngu-1 are the gate/up tiles (as nmoe_grouped_gateup_kernel's
 * grid), the blocks after them the down tiles of nmoe_ffn_dn_rows(NW) rows
 * (as nmoe_grouped_down_kernel's grid, from block ngu on, over the second
 * list of rank[]: the down tiles' order, nmoe_down_entry).  A down tile
 * waits (bounded) for its expert's gate/up tiles, which count themselves in
 * done[] (zeroed by the preparation launch) at the expert's gate/up entry,
 * so the down tiles of the experts finished first fill the CUs that the
 * last gate/up tiles leave idle, instead of waiting for the whole gate/up
 * launch to end.
 *
 * Where the tiles run: blocks are dealt to the eight dies in turn, block b
 * to die (b + c) mod 8 with c fixed within the launch (checked at context
 * creation, else this kernel is not used), and ngu is a multiple of 8, so
 * the gate/up and down tiles of one expert (the same entry mod 8 in either
 * order) run on one die and its L2 holds their act rows (nmoe_wait_tiles
 * checks it).
 * A die starts its blocks in index order, so every gate/up block a down
 * block waits for has started before it, and gate/up blocks wait for
 * nothing: each wait ends. */
template <int BITS, int XPL, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
nmoe_grouped_ffn_kernel(const uint8_t *pack, const uint16_t *xhi, const uint16_t *xlo, const uint16_t *xs3,
                        const uint32_t *perm, const uint4 *rank, int k, int nrows, uint16_t *ahi, uint16_t *alo,
                        float *as, float *y, int ngu, uint32_t *done, uint32_t *sync, uint32_t spin, uint64_t *tl) {
    nmoe_gtl_begin(tl);
    typedef nmoe_gu_lds_types<BITS, XPL, NW> TG;
    constexpr int NTD = nmoe_ffn_dn_rows(NW);
    typedef nmoe_dn_lds_types<BITS, NW, NTD> TD;
    constexpr int NS = nmoe_ffn_stages(BITS, XPL, NW);
    union StageV {
        typename TG::StageU gu;
        typename TD::StageU dn;
    };
    union ScalesV {
        typename TG::Scales gu;
        typename TD::Scales dn;
    };
    static_assert(sizeof(StageV) * NS + sizeof(ScalesV) + 4 * NMOE_MCHUNK * (1 + NW) ==
                      (size_t)nmoe_ffn_lds(BITS, XPL, NW, NS),
                  "LDS size");
    __shared__ ScalesV s_s;
    __shared__ StageV s_st0, s_st1, s_st2, s_st3;
    __shared__ uint32_t s_tok[NMOE_MCHUNK]; /* the gate/up tile's tokens, the down tile's output slots */
    __shared__ float s_as[NW][NMOE_MCHUNK];
    constexpr int NTG = NMOE_INTER / TG::NT, NTILED = NMOE_HIDDEN / NTD;
    int es, nt;
    if ((int)blockIdx.x < ngu) {
        nmoe_die_tile(blockIdx.x, NTG, es, nt);
        nmoe_gu_tile<BITS, XPL, NW, NS, true>(pack, xhi, xlo, xs3, perm, rank, k, 1, nrows, ahi, alo, as, es, nt, 0,
                                              s_s.gu, s_st0.gu, s_st1.gu, s_st2.gu, s_st3.gu, s_tok, s_as, done);
        nmoe_gtl_end(tl, 1, rank, es, nt, 0, nrows);
    } else {
        /* the down tiles' order (the dispatch's second list) */
        nmoe_die_tile(blockIdx.x - ngu, NTILED, es, nt);
        nmoe_dn_tile<BITS, NW, NTD, NS, true>(pack, ahi, alo, as, perm, rank + NMOE_EXPERTS, 1, nrows, y, es, nt, 0,
                                              s_s.dn, s_st0.dn, s_st1.dn, s_st2.dn, s_st3.dn, s_tok, done, NTG, sync,
                                              spin, tl);
        nmoe_gtl_end(tl, 2, rank + NMOE_EXPERTS, es, nt, 0, nrows);
    }
}

/* ------------------------------------------------------------ combine */

/* out[t] = h_mid[t] + sum_{s<k} w[t][s] y[t*k+s] in slot order
 * (kernels.metal:1394-1423) (+ sigmoid(g) * shared_out); a slot whose index
 * is outside the layer contributes nothing (runtime.m:2977-2981). */
/* A set status word (a bounded wait of this or an earlier launch gave up
 * and the host has not read the status yet) makes the combine write NaN:
 * y may rest on a dispatch that never completed. */
__device__ __forceinline__ bool nmoe_status_set(const uint32_t *status) {
    return __hip_atomic_load((nmoe_g32 *)status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}

/* The same for rows not 16-byte aligned: one row per thread. */
__global__ void __launch_bounds__(256) nmoe_grouped_combine_rows_kernel(const float *y, const uint32_t *idx,
                                                                         const float *w, int k, const float *h_mid,
                                                                         const float *shared_out,
                                                                         const float *shared_gate_raw,
                                                                         const uint32_t *status, float *out) {
    const int t = blockIdx.y, r = blockIdx.x * 256 + threadIdx.x;
    float moe = 0.0f;
    for (int s = 0; s < k; s++) {
        const size_t q = (size_t)t * k + s;
        if (idx[(size_t)t * NMOE_MAX_K + s] < NMOE_EXPERTS) moe += w[(size_t)t * NMOE_MAX_K + s] * y[q * NMOE_HIDDEN + r];
    }
    float o = h_mid[(size_t)t * NMOE_HIDDEN + r] + moe;
    if (shared_out != NULL) o = o + nmoe_sigmoid_dev(shared_gate_raw[t]) * shared_out[(size_t)t * NMOE_HIDDEN + r];
    out[(size_t)t * NMOE_HIDDEN + r] = nmoe_status_set(status) ? __builtin_nanf("") : o;
}

__global__ void __launch_bounds__(64) nmoe_grouped_combine_kernel(const float *y, const uint32_t *idx,
                                                                   const float *w, int k, const float *h_mid,
                                                                   const float *shared_out,
                                                                   const float *shared_gate_raw,
                                                                   const uint32_t *status, float *out) {
    /* four consecutive rows per thread, one wavefront a block (eight blocks a
     * token, so that 64 tokens already spread over every CU); all k partial
     * rows are loaded before the sum (an invalid slot's row was never
     * written: its value is dropped by the select, never multiplied into
     * the sum) */
    const int t = blockIdx.y, r = 4 * (blockIdx.x * 64 + threadIdx.x);
    float4 yv[NMOE_MAX_K];
#pragma unroll
    for (int s = 0; s < NMOE_MAX_K; s++)
        if (s < k) yv[s] = *(const float4 *)(y + ((size_t)t * k + s) * NMOE_HIDDEN + r);
    const float4 h = *(const float4 *)(h_mid + (size_t)t * NMOE_HIDDEN + r);
    float m[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < NMOE_MAX_K; s++) {
        if (s >= k) break;
        const bool valid = idx[(size_t)t * NMOE_MAX_K + s] < NMOE_EXPERTS;
        const float ws = w[(size_t)t * NMOE_MAX_K + s];
        const float v[4] = {yv[s].x, yv[s].y, yv[s].z, yv[s].w};
#pragma unroll
        for (int i = 0; i < 4; i++) m[i] = valid ? m[i] + ws * v[i] : m[i];
    }
    float o[4] = {h.x + m[0], h.y + m[1], h.z + m[2], h.w + m[3]};
    if (shared_out != NULL) {
        const float g = nmoe_sigmoid_dev(shared_gate_raw[t]);
        const float4 sh = *(const float4 *)(shared_out + (size_t)t * NMOE_HIDDEN + r);
        o[0] = o[0] + g * sh.x, o[1] = o[1] + g * sh.y, o[2] = o[2] + g * sh.z, o[3] = o[3] + g * sh.w;
    }
    if (nmoe_status_set(status)) o[0] = o[1] = o[2] = o[3] = __builtin_nanf("");
    *(float4 *)(out + (size_t)t * NMOE_HIDDEN + r) = make_float4(o[0], o[1], o[2], o[3]);
}

/* ------------------------------------------------------------ stripes */

/* dst = src with each expert's three code matrices stripe-major
 * (nmoe_stripe_word) and everything else (scales, biases) in place: one
 * 16-byte word a thread, which never straddles a group (q4 groups are 32
 * bytes, q2 16).  The matrices all hold wpm words: gate and up 512 rows,
 * down 2,048 rows. */
template <int BITS>
__global__ void __launch_bounds__(256) nmoe_stripe_kernel(const uint4 *src, uint4 *dst) {
    using L = nmoe_layout<BITS>;
    using Q = nmoe_q<BITS>;
    constexpr uint32_t E16 = L::expert_size / 16u, GW = nmoe_gwords<BITS>();
    const uint32_t mat[3] = {L::gate_w, L::up_w, L::down_w};
    const uint32_t wpr[3] = {(uint32_t)Q::WPR_G, (uint32_t)Q::WPR_G, (uint32_t)Q::WPR_D};
    constexpr uint32_t MW = (uint32_t)NMOE_INTER * Q::WPR_G; /* words a matrix */
    static_assert((uint32_t)NMOE_HIDDEN * Q::WPR_D == MW, "three matrices of the same size");
    const uint64_t n = (uint64_t)NMOE_EXPERTS * E16;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t e = (uint32_t)(i / E16), b = 16u * (uint32_t)(i % E16); /* expert, byte in the expert */
        uint32_t to = b;
#pragma unroll
        for (int m = 0; m < 3; m++)
            if (b >= mat[m] && b < mat[m] + 4u * MW) {
                const uint32_t wd = (b - mat[m]) / 4u, r = wd / wpr[m], c = wd % wpr[m];
                to = mat[m] + 4u * (nmoe_stripe_word(r, c / GW, GW, wpr[m]) + c % GW);
            }
        dst[(uint64_t)e * E16 + to / 16u] = src[i];
    }
}

int nmoe_pack_stripe(nmoe_hip_ctx *ctx, int layer) {
    const nmoe_pack_slot *slot = &ctx->packs[layer];
    const dim3 grid(ctx->num_cus * 8);
    if (slot->bits == 4)
        hipLaunchKernelGGL(nmoe_stripe_kernel<4>, grid, dim3(256), 0, ctx->stream, (const uint4 *)slot->dev,
                           (uint4 *)slot->stripes);
    else
        hipLaunchKernelGGL(nmoe_stripe_kernel<2>, grid, dim3(256), 0, ctx->stream, (const uint4 *)slot->dev,
                           (uint4 *)slot->stripes);
    NMOE_HIP_TRY(ctx, hipGetLastError());
    /* complete before the call returns, as the upload's copy is: a grouped
     * call may follow on any stream */
    NMOE_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return NMOE_HIP_OK;
}

/* ------------------------------------------------------------ host */

extern "C" int nmoe_grouped_init(nmoe_hip_ctx *ctx) {
    const size_t mt = (size_t)ctx->max_tokens, rows = mt * NMOE_MAX_K;
    ctx->grouped_min_tokens = 8;
    if (hipMalloc((void **)&ctx->g_counts, NMOE_DISPATCH_MAX * NMOE_EXPERTS * sizeof(uint64_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_perm, rows * sizeof(uint32_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_offsets, (NMOE_EXPERTS + 1) * sizeof(uint32_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_rank, 2 * NMOE_EXPERTS * 4 * sizeof(uint32_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_xhi, mt * NMOE_HIDDEN * sizeof(uint16_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_xlo, mt * NMOE_HIDDEN * sizeof(uint16_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_xs, mt * 3 * (NMOE_HIDDEN / NMOE_GROUP) * sizeof(uint16_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_ahi, rows * NMOE_INTER * sizeof(uint16_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_alo, rows * NMOE_INTER * sizeof(uint16_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_as, rows * (NMOE_INTER / NMOE_GROUP) * sizeof(float)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_y, rows * NMOE_HIDDEN * sizeof(float)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_done, NMOE_SCHED_WORDS * sizeof(uint32_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->g_tags, rows * sizeof(uint64_t)) != hipSuccess)
        return NMOE_HIP_ENOMEM;
    ctx->grouped_one_launch = ctx->xcd_placed;
    ctx->skew_tiles = -1;
    /* the dispatch's words start in range (epoch 0, which no launch takes):
     * a launch whose wait for the slices' histograms gives up then reads
     * zeros, never uninitialised counts */
    if (hipMemset(ctx->g_counts, 0, NMOE_DISPATCH_MAX * NMOE_EXPERTS * sizeof(uint64_t)) != hipSuccess ||
        hipMemset(ctx->g_perm, 0, rows * sizeof(uint32_t)) != hipSuccess ||
        hipMemset(ctx->g_offsets, 0, (NMOE_EXPERTS + 1) * sizeof(uint32_t)) != hipSuccess ||
        hipMemset(ctx->g_rank, 0, 2 * NMOE_EXPERTS * 4 * sizeof(uint32_t)) != hipSuccess ||
        hipMemset(ctx->g_done, 0, NMOE_SCHED_WORDS * sizeof(uint32_t)) != hipSuccess ||
        hipMemset(ctx->g_tags, 0, rows * sizeof(uint64_t)) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess)
        return NMOE_HIP_EHIP;
    return NMOE_HIP_OK;
}

extern "C" void nmoe_grouped_free(nmoe_hip_ctx *ctx) {
    void *p[] = {ctx->g_counts, ctx->g_perm, ctx->g_offsets, ctx->g_rank, ctx->g_xhi, ctx->g_xlo,
                 ctx->g_xs,     ctx->g_ahi,  ctx->g_alo,     ctx->g_as,   ctx->g_y,   ctx->g_done, ctx->g_tags};
    for (void *q : p)
        if (q != NULL) (void)hipFree(q);
}

/* D1 + D2 into perm / offsets (any device buffers of T*k and 257 words). */
extern "C" int nmoe_grouped_dispatch(nmoe_hip_ctx *ctx, const uint32_t *idx, int ntok, int k, uint32_t *perm,
                                     uint32_t *offsets, hipStream_t s) {
    const int nd = nmoe_dispatch_blocks(ntok * k);
#define NMOE_DISPATCH_LAUNCH(M)                                                                                        \
    hipLaunchKernelGGL((nmoe_grouped_prep_kernel<4, uint16_t, false, M>), dim3(nd), dim3(256), 0, s, idx, ntok, k, nd, \
                       ctx->g_counts, perm, offsets, (uint4 *)ctx->g_rank, ctx->sync, ctx->spin_limit,                 \
                       (const uint16_t *)NULL, (uint16_t *)NULL, (uint16_t *)NULL, (uint16_t *)NULL,                   \
                       (const float *)NULL, (uint32_t *)NULL, (float *)NULL, (uint32_t *)NULL, -1, (uint64_t *)NULL,    \
                       (uint64_t *)NULL)
    if (nd > 1)
        NMOE_DISPATCH_LAUNCH(true);
    else
        NMOE_DISPATCH_LAUNCH(false);
#undef NMOE_DISPATCH_LAUNCH
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? NMOE_HIP_OK : nmoe_hip_check(ctx, e, "dispatch launch");
}

/* logits != NULL: the routing from those logits in the preparation launch
 * (idx / w are then its outputs, [ntok][8]); else idx / w are given. */
template <int BITS>
static int nmoe_grouped_run(nmoe_hip_ctx *ctx, const uint8_t *pack, const void *x, int x_dtype, int ntok, int k,
                            const uint32_t *idx, const float *w, const float *h_mid, const float *shared_out,
                            const float *shared_gate_raw, float *out, hipStream_t s, const float *logits = NULL) {
    const bool bf = x_dtype == NMOE_HIP_BF16;
    const int nd = nmoe_dispatch_blocks(ntok * k);
    const dim3 gprep(nd + (logits != NULL ? (ntok + 3) / 4 : 0) + ntok);
    uint32_t *ri = (uint32_t *)idx;
    float *rw = (float *)w;
    /* two pass lanes once an expert averages more than half a pass: the
     * passes of a large expert's tile then run in blocks of their own, side
     * by side (on the same die, so the second reads the codes from L2) */
    const int lanes = (long)ntok * k > (long)NMOE_EXPERTS * NMOE_MCHUNK / 2 ? 2 : 1;
    /* gate/up and down in one launch where the blocks' dies are known (one
     * pass lane) */
    const bool one = ctx->grouped_one_launch && ctx->xcd_placed && lanes == 1;
    uint32_t *done = one ? ctx->g_done : NULL;
    const int skew = one ? ctx->skew_tiles : -1;
    if (one) ctx->skew_tiles = -1;
    /* timeline builds: 4 stamps a block of the preparation launch */
    uint64_t *tlp = nmoe_tl_take(ctx, (int)((4 * (size_t)gprep.x + NMOE_TL_SLOT_WORDS - 1) / NMOE_TL_SLOT_WORDS));
#define NMOE_PREP_M(XT, R, XLO, M)                                                                                      \
    hipLaunchKernelGGL((nmoe_grouped_prep_kernel<BITS, XT, R, M>), gprep, dim3(256), 0, s, idx, ntok, k, nd,              \
                       ctx->g_counts, ctx->g_perm, ctx->g_offsets, (uint4 *)ctx->g_rank, ctx->sync, ctx->spin_limit,    \
                       (const XT *)x, ctx->g_xhi, XLO, ctx->g_xs, logits, ri, rw, done, skew, ctx->g_tags, tlp)
    /* (one slice: the form without the slices' histogram exchange, and its registers) */
#define NMOE_PREP(XT, R, XLO)                 \
    do {                                      \
        if (nd > 1)                           \
            NMOE_PREP_M(XT, R, XLO, true);    \
        else                                  \
            NMOE_PREP_M(XT, R, XLO, false);   \
    } while (0)
    if (logits != NULL) {
        if (bf)
            NMOE_PREP(uint16_t, true, (uint16_t *)NULL);
        else
            NMOE_PREP(float, true, ctx->g_xlo);
    } else {
        if (bf)
            NMOE_PREP(uint16_t, false, (uint16_t *)NULL);
        else
            NMOE_PREP(float, false, ctx->g_xlo);
    }
#undef NMOE_PREP
#undef NMOE_PREP_M
    constexpr int NW = NMOE_GROUPED_NW;
    const dim3 blk(64 * NW);
    const dim3 ggu(lanes * NMOE_EXPERTS * (NMOE_INTER / nmoe_gu_rows(bf ? 1 : 2, NW))),
        gdn(lanes * NMOE_EXPERTS * (NMOE_HIDDEN / nmoe_dn_rows(NW)));
    const uint16_t *xhi = (const uint16_t *)ctx->g_xhi, *xlo = (const uint16_t *)ctx->g_xlo;
    const uint32_t *perm = (const uint32_t *)ctx->g_perm;
    const uint4 *rank = (const uint4 *)ctx->g_rank;
    const uint16_t *ahi = (const uint16_t *)ctx->g_ahi, *alo = (const uint16_t *)ctx->g_alo;
    const uint16_t *xs3 = ctx->g_xs;
    const float *as = (const float *)ctx->g_as;
    const int nrows = ntok * k;
    /* timeline builds: 4 stamps a block of the GEMM launches */
    const dim3 gffn(ggu.x + NMOE_EXPERTS * (NMOE_HIDDEN / nmoe_ffn_dn_rows(NW)));
    const size_t tl_recs = one ? gffn.x : ggu.x + gdn.x;
    const int tl_slots = (int)((4 * tl_recs + NMOE_TL_SLOT_WORDS - 1) / NMOE_TL_SLOT_WORDS);
    uint64_t *tl = nmoe_tl_take(ctx, tl_slots);
    if (one) {
        /* gate/up tiles, then the down tiles of nmoe_ffn_dn_rows rows, in one grid */
        if (bf)
            hipLaunchKernelGGL((nmoe_grouped_ffn_kernel<BITS, 1, NW>), gffn, blk, 0, s, pack, xhi, xlo, xs3, perm, rank,
                               k, nrows, ctx->g_ahi, ctx->g_alo, ctx->g_as, ctx->g_y, (int)ggu.x, done, ctx->sync,
                               ctx->spin_limit, tl);
        else
            hipLaunchKernelGGL((nmoe_grouped_ffn_kernel<BITS, 2, NW>), gffn, blk, 0, s, pack, xhi, xlo, xs3, perm, rank,
                               k, nrows, ctx->g_ahi, ctx->g_alo, ctx->g_as, ctx->g_y, (int)ggu.x, done, ctx->sync,
                               ctx->spin_limit, tl);
    } else {
        /* gate/up, then down */
        if (bf)
            hipLaunchKernelGGL((nmoe_grouped_gateup_kernel<BITS, 1, NW>), ggu, blk, 0, s, pack, xhi, xlo, xs3, perm,
                               rank, k, lanes, nrows, ctx->g_ahi, ctx->g_alo, ctx->g_as, tl);
        else
            hipLaunchKernelGGL((nmoe_grouped_gateup_kernel<BITS, 2, NW>), ggu, blk, 0, s, pack, xhi, xlo, xs3, perm,
                               rank, k, lanes, nrows, ctx->g_ahi, ctx->g_alo, ctx->g_as, tl);
        hipLaunchKernelGGL((nmoe_grouped_down_kernel<BITS, NW>), gdn, blk, 0, s, pack, ahi, alo, as, perm, rank, lanes,
                           nrows, ctx->g_y, tl == NULL ? tl : tl + 4 * (size_t)ggu.x);
    }
    const uint32_t *status = ctx->sync + NMOE_SYNC_STATUS;
    if (nmoe_aligned(h_mid, 16) && nmoe_aligned(out, 16) && (shared_out == NULL || nmoe_aligned(shared_out, 16)))
        hipLaunchKernelGGL(nmoe_grouped_combine_kernel, dim3(NMOE_HIDDEN / 256, ntok), dim3(64), 0, s,
                           (const float *)ctx->g_y, idx, w, k, h_mid, shared_out, shared_gate_raw, status, out);
    else
        hipLaunchKernelGGL(nmoe_grouped_combine_rows_kernel, dim3(NMOE_HIDDEN / 256, ntok), dim3(256), 0, s,
                           (const float *)ctx->g_y, idx, w, k, h_mid, shared_out, shared_gate_raw, status, out);
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

/* The routing from given logits ([ntok][256]) in the preparation launch,
 * then the grouped experts: idx / w ([ntok][8]) receive the routing. */
extern "C" int nmoe_grouped_experts_routed(nmoe_hip_ctx *ctx, int bits, const uint8_t *pack, const float *logits,
                                           const void *x, int x_dtype, int ntok, int k, uint32_t *idx, float *w,
                                           const float *h_mid, const float *shared_out, const float *shared_gate_raw,
                                           float *out, hipStream_t s) {
    if (bits == 4)
        return nmoe_grouped_run<4>(ctx, pack, x, x_dtype, ntok, k, idx, w, h_mid, shared_out, shared_gate_raw, out, s,
                                   logits);
    return nmoe_grouped_run<2>(ctx, pack, x, x_dtype, ntok, k, idx, w, h_mid, shared_out, shared_gate_raw, out, s,
                               logits);
}
