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
 * and the step is one launch of 256 blocks x 10 wavefronts (8 workers that
 * stream and multiply expert rows, 2 control wavefronts that route).
 *
 * Blocks form 8 groups of 32 (group g = block % 8, j = block / 8); group g
 * streams expert slot g.
 *
 *   N  (stack variant) every block derives x = RMSNorm(h) itself, bit-exact
 *      with math.m:34-65.
 *   R  block b computes router row b in its candidate wavefront: the 1 MB
 *      router is read once per step (one 4 KB row per block).
 *   T  every block waits for all 256 logits and routes the token: the
 *      candidate wavefront selects the k largest logits, the exact
 *      wavefront runs math.m's softmax / top-k / renormalise bit for bit.
 *   P  block j of group g issues all weight loads of slot g at once: gate/up
 *      rows 16j..16j+15 and down rows 64j..64j+63 (~55 KB per block, the
 *      whole 14 MB of expert weights in flight across the grid).
 *   G  gate/up dot products + SwiGLU -> act[g][512].
 *   D  block j waits for act[g], computes y_g = down_g . act[g] for rows
 *      64j..64j+63 -> ypart[g].
 *   C  block j of group j % K (XBLOCK: of group 0, so that all combining
 *      blocks share a die) polls the other groups' partials of rows
 *      64j..64j+63 and combines out = h_mid + sum_s w_s y_s
 *      (+ sigmoid(g) * shared) in slot order.
 *
 * The candidates (the k largest logits) are handed to the workers one
 * selection round at a time, so group s starts streaming expert s while
 * later rounds and the exact softmax still run; the exact result confirms
 * each group's expert (or re-points it, on probability ties) before act is
 * published.  The expert weights are loaded non-temporally: read once per
 * step, they would otherwise evict the routers from the memory-side cache.
 *
 * Values a block waits for cross blocks as 64-bit (epoch, value) words
 * written and read with one device-coherent (sc1) access each; a consumer
 * polls the words it needs until all carry this launch's epoch.  That merges
 * "wait" and "fetch" into one memory round trip: no barrier counter and no
 * L2-wide cache maintenance.  The epoch is the launch count, kept per block
 * (each block increments its own word once per launch, so all agree).  The
 * combine of a chunk polls the chunk's K-1 other partials in one block.
 * Idle groups (K < 8) exit after their router row (XBLOCK: and their
 * shared-down rows).  Every wait is bounded.
 *
 * Forms (XMODE): x given (fp32 / bf16), x = RMSNorm(h) (XNORM), the whole
 * MoE half of a model layer (XBLOCK: weighted norms, the shared expert in
 * phases S1/S2, the next layer's norm N), and the layer loop of one token
 * (XSTACK, nmoe_fused_stack_kernel): all layers in one launch, with the
 * routing kept inside each die (the die's 32 blocks compute all 256 logits
 * from router rows fetched into LDS a layer ahead), every block combining
 * its chunk so that each die holds the whole next h, and the next layer's
 * norm from the combining blocks' partial sums of squares.  In the loop,
 * layer l's words carry epoch e + l, and the regions a die a layer ahead
 * could overwrite early (logits, partials) come in two sets by layer parity.
 */
#include <string.h>

#include "nmoe_device.h"

#pragma clang fp contract(off)

static __constant__ uint64_t nmoe_fused_exp2_tab[32] = NMOE_EXP2_TAB32;

#define NMOE_FUSED_BLOCKS 256
#define NMOE_FUSED_GROUPS 8
#define NMOE_FUSED_GROUP_BLOCKS (NMOE_FUSED_BLOCKS / NMOE_FUSED_GROUPS) /* 32 */
#define NMOE_FUSED_CHUNK (NMOE_HIDDEN / NMOE_FUSED_GROUP_BLOCKS)         /* 64 output rows per block */
#define NMOE_FUSED_GU_ROWS (NMOE_INTER / NMOE_FUSED_GROUP_BLOCKS)        /* 16 gate/up rows per block */
#define NMOE_FUSED_S2_ROWS (NMOE_FUSED_CHUNK / NMOE_FUSED_GROUPS)        /* 8 shared-down rows per block */
#define NMOE_FUSED_WORKERS 8 /* worker wavefronts per block, plus two control wavefronts */
#define NMOE_FUSED_THREADS (64 * (NMOE_FUSED_WORKERS + 2))
#define NMOE_FUSED_CTRL NMOE_FUSED_WORKERS        /* router row, candidate selection */
#define NMOE_FUSED_EXACT (NMOE_FUSED_WORKERS + 1) /* exact routing, group assignment */


/* exchange scratch layout (64-bit tagged words) */
/* Words that many blocks poll sit 64 bytes apart (SP words): polling a
 * densely packed word array from every block serialises on its few cache
 * lines (measured: the last of 256 packed words is seen ~2.6 us after it is
 * written by 256 polling blocks, ~1.2 us when the words are 64 B apart). */
#define NMOE_XCH_SP 8
/* The act words of a group are polled by the group's own 32 blocks on one
 * die and sit densely packed: 16 rows of one writer block share one
 * 128-byte line, so a poll round is 32 line reads per block. */
#define NMOE_XCH_ASP 1
#define NMOE_XCH_LOGITS 0
#define NMOE_XCH_ACT (NMOE_XCH_SP * NMOE_EXPERTS)
#define NMOE_XCH_YPART (NMOE_XCH_ACT + NMOE_XCH_SP * NMOE_FUSED_GROUPS * NMOE_INTER)
#define NMOE_XCH_WORDS (NMOE_XCH_YPART + NMOE_FUSED_GROUPS * NMOE_HIDDEN) /* tagged partials, polled by one block */
static_assert(NMOE_XCH_WORDS * sizeof(uint64_t) == NMOE_FUSED_XCH_BYTES, "exchange size as the host allocates it");
/* The whole-block form (XBLOCK) adds: the shared expert's activations
 * [512] (dense: every block reads all of them once, mostly after they are
 * written), each combining block's sum of squares of its output rows (a
 * double as two words), its output rows themselves (read only on the
 * exact-replay path of the next-layer norm) and the shared expert's down
 * rows [2048] (each polled by the one combining block of its chunk). */
#define NMOE_XCH_SHACT NMOE_XCH_WORDS
#define NMOE_XCH_NSQ (NMOE_XCH_SHACT + NMOE_INTER)
#define NMOE_XCH_NOUT (NMOE_XCH_NSQ + 2 * NMOE_FUSED_GROUP_BLOCKS)
#define NMOE_XCH_SHD (NMOE_XCH_NOUT + NMOE_HIDDEN)
#define NMOE_XCH_WORDS_BLOCK (NMOE_XCH_SHD + NMOE_HIDDEN)
static_assert(NMOE_XCH_WORDS_BLOCK * sizeof(uint64_t) == NMOE_FUSED_XCH_BYTES_BLOCK, "the whole-block exchange size");
/* The stack form (XSTACK) routes within each die: per die and layer
 * parity the 256 logits its 32 blocks compute (8 each, dense), per die
 * the 2048 words of the next h its blocks gather followed by its 32
 * blocks' sums of squares (a double as two words each), and a second set of
 * partial-sum words (dies may run up to a layer apart once routing no
 * longer crosses them; alternating by layer parity, no block overwrites a
 * partial or a logit another block still waits for). */
#define NMOE_XCH_LGD NMOE_XCH_WORDS_BLOCK
#define NMOE_XCH_HG (NMOE_XCH_LGD + 2 * NMOE_FUSED_GROUPS * NMOE_EXPERTS)
#define NMOE_XCH_HGS (NMOE_HIDDEN + 2 * NMOE_FUSED_GROUP_BLOCKS) /* a die's words */
#define NMOE_XCH_YPART2 (NMOE_XCH_HG + NMOE_FUSED_GROUPS * NMOE_XCH_HGS)
#define NMOE_XCH_WORDS_STACK (NMOE_XCH_YPART2 + NMOE_FUSED_GROUPS * NMOE_HIDDEN)
static_assert(NMOE_XCH_WORDS_STACK * sizeof(uint64_t) == NMOE_FUSED_XCH_BYTES_STACK, "the stack exchange size");

/* x sources: XF32 / XBF16 = activations given; XNORM = x is RMSNorm(h);
 * XBLOCK = the whole MoE half of a layer: x is the weighted RMSNorm of h,
 * with the shared expert and the next layer's input norm optional. */
#define NMOE_XF32 0
#define NMOE_XBF16 1
#define NMOE_XNORM 2
#define NMOE_XBLOCK 3
/* XSTACK: all layers of one token in one launch (per layer as XNORM:
 * x_l = RMSNorm(h_l), h_{l+1} = h_l + MoE_l(x_l)) */
#define NMOE_XSTACK 4

/* ROUTE: routing given (idx_in / w_in), or computed from a bf16 or a q4 router */
#define NMOE_ROUTE_GIVEN 0
#define NMOE_ROUTE_BF16 1
#define NMOE_ROUTE_Q4 2

struct nmoe_fused_args {
    const uint8_t *pack;
    const uint16_t *router_w; /* bf16 [256][2048] (routing), or NULL with router_q4 */
    const uint32_t *router_q4; /* q4 [256][256] words, scales/biases bf16 [256][32] (routing) */
    const uint16_t *router_s;
    const uint16_t *router_b;
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
    int xcd_local; /* act travels through the die's L2 (a group's blocks share a die) */
    uint32_t spin; /* unsuccessful poll rounds a wait tolerates before it gives up */
    uint32_t epoch_arg; /* nonzero: the launch epoch (no per-block epoch words) */
    /* XBLOCK only */
    const uint16_t *norm_w; /* bf16 [2048] weight of x's RMSNorm (NULL: unit) */
    const uint16_t *next_w; /* bf16 [2048] weight of the next-layer norm (NULL: unit) */
    int add_one;            /* the weights enter as 1 + w */
    float *next_x;          /* RMSNorm(out, next_w), or NULL */
    nmoe_hip_shared_expert sh; /* the shared expert (sh.gate.w == NULL: none) */
    /* XSTACK: x = h_seq row 0, out = rows 1..nl, idx_out / w_out 8 per layer */
    int nl;
    uint64_t *tl; /* NMOE_TIMELINE builds: this launch's stamps [layers][256][16], or NULL */
};

/* When each worker asks for its down rows.  0: in the same burst as its
 * gate/up rows; 1 (default): once it has used its gate/up rows; 2: once
 * every group's candidate is known, so that the whole chip's gate/up
 * requests are ahead of the down requests; 3: once it has published its
 * act, for the confirmed expert.  Measured (q4 top-8, us): C1 step 11.62 /
 * 11.33 / 11.39 / 11.86, C3 layer 10.85 / 10.26 / 10.83 / 10.78, MoE block
 * 15.2 / 15.05 / 15.1 / 15.6.  With 1 the gate/up burst is a third smaller,
 * so it is issued sooner and the gate/up rows (two thirds of the bytes)
 * arrive sooner, while the down rows still arrive before the act exchange
 * ends; 3 waits a memory round trip too long. */
#ifndef NMOE_FUSED_DOWN_AFTER
#define NMOE_FUSED_DOWN_AFTER 1
#endif

/* Phase timeline (NMOE_TIMELINE builds): the real-time clock at a phase
 * boundary, written by the one lane that calls it to this block's stamp of
 * event ev (the order of nmoe_hip.py's TL_EVENTS) in layer ly's slot.  The
 * store is a vector store written out, so that nothing moves it. */
enum {
    NMOE_TL_START, NMOE_TL_X, NMOE_TL_LOGIT, NMOE_TL_LOGITS_IN, NMOE_TL_CAND0, NMOE_TL_CANDS, NMOE_TL_CONFIRM,
    NMOE_TL_LOADS, NMOE_TL_GU, NMOE_TL_ACT_PUB, NMOE_TL_ACT_IN, NMOE_TL_DOWN, NMOE_TL_PARTS_IN, NMOE_TL_OUT,
    NMOE_TL_NEXT, NMOE_TL_END
};
static_assert(NMOE_TL_END + 1 == NMOE_TL_EVENTS, "one stamp an event");
__device__ __forceinline__ void nmoe_tl_stamp(uint64_t *tl, int ly, int ev, float after = 0.0f) {
    if constexpr (NMOE_TIMELINE) {
        if (tl != nullptr) {
            asm volatile("" ::"v"(after)); /* a value the stamp must follow */
            const uint64_t t = __builtin_amdgcn_s_memrealtime();
            uint64_t *p = tl + ((size_t)ly * NMOE_FUSED_BLOCKS + blockIdx.x) * NMOE_TL_EVENTS + ev;
            asm volatile("global_store_dwordx2 %0, %1, off" ::"v"(p), "v"(t) : "memory");
        }
    }
}

/* XSTACK's layer table, passed by value (kernel arguments: no upload, no
 * allocation): per layer the resident pack, the router words (bf16 rows or
 * q4 words) and the q4 router's scales and biases. */
#define NMOE_STACK_MAX_LAYERS 64
struct nmoe_stack_tab {
    const void *p[4 * NMOE_STACK_MAX_LAYERS];
};

/* Die-local exchange: words written and read only by blocks of one
 * accelerator die meet in that die's L2.  The store is a plain one (the
 * vector L1 writes through to L2, and the line stays there); the load is a
 * system-scope one (sc0 sc1), which bypasses the L1 and is served by the
 * L2.  Round trip about 0.55 us instead of 0.85 us through device-coherent
 * memory, and no traffic on the fabric the expert rows stream over. */
__device__ __forceinline__ void nmoe_st_tagged_die(uint64_t *p, uint32_t epoch, float v) {
    const uint64_t w = ((uint64_t)epoch << 32) | __float_as_uint(v);
    asm volatile("global_store_dwordx2 %0, %1, off" ::"v"(p), "v"(w) : "memory");
}
__device__ __forceinline__ uint64_t nmoe_ld_tagged_die(const uint64_t *p) {
    return __hip_atomic_load((nmoe_g64 *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

/* A 16-byte load marked non-temporal (the expert weights are read once per
 * step). */
typedef unsigned int nmoe_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 nmoe_ld_nt4(const uint4 *p) {
    const nmoe_u32x4 v = __builtin_nontemporal_load((const nmoe_u32x4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
typedef __attribute__((address_space(1))) nmoe_u32x4 nmoe_gv4;
typedef __attribute__((address_space(1))) uint16_t nmoe_g16;
__device__ __forceinline__ uint4 nmoe_ld_nt4(const nmoe_gv4 *p) {
    const nmoe_u32x4 v = __builtin_nontemporal_load(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

/* A bounded wait that gave up: the status word tells the host, and the
 * block's LDS flag makes everything the block publishes from then on NaN,
 * so a result computed from words that never arrived cannot pass for a
 * valid one.  Nothing read afterwards is used as an address without a
 * clamp, so the block still finishes in bounds. */
__device__ __forceinline__ void nmoe_wait_expired(uint32_t *status, uint32_t *bad) {
    __hip_atomic_store((nmoe_g32 *)status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(bad, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

/* Polls n tagged words until all carry `epoch` (at most `spin` unsuccessful
 * rounds); returns the values (a word that never arrived leaves v[i] as it
 * was).  Each lane polls its own words. */
template <int N>
__device__ __forceinline__ void nmoe_poll(const uint64_t *const p[N], uint32_t epoch, float v[N], uint32_t *status,
                                          uint32_t *bad, uint32_t spin, bool die_local = false,
                                          uint32_t need = (1u << N) - 1u) {
    /* a word, once seen with this epoch, is not loaded again: after the
     * first round only the stragglers' words are re-polled, which keeps the
     * polling traffic off the memory channels the late writers need.  need:
     * the words to wait for (the others are left untouched) */
    uint32_t spins = 0;
    if (need == 0) return;
    for (;;) {
        uint64_t w[N];
#pragma unroll
        for (int i = 0; i < N; i++) /* all loads of a round in flight together */
            if (need & (1u << i)) w[i] = die_local ? nmoe_ld_tagged_die(p[i]) : nmoe_ld_tagged(p[i]);
#pragma unroll
        for (int i = 0; i < N; i++)
            if ((need & (1u << i)) && nmoe_tag_is(w[i], epoch)) {
                v[i] = nmoe_tag_val(w[i]);
                need &= ~(1u << i);
            }
        if (need == 0) return;
        __builtin_amdgcn_s_sleep(1);
        if (++spins > spin) {
            nmoe_wait_expired(status, bad);
            return;
        }
    }
}

/* nmoe_poll with two rounds in flight: loads return in order, so while one
 * round's words are checked the next round is already on its way, and a
 * word that lands just after a round was issued is seen about one round
 * trip later instead of two.  All N words are loaded each round (they
 * must be valid addresses); only those in `need` are waited for. */
template <int N>
__device__ __forceinline__ bool nmoe_poll2(const uint64_t *const p[N], uint32_t epoch, float v[N], uint32_t *status,
                                           uint32_t *bad, uint32_t spin, uint32_t need) {
    if (need == 0) return false;
    uint32_t spins = 0;
    uint64_t wa[N], wb[N];
    auto issue = [&](uint64_t(&w)[N]) { /* every word, so each round is N loads and the wait is vmcnt(N) */
#pragma unroll
        for (int i = 0; i < N; i++) w[i] = nmoe_ld_tagged(p[i]);
    };
    auto check = [&](const uint64_t(&w)[N]) {
#pragma unroll
        for (int i = 0; i < N; i++)
            if ((need & (1u << i)) && nmoe_tag_is(w[i], epoch)) {
                v[i] = nmoe_tag_val(w[i]);
                need &= ~(1u << i);
            }
    };
    issue(wa);
    for (;;) { /* the barriers keep each round's loads ahead of the previous round's check */
        __builtin_amdgcn_s_sleep(4);
        issue(wb);
        __builtin_amdgcn_sched_barrier(0);
        check(wa);
        if (need == 0) return false;
        __builtin_amdgcn_s_sleep(4);
        issue(wa);
        __builtin_amdgcn_sched_barrier(0);
        check(wb);
        if (need == 0) return false;
        if (++spins > spin / 2) {
            nmoe_wait_expired(status, bad);
            return true;
        }
    }
}

/* Waits (bounded) until the LDS word *w exceeds v: a hand-off from another
 * wavefront of the block that needs no block-wide barrier.  An LDS poll
 * round is about 32 times shorter than a round trip to memory, so the bound
 * is 32 times the rounds of the memory polls: the waiting wavefront then
 * gives up no sooner than the wavefront it waits for. */
/* An LDS word read by another wavefront's hand-off: ds_read_b32 written
 * out, followed by its own lgkmcnt wait.  An atomic LDS load would do, but
 * it reaches the compiler's wait placement without the alias scope that
 * tells it which LDS variable it reads; in a kernel that also loads LDS
 * directly from memory (the stack's router rows, the block form's
 * shared-down rows) the compiler then makes it wait for every load in
 * flight, the expert weight stream included.  The clobbers keep the
 * surrounding LDS accesses in program order; the hardware completes one
 * wavefront's LDS accesses in order.  The address operand is the LDS
 * offset: the low 32 bits of a generic pointer into LDS (the shared
 * aperture's base has none set), as the compiler's own generic-to-LDS
 * conversion takes it. */
__device__ __forceinline__ uint32_t nmoe_lds_read_flag(const uint32_t *w) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"((uint32_t)(size_t)w) : "memory");
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v) : : "memory");
    return v;
}

__device__ __forceinline__ void nmoe_lds_wait_above(uint32_t *w, uint32_t v, uint32_t *status, uint32_t *bad,
                                                    uint32_t spin) {
    uint32_t spins = 0;
    while (nmoe_lds_read_flag(w) <= v) {
        __builtin_amdgcn_s_sleep(1);
        if (++spins > 32u * spin) {
            nmoe_wait_expired(status, bad);
            return;
        }
    }
}

__device__ __forceinline__ bool nmoe_lds_flag(uint32_t *f) { return nmoe_lds_read_flag(f) != 0u; }

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
        if (XMODE == NMOE_XNORM || XMODE == NMOE_XBLOCK || XMODE == NMOE_XSTACK)
            for (int i = 0; i < n; i++) out[i] = (float)((double)out[i] * rinv);
    }
}

/* The weight math.m:34-65 multiplies by: bf16 w (+1 for the model's
 * zero-centred norms, math.m:58-60), 1 without a weight tensor. */
__device__ __forceinline__ float nmoe_norm_weight(const uint16_t *w, int c, int add_one) {
    if (w == NULL) return 1.0f;
    const float v = nmoe_bf16f(w[c]);
    return add_one ? v + 1.0f : v;
}

/* A tagged word with a raw 32-bit payload (halves of a double). */
__device__ __forceinline__ void nmoe_st_tagged_u32(uint64_t *p, uint32_t epoch, uint32_t v) {
    __hip_atomic_store((nmoe_g64 *)p, ((uint64_t)epoch << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

template <int BITS, int ROUTE, int XMODE>
__device__ __forceinline__ void nmoe_fused_body(nmoe_fused_args a, const nmoe_stack_tab *stab) {
    using Q = nmoe_q<BITS>;
    using L = nmoe_layout<BITS>;
    constexpr int RPS = NMOE_WAVE / Q::LPR_G;   /* gate/up rows per wave step: 1 (q4) / 2 (q2) */
    constexpr int GSTEPS = NMOE_FUSED_GU_ROWS / NMOE_FUSED_WORKERS / RPS; /* gate/up rows per worker, in steps */
    constexpr int RPW_D = NMOE_WAVE / Q::LPR_D; /* down rows per wave step: 4 (q4) / 8 (q2) */
    constexpr int DSTEPS = NMOE_FUSED_CHUNK / NMOE_FUSED_WORKERS / RPW_D; /* down rows per worker, in steps */
    static_assert(GSTEPS >= 1 && DSTEPS >= 1, "rows split evenly over the worker wavefronts");
    constexpr bool STK = XMODE == NMOE_XSTACK;
    constexpr bool NORM = XMODE == NMOE_XNORM || XMODE == NMOE_XBLOCK || STK; /* x = RMSNorm(h) in the block */
    constexpr bool BLK = XMODE == NMOE_XBLOCK;
    __shared__ uint64_t s_tab[32];
    __shared__ float s_scratch[NMOE_EXPERTS];
    __shared__ float s_lg[NMOE_EXPERTS]; /* the token's logits, candidate -> exact wavefront */
    __shared__ float s_act[NMOE_INTER];
    __shared__ float s_y[NMOE_FUSED_CHUNK];
    __shared__ uint32_t s_t[4 * NMOE_MAX_K];
    __shared__ uint32_t s_cand[NMOE_MAX_K];  /* expert group g starts loading (entry + 1; 0 = not yet) */
    __shared__ uint32_t s_gx[NMOE_MAX_K];    /* expert group g streams */
    __shared__ uint32_t s_slotg[NMOE_MAX_K]; /* group streaming slot s */
    __shared__ float s_w[NMOE_MAX_K];
    __shared__ double s_dd[8];
    __shared__ float s_f[1];
    __shared__ uint32_t s_epoch;
    __shared__ uint32_t s_ncand, s_confirm, s_lgok; /* control -> workers / control -> control hand-offs */
    __shared__ uint32_t s_bad; /* a wait of this block gave up: what it publishes is NaN */
    __shared__ __align__(16) float s_h[NORM ? NMOE_HIDDEN : 4];
    /* XBLOCK: the shared expert (gate values of this block's two rows, the
     * combining block's copy of all 512 activations, its 64 shared-down
     * rows and gate score) and the hand-offs between the wavefronts */
    __shared__ __align__(16) float s_sact[BLK ? NMOE_INTER : 4];
    __shared__ float s_shg[2], s_sgr[1];
    __shared__ uint32_t s_shok;
    /* XBLOCK: the block's 8 shared-down rows (codes; scales, then biases),
     * loaded while the logits are exchanged; s_s2ok: they are in */
    __shared__ __align__(16) uint8_t s_s2w[BLK ? NMOE_FUSED_S2_ROWS * (NMOE_INTER / 2) : 16];
    __shared__ uint16_t s_s2sb[BLK ? 2 * NMOE_FUSED_S2_ROWS * (NMOE_INTER / NMOE_GROUP) : 2];
    __shared__ uint32_t s_s2ok;
    /* XSTACK: h of this layer and the next (the gather of the next one
     * never touches the rows the combine still reads), the layer's router
     * rows 8j .. 8j+7 (fetched a layer ahead; bf16: 8 x 4 KB; q4: 8 x 1 KB
     * of words, then 8 x 64 B of scales and of biases), the layer table */
    __shared__ __align__(16) float s_hin[2][STK ? NMOE_HIDDEN : 4];
    __shared__ __align__(16) uint32_t s_rrow[STK ? 8 * NMOE_HIDDEN / 2 : 4];
    __shared__ const void *s_stk[STK ? 4 * NMOE_STACK_MAX_LAYERS : 1];
    __shared__ double s_rinv; /* XSTACK: the next layer's 1 / rms, or -1 (the block computes it) */

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (!STK && tid == 0) nmoe_tl_stamp(a.tl, 0, NMOE_TL_START);
    const bool ctrl = wave >= NMOE_FUSED_CTRL; /* either control wavefront */
    const bool cwave = wave == NMOE_FUSED_CTRL;
    const int g = blockIdx.x % NMOE_FUSED_GROUPS, j = blockIdx.x / NMOE_FUSED_GROUPS;
    const int k = a.k;
    /* this block combines rows 64j .. 64j+63: XSTACK every die; XBLOCK the
     * blocks of group 0, all on one die, so that the next-layer norm's
     * partial sums never leave it; otherwise group j % k */
    const bool comb = STK || (BLK ? g == 0 : g == j % k);
    const bool has_sh = BLK && a.sh.gate.w != NULL;
    uint32_t *status = a.sync + NMOE_SYNC_STATUS;

    /* Independent loads go out first and unconditionally (loads retire in
     * order, so a later wait on one of them must not cover the big ones):
     * the launch epoch, the exp2 table entry, the residual row this thread
     * may combine; then the control wavefront's router row and x columns.
     * The epoch is the block's own launch count, or the host's when given. */
    uint32_t *ep = a.sync + NMOE_SYNC_EPOCH(blockIdx.x);
    const uint32_t ep_old = a.epoch_arg != 0u ? 0u : nmoe_ld_u32_dev(ep);
    const uint64_t tab_v = nmoe_fused_exp2_tab[tid & 31];
    const int crow = j * NMOE_FUSED_CHUNK + (tid & (NMOE_FUSED_CHUNK - 1));
    /* XBLOCK may write out over h_mid: only the combining block reads the
     * rows it will overwrite (every block's reads of h end before its first
     * barrier, long before any block writes out) */
    const float hm = STK ? 0.0f : !BLK || comb ? a.h_mid[crow] : 0.0f;
    const float sh = !BLK && a.shared_out != NULL ? a.shared_out[crow] : 0.0f;
    const float sgr = !BLK && a.shared_out != NULL ? a.shared_gate_raw[0] : 0.0f;
    /* XBLOCK: the norm weights this thread multiplies by, loaded with the
     * other independent loads (read where they are used, each is a memory
     * round trip in the middle of the norm and of the next-layer norm) */
    float nwv[BLK ? 8 : 1];
    float nxw = 1.0f;
    if (BLK) {
        if (tid < NMOE_HIDDEN / 8)
#pragma unroll
            for (int i = 0; i < 8; i++) nwv[i] = nmoe_norm_weight(a.norm_w, 8 * tid + i, a.add_one);
        if (comb && tid < NMOE_FUSED_CHUNK) nxw = nmoe_norm_weight(a.next_w, crow, a.add_one);
    }
    uint4 wv0[4]; /* the router row (not XSTACK: there it comes from LDS) */
    uint32_t wq0[4];
    uint16_t rsr0[4], rbr0[4];
    float xs_r0[32];
    if (ROUTE && cwave && !STK) {
        if (ROUTE == NMOE_ROUTE_Q4) {
            /* q4 router row: words lane + 64q (columns 8 word .. +7) and their
             * groups' scale and bias, kept raw until the dot product */
            const uint32_t *rowq = a.router_q4 + (size_t)blockIdx.x * (NMOE_HIDDEN / 8);
            const size_t g0 = (size_t)blockIdx.x * (NMOE_HIDDEN / NMOE_GROUP);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                wq0[q] = rowq[lane + 64 * q];
                rsr0[q] = a.router_s[g0 + (lane + 64 * q) / 8];
                rbr0[q] = a.router_b[g0 + (lane + 64 * q) / 8];
            }
        } else {
            const uint4 *row = (const uint4 *)(a.router_w + (size_t)blockIdx.x * NMOE_HIDDEN);
#pragma unroll
            for (int q = 0; q < 4; q++) wv0[q] = row[lane + 64 * q];
        }
        if (!NORM)
#pragma unroll
            for (int q = 0; q < 4; q++) nmoe_x_cols<XMODE>(a.x, (lane + 64 * q) * 8, 8, 1.0, xs_r0 + 8 * q);
    }
    /* XBLOCK, combining block: the shared expert's gate-score row
     * (kernels.metal:510-513), a router-like row the candidate wavefront
     * reduces after its router row */
    uint32_t sq_w[4];
    uint16_t sq_s[4], sq_b[4];
    if (has_sh && cwave && comb) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            sq_w[q] = a.sh.score.w[lane + 64 * q];
            sq_s[q] = a.sh.score.scales[(lane + 64 * q) / 8];
            sq_b[q] = a.sh.score.biases[(lane + 64 * q) / 8];
        }
    }
    if (tid < 32) s_tab[tid] = tab_v;
    /* XSTACK: router rows 8j .. 8j+7 of a layer into LDS (the exact
     * wavefront, a layer ahead of their use), by loads that write LDS
     * directly: no registers held, all 32 KB in flight at once.  The wave
     * waits for them (vmcnt) before the next layer's first barrier. */
    typedef __attribute__((address_space(3))) void nmoe_lds_void;
    auto load_rrow = [&](const void *rw, const void *rs, const void *rb) {
        const int j8 = 8 * (blockIdx.x / NMOE_FUSED_GROUPS);
        if (ROUTE == NMOE_ROUTE_Q4) {
            const uint8_t *w = (const uint8_t *)rw + (size_t)j8 * (NMOE_HIDDEN / 2);
#pragma unroll
            for (int i = 0; i < 8; i++)
                __builtin_amdgcn_global_load_lds(w + 1024 * i + 16 * lane, (nmoe_lds_void *)((uint8_t *)s_rrow + 1024 * i),
                                                 16, 0, 0);
            if (lane < 32) {
                const uint8_t *sc = (const uint8_t *)rs + (size_t)j8 * (NMOE_HIDDEN / NMOE_GROUP) * 2;
                const uint8_t *bi = (const uint8_t *)rb + (size_t)j8 * (NMOE_HIDDEN / NMOE_GROUP) * 2;
                __builtin_amdgcn_global_load_lds(sc + 16 * lane, (nmoe_lds_void *)((uint8_t *)s_rrow + 8192), 16, 0, 0);
                __builtin_amdgcn_global_load_lds(bi + 16 * lane, (nmoe_lds_void *)((uint8_t *)s_rrow + 8704), 16, 0, 0);
            }
        } else {
            const uint8_t *w = (const uint8_t *)rw + (size_t)j8 * NMOE_HIDDEN * 2;
#pragma unroll
            for (int i = 0; i < 32; i++)
                __builtin_amdgcn_global_load_lds(w + 1024 * i + 16 * lane, (nmoe_lds_void *)((uint8_t *)s_rrow + 1024 * i),
                                                 16, 0, 0);
        }
    };
    if (STK) { /* the layer table, h_0 and layer 0's router row */
        if (tid < 4 * a.nl) s_stk[tid] = stab->p[tid];
        if (tid < NMOE_HIDDEN / 4) ((float4 *)s_hin[0])[tid] = ((const float4 *)a.x)[tid];
        if (wave == NMOE_FUSED_EXACT) load_rrow(stab->p[1], stab->p[2], stab->p[3]);
    }
    const int nl = STK ? a.nl : 1;
    auto layer = [&](const int ly) {
    if (STK && wave == NMOE_FUSED_EXACT) __builtin_amdgcn_s_waitcnt(0); /* this layer's router rows are in LDS */
    if (STK) __syncthreads(); /* the layer before is done: h_l, its router rows and the LDS hand-offs are free */
    if (STK && threadIdx.x == 0) nmoe_tl_stamp(a.tl, ly, NMOE_TL_START);
    /* XSTACK: an opaque copy of the thread index, so that the per-lane
     * addresses derived from it are recomputed in each layer instead of
     * hoisted out of the loop and kept live across all of it (the wave
     * index stays the uniform one) */
    int tid_o = (int)threadIdx.x;
    if (STK) asm volatile("" : "+v"(tid_o));
    const int tid = tid_o, lane = tid_o & 63;
    uint4 wv[4];
    uint32_t wq[4];
    uint16_t rsr[4], rbr[4];
    float xs_r[32], lv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (!STK) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            wv[q] = wv0[q];
            wq[q] = wq0[q];
            rsr[q] = rsr0[q];
            rbr[q] = rbr0[q];
        }
#pragma unroll
        for (int c = 0; c < 32; c++) xs_r[c] = xs_r0[c];
    }
    /* XSTACK: an opaque copy of the exchange base, so that no per-lane
     * exchange address is hoisted out of the layer loop (they would stay
     * live across every layer) */
    uint64_t *xch = a.xch;
    if (STK) asm volatile("" : "+s"(xch));
    const uint8_t *pack = STK ? (const uint8_t *)s_stk[4 * ly] : a.pack;
    uint64_t *xlg = xch + NMOE_XCH_LOGITS;
    uint64_t *xlgd = xch + NMOE_XCH_LGD + (ly & 1) * (NMOE_FUSED_GROUPS * NMOE_EXPERTS) + g * NMOE_EXPERTS; /* XSTACK */
    uint64_t *xact = xch + NMOE_XCH_ACT + NMOE_XCH_ASP * g * NMOE_INTER;
    uint64_t *ypart = xch + (STK && (ly & 1) ? NMOE_XCH_YPART2 : NMOE_XCH_YPART);
    if (tid < NMOE_MAX_K) { /* in-range defaults for every routing word a wait may leave unwritten */
        s_cand[tid] = 0u;
        s_gx[tid] = 0u;
        s_slotg[tid] = (uint32_t)tid;
        s_w[tid] = 0.0f;
        s_t[tid] = 0u;
        s_t[NMOE_MAX_K + tid] = 0u;
    }
    if (NORM) {
        /* x = h / rms (times the norm weight, XBLOCK) once per block, into
         * LDS in the workers' swizzled chunk order (as the act): the workers
         * then hold no raw h and do no double arithmetic of their own */
        const float *hsrc = STK ? s_hin[ly & 1] : (const float *)a.x;
        /* XSTACK after layer 0: from the 32 partial sums of squares the
         * candidate wavefront summed while h was gathered */
        const double ri_pre = STK && ly > 0 ? s_rinv : -1.0;
        /* the thread's 8 h values (columns 8 tid ..), loaded once for both
         * the norm and x */
        float hv8[8];
        const double rinv = ri_pre >= 0.0 ? ri_pre : 1.0 / (double)nmoe_block_rms_exact(hsrc, a.eps, s_h, s_dd, s_f, hv8);
        if (tid < NMOE_HIDDEN / 8) {
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const int c0 = 8 * tid + 4 * q;
                float4 v;
                if (ri_pre >= 0.0) {
                    nmoe_x_cols<XMODE>(hsrc, c0, 4, rinv, &v.x);
                } else { /* x = h / rms as (float)(h * (1 / rms)), as nmoe_x_cols computes it */
                    v.x = (float)((double)hv8[4 * q] * rinv);
                    v.y = (float)((double)hv8[4 * q + 1] * rinv);
                    v.z = (float)((double)hv8[4 * q + 2] * rinv);
                    v.w = (float)((double)hv8[4 * q + 3] * rinv);
                }
                if constexpr (BLK) {
                    if (a.norm_w != NULL) { /* math.m:63: (h / rms) * weight */
                        v.x = v.x * nwv[4 * q];
                        v.y = v.y * nwv[4 * q + 1];
                        v.z = v.z * nwv[4 * q + 2];
                        v.w = v.w * nwv[4 * q + 3];
                    }
                }
                ((float4 *)s_h)[nmoe_act_slot<Q::CPL / 4>(c0) / 4] = v;
            }
        }
    }
    /* after the norm: thread 0 waits here for the launch epoch it loaded at
     * the start (a memory round trip), not before its loads of h */
    if (tid == 0) {
        if (ly == 0) {
            /* XSTACK: layer l runs with epoch e + l, and the block's word
             * keeps the last one it uses */
            uint32_t e = a.epoch_arg;
            if (e == 0u) {
                /* epochs skip 0, the tag of a cleared word: a launch whose
                 * epochs would reach it after 2^32 - 1 starts again at 1 */
                e = ep_old + 1u;
                if (e == 0u || e + (uint32_t)(nl - 1) < e) e = 1u;
                __hip_atomic_store((nmoe_g32 *)ep, e + (uint32_t)(nl - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            s_epoch = e;
            s_bad = 0u;
            s_shok = 0u;
            s_s2ok = 0u;
        }
        s_ncand = 0u;
        s_confirm = 0u;
        s_lgok = 0u;
    }
    __syncthreads();
    if (tid == 0) nmoe_tl_stamp(a.tl, ly, NMOE_TL_X);
    const uint32_t epoch = s_epoch + (STK ? (uint32_t)ly : 0u);

    /* ---- S2 (XBLOCK, every block's candidate wavefront after its routing):
     * shared-down rows 64j + 8g .. +7 (kernels.metal:1520-1537), published
     * for the block that combines chunk j.  All 512 shared activations into
     * LDS, then 16 lanes a row (32 columns each, the routed down rows' form
     * s * sum(q a) + b * sum(a) per 64-column group), four rows a step. */
    const int s2r0 = j * NMOE_FUSED_CHUNK + NMOE_FUSED_S2_ROWS * g;
    auto shared_rows = [&]() {
        const uint64_t *ps[8];
        float v[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int q = 0; q < 8; q++) ps[q] = a.xch + NMOE_XCH_SHACT + lane + 64 * q;
        nmoe_poll<8>(ps, epoch, v, status, &s_bad, a.spin);
#pragma unroll
        for (int q = 0; q < 8; q++) s_sact[lane + 64 * q] = v[q];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        nmoe_lds_wait_above(&s_s2ok, 0u, status, &s_bad, a.spin); /* the rows */
        /* the multiply-adds below the workers' priority: they fill the
         * workers' waits (their loads, the act exchange), and the combine
         * needs them only after the workers are done */
        __builtin_amdgcn_s_setprio(0);
        const int dl16 = lane & 15, rsub = lane >> 4;
        float av[32];
#pragma unroll
        for (int c = 0; c < 8; c++) *(float4 *)(av + 4 * c) = ((const float4 *)s_sact)[8 * dl16 + c];
        float asum = 0.0f;
#pragma unroll
        for (int c = 0; c < 32; c++) asum += av[c];
        const bool poisoned = nmoe_lds_flag(&s_bad);
#pragma unroll
        for (int st = 0; st < NMOE_FUSED_S2_ROWS / 4; st++) {
            const int rr = 4 * st + rsub;
            const uint4 dw = *(const uint4 *)(s_s2w + rr * (NMOE_INTER / 2) + 16 * dl16);
            const float sc = nmoe_bf16f(s_s2sb[rr * (NMOE_INTER / NMOE_GROUP) + dl16 / 2]);
            const float bi = nmoe_bf16f(s_s2sb[NMOE_FUSED_S2_ROWS * (NMOE_INTER / NMOE_GROUP) +
                                                rr * (NMOE_INTER / NMOE_GROUP) + dl16 / 2]);
            float y = __builtin_fmaf(sc, nmoe_dot16<4>(dw, av), bi * asum);
            y = nmoe_dpp_group_sum<16>(y);
            if (dl16 == 0) nmoe_st_tagged(a.xch + NMOE_XCH_SHD + s2r0 + rr, epoch, poisoned ? __builtin_nanf("") : y);
        }
    };
    if (has_sh && wave == NMOE_FUSED_EXACT) {
        /* the block's shared-down rows into LDS (2 KB of codes by loads that
         * write LDS directly, 256 B of scales and biases), while the logits
         * are exchanged (at the start they would delay the loads of h).
         * This wavefront is idle until the logits are in, long after. */
        typedef __attribute__((address_space(3))) void nmoe_lds_void_sd;
        const uint8_t *cw = (const uint8_t *)a.sh.down.w + (size_t)s2r0 * (NMOE_INTER / 2);
        constexpr int WB = NMOE_FUSED_S2_ROWS * (NMOE_INTER / 2), SN = NMOE_FUSED_S2_ROWS * (NMOE_INTER / NMOE_GROUP);
        static_assert(WB % 1024 == 0 && SN == NMOE_WAVE, "16-byte loads of whole rows; one scale a lane");
#pragma unroll
        for (int i = 0; i < WB / 1024; i++)
            __builtin_amdgcn_global_load_lds(cw + 1024 * i + 16 * lane, (nmoe_lds_void_sd *)(s_s2w + 1024 * i), 16, 0, 0);
        s_s2sb[lane] = a.sh.down.scales[(size_t)s2r0 * (NMOE_INTER / NMOE_GROUP) + lane];
        s_s2sb[SN + lane] = a.sh.down.biases[(size_t)s2r0 * (NMOE_INTER / NMOE_GROUP) + lane];
        __builtin_amdgcn_s_waitcnt(0);
        if (lane == 0) __hip_atomic_store(&s_s2ok, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }

    if (STK && !ctrl) {
        /* ---- R (XSTACK, worker wavefront w): router row 8j + w from LDS,
         * published to this die's logit words (the die's 32 blocks cover
         * all 256 rows, so routing never leaves the die) */
        float xq[32];
#pragma unroll
        for (int c = 0; c < 8; c++)
            *(float4 *)(xq + 4 * c) =
                ((const float4 *)s_h)[nmoe_act_slot<Q::CPL / 4>(8 * lane + 512 * (c >> 1) + 4 * (c & 1)) / 4];
        float logit;
        if (ROUTE == NMOE_ROUTE_Q4) {
            uint32_t w4[4];
            uint16_t s4[4], b4[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                w4[q] = s_rrow[256 * wave + lane + 64 * q];
                s4[q] = ((const uint16_t *)s_rrow)[4096 + 32 * wave + (lane + 64 * q) / 8];
                b4[q] = ((const uint16_t *)s_rrow)[4352 + 32 * wave + (lane + 64 * q) / 8];
            }
            logit = nmoe_router_row_q4(w4, s4, b4, xq);
        } else {
            uint4 w4[4];
#pragma unroll
            for (int q = 0; q < 4; q++) w4[q] = ((const uint4 *)s_rrow)[256 * wave + lane + 64 * q];
            logit = nmoe_router_row_bf16(w4, xq);
        }
        if (nmoe_lds_flag(&s_bad)) logit = __builtin_nanf(""); /* a layer before went wrong: so do all after */
        if (lane == 0) {
            if (a.xcd_local)
                nmoe_st_tagged_die(xlgd + 8 * j + wave, epoch, logit);
            else
                nmoe_st_tagged(xlgd + 8 * j + wave, epoch, logit);
            if (wave == 0) nmoe_tl_stamp(a.tl, ly, NMOE_TL_LOGIT);
        }
    }
    if (has_sh && wave < 4) {
        /* ---- S1 (XBLOCK, every block): shared gate/up rows 2b, 2b+1
         * (kernels.metal:421-469) in the router's per-element form, while
         * the routing runs: wavefronts 0, 1 reduce the gate rows, 2, 3 the
         * up rows and publish SiLU(gate) * up for every block's
         * shared-down rows */
        const int srow = 2 * blockIdx.x + (wave & 1);
        const nmoe_hip_qtensor T = wave < 2 ? a.sh.gate : a.sh.up;
        uint32_t w4[4];
        uint16_t s4[4], b4[4];
        float xq[32];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            w4[q] = T.w[(size_t)srow * (NMOE_HIDDEN / 8) + lane + 64 * q];
            s4[q] = T.scales[(size_t)srow * (NMOE_HIDDEN / NMOE_GROUP) + (lane + 64 * q) / 8];
            b4[q] = T.biases[(size_t)srow * (NMOE_HIDDEN / NMOE_GROUP) + (lane + 64 * q) / 8];
        }
#pragma unroll
        for (int c = 0; c < 8; c++)
            *(float4 *)(xq + 4 * c) =
                ((const float4 *)s_h)[nmoe_act_slot<Q::CPL / 4>(8 * lane + 512 * (c >> 1) + 4 * (c & 1)) / 4];
        const float v = nmoe_router_row_q4(w4, s4, b4, xq);
        if (wave < 2) {
            if (lane == 0) {
                s_shg[wave] = v;
                __hip_atomic_fetch_add(&s_shok, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        } else {
            nmoe_lds_wait_above(&s_shok, 1u, status, &s_bad, a.spin);
            float act = nmoe_silu_dev(s_shg[wave & 1]) * v;
            if (nmoe_lds_flag(&s_bad)) act = __builtin_nanf("");
            if (lane == 0) nmoe_st_tagged(a.xch + NMOE_XCH_SHACT + srow, epoch, act);
        }
    }

    if (ROUTE && cwave) {
        /* the control wavefronts share SIMDs with workers: their routing is
         * on the critical path, the workers' multiply-adds mostly are not */
        __builtin_amdgcn_s_setprio(2);
        /* ---- R (candidate wavefront): router row blockIdx.x (XSTACK: the
         * worker wavefronts, below) */
        if (NORM && !STK)
#pragma unroll
            for (int c = 0; c < 8; c++)
                *(float4 *)(xs_r + 4 * c) =
                    ((const float4 *)s_h)[nmoe_act_slot<Q::CPL / 4>(8 * lane + 512 * (c >> 1) + 4 * (c & 1)) / 4];
        if (!STK) {
            const float logit =
                ROUTE == NMOE_ROUTE_Q4 ? nmoe_router_row_q4(wq, rsr, rbr, xs_r) : nmoe_router_row_bf16(wv, xs_r);
            if (lane == 0) {
                nmoe_st_tagged(xlg + NMOE_XCH_SP * blockIdx.x, epoch, logit);
                nmoe_tl_stamp(a.tl, ly, NMOE_TL_LOGIT);
            }
        }
        if (has_sh && comb) { /* the shared expert's gate score, same x */
            const float v = nmoe_router_row_q4(sq_w, sq_s, sq_b, xs_r);
            if (lane == 0) s_sgr[0] = v;
        }
        if (g < k || STK) {
            /* ---- T: wait for all 256 logits and hand them to the exact
             * wavefront; the candidates are the k largest logits, published
             * one per selection round so that group s starts streaming its
             * expert as soon as candidate s is known.  Their probabilities
             * are the k largest too, up to ties, which the exact routing
             * settles. */
            const uint64_t *pl[4] = {xlg + NMOE_XCH_SP * lane, xlg + NMOE_XCH_SP * (lane + 64),
                                     xlg + NMOE_XCH_SP * (lane + 128), xlg + NMOE_XCH_SP * (lane + 192)};
            const uint64_t *pd[4] = {xlgd + lane, xlgd + lane + 64, xlgd + lane + 128, xlgd + lane + 192};
            if (STK) /* this die's 256 logits */
                nmoe_poll<4>(pd, epoch, lv, status, &s_bad, a.spin, a.xcd_local != 0);
            else
                nmoe_poll<4>(pl, epoch, lv, status, &s_bad, a.spin);
#pragma unroll
            for (int q = 0; q < 4; q++) s_lg[lane + 64 * q] = lv[q];
            if (lane == 0) {
                __hip_atomic_store(&s_lgok, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
                nmoe_tl_stamp(a.tl, ly, NMOE_TL_LOGITS_IN);
            }
            /* one wave maximum per round: the key's top 24 bits with the
             * complemented entry below make every key distinct and name
             * its entry (logits that agree in those bits go lowest entry
             * first; the exact routing corrects that where it matters).
             * Each lane keeps its four keys sorted, so a round reduces one
             * value and the winning lane shifts its next key up. */
            uint32_t key[4];
#pragma unroll
            for (int q = 0; q < 4; q++) key[q] = (nmoe_fkey(lv[q]) & 0xffffff00u) | (uint32_t)(255 - lane - 64 * q);
            {
                const uint32_t a0 = max(key[0], key[1]), b0 = min(key[0], key[1]);
                const uint32_t a1 = max(key[2], key[3]), b1 = min(key[2], key[3]);
                const uint32_t x = min(a0, a1), y = max(b0, b1);
                key[0] = max(a0, a1);
                key[1] = max(x, y);
                key[2] = min(x, y);
                key[3] = min(b0, b1);
            }
#pragma unroll
            for (int s = 0; s < NMOE_MAX_K; s++) {
                if (s < k) {
                    const uint32_t best = nmoe_wave_max_u32(key[0]);
                    if (lane == 0) {
                        __hip_atomic_store(&s_cand[s], 256u - (best & 255u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                        if (s == 0) nmoe_tl_stamp(a.tl, ly, NMOE_TL_CAND0);
                    }
                    if (key[0] == best) {
                        key[0] = key[1];
                        key[1] = key[2];
                        key[2] = key[3];
                        key[3] = 0u;
                    }
                }
            }
            if (lane == 0) {
                __hip_atomic_store(&s_ncand, (uint32_t)k, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
                nmoe_tl_stamp(a.tl, ly, NMOE_TL_CANDS);
            }
        }
        if (has_sh) shared_rows(); /* (an idle group's block: right after its logit) */
    }
    if (ROUTE && wave == NMOE_FUSED_EXACT && (g < k || STK)) {
        /* ---- exact routing (math.m softmax / top-k / renormalise), from
         * the moment the logits are in, alongside the candidate rounds and
         * the expert loads; then the expert of each group. */
        __builtin_amdgcn_s_setprio(2);
        nmoe_lds_wait_above(&s_lgok, 0u, status, &s_bad, a.spin);
        float l[4], p[4];
#pragma unroll
        for (int q = 0; q < 4; q++) l[q] = s_lg[lane + 64 * q];
        nmoe_wave_softmax(l, NMOE_EXPERTS, s_scratch, s_tab, p);
#pragma unroll
        for (int q = 0; q < 4; q++) s_scratch[lane + 64 * q] = p[q];
        nmoe_lds_wait_above(&s_ncand, (uint32_t)(k - 1), status, &s_bad, a.spin);
        /* lane s < k: group s's candidate and its probability.  With p8 the
         * smallest of these, math.m's top-k is {p > p8} plus the lowest
         * entries with p == p8, since p8 is at most the k-th largest
         * probability and equal to it once fewer than k exceed it; when
         * every p > p8 and every p == p8 belongs to a candidate, the top-k
         * is the candidate set, each group keeps its expert and only the
         * slot order (probability, ties to the lower entry) is left. */
        const bool mine = lane < k;
        const uint32_t sc = mine ? s_cand[lane] : 0u; /* 1..256 once published */
        const uint32_t c = sc != 0u ? min(sc - 1u, (uint32_t)(NMOE_EXPERTS - 1)) : 0u;
        const uint32_t pcb = mine ? __float_as_uint(s_scratch[c]) : 0xffffffffu; /* p >= 0: bits order like values */
        uint32_t p8 = 0xffffffffu;
#pragma unroll
        for (int t = 0; t < NMOE_MAX_K; t++)
            if (t < k) p8 = min(p8, (uint32_t)__builtin_amdgcn_readlane((int)pcb, t));
        int ngt = 0, neq = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            ngt += __popcll(__ballot(__float_as_uint(p[q]) > p8));
            neq += __popcll(__ballot(__float_as_uint(p[q]) == p8));
        }
        const int cgt = __popcll(__ballot(mine && pcb > p8)), ceq = __popcll(__ballot(mine && pcb == p8));
        if (ngt == cgt && neq == ceq) {
            int slot = 0;
#pragma unroll
            for (int t = 0; t < NMOE_MAX_K; t++) {
                if (t < k) {
                    const uint32_t pt = (uint32_t)__builtin_amdgcn_readlane((int)pcb, t);
                    const uint32_t ct = (uint32_t)__builtin_amdgcn_readlane((int)c, t);
                    slot += (pt > pcb || (pt == pcb && ct < c)) ? 1 : 0;
                }
            }
            if (mine) {
                s_gx[lane] = c;
                s_slotg[slot] = (uint32_t)lane;
                s_t[slot] = c;
                s_t[NMOE_MAX_K + slot] = pcb;
            } else if (lane < NMOE_MAX_K) {
                s_t[lane] = 0u; /* unused slots: entry 0, weight 0 */
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            /* math.m:134-153 in slot order */
            const float pq = mine ? __uint_as_float(s_t[NMOE_MAX_K + lane]) : 0.0f;
            float sum = 0.0f;
#pragma unroll
            for (int q = 0; q < NMOE_MAX_K; q++)
                if (q < k) sum += __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(pq), q));
            const float rinv = sum == 0.0f ? 1.0f / (float)k : 1.0f / sum;
            if (lane < NMOE_MAX_K) s_w[lane] = mine ? (sum == 0.0f ? rinv : pq * rinv) : 0.0f;
        } else {
            /* ties at the boundary (or candidates cut short by their 24-bit
             * keys): the full selection; a candidate outside it hands its
             * group to a selected expert no group holds yet */
            uint32_t si[NMOE_MAX_K], cand[NMOE_MAX_K], key[4], selkey[NMOE_MAX_K];
            float sw[NMOE_MAX_K], sel_v[NMOE_MAX_K];
#pragma unroll
            for (int q = 0; q < 4; q++) key[q] = __float_as_uint(p[q]) + 1u;
            nmoe_wave_top_keys(key, k, si, selkey);
#pragma unroll
            for (int q = 0; q < NMOE_MAX_K; q++) sel_v[q] = q < k ? __uint_as_float(selkey[q] - 1u) : 0.0f;
            nmoe_renormalize(sel_v, k, sw);
#pragma unroll
            for (int q = 0; q < NMOE_MAX_K; q++) cand[q] = (uint32_t)__builtin_amdgcn_readlane((int)c, q);
            uint32_t ct = 0, et = 0;
            float wt = 0.0f;
            bool c_in_e = false, e_in_c = false;
#pragma unroll
            for (int q = 0; q < NMOE_MAX_K; q++) {
                if (q == lane) {
                    ct = cand[q];
                    et = si[q];
                    wt = sw[q];
                }
            }
#pragma unroll
            for (int q = 0; q < NMOE_MAX_K; q++) {
                if (q < k) {
                    c_in_e = c_in_e || ct == si[q];
                    e_in_c = e_in_c || et == cand[q];
                }
            }
            const uint64_t fm = __ballot(lane < k && !c_in_e); /* groups to re-point */
            const uint64_t mm = __ballot(lane < k && !e_in_c); /* slots no group holds */
            uint32_t xg = ct;
            if (fm != 0) {
                const int fr = (int)__builtin_popcountll(fm & ((1ull << lane) - 1ull));
#pragma unroll
                for (int q = 0; q < NMOE_MAX_K; q++)
                    if (((mm >> q) & 1) && (int)__builtin_popcountll(mm & ((1ull << q) - 1ull)) == fr &&
                        ((fm >> lane) & 1))
                        xg = si[q];
            }
            uint32_t sg = 0;
#pragma unroll
            for (int q = 0; q < NMOE_MAX_K; q++)
                if (q < k && (uint32_t)__builtin_amdgcn_readlane((int)xg, q) == et) sg = (uint32_t)q;
            if (lane < NMOE_MAX_K) {
                s_gx[lane] = xg;
                s_slotg[lane] = sg;
                s_w[lane] = wt;
                s_t[lane] = et; /* written out at the end */
            }
        }
        if (lane == 0) {
            __hip_atomic_store(&s_confirm, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            nmoe_tl_stamp(a.tl, ly, NMOE_TL_CONFIRM);
        }
        /* XSTACK: the next layer's router row, while this layer streams
         * (the candidate wavefront read this one before the logits came).
         * This wavefront has nothing else to do until the block's next
         * barrier, so it waits for those loads here: then no direct LDS load
         * is pending where its path joins the workers', and the compiler
         * keeps the workers' waits for their weight rows exact (with one
         * pending, loads of two kinds share the counter and every wait after
         * the join becomes a wait for all loads) */
        if (STK && ly + 1 < nl) {
            load_rrow(s_stk[4 * (ly + 1) + 1], s_stk[4 * (ly + 1) + 2], s_stk[4 * (ly + 1) + 3]);
            __builtin_amdgcn_s_waitcnt(0);
        }
    }
    if (!ROUTE) {
        if (tid < NMOE_MAX_K) {
            uint32_t e = tid < k ? a.idx_in[tid] : 0u;
            float wv_in = tid < k ? a.w_in[tid] : 0.0f;
            /* an index outside the layer is an invalid slot: weight 0, as
             * for a failed expert read (runtime.m:2977-2981) */
            s_w[tid] = e < NMOE_EXPERTS ? wv_in : 0.0f;
            s_cand[tid] = e < NMOE_EXPERTS ? e + 1u : 1u;
            s_gx[tid] = e < NMOE_EXPERTS ? e : 0u;
            s_slotg[tid] = tid;
        }
        __syncthreads();
    }
    if (!STK && g >= k) return; /* group g streams one expert (XSTACK: idle groups still combine) */
    const bool active = !STK || g < k;

    /* ---- P (workers): issue all weight loads of this wavefront */
    const int gsub = lane / Q::LPR_G, gl = lane % Q::LPR_G, ggrp = gl * Q::CPL / NMOE_GROUP;
    const int dsub = lane / Q::LPR_D, dl = lane % Q::LPR_D, dgrp = dl * Q::CPL / NMOE_GROUP;
    const int grow0 = j * NMOE_FUSED_GU_ROWS + (NMOE_FUSED_GU_ROWS / NMOE_FUSED_WORKERS) * wave + gsub;
    const int drow0 = j * NMOE_FUSED_CHUNK + (NMOE_FUSED_CHUNK / NMOE_FUSED_WORKERS) * wave + dsub;
    /* the burst holds raw loads only: unpacking x or combining a scale with
     * its bias inside it would make the wave wait for those loads before
     * issuing the rest */
    constexpr int XV = XMODE == NMOE_XBF16 ? Q::CPL / 8 : Q::CPL / 4; /* 16-byte x chunks per lane */
    uint4 xr[XV];
    uint4 gwv[GSTEPS], uwv[GSTEPS], dwv[DSTEPS];
    uint32_t gsc[GSTEPS], gbi[GSTEPS], usc[GSTEPS], ubi[GSTEPS], dsc[DSTEPS], dbi[DSTEPS];
    /* the weights through a global-memory pointer (the stack form takes the
     * pack from its layer table in LDS as a generic one): as global loads
     * they complete in order, so the gate/up rows are used while the down
     * rows are still in flight (flat loads would make the first use wait for
     * all of them) */
    auto load_gate_up = [&](uint32_t e) {
        const nmoe_gu8 *ex = (const nmoe_gu8 *)pack + (size_t)e * L::expert_size;
#pragma unroll
        for (int i = 0; i < GSTEPS; i++) {
            int row = grow0 + i * RPS;
            gwv[i] = nmoe_ld_nt4((const nmoe_gv4 *)(ex + L::gate_w) + (size_t)row * (Q::WPR_G / 4) + gl);
            uwv[i] = nmoe_ld_nt4((const nmoe_gv4 *)(ex + L::up_w) + (size_t)row * (Q::WPR_G / 4) + gl);
            const nmoe_g16 *gs = (const nmoe_g16 *)(ex + L::gate_s) + row * Q::GPR_G + ggrp;
            const nmoe_g16 *us = (const nmoe_g16 *)(ex + L::up_s) + row * Q::GPR_G + ggrp;
            gsc[i] = __builtin_nontemporal_load(gs);
            gbi[i] = __builtin_nontemporal_load(gs + NMOE_INTER * Q::GPR_G);
            usc[i] = __builtin_nontemporal_load(us);
            ubi[i] = __builtin_nontemporal_load(us + NMOE_INTER * Q::GPR_G);
        }
    };
    auto load_down = [&](uint32_t e) {
        const nmoe_gu8 *ex = (const nmoe_gu8 *)pack + (size_t)e * L::expert_size;
#pragma unroll
        for (int i = 0; i < DSTEPS; i++) {
            int row = drow0 + i * RPW_D;
            dwv[i] = nmoe_ld_nt4((const nmoe_gv4 *)(ex + L::down_w) + (size_t)row * (Q::WPR_D / 4) + dl);
            const nmoe_g16 *ds = (const nmoe_g16 *)(ex + L::down_s) + row * Q::GPR_D + dgrp;
            dsc[i] = __builtin_nontemporal_load(ds);
            dbi[i] = __builtin_nontemporal_load(ds + NMOE_HIDDEN * Q::GPR_D);
        }
    };
    auto load_expert = [&](uint32_t e) {
        load_gate_up(e);
        __builtin_amdgcn_sched_barrier(0); /* gate/up rows ahead of the down rows */
        load_down(e);
    };
    float xs[Q::CPL];
    /* ---- G (workers): gate/up + SwiGLU -> act[g], published once the
     * control wavefront has confirmed the expert */
    float actv[GSTEPS];
    auto gate_up = [&]() {
        float xsum = 0.0f;
#pragma unroll
        for (int c = 0; c < Q::CPL; c++) xsum += xs[c];
#pragma unroll
        for (int i = 0; i < GSTEPS; i++) {
            float gv = __builtin_fmaf(nmoe_bf16f(gsc[i]), nmoe_dot16<BITS>(gwv[i], xs), nmoe_bf16f(gbi[i]) * xsum);
            float uv = __builtin_fmaf(nmoe_bf16f(usc[i]), nmoe_dot16<BITS>(uwv[i], xs), nmoe_bf16f(ubi[i]) * xsum);
            gv = nmoe_lanes_sum<Q::LPR_G>(gv);
            uv = nmoe_lanes_sum<Q::LPR_G>(uv);
            actv[i] = nmoe_silu_dev(gv) * uv;
        }
    };
    uint32_t cand_g = 0;
    if (!ctrl && active) {
        /* x first: loads retire in order, so G can start while down rows stream */
        const uint4 *xp = (const uint4 *)a.x + gl * XV;
        if (!NORM)
#pragma unroll
            for (int c = 0; c < XV; c++) xr[c] = xp[c];
        if (ROUTE) /* candidate g published by the control wavefront */
            nmoe_lds_wait_above(&s_cand[g], 0u, status, &s_bad, a.spin);
        const uint32_t cg = s_cand[g]; /* 0 only if that wait gave up */
        cand_g = cg != 0u ? min(cg - 1u, (uint32_t)(NMOE_EXPERTS - 1)) : 0u;
        __builtin_amdgcn_sched_barrier(0);
        if (NMOE_FUSED_DOWN_AFTER == 0 || (NMOE_FUSED_DOWN_AFTER == 2 && !ROUTE) ||
            (NMOE_FUSED_DOWN_AFTER == 3 && !ROUTE)) {
            load_expert(cand_g);
        } else {
            load_gate_up(cand_g);
            if (NMOE_FUSED_DOWN_AFTER == 2) { /* the down rows once every group's gate/up rows are asked for */
                nmoe_lds_wait_above(&s_ncand, (uint32_t)(k - 1), status, &s_bad, a.spin);
                __builtin_amdgcn_sched_barrier(0);
                load_down(cand_g);
            }
        }
        /* keep every weight load above in one burst: no compute hoisted into it */
        __builtin_amdgcn_sched_barrier(0);
        if (tid == 0) nmoe_tl_stamp(a.tl, ly, NMOE_TL_LOADS);
        /* x as floats, and G right away: the first use of the weight
         * registers stays on this path, so the compiler waits for the gate/up
         * rows only (where the control wavefronts' path joins this one, it
         * would wait for every load in flight: their direct LDS loads count
         * in the same counter) */
#pragma unroll
        for (int c = 0; c < XV; c++) {
            if (NORM) {
                *(float4 *)(xs + 4 * c) = ((const float4 *)s_h)[nmoe_act_slot<Q::CPL / 4>(4 * (gl * XV + c)) / 4];
            } else if (XMODE == NMOE_XBF16) {
                nmoe_unpack_bf16x8(xr[c], xs + 8 * c);
            } else {
                xs[4 * c] = __uint_as_float(xr[c].x);
                xs[4 * c + 1] = __uint_as_float(xr[c].y);
                xs[4 * c + 2] = __uint_as_float(xr[c].z);
                xs[4 * c + 3] = __uint_as_float(xr[c].w);
            }
        }
        gate_up();
        if (tid == 0) nmoe_tl_stamp(a.tl, ly, NMOE_TL_GU, actv[GSTEPS - 1]);
        if (NMOE_FUSED_DOWN_AFTER == 1) {
            /* the down rows behind the gate/up rows the whole chip asked for */
            __builtin_amdgcn_sched_barrier(0);
            load_down(cand_g);
        }
    }
    if (!ctrl && active) {
        if (ROUTE) {
            nmoe_lds_wait_above(&s_confirm, 0u, status, &s_bad, a.spin);
            const uint32_t xg = min(s_gx[g], (uint32_t)(NMOE_EXPERTS - 1));
            if (xg != cand_g) { /* probability tie at the boundary: redo with the selected expert */
                if (NMOE_FUSED_DOWN_AFTER == 3)
                    load_gate_up(xg);
                else
                    load_expert(xg);
                gate_up();
                cand_g = xg;
            }
        }
        if (ROUTE && nmoe_lds_flag(&s_bad)) /* the routing this act rests on is not the token's */
#pragma unroll
            for (int i = 0; i < GSTEPS; i++) actv[i] = __builtin_nanf("");
        if (gl == 0) {
#pragma unroll
            for (int i = 0; i < GSTEPS; i++) {
                if (a.xcd_local)
                    nmoe_st_tagged_die(xact + NMOE_XCH_ASP * (grow0 + i * RPS), epoch, actv[i]);
                else
                    nmoe_st_tagged(xact + NMOE_XCH_ASP * (grow0 + i * RPS), epoch, actv[i]);
            }
        }
        if (tid == 0) nmoe_tl_stamp(a.tl, ly, NMOE_TL_ACT_PUB);
        if (NMOE_FUSED_DOWN_AFTER == 3 && ROUTE) { /* the down rows of the confirmed expert, after its act is out */
            __builtin_amdgcn_sched_barrier(0);
            load_down(cand_g);
        }
    }

    /* q4: the down codes as floats while the act is in flight, so that D is
     * multiply-adds only (q2 has no registers to spare for this) */
    constexpr bool DPRE = BITS == 4;
    float dwf[DPRE ? DSTEPS : 1][DPRE ? Q::CPL : 1];
    if (DPRE && !ctrl && active)
#pragma unroll
        for (int i = 0; i < DSTEPS; i++) nmoe_unpack_q4(dwv[i], dwf[i]);

    /* ---- D (workers): wait for act[g], then y_g for rows 64j..64j+63 */
    if (!ctrl && active) {
        constexpr int APT = NMOE_INTER / (64 * NMOE_FUSED_WORKERS); /* act words per worker thread */
        const uint64_t *pa[APT];
        float av[APT];
#pragma unroll
        for (int q = 0; q < APT; q++) {
            pa[q] = xact + NMOE_XCH_ASP * (tid + 64 * NMOE_FUSED_WORKERS * q);
            av[q] = 0.0f;
        }
        nmoe_poll<APT>(pa, epoch, av, status, &s_bad, a.spin, a.xcd_local != 0);
#pragma unroll
        for (int q = 0; q < APT; q++) s_act[nmoe_act_slot<Q::CPL / 4>(tid + 64 * NMOE_FUSED_WORKERS * q)] = av[q];
        if (tid == 0) nmoe_tl_stamp(a.tl, ly, NMOE_TL_ACT_IN);
    }
    __syncthreads();
    if (!ctrl && active) {
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
            const float dot = DPRE ? nmoe_dot_f4(dwf[i], as) : nmoe_dot16<BITS>(dwv[i], as);
            float y = __builtin_fmaf(nmoe_bf16f(dsc[i]), dot, nmoe_bf16f(dbi[i]) * asum);
            y = nmoe_dpp_group_sum<Q::LPR_D>(y);
            if (dl == 0) s_y[(NMOE_FUSED_CHUNK / NMOE_FUSED_WORKERS) * wave + dsub + i * RPW_D] = y;
        }
    }
    __syncthreads();
    if (tid == 0) nmoe_tl_stamp(a.tl, ly, NMOE_TL_DOWN);
    /* ---- C: group j % K combines rows 64j..64j+63 (out = h_mid + sum_s
     * w_s y_s in slot order); the other groups publish their partials as
     * tagged words and are done.  The combiner polls the K-1 partials of its
     * chunk: one round trip after the last one is written. */
    const int row = j * NMOE_FUSED_CHUNK + tid;
    const bool poisoned = nmoe_lds_flag(&s_bad); /* every wait of the block is behind the barrier above */
    float rv = 0.0f; /* the combining thread's out row */
    uint64_t *xhg = xch + NMOE_XCH_HG + g * NMOE_XCH_HGS; /* XSTACK: the die's next h */
    if (tid < NMOE_FUSED_CHUNK) {
        if (!comb || (STK && active))
            nmoe_st_tagged(ypart + g * NMOE_HIDDEN + row, epoch, poisoned ? __builtin_nanf("") : s_y[tid]);
        if (comb) {
            /* the k - 1 other groups' partials and (XBLOCK) the shared
             * expert's down row */
            constexpr int NP = BLK ? NMOE_MAX_K + 1 : NMOE_MAX_K;
            const uint64_t *pp[NP];
            float ys[NP];
#pragma unroll
            for (int q = 0; q < NMOE_MAX_K; q++) {
                pp[q] = ypart + q * NMOE_HIDDEN + row;
                ys[q] = s_y[tid];
            }
            if constexpr (BLK) {
                pp[NMOE_MAX_K] = a.xch + NMOE_XCH_SHD + row;
                ys[NMOE_MAX_K] = 0.0f;
            }
            /* everything but the partials before the wait: slot s's weight
             * and the group that streams it (usually group s), the shared
             * expert's gate */
            float wsl[NMOE_MAX_K];
            uint32_t sgl[NMOE_MAX_K];
            bool ident = true;
#pragma unroll
            for (int s = 0; s < NMOE_MAX_K; s++) {
                wsl[s] = s < k ? s_w[s] : 0.0f;
                sgl[s] = s < k ? s_slotg[s] : (uint32_t)s;
                ident = ident && sgl[s] == (uint32_t)s;
            }
            const bool shared_term = BLK ? has_sh : a.shared_out != NULL;
            const float gsig = shared_term ? nmoe_sigmoid_dev(BLK ? s_sgr[0] : sgr) : 0.0f;
            const uint32_t need = (((1u << k) - 1u) & ~(active ? 1u << g : 0u)) | (has_sh ? 1u << NMOE_MAX_K : 0u);
            const bool expired = nmoe_poll2<NP>(pp, epoch, ys, status, &s_bad, a.spin, need);
            if (tid == 0) nmoe_tl_stamp(a.tl, ly, NMOE_TL_PARTS_IN);
            const float shv = BLK ? ys[NP - 1] : sh; /* (XBLOCK without a shared expert: unused) */
            /* slot order: slot s is streamed by group sgl[s] */
            float moe = 0.0f;
            if (ident) {
#pragma unroll
                for (int s = 0; s < NMOE_MAX_K; s++)
                    if (s < k) moe += wsl[s] * ys[s];
            } else {
#pragma unroll
                for (int s = 0; s < NMOE_MAX_K; s++) {
                    if (s < k) {
                        float y = ys[0];
#pragma unroll
                        for (int q = 1; q < NMOE_MAX_K; q++)
                            if (sgl[s] == (uint32_t)q) y = ys[q];
                        moe += wsl[s] * y;
                    }
                }
            }
            float r = (STK ? s_hin[ly & 1][row] : hm) + moe;
            if (shared_term) r = r + gsig * shv;
            rv = poisoned || expired ? __builtin_nanf("") : r;
            if (!STK) {
                a.out[row] = rv;
                if (tid == 0) nmoe_tl_stamp(a.tl, ly, NMOE_TL_OUT);
            } else {
                /* every die holds the same rows: one writes them out, each
                 * publishes them to its own 32 blocks */
                if (g == (j & (NMOE_FUSED_GROUPS - 1))) a.out[(size_t)ly * NMOE_HIDDEN + row] = rv;
                if (a.xcd_local)
                    nmoe_st_tagged_die(xhg + row, epoch, rv);
                else
                    nmoe_st_tagged(xhg + row, epoch, rv);
                /* and the sum of their squares for the next layer's norm
                 * (a tree of depth 6; the 32 partials' tree adds 5) */
                const double ps = nmoe_wave_sq_tree(rv);
                if (tid < 2) {
                    const uint64_t pb = __builtin_bit_cast(uint64_t, ps);
                    const uint32_t half = tid == 0 ? (uint32_t)pb : (uint32_t)(pb >> 32);
                    if (a.xcd_local)
                        nmoe_st_tagged_die(xhg + NMOE_HIDDEN + 2 * j + tid, epoch, __uint_as_float(half));
                    else
                        nmoe_st_tagged_u32(xhg + NMOE_HIDDEN + 2 * j + tid, epoch, half);
                }
            }
        }
    }
    if (BLK && comb && a.next_x != NULL && wave == 0) {
        /* ---- N (XBLOCK): the next layer's input norm of out
         * (runtime.m:2893-2900, math.m:34-65).  Each combining block
         * publishes the sum of its 64 squares (a tree of depth 6) and its
         * rows; each adds the 32 partials in one fixed order (depth 5), so
         * all reach the same mean square: the float math.m's long double
         * sum rounds to where no rounding midpoint is near, or else the
         * replay of that x87 sum over all 2048 rows in index order.  The
         * combining blocks all run on one die when blocks are dealt
         * round-robin over the dies (xcd_local): then these words stay in
         * that die's L2. */
        const double sq = nmoe_wave_sq_tree(rv);
        uint64_t *nsq = a.xch + NMOE_XCH_NSQ;
        const bool dl = a.xcd_local != 0;
        auto put = [&](uint64_t *p, uint32_t v) {
            if (dl)
                nmoe_st_tagged_die(p, epoch, __uint_as_float(v));
            else
                nmoe_st_tagged_u32(p, epoch, v);
        };
        if (lane < 2) {
            const uint64_t sb = __builtin_bit_cast(uint64_t, sq);
            put(nsq + 2 * j + lane, lane == 0 ? (uint32_t)sb : (uint32_t)(sb >> 32));
        }
        put(a.xch + NMOE_XCH_NOUT + row, __float_as_uint(rv));
        const int src = lane & (NMOE_FUSED_GROUP_BLOCKS - 1); /* lanes 32..63 poll nothing */
        const uint64_t *pq[2] = {nsq + 2 * src, nsq + 2 * src + 1};
        float pv[2] = {0.0f, 0.0f};
        nmoe_poll<2>(pq, epoch, pv, status, &s_bad, a.spin, dl, lane < NMOE_FUSED_GROUP_BLOCKS ? 3u : 0u);
        const double ps = lane < NMOE_FUSED_GROUP_BLOCKS
                              ? __builtin_bit_cast(double, ((uint64_t)__float_as_uint(pv[1]) << 32) | __float_as_uint(pv[0]))
                              : 0.0;
        float mean = nmoe_mean_sq_from_sum(nmoe_sum32_tree(ps));
        if (mean < 0.0f) {
            /* near a rounding midpoint (or tiny values): all 2048 rows, the
             * x87 running sum in index order (s_h is free: x is consumed) */
            for (int i0 = 0; i0 < NMOE_HIDDEN; i0 += 4 * NMOE_WAVE) {
                const uint64_t *po[4] = {a.xch + NMOE_XCH_NOUT + i0 + lane, a.xch + NMOE_XCH_NOUT + i0 + lane + 64,
                                         a.xch + NMOE_XCH_NOUT + i0 + lane + 128,
                                         a.xch + NMOE_XCH_NOUT + i0 + lane + 192};
                float ov[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                nmoe_poll<4>(po, epoch, ov, status, &s_bad, a.spin, dl);
#pragma unroll
                for (int q = 0; q < 4; q++) s_h[i0 + lane + 64 * q] = ov[q];
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            float t = 0.0f;
            if (lane == 0) {
                nmoe_x87 acc = nmoe_x87_zero();
                for (int i = 0; i < NMOE_HIDDEN; i++) acc = nmoe_x87_add(acc, nmoe_x87_square(s_h[i]));
                acc.e -= 11; /* / 2048, exact */
                t = nmoe_x87_to_float(acc);
            }
            mean = nmoe_readlane_f(t, 0);
        }
        float rms = nmoe_sqrtf_rn(mean + a.eps);
        rms = rms == 0.0f ? 1.0f : rms;
        float xn = (float)((double)rv * (1.0 / (double)rms));
        xn = a.next_w != NULL ? xn * nxw : xn;
        a.next_x[row] = nmoe_lds_flag(&s_bad) ? __builtin_nanf("") : xn; /* a partial that never came */
        if (lane == 0) nmoe_tl_stamp(a.tl, ly, NMOE_TL_NEXT);
    }
    if (ROUTE && blockIdx.x == 0 && cwave) {
        const int o = STK ? NMOE_MAX_K * ly : 0;
        if (lane < NMOE_MAX_K) {
            if (a.idx_out != NULL) a.idx_out[o + lane] = min(s_t[lane], (uint32_t)(NMOE_EXPERTS - 1));
            if (a.w_out != NULL) a.w_out[o + lane] = poisoned ? __builtin_nanf("") : s_w[lane];
        }
        if (a.logits_out != NULL)
#pragma unroll
            for (int q = 0; q < 4; q++) a.logits_out[lane + 64 * q] = lv[q];
    }
    if (STK && ly + 1 < nl && tid < NMOE_HIDDEN / 4) {
        /* ---- H (XSTACK): the die's 32 blocks gather h_{l+1} (all of it,
         * 4 words a thread) into the other h buffer */
        const uint64_t *ph[4] = {xhg + tid, xhg + tid + 512, xhg + tid + 1024, xhg + tid + 1536};
        float hv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        nmoe_poll<4>(ph, epoch, hv, status, &s_bad, a.spin, a.xcd_local != 0);
#pragma unroll
        for (int q = 0; q < 4; q++) s_hin[(ly + 1) & 1][tid + 512 * q] = hv[q];
        if (tid == 0) nmoe_tl_stamp(a.tl, ly, NMOE_TL_NEXT);
    }
    if (STK && ly + 1 < nl && cwave) {
        /* ---- H (XSTACK, candidate wavefront): the die's 32 sums of
         * squares (lanes 0..31, two words each) -> the next layer's 1 / rms,
         * or -1 where the float mean needs the x87 replay */
        const int src = lane & (NMOE_FUSED_GROUP_BLOCKS - 1);
        const uint64_t *pq[2] = {xhg + NMOE_HIDDEN + 2 * src, xhg + NMOE_HIDDEN + 2 * src + 1};
        float pv[2] = {0.0f, 0.0f};
        nmoe_poll<2>(pq, epoch, pv, status, &s_bad, a.spin, a.xcd_local != 0, lane < NMOE_FUSED_GROUP_BLOCKS ? 3u : 0u);
        const double ps = lane < NMOE_FUSED_GROUP_BLOCKS
                              ? __builtin_bit_cast(double, ((uint64_t)__float_as_uint(pv[1]) << 32) | __float_as_uint(pv[0]))
                              : 0.0;
        const float mean = nmoe_mean_sq_from_sum(nmoe_sum32_tree(ps));
        double ri = -1.0;
        if (mean >= 0.0f) {
            float rms = nmoe_sqrtf_rn(mean + a.eps);
            rms = rms == 0.0f ? 1.0f : rms;
            ri = 1.0 / (double)rms;
        }
        if (lane == 0) s_rinv = ri;
    }
    if (threadIdx.x == 0) nmoe_tl_stamp(a.tl, ly, NMOE_TL_END);
    };
    if constexpr (STK) {
        for (int ly = 0; ly < nl; ly++) layer(ly);
    } else {
        layer(0);
    }
}

template <int BITS, int ROUTE, int XMODE>
__global__ void __launch_bounds__(NMOE_FUSED_THREADS) nmoe_fused_decode_kernel(nmoe_fused_args a) {
    nmoe_fused_body<BITS, ROUTE, XMODE>(a, nullptr);
}

/* XSTACK: the token's layers in one launch (the layer table by value) */
template <int BITS, int ROUTE>
__global__ void __launch_bounds__(NMOE_FUSED_THREADS) nmoe_fused_stack_kernel(nmoe_fused_args a, nmoe_stack_tab t) {
    nmoe_fused_body<BITS, ROUTE, NMOE_XSTACK>(a, &t);
}

/* ----------------------------------------------------------- launching */

template <int BITS, int ROUTE, int XMODE>
static hipError_t nmoe_fused_launch(const nmoe_fused_args &args, hipStream_t s) {
    hipLaunchKernelGGL((nmoe_fused_decode_kernel<BITS, ROUTE, XMODE>), dim3(NMOE_FUSED_BLOCKS), dim3(NMOE_FUSED_THREADS), 0, s, args);
    return hipGetLastError();
}

template <int BITS, int ROUTE, int XMODE>
static int nmoe_fused_fits(int num_cus) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, nmoe_fused_decode_kernel<BITS, ROUTE, XMODE>, NMOE_FUSED_THREADS, 0) !=
        hipSuccess)
        return 0;
    return per_cu >= 1 && per_cu * num_cus >= NMOE_FUSED_BLOCKS;
}

/* Every x form the launcher may use with this router kind (the RMSNorm
 * form needs the kernel to route). */
template <int BITS, int ROUTE>
static int nmoe_stack_fits(int num_cus) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, nmoe_fused_stack_kernel<BITS, ROUTE>, NMOE_FUSED_THREADS,
                                                     0) != hipSuccess)
        return 0;
    return per_cu >= 1 && per_cu * num_cus >= NMOE_FUSED_BLOCKS;
}

template <int BITS, int ROUTE>
static int nmoe_fused_fits_all(int num_cus) {
    int ok = nmoe_fused_fits<BITS, ROUTE, NMOE_XBF16>(num_cus) && nmoe_fused_fits<BITS, ROUTE, NMOE_XF32>(num_cus);
    if constexpr (ROUTE != NMOE_ROUTE_GIVEN)
        ok = ok && nmoe_fused_fits<BITS, ROUTE, NMOE_XNORM>(num_cus) && nmoe_fused_fits<BITS, ROUTE, NMOE_XBLOCK>(num_cus) &&
             nmoe_stack_fits<BITS, ROUTE>(num_cus);
    return ok;
}

/* Which die each block runs on. */
__global__ void nmoe_xcc_probe_kernel(uint32_t *out) {
    if (threadIdx.x == 0) out[blockIdx.x] = nmoe_xcc_id();
}

/* *placed = 1 when the blocks of a 256-block grid go round-robin over the
 * 8 dies -- block b on die (b + c) % 8, c fixed within a launch (the
 * dispatcher continues its rotation from the previous launch, so c varies
 * between launches).  The blocks of a group (b % 8 equal) then share a die
 * and its L2, which the die-local exchange relies on.  Checked over launches
 * with different rotations (a 1-block launch in between shifts c).  Runs on
 * stream s and waits for that stream only (never for the whole device), so
 * it can run while another stream is being captured into a graph; it must
 * not run on a stream that is itself capturing. */
extern "C" int nmoe_probe_xcd_placement(uint32_t *d, int *placed, hipStream_t s) {
    uint32_t h[NMOE_FUSED_BLOCKS];
    *placed = 0;
    int ok = 1;
    for (int rep = 0; rep < 4 && ok; rep++) {
        hipLaunchKernelGGL(nmoe_xcc_probe_kernel, dim3(NMOE_FUSED_BLOCKS), dim3(NMOE_FUSED_THREADS), 0, s, d);
        if (hipGetLastError() != hipSuccess || hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess)
            return NMOE_HIP_EHIP;
        const uint32_t c = h[0] % NMOE_FUSED_GROUPS;
        for (int b = 0; b < NMOE_FUSED_BLOCKS; b++) ok = ok && h[b] == (uint32_t)(b + c) % NMOE_FUSED_GROUPS;
        hipLaunchKernelGGL(nmoe_xcc_probe_kernel, dim3(1 + rep), dim3(64), 0, s, d); /* shift the rotation */
    }
    if (hipStreamSynchronize(s) != hipSuccess) return NMOE_HIP_EHIP;
    *placed = ok;
    return NMOE_HIP_OK;
}

/* The fused path needs all 256 blocks resident at once (its blocks wait for
 * each other's exchange words): 1 when every variant's occupancy allows
 * that on num_cus compute units. */
extern "C" int nmoe_fused_resident(int num_cus) {
    int ok = 1;
#define NMOE_FITS_ALL(B, R) \
    ok = ok && nmoe_fused_fits_all<B, R>(num_cus)
    NMOE_FITS_ALL(4, NMOE_ROUTE_BF16);
    NMOE_FITS_ALL(4, NMOE_ROUTE_Q4);
    NMOE_FITS_ALL(4, NMOE_ROUTE_GIVEN);
    NMOE_FITS_ALL(2, NMOE_ROUTE_BF16);
    NMOE_FITS_ALL(2, NMOE_ROUTE_Q4);
    NMOE_FITS_ALL(2, NMOE_ROUTE_GIVEN);
#undef NMOE_FITS_ALL
    return ok;
}

extern "C" int nmoe_decode_init(nmoe_hip_ctx *ctx) {
    const int ok = nmoe_fused_resident(ctx->num_cus);
    ctx->fused_blocks = ok ? NMOE_FUSED_BLOCKS : 0;
    ctx->xcd_placed = 0;
    ctx->xch_bytes = NMOE_FUSED_XCH_BYTES_STACK;
    if (hipMalloc((void **)&ctx->xch, ctx->xch_bytes) != hipSuccess) return NMOE_HIP_ENOMEM;
    if (ok) { /* the probe writes into the exchange buffer, cleared afterwards */
        int r = nmoe_probe_xcd_placement((uint32_t *)ctx->xch, &ctx->xcd_placed, ctx->stream);
        if (r != NMOE_HIP_OK) return r;
    }
    ctx->use_xcd_local = ctx->xcd_placed;
    if (hipMemset(ctx->xch, 0, ctx->xch_bytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
        return NMOE_HIP_EHIP;
    return NMOE_HIP_OK;
}

template <int BITS, int ROUTE>
static hipError_t nmoe_fused_launch_x(int xmode, const nmoe_fused_args &a, hipStream_t s) {
    if (xmode == NMOE_XBF16) return nmoe_fused_launch<BITS, ROUTE, NMOE_XBF16>(a, s);
    if (xmode == NMOE_XF32) return nmoe_fused_launch<BITS, ROUTE, NMOE_XF32>(a, s);
    if constexpr (ROUTE != NMOE_ROUTE_GIVEN) {
        if (xmode == NMOE_XNORM) return nmoe_fused_launch<BITS, ROUTE, NMOE_XNORM>(a, s);
        if (xmode == NMOE_XBLOCK) return nmoe_fused_launch<BITS, ROUTE, NMOE_XBLOCK>(a, s);
    }
    return hipErrorInvalidValue;
}

/* One token through the fused launch, every buffer given: xch
 * (NMOE_FUSED_XCH_BYTES), sync (NMOE_SYNC_WORDS words: status and the
 * per-block epochs), epoch 0 = the blocks' own launch counts, else the
 * launch epoch (the caller never repeats one while words of an earlier
 * launch with it may remain).  route != 0: routing computed from `router`
 * (bf16 or q4); else given by idx_in / w_in.  xmode: NMOE_XF32 / NMOE_XBF16
 * / NMOE_XNORM / NMOE_XBLOCK (blk: its norm weights, next-layer norm and
 * shared expert; xch then NMOE_FUSED_XCH_BYTES_BLOCK).  tl: the launch's
 * timeline stamps (NMOE_TIMELINE builds), or NULL. */
extern "C" hipError_t nmoe_fused_launch_core(int bits, int route, const void *x, int xmode, float eps, int k,
                                             const nmoe_hip_router *router, const uint32_t *idx_in, const float *w_in,
                                             const float *h_mid, const float *shared_out, const float *shared_gate_raw,
                                             float *out, uint32_t *idx_out, float *w_out, float *logits_out,
                                             const uint8_t *pack, uint64_t *xch, uint32_t *sync, int xcd_local,
                                             uint32_t spin, uint32_t epoch, const nmoe_block_ext *blk,
                                             hipStream_t s, uint64_t *tl) {
    nmoe_fused_args a;
    memset(&a, 0, sizeof(a));
    a.tl = tl;
    if (blk != NULL) {
        a.norm_w = blk->norm_w;
        a.next_w = blk->next_w;
        a.add_one = blk->add_one;
        a.next_x = blk->next_x;
        a.sh = blk->sh;
    }
    a.pack = pack;
    const bool q4r = router != NULL && router->kind == NMOE_HIP_ROUTER_Q4;
    a.router_w = router != NULL && !q4r ? router->w_bf16 : NULL;
    a.router_q4 = q4r ? router->w_q4 : NULL;
    a.router_s = q4r ? router->scales : NULL;
    a.router_b = q4r ? router->biases : NULL;
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
    a.xch = xch;
    a.sync = sync;
    a.xcd_local = xcd_local;
    a.spin = spin;
    a.epoch_arg = epoch;
    hipError_t e = hipErrorInvalidValue;
    const int r = !route ? NMOE_ROUTE_GIVEN : q4r ? NMOE_ROUTE_Q4 : NMOE_ROUTE_BF16;
    if (bits == 4)
        e = r == NMOE_ROUTE_Q4     ? nmoe_fused_launch_x<4, NMOE_ROUTE_Q4>(xmode, a, s)
            : r == NMOE_ROUTE_BF16 ? nmoe_fused_launch_x<4, NMOE_ROUTE_BF16>(xmode, a, s)
                                   : nmoe_fused_launch_x<4, NMOE_ROUTE_GIVEN>(xmode, a, s);
    else
        e = r == NMOE_ROUTE_Q4     ? nmoe_fused_launch_x<2, NMOE_ROUTE_Q4>(xmode, a, s)
            : r == NMOE_ROUTE_BF16 ? nmoe_fused_launch_x<2, NMOE_ROUTE_BF16>(xmode, a, s)
                                   : nmoe_fused_launch_x<2, NMOE_ROUTE_GIVEN>(xmode, a, s);
    return e;
}

extern "C" int nmoe_fused_decode(nmoe_hip_ctx *ctx, int bits, int route, const void *x, int xmode, float eps, int k,
                                 const nmoe_hip_router *router, const uint32_t *idx_in, const float *w_in,
                                 const float *h_mid, const float *shared_out, const float *shared_gate_raw, float *out,
                                 uint32_t *idx_out, float *w_out, float *logits_out, const uint8_t *pack,
                                 hipStream_t s) {
    const hipError_t e = nmoe_fused_launch_core(bits, route, x, xmode, eps, k, router, idx_in, w_in, h_mid, shared_out,
                                                shared_gate_raw, out, idx_out, w_out, logits_out, pack, ctx->xch,
                                                ctx->sync, ctx->use_xcd_local, ctx->spin_limit, 0u, NULL, s,
                                                nmoe_tl_take(ctx, 1));
    if (e != hipSuccess) return nmoe_hip_check(ctx, e, "fused decode launch");
    return NMOE_HIP_OK;
}

/* The whole MoE half of one token's layer in one launch (XBLOCK): the
 * weighted RMSNorm of h_mid, routing, the shared expert, the experts, the
 * combine into out (which may alias h_mid) and the next layer's norm. */
extern "C" int nmoe_fused_block(nmoe_hip_ctx *ctx, int bits, const nmoe_hip_router *router, const float *h_mid,
                                float eps, int k, const nmoe_block_ext *blk, float *out, uint32_t *idx_out,
                                float *w_out, float *logits_out, const uint8_t *pack, hipStream_t s) {
    const hipError_t e = nmoe_fused_launch_core(bits, 1, h_mid, NMOE_XBLOCK, eps, k, router, NULL, NULL, h_mid, NULL, NULL,
                                                out, idx_out, w_out, logits_out, pack, ctx->xch, ctx->sync,
                                                ctx->use_xcd_local, ctx->spin_limit, 0u, blk, s, nmoe_tl_take(ctx, 1));
    if (e != hipSuccess) return nmoe_hip_check(ctx, e, "fused block launch");
    return NMOE_HIP_OK;
}

/* Every layer of one token in one launch (XSTACK), at most
 * NMOE_STACK_MAX_LAYERS: layer l streams packs[l] and routes with
 * routers[l] (all of one kind, q4r), x_l = RMSNorm(h_l) (unit weight),
 * h_seq rows 1..nl receive h_{l+1} = h_l + MoE_l(x_l), idx_seq / w_seq
 * (nullable) 8 words per layer. */
extern "C" int nmoe_fused_stack(nmoe_hip_ctx *ctx, int bits, int q4r, int nl, const uint8_t *const *packs,
                                const nmoe_hip_router *routers, float *h_seq, float eps, int k, uint32_t *idx_seq,
                                float *w_seq, hipStream_t s) {
    if (nl < 1 || nl > NMOE_STACK_MAX_LAYERS) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "stack of %d layers", nl);
    nmoe_fused_args a;
    memset(&a, 0, sizeof(a));
    nmoe_stack_tab t;
    memset(&t, 0, sizeof(t));
    for (int l = 0; l < nl; l++) {
        t.p[4 * l] = packs[l];
        t.p[4 * l + 1] = q4r ? (const void *)routers[l].w_q4 : (const void *)routers[l].w_bf16;
        t.p[4 * l + 2] = q4r ? routers[l].scales : NULL;
        t.p[4 * l + 3] = q4r ? routers[l].biases : NULL;
    }
    a.x = h_seq;
    a.out = h_seq + NMOE_HIDDEN;
    a.eps = eps;
    a.k = k;
    a.idx_out = idx_seq;
    a.w_out = w_seq;
    a.xch = ctx->xch;
    a.sync = ctx->sync;
    a.xcd_local = ctx->use_xcd_local;
    a.spin = ctx->spin_limit;
    a.nl = nl;
    a.tl = nmoe_tl_take(ctx, nl);
    if (bits == 4) {
        if (q4r)
            hipLaunchKernelGGL((nmoe_fused_stack_kernel<4, NMOE_ROUTE_Q4>), dim3(NMOE_FUSED_BLOCKS), dim3(NMOE_FUSED_THREADS), 0, s, a, t);
        else
            hipLaunchKernelGGL((nmoe_fused_stack_kernel<4, NMOE_ROUTE_BF16>), dim3(NMOE_FUSED_BLOCKS), dim3(NMOE_FUSED_THREADS), 0, s, a, t);
    } else {
        if (q4r)
            hipLaunchKernelGGL((nmoe_fused_stack_kernel<2, NMOE_ROUTE_Q4>), dim3(NMOE_FUSED_BLOCKS), dim3(NMOE_FUSED_THREADS), 0, s, a, t);
        else
            hipLaunchKernelGGL((nmoe_fused_stack_kernel<2, NMOE_ROUTE_BF16>), dim3(NMOE_FUSED_BLOCKS), dim3(NMOE_FUSED_THREADS), 0, s, a, t);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return nmoe_hip_check(ctx, e, "fused stack launch");
    return NMOE_HIP_OK;
}
