/*
 * nmoe_hip_internal.h -- shared definitions of libnmoe_hip.so (not installed).
 */
#ifndef NMOE_HIP_INTERNAL_H
#define NMOE_HIP_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>

#include "nmoe_exact.h"
#include "nmoe_hip.h"

#define NMOE_WAVE 64
#define NMOE_HIDDEN NMOE_HIP_HIDDEN
#define NMOE_INTER NMOE_HIP_INTER
#define NMOE_EXPERTS NMOE_HIP_EXPERTS
#define NMOE_GROUP NMOE_HIP_GROUP
#define NMOE_MAX_K NMOE_HIP_MAX_K

/* Pack component offsets (scripts/convert_qwen36.py:38-64, runtime.m:2240-2252):
 * gate w/s/b, up w/s/b, down w/s/b. */
#define NMOE_Q4_OFFSETS {0u, 524288u, 557056u, 589824u, 1114112u, 1146880u, 1179648u, 1703936u, 1736704u}
#define NMOE_Q2_OFFSETS {0u, 262144u, 294912u, 327680u, 589824u, 622592u, 655360u, 917504u, 950272u}

template <int BITS>
struct nmoe_layout;

template <>
struct nmoe_layout<4> {
    static constexpr uint32_t expert_size = NMOE_HIP_EXPERT_SIZE_Q4;
    static constexpr uint32_t gate_w = 0u, gate_s = 524288u, gate_b = 557056u;
    static constexpr uint32_t up_w = 589824u, up_s = 1114112u, up_b = 1146880u;
    static constexpr uint32_t down_w = 1179648u, down_s = 1703936u, down_b = 1736704u;
};

template <>
struct nmoe_layout<2> {
    static constexpr uint32_t expert_size = NMOE_HIP_EXPERT_SIZE_Q2;
    static constexpr uint32_t gate_w = 0u, gate_s = 262144u, gate_b = 294912u;
    static constexpr uint32_t up_w = 327680u, up_s = 589824u, up_b = 622592u;
    static constexpr uint32_t down_w = 655360u, down_s = 917504u, down_b = 950272u;
};

/* Device scratch words used by persistent kernels.  Each counter sits on
 * its own 128-byte line. */
#define NMOE_SYNC_STATUS 0     /* set to 1 by a kernel whose bounded wait expired */
#define NMOE_SYNC_WORDS 8192   /* status + per-block launch epochs of the fused kernel */
#define NMOE_SYNC_EPOCH(b) (64 + 16 * (b))     /* per-block launch epochs, 64 bytes apart */
#define NMOE_SYNC_PREP_EPOCH 4368              /* preparation launches so far (the epoch of their tagged words - 1) */
#define NMOE_SYNC_BLOCKS 256
/* The fused launch's exchange words (tagged logits, act and partial y),
 * and with the whole-block form's shared activations and next-norm sums. */
#define NMOE_FUSED_XCH_BYTES 409600u
#define NMOE_FUSED_XCH_BYTES_BLOCK 446976u
#define NMOE_FUSED_XCH_BYTES_STACK 745984u /* the block form's words + the layer loop's */

/* The whole-block parts of a fused launch (XBLOCK): norm weights, the
 * next-layer norm output and the shared expert. */
struct nmoe_block_ext {
    const uint16_t *norm_w;
    const uint16_t *next_w;
    int add_one;
    float *next_x;
    nmoe_hip_shared_expert sh; /* sh.gate.w == NULL: none */
};

struct nmoe_pack_slot {
    void *dev;     /* the layer's pack as uploaded (256 experts, row-major codes) */
    void *stripes; /* the same pack with stripe-major codes, read by the grouped GEMMs */
    int bits;
    size_t bytes;
};

struct nmoe_buf_entry {
    char label[64];
    void *dev;
    size_t size;
};

/* 1 in the phase-timeline build (make timeline -> libnmoe_hip_tl.so): the
 * fused launches stamp the device's real-time clock at their phase
 * boundaries into the buffer nmoe_hip_set_timeline names.  0 in the product
 * build, where the stamps compile to nothing. */
#ifndef NMOE_TIMELINE
#define NMOE_TIMELINE 0
#endif
#define NMOE_TL_EVENTS 16
/* one timeline slot: the stamps of one fused launch (256 blocks x 16
 * events), or of 1,024 blocks of a grouped GEMM launch (4 words each) */
#define NMOE_TL_SLOT_WORDS (256 * NMOE_TL_EVENTS)

struct nmoe_hip_ctx {
    int device;
    int num_cus;
    int max_tokens;
    hipStream_t stream;
    nmoe_pack_slot packs[NMOE_HIP_MAX_LAYERS];
    nmoe_buf_entry *bufs;
    int nbufs;
    int capbufs;
    /* scratch, sized for max_tokens at create */
    float *act;      /* [max_tokens][8][512] SwiGLU activations */
    float *logits;   /* [max_tokens][256] */
    uint32_t *idx;   /* [max_tokens][8] routing scratch for nmoe_moe_layer */
    float *w;        /* [max_tokens][8] */
    uint32_t *sync;  /* NMOE_SYNC_WORDS */
    uint64_t *xch;   /* fused kernel's cross-block exchange (tagged logits, act, partial y) */
    size_t xch_bytes;
    int fused_blocks;     /* persistent decode grid (0 = not resident-capable) */
    int use_fused;        /* NMOE_HIP_OPT_FUSED_DECODE */
    int xcd_placed;       /* blocks dealt round-robin over 8 dies (checked at create) */
    int use_xcd_local;    /* NMOE_HIP_OPT_XCD_LOCAL */
    uint32_t spin_limit;  /* NMOE_HIP_OPT_SPIN_LIMIT: poll rounds before a bounded wait gives up */
    int sync_check;       /* NMOE_HIP_OPT_SYNC_CHECK */
    int stack_loop;       /* NMOE_HIP_OPT_STACK_LOOP */
    /* phase timeline (builds with NMOE_TIMELINE only): [tl_slots][256][16]
     * stamps, one slot a launch (a layer of a stack launch), in turn */
    uint64_t *tl;
    int tl_slots, tl_next;
    /* grouped (matrix-core) path for many tokens, sized for max_tokens */
    int grouped_min_tokens; /* NMOE_HIP_OPT_GROUPED_MIN_TOKENS */
    int grouped_one_launch; /* NMOE_HIP_OPT_GROUPED_ONE_LAUNCH */
    int skew_tiles;         /* NMOE_HIP_OPT_SKEW_TILES: rank, or -1 */
    uint32_t *g_done;       /* [256] the one-launch form's gate/up tiles done per expert rank */
    uint64_t *g_tags;       /* [T*8] routed entries of the preparation launch: epoch << 32 | expert */
    uint64_t *g_counts;     /* [64][256] per-slice expert histograms, each word epoch << 32 | count */
    uint32_t *g_perm;       /* [T*8] entries grouped by expert */
    uint32_t *g_offsets;    /* [257] */
    uint32_t *g_rank;       /* [2][256][4] the expert order (expert, first entry, entries, entry), then the
                               same entries in the one-launch down tiles' order */
    uint16_t *g_xhi, *g_xlo; /* [T][2048] x in operand order (bf16 hi / lo) */
    uint16_t *g_xs;         /* [T][3][32] group sums of x as three bf16 parts */
    uint16_t *g_ahi, *g_alo; /* [T*8][512] act (bf16 hi / lo), by permuted row */
    float *g_as;            /* [T*8][8] group sums of act */
    float *g_y;             /* [T*8][2048] per-entry expert outputs */
    float *s_act;           /* [T][512] shared-expert activations */
    /* the MoE blocks of the model weights loaded by nmoe_hip_load_model_weights */
    nmoe_hip_moe_block blocks[NMOE_HIP_MAX_LAYERS];
    unsigned char block_set[NMOE_HIP_MAX_LAYERS];
    char err[256];
};

int nmoe_fail(nmoe_hip_ctx *ctx, int code, const char *fmt, ...);
/* With NMOE_HIP_OPT_SYNC_CHECK set: waits for `stream` and turns an expired
 * bounded wait into NMOE_HIP_ETIMEDOUT (nmoe_hip_check_device_status);
 * otherwise returns NMOE_HIP_OK at once. */
extern "C" int nmoe_sync_check(nmoe_hip_ctx *ctx, void *stream);
int nmoe_hip_check(nmoe_hip_ctx *ctx, hipError_t e, const char *what);
/* The next n timeline slots of the context (NMOE_TIMELINE builds; NULL
 * when no timeline buffer is set). */
uint64_t *nmoe_tl_take(nmoe_hip_ctx *ctx, int n);
/* Writes the stripe-major copy of layer's pack (after every write of the
 * pack) and waits for it. */
int nmoe_pack_stripe(nmoe_hip_ctx *ctx, int layer);

#define NMOE_HIP_TRY(ctx, call)                                   \
    do {                                                          \
        hipError_t nmoe_e_ = (call);                              \
        if (nmoe_e_ != hipSuccess) return nmoe_hip_check((ctx), nmoe_e_, #call); \
    } while (0)

static inline hipStream_t nmoe_stream_of(nmoe_hip_ctx *ctx, void *stream) {
    return stream != NULL ? (hipStream_t)stream : ctx->stream;
}

static inline int nmoe_aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

/* ---------------------------------------------------------------- device */

__device__ __forceinline__ float nmoe_bf16f(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint32_t nmoe_f32_to_bf16_bits(float f) {
    uint32_t b = __float_as_uint(f);
    return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

#endif
