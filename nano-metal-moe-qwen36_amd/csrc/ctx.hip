/*
 * ctx.hip -- context, device buffers, resident expert packs, the synthetic
 * pack generator and the bit-exact dequant probe.
 *
 * The reference keeps one Metal device/queue and a label -> buffer registry
 * (src/backend/metal_backend.m:156-183, 263-277) and maps each layer's expert
 * file for pread into eight fixed 2 MB-aligned I/O buffers per token
 * (src/runtime.m:1542-1634, 2426-2465).  Here every layer pack is copied
 * once into HBM (288 GB holds all 40 q4 layers, 18.1 GB) and stays there,
 * so the per-token path has no host copy and no host/device handshake.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "nmoe_device.h"

#pragma clang fp contract(off)

int nmoe_fail(nmoe_hip_ctx *ctx, int code, const char *fmt, ...) {
    if (ctx != NULL) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(ctx->err, sizeof(ctx->err), fmt, ap);
        va_end(ap);
    }
    return code;
}

int nmoe_hip_check(nmoe_hip_ctx *ctx, hipError_t e, const char *what) {
    return nmoe_fail(ctx, NMOE_HIP_EHIP, "%s failed: %s", what, hipGetErrorString(e));
}

extern "C" int nmoe_hip_create(int device, int max_tokens, nmoe_hip_ctx **out) {
    if (out == NULL) return NMOE_HIP_EINVAL;
    *out = NULL;
    if (max_tokens < 1 || max_tokens > (1 << 16)) return NMOE_HIP_EINVAL;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return NMOE_HIP_ENODEV;
    if (hipSetDevice(device) != hipSuccess) return NMOE_HIP_ENODEV;
    nmoe_hip_ctx *ctx = (nmoe_hip_ctx *)calloc(1, sizeof(nmoe_hip_ctx));
    if (ctx == NULL) return NMOE_HIP_ENOMEM;
    ctx->device = device;
    ctx->max_tokens = max_tokens;
    ctx->use_fused = 1;
    ctx->stack_loop = 1;
    ctx->spin_limit = NMOE_SPIN_LIMIT;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess || hipStreamCreate(&ctx->stream) != hipSuccess) {
        free(ctx);
        return NMOE_HIP_ENODEV;
    }
    ctx->num_cus = prop.multiProcessorCount;
    size_t mt = (size_t)max_tokens;
    size_t bytes_act = mt * NMOE_MAX_K * NMOE_INTER * sizeof(float);
    size_t bytes_logits = mt * NMOE_EXPERTS * sizeof(float);
    size_t bytes_idx = mt * NMOE_MAX_K * sizeof(uint32_t);
    if (hipMalloc((void **)&ctx->act, bytes_act) != hipSuccess ||
        hipMalloc((void **)&ctx->logits, bytes_logits) != hipSuccess ||
        hipMalloc((void **)&ctx->idx, bytes_idx) != hipSuccess ||
        hipMalloc((void **)&ctx->w, bytes_idx) != hipSuccess ||
        hipMalloc((void **)&ctx->s_act, mt * NMOE_INTER * sizeof(float)) != hipSuccess ||
        hipMalloc((void **)&ctx->sync, NMOE_SYNC_WORDS * sizeof(uint32_t)) != hipSuccess ||
        hipMemset(ctx->sync, 0, NMOE_SYNC_WORDS * sizeof(uint32_t)) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        nmoe_hip_destroy(ctx);
        return NMOE_HIP_ENOMEM;
    }
    extern int nmoe_decode_init(nmoe_hip_ctx *);
    if (nmoe_decode_init(ctx) != NMOE_HIP_OK) {
        nmoe_hip_destroy(ctx);
        return NMOE_HIP_ENODEV;
    }
    extern int nmoe_grouped_init(nmoe_hip_ctx *);
    if (nmoe_grouped_init(ctx) != NMOE_HIP_OK) {
        nmoe_hip_destroy(ctx);
        return NMOE_HIP_ENOMEM;
    }
    *out = ctx;
    return NMOE_HIP_OK;
}

extern "C" void nmoe_hip_destroy(nmoe_hip_ctx *ctx) {
    if (ctx == NULL) return;
    hipSetDevice(ctx->device);
    if (ctx->stream != NULL) hipStreamSynchronize(ctx->stream);
    for (int l = 0; l < NMOE_HIP_MAX_LAYERS; l++)
        if (ctx->packs[l].dev != NULL) {
            hipFree(ctx->packs[l].dev);
            hipFree(ctx->packs[l].stripes);
        }
    for (int i = 0; i < ctx->nbufs; i++) hipFree(ctx->bufs[i].dev);
    free(ctx->bufs);
    hipFree(ctx->act);
    hipFree(ctx->logits);
    hipFree(ctx->idx);
    hipFree(ctx->w);
    hipFree(ctx->s_act);
    hipFree(ctx->sync);
    hipFree(ctx->xch);
    extern void nmoe_grouped_free(nmoe_hip_ctx *);
    nmoe_grouped_free(ctx);
    if (ctx->stream != NULL) hipStreamDestroy(ctx->stream);
    free(ctx);
}

extern "C" int nmoe_hip_set_option(nmoe_hip_ctx *ctx, int option, int value) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (option == NMOE_HIP_OPT_FUSED_DECODE) {
        ctx->use_fused = value != 0;
        return NMOE_HIP_OK;
    }
    if (option == NMOE_HIP_OPT_GROUPED_MIN_TOKENS) {
        if (value < 1) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "grouped path minimum %d < 1", value);
        ctx->grouped_min_tokens = value;
        return NMOE_HIP_OK;
    }
    if (option == NMOE_HIP_OPT_XCD_LOCAL) {
        if (value != 0 && !ctx->xcd_placed)
            return nmoe_fail(ctx, NMOE_HIP_EINVAL, "this device does not deal a launch's blocks round-robin over 8 dies");
        ctx->use_xcd_local = value != 0;
        return NMOE_HIP_OK;
    }
    if (option == NMOE_HIP_OPT_SPIN_LIMIT) {
        if (value < 0 || value > NMOE_HIP_SPIN_LIMIT_MAX)
            return nmoe_fail(ctx, NMOE_HIP_EINVAL, "spin limit %d outside 0..%d", value, NMOE_HIP_SPIN_LIMIT_MAX);
        ctx->spin_limit = value == 0 ? NMOE_SPIN_LIMIT : (uint32_t)value;
        return NMOE_HIP_OK;
    }
    if (option == NMOE_HIP_OPT_SYNC_CHECK) {
        ctx->sync_check = value != 0;
        return NMOE_HIP_OK;
    }
    if (option == NMOE_HIP_OPT_STACK_LOOP) {
        ctx->stack_loop = value != 0;
        return NMOE_HIP_OK;
    }
    if (option == NMOE_HIP_OPT_SKEW_TILES) {
        if (value < 0 || value >= NMOE_EXPERTS)
            return nmoe_fail(ctx, NMOE_HIP_EINVAL, "expert rank %d outside 0..%d", value, NMOE_EXPERTS - 1);
        ctx->skew_tiles = value;
        return NMOE_HIP_OK;
    }
    if (option == NMOE_HIP_OPT_GROUPED_ONE_LAUNCH) {
        if (value != 0 && !ctx->xcd_placed)
            return nmoe_fail(ctx, NMOE_HIP_EINVAL, "this device does not deal a launch's blocks round-robin over 8 dies");
        ctx->grouped_one_launch = value != 0;
        return NMOE_HIP_OK;
    }
    if (option == NMOE_HIP_OPT_SKEW_EPOCH) {
        /* Moves block `value`'s launch epoch one ahead of the others, so the
         * next fused launch cannot complete: its bounded waits expire and it
         * reports ETIMEDOUT, the failure a block that is not resident would
         * cause.  Synchronous; for tests of that path. */
        if (value < 0 || value >= NMOE_SYNC_BLOCKS)
            return nmoe_fail(ctx, NMOE_HIP_EINVAL, "block %d outside 0..%d", value, NMOE_SYNC_BLOCKS - 1);
        uint32_t ep = 0;
        NMOE_HIP_TRY(ctx, hipSetDevice(ctx->device));
        NMOE_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        NMOE_HIP_TRY(ctx, hipMemcpy(&ep, ctx->sync + NMOE_SYNC_EPOCH(value), sizeof(ep), hipMemcpyDeviceToHost));
        ep += 1u;
        NMOE_HIP_TRY(ctx, hipMemcpy(ctx->sync + NMOE_SYNC_EPOCH(value), &ep, sizeof(ep), hipMemcpyHostToDevice));
        return NMOE_HIP_OK;
    }
    return nmoe_fail(ctx, NMOE_HIP_EINVAL, "unknown option %d", option);
}

extern "C" int nmoe_hip_set_timeline(nmoe_hip_ctx *ctx, void *stamps, int slots) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
#if NMOE_TIMELINE
    if ((stamps == NULL) != (slots == 0) || slots < 0 || (stamps != NULL && !nmoe_aligned(stamps, 8)))
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "timeline: a buffer of slots x 256 x 16 stamps, or NULL and 0");
    ctx->tl = (uint64_t *)stamps;
    ctx->tl_slots = slots;
    ctx->tl_next = 0;
    return NMOE_HIP_OK;
#else
    (void)stamps;
    (void)slots;
    return nmoe_fail(ctx, NMOE_HIP_EINVAL, "this library was built without the phase timeline (NMOE_TIMELINE)");
#endif
}

uint64_t *nmoe_tl_take(nmoe_hip_ctx *ctx, int n) {
    if (!NMOE_TIMELINE || ctx->tl == NULL || n > ctx->tl_slots) return NULL;
    if (ctx->tl_next + n > ctx->tl_slots) ctx->tl_next = 0;
    uint64_t *p = ctx->tl + (size_t)ctx->tl_next * NMOE_TL_SLOT_WORDS;
    ctx->tl_next += n;
    return p;
}

extern "C" int nmoe_sync_check(nmoe_hip_ctx *ctx, void *stream) {
    if (!ctx->sync_check) return NMOE_HIP_OK;
    NMOE_HIP_TRY(ctx, hipStreamSynchronize(nmoe_stream_of(ctx, stream)));
    return nmoe_hip_check_device_status(ctx);
}

extern "C" const char *nmoe_hip_last_error(const nmoe_hip_ctx *ctx) { return ctx != NULL ? ctx->err : "no context"; }

extern "C" void *nmoe_hip_stream(nmoe_hip_ctx *ctx) { return ctx != NULL ? (void *)ctx->stream : NULL; }

extern "C" int nmoe_hip_device_cus(const nmoe_hip_ctx *ctx) { return ctx != NULL ? ctx->num_cus : 0; }

extern "C" int nmoe_hip_synchronize(nmoe_hip_ctx *ctx) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    NMOE_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return NMOE_HIP_OK;
}

extern "C" int nmoe_hip_check_device_status(nmoe_hip_ctx *ctx) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    uint32_t status = 0;
    NMOE_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    NMOE_HIP_TRY(ctx, hipMemcpy(&status, ctx->sync + NMOE_SYNC_STATUS, sizeof(status), hipMemcpyDeviceToHost));
    if (status != 0) {
        /* An aborted launch leaves the blocks' epochs unequal.  Every epoch
         * moves past the largest one (exchange words only ever carry past
         * epochs, so none can match a future one -- including copies still
         * held in a die's L2), and the status restarts from 0.  (A host
         * copy of the words; this is the error path.) */
        uint32_t *words = (uint32_t *)malloc(NMOE_SYNC_WORDS * sizeof(uint32_t));
        if (words == NULL) return nmoe_fail(ctx, NMOE_HIP_ENOMEM, "host copy of the sync words");
        hipError_t e = hipMemcpy(words, ctx->sync, NMOE_SYNC_WORDS * sizeof(uint32_t), hipMemcpyDeviceToHost);
        if (e == hipSuccess) {
            uint32_t top = 0;
            for (int b = 0; b < NMOE_SYNC_BLOCKS; b++)
                if (words[NMOE_SYNC_EPOCH(b)] > top) top = words[NMOE_SYNC_EPOCH(b)];
            for (int b = 0; b < NMOE_SYNC_BLOCKS; b++) words[NMOE_SYNC_EPOCH(b)] = top + 1u;
            words[NMOE_SYNC_STATUS] = 0u;
            /* routed entries and histogram words of the aborted launch may
             * carry the epoch after it: the next launch takes one past that */
            words[NMOE_SYNC_PREP_EPOCH] += 2u;
            e = hipMemcpy(ctx->sync, words, NMOE_SYNC_WORDS * sizeof(uint32_t), hipMemcpyHostToDevice);
        }
        free(words);
        NMOE_HIP_TRY(ctx, e);
        NMOE_HIP_TRY(ctx, hipDeviceSynchronize());
        return nmoe_fail(ctx, NMOE_HIP_ETIMEDOUT, "a persistent kernel's bounded wait expired (status %u)", status);
    }
    return NMOE_HIP_OK;
}

/* ------------------------------------------------------------- buffers */

static int nmoe_buf_add(nmoe_hip_ctx *ctx, const char *label, void *dev, size_t size) {
    if (ctx->nbufs == ctx->capbufs) {
        int cap = ctx->capbufs ? ctx->capbufs * 2 : 16;
        nmoe_buf_entry *nb = (nmoe_buf_entry *)realloc(ctx->bufs, sizeof(nmoe_buf_entry) * (size_t)cap);
        if (nb == NULL) return NMOE_HIP_ENOMEM;
        ctx->bufs = nb;
        ctx->capbufs = cap;
    }
    nmoe_buf_entry *e = &ctx->bufs[ctx->nbufs++];
    snprintf(e->label, sizeof(e->label), "%s", label);
    e->dev = dev;
    e->size = size;
    return NMOE_HIP_OK;
}

extern "C" void *nmoe_hip_lookup_buffer(const nmoe_hip_ctx *ctx, const char *label) {
    if (ctx == NULL || label == NULL) return NULL;
    for (int i = 0; i < ctx->nbufs; i++)
        if (strncmp(ctx->bufs[i].label, label, sizeof(ctx->bufs[i].label)) == 0) return ctx->bufs[i].dev;
    return NULL;
}

extern "C" int nmoe_hip_register_state_buffer(nmoe_hip_ctx *ctx, const char *label, size_t size, void **dev_out) {
    if (ctx == NULL || label == NULL || dev_out == NULL || size == 0) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "bad args");
    if (nmoe_hip_lookup_buffer(ctx, label) != NULL)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "buffer label '%s' already registered", label);
    void *dev = NULL;
    NMOE_HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (hipMalloc(&dev, size) != hipSuccess) return nmoe_fail(ctx, NMOE_HIP_ENOMEM, "hipMalloc(%zu) failed", size);
    if (hipMemset(dev, 0, size) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        hipFree(dev);
        return nmoe_fail(ctx, NMOE_HIP_EHIP, "zero-fill of '%s' failed", label);
    }
    int rc = nmoe_buf_add(ctx, label, dev, size);
    if (rc != NMOE_HIP_OK) {
        hipFree(dev);
        return nmoe_fail(ctx, rc, "registry full");
    }
    *dev_out = dev;
    return NMOE_HIP_OK;
}

extern "C" int nmoe_hip_register_shared_buffer(nmoe_hip_ctx *ctx, const char *label, const void *host, size_t size,
                                               void **dev_out) {
    if (host == NULL) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "NULL host data");
    int rc = nmoe_hip_register_state_buffer(ctx, label, size, dev_out);
    if (rc != NMOE_HIP_OK) return rc;
    NMOE_HIP_TRY(ctx, hipMemcpy(*dev_out, host, size, hipMemcpyHostToDevice));
    return NMOE_HIP_OK;
}

extern "C" int nmoe_hip_copy_to_device(nmoe_hip_ctx *ctx, void *dev, const void *host, size_t size) {
    if (ctx == NULL || dev == NULL || host == NULL) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "bad args");
    NMOE_HIP_TRY(ctx, hipMemcpyAsync(dev, host, size, hipMemcpyHostToDevice, ctx->stream));
    NMOE_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return NMOE_HIP_OK;
}

extern "C" int nmoe_hip_copy_to_host(nmoe_hip_ctx *ctx, void *host, const void *dev, size_t size) {
    if (ctx == NULL || dev == NULL || host == NULL) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "bad args");
    NMOE_HIP_TRY(ctx, hipMemcpyAsync(host, dev, size, hipMemcpyDeviceToHost, ctx->stream));
    NMOE_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return NMOE_HIP_OK;
}

/* --------------------------------------------------------------- packs */

extern "C" size_t nmoe_hip_expert_size(int bits) {
    return bits == 4 ? NMOE_HIP_EXPERT_SIZE_Q4 : bits == 2 ? NMOE_HIP_EXPERT_SIZE_Q2 : 0u;
}

static int nmoe_pack_alloc(nmoe_hip_ctx *ctx, int layer, int bits, void **dev_out) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (layer < 0 || layer >= NMOE_HIP_MAX_LAYERS)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "layer %d outside 0..%d", layer, NMOE_HIP_MAX_LAYERS - 1);
    if (bits != 4 && bits != 2) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "bits must be 4 or 2, got %d", bits);
    size_t bytes = (size_t)NMOE_EXPERTS * nmoe_hip_expert_size(bits);
    nmoe_pack_slot *slot = &ctx->packs[layer];
    NMOE_HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (slot->dev != NULL && slot->bytes != bytes) {
        NMOE_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        hipFree(slot->dev);
        hipFree(slot->stripes);
        slot->dev = slot->stripes = NULL;
    }
    if (slot->dev == NULL) {
        /* the pack and its stripe-major copy for the grouped GEMMs */
        if (hipMalloc(&slot->dev, bytes) != hipSuccess) {
            slot->dev = NULL;
            return nmoe_fail(ctx, NMOE_HIP_ENOMEM, "hipMalloc of layer %d pack (%zu bytes) failed", layer, bytes);
        }
        if (hipMalloc(&slot->stripes, bytes) != hipSuccess) {
            hipFree(slot->dev);
            slot->dev = slot->stripes = NULL;
            return nmoe_fail(ctx, NMOE_HIP_ENOMEM, "hipMalloc of layer %d stripe-major pack (%zu bytes) failed", layer,
                             bytes);
        }
    }
    slot->bits = bits;
    slot->bytes = bytes;
    *dev_out = slot->dev;
    return NMOE_HIP_OK;
}

extern "C" int nmoe_hip_upload_layer_pack(nmoe_hip_ctx *ctx, int layer, int bits, const void *host, size_t size) {
    if (ctx == NULL || host == NULL) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "bad args");
    size_t want = (size_t)NMOE_EXPERTS * nmoe_hip_expert_size(bits);
    if (want == 0) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "bits must be 4 or 2, got %d", bits);
    /* runtime.m:2444-2451 rejects a layer file shorter than 256 experts */
    if (size != want)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "layer %d pack has %zu bytes, expected %zu (256 x %zu)", layer, size, want,
                         nmoe_hip_expert_size(bits));
    void *dev = NULL;
    int rc = nmoe_pack_alloc(ctx, layer, bits, &dev);
    if (rc != NMOE_HIP_OK) return rc;
    NMOE_HIP_TRY(ctx, hipMemcpy(dev, host, size, hipMemcpyHostToDevice));
    return nmoe_pack_stripe(ctx, layer);
}

extern "C" const void *nmoe_hip_layer_pack(const nmoe_hip_ctx *ctx, int layer, int *bits_out) {
    if (ctx == NULL || layer < 0 || layer >= NMOE_HIP_MAX_LAYERS) return NULL;
    if (bits_out != NULL) *bits_out = ctx->packs[layer].bits;
    return ctx->packs[layer].dev;
}

/* ----------------------------------------------------------- generator */

#define NMOE_GOLDEN 0x9E3779B97F4A7C15ull

__host__ __device__ __forceinline__ uint64_t nmoe_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__host__ __device__ __forceinline__ uint64_t nmoe_syn_stream(uint64_t seed, uint32_t layer, uint32_t expert,
                                                            uint32_t tag) {
    uint64_t s = nmoe_mix64(seed + NMOE_GOLDEN);
    return nmoe_mix64(s ^ (((uint64_t)layer << 40) | ((uint64_t)expert << 16) | (uint64_t)tag));
}

__device__ __forceinline__ uint64_t nmoe_syn_rand64(uint64_t stream, uint64_t i) {
    return nmoe_mix64(stream + (i + 1) * NMOE_GOLDEN);
}

/* Irwin-Hall(12): twelve 16-bit uniforms (u + 1/2)/65536 summed, minus 6
 * (exact in fp32; the only rounding is the final multiply by sigma). */
__device__ __forceinline__ float nmoe_syn_normal(uint64_t stream, uint64_t i) {
    uint32_t sum = 0;
#pragma unroll
    for (uint64_t j = 0; j < 3; j++) {
        uint64_t r = nmoe_syn_rand64(stream, 3 * i + j);
        sum += (uint32_t)(r & 0xFFFF) + (uint32_t)((r >> 16) & 0xFFFF) + (uint32_t)((r >> 32) & 0xFFFF) +
               (uint32_t)(r >> 48);
    }
    return (float)(sum + 6u) * (1.0f / 65536.0f) - 6.0f;
}

/* All three matrices of an expert hold the same number of packed words
 * (q4: 131072, q2: 65536) and the same number of groups (16384). */
__global__ void nmoe_synth_words_kernel(uint32_t *pack, uint64_t seed, uint32_t layer, uint32_t esz_words,
                                        uint32_t wpm, uint32_t off_up_words, uint32_t off_down_words) {
    uint64_t pairs_per_expert = (uint64_t)3 * (wpm / 2);
    uint64_t total = pairs_per_expert * NMOE_EXPERTS;
    for (uint64_t p = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; p < total; p += (uint64_t)gridDim.x * blockDim.x) {
        uint32_t e = (uint32_t)(p / pairs_per_expert);
        uint32_t r = (uint32_t)(p % pairs_per_expert);
        uint32_t m = r / (wpm / 2);
        uint32_t jp = r % (wpm / 2);
        uint64_t st = nmoe_syn_stream(seed, layer, e, 2u * m);
        uint64_t v = nmoe_syn_rand64(st, jp);
        uint32_t base = m == 0 ? 0u : (m == 1 ? off_up_words : off_down_words);
        uint2 *dst = (uint2 *)(pack + (uint64_t)e * esz_words + base) + jp;
        *dst = make_uint2((uint32_t)v, (uint32_t)(v >> 32));
    }
}

__global__ void nmoe_synth_scales_kernel(uint16_t *pack16, uint64_t seed, uint32_t layer, uint32_t esz_halfs,
                                         uint32_t s0, uint32_t s1, uint32_t s2, uint32_t ngroups, float sigma,
                                         int bits) {
    uint64_t per_expert = (uint64_t)3 * ngroups;
    uint64_t total = per_expert * NMOE_EXPERTS;
    for (uint64_t p = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; p < total; p += (uint64_t)gridDim.x * blockDim.x) {
        uint32_t e = (uint32_t)(p / per_expert);
        uint32_t r = (uint32_t)(p % per_expert);
        uint32_t m = r / ngroups;
        uint32_t g = r % ngroups;
        uint64_t st = nmoe_syn_stream(seed, layer, e, 2u * m + 1u);
        uint32_t s16 = nmoe_f32_to_bf16_bits(nmoe_syn_normal(st, g) * sigma);
        float s = nmoe_bf16f(s16);
        uint32_t b16 = nmoe_f32_to_bf16_bits(bits == 4 ? -8.0f * s : -1.5f * s);
        uint32_t so = m == 0 ? s0 : (m == 1 ? s1 : s2);
        uint16_t *base = pack16 + (uint64_t)e * esz_halfs + so;
        base[g] = (uint16_t)s16;
        base[ngroups + g] = (uint16_t)b16; /* biases follow the scales */
    }
}

__global__ void nmoe_synth_bf16_kernel(uint16_t *dst, uint64_t n, uint64_t stream, float sigma) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = (uint16_t)nmoe_f32_to_bf16_bits(nmoe_syn_normal(stream, i) * sigma);
}

extern "C" int nmoe_hip_synth_layer_pack(nmoe_hip_ctx *ctx, int layer, int bits, uint64_t seed, float sigma) {
    void *dev = NULL;
    int rc = nmoe_pack_alloc(ctx, layer, bits, &dev);
    if (rc != NMOE_HIP_OK) return rc;
    uint32_t esz = (uint32_t)nmoe_hip_expert_size(bits);
    uint32_t wpm = bits == 4 ? 131072u : 65536u;
    uint32_t up_w = bits == 4 ? nmoe_layout<4>::up_w : nmoe_layout<2>::up_w;
    uint32_t down_w = bits == 4 ? nmoe_layout<4>::down_w : nmoe_layout<2>::down_w;
    uint32_t gs = bits == 4 ? nmoe_layout<4>::gate_s : nmoe_layout<2>::gate_s;
    uint32_t us = bits == 4 ? nmoe_layout<4>::up_s : nmoe_layout<2>::up_s;
    uint32_t ds = bits == 4 ? nmoe_layout<4>::down_s : nmoe_layout<2>::down_s;
    int blocks = ctx->num_cus * 8;
    hipLaunchKernelGGL(nmoe_synth_words_kernel, dim3(blocks), dim3(256), 0, ctx->stream, (uint32_t *)dev, seed,
                       (uint32_t)layer, esz / 4u, wpm, up_w / 4u, down_w / 4u);
    NMOE_HIP_TRY(ctx, hipGetLastError());
    hipLaunchKernelGGL(nmoe_synth_scales_kernel, dim3(blocks), dim3(256), 0, ctx->stream, (uint16_t *)dev, seed,
                       (uint32_t)layer, esz / 2u, gs / 2u, us / 2u, ds / 2u, 16384u, sigma, bits);
    NMOE_HIP_TRY(ctx, hipGetLastError());
    return nmoe_pack_stripe(ctx, layer);
}

extern "C" int nmoe_hip_synth_bf16(nmoe_hip_ctx *ctx, uint16_t *dev, size_t n, uint64_t seed, uint32_t layer,
                                   uint32_t tag, float sigma, void *stream) {
    if (ctx == NULL || dev == NULL) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "bad args");
    if (n == 0) return NMOE_HIP_OK;
    uint64_t st = nmoe_syn_stream(seed, layer, 0xFFFFu, tag);
    int blocks = (int)((n + 255) / 256);
    if (blocks > ctx->num_cus * 8) blocks = ctx->num_cus * 8;
    hipLaunchKernelGGL(nmoe_synth_bf16_kernel, dim3(blocks), dim3(256), 0, nmoe_stream_of(ctx, stream), dev,
                       (uint64_t)n, st, sigma);
    NMOE_HIP_TRY(ctx, hipGetLastError());
    return NMOE_HIP_OK;
}

/* ------------------------------------------------------- dequant probe */

/* One thread per output element: q = field of the packed word, out =
 * fma(q, scale, bias).  q*scale is exact (<= 4 + 8 significant bits), so the
 * fused and unfused forms (kernels.metal:1083, math.m:230) agree bit for bit. */
template <int BITS>
__global__ void nmoe_dequant_rows_kernel(const uint32_t *packed, const uint16_t *scales, const uint16_t *biases,
                                         int rows, int in_dim, float *out) {
    constexpr int VPW = 32 / BITS;
    constexpr uint32_t MASK = (1u << BITS) - 1u;
    uint64_t total = (uint64_t)rows * (uint64_t)in_dim;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x) {
        uint64_t r = i / (uint64_t)in_dim;
        uint32_t c = (uint32_t)(i % (uint64_t)in_dim);
        uint32_t word = packed[r * (uint64_t)(in_dim / VPW) + c / VPW];
        uint32_t q = (word >> ((c % VPW) * BITS)) & MASK;
        uint64_t g = r * (uint64_t)(in_dim / NMOE_GROUP) + c / NMOE_GROUP;
        out[i] = __builtin_fmaf((float)q, nmoe_bf16f(scales[g]), nmoe_bf16f(biases[g]));
    }
}

extern "C" int nmoe_dequant_rows(nmoe_hip_ctx *ctx, int bits, const uint32_t *packed, const uint16_t *scales,
                                 const uint16_t *biases, int rows, int in_dim, float *out, void *stream) {
    if (ctx == NULL || packed == NULL || scales == NULL || biases == NULL || out == NULL)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "NULL argument");
    if (bits != 4 && bits != 2) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "bits must be 4 or 2");
    if (rows < 0 || in_dim <= 0 || in_dim % NMOE_GROUP != 0)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "in_dim must be a positive multiple of 64");
    if (rows == 0) return NMOE_HIP_OK;
    uint64_t total = (uint64_t)rows * (uint64_t)in_dim;
    int blocks = (int)((total + 255) / 256);
    if (blocks > ctx->num_cus * 16) blocks = ctx->num_cus * 16;
    hipStream_t s = nmoe_stream_of(ctx, stream);
    if (bits == 4)
        hipLaunchKernelGGL(nmoe_dequant_rows_kernel<4>, dim3(blocks), dim3(256), 0, s, packed, scales, biases, rows,
                           in_dim, out);
    else
        hipLaunchKernelGGL(nmoe_dequant_rows_kernel<2>, dim3(blocks), dim3(256), 0, s, packed, scales, biases, rows,
                           in_dim, out);
    NMOE_HIP_TRY(ctx, hipGetLastError());
    return NMOE_HIP_OK;
}

/* The model weights' MoE blocks (set by host/weights.c). */
extern "C" int nmoe_ctx_set_block(nmoe_hip_ctx *ctx, int layer, const nmoe_hip_moe_block *b) {
    if (ctx == NULL || b == NULL || layer < 0 || layer >= NMOE_HIP_MAX_LAYERS) return NMOE_HIP_EINVAL;
    ctx->blocks[layer] = *b;
    ctx->block_set[layer] = 1;
    return NMOE_HIP_OK;
}

extern "C" int nmoe_hip_layer_block(const nmoe_hip_ctx *ctx, int layer, nmoe_hip_moe_block *out) {
    if (ctx == NULL || out == NULL || layer < 0 || layer >= NMOE_HIP_MAX_LAYERS) return NMOE_HIP_EINVAL;
    if (!ctx->block_set[layer]) return NMOE_HIP_ENOENT;
    *out = ctx->blocks[layer];
    return NMOE_HIP_OK;
}

/* Error hook for the C host files of the library. */
extern "C" int nmoe_host_fail(nmoe_hip_ctx *ctx, int code, const char *msg) { return nmoe_fail(ctx, code, "%s", msg); }
