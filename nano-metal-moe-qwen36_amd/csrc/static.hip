/*
 * static.hip -- nmoe_moe_layer_static: the per-layer MoE call for callers
 * that cannot allocate device memory (code under graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  It has no counterpart in
 * the reference, whose runtime allocates every buffer once at start-up
 * (src/runtime.m:1542-1584, 2467-2569).
 *
 * Everything the kernels need beyond the caller's inputs and outputs lives
 * in `scratch`, a file-scope device array of fixed size: every GPU the
 * library runs on holds its own copy until the process ends.  Host code
 * never passes the array's name to a kernel (on the host it is only a
 * stand-in for the symbol); the device address of each GPU's copy comes
 * from hipGetSymbolAddress, once per device, at the entry point's first call
 * on that device, and only that address reaches the kernels.
 *
 * Layout of scratch (bytes from its start, each part 256-byte aligned):
 *   xch     the fused launch's exchange words (one token per launch)
 *   sync    its status word (set when a bounded wait gives up) and the
 *           per-block launch epochs: each launch's blocks count their own
 *           launches on the device, so every replay of a call captured into
 *           a graph takes a new epoch, as every eager call does
 *   act     [16][8][512] fp32 SwiGLU activations of the per-token kernels
 *   logits  [16][256] fp32
 *   idx, w  [16][8] routing, used when the caller passes none
 *   probe   [256] u32: the die-placement probe
 * Calls share their GPU's copy and leave their contents in it; calls that
 * overlap on one GPU (two host threads, or two streams without ordering)
 * race.  The array starts zeroed (so the first epoch is 1); epochs skip 0
 * and wrap after 2^32 - 1 launches, so an exchange word that no launch
 * rewrote for that many launches could be taken as current.
 *
 * Set-up needs no stream work except the die-placement probe (a launch and
 * a copy back, which a stream being captured cannot do).  A call whose
 * stream is capturing therefore skips the probe and uses the
 * device-coherent exchange (correct wherever the blocks run); the first
 * call on a stream that is not capturing runs the probe, and later calls
 * use the die-local exchange where the probe allows it.  Launches of either
 * kind may follow each other: a launch accepts only words that carry its
 * own epoch, which only its own blocks write.
 */
#include <atomic>
#include <mutex>

#include "nmoe_device.h"

#define NMOE_STATIC_MAX_DEVICES 64
#define NMOE_STATIC_XCH 0u
#define NMOE_STATIC_SYNC (NMOE_STATIC_XCH + NMOE_FUSED_XCH_BYTES)
#define NMOE_STATIC_ACT (NMOE_STATIC_SYNC + NMOE_SYNC_WORDS * 4u)
#define NMOE_STATIC_LOGITS (NMOE_STATIC_ACT + NMOE_HIP_STATIC_MAX_TOKENS * NMOE_MAX_K * NMOE_INTER * 4u)
#define NMOE_STATIC_IDX (NMOE_STATIC_LOGITS + NMOE_HIP_STATIC_MAX_TOKENS * NMOE_EXPERTS * 4u)
#define NMOE_STATIC_W (NMOE_STATIC_IDX + NMOE_HIP_STATIC_MAX_TOKENS * NMOE_MAX_K * 4u)
#define NMOE_STATIC_PROBE (NMOE_STATIC_W + NMOE_HIP_STATIC_MAX_TOKENS * NMOE_MAX_K * 4u)
#define NMOE_STATIC_BYTES (NMOE_STATIC_PROBE + NMOE_EXPERTS * 4u)
static_assert(NMOE_STATIC_SYNC % 256 == 0 && NMOE_STATIC_ACT % 256 == 0 && NMOE_STATIC_LOGITS % 256 == 0 &&
                  NMOE_STATIC_IDX % 256 == 0 && NMOE_STATIC_W % 256 == 0 && NMOE_STATIC_PROBE % 256 == 0,
              "scratch parts 256-byte aligned");
static_assert(NMOE_STATIC_BYTES == NMOE_HIP_STATIC_SCRATCH_BYTES, "the size the header states");

static __device__ __align__(256) uint8_t scratch[NMOE_STATIC_BYTES];

extern "C" hipError_t nmoe_fused_launch_core(int bits, int route, const void *x, int xmode, float eps, int k,
                                             const nmoe_hip_router *router, const uint32_t *idx_in, const float *w_in,
                                             const float *h_mid, const float *shared_out, const float *shared_gate_raw,
                                             float *out, uint32_t *idx_out, float *w_out, float *logits_out,
                                             const uint8_t *pack, uint64_t *xch, uint32_t *sync, int xcd_local,
                                             uint32_t spin, uint32_t epoch, const nmoe_block_ext *blk,
                                             hipStream_t s, uint64_t *tl);
extern "C" int nmoe_fused_resident(int num_cus);
extern "C" int nmoe_probe_xcd_placement(uint32_t *d, int *placed, hipStream_t s);
extern "C" hipError_t nmoe_router_logits_launch(const nmoe_hip_router *router, const void *x, int x_dtype, int ntok,
                                               float *logits, hipStream_t s);
extern "C" hipError_t nmoe_topk_launch(const float *logits, int ntok, int num_experts, int k, uint32_t *idx, float *w,
                                      float *probs, hipStream_t s);
extern "C" hipError_t nmoe_experts_launch(int bits, const uint8_t *pack, const void *x, int x_dtype, int ntok, int k,
                                         const uint32_t *idx, const float *w, const float *h_mid,
                                         const float *shared_out, const float *shared_gate_raw, float *out,
                                         float *act, hipStream_t s);

/* Per-device state, set up once with the device current. */
struct nmoe_static_dev {
    std::atomic<int> ready;  /* 1 once set up, -1 if set-up failed */
    std::atomic<int> probed; /* 0: placement not probed yet, 1: probed, -1: the probe failed */
    uint8_t *ptr;            /* this device's copy of scratch */
    int fused;               /* the 256-block fused grid is resident-capable */
    std::atomic<int> xcd_local; /* blocks dealt round-robin over the 8 dies (probed) */
};
static nmoe_static_dev nmoe_static_devs[NMOE_STATIC_MAX_DEVICES];
static std::mutex nmoe_static_lock;

/* 1 when work issued to s is being captured into a graph (or the runtime
 * cannot tell: then the probe is not run either). */
static int nmoe_static_capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) return 1;
    return st != hipStreamCaptureStatusNone;
}

static int nmoe_static_setup(int dev, hipStream_t s, nmoe_static_dev **out) {
    nmoe_static_dev *d = &nmoe_static_devs[dev];
    if (d->ready.load(std::memory_order_acquire) == 0) {
        std::lock_guard<std::mutex> g(nmoe_static_lock);
        if (d->ready.load(std::memory_order_relaxed) == 0) {
            int rc = NMOE_HIP_OK, cus = 0;
            void *p = NULL;
            if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == NULL)
                rc = NMOE_HIP_EHIP;
            else if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
                rc = NMOE_HIP_ENODEV;
            if (rc == NMOE_HIP_OK) {
                d->ptr = (uint8_t *)p;
                d->fused = nmoe_fused_resident(cus);
            }
            d->xcd_local.store(0, std::memory_order_relaxed);
            d->probed.store(d->fused ? 0 : 1, std::memory_order_relaxed);
            d->ready.store(rc == NMOE_HIP_OK ? 1 : -1, std::memory_order_release);
        }
    }
    if (d->ready.load(std::memory_order_acquire) != 1) return NMOE_HIP_EHIP;
    if (d->probed.load(std::memory_order_acquire) == 0 && !nmoe_static_capturing(s)) {
        std::lock_guard<std::mutex> g(nmoe_static_lock);
        if (d->probed.load(std::memory_order_relaxed) == 0) {
            int placed = 0;
            const int rc = nmoe_probe_xcd_placement((uint32_t *)(d->ptr + NMOE_STATIC_PROBE), &placed, s);
            d->xcd_local.store(rc == NMOE_HIP_OK ? placed : 0, std::memory_order_relaxed);
            d->probed.store(rc == NMOE_HIP_OK ? 1 : -1, std::memory_order_release);
            if (rc != NMOE_HIP_OK) return rc;
        }
    }
    *out = d;
    return NMOE_HIP_OK;
}

static int nmoe_static_router_ok(const nmoe_hip_router *r) {
    if (r == NULL || r->num_experts != NMOE_EXPERTS) return 0;
    if (r->kind == NMOE_HIP_ROUTER_BF16) return r->w_bf16 != NULL && nmoe_aligned(r->w_bf16, 16);
    if (r->kind == NMOE_HIP_ROUTER_Q4)
        return r->w_q4 != NULL && r->scales != NULL && r->biases != NULL && nmoe_aligned(r->w_q4, 4);
    return 0;
}

extern "C" int nmoe_moe_layer_static(const void *layer_pack, int bits, const nmoe_hip_router *router, const void *x,
                                     int x_dtype, int ntok, int k, const float *h_mid, const float *shared_out,
                                     const float *shared_gate_raw, float *out, uint32_t *idx, float *w,
                                     void *stream) {
    if (ntok < 1 || ntok > NMOE_HIP_STATIC_MAX_TOKENS) return NMOE_HIP_EINVAL; /* beyond what scratch holds */
    if (layer_pack == NULL || !nmoe_aligned(layer_pack, 16) || (bits != 4 && bits != 2)) return NMOE_HIP_EINVAL;
    if (!nmoe_static_router_ok(router) || k < 1 || k > NMOE_MAX_K) return NMOE_HIP_EINVAL;
    if (x == NULL || !nmoe_aligned(x, 16) || (x_dtype != NMOE_HIP_F32 && x_dtype != NMOE_HIP_BF16))
        return NMOE_HIP_EINVAL;
    if (h_mid == NULL || out == NULL || !nmoe_aligned(h_mid, 4) || !nmoe_aligned(out, 4)) return NMOE_HIP_EINVAL;
    if ((shared_out == NULL) != (shared_gate_raw == NULL)) return NMOE_HIP_EINVAL;
    if ((idx != NULL && !nmoe_aligned(idx, 4)) || (w != NULL && !nmoe_aligned(w, 4))) return NMOE_HIP_EINVAL;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NMOE_STATIC_MAX_DEVICES) return NMOE_HIP_ENODEV;
    hipStream_t s = (hipStream_t)stream;
    nmoe_static_dev *d = NULL;
    int rc = nmoe_static_setup(dev, s, &d);
    if (rc != NMOE_HIP_OK) return rc;
    uint8_t *ptr = d->ptr;
    const uint8_t *pack = (const uint8_t *)layer_pack;
    if (ntok == 1 && d->fused) { /* epoch 0: the blocks count their launches on the device */
        const hipError_t e = nmoe_fused_launch_core(
            bits, 1, x, x_dtype, 0.0f, k, router, NULL, NULL, h_mid, shared_out, shared_gate_raw, out, idx, w, NULL, pack,
            (uint64_t *)(ptr + NMOE_STATIC_XCH), (uint32_t *)(ptr + NMOE_STATIC_SYNC),
            d->xcd_local.load(std::memory_order_relaxed), NMOE_SPIN_LIMIT, 0u, NULL, s, NULL);
        return e == hipSuccess ? NMOE_HIP_OK : NMOE_HIP_EHIP;
    }
    /* several tokens: router, top-k and the per-token expert kernels */
    float *logits = (float *)(ptr + NMOE_STATIC_LOGITS), *act = (float *)(ptr + NMOE_STATIC_ACT);
    uint32_t *ri = idx != NULL ? idx : (uint32_t *)(ptr + NMOE_STATIC_IDX);
    float *rw = w != NULL ? w : (float *)(ptr + NMOE_STATIC_W);
    if (nmoe_router_logits_launch(router, x, x_dtype, ntok, logits, s) != hipSuccess ||
        nmoe_topk_launch(logits, ntok, NMOE_EXPERTS, k, ri, rw, NULL, s) != hipSuccess ||
        nmoe_experts_launch(bits, pack, x, x_dtype, ntok, k, ri, rw, h_mid, shared_out, shared_gate_raw, out, act, s) !=
            hipSuccess)
        return NMOE_HIP_EHIP;
    return NMOE_HIP_OK;
}
