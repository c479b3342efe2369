/*
 * nmoe_hip.h -- C ABI of libnmoe_hip.so: the routed-expert MoE step of
 * Qwen3.6-35B-A3B on AMD Instinct MI355X (gfx950).
 *
 * Plain C, includable from C, C++ and Objective-C (the guard style of the
 * reference's include/nmoe/backend.h:7-9,69-71).  No HIP or torch types
 * appear in the signatures: device memory is passed as `void *` / typed
 * pointers, streams as `void *` (a hipStream_t; NULL = the context's stream).
 *
 * Replaces, in the reference (file:line relative to the reference root):
 *   - the Metal backend's device/queue/buffer registry for this path
 *       include/nmoe/backend.h:55-67, src/backend/metal_backend.m:156-183
 *   - the expert-pack residency (mmap + pread of packed_experts/layer_XX.bin)
 *       src/runtime.m:2426-2465, 1588-1634; include/nmoe/expert_io.h:21-24
 *   - the router + top-k:  metal/kernels.metal:472-513 (logits),
 *       src/runtime.m:1498-1511 -> src/math.m:67-153 (softmax/top-k/renorm)
 *   - the expert kernels: metal/kernels.metal:562-640 (gate/up + SwiGLU),
 *       642-714 and 1456-1542 (down + weighted combine), 1394-1454 (combine)
 *   - the per-layer MoE call NMOEPipelinedExpertTail, src/runtime.m:2908-2999
 *
 * Conventions (every entry point):
 *   - returns 0 (NMOE_HIP_OK) or a negative NMOE_HIP_E* code; the message is
 *     available from nmoe_hip_last_error();
 *   - arguments are validated on the host before any launch;
 *   - calls that launch work are asynchronous and stream-ordered and never
 *     allocate (all scratch is sized at nmoe_hip_create);
 *   - a context is not thread-safe and its launches must be ordered on one
 *     stream (the persistent kernels share the context's barrier words).
 */
#ifndef NMOE_HIP_H
#define NMOE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Model constants (src/runtime.m:31-48, scripts/convert_qwen36.py:31-36). */
#define NMOE_HIP_HIDDEN 2048
#define NMOE_HIP_INTER 512
#define NMOE_HIP_EXPERTS 256
#define NMOE_HIP_GROUP 64
#define NMOE_HIP_MAX_K 8 /* kNMOEMaxExperts, src/runtime.m:43 */
#define NMOE_HIP_MAX_LAYERS 64

/* Expert pack sizes, src/expert_io.m:90-99. */
#define NMOE_HIP_EXPERT_SIZE_Q4 1769472u
#define NMOE_HIP_EXPERT_SIZE_Q2 983040u

/* Status codes. */
#define NMOE_HIP_OK 0
#define NMOE_HIP_EINVAL (-22)   /* bad argument: NULL, K outside 1..8, size, alignment */
#define NMOE_HIP_ENOMEM (-12)   /* device allocation failed (create / upload only) */
#define NMOE_HIP_ENODEV (-19)   /* no such device / HIP runtime error at create */
#define NMOE_HIP_ENOENT (-2)    /* layer pack or buffer label not present */
#define NMOE_HIP_EIO (-5)       /* file read failed / wrong file size */
#define NMOE_HIP_EHIP (-71)     /* a HIP runtime call failed */
#define NMOE_HIP_ETIMEDOUT (-110) /* a persistent kernel hit its bounded wait */

/* Element types for activations passed in. */
#define NMOE_HIP_F32 0
#define NMOE_HIP_BF16 1

/* Exported symbols (the library is built with -fvisibility=hidden). */
#if defined(__GNUC__) || defined(__clang__)
#define NMOE_HIP_API __attribute__((visibility("default")))
#else
#define NMOE_HIP_API
#endif

typedef struct nmoe_hip_ctx nmoe_hip_ctx;

/* ---- context (replaces nmoe_backend_create/destroy, backend.h:55-56, and the
 *      one-time buffer set-up NMOEInitExpertIOBuffers, runtime.m:1542-1584) */

/* max_tokens bounds ntok for every later call; scratch for that many tokens
 * is allocated here, once. */
NMOE_HIP_API int nmoe_hip_create(int device, int max_tokens, nmoe_hip_ctx **out);
NMOE_HIP_API void nmoe_hip_destroy(nmoe_hip_ctx *ctx);
NMOE_HIP_API const char *nmoe_hip_last_error(const nmoe_hip_ctx *ctx);
NMOE_HIP_API void *nmoe_hip_stream(nmoe_hip_ctx *ctx);
NMOE_HIP_API int nmoe_hip_synchronize(nmoe_hip_ctx *ctx);
/* Number of compute units of the context's device. */
NMOE_HIP_API int nmoe_hip_device_cus(const nmoe_hip_ctx *ctx);
/* Reads (and clears) the device-side status word that persistent kernels set
 * when a bounded wait expires: returns 0 or NMOE_HIP_ETIMEDOUT.  Synchronous. */
NMOE_HIP_API int nmoe_hip_check_device_status(nmoe_hip_ctx *ctx);

/* Path options (the counterpart of the reference's experiment toggles,
 * NMOE_FUSED_DOWN_COMBINE_Q4 / NMOE_PIPELINE etc., runtime.m:1426-1496).
 * NMOE_HIP_OPT_FUSED_DECODE (default 1): single-token calls run as one
 * persistent launch; 0 selects the multi-launch kernels.
 * NMOE_HIP_OPT_XCD_LOCAL (default 1 where the device deals the blocks of a
 * launch round-robin over its 8 accelerator dies, checked at create): the
 * fused launch exchanges values that stay within a group of blocks on one
 * die through that die's L2; 0 sends them through device-coherent memory
 * like the rest. */
#define NMOE_HIP_OPT_FUSED_DECODE 1
#define NMOE_HIP_OPT_XCD_LOCAL 2
/* NMOE_HIP_OPT_GROUPED_MIN_TOKENS (default 8): calls with at least this many
 * tokens run the experts as grouped GEMMs on the matrix cores (dispatch
 * permutation, then each expert's weights read once for all its tokens);
 * fewer tokens run the per-token kernels. */
#define NMOE_HIP_OPT_GROUPED_MIN_TOKENS 3
/* NMOE_HIP_OPT_SPIN_LIMIT (default 0 = 2^20): unsuccessful poll rounds a
 * persistent kernel's bounded wait tolerates before it gives up (a round
 * trip to memory is about 1 us); at most NMOE_HIP_SPIN_LIMIT_MAX.  A wait
 * that gives up sets the device status word (nmoe_hip_check_device_status
 * returns NMOE_HIP_ETIMEDOUT) and makes every output the launch still writes
 * NaN, so the failure also shows in the data without a host round trip. */
#define NMOE_HIP_OPT_SPIN_LIMIT 4
#define NMOE_HIP_SPIN_LIMIT_MAX (1 << 26)
/* NMOE_HIP_OPT_SYNC_CHECK (default 0): 1 makes nmoe_moe_experts_*,
 * nmoe_moe_layer, nmoe_moe_layer_rmsnorm and nmoe_moe_stack wait for their
 * stream and return NMOE_HIP_ETIMEDOUT when a bounded wait expired (the
 * call is then synchronous; nmoe_moe_stack checks once, after its last
 * layer). */
#define NMOE_HIP_OPT_SYNC_CHECK 5
/* NMOE_HIP_OPT_SKEW_EPOCH (value = block 0..255; for tests of the failure
 * path): moves that block's launch epoch one ahead, so the next fused
 * launch cannot complete and ends through its bounded waits, as a launch
 * whose blocks are not all resident would.  nmoe_hip_check_device_status
 * then realigns the epochs.  Synchronous. */
#define NMOE_HIP_OPT_SKEW_EPOCH 6
/* NMOE_HIP_OPT_STACK_LOOP (default 1): nmoe_moe_stack runs the token's
 * layers in one persistent launch (up to 64 layers per launch; the next
 * layer's router row is fetched while the current one streams, and no
 * launch boundary separates the layers) when all its packs have one bit
 * width and all its routers one kind; 0 runs one launch per layer. */
#define NMOE_HIP_OPT_STACK_LOOP 7
/* NMOE_HIP_OPT_GROUPED_ONE_LAUNCH (default 1 where the device deals the
 * blocks of a launch round-robin over its 8 dies, checked at create): the
 * grouped path runs gate/up and down in one launch, each down tile starting
 * once its expert's gate/up tiles are done (a bounded wait); 0 runs them as
 * two launches.  The results are the same to the grouped path's
 * tolerance. */
#define NMOE_HIP_OPT_GROUPED_ONE_LAUNCH 8
/* NMOE_HIP_OPT_SKEW_TILES (value = expert rank 0..255, by entries, most
 * first; for tests of the failure path): the next one-launch grouped call
 * starts that rank's count of finished gate/up tiles at an impossible
 * value, so its down tiles find the count wrong, as they would had the
 * tiles run on another die: the call's outputs are NaN and
 * nmoe_hip_check_device_status returns NMOE_HIP_ETIMEDOUT.  Once. */
#define NMOE_HIP_OPT_SKEW_TILES 9
NMOE_HIP_API int nmoe_hip_set_option(nmoe_hip_ctx *ctx, int option, int value);

/* Per-stage timing of the fused launches (the counterpart of the
 * reference's --timing stage clocks, src/runtime.m:56-78, 2139-2143,
 * 3843-3894).  Only a library built with the phase timeline
 * (libnmoe_hip_tl.so, `make timeline`) records it; the product build returns
 * NMOE_HIP_EINVAL.  stamps: device memory of slots x 256 x 16 uint64; each
 * fused launch (each layer of a stack launch) takes the next slot in turn,
 * and block b writes the device's real-time clock at its phase boundaries
 * to stamps[slot][b][event] (events in nmoe_hip.py's TL_EVENTS; unwritten
 * stamps keep their contents).  The grouped path's launches (the
 * preparation, then the GEMM launch or launches) take the next slots as
 * well, 4 words a block from the slot's start: the clock at its start, at a
 * ready point and at its end, and what it ran (entries << 32 | kind << 28 |
 * die << 24 | expert entry or block << 8 | tile; kind 1 gate/up, 2 down,
 * 3 routing, 4 dispatch, 5 x planes).  NULL and 0 stop the recording. */
NMOE_HIP_API int nmoe_hip_set_timeline(nmoe_hip_ctx *ctx, void *stamps, int slots);

/* ---- buffers (backend.h:64-66: register_shared_buffer / register_state_buffer
 *      / lookup_shared_buffer).  The context owns them until destroy. */
NMOE_HIP_API int nmoe_hip_register_state_buffer(nmoe_hip_ctx *ctx, const char *label, size_t size, void **dev_out);
NMOE_HIP_API int nmoe_hip_register_shared_buffer(nmoe_hip_ctx *ctx, const char *label, const void *host, size_t size,
                                    void **dev_out);
NMOE_HIP_API void *nmoe_hip_lookup_buffer(const nmoe_hip_ctx *ctx, const char *label);
NMOE_HIP_API int nmoe_hip_copy_to_device(nmoe_hip_ctx *ctx, void *dev, const void *host, size_t size);
NMOE_HIP_API int nmoe_hip_copy_to_host(nmoe_hip_ctx *ctx, void *host, const void *dev, size_t size);

/* ---- expert packs (expert_io.h:21-24; runtime.m:2426-2465 NMOELoadExpertLayer).
 * A layer pack is the layer_XX.bin bytes unchanged: 256 experts of
 * nmoe_hip_expert_size(bits) bytes each, component offsets as
 * convert_qwen36.py:38-64.  Packs stay resident in HBM until destroy.
 * Each resident layer also holds a second copy of the same size, written on
 * the device after every upload or synthesis, whose code matrices the
 * grouped (many-token) path reads stripe-major: a layer takes twice its
 * pack's bytes of device memory (ENOMEM when either does not fit), and the
 * pack must be changed only through these calls. */
NMOE_HIP_API size_t nmoe_hip_expert_size(int bits);
NMOE_HIP_API int nmoe_hip_upload_layer_pack(nmoe_hip_ctx *ctx, int layer, int bits, const void *host, size_t size);
NMOE_HIP_API int nmoe_hip_load_layer_file(nmoe_hip_ctx *ctx, int layer, int bits, const char *path);

/* Validates an expert directory's layout.json against the fixed pack layout.
 * Accepts the converter's schema {expert_size, num_layers, num_experts,
 * components[{name, offset, size}]} (scripts/convert_qwen36.py:341-360) and
 * the richer one src/expert_io.m:230-320 reads (bits/quant, per-component
 * dtype/shape/logical_shape).  bits comes from bits/quant, else from
 * expert_size; num_layers is 0 when absent.  No context needed; err
 * (nullable) receives the reason.  EINVAL on a mismatch, ENOENT when the file
 * cannot be opened. */
NMOE_HIP_API int nmoe_hip_validate_layout(const char *layout_json_path, int *bits, int *num_layers, char *err,
                                          size_t err_len);
/* Validates dir/layout.json, then makes dir/layer_00.bin .. layer_{n-1}.bin
 * resident as layers 0..n-1 (each with nmoe_hip_load_layer_file's size
 * check); n = nlayers if > 0, else num_layers of the file.  bits_out and
 * layers_out (nullable) receive the quantisation and the layers loaded. */
NMOE_HIP_API int nmoe_hip_load_expert_dir(nmoe_hip_ctx *ctx, const char *dir, int nlayers, int *bits_out,
                                          int *layers_out);
/* Device address of a resident layer pack (NULL if absent), read-only: the
 * bytes as uploaded, not the grouped path's stripe-major copy. */
NMOE_HIP_API const void *nmoe_hip_layer_pack(const nmoe_hip_ctx *ctx, int layer, int *bits_out);
/* Allocates layer `layer` and fills it with the repository's synthetic
 * generator (counter-based SplitMix64; codes uniform, scales bf16 of an
 * Irwin-Hall(12) normal times sigma, bias = bf16(-8*scale) for q4 and
 * bf16(-1.5*scale) for q2).  Bench/test data; no reference counterpart. */
NMOE_HIP_API int nmoe_hip_synth_layer_pack(nmoe_hip_ctx *ctx, int layer, int bits, uint64_t seed, float sigma);
/* Fills n bf16 values with the same generator (tag selects the stream). */
NMOE_HIP_API int nmoe_hip_synth_bf16(nmoe_hip_ctx *ctx, uint16_t *dev, size_t n, uint64_t seed, uint32_t layer, uint32_t tag,
                        float sigma, void *stream);

/* ---- router.  Either a dense bf16 router [E][hidden] (the benchmark
 * configs) or the reference model's q4 router (runtime.m:2357, evaluated by
 * kernels.metal:472-513): u32 [E][hidden/8], bf16 scales/biases [E][hidden/64]. */
#define NMOE_HIP_ROUTER_BF16 0
#define NMOE_HIP_ROUTER_Q4 1
typedef struct nmoe_hip_router {
    int kind;
    int num_experts; /* 256 */
    const uint16_t *w_bf16;
    const uint32_t *w_q4;
    const uint16_t *scales;
    const uint16_t *biases;
} nmoe_hip_router;

/* logits[ntok][E] = router . x (fp32 accumulate, fixed reduction order). */
NMOE_HIP_API int nmoe_moe_router_logits(nmoe_hip_ctx *ctx, const nmoe_hip_router *router, const void *x, int x_dtype,
                           int ntok, float *logits, void *stream);
/* math.m softmax -> top-k (ties to the lower index) -> renormalise, per token
 * (runtime.m:1498-1511).  idx/w: [ntok][8], unused slots idx 0 / w 0
 * (kernels.metal:1767-1775).  probs (nullable): [ntok][E] softmax output. */
NMOE_HIP_API int nmoe_moe_topk(nmoe_hip_ctx *ctx, const float *logits, int ntok, int num_experts, int k, uint32_t *idx,
                  float *w, float *probs, void *stream);
/* router logits + top-k.  logits (nullable) receives the logits. */
NMOE_HIP_API int nmoe_moe_route(nmoe_hip_ctx *ctx, const nmoe_hip_router *router, const void *x, int x_dtype, int ntok, int k,
                   uint32_t *idx, float *w, float *logits, void *stream);

/* ---- routed experts with the routing given (the expert phase,
 * runtime.m:2778-2903):
 *   out[t] = h_mid[t] + sum_s w[t][s] * down_e(SwiGLU(gate_e x[t], up_e x[t]))
 *            (+ sigmoid(shared_gate_raw[t]) * shared_out[t])
 * with e = idx[t][s], the sum over slots in order (kernels.metal:1394-1423).
 * x: [ntok][2048] fp32 or bf16; h_mid, out, shared_out: fp32 [ntok][2048];
 * shared_gate_raw: fp32 [ntok]; shared_* both NULL or both set.  out may
 * alias h_mid (the residual is updated in place, runtime.m:2827-2831). */
NMOE_HIP_API int nmoe_moe_experts_q4(nmoe_hip_ctx *ctx, int layer, const void *x, int x_dtype, int ntok, int k,
                        const uint32_t *idx, const float *w, const float *h_mid, const float *shared_out,
                        const float *shared_gate_raw, float *out, void *stream);
NMOE_HIP_API int nmoe_moe_experts_q2(nmoe_hip_ctx *ctx, int layer, const void *x, int x_dtype, int ntok, int k,
                        const uint32_t *idx, const float *w, const float *h_mid, const float *shared_out,
                        const float *shared_gate_raw, float *out, void *stream);

/* ---- dispatch permutation for batched tokens (no reference counterpart:
 * the reference runs its MoE tail once per token, runtime.m:3816).  The
 * entries q = t*k + s of idx [ntok][8] (slots s < k) sorted stably by
 * expert -- ties by t, then s: perm [ntok*k] lists the entries of expert 0,
 * then expert 1, ...; offsets [257]: expert e owns perm[offsets[e] ..
 * offsets[e+1]).  Entries whose index is >= 256 are left out (offsets[256]
 * counts the rest). */
NMOE_HIP_API int nmoe_moe_dispatch(nmoe_hip_ctx *ctx, const uint32_t *idx, int ntok, int k, uint32_t *perm,
                                   uint32_t *offsets, void *stream);

/* ---- the shared expert (metal/kernels.metal:421-469 and 510-513: rows 0-511
 * and 768 of nmoe_route_shared_q4; :1520-1537: the shared down of
 * nmoe_expert_down_combine_q4; tensors mlp.shared_expert.{gate,up,down}_proj
 * and mlp.shared_expert_gate, src/runtime.m:2360-2369):
 *   act[t]             = SiLU(Wg . x[t]) * (Wu . x[t])   Wg, Wu: q4 [512][2048]
 *   shared_out[t]      = Wd . act[t]                     Wd: q4 [2048][512]
 *   shared_gate_raw[t] = Ws . x[t]                       Ws: q4 [1][2048]
 * A q4 tensor is the model's own quantised tensor, unchanged: w u32
 * [rows][cols/8] (column 8w+v in nibble v), scales and biases bf16
 * [rows][cols/64], weight = q*scale + bias.  The outputs are the
 * shared_out / shared_gate_raw inputs of the expert and layer calls, whose
 * combine adds sigmoid(shared_gate_raw) * shared_out (kernels.metal:1539-1541).
 * x: [ntok][2048] fp32 or bf16; shared_out fp32 [ntok][2048];
 * shared_gate_raw fp32 [ntok]. */
typedef struct nmoe_hip_qtensor {
    const uint32_t *w;
    const uint16_t *scales;
    const uint16_t *biases;
} nmoe_hip_qtensor;

typedef struct nmoe_hip_shared_expert {
    nmoe_hip_qtensor gate;  /* [512][2048] */
    nmoe_hip_qtensor up;    /* [512][2048] */
    nmoe_hip_qtensor down;  /* [2048][512] */
    nmoe_hip_qtensor score; /* [1][2048] */
} nmoe_hip_shared_expert;

NMOE_HIP_API int nmoe_moe_shared_expert(nmoe_hip_ctx *ctx, const nmoe_hip_shared_expert *se, const void *x,
                                        int x_dtype, int ntok, float *shared_out, float *shared_gate_raw,
                                        void *stream);

/* ---- the whole per-layer MoE call (NMOEPipelinedExpertTail,
 * runtime.m:2908-2999, with routing on the device and no host round trip):
 * route x, run the selected experts of resident layer `layer`, combine into
 * out.  idx/w/logits (nullable) receive the routing. */
NMOE_HIP_API int nmoe_moe_layer(nmoe_hip_ctx *ctx, int layer, const nmoe_hip_router *router, const void *x, int x_dtype,
                   int ntok, int k, const float *h_mid, const float *shared_out, const float *shared_gate_raw,
                   float *out, uint32_t *idx, float *w, float *logits, void *stream);

/* ---- the per-layer call with the layer's input RMSNorm in front
 * (math.m:34-65, unit weight, bit-exact), the way the reference runs the next
 * layer's input norm right after the combine (runtime.m:2893-2900):
 *   h_out = h_in + MoE(RMSNorm(h_in)).
 * One token, bf16 or q4 router; h_out must not alias h_in. */
NMOE_HIP_API int nmoe_moe_layer_rmsnorm(nmoe_hip_ctx *ctx, int layer, const nmoe_hip_router *router,
                                        const float *h_in, float eps, int k, float *h_out, uint32_t *idx, float *w,
                                        float *logits, void *stream);

/* ---- the MoE half of one layer, whole, for one token in one launch: the
 * route/shared stage of the attention step's tail (src/runtime.m:3144-3201:
 * post-attention RMSNorm, the q4 router, the shared expert's gate/up and
 * score, kernels.metal:384-514), the expert tail NMOEPipelinedExpertTail
 * (runtime.m:2908-2999, the shared down in the combine, kernels.metal:
 * 1456-1542) and the next layer's input norm (runtime.m:2893-2900):
 *   x      = RMSNorm(h_mid) * w_post       (math.m:34-65; w = 1 + weight with
 *                                           add_one, unit weight when NULL)
 *   idx, w = softmax / top-k / renormalise of router . x
 *   out    = h_mid + sum_s w_s down_s(SwiGLU(gate_s x, up_s x))
 *            + sigmoid(score . x) * shared_down(SwiGLU(shared_gate x, shared_up x))
 *   next_x = RMSNorm(out) * w_next         (when next_x is not NULL)
 * out may alias h_mid (the residual is updated in place, runtime.m:2827-2831);
 * h_mid 16-byte aligned.  nmoe_hip_layer_block fills the descriptor from
 * weights loaded by nmoe_hip_load_model_weights. */
typedef struct nmoe_hip_moe_block {
    nmoe_hip_router router;        /* the layer's router: the model's q4 .mlp.gate, or bf16 */
    int has_shared;                /* 1: `shared` holds the layer's shared expert */
    nmoe_hip_shared_expert shared; /* .mlp.shared_expert.{gate,up,down}_proj, .mlp.shared_expert_gate */
    const uint16_t *post_norm;     /* bf16 [2048] post_attention_layernorm.weight, NULL = unit */
    const uint16_t *next_norm;     /* bf16 [2048] the next layer's input_layernorm.weight, NULL = unit */
    int add_one;                   /* 1: the norm weights enter as 1 + w (the model's, runtime.m:3149, 2898) */
    float eps;                     /* rms_norm_eps */
} nmoe_hip_moe_block;

NMOE_HIP_API int nmoe_moe_block(nmoe_hip_ctx *ctx, int layer, const nmoe_hip_moe_block *blk, const float *h_mid,
                                int k, float *out, float *next_x, uint32_t *idx, float *w, float *logits,
                                void *stream);

/* ---- the model's non-expert weights of the MoE path, from the converter's
 * model_weights.bin / model_weights.json (scripts/convert_qwen36.py:266-327;
 * read by src/manifest.m:229-316).  For layers 0 .. n-1 (n = nlayers, or
 * config.num_hidden_layers when 0) the tensors the MoE block needs
 * (runtime.m:2349-2369: input_layernorm / post_attention_layernorm .weight
 * BF16; mlp.gate, mlp.shared_expert.{gate,up,down}_proj, mlp.shared_expert_gate
 * as .weight U32 + .scales/.biases BF16) are checked -- present, dtype and
 * range as NMOETensorPointer (runtime.m:2271-2299), size as the kernels read
 * them -- and made resident; the manifest may take any of the shapes the
 * reference's reader walks.  layers_out (nullable) receives n. */
NMOE_HIP_API int nmoe_hip_load_model_weights(nmoe_hip_ctx *ctx, const char *bin_path, const char *json_path,
                                             int nlayers, int *layers_out);
/* The MoE block of a loaded layer: q4 router, shared expert, its
 * post-attention norm, the next layer's input norm (NULL for the last
 * loaded layer), add_one 1, eps = config.rms_norm_eps.  ENOENT if the
 * layer's weights are not loaded. */
NMOE_HIP_API int nmoe_hip_layer_block(const nmoe_hip_ctx *ctx, int layer, nmoe_hip_moe_block *out);

/* ---- routing from given router logits and the routed experts in one call
 * (runtime.m:1498-1511 routing, then the expert tail of
 * NMOEPipelinedExpertTail, runtime.m:2908-2999), for callers whose router
 * logits are already on the device (batched decode, prompt processing: the
 * reference's prompt loop runs the same per-token step, runtime.m:3814-3818).
 * logits: fp32 [ntok][256]; idx / w: [ntok][8] receive the routing, bit for
 * bit nmoe_moe_topk's (math.m softmax / top-k / renormalise); out as
 * nmoe_moe_experts_q4/q2 on the layer's pack (either width).  From
 * NMOE_HIP_OPT_GROUPED_MIN_TOKENS tokens on, the routing runs inside the
 * grouped path's first launch instead of a launch of its own. */
NMOE_HIP_API int nmoe_moe_experts_from_logits(nmoe_hip_ctx *ctx, int layer, const float *logits, const void *x,
                                              int x_dtype, int ntok, int k, const float *h_mid,
                                              const float *shared_out, const float *shared_gate_raw, float *out,
                                              uint32_t *idx, float *w, void *stream);

/* ---- the routed-expert stack of one decode token (the layer loop of
 * NMOEProcessToken, runtime.m:3732-3777, restricted to the MoE tails):
 * h_seq[l+1] = h_seq[l] + MoE_l(RMSNorm(h_seq[l])) for l < nlayers.
 * layers[l]: resident pack of layer l; routers[l]: its router (bf16 or q4).
 * h_seq: fp32 [nlayers+1][2048] (row 0 = input, 16-byte aligned);
 * idx_seq / w_seq: nullable [nlayers][8].  One launch for all layers
 * (NMOE_HIP_OPT_STACK_LOOP), else one per layer; the results are the
 * same bits either way. */
NMOE_HIP_API int nmoe_moe_stack(nmoe_hip_ctx *ctx, int nlayers, const int *layers, const nmoe_hip_router *routers,
                                int k, float eps, float *h_seq, uint32_t *idx_seq, float *w_seq, void *stream);

/* ---- the per-layer MoE call without allocation and without a context.
 * No counterpart in the reference (its runtime allocates every buffer at
 * start-up, runtime.m:1542-1584).  It is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  Same computation as nmoe_moe_layer on
 * the current device: layer_pack is a resident layer (256 experts of
 * nmoe_hip_expert_size(bits) bytes, e.g. nmoe_hip_layer_pack's address),
 * router a 256-expert router, and for ntok > 1 the per-token kernels run
 * (never the grouped ones).  Calls no hipMalloc/hipFree and no allocating
 * library routine: its scratch is a fixed device array of
 * NMOE_HIP_STATIC_SCRATCH_BYTES per GPU, held until the process ends, so
 * ntok is at most NMOE_HIP_STATIC_MAX_TOKENS (EINVAL beyond).  Calls share
 * that array: calls that overlap on one GPU race.  idx/w (nullable) receive
 * the routing.  A bounded wait that gives up shows as NaN in out and w
 * (there is no context to hold a status).  Any call, the first on a device
 * included, may be made while `stream` is being captured into a HIP graph:
 * it then only launches kernels on it (the one-time die-placement check,
 * a launch and a copy back, waits for the first call on a stream that is
 * not capturing), and every replay of the graph is a new launch with its
 * own synchronisation epoch, counted on the device. */
#define NMOE_HIP_STATIC_MAX_TOKENS 16
#define NMOE_HIP_STATIC_SCRATCH_BYTES 722944u
NMOE_HIP_API int nmoe_moe_layer_static(const void *layer_pack, int bits, const nmoe_hip_router *router,
                                       const void *x, int x_dtype, int ntok, int k, const float *h_mid,
                                       const float *shared_out, const float *shared_gate_raw, float *out,
                                       uint32_t *idx, float *w, void *stream);

/* ---- the streaming ceiling of the decode step (a measurement entry point;
 * no reference counterpart, like the reference's matvec micro-benchmark
 * scripts/matvec_bench.m): reads `bytes` (a multiple of 16) from src once,
 * with the fused step's expert-load pattern (256 blocks of 512 threads, 8
 * non-temporal 16-byte loads a thread in flight before any is used, in
 * rounds of 16 MiB), folding them into sink[2048] words.  Its launch time
 * is the floor of the step's expert phase: the step's expert bytes streamed
 * from a cold start with no routing before and no exchange after. */
NMOE_HIP_API int nmoe_hip_read_probe(nmoe_hip_ctx *ctx, const void *src, size_t bytes, uint32_t *sink, void *stream);

/* The same read at any launch shape: `blocks` (1..8192) blocks of `threads`
 * (64..1024, a multiple of 64), `loads` (1, 2, 4, 8 or 16) 16-byte loads a
 * thread a round.  Block b reads the 16-byte items [b*per, min((b+1)*per, n)),
 * per = ceil(n / blocks), in rounds of threads*loads items; sink receives
 * blocks*threads/64 words, word b*(threads/64)+w the XOR of every 32-bit
 * word wavefront w of block b read.  For the sweep of the part's sustained
 * read rate against size and shape; a 16-byte read gives the period of a
 * near-empty launch of the grid. */
NMOE_HIP_API int nmoe_hip_read_probe_grid(nmoe_hip_ctx *ctx, const void *src, size_t bytes, int blocks, int threads,
                                          int loads, uint32_t *sink, void *stream);

/* ---- bit-exact dequant probe (kernels.metal:1066-1106 nmoe_dequant_row_q4/q2,
 * math.m:206-234): out[r][c] = q*scale + bias for `rows` rows of `in_dim`. */
NMOE_HIP_API int nmoe_dequant_rows(nmoe_hip_ctx *ctx, int bits, const uint32_t *packed, const uint16_t *scales,
                      const uint16_t *biases, int rows, int in_dim, float *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif
