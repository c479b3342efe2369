/*
 * stack.c -- the routed-expert layer loop of one decode token (plain C).
 *
 * The reference's NMOEProcessToken (src/runtime.m:3712-3777) walks the 40
 * layers; each layer ends with the MoE tail and the next layer's input
 * RMSNorm (runtime.m:2893-2900).  The layers run as one persistent
 * launch (up to 64 layers each) when they share a bit width and a router
 * kind; otherwise, or with NMOE_HIP_OPT_STACK_LOOP off, this loop issues
 * one fused launch per layer (nmoe_moe_layer_rmsnorm), all on one stream,
 * with no host synchronisation between layers.
 */
#include <stddef.h>

#include "nmoe_hip.h"

int nmoe_host_fail(nmoe_hip_ctx *ctx, int code, const char *msg);
int nmoe_layer_rmsnorm_launch(nmoe_hip_ctx *ctx, int layer, const nmoe_hip_router *router, const float *h_in,
                              float eps, int k, float *h_out, uint32_t *idx, float *w, float *logits, void *stream);
int nmoe_sync_check(nmoe_hip_ctx *ctx, void *stream);
int nmoe_stack_loop_launch(nmoe_hip_ctx *ctx, int nlayers, const int *layers, const nmoe_hip_router *routers, int k,
                           float eps, float *h_seq, uint32_t *idx_seq, float *w_seq, void *stream);

int nmoe_moe_stack(nmoe_hip_ctx *ctx, int nlayers, const int *layers, const nmoe_hip_router *routers, int k,
                   float eps, float *h_seq, uint32_t *idx_seq, float *w_seq, void *stream) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (nlayers < 1 || layers == NULL || routers == NULL || h_seq == NULL)
        return nmoe_host_fail(ctx, NMOE_HIP_EINVAL, "nlayers >= 1, layers, routers and h_seq are required");
    int rc = nmoe_stack_loop_launch(ctx, nlayers, layers, routers, k, eps, h_seq, idx_seq, w_seq, stream);
    if (rc != 1) return rc != NMOE_HIP_OK ? rc : nmoe_sync_check(ctx, stream);
    for (int l = 0; l < nlayers; l++) {
        rc = nmoe_layer_rmsnorm_launch(ctx, layers[l], &routers[l], h_seq + (size_t)l * NMOE_HIP_HIDDEN, eps, k,
                                           h_seq + (size_t)(l + 1) * NMOE_HIP_HIDDEN,
                                           idx_seq != NULL ? idx_seq + (size_t)l * NMOE_HIP_MAX_K : NULL,
                                           w_seq != NULL ? w_seq + (size_t)l * NMOE_HIP_MAX_K : NULL, NULL, stream);
        if (rc != NMOE_HIP_OK) return rc;
    }
    return nmoe_sync_check(ctx, stream);
}
