/*
 * abi_client.c -- a plain C caller of include/nmoe_hip.h, linked against
 * libnmoe_hip.so the way the reference's host would link it (the
 * reference's callers of the per-layer MoE call are Objective-C,
 * src/runtime.m:3198-3201, 3544-3547; Objective-C is a superset of C).
 * tests/test_c_boundary.py compiles this file as C11, as C++17 and as
 * Objective-C, with warnings as errors.
 *
 *   abi_client layout   prints the sizes and field offsets of the header's
 *                       structs (the binding's ctypes layouts must match)
 *   abi_client cpu DIR  argument validation and the calls that need no GPU
 *                       (DIR: tests/golden, for the layout.json fixtures)
 *   abi_client gpu OUT  one q4 top-8 decode step through nmoe_moe_layer on
 *                       device 0 with the repository's synthetic layer,
 *                       router and input (seed 0, layer 0); writes idx[8],
 *                       w[8] and out[2048] to OUT for the test to check
 *                       against the oracle; then a 3-layer nmoe_moe_stack
 *                       on that layer, as one launch and as one launch per
 *                       layer, which must agree bit for bit
 */
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "nmoe_hip.h"

static int failures = 0;

#define EXPECT(cond)                                                   \
    do {                                                               \
        if (!(cond)) {                                                 \
            fprintf(stderr, "%s:%d: failed: %s\n", __FILE__, __LINE__, #cond); \
            failures++;                                                \
        }                                                              \
    } while (0)

static int run_layout(void) {
    printf("router %zu %zu %zu %zu %zu %zu %zu\n", sizeof(nmoe_hip_router), offsetof(nmoe_hip_router, kind),
           offsetof(nmoe_hip_router, num_experts), offsetof(nmoe_hip_router, w_bf16), offsetof(nmoe_hip_router, w_q4),
           offsetof(nmoe_hip_router, scales), offsetof(nmoe_hip_router, biases));
    printf("qtensor %zu %zu %zu %zu\n", sizeof(nmoe_hip_qtensor), offsetof(nmoe_hip_qtensor, w),
           offsetof(nmoe_hip_qtensor, scales), offsetof(nmoe_hip_qtensor, biases));
    printf("shared %zu %zu %zu %zu %zu\n", sizeof(nmoe_hip_shared_expert), offsetof(nmoe_hip_shared_expert, gate),
           offsetof(nmoe_hip_shared_expert, up), offsetof(nmoe_hip_shared_expert, down),
           offsetof(nmoe_hip_shared_expert, score));
    printf("block %zu %zu %zu %zu %zu %zu %zu %zu\n", sizeof(nmoe_hip_moe_block), offsetof(nmoe_hip_moe_block, router),
           offsetof(nmoe_hip_moe_block, has_shared), offsetof(nmoe_hip_moe_block, shared),
           offsetof(nmoe_hip_moe_block, post_norm), offsetof(nmoe_hip_moe_block, next_norm),
           offsetof(nmoe_hip_moe_block, add_one), offsetof(nmoe_hip_moe_block, eps));
    return 0;
}

static int run_cpu(const char *golden_dir) {
    nmoe_hip_ctx *ctx = NULL;
    EXPECT(nmoe_hip_create(0, 0, &ctx) == NMOE_HIP_EINVAL && ctx == NULL);
    EXPECT(nmoe_hip_create(0, 1 << 20, &ctx) == NMOE_HIP_EINVAL);
    EXPECT(nmoe_hip_create(0, 8, NULL) == NMOE_HIP_EINVAL);
    EXPECT(nmoe_hip_expert_size(4) == NMOE_HIP_EXPERT_SIZE_Q4);
    EXPECT(nmoe_hip_expert_size(2) == NMOE_HIP_EXPERT_SIZE_Q2);
    EXPECT(nmoe_hip_expert_size(3) == 0);
    EXPECT(strcmp(nmoe_hip_last_error(NULL), "no context") == 0);
    EXPECT(nmoe_hip_synchronize(NULL) == NMOE_HIP_EINVAL);
    EXPECT(nmoe_hip_set_option(NULL, NMOE_HIP_OPT_FUSED_DECODE, 1) == NMOE_HIP_EINVAL);
    EXPECT(nmoe_hip_device_cus(NULL) == 0);
    EXPECT(nmoe_hip_stream(NULL) == NULL);
    EXPECT(nmoe_hip_lookup_buffer(NULL, "x") == NULL);
    EXPECT(nmoe_hip_layer_pack(NULL, 0, NULL) == NULL);
    nmoe_hip_destroy(NULL);
    nmoe_hip_router r;
    memset(&r, 0, sizeof(r));
    r.kind = NMOE_HIP_ROUTER_BF16;
    r.num_experts = NMOE_HIP_EXPERTS;
    EXPECT(nmoe_moe_layer(NULL, 0, &r, NULL, NMOE_HIP_F32, 1, 8, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL) ==
           NMOE_HIP_EINVAL);
    EXPECT(nmoe_moe_stack(NULL, 1, NULL, NULL, 8, 1e-6f, NULL, NULL, NULL, NULL) == NMOE_HIP_EINVAL);
    EXPECT(nmoe_moe_experts_q4(NULL, 0, NULL, NMOE_HIP_F32, 1, 8, NULL, NULL, NULL, NULL, NULL, NULL, NULL) ==
           NMOE_HIP_EINVAL);
    /* the no-allocation call checks its arguments before it touches a device */
    EXPECT(nmoe_moe_layer_static(NULL, 4, &r, NULL, NMOE_HIP_F32, NMOE_HIP_STATIC_MAX_TOKENS + 1, 8, NULL, NULL, NULL,
                                 NULL, NULL, NULL, NULL) == NMOE_HIP_EINVAL);
    EXPECT(nmoe_moe_layer_static(NULL, 4, &r, NULL, NMOE_HIP_F32, 1, 8, NULL, NULL, NULL, NULL, NULL, NULL, NULL) ==
           NMOE_HIP_EINVAL);
    /* layout validation needs no context */
    char path[4096], err[256];
    int bits = 0, nl = -1;
    snprintf(path, sizeof path, "%s/layout_q4.json", golden_dir);
    EXPECT(nmoe_hip_validate_layout(path, &bits, &nl, err, sizeof err) == NMOE_HIP_OK && bits == 4);
    snprintf(path, sizeof path, "%s/layout_q2.json", golden_dir);
    EXPECT(nmoe_hip_validate_layout(path, &bits, &nl, err, sizeof err) == NMOE_HIP_OK && bits == 2);
    snprintf(path, sizeof path, "%s/does_not_exist.json", golden_dir);
    EXPECT(nmoe_hip_validate_layout(path, &bits, &nl, err, sizeof err) == NMOE_HIP_ENOENT);
    printf("cpu checks: %d failed\n", failures);
    return failures != 0;
}

#define CHECK(call)                                                                  \
    do {                                                                             \
        int rc_ = (call);                                                            \
        if (rc_ != NMOE_HIP_OK) {                                                    \
            fprintf(stderr, "%s -> %d: %s\n", #call, rc_, nmoe_hip_last_error(ctx)); \
            nmoe_hip_destroy(ctx);                                                   \
            return 1;                                                                \
        }                                                                            \
    } while (0)

static int run_gpu(const char *out_path) {
    nmoe_hip_ctx *ctx = NULL;
    if (nmoe_hip_create(0, 4, &ctx) != NMOE_HIP_OK) {
        fprintf(stderr, "nmoe_hip_create failed\n");
        return 1;
    }
    printf("device 0: %d CUs\n", nmoe_hip_device_cus(ctx));
    void *router = NULL, *x = NULL, *h = NULL, *out = NULL, *idx = NULL, *w = NULL;
    CHECK(nmoe_hip_synth_layer_pack(ctx, 0, 4, 0, 0.02f));
    CHECK(nmoe_hip_register_state_buffer(ctx, "router", (size_t)256 * 2048 * 2, &router));
    CHECK(nmoe_hip_register_state_buffer(ctx, "x", 2048 * 2, &x));
    CHECK(nmoe_hip_register_state_buffer(ctx, "h", 2048 * 4, &h));
    CHECK(nmoe_hip_register_state_buffer(ctx, "out", 2048 * 4, &out));
    CHECK(nmoe_hip_register_state_buffer(ctx, "idx", 32, &idx));
    CHECK(nmoe_hip_register_state_buffer(ctx, "w", 32, &w));
    CHECK(nmoe_hip_synth_bf16(ctx, (uint16_t *)router, (size_t)256 * 2048, 0, 0, 16, 0.02f, NULL));
    CHECK(nmoe_hip_synth_bf16(ctx, (uint16_t *)x, 2048, 0, 0, 17, 1.0f, NULL));
    /* h_mid stays zero (registered buffers are zero-filled): out = the MoE term */
    nmoe_hip_router r;
    memset(&r, 0, sizeof(r));
    r.kind = NMOE_HIP_ROUTER_BF16;
    r.num_experts = NMOE_HIP_EXPERTS;
    r.w_bf16 = (const uint16_t *)router;
    CHECK(nmoe_moe_layer(ctx, 0, &r, x, NMOE_HIP_BF16, 1, 8, (const float *)h, NULL, NULL, (float *)out,
                         (uint32_t *)idx, (float *)w, NULL, NULL));
    CHECK(nmoe_hip_synchronize(ctx));
    CHECK(nmoe_hip_check_device_status(ctx));
    uint32_t hi[8];
    float hw[8];
    float *ho = (float *)malloc(2048 * sizeof(float));
    if (ho == NULL) return 1;
    CHECK(nmoe_hip_copy_to_host(ctx, hi, idx, sizeof hi));
    CHECK(nmoe_hip_copy_to_host(ctx, hw, w, sizeof hw));
    CHECK(nmoe_hip_copy_to_host(ctx, ho, out, 2048 * sizeof(float)));
    FILE *f = fopen(out_path, "wb");
    int ok = f != NULL && fwrite(hi, sizeof hi, 1, f) == 1 && fwrite(hw, sizeof hw, 1, f) == 1 &&
             fwrite(ho, 2048 * sizeof(float), 1, f) == 1;
    if (f != NULL) fclose(f);
    printf("experts %u %u %u %u %u %u %u %u\n", hi[0], hi[1], hi[2], hi[3], hi[4], hi[5], hi[6], hi[7]);

    /* the token's layer loop (three entries of layer 0, the step's out as
     * h_0): one persistent launch, then one launch per layer */
    enum { NL = 3 };
    const int layers[NL] = {0, 0, 0};
    const nmoe_hip_router routers[NL] = {r, r, r};
    void *hseq = NULL, *iseq = NULL;
    float *hh[2] = {NULL, NULL};
    uint32_t si[2][NL * 8];
    CHECK(nmoe_hip_register_state_buffer(ctx, "hseq", (NL + 1) * 2048 * 4, &hseq));
    CHECK(nmoe_hip_register_state_buffer(ctx, "iseq", NL * 8 * 4, &iseq));
    for (int loop = 0; loop < 2; loop++) {
        hh[loop] = (float *)malloc((NL + 1) * 2048 * sizeof(float));
        if (hh[loop] == NULL) return 1;
        CHECK(nmoe_hip_set_option(ctx, NMOE_HIP_OPT_STACK_LOOP, loop));
        CHECK(nmoe_hip_copy_to_device(ctx, hseq, ho, 2048 * sizeof(float)));
        CHECK(nmoe_moe_stack(ctx, NL, layers, routers, 8, 1e-6f, (float *)hseq, (uint32_t *)iseq, NULL, NULL));
        CHECK(nmoe_hip_synchronize(ctx));
        CHECK(nmoe_hip_check_device_status(ctx));
        CHECK(nmoe_hip_copy_to_host(ctx, hh[loop], hseq, (NL + 1) * 2048 * sizeof(float)));
        CHECK(nmoe_hip_copy_to_host(ctx, si[loop], iseq, sizeof si[loop]));
    }
    const int same = memcmp(hh[0], hh[1], (NL + 1) * 2048 * sizeof(float)) == 0 && memcmp(si[0], si[1], sizeof si[0]) == 0;
    printf("stack: one launch equals one launch per layer: %s\n", same ? "yes" : "NO");
    free(hh[0]);
    free(hh[1]);
    free(ho);
    nmoe_hip_destroy(ctx);
    return ok && same ? 0 : 1;
}

int main(int argc, char **argv) {
    if (argc >= 2 && strcmp(argv[1], "layout") == 0) return run_layout();
    if (argc >= 3 && strcmp(argv[1], "cpu") == 0) return run_cpu(argv[2]);
    if (argc >= 3 && strcmp(argv[1], "gpu") == 0) return run_gpu(argv[2]);
    fprintf(stderr, "usage: abi_client layout | cpu GOLDEN_DIR | gpu OUT\n");
    return 2;
}
