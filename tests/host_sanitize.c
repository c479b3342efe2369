/*
 * host_sanitize.c -- runs the library's plain-C host code (host/json.c,
 * layout.c, weights.c, pack_io.c) and the CPU oracle on the files named on
 * the command line, built by tests/test_host_sanitize.py with
 * -fsanitize=address,undefined so that any out-of-bounds access, leak or
 * undefined operation on hostile input ends the run with a report.
 *
 * The device side of the library (context, buffers, uploads) is replaced
 * by the host-memory stand-ins below: the host code only hands them
 * pointers and sizes, which they check and copy.  TEST INFRASTRUCTURE: not
 * part of libnmoe_hip.so.
 *
 *   host_sanitize json FILE              jparse_text on the file's exact bytes
 *                                        (no terminating NUL)
 *   host_sanitize layout FILE            nmoe_hip_validate_layout
 *   host_sanitize weights BIN JSON N     nmoe_hip_load_model_weights
 *   host_sanitize layer FILE BITS        nmoe_hip_load_layer_file
 *   host_sanitize expdir DIR N           nmoe_hip_load_expert_dir
 *   host_sanitize oracle                 the oracle's routing, norm and dequant
 *                                        on non-finite and extreme values
 * Prints "rc=<status>" and exits 0 when nothing was detected.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../nano-metal-moe-qwen36_amd/host/json.h"
#include "../oracle/nmoe_oracle.h"
#include "nmoe_hip.h"

/* ---- stand-ins for the device side: host buffers behind labels */
#define MAXBUF 256
static struct {
    char label[64];
    unsigned char *p;
    size_t n;
} bufs[MAXBUF];
static int nbufs;
static char ctx_storage[64];
#define CTX ((nmoe_hip_ctx *)(void *)ctx_storage)

int nmoe_host_fail(nmoe_hip_ctx *ctx, int code, const char *msg) {
    (void)ctx;
    fprintf(stderr, "fail %d: %s\n", code, msg);
    return code;
}

int nmoe_ctx_set_block(nmoe_hip_ctx *ctx, int layer, const nmoe_hip_moe_block *b) {
    (void)ctx;
    if (layer < 0 || layer >= NMOE_HIP_MAX_LAYERS || b == NULL) abort();
    return NMOE_HIP_OK;
}

void *nmoe_hip_lookup_buffer(const nmoe_hip_ctx *ctx, const char *label) {
    (void)ctx;
    for (int i = 0; i < nbufs; i++)
        if (strcmp(bufs[i].label, label) == 0) return bufs[i].p;
    return NULL;
}

int nmoe_hip_register_shared_buffer(nmoe_hip_ctx *ctx, const char *label, const void *host, size_t size,
                                    void **dev_out) {
    (void)ctx;
    if (nbufs == MAXBUF || strlen(label) >= sizeof bufs[0].label) return NMOE_HIP_ENOMEM;
    unsigned char *p = (unsigned char *)malloc(size);
    if (p == NULL) return NMOE_HIP_ENOMEM;
    memcpy(p, host, size);
    strcpy(bufs[nbufs].label, label);
    bufs[nbufs].p = p;
    bufs[nbufs].n = size;
    nbufs++;
    *dev_out = p;
    return NMOE_HIP_OK;
}

int nmoe_hip_copy_to_device(nmoe_hip_ctx *ctx, void *dev, const void *host, size_t size) {
    (void)ctx;
    for (int i = 0; i < nbufs; i++)
        if (bufs[i].p == dev) {
            if (size > bufs[i].n) abort();
            memcpy(dev, host, size);
            return NMOE_HIP_OK;
        }
    abort();
}

size_t nmoe_hip_expert_size(int bits) {
    return bits == 4 ? NMOE_HIP_EXPERT_SIZE_Q4 : bits == 2 ? NMOE_HIP_EXPERT_SIZE_Q2 : 0;
}

int nmoe_hip_upload_layer_pack(nmoe_hip_ctx *ctx, int layer, int bits, const void *bytes, size_t n) {
    (void)ctx;
    if (layer < 0 || layer >= NMOE_HIP_MAX_LAYERS || n != NMOE_HIP_EXPERTS * nmoe_hip_expert_size(bits)) abort();
    /* touch every byte handed over */
    unsigned x = 0;
    for (size_t i = 0; i < n; i += 4096) x += ((const unsigned char *)bytes)[i];
    x += ((const unsigned char *)bytes)[n - 1];
    return x == 0xFFFFFFFFu ? NMOE_HIP_EIO : NMOE_HIP_OK;
}

static void free_bufs(void) {
    for (int i = 0; i < nbufs; i++) free(bufs[i].p);
    nbufs = 0;
}

/* ---- the oracle on non-finite and extreme values */
static int run_oracle(void) {
    const float specials[] = {0.0f, -0.0f, 1.0f, -1.0f, 1e-45f, -1e-45f, 3.4e38f, -3.4e38f, INFINITY, -INFINITY, NAN};
    const int ns = (int)(sizeof specials / sizeof specials[0]);
    float lg[ORC_EXPERTS], w8[ORC_MAX_K], probs[ORC_EXPERTS];
    uint32_t idx8[ORC_MAX_K];
    for (int a = 0; a < ns; a++)
        for (int b = 0; b < ns; b++) {
            for (int e = 0; e < ORC_EXPERTS; e++) lg[e] = (e % 3 == 0) ? specials[a] : specials[b];
            for (int k = 1; k <= ORC_MAX_K; k++) {
                orc_route(lg, ORC_EXPERTS, k, idx8, w8, probs);
                orc_route(lg, 3, k, idx8, w8, NULL); /* fewer experts than k */
                for (int s = 0; s < ORC_MAX_K; s++)
                    if (idx8[s] >= ORC_EXPERTS) abort();
            }
        }
    float h[ORC_HIDDEN], x[ORC_HIDDEN];
    uint16_t wn[ORC_HIDDEN];
    for (int a = 0; a < ns; a++) {
        for (int i = 0; i < ORC_HIDDEN; i++) {
            h[i] = specials[(a + i) % ns];
            wn[i] = (uint16_t)(0x3F80u + (unsigned)i);
        }
        orc_rms_norm(h, NULL, x, ORC_HIDDEN, 1e-6f, 0);
        orc_rms_norm(h, wn, x, ORC_HIDDEN, 0.0f, 1);
    }
    /* dequant rows with every scale / bias bit pattern class */
    uint32_t packed[ORC_HIDDEN / 8];
    uint16_t sc[ORC_HIDDEN / 64], bi[ORC_HIDDEN / 64];
    float row[ORC_HIDDEN];
    const uint16_t sb[] = {0x0000u, 0x8000u, 0x0001u, 0x7F7Fu, 0x7F80u, 0xFF80u, 0x7FC0u, 0x3F80u};
    for (int i = 0; i < ORC_HIDDEN / 8; i++) packed[i] = 0x9E3779B9u * (uint32_t)(i + 1);
    for (int a = 0; a < 8; a++)
        for (int b = 0; b < 8; b++) {
            for (int g = 0; g < ORC_HIDDEN / 64; g++) {
                sc[g] = sb[a];
                bi[g] = sb[b];
            }
            orc_dequant_row(packed, sc, bi, row, ORC_HIDDEN, 4);
            orc_dequant_row(packed, sc, bi, row, ORC_HIDDEN, 2);
        }
    printf("rc=0\n");
    return 0;
}

/* ---- the file's exact bytes, with no terminator after them */
static char *read_exact(const char *path, size_t *len) {
    FILE *f = fopen(path, "rb");
    if (f == NULL) return NULL;
    if (fseek(f, 0, SEEK_END) != 0) {
        fclose(f);
        return NULL;
    }
    long n = ftell(f);
    if (n < 0 || fseek(f, 0, SEEK_SET) != 0) {
        fclose(f);
        return NULL;
    }
    char *p = (char *)malloc(n > 0 ? (size_t)n : 1);
    if (p != NULL && n > 0 && fread(p, 1, (size_t)n, f) != (size_t)n) {
        free(p);
        p = NULL;
    }
    fclose(f);
    *len = (size_t)n;
    return p;
}

int main(int argc, char **argv) {
    if (argc < 2) return 2;
    const char *cmd = argv[1];
    int rc;
    if (strcmp(cmd, "oracle") == 0) return run_oracle();
    if (strcmp(cmd, "json") == 0 && argc == 3) {
        size_t len = 0;
        char *text = read_exact(argv[2], &len);
        if (text == NULL) return 3;
        jv root;
        rc = jparse_text(text, len, &root);
        if (rc == 0) {
            unsigned long long v;
            (void)jint(&root, &v);
            (void)jget(&root, "a");
            jv_free(&root);
        }
        free(text);
    } else if (strcmp(cmd, "layout") == 0 && argc == 3) {
        char err[128];
        int bits = 0, nl = 0;
        rc = nmoe_hip_validate_layout(argv[2], &bits, &nl, err, sizeof err);
        if (rc != 0) fprintf(stderr, "layout: %s\n", err);
    } else if (strcmp(cmd, "weights") == 0 && argc == 5) {
        int got = 0;
        rc = nmoe_hip_load_model_weights(CTX, argv[2], argv[3], atoi(argv[4]), &got);
    } else if (strcmp(cmd, "layer") == 0 && argc == 4) {
        rc = nmoe_hip_load_layer_file(CTX, 0, atoi(argv[3]), argv[2]);
    } else if (strcmp(cmd, "expdir") == 0 && argc == 4) {
        int bits = 0, got = 0;
        rc = nmoe_hip_load_expert_dir(CTX, argv[2], atoi(argv[3]), &bits, &got);
    } else {
        return 2;
    }
    free_bufs();
    printf("rc=%d\n", rc);
    return 0;
}
