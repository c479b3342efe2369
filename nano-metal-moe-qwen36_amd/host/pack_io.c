/*
 * pack_io.c -- host side of expert-pack residency (plain C).
 *
 * The reference maps packed_experts/layer_XX.bin (src/runtime.m:2426-2465,
 * NMOELoadExpertLayer: open, fstat, reject files shorter than 256 experts,
 * mmap MAP_PRIVATE) and preads the K selected experts per token into fixed
 * I/O buffers (runtime.m:1588-1634).  Here the file is read once and copied
 * to HBM, where it stays: the byte layout (convert_qwen36.py:38-64,
 * 341-413) is uploaded unchanged, with no transcoding.
 */
#define _FILE_OFFSET_BITS 64
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include "nmoe_hip.h"

int nmoe_host_fail(nmoe_hip_ctx *ctx, int code, const char *msg);

static int nmoe_read_fully(int fd, unsigned char *dst, size_t size) {
    size_t done = 0;
    while (done < size) {
        ssize_t got = pread(fd, dst + done, size - done, (off_t)done);
        if (got < 0) {
            if (errno == EINTR) continue;
            return -1;
        }
        if (got == 0) return -1; /* unexpected EOF (expert_io.m:74-79) */
        done += (size_t)got;
    }
    return 0;
}

int nmoe_hip_load_layer_file(nmoe_hip_ctx *ctx, int layer, int bits, const char *path) {
    if (ctx == NULL || path == NULL) return NMOE_HIP_EINVAL;
    size_t esz = nmoe_hip_expert_size(bits);
    if (esz == 0) return nmoe_host_fail(ctx, NMOE_HIP_EINVAL, "bits must be 4 or 2");
    size_t want = (size_t)NMOE_HIP_EXPERTS * esz;
    int fd = open(path, O_RDONLY);
    if (fd < 0) return nmoe_host_fail(ctx, NMOE_HIP_ENOENT, "cannot open layer file");
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return nmoe_host_fail(ctx, NMOE_HIP_EIO, "fstat failed on layer file");
    }
    /* runtime.m:2444-2451: a layer file must hold all 256 experts */
    if ((size_t)st.st_size < want) {
        close(fd);
        return nmoe_host_fail(ctx, NMOE_HIP_EIO, "layer file has the wrong size (shorter than 256 experts)");
    }
    unsigned char *buf = (unsigned char *)malloc(want);
    if (buf == NULL) {
        close(fd);
        return nmoe_host_fail(ctx, NMOE_HIP_ENOMEM, "host staging buffer allocation failed");
    }
    int rc = nmoe_read_fully(fd, buf, want);
    close(fd);
    if (rc != 0) {
        free(buf);
        return nmoe_host_fail(ctx, NMOE_HIP_EIO, "read of layer file failed");
    }
    rc = nmoe_hip_upload_layer_pack(ctx, layer, bits, buf, want);
    free(buf);
    return rc;
}
