/*
 * weights.c -- the model's non-expert weights that the MoE block needs,
 * from the converter's model_weights.bin + model_weights.json (plain C).
 *
 * The converter writes every non-expert tensor of the model into one file
 * (scripts/convert_qwen36.py:266-327): 2-D ".weight" matrices quantised to
 * q4 as three blobs base.weight (U32 [rows][cols/8]), base.scales and
 * base.biases (BF16 [rows][cols/64]), 1-D tensors as BF16 (A_log as F32),
 * each blob 64-byte aligned, and a manifest {"tensors": {name: {offset,
 * size, shape, dtype}}, "config": {...}}.  The reference maps the file and
 * looks tensors up by name (src/manifest.m:229-316, runtime.m:2271-2299,
 * 2339-2369).  Here the tensors of the MoE path (per layer: the two norms,
 * the q4 router mlp.gate, the shared expert and its gate) are checked and
 * made resident in HBM, one device buffer per layer, and each layer's MoE
 * block descriptor is kept in the context.
 */
#define _POSIX_C_SOURCE 200809L
#include <ctype.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include "json.h"
#include "nmoe_hip.h"

int nmoe_host_fail(nmoe_hip_ctx *ctx, int code, const char *msg);
int nmoe_ctx_set_block(nmoe_hip_ctx *ctx, int layer, const nmoe_hip_moe_block *b);

typedef struct {
    const char *name; /* points into the parsed JSON */
    unsigned long long offset, size;
    char dtype[8];
} wtensor;

typedef struct {
    wtensor *t;
    int n, cap;
} wlist;

static int looks_like_tensor(const jv *o) {
    return o != NULL && o->type == J_OBJ && jget(o, "offset") != NULL && jget(o, "size") != NULL &&
           jget(o, "dtype") != NULL;
}

static int add_tensor(wlist *L, const char *name, const jv *o) {
    unsigned long long off = 0, sz = 0;
    const jv *dt = jget(o, "dtype");
    if (jint(jget(o, "offset"), &off) != 0 || jint(jget(o, "size"), &sz) != 0 || dt->type != J_STR) return 0;
    if (L->n == L->cap) {
        int cap = L->cap ? 2 * L->cap : 64;
        wtensor *t = (wtensor *)realloc(L->t, sizeof(wtensor) * (size_t)cap);
        if (t == NULL) return -1;
        L->t = t;
        L->cap = cap;
    }
    wtensor *w = &L->t[L->n++];
    w->name = name;
    w->offset = off;
    w->size = sz;
    memset(w->dtype, 0, sizeof(w->dtype));
    for (int i = 0; i < 7 && dt->str[i]; i++) w->dtype[i] = (char)toupper((unsigned char)dt->str[i]);
    return 0;
}

/* The manifest shapes the reference accepts (src/manifest.m:113-190): a
 * tensor is an object with offset, size and dtype, named by its key or by a
 * "name" member; "tensors", "entries", "weights" and "weight_map" hold them;
 * other members are searched except metadata, config, model and version. */
static int walk(wlist *L, const char *hint, const jv *node) {
    if (node == NULL) return 0;
    if (node->type == J_OBJ) {
        if (looks_like_tensor(node) && hint != NULL) return add_tensor(L, hint, node);
        const char *holders[3] = {"tensors", "entries", "weights"};
        for (int h = 0; h < 3; h++)
            if (jget(node, holders[h]) != NULL) return walk(L, NULL, jget(node, holders[h]));
        const jv *map = jget(node, "weight_map");
        if (map != NULL && map->type == J_OBJ) {
            for (int i = 0; i < map->n; i++)
                if (walk(L, map->keys[i], &map->kids[i]) != 0) return -1;
            return 0;
        }
        for (int i = 0; i < node->n; i++) {
            const jv *v = &node->kids[i];
            const char *key = node->keys[i];
            if (v->type != J_OBJ && v->type != J_ARR) continue;
            if (looks_like_tensor(v) || (strcmp(key, "metadata") != 0 && strcmp(key, "config") != 0 &&
                                         strcmp(key, "model") != 0 && strcmp(key, "version") != 0))
                if (walk(L, key, v) != 0) return -1;
        }
        return 0;
    }
    if (node->type == J_ARR) {
        for (int i = 0; i < node->n; i++) {
            const jv *it = &node->kids[i];
            if (it->type == J_OBJ) {
                const jv *nm = jget(it, "name");
                const char *name = nm != NULL && nm->type == J_STR ? nm->str : hint;
                if (looks_like_tensor(it) && name != NULL) {
                    if (add_tensor(L, name, it) != 0) return -1;
                } else if (walk(L, name, it) != 0) {
                    return -1;
                }
            } else if (walk(L, hint, it) != 0) {
                return -1;
            }
        }
    }
    return 0;
}

static const wtensor *find(const wlist *L, const char *name) {
    for (int i = 0; i < L->n; i++)
        if (strcmp(L->t[i].name, name) == 0) return &L->t[i];
    return NULL;
}

/* One layer's MoE-path tensors: name suffix, dtype, exact size in bytes. */
typedef struct {
    const char *suffix, *dtype;
    unsigned long long size;
} wneed;

#define NMOE_W_NEEDS 17
static const wneed nmoe_w_needs[NMOE_W_NEEDS] = {
    {".mlp.gate.weight", "U32", 256ull * 256 * 4},
    {".mlp.gate.scales", "BF16", 256ull * 32 * 2},
    {".mlp.gate.biases", "BF16", 256ull * 32 * 2},
    {".mlp.shared_expert.gate_proj.weight", "U32", 512ull * 256 * 4},
    {".mlp.shared_expert.gate_proj.scales", "BF16", 512ull * 32 * 2},
    {".mlp.shared_expert.gate_proj.biases", "BF16", 512ull * 32 * 2},
    {".mlp.shared_expert.up_proj.weight", "U32", 512ull * 256 * 4},
    {".mlp.shared_expert.up_proj.scales", "BF16", 512ull * 32 * 2},
    {".mlp.shared_expert.up_proj.biases", "BF16", 512ull * 32 * 2},
    {".mlp.shared_expert.down_proj.weight", "U32", 2048ull * 64 * 4},
    {".mlp.shared_expert.down_proj.scales", "BF16", 2048ull * 8 * 2},
    {".mlp.shared_expert.down_proj.biases", "BF16", 2048ull * 8 * 2},
    {".mlp.shared_expert_gate.weight", "U32", 256ull * 4},
    {".mlp.shared_expert_gate.scales", "BF16", 32ull * 2},
    {".mlp.shared_expert_gate.biases", "BF16", 32ull * 2},
    {".input_layernorm.weight", "BF16", 2048ull * 2},
    {".post_attention_layernorm.weight", "BF16", 2048ull * 2},
};

#define WFAIL(code, ...)                            \
    do {                                            \
        snprintf(msg, sizeof msg, __VA_ARGS__);     \
        rc = nmoe_host_fail(ctx, (code), msg);      \
        goto done;                                  \
    } while (0)

int nmoe_hip_load_model_weights(nmoe_hip_ctx *ctx, const char *bin_path, const char *json_path, int nlayers,
                                int *layers_out) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (bin_path == NULL || json_path == NULL || nlayers < 0 || nlayers > NMOE_HIP_MAX_LAYERS)
        return nmoe_host_fail(ctx, NMOE_HIP_EINVAL, "bin_path, json_path and nlayers 0..64 are required");
    char msg[512];
    int rc = NMOE_HIP_OK, fd = -1;
    size_t len = 0;
    char *text = jread_file(json_path, &len);
    unsigned char *stage = NULL;
    jv root;
    memset(&root, 0, sizeof(root));
    wlist L = {NULL, 0, 0};
    if (text == NULL) WFAIL(NMOE_HIP_ENOENT, "cannot read %s", json_path);
    if (jparse_text(text, len, &root) != 0) WFAIL(NMOE_HIP_EINVAL, "%s is not valid JSON", json_path);
    if (walk(&L, NULL, &root) != 0) WFAIL(NMOE_HIP_ENOMEM, "manifest too large");
    if (L.n == 0) WFAIL(NMOE_HIP_EINVAL, "%s holds no tensors", json_path);
    const jv *cfg = jget(&root, "config");
    float eps = 1e-6f;
    const jv *ev = jget(cfg, "rms_norm_eps");
    if (ev != NULL && (ev->type != J_NUM || !(ev->num >= 0.0 && ev->num < 1.0)))
        WFAIL(NMOE_HIP_EINVAL, "config.rms_norm_eps must be a number in [0, 1)");
    if (ev != NULL) eps = (float)ev->num;
    unsigned long long cl = 0;
    int n = nlayers;
    if (n == 0 && jint(jget(cfg, "num_hidden_layers"), &cl) == 0) n = (int)cl;
    if (n < 1 || n > NMOE_HIP_MAX_LAYERS) WFAIL(NMOE_HIP_EINVAL, "layer count %d outside 1..64 (pass nlayers)", n);
    fd = open(bin_path, O_RDONLY);
    struct stat st;
    if (fd < 0 || fstat(fd, &st) != 0) WFAIL(NMOE_HIP_ENOENT, "cannot open %s", bin_path);
    /* one layer's buffer: the 17 tensors back to back, each 256-byte aligned */
    size_t offs[NMOE_W_NEEDS], total = 0;
    for (int i = 0; i < NMOE_W_NEEDS; i++) {
        offs[i] = total;
        total += (size_t)((nmoe_w_needs[i].size + 255u) & ~255ull);
    }
    stage = (unsigned char *)calloc(1, total);
    if (stage == NULL) WFAIL(NMOE_HIP_ENOMEM, "host staging buffer");
    void *devs[NMOE_HIP_MAX_LAYERS];
    for (int l = 0; l < n; l++) {
        for (int i = 0; i < NMOE_W_NEEDS; i++) {
            char name[160];
            snprintf(name, sizeof name, "model.layers.%d%s", l, nmoe_w_needs[i].suffix);
            const wtensor *t = find(&L, name);
            /* runtime.m:2278-2297: missing tensor, wrong dtype, out of range */
            if (t == NULL) WFAIL(NMOE_HIP_ENOENT, "missing tensor %s", name);
            if (strcmp(t->dtype, nmoe_w_needs[i].dtype) != 0)
                WFAIL(NMOE_HIP_EINVAL, "tensor %s has dtype %s, expected %s", name, t->dtype, nmoe_w_needs[i].dtype);
            if (t->offset + t->size > (unsigned long long)st.st_size || t->offset + t->size < t->offset)
                WFAIL(NMOE_HIP_EIO, "tensor %s is out of range of %s", name, bin_path);
            if (t->size != nmoe_w_needs[i].size)
                WFAIL(NMOE_HIP_EINVAL, "tensor %s has %llu bytes, expected %llu", name, t->size, nmoe_w_needs[i].size);
            size_t got = 0;
            while (got < t->size) {
                ssize_t r = pread(fd, stage + offs[i] + got, (size_t)t->size - got, (off_t)(t->offset + got));
                if (r <= 0) WFAIL(NMOE_HIP_EIO, "read of %s failed", name);
                got += (size_t)r;
            }
        }
        char label[48];
        snprintf(label, sizeof label, "nmoe.model.layer.%d", l);
        void *dev = nmoe_hip_lookup_buffer(ctx, label);
        if (dev != NULL) {
            rc = nmoe_hip_copy_to_device(ctx, dev, stage, total);
        } else {
            rc = nmoe_hip_register_shared_buffer(ctx, label, stage, total, &dev);
        }
        if (rc != NMOE_HIP_OK) goto done;
        devs[l] = dev;
    }
    for (int l = 0; l < n; l++) {
        const unsigned char *d = (const unsigned char *)devs[l];
#define P(i) ((const void *)(d + offs[i]))
        nmoe_hip_moe_block b;
        memset(&b, 0, sizeof(b));
        b.router.kind = NMOE_HIP_ROUTER_Q4;
        b.router.num_experts = NMOE_HIP_EXPERTS;
        b.router.w_q4 = (const uint32_t *)P(0);
        b.router.scales = (const uint16_t *)P(1);
        b.router.biases = (const uint16_t *)P(2);
        b.has_shared = 1;
        nmoe_hip_qtensor *q[4] = {&b.shared.gate, &b.shared.up, &b.shared.down, &b.shared.score};
        for (int m = 0; m < 4; m++) {
            q[m]->w = (const uint32_t *)P(3 + 3 * m);
            q[m]->scales = (const uint16_t *)P(4 + 3 * m);
            q[m]->biases = (const uint16_t *)P(5 + 3 * m);
        }
        b.post_norm = (const uint16_t *)P(16);
        /* the next layer's input norm follows the combine (runtime.m:2893-2900) */
        b.next_norm = l + 1 < n ? (const uint16_t *)((const unsigned char *)devs[l + 1] + offs[15]) : NULL;
        b.add_one = 1; /* runtime.m:3149, 2898 */
        b.eps = eps;
#undef P
        rc = nmoe_ctx_set_block(ctx, l, &b);
        if (rc != NMOE_HIP_OK) goto done;
    }
    if (layers_out != NULL) *layers_out = n;
done:
    if (fd >= 0) close(fd);
    free(stage);
    free(L.t);
    jv_free(&root);
    free(text);
    return rc;
}
