/*
 * layout.c -- validation of an expert directory's layout.json, and loading
 * the directory's layer files into HBM (plain C).
 *
 * The converter writes {expert_size, num_layers, num_experts,
 * components[{name, offset, size}]} (scripts/convert_qwen36.py:341-360).
 * The reference's own validator (src/expert_io.m:230-320) expects more keys
 * -- bits/quant and per-component dtype/shape -- and would reject that
 * file; it is never called, and the runtime relies on fixed offsets
 * (src/runtime.m:2240-2252) and the file size (runtime.m:2444-2451).  This
 * validator accepts both schemas: the quantisation comes from bits/quant
 * (2/4, "q2"/"q4", "2"/"4") when present, else from expert_size; when both
 * are present they must agree; dtype, shape and logical_shape are checked
 * when present.  The components must be the nine of the fixed pack layout,
 * in order, with their offsets and sizes.
 */
#include <ctype.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "nmoe_hip.h"

int nmoe_host_fail(nmoe_hip_ctx *ctx, int code, const char *msg);

#include "json.h"

/* ------------------------------------------------------------ the layout */

typedef struct {
    const char *name;
    unsigned long long rows, logical_cols, packed_cols, elem;
} nmoe_component;

/* The nine components of one expert (convert_qwen36.py:38-64; the same table
 * expert_io.m:132-181 builds): weight u32 [rows][cols*bits/32], scales and
 * biases u16 [rows][cols/64], packed back to back. */
static void nmoe_components(int bits, nmoe_component c[9]) {
    const unsigned long long vpw = 32u / (unsigned)bits;
    const char *names[9] = {"gate_proj.weight", "gate_proj.scales", "gate_proj.biases",
                            "up_proj.weight",   "up_proj.scales",   "up_proj.biases",
                            "down_proj.weight", "down_proj.scales", "down_proj.biases"};
    const unsigned long long rows[3] = {512, 512, 2048}, cols[3] = {2048, 2048, 512};
    for (int m = 0; m < 3; m++) {
        c[3 * m] = (nmoe_component){names[3 * m], rows[m], cols[m], cols[m] / vpw, 4};
        c[3 * m + 1] = (nmoe_component){names[3 * m + 1], rows[m], cols[m], cols[m] / 64, 2};
        c[3 * m + 2] = (nmoe_component){names[3 * m + 2], rows[m], cols[m], cols[m] / 64, 2};
    }
}

static int nmoe_quant_bits(const jv *q) {
    if (q == NULL) return 0;
    if (q->type == J_NUM) return q->num == 4.0 ? 4 : q->num == 2.0 ? 2 : -1;
    if (q->type == J_STR) {
        char t[8] = {0};
        for (int i = 0; i < 7 && q->str[i]; i++) t[i] = (char)tolower((unsigned char)q->str[i]);
        if (strcmp(t, "q4") == 0 || strcmp(t, "4") == 0) return 4;
        if (strcmp(t, "q2") == 0 || strcmp(t, "2") == 0) return 2;
    }
    return -1;
}

#define LFAIL(...)                                       \
    do {                                                 \
        if (err != NULL && err_len > 0) snprintf(err, err_len, __VA_ARGS__); \
        rc = NMOE_HIP_EINVAL;                            \
        goto done;                                       \
    } while (0)

int nmoe_hip_validate_layout(const char *path, int *bits_out, int *num_layers_out, char *err, size_t err_len) {
    if (err != NULL && err_len > 0) err[0] = 0;
    if (path == NULL) return NMOE_HIP_EINVAL;
    FILE *f = fopen(path, "rb");
    if (f == NULL) {
        if (err != NULL && err_len > 0) snprintf(err, err_len, "cannot open %s", path);
        return NMOE_HIP_ENOENT;
    }
    char *text = (char *)malloc(1 << 20);
    size_t len = text != NULL ? fread(text, 1, (1 << 20) - 1, f) : 0;
    int toolong = text != NULL && !feof(f);
    fclose(f);
    if (text == NULL) return NMOE_HIP_ENOMEM;
    text[len] = 0; /* strtod stops at the terminator */
    jv root;
    memset(&root, 0, sizeof(root));
    int rc = NMOE_HIP_OK;
    if (toolong) LFAIL("layout file larger than 1 MiB");
    if (jparse_text(text, len, &root) != 0) LFAIL("layout is not valid JSON (or has trailing characters)");
    if (root.type != J_OBJ) LFAIL("layout must be a JSON object");

    const jv *qv = jget(&root, "bits");
    if (qv == NULL) qv = jget(&root, "quant");
    int qbits = nmoe_quant_bits(qv);
    if (qbits < 0) LFAIL("bits/quant must be 2, 4, \"q2\" or \"q4\"");
    unsigned long long esz = 0;
    const jv *ev = jget(&root, "expert_size");
    int sbits = 0;
    if (ev != NULL) {
        if (jint(ev, &esz) != 0) LFAIL("expert_size must be a non-negative integer");
        sbits = esz == NMOE_HIP_EXPERT_SIZE_Q4 ? 4 : esz == NMOE_HIP_EXPERT_SIZE_Q2 ? 2 : -1;
        if (sbits < 0) LFAIL("expert_size %llu is neither %u (q4) nor %u (q2)", esz, NMOE_HIP_EXPERT_SIZE_Q4,
                             NMOE_HIP_EXPERT_SIZE_Q2);
    }
    if (qbits == 0 && sbits == 0) LFAIL("neither bits/quant nor expert_size: cannot tell q4 from q2");
    if (qbits != 0 && sbits != 0 && qbits != sbits) LFAIL("bits/quant (q%d) and expert_size (q%d) disagree", qbits, sbits);
    const int bits = qbits != 0 ? qbits : sbits;

    unsigned long long v;
    const jv *ne = jget(&root, "num_experts");
    if (ne != NULL && (jint(ne, &v) != 0 || v != NMOE_HIP_EXPERTS)) LFAIL("num_experts must be %d", NMOE_HIP_EXPERTS);
    int nl = 0;
    const jv *nlv = jget(&root, "num_layers");
    if (nlv != NULL) {
        if (jint(nlv, &v) != 0 || v < 1 || v > NMOE_HIP_MAX_LAYERS) LFAIL("num_layers must be 1..%d", NMOE_HIP_MAX_LAYERS);
        nl = (int)v;
    }

    const jv *comps = jget(&root, "components");
    if (comps == NULL || comps->type != J_ARR || comps->n != 9) LFAIL("components must be an array of 9 entries");
    nmoe_component want[9];
    nmoe_components(bits, want);
    unsigned long long off = 0;
    for (int i = 0; i < 9; i++) {
        const jv *c = &comps->kids[i];
        const unsigned long long size = want[i].rows * want[i].packed_cols * want[i].elem;
        const jv *nm = jget(c, "name");
        if (c->type != J_OBJ || nm == NULL || nm->type != J_STR) LFAIL("component %d: missing name", i);
        if (strcmp(nm->str, want[i].name) != 0) LFAIL("component %d is %s, expected %s", i, nm->str, want[i].name);
        unsigned long long o2, s2;
        if (jint(jget(c, "offset"), &o2) != 0 || jint(jget(c, "size"), &s2) != 0)
            LFAIL("component %s: offset and size must be integers", want[i].name);
        if (o2 != off || s2 != size)
            LFAIL("component %s: offset/size %llu/%llu, expected %llu/%llu", want[i].name, o2, s2, off, size);
        const jv *dt = jget(c, "dtype");
        if (dt != NULL) {
            const char *wd = want[i].elem == 4 ? "u32" : "u16";
            char t[16] = {0};
            if (dt->type != J_STR) LFAIL("component %s: dtype must be a string", want[i].name);
            for (int j = 0; j < 15 && dt->str[j]; j++) t[j] = (char)tolower((unsigned char)dt->str[j]);
            if (strcmp(t, wd) != 0) LFAIL("component %s: dtype %s, expected %s", want[i].name, dt->str, wd);
        }
        const char *shk[2] = {"shape", "logical_shape"};
        for (int sk = 0; sk < 2; sk++) {
            const jv *sh = jget(c, shk[sk]);
            if (sh == NULL) continue;
            unsigned long long r0, c0;
            const unsigned long long wc = sk == 0 ? want[i].packed_cols : want[i].logical_cols;
            if (sh->type != J_ARR || sh->n != 2 || jint(&sh->kids[0], &r0) != 0 || jint(&sh->kids[1], &c0) != 0)
                LFAIL("component %s: %s must be [rows, cols]", want[i].name, shk[sk]);
            if (r0 != want[i].rows || c0 != wc)
                LFAIL("component %s: %s [%llu, %llu], expected [%llu, %llu]", want[i].name, shk[sk], r0, c0, want[i].rows,
                      wc);
        }
        off += size;
    }
    if (esz != 0 && off != esz) LFAIL("components end at %llu, expert_size is %llu", off, esz);
    if (bits_out != NULL) *bits_out = bits;
    if (num_layers_out != NULL) *num_layers_out = nl;
done:
    jv_free(&root);
    free(text);
    return rc;
}

int nmoe_hip_load_expert_dir(nmoe_hip_ctx *ctx, const char *dir, int nlayers, int *bits_out, int *layers_out) {
    if (ctx == NULL || dir == NULL) return NMOE_HIP_EINVAL;
    char path[4096], err[256];
    if (snprintf(path, sizeof path, "%s/layout.json", dir) >= (int)sizeof path)
        return nmoe_host_fail(ctx, NMOE_HIP_EINVAL, "directory path too long");
    int bits = 0, nl = 0;
    int rc = nmoe_hip_validate_layout(path, &bits, &nl, err, sizeof err);
    if (rc != NMOE_HIP_OK) return nmoe_host_fail(ctx, rc, err[0] ? err : "layout.json rejected");
    const int n = nlayers > 0 ? nlayers : nl;
    if (n < 1 || n > NMOE_HIP_MAX_LAYERS)
        return nmoe_host_fail(ctx, NMOE_HIP_EINVAL, "no layer count: pass nlayers or give num_layers in layout.json");
    if (nl > 0 && n > nl) return nmoe_host_fail(ctx, NMOE_HIP_EINVAL, "nlayers exceeds num_layers of layout.json");
    for (int l = 0; l < n; l++) {
        if (snprintf(path, sizeof path, "%s/layer_%02d.bin", dir, l) >= (int)sizeof path)
            return nmoe_host_fail(ctx, NMOE_HIP_EINVAL, "directory path too long");
        rc = nmoe_hip_load_layer_file(ctx, l, bits, path);
        if (rc != NMOE_HIP_OK) return rc;
        if (layers_out != NULL) *layers_out = l + 1;
    }
    if (bits_out != NULL) *bits_out = bits;
    return NMOE_HIP_OK;
}
