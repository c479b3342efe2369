/*
 * json.c -- a small JSON reader for the converter's metadata files
 * (layout.json, model_weights.json): numbers, strings, arrays, objects,
 * true/false/null; nesting up to 32 levels; \\uXXXX escapes become '?'
 * (the files are ASCII); numbers must be finite doubles.  Plain C.
 */
#include <ctype.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "json.h"


typedef struct {
    const char *p, *end;
    int depth;
} jparser;

void jv_free(jv *v) {
    if (v == NULL) return;
    free(v->str);
    for (int i = 0; i < v->n; i++) {
        jv_free(&v->kids[i]);
        if (v->keys != NULL) free(v->keys[i]);
    }
    free(v->kids);
    free(v->keys);
}

static void jskip(jparser *ps) {
    while (ps->p < ps->end && isspace((unsigned char)*ps->p)) ps->p++;
}

static int jparse(jparser *ps, jv *out);

static int jstring(jparser *ps, char **out) {
    if (ps->p >= ps->end || *ps->p != '"') return -1;
    ps->p++;
    size_t cap = 16, len = 0;
    char *s = (char *)malloc(cap);
    if (s == NULL) return -1;
    while (ps->p < ps->end && *ps->p != '"') {
        char c = *ps->p++;
        if (c == '\\') {
            if (ps->p >= ps->end) break;
            char e = *ps->p++;
            c = e == 'n' ? '\n' : e == 't' ? '\t' : e == 'r' ? '\r' : e == 'b' ? '\b' : e == 'f' ? '\f' : e;
            if (e == 'u') { /* the layout uses ASCII only: keep \uXXXX as '?' */
                if (ps->end - ps->p < 4) break;
                ps->p += 4;
                c = '?';
            }
        }
        if (len + 2 > cap) {
            char *t = (char *)realloc(s, cap *= 2);
            if (t == NULL) {
                free(s);
                return -1;
            }
            s = t;
        }
        s[len++] = c;
    }
    if (ps->p >= ps->end) {
        free(s);
        return -1;
    }
    ps->p++; /* closing quote */
    s[len] = 0;
    *out = s;
    return 0;
}

/* Appends a member, the room doubling as it fills (a member at a time
 * would copy the array once per member: quadratic in its length). */
static int jpush(jv *v, jv *kid, char *key) {
    if (v->n == v->cap) {
        if (v->cap > (1 << 26)) return -1;
        const int cap = v->cap ? 2 * v->cap : 8;
        jv *k2 = (jv *)realloc(v->kids, sizeof(jv) * (size_t)cap);
        if (k2 == NULL) return -1;
        v->kids = k2;
        if (v->type == J_OBJ) {
            char **kk = (char **)realloc(v->keys, sizeof(char *) * (size_t)cap);
            if (kk == NULL) return -1;
            v->keys = kk;
        }
        v->cap = cap;
    }
    if (v->type == J_OBJ) v->keys[v->n] = key;
    v->kids[v->n++] = *kid;
    return 0;
}

static int jparse(jparser *ps, jv *out) {
    memset(out, 0, sizeof(*out));
    if (++ps->depth > 32) return -1;
    jskip(ps);
    if (ps->p >= ps->end) return -1;
    char c = *ps->p;
    int rc = 0;
    if (c == '{' || c == '[') {
        out->type = c == '{' ? J_OBJ : J_ARR;
        ps->p++;
        jskip(ps);
        if (ps->p < ps->end && *ps->p == (c == '{' ? '}' : ']')) {
            ps->p++;
        } else {
            for (;;) {
                char *key = NULL;
                jskip(ps);
                if (out->type == J_OBJ) {
                    if (jstring(ps, &key) != 0) return -1;
                    jskip(ps);
                    if (ps->p >= ps->end || *ps->p != ':') {
                        free(key);
                        return -1;
                    }
                    ps->p++;
                }
                jv kid;
                if (jparse(ps, &kid) != 0 || jpush(out, &kid, key) != 0) {
                    jv_free(&kid);
                    free(key);
                    return -1;
                }
                jskip(ps);
                if (ps->p < ps->end && *ps->p == ',') {
                    ps->p++;
                    continue;
                }
                if (ps->p < ps->end && *ps->p == (out->type == J_OBJ ? '}' : ']')) {
                    ps->p++;
                    break;
                }
                return -1;
            }
        }
    } else if (c == '"') {
        out->type = J_STR;
        rc = jstring(ps, &out->str);
    } else if (c == '-' || isdigit((unsigned char)c)) {
        /* a JSON number: the token (sign, digits, '.', exponent) copied out,
         * so that strtod never reads past the text (which need not be
         * NUL-terminated) and never sees the nan / inf / hex forms it would
         * also accept; a value beyond double range is an error */
        char tok[64];
        size_t tl = 0;
        while (ps->p + tl < ps->end && tl < sizeof tok - 1 &&
               (isdigit((unsigned char)ps->p[tl]) || ps->p[tl] == '-' || ps->p[tl] == '+' || ps->p[tl] == '.' ||
                ps->p[tl] == 'e' || ps->p[tl] == 'E'))
            tl++;
        if (tl == sizeof tok - 1) return -1;
        memcpy(tok, ps->p, tl);
        tok[tl] = 0;
        char *e = NULL;
        out->type = J_NUM;
        out->num = strtod(tok, &e);
        if (e == tok || !isfinite(out->num)) return -1;
        ps->p += e - tok;
    } else if (ps->end - ps->p >= 4 && strncmp(ps->p, "true", 4) == 0) {
        out->type = J_BOOL, out->num = 1, ps->p += 4;
    } else if (ps->end - ps->p >= 5 && strncmp(ps->p, "false", 5) == 0) {
        out->type = J_BOOL, ps->p += 5;
    } else if (ps->end - ps->p >= 4 && strncmp(ps->p, "null", 4) == 0) {
        out->type = J_NULL, ps->p += 4;
    } else {
        return -1;
    }
    ps->depth--;
    return rc;
}

const jv *jget(const jv *o, const char *key) {
    if (o == NULL || o->type != J_OBJ) return NULL;
    for (int i = 0; i < o->n; i++)
        if (strcmp(o->keys[i], key) == 0) return &o->kids[i];
    return NULL;
}

int jint(const jv *v, unsigned long long *out) {
    /* the range test first (it also rejects NaN), so that the cast below is
     * defined */
    if (v == NULL || v->type != J_NUM || !(v->num >= 0.0 && v->num <= 9.0e15) ||
        v->num != (double)(unsigned long long)v->num)
        return -1;
    *out = (unsigned long long)v->num;
    return 0;
}


int jparse_text(const char *text, size_t len, jv *out) {
    jparser ps = {text, text + len, 0};
    if (jparse(&ps, out) != 0) {
        jv_free(out);
        memset(out, 0, sizeof(*out));
        return -1;
    }
    jskip(&ps);
    if (ps.p != ps.end) {
        jv_free(out);
        memset(out, 0, sizeof(*out));
        return -1;
    }
    return 0;
}

char *jread_file(const char *path, size_t *len_out) {
    FILE *f = fopen(path, "rb");
    if (f == NULL) return NULL;
    char *buf = NULL;
    long n = -1;
    if (fseek(f, 0, SEEK_END) == 0 && (n = ftell(f)) >= 0 && fseek(f, 0, SEEK_SET) == 0) {
        buf = (char *)malloc((size_t)n + 1);
        if (buf != NULL && fread(buf, 1, (size_t)n, f) != (size_t)n) {
            free(buf);
            buf = NULL;
        }
    }
    fclose(f);
    if (buf != NULL) {
        buf[n] = 0;
        *len_out = (size_t)n;
    }
    return buf;
}
