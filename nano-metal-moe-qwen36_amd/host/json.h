/*
 * json.h -- the small JSON reader of the host code (json.c); not installed.
 */
#ifndef NMOE_HOST_JSON_H
#define NMOE_HOST_JSON_H

#include <stddef.h>

enum { J_NULL, J_BOOL, J_NUM, J_STR, J_ARR, J_OBJ };

typedef struct jv {
    int type;
    double num;
    char *str;           /* J_STR: value; object members: key */
    struct jv *kids;     /* J_ARR / J_OBJ: children (objects: each child's str_key set) */
    char **keys;         /* J_OBJ: member keys, parallel to kids */
    int n;
    int cap;             /* J_ARR / J_OBJ: room in kids (and keys) */
} jv;

void jv_free(jv *v);
/* Parses the whole of text[0..len) into out (0), or -1 on a syntax error. */
int jparse_text(const char *text, size_t len, jv *out);
/* The file's bytes, NUL-terminated (free() them), or NULL. */
char *jread_file(const char *path, size_t *len_out);
/* Member `key` of object o, or NULL. */
const jv *jget(const jv *o, const char *key);
/* A non-negative integral number below 2^53 (0), else -1. */
int jint(const jv *v, unsigned long long *out);

#endif
