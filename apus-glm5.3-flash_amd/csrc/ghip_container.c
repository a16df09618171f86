/*
 * ghip_container.c — the converted-container index, host side (C11).
 *
 * A converted v2 container (the format the reference's expert cache opens,
 * c/gcache.h:832-930; schema tests/m1/README.md:21-55) is a directory with
 * apus.index.json and safetensors shards. The index names, per routed
 * expert, one contiguous slab record {block "layers.<n>", expert, shard,
 * offset (file-absolute), nbytes}; the slab holds the six members in the
 * pinned order gate.w | gate.s | up.w | up.s | down.w | down.s. This file
 * parses the index (a small JSON reader: objects, arrays, strings, numbers,
 * literals) and returns one layer's slab records; the store loads them
 * (apus_ghip_store_load_container, one pread per slab).
 */
#include <errno.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "backend_hip.h"
#include "ghip_internal.h"

/* v is a non-negative integer <= max (JSON numbers are read as doubles) */
static int jn_index(double v, double max) {
    return v >= 0.0 && v <= max && v == (double)(uint64_t)v;
}

/* ---- a small JSON reader --------------------------------------------- */

typedef enum { JN_NULL, JN_BOOL, JN_NUM, JN_STR, JN_ARR, JN_OBJ } JKind;

typedef struct JNode {
    JKind kind;
    double num;
    char *str;                  /* JN_STR value; key of an object member */
    struct JNode *kids;         /* array elements / object members */
    size_t n, cap;
    char *key;
} JNode;

typedef struct {
    const char *p, *end;
    char *err;
    size_t errcap;
    int depth;
} JParser;

static void jn_free(JNode *n) {
    if (!n) return;
    for (size_t i = 0; i < n->n; i++) jn_free(&n->kids[i]);
    free(n->kids);
    free(n->str);
    free(n->key);
    n->kids = NULL;
    n->str = NULL;
    n->key = NULL;
}

static int jp_fail(JParser *jp, const char *what) {
    if (jp->err && jp->errcap && !jp->err[0])
        snprintf(jp->err, jp->errcap, "index json: %s", what);
    return 1;
}

static void jp_ws(JParser *jp) {
    while (jp->p < jp->end && (*jp->p == ' ' || *jp->p == '\t' || *jp->p == '\n'
                               || *jp->p == '\r'))
        jp->p++;
}

static int jp_string(JParser *jp, char **out) {
    if (jp->p >= jp->end || *jp->p != '"') return jp_fail(jp, "string expected");
    jp->p++;
    size_t cap = 16, n = 0;
    char *s = (char *)malloc(cap);
    if (!s) return jp_fail(jp, "out of memory");
    while (jp->p < jp->end && *jp->p != '"') {
        char c = *jp->p++;
        if (c == '\\') {
            if (jp->p >= jp->end) break;
            char e = *jp->p++;
            switch (e) {
            case 'n': c = '\n'; break;
            case 't': c = '\t'; break;
            case 'r': c = '\r'; break;
            case 'b': c = '\b'; break;
            case 'f': c = '\f'; break;
            case 'u': {
                /* \uXXXX: code points below 0x80 kept, others as '?' (the
                 * index keys and shard names used here are ASCII) */
                unsigned v = 0;
                for (int i = 0; i < 4; i++) {
                    if (jp->p >= jp->end) { free(s); return jp_fail(jp, "bad \\u escape"); }
                    char h = *jp->p++;
                    v <<= 4;
                    if (h >= '0' && h <= '9') v |= (unsigned)(h - '0');
                    else if (h >= 'a' && h <= 'f') v |= (unsigned)(h - 'a' + 10);
                    else if (h >= 'A' && h <= 'F') v |= (unsigned)(h - 'A' + 10);
                    else { free(s); return jp_fail(jp, "bad \\u escape"); }
                }
                c = v < 0x80 ? (char)v : '?';
                break;
            }
            default: c = e; break;             /* \" \\ \/ */
            }
        }
        if (n + 1 >= cap) {
            cap *= 2;
            char *t = (char *)realloc(s, cap);
            if (!t) { free(s); return jp_fail(jp, "out of memory"); }
            s = t;
        }
        s[n++] = c;
    }
    if (jp->p >= jp->end) { free(s); return jp_fail(jp, "unterminated string"); }
    jp->p++;
    s[n] = 0;
    *out = s;
    return 0;
}

static int jp_value(JParser *jp, JNode *out);

static int jn_push(JNode *parent, JNode *kid) {
    if (parent->n == parent->cap) {
        size_t nc = parent->cap ? 2 * parent->cap : 8;
        JNode *t = (JNode *)realloc(parent->kids, nc * sizeof(JNode));
        if (!t) return 1;
        parent->kids = t;
        parent->cap = nc;
    }
    parent->kids[parent->n++] = *kid;
    return 0;
}

static int jp_value(JParser *jp, JNode *out) {
    memset(out, 0, sizeof *out);
    jp_ws(jp);
    if (jp->p >= jp->end) return jp_fail(jp, "unexpected end");
    if (++jp->depth > 64) return jp_fail(jp, "nesting too deep");
    char c = *jp->p;
    int rc = 0;
    if (c == '{' || c == '[') {
        const int obj = c == '{';
        out->kind = obj ? JN_OBJ : JN_ARR;
        jp->p++;
        jp_ws(jp);
        if (jp->p < jp->end && *jp->p == (obj ? '}' : ']')) {
            jp->p++;
        } else {
            for (;;) {
                JNode kid;
                char *key = NULL;
                if (obj) {
                    jp_ws(jp);
                    if (jp_string(jp, &key)) { rc = 1; break; }
                    jp_ws(jp);
                    if (jp->p >= jp->end || *jp->p != ':') {
                        free(key);
                        rc = jp_fail(jp, "':' expected");
                        break;
                    }
                    jp->p++;
                }
                if (jp_value(jp, &kid)) { free(key); jn_free(&kid); rc = 1; break; }
                kid.key = key;
                if (jn_push(out, &kid)) { jn_free(&kid); rc = jp_fail(jp, "out of memory"); break; }
                jp_ws(jp);
                if (jp->p < jp->end && *jp->p == ',') { jp->p++; continue; }
                if (jp->p < jp->end && *jp->p == (obj ? '}' : ']')) { jp->p++; break; }
                rc = jp_fail(jp, obj ? "',' or '}' expected" : "',' or ']' expected");
                break;
            }
        }
    } else if (c == '"') {
        out->kind = JN_STR;
        rc = jp_string(jp, &out->str);
    } else if (c == 't' && jp->end - jp->p >= 4 && !strncmp(jp->p, "true", 4)) {
        out->kind = JN_BOOL;
        out->num = 1;
        jp->p += 4;
    } else if (c == 'f' && jp->end - jp->p >= 5 && !strncmp(jp->p, "false", 5)) {
        out->kind = JN_BOOL;
        jp->p += 5;
    } else if (c == 'n' && jp->end - jp->p >= 4 && !strncmp(jp->p, "null", 4)) {
        out->kind = JN_NULL;
        jp->p += 4;
    } else if (c == '-' || (c >= '0' && c <= '9')) {
        /* the buffer is NUL-terminated, so strtod stops inside it */
        char *e = NULL;
        out->kind = JN_NUM;
        out->num = strtod(jp->p, &e);
        if (!e || e == jp->p) rc = jp_fail(jp, "bad number");
        else jp->p = e;
    } else {
        rc = jp_fail(jp, "unexpected character");
    }
    jp->depth--;
    return rc;
}

static const JNode *jn_get(const JNode *obj, const char *key) {
    if (!obj || obj->kind != JN_OBJ) return NULL;
    for (size_t i = 0; i < obj->n; i++)
        if (obj->kids[i].key && !strcmp(obj->kids[i].key, key)) return &obj->kids[i];
    return NULL;
}

/* ---- the index --------------------------------------------------------- */

static void cerr(char *err, size_t errcap, const char *fmt, ...) {
    if (!err || !errcap) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errcap, fmt, ap);
    va_end(ap);
}

int ghip_container_layer(const char *dir, int layer, size_t slab_bytes,
                         GhipSlabRec **out, int *n_out, char *err, size_t errcap) {
    *out = NULL;
    *n_out = 0;
    if (err && errcap) err[0] = 0;
    char path[4096];
    if (!dir || snprintf(path, sizeof path, "%s/apus.index.json", dir) >= (int)sizeof path) {
        cerr(err, errcap, "container: bad directory");
        return 1;
    }
    FILE *f = fopen(path, "rb");
    if (!f) {
        cerr(err, errcap, "container: cannot open %s: %s", path, strerror(errno));
        return 1;
    }
    fseek(f, 0, SEEK_END);
    long len = ftell(f);
    fseek(f, 0, SEEK_SET);
    char *buf = len >= 0 ? (char *)malloc((size_t)len + 1) : NULL;
    if (!buf || fread(buf, 1, (size_t)len, f) != (size_t)len) {
        fclose(f);
        free(buf);
        cerr(err, errcap, "container: cannot read %s", path);
        return 1;
    }
    fclose(f);
    buf[len] = 0;
    JParser jp = { buf, buf + len, err, errcap, 0 };
    JNode root;
    int rc = jp_value(&jp, &root);
    free(buf);
    if (rc) { jn_free(&root); return 1; }
    /* c/gcache.h:868-882: a glm5_next container, format version 2 */
    const JNode *fv = jn_get(&root, "format_version");
    const JNode *mt = jn_get(&root, "model_type");
    const JNode *slabs = jn_get(&root, "expert_slabs");
    if (!fv || fv->kind != JN_NUM || (long)fv->num != 2 || !mt || mt->kind != JN_STR
        || strcmp(mt->str, "glm5_next") || !slabs || slabs->kind != JN_ARR) {
        cerr(err, errcap, "container: apus.index.json is not a glm5_next v2 container");
        jn_free(&root);
        return 1;
    }
    GhipSlabRec *recs = (GhipSlabRec *)calloc(slabs->n ? slabs->n : 1, sizeof *recs);
    int n = 0;
    rc = recs == NULL;
    for (size_t i = 0; i < slabs->n && !rc; i++) {
        const JNode *r = &slabs->kids[i];
        const JNode *blk = jn_get(r, "block"), *ex = jn_get(r, "expert");
        const JNode *sh = jn_get(r, "shard"), *off = jn_get(r, "offset");
        const JNode *nb = jn_get(r, "nbytes");
        int l = -1;
        if (!blk || blk->kind != JN_STR || sscanf(blk->str, "layers.%d", &l) != 1 || !ex
            || ex->kind != JN_NUM || !sh || sh->kind != JN_STR || !off || off->kind != JN_NUM
            || !nb || nb->kind != JN_NUM || !jn_index(ex->num, (double)INT32_MAX)
            || !jn_index(off->num, 9007199254740992.0)
            || !jn_index(nb->num, 9007199254740992.0)) {
            /* the expert id must be an int (c/gcache.h:911-913 parses it as a
             * long and bounds it); offsets and sizes integral and exact in a
             * double */
            cerr(err, errcap, "container: bad slab record %zu", i);
            rc = 1;
            break;
        }
        if (l != layer) continue;
        /* c/gcache.h:912-920: the record must hold exactly one slab */
        if ((uint64_t)nb->num != (uint64_t)slab_bytes) {
            cerr(err, errcap, "container: slab record (layers.%d, %d) holds %llu bytes, "
                 "want %zu", l, (int)ex->num, (unsigned long long)nb->num, slab_bytes);
            rc = 1;
            break;
        }
        if (strlen(sh->str) >= sizeof recs[n].shard || strchr(sh->str, '/')) {
            cerr(err, errcap, "container: bad shard name in record %zu", i);
            rc = 1;
            break;
        }
        recs[n].expert = (int)ex->num;
        strcpy(recs[n].shard, sh->str);
        recs[n].offset = (uint64_t)off->num;
        recs[n].nbytes = (uint64_t)nb->num;
        n++;
    }
    jn_free(&root);
    if (rc) {
        free(recs);
        return 1;
    }
    *out = recs;
    *n_out = n;
    return 0;
}

int apus_ghip_container_slab(const char *dir, int layer, int expert, size_t slab_bytes,
                             char *shard, size_t shard_cap, uint64_t *offset,
                             char *err, size_t errcap) {
    GhipSlabRec *recs = NULL;
    int n = 0;
    if (ghip_container_layer(dir, layer, slab_bytes, &recs, &n, err, errcap)) return 1;
    int rc = 1;
    for (int i = 0; i < n; i++)
        if (recs[i].expert == expert) {
            if (shard && shard_cap) snprintf(shard, shard_cap, "%s", recs[i].shard);
            if (offset) *offset = recs[i].offset;
            rc = 0;
            break;
        }
    if (rc) cerr(err, errcap, "container: no slab record for (layers.%d, %d)", layer, expert);
    free(recs);
    return rc;
}
