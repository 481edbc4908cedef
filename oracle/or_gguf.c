/* or_gguf.c - oracle GGUF v3 writer and mmap loader (TEST INFRASTRUCTURE).
 *
 * Format (reference src/ornith_gguf_write.c:1-11, 218-474):
 *   "GGUF" u32 version | u64 n_tensors | u64 n_kv
 *   n_kv x { str key | u32 vtype | value }
 *   n_tensors x { str name | u32 n_dims | u64 dims[] | u32 type | u64 offset }
 *   zero pad to the alignment (32, or general.alignment) | tensor data, each
 *   tensor zero-padded to the alignment. str = u64 length + bytes.
 */
#define _POSIX_C_SOURCE 200809L
#include "oracle.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <fcntl.h>
#include <unistd.h>
#include <sys/mman.h>
#include <sys/stat.h>

void orc_seterr(const char *fmt, ...);

enum { VT_U8 = 0, VT_I8, VT_U16, VT_I16, VT_U32, VT_I32, VT_F32, VT_BOOL,
       VT_STR, VT_ARR, VT_U64, VT_I64, VT_F64 };

/* ---- writer --------------------------------------------------------------- */
typedef struct { uint8_t *p; size_t n, cap; } bytes;
static int b_put(bytes *b, const void *src, size_t n) {
    if (b->n + n > b->cap) {
        size_t cap = b->cap ? b->cap : 256;
        while (cap < b->n + n) cap *= 2;
        uint8_t *q = realloc(b->p, cap);
        if (!q) return -1;
        b->p = q; b->cap = cap;
    }
    memcpy(b->p + b->n, src, n); b->n += n; return 0;
}
static int b_u32(bytes *b, uint32_t v) { return b_put(b, &v, 4); }
static int b_u64(bytes *b, uint64_t v) { return b_put(b, &v, 8); }
static int b_str(bytes *b, const char *s) {
    const uint64_t n = strlen(s);
    return b_u64(b, n) || b_put(b, s, n);
}

typedef struct { char *key; uint32_t vt; bytes val; } wkv;
typedef struct { char name[256]; uint32_t nd; uint64_t dims[4]; uint32_t type;
                 const void *data; uint64_t nbytes; } wten;
struct orc_writer { wkv *kv; size_t nkv; wten *t; size_t nt; int bad; };

orc_writer *orc_writer_new(void) { return calloc(1, sizeof(orc_writer)); }
void orc_writer_free(orc_writer *w) {
    if (!w) return;
    for (size_t i = 0; i < w->nkv; i++) { free(w->kv[i].key); free(w->kv[i].val.p); }
    free(w->kv); free(w->t); free(w);
}
static wkv *add_kv(orc_writer *w, const char *key, uint32_t vt) {
    wkv *k = realloc(w->kv, (w->nkv + 1) * sizeof *k);
    if (!k) { w->bad = 1; return NULL; }
    w->kv = k;
    k = &w->kv[w->nkv++];
    memset(k, 0, sizeof *k);
    k->key = strdup(key); k->vt = vt;
    return k;
}
int orc_w_string(orc_writer *w, const char *key, const char *val) {
    wkv *k = add_kv(w, key, VT_STR); return k ? b_str(&k->val, val) : ORC_ERR_OOM;
}
int orc_w_u32(orc_writer *w, const char *key, uint32_t v) {
    wkv *k = add_kv(w, key, VT_U32); return k ? b_u32(&k->val, v) : ORC_ERR_OOM;
}
int orc_w_f32(orc_writer *w, const char *key, float v) {
    wkv *k = add_kv(w, key, VT_F32); return k ? b_put(&k->val, &v, 4) : ORC_ERR_OOM;
}
int orc_w_arr_str(orc_writer *w, const char *key, const char *const *vals, size_t n) {
    wkv *k = add_kv(w, key, VT_ARR);
    if (!k) return ORC_ERR_OOM;
    int e = b_u32(&k->val, VT_STR) || b_u64(&k->val, n);
    for (size_t i = 0; i < n && !e; i++) e = b_str(&k->val, vals[i]);
    return e ? ORC_ERR_OOM : ORC_OK;
}
int orc_w_tensor(orc_writer *w, const char *name, uint32_t nd, const uint64_t *dims,
                 uint32_t type, const void *data, uint64_t nbytes) {
    wten *t = realloc(w->t, (w->nt + 1) * sizeof *t);
    if (!t) return ORC_ERR_OOM;
    w->t = t;
    t = &w->t[w->nt++];
    memset(t, 0, sizeof *t);
    snprintf(t->name, sizeof t->name, "%s", name);
    t->nd = nd; memcpy(t->dims, dims, nd * 8); t->type = type;
    t->data = data; t->nbytes = nbytes;
    return ORC_OK;
}
static uint64_t up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

int orc_writer_write(orc_writer *w, const char *path) {
    bytes h = {0};
    int e = b_put(&h, "GGUF", 4) || b_u32(&h, 3) || b_u64(&h, w->nt) || b_u64(&h, w->nkv);
    for (size_t i = 0; i < w->nkv && !e; i++)
        e = b_str(&h, w->kv[i].key) || b_u32(&h, w->kv[i].vt) ||
            b_put(&h, w->kv[i].val.p, w->kv[i].val.n);
    uint64_t off = 0;
    for (size_t i = 0; i < w->nt && !e; i++) {
        const wten *t = &w->t[i];
        e = b_str(&h, t->name) || b_u32(&h, t->nd);
        for (uint32_t d = 0; d < t->nd && !e; d++) e = b_u64(&h, t->dims[d]);
        e = e || b_u32(&h, t->type) || b_u64(&h, off);
        off = up(off + t->nbytes, 32);
    }
    if (e || w->bad) { free(h.p); orc_seterr("oom building header"); return ORC_ERR_OOM; }
    FILE *f = fopen(path, "wb");
    if (!f) { free(h.p); orc_seterr("cannot open %s", path); return ORC_ERR_IO; }
    static const uint8_t zero[32];
    int ok = fwrite(h.p, 1, h.n, f) == h.n;
    uint64_t pos = h.n;
    free(h.p);
    if (ok && up(pos, 32) > pos) { ok = fwrite(zero, 1, up(pos, 32) - pos, f) == up(pos, 32) - pos; pos = up(pos, 32); }
    for (size_t i = 0; i < w->nt && ok; i++) {
        const wten *t = &w->t[i];
        if (t->nbytes) ok = fwrite(t->data, 1, t->nbytes, f) == t->nbytes;
        pos += t->nbytes;
        const uint64_t pad = up(pos, 32) - pos;
        if (ok && pad) ok = fwrite(zero, 1, pad, f) == pad;
        pos += pad;
    }
    if (fclose(f) != 0) ok = 0;
    if (!ok) { orc_seterr("short write to %s", path); return ORC_ERR_IO; }
    return ORC_OK;
}

/* ---- mmap loader ---------------------------------------------------------- */
typedef struct { char *key; uint32_t vt; const uint8_t *val; size_t len; } lkv;
struct orc_gguf {
    uint8_t *map; size_t size;
    lkv *kv; uint64_t nkv;
    orc_tensor *t; uint64_t nt;
    uint32_t alignment;
};

typedef struct { const uint8_t *p, *end; } cur;
static int c_take(cur *c, void *dst, size_t n) {
    if ((size_t)(c->end - c->p) < n) return -1;
    if (dst) memcpy(dst, c->p, n);
    c->p += n; return 0;
}
static size_t scalar_size(uint32_t vt) {
    switch (vt) {
    case VT_U8: case VT_I8: case VT_BOOL: return 1;
    case VT_U16: case VT_I16: return 2;
    case VT_U32: case VT_I32: case VT_F32: return 4;
    case VT_U64: case VT_I64: case VT_F64: return 8;
    default: return 0;
    }
}
static int skip_value(cur *c, uint32_t vt, int depth) {
    if (vt == VT_STR) { uint64_t n; return c_take(c, &n, 8) || c_take(c, NULL, n); }
    if (vt == VT_ARR) {
        uint32_t et; uint64_t n;
        if (depth > 4 || c_take(c, &et, 4) || c_take(c, &n, 8)) return -1;
        for (uint64_t i = 0; i < n; i++) if (skip_value(c, et, depth + 1)) return -1;
        return 0;
    }
    const size_t s = scalar_size(vt);
    return s ? c_take(c, NULL, s) : -1;
}

void orc_gguf_free(orc_gguf *g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->size);
    for (uint64_t i = 0; i < g->nkv; i++) free(g->kv[i].key);
    free(g->kv); free(g->t); free(g);
}

int orc_gguf_load(const char *path, orc_gguf **out) {
    *out = NULL;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) { orc_seterr("cannot open %s", path); return ORC_ERR_IO; }
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); orc_seterr("fstat %s", path); return ORC_ERR_IO; }
    const size_t size = (size_t)st.st_size;
    uint8_t *map = size ? mmap(NULL, size, PROT_READ, MAP_PRIVATE, fd, 0) : MAP_FAILED;
    close(fd);
    if (map == MAP_FAILED) { orc_seterr("mmap %s failed", path); return ORC_ERR_IO; }
    orc_gguf *g = calloc(1, sizeof *g);
    g->map = map; g->size = size; g->alignment = 32;
    cur c = { map, map + size };
    uint32_t ver; uint64_t nt, nkv;
    if (size < 4 || memcmp(map, "GGUF", 4) != 0) { orc_gguf_free(g); orc_seterr("not a GGUF file (bad magic)"); return ORC_ERR_FORMAT; }
    c.p += 4;
    if (c_take(&c, &ver, 4) || c_take(&c, &nt, 8) || c_take(&c, &nkv, 8)) {
        orc_gguf_free(g); orc_seterr("truncated GGUF header"); return ORC_ERR_FORMAT;
    }
    if (ver < 2 || ver > 3) { orc_gguf_free(g); orc_seterr("unsupported GGUF version %u", ver); return ORC_ERR_UNSUPPORTED; }
    if (nt > (1u << 24) || nkv > (1u << 24)) { orc_gguf_free(g); orc_seterr("implausible counts"); return ORC_ERR_FORMAT; }
    g->kv = calloc(nkv ? nkv : 1, sizeof(lkv));
    g->t = calloc(nt ? nt : 1, sizeof(orc_tensor));
    for (uint64_t i = 0; i < nkv; i++) {
        uint64_t kl;
        if (c_take(&c, &kl, 8) || (size_t)(c.end - c.p) < kl) goto bad;
        lkv *k = &g->kv[g->nkv++];
        k->key = strndup((const char *)c.p, kl); c.p += kl;
        if (c_take(&c, &k->vt, 4)) goto bad;
        k->val = c.p;
        if (skip_value(&c, k->vt, 0)) goto bad;
        k->len = (size_t)(c.p - k->val);
        if (strcmp(k->key, "general.alignment") == 0 && k->vt == VT_U32) {
            uint32_t a; memcpy(&a, k->val, 4);
            if (a) g->alignment = a;
        }
    }
    uint64_t *offs = calloc(nt ? nt : 1, 8);
    for (uint64_t i = 0; i < nt; i++) {
        orc_tensor *t = &g->t[i];
        uint64_t nl;
        if (c_take(&c, &nl, 8) || (size_t)(c.end - c.p) < nl) { free(offs); goto bad; }
        snprintf(t->name, sizeof t->name, "%.*s", (int)(nl < 255 ? nl : 255), (const char *)c.p);
        c.p += nl;
        if (c_take(&c, &t->n_dims, 4) || t->n_dims > 4) { free(offs); goto bad; }
        t->n_elements = 1;
        for (uint32_t d = 0; d < t->n_dims; d++) {
            if (c_take(&c, &t->dims[d], 8)) { free(offs); goto bad; }
            t->n_elements *= t->dims[d];
        }
        if (c_take(&c, &t->type, 4) || c_take(&c, &offs[i], 8)) { free(offs); goto bad; }
    }
    g->nt = nt;
    const uint64_t data0 = up((uint64_t)(c.p - map), g->alignment);
    if (data0 > size) { free(offs); orc_gguf_free(g); orc_seterr("data section starts past EOF"); return ORC_ERR_FORMAT; }
    for (uint64_t i = 0; i < nt; i++) {
        orc_tensor *t = &g->t[i];
        t->nbytes = orc_row_bytes(t->type, t->n_elements);
        if (!t->nbytes && t->n_elements) {
            free(offs); orc_gguf_free(g);
            orc_seterr("tensor '%s': cannot size type %u", t->name, t->type);
            return ORC_ERR_UNSUPPORTED;
        }
        if (offs[i] > size - data0 || t->nbytes > size - data0 - offs[i]) {
            free(offs); orc_gguf_free(g);
            orc_seterr("tensor '%s' data extends past EOF", t->name);
            return ORC_ERR_FORMAT;
        }
        t->data = map + data0 + offs[i];
    }
    free(offs);
    *out = g;
    return ORC_OK;
bad:
    orc_gguf_free(g);
    orc_seterr("malformed GGUF metadata or tensor index");
    return ORC_ERR_FORMAT;
}

uint64_t orc_gguf_n_tensors(const orc_gguf *g) { return g->nt; }
const orc_tensor *orc_gguf_tensor(const orc_gguf *g, uint64_t i) { return i < g->nt ? &g->t[i] : NULL; }
const orc_tensor *orc_gguf_find(const orc_gguf *g, const char *name) {
    for (uint64_t i = 0; i < g->nt; i++) if (strcmp(g->t[i].name, name) == 0) return &g->t[i];
    return NULL;
}

/* metadata lookups used by the model loader (src/ornith_rforward.c:38-70) */
const void *orc_gguf_kv(const orc_gguf *g, const char *key, uint32_t *vt, size_t *len) {
    for (uint64_t i = 0; i < g->nkv; i++)
        if (strcmp(g->kv[i].key, key) == 0) { *vt = g->kv[i].vt; *len = g->kv[i].len; return g->kv[i].val; }
    return NULL;
}
