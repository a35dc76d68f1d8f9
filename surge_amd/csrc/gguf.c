/* gguf.c - read-only GGUF v3 reader over an mmap of the file.
 *
 * Interface: the reference's sg_gguf_* (reference surge.h:13-46); behaviour
 * follows reference src/gguf.c: v3 only, metadata scalars/strings/arrays,
 * tensor table, data section at the file's general.alignment (default 32,
 * gguf.c:435-441), Q8_0 sized as 34 bytes per 32 elements (gguf.c:153-177).
 * Every length read from the file is bounds-checked against the mapping, so
 * a truncated or corrupt file is an error, never an out-of-bounds read.
 */
#define _GNU_SOURCE
#include "surge.h"

#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

typedef struct {
    char *key;
    sg_gguf_kv_type type;
    const uint8_t *val;          /* points at the value bytes in the mapping */
    sg_gguf_kv_type elem;        /* arrays: element type */
    uint64_t count;              /* arrays: element count */
    char *str;                   /* strings: NUL-terminated copy */
} gkv;

struct sg_gguf {
    uint8_t *base;
    size_t size;
    uint32_t version;
    uint64_t n_kv, n_tensors;
    gkv *kv;
    sg_tensor *tensors;
};

typedef struct { const uint8_t *p, *end; bool ok; } cursor;

static bool need(cursor *c, uint64_t n) {
    if (!c->ok || (uint64_t)(c->end - c->p) < n) { c->ok = false; return false; }
    return true;
}
static uint32_t rd32(cursor *c) { uint32_t v = 0; if (need(c, 4)) { memcpy(&v, c->p, 4); c->p += 4; } return v; }
static uint64_t rd64(cursor *c) { uint64_t v = 0; if (need(c, 8)) { memcpy(&v, c->p, 8); c->p += 8; } return v; }

/* A GGUF string: u64 length then bytes (not NUL-terminated in the file). */
static char *rdstr(cursor *c) {
    uint64_t n = rd64(c);
    if (!need(c, n) || n > (1u << 20)) { c->ok = false; return NULL; }
    char *s = malloc(n + 1);
    if (!s) { c->ok = false; return NULL; }
    memcpy(s, c->p, n);
    s[n] = 0;
    c->p += n;
    return s;
}

static uint64_t scalar_size(sg_gguf_kv_type t) {
    switch (t) {
    case SG_GGUF_U8: case SG_GGUF_I8: case SG_GGUF_BOOL: return 1;
    case SG_GGUF_U16: case SG_GGUF_I16: return 2;
    case SG_GGUF_U32: case SG_GGUF_I32: case SG_GGUF_F32: return 4;
    case SG_GGUF_U64: case SG_GGUF_I64: case SG_GGUF_F64: return 8;
    default: return 0;
    }
}

static bool skip_value(cursor *c, sg_gguf_kv_type t, uint64_t *elem, uint64_t *count) {
    if (t == SG_GGUF_STR) { uint64_t n = rd64(c); if (!need(c, n)) return false; c->p += n; return true; }
    if (t == SG_GGUF_ARR) {
        uint32_t et = rd32(c);
        uint64_t n = rd64(c);
        if (!c->ok || et == SG_GGUF_ARR) return false;
        if (elem) *elem = et;
        if (count) *count = n;
        if (et == SG_GGUF_STR) {
            for (uint64_t i = 0; i < n; i++) {
                uint64_t l = rd64(c);
                if (!need(c, l)) return false;
                c->p += l;
            }
            return true;
        }
        uint64_t es = scalar_size((sg_gguf_kv_type)et);
        if (!es || n > UINT64_MAX / es || !need(c, n * es)) return false;
        c->p += n * es;
        return true;
    }
    uint64_t s = scalar_size(t);
    if (!s || !need(c, s)) return false;
    c->p += s;
    return true;
}

/* Bytes of a tensor of `elems` elements, or 0 for an unsupported type or a
 * Q8_0 count that is not whole blocks. */
static uint64_t tensor_bytes(sg_tensor_type t, uint64_t elems) {
    switch (t) {
    case SG_T_F32: return elems * 4;
    case SG_T_F16: case SG_T_BF16: return elems * 2;
    case SG_T_Q8_0: return (elems % 32) ? 0 : elems / 32 * 34;
    default: return 0;
    }
}

void sg_gguf_close(sg_gguf *g) {
    if (!g) return;
    if (g->kv) for (uint64_t i = 0; i < g->n_kv; i++) { free(g->kv[i].key); free(g->kv[i].str); }
    if (g->tensors) for (uint64_t i = 0; i < g->n_tensors; i++) free((char *)g->tensors[i].name);
    free(g->kv);
    free(g->tensors);
    if (g->base) munmap(g->base, g->size);
    free(g);
}

sg_err sg_gguf_open(const char *path, sg_gguf **out) {
    if (!out) return (sg_err){"gguf: invalid arguments"};
    *out = NULL;
    if (!path) return (sg_err){"gguf: invalid arguments"};
    int fd = open(path, O_RDONLY);
    if (fd < 0) return (sg_err){"gguf: cannot open file"};
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size < 24) { close(fd); return (sg_err){"gguf: file too small"}; }
    void *map = mmap(NULL, (size_t)sb.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return (sg_err){"gguf: mmap failed"};
    sg_gguf *g = calloc(1, sizeof *g);
    if (!g) { munmap(map, (size_t)sb.st_size); return (sg_err){"gguf: out of memory"}; }
    g->base = map;
    g->size = (size_t)sb.st_size;

    cursor c = { g->base, g->base + g->size, true };
    if (memcmp(c.p, "GGUF", 4) != 0) { sg_gguf_close(g); return (sg_err){"gguf: bad magic"}; }
    c.p += 4;
    g->version = rd32(&c);
    if (g->version != 3) { sg_gguf_close(g); return (sg_err){"gguf: only version 3 is supported"}; }
    g->n_tensors = rd64(&c);
    g->n_kv = rd64(&c);
    if (g->n_tensors > (1u << 24) || g->n_kv > (1u << 24)) {
        sg_gguf_close(g);
        return (sg_err){"gguf: implausible tensor or metadata count"};
    }
    g->kv = calloc(g->n_kv ? g->n_kv : 1, sizeof *g->kv);
    g->tensors = calloc(g->n_tensors ? g->n_tensors : 1, sizeof *g->tensors);
    if (!g->kv || !g->tensors) { sg_gguf_close(g); return (sg_err){"gguf: out of memory"}; }

    uint32_t align = 32;
    for (uint64_t i = 0; i < g->n_kv && c.ok; i++) {
        gkv *kv = &g->kv[i];
        kv->key = rdstr(&c);
        kv->type = (sg_gguf_kv_type)rd32(&c);
        kv->val = c.p;
        if (kv->type == SG_GGUF_STR) {
            cursor sc = c;
            kv->str = rdstr(&sc);
        }
        uint64_t elem = 0;
        if (!c.ok || !skip_value(&c, kv->type, &elem, &kv->count)) { c.ok = false; break; }
        kv->elem = (sg_gguf_kv_type)elem;
        if (kv->key && strcmp(kv->key, "general.alignment") == 0 && kv->type == SG_GGUF_U32) {
            memcpy(&align, kv->val, 4);
        }
    }
    if (!c.ok) { sg_gguf_close(g); return (sg_err){"gguf: truncated or corrupt metadata"}; }
    if (align == 0 || (align & (align - 1))) { sg_gguf_close(g); return (sg_err){"gguf: bad alignment"}; }

    uint64_t *offs = calloc(g->n_tensors ? g->n_tensors : 1, sizeof *offs);
    if (!offs) { sg_gguf_close(g); return (sg_err){"gguf: out of memory"}; }
    for (uint64_t i = 0; i < g->n_tensors && c.ok; i++) {
        sg_tensor *t = &g->tensors[i];
        t->name = rdstr(&c);
        t->n_dims = rd32(&c);
        if (t->n_dims == 0 || t->n_dims > 4) { c.ok = false; break; }
        uint64_t elems = 1;
        for (uint32_t d = 0; d < t->n_dims; d++) {
            t->dims[d] = rd64(&c);
            if (t->dims[d] && elems > UINT64_MAX / t->dims[d]) c.ok = false;
            elems *= t->dims[d];
        }
        t->type = (sg_tensor_type)rd32(&c);
        offs[i] = rd64(&c);
        t->nbytes = tensor_bytes(t->type, elems);
        if (!t->nbytes && elems) c.ok = false;
    }
    if (!c.ok) { free(offs); sg_gguf_close(g); return (sg_err){"gguf: truncated or corrupt tensor table"}; }
    uint64_t data0 = (uint64_t)(c.p - g->base);
    data0 = (data0 + align - 1) / align * align;
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        sg_tensor *t = &g->tensors[i];
        if (offs[i] % align || data0 + offs[i] > g->size || t->nbytes > g->size - data0 - offs[i]) {
            free(offs);
            sg_gguf_close(g);
            return (sg_err){"gguf: tensor data lies outside the file"};
        }
        t->data = g->base + data0 + offs[i];
    }
    free(offs);
    *out = g;
    return SG_OK;
}

static const gkv *find(const sg_gguf *g, const char *key) {
    if (!g || !key) return NULL;
    for (uint64_t i = 0; i < g->n_kv; i++)
        if (g->kv[i].key && strcmp(g->kv[i].key, key) == 0) return &g->kv[i];
    return NULL;
}

bool sg_gguf_get_u32(const sg_gguf *g, const char *key, uint32_t *out) {
    const gkv *kv = find(g, key);
    if (!kv || !out) return false;
    if (kv->type == SG_GGUF_U32 || kv->type == SG_GGUF_I32) { memcpy(out, kv->val, 4); return true; }
    if (kv->type == SG_GGUF_U64) {
        uint64_t v; memcpy(&v, kv->val, 8);
        if (v > UINT32_MAX) return false;
        *out = (uint32_t)v;
        return true;
    }
    return false;
}

bool sg_gguf_get_f32(const sg_gguf *g, const char *key, float *out) {
    const gkv *kv = find(g, key);
    if (!kv || !out) return false;
    if (kv->type == SG_GGUF_F32) { memcpy(out, kv->val, 4); return true; }
    if (kv->type == SG_GGUF_F64) { double d; memcpy(&d, kv->val, 8); *out = (float)d; return true; }
    return false;
}

bool sg_gguf_get_str(const sg_gguf *g, const char *key, const char **out) {
    const gkv *kv = find(g, key);
    if (!kv || !out || kv->type != SG_GGUF_STR || !kv->str) return false;
    *out = kv->str;     /* owned by g, valid until sg_gguf_close */
    return true;
}

bool sg_gguf_get_arr(const sg_gguf *g, const char *key, sg_gguf_kv_type *elem_type,
                     const void **data, uint64_t *count) {
    const gkv *kv = find(g, key);
    if (!kv || kv->type != SG_GGUF_ARR) return false;
    if (elem_type) *elem_type = kv->elem;
    if (data) *data = kv->val + 12;      /* past elem type (u32) and count (u64) */
    if (count) *count = kv->count;
    return true;
}

uint32_t sg_gguf_version(const sg_gguf *g) { return g ? g->version : 0; }
uint64_t sg_gguf_kv_count(const sg_gguf *g) { return g ? g->n_kv : 0; }
uint64_t sg_gguf_tensor_count(const sg_gguf *g) { return g ? g->n_tensors : 0; }

const sg_tensor *sg_gguf_tensor(const sg_gguf *g, const char *name) {
    if (!g || !name) return NULL;
    for (uint64_t i = 0; i < g->n_tensors; i++)
        if (g->tensors[i].name && strcmp(g->tensors[i].name, name) == 0) return &g->tensors[i];
    return NULL;
}

const sg_tensor *sg_gguf_tensor_at(const sg_gguf *g, uint64_t i) {
    return (g && i < g->n_tensors) ? &g->tensors[i] : NULL;
}
