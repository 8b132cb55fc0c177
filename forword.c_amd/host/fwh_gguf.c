/*
 * GGUF v2/v3 reader over a file mmap or an in-memory image.
 *
 * Follows the container rules the reference enforces in gguf_open
 * (gguf.c:256-353): magic "GGUF", version 2..3, at most 10M tensors/keys,
 * n_dims 1..4, element-count overflow checks, per-type byte sizes with whole
 * blocks per row (gguf.c:187-253), `general.alignment` (power of two <= 4096,
 * default 32, gguf.c:289-292), data section at the aligned end of the
 * descriptors, and every tensor's bytes inside the file (gguf.c:343-351).
 * Metadata values are kept as pointers into the image and decoded on demand.
 */
#define _POSIX_C_SOURCE 200809L
#include "fw_host.h"

#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#define GGUF_MAGIC_LE 0x46554747u
#define GGUF_MAX_ITEMS 10000000u
#define GGUF_MAX_STR (64u * 1024u * 1024u)

enum { VT_U8 = 0, VT_I8, VT_U16, VT_I16, VT_U32, VT_I32, VT_F32, VT_BOOL, VT_STR, VT_ARR,
       VT_U64, VT_I64, VT_F64 };

typedef struct {
    const char *key;
    uint64_t    key_len;
    uint32_t    type;
    const uint8_t *val;     /* start of the value in the image */
} kv_t;

struct fwh_gguf {
    const uint8_t *base;
    size_t         size;
    void          *map;      /* non-NULL when we own an mmap */
    int            fd;
    uint32_t       version;
    uint32_t       alignment;
    uint64_t       data_offset;
    kv_t          *kvs;
    size_t         n_kvs;
    forword_gpu_tensor_t *tensors;
    char         **names;    /* owned copies of tensor names */
    size_t         n_tensors;
};

typedef struct { const uint8_t *p, *end; } rd_t;

static void seterr(char *buf, size_t cap, const char *fmt, ...)
{
    if (!buf || !cap) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, cap, fmt, ap);
    va_end(ap);
}

static int rd_take(rd_t *r, void *out, size_t n)
{
    if ((size_t)(r->end - r->p) < n) return -1;
    if (out) memcpy(out, r->p, n);
    r->p += n;
    return 0;
}
static int rd_u32(rd_t *r, uint32_t *v) { return rd_take(r, v, 4); }
static int rd_u64(rd_t *r, uint64_t *v) { return rd_take(r, v, 8); }

static int rd_str(rd_t *r, const char **s, uint64_t *len)
{
    uint64_t n;
    if (rd_u64(r, &n) || n > GGUF_MAX_STR || n > (uint64_t)(r->end - r->p)) return -1;
    if (s) *s = (const char *)r->p;
    if (len) *len = n;
    r->p += n;
    return 0;
}

static size_t scalar_size(uint32_t t)
{
    switch (t) {
    case VT_U8: case VT_I8: case VT_BOOL: return 1;
    case VT_U16: case VT_I16: return 2;
    case VT_U32: case VT_I32: case VT_F32: return 4;
    case VT_U64: case VT_I64: case VT_F64: return 8;
    default: return 0;
    }
}

static int rd_skip(rd_t *r, uint32_t type, unsigned depth)
{
    if (depth > 8) return -1;
    if (type == VT_STR) return rd_str(r, NULL, NULL);
    if (type == VT_ARR) {
        uint32_t et; uint64_t cnt;
        if (rd_u32(r, &et) || rd_u64(r, &cnt) || cnt > GGUF_MAX_ITEMS) return -1;
        size_t es = scalar_size(et);
        if (es) {                                  /* fixed-size elements: one jump */
            if (cnt > (uint64_t)(r->end - r->p) / es) return -1;
            r->p += cnt * es;
            return 0;
        }
        for (uint64_t i = 0; i < cnt; i++)
            if (rd_skip(r, et, depth + 1)) return -1;
        return 0;
    }
    size_t n = scalar_size(type);
    if (!n) return -1;
    return rd_take(r, NULL, n);
}

/* Byte size of a tensor (gguf.c:187-253): 0 ok, 1 unknown type, -1 invalid. */
static int tensor_bytes(uint32_t type, uint32_t n_dims, const uint64_t *dims, uint64_t elems,
                        uint64_t *bytes)
{
    uint64_t bs = 1, bb = 0;
    *bytes = 0;
    switch (type) {
    case 0: bb = 4; break;  case 1: bb = 2; break;  case 24: bb = 1; break;
    case 25: bb = 2; break; case 26: bb = 4; break; case 27: bb = 8; break;
    case 28: bb = 8; break; case 30: bb = 2; break;
    case 2: bs = 32; bb = 18; break;  case 3: bs = 32; bb = 20; break;
    case 6: bs = 32; bb = 22; break;  case 7: bs = 32; bb = 24; break;
    case 8: bs = 32; bb = 34; break;  case 9: bs = 32; bb = 40; break;
    case 10: bs = 256; bb = 84; break;  case 11: bs = 256; bb = 110; break;
    case 12: bs = 256; bb = 144; break; case 13: bs = 256; bb = 176; break;
    case 14: bs = 256; bb = 210; break; case 15: bs = 256; bb = 292; break;
    default: return 1;
    }
    if (n_dims == 0) return -1;
    if (elems == 0) return 0;
    if (dims[0] % bs || elems % bs) return -1;
    uint64_t blocks = elems / bs;
    if (blocks > UINT64_MAX / bb) return -1;
    *bytes = blocks * bb;
    return 0;
}

static fwh_gguf_t *parse(fwh_gguf_t *g, char *errbuf, size_t errcap)
{
    rd_t r = { g->base, g->base + g->size };
    uint32_t magic;
    uint64_t n_tensors, n_kv;
    if (rd_u32(&r, &magic) || magic != GGUF_MAGIC_LE || rd_u32(&r, &g->version) ||
        rd_u64(&r, &n_tensors) || rd_u64(&r, &n_kv)) {
        seterr(errbuf, errcap, "not a valid GGUF header");
        return NULL;
    }
    if (g->version < 2 || g->version > 3 || n_tensors > GGUF_MAX_ITEMS || n_kv > GGUF_MAX_ITEMS) {
        seterr(errbuf, errcap, "unsupported GGUF version/counts");
        return NULL;
    }
    g->alignment = 32;
    g->kvs = (kv_t *)calloc(n_kv ? n_kv : 1, sizeof(kv_t));
    g->tensors = (forword_gpu_tensor_t *)calloc(n_tensors ? n_tensors : 1, sizeof(forword_gpu_tensor_t));
    g->names = (char **)calloc(n_tensors ? n_tensors : 1, sizeof(char *));
    if (!g->kvs || !g->tensors || !g->names) { seterr(errbuf, errcap, "out of memory"); return NULL; }

    for (uint64_t i = 0; i < n_kv; i++) {
        kv_t *kv = &g->kvs[g->n_kvs];
        if (rd_str(&r, &kv->key, &kv->key_len) || rd_u32(&r, &kv->type)) {
            seterr(errbuf, errcap, "malformed metadata entry %llu", (unsigned long long)i);
            return NULL;
        }
        kv->val = r.p;
        if (rd_skip(&r, kv->type, 0)) {
            seterr(errbuf, errcap, "malformed metadata entry %llu", (unsigned long long)i);
            return NULL;
        }
        g->n_kvs++;
        if (kv->key_len == 17 && !memcmp(kv->key, "general.alignment", 17)) {
            uint64_t a = 0;
            if (kv->type == VT_U32 || kv->type == VT_I32) { uint32_t v; memcpy(&v, kv->val, 4); a = v; }
            else if (kv->type == VT_U64 || kv->type == VT_I64) memcpy(&a, kv->val, 8);
            else if (kv->type == VT_U16) { uint16_t v; memcpy(&v, kv->val, 2); a = v; }
            else if (kv->type == VT_U8) a = kv->val[0];
            if (a > 0 && a <= 4096 && (a & (a - 1)) == 0) g->alignment = (uint32_t)a;
        }
    }

    for (uint64_t i = 0; i < n_tensors; i++) {
        forword_gpu_tensor_t *t = &g->tensors[g->n_tensors];
        const char *nm; uint64_t nl;
        if (rd_str(&r, &nm, &nl) || rd_u32(&r, &t->n_dims) || t->n_dims == 0 || t->n_dims > 4) {
            seterr(errbuf, errcap, "malformed tensor descriptor %llu", (unsigned long long)i);
            return NULL;
        }
        char *copy = (char *)malloc(nl + 1);
        if (!copy) { seterr(errbuf, errcap, "out of memory"); return NULL; }
        memcpy(copy, nm, nl);
        copy[nl] = '\0';
        g->names[g->n_tensors] = copy;
        t->name = copy;
        uint64_t elems = 1;
        for (uint32_t d = 0; d < t->n_dims; d++) {
            if (rd_u64(&r, &t->dims[d]) || (t->dims[d] && elems > UINT64_MAX / t->dims[d])) {
                seterr(errbuf, errcap, "invalid tensor dimensions");
                g->n_tensors++;
                return NULL;
            }
            elems *= t->dims[d];
        }
        for (uint32_t d = t->n_dims; d < 4; d++) t->dims[d] = 1;
        if (rd_u32(&r, &t->ggml_type) || rd_u64(&r, &t->offset)) {
            seterr(errbuf, errcap, "truncated tensor descriptor");
            g->n_tensors++;
            return NULL;
        }
        if (tensor_bytes(t->ggml_type, t->n_dims, t->dims, elems, &t->byte_size) < 0) {
            seterr(errbuf, errcap, "invalid dimensions for tensor '%s'", copy);
            g->n_tensors++;
            return NULL;
        }
        g->n_tensors++;
    }

    uint64_t after = (uint64_t)(r.p - g->base);
    uint64_t aligned = (after + g->alignment - 1) & ~((uint64_t)g->alignment - 1);
    if (aligned > g->size) { seterr(errbuf, errcap, "tensor data offset outside file"); return NULL; }
    g->data_offset = aligned;
    for (size_t i = 0; i < g->n_tensors; i++) {
        const forword_gpu_tensor_t *t = &g->tensors[i];
        if (t->offset > g->size - g->data_offset) {
            seterr(errbuf, errcap, "tensor '%s' offset outside file", t->name);
            return NULL;
        }
        if (t->byte_size > g->size - g->data_offset - t->offset) {
            seterr(errbuf, errcap, "tensor '%s' extends beyond file", t->name);
            return NULL;
        }
    }
    return g;
}

fwh_gguf_t *fwh_gguf_open_memory(const void *image, size_t size, char *errbuf, size_t errcap)
{
    if (!image || size < 24) { seterr(errbuf, errcap, "invalid or too-small image"); return NULL; }
    fwh_gguf_t *g = (fwh_gguf_t *)calloc(1, sizeof(*g));
    if (!g) { seterr(errbuf, errcap, "out of memory"); return NULL; }
    g->fd = -1;
    g->base = (const uint8_t *)image;
    g->size = size;
    if (!parse(g, errbuf, errcap)) { fwh_gguf_close(g); return NULL; }
    return g;
}

fwh_gguf_t *fwh_gguf_open(const char *path, char *errbuf, size_t errcap)
{
    fwh_gguf_t *g = (fwh_gguf_t *)calloc(1, sizeof(*g));
    if (!g) { seterr(errbuf, errcap, "out of memory"); return NULL; }
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) {
        seterr(errbuf, errcap, "open %s: %s", path, strerror(errno));
        free(g);
        return NULL;
    }
    struct stat st;
    if (fstat(g->fd, &st) || st.st_size < 24) {
        seterr(errbuf, errcap, "invalid or too-small file");
        fwh_gguf_close(g);
        return NULL;
    }
    g->size = (size_t)st.st_size;
    g->map = mmap(NULL, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (g->map == MAP_FAILED) {
        g->map = NULL;
        seterr(errbuf, errcap, "mmap: %s", strerror(errno));
        fwh_gguf_close(g);
        return NULL;
    }
    g->base = (const uint8_t *)g->map;
    if (!parse(g, errbuf, errcap)) { fwh_gguf_close(g); return NULL; }
    return g;
}

void fwh_gguf_close(fwh_gguf_t *g)
{
    if (!g) return;
    for (size_t i = 0; i < g->n_tensors; i++) free(g->names[i]);
    free(g->names);
    free(g->tensors);
    free(g->kvs);
    if (g->map) munmap(g->map, g->size);
    if (g->fd >= 0) close(g->fd);
    free(g);
}

uint32_t fwh_gguf_version(const fwh_gguf_t *g) { return g ? g->version : 0; }
uint32_t fwh_gguf_alignment(const fwh_gguf_t *g) { return g ? g->alignment : 0; }
uint64_t fwh_gguf_data_offset(const fwh_gguf_t *g) { return g ? g->data_offset : 0; }
size_t fwh_gguf_n_tensors(const fwh_gguf_t *g) { return g ? g->n_tensors : 0; }
const forword_gpu_tensor_t *fwh_gguf_tensors(const fwh_gguf_t *g) { return g ? g->tensors : NULL; }

const void *fwh_gguf_data(const fwh_gguf_t *g, size_t *size_out)
{
    if (size_out) *size_out = g ? g->size - g->data_offset : 0;
    return g ? g->base + g->data_offset : NULL;
}

long fwh_gguf_find_tensor(const fwh_gguf_t *g, const char *name)
{
    if (!g || !name) return -1;
    for (size_t i = 0; i < g->n_tensors; i++)
        if (!strcmp(g->tensors[i].name, name)) return (long)i;
    return -1;
}

static const kv_t *find_kv(const fwh_gguf_t *g, const char *key)
{
    if (!g || !key) return NULL;
    size_t kl = strlen(key);
    for (size_t i = 0; i < g->n_kvs; i++)
        if (g->kvs[i].key_len == kl && !memcmp(g->kvs[i].key, key, kl)) return &g->kvs[i];
    return NULL;
}

int fwh_gguf_kv_type(const fwh_gguf_t *g, const char *key)
{
    const kv_t *kv = find_kv(g, key);
    return kv ? (int)kv->type : -1;
}

int fwh_gguf_get_u32(const fwh_gguf_t *g, const char *key, uint32_t *out)
{
    const kv_t *kv = find_kv(g, key);
    if (!kv || (kv->type != VT_U32 && kv->type != VT_I32)) return -1;
    memcpy(out, kv->val, 4);
    return 0;
}

int fwh_gguf_get_f32(const fwh_gguf_t *g, const char *key, float *out)
{
    const kv_t *kv = find_kv(g, key);
    if (!kv || kv->type != VT_F32) return -1;
    memcpy(out, kv->val, 4);
    return 0;
}

int fwh_gguf_get_str(const fwh_gguf_t *g, const char *key, char *buf, size_t cap)
{
    const kv_t *kv = find_kv(g, key);
    if (!kv || kv->type != VT_STR || !buf || !cap) return -1;
    uint64_t n;
    memcpy(&n, kv->val, 8);
    size_t c = n < cap - 1 ? (size_t)n : cap - 1;
    memcpy(buf, kv->val + 8, c);
    buf[c] = '\0';
    return 0;
}

int64_t fwh_gguf_array_len(const fwh_gguf_t *g, const char *key)
{
    const kv_t *kv = find_kv(g, key);
    if (!kv || kv->type != VT_ARR) return -1;
    uint64_t n;
    memcpy(&n, kv->val + 4, 8);
    return (int64_t)n;
}
