/*
 * gguf_write.c -- a GGUF v3 writer for synthetic models.
 *
 * The reference ships a GGUF v3 reader only (slm/gguf.c:172-261); this
 * writes files it reads: the header (magic "GGUF", version 3, tensor and
 * key counts), the key/value section, the tensor-info section, padding
 * to `general.alignment` (32 unless a u32 key overrides it,
 * slm/gguf.c:173,219-227), then every tensor's bytes at its recorded
 * offset from the aligned data start, each offset itself a multiple of
 * the alignment. Integers are little-endian; strings are a u64 length
 * and the bytes, no terminator (slm/gguf.c:122-128).
 *
 * Usage: gw_init(); gw_kv_*(...) and gw_tensor(...) in any order (keys
 * and tensors keep their call order); gw_write(path); gw_free().
 * Tensor data is borrowed until gw_write returns.
 */
#ifndef GGUF_WRITE_C
#define GGUF_WRITE_C

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum {
    GW_U32 = 4, GW_I32 = 5, GW_F32 = 6, GW_STR = 8, GW_ARRAY = 9
};

struct gw_buf {
    uint8_t *p;
    size_t n, cap;
};

struct gw_tensor {
    char name[96];
    uint32_t n_dims;
    uint64_t shape[4];
    uint32_t type;
    const void *data;
    uint64_t bytes;
    uint64_t offset;
};

struct gw {
    struct gw_buf kv;          /* encoded key/value pairs */
    uint64_t n_kv;
    struct gw_tensor *t;
    uint64_t n_t, cap_t;
    uint32_t alignment;
};

static void gw_put(struct gw_buf *b, const void *src, size_t n) {
    if (b->n + n > b->cap) {
        size_t cap = b->cap ? b->cap : 4096;
        while (cap < b->n + n) cap *= 2;
        uint8_t *q = (uint8_t *)realloc(b->p, cap);
        if (!q) {
            fprintf(stderr, "gguf_write: out of memory\n");
            abort();
        }
        b->p = q;
        b->cap = cap;
    }
    memcpy(b->p + b->n, src, n);
    b->n += n;
}

static void gw_u32(struct gw_buf *b, uint32_t v) { gw_put(b, &v, 4); }
static void gw_u64(struct gw_buf *b, uint64_t v) { gw_put(b, &v, 8); }
static void gw_str(struct gw_buf *b, const char *s, uint64_t n) {
    gw_u64(b, n);
    gw_put(b, s, (size_t)n);
}

static void gw_init(struct gw *w) {
    memset(w, 0, sizeof(*w));
    w->alignment = 32;
}

static void gw_free(struct gw *w) {
    free(w->kv.p);
    free(w->t);
    memset(w, 0, sizeof(*w));
}

static void gw_key(struct gw *w, const char *key, uint32_t type) {
    gw_str(&w->kv, key, strlen(key));
    gw_u32(&w->kv, type);
    w->n_kv++;
}

static void gw_kv_u32(struct gw *w, const char *key, uint32_t v) {
    gw_key(w, key, GW_U32);
    gw_u32(&w->kv, v);
    if (strcmp(key, "general.alignment") == 0) w->alignment = v;
}

static void gw_kv_f32(struct gw *w, const char *key, float v) {
    gw_key(w, key, GW_F32);
    gw_put(&w->kv, &v, 4);
}

static void gw_kv_str(struct gw *w, const char *key, const char *s) {
    gw_key(w, key, GW_STR);
    gw_str(&w->kv, s, strlen(s));
}

static void gw_kv_i32_array(struct gw *w, const char *key, const int32_t *v, uint64_t n) {
    gw_key(w, key, GW_ARRAY);
    gw_u32(&w->kv, GW_I32);
    gw_u64(&w->kv, n);
    for (uint64_t i = 0; i < n; i++) gw_put(&w->kv, &v[i], 4);
}

/* An array of n strings; name(i, buf, cap) writes string i into buf and
 * returns its length. */
static void gw_kv_str_array(struct gw *w, const char *key, uint64_t n,
                            size_t (*name)(uint64_t i, char *buf, size_t cap)) {
    gw_key(w, key, GW_ARRAY);
    gw_u32(&w->kv, GW_STR);
    gw_u64(&w->kv, n);
    char tmp[256];
    for (uint64_t i = 0; i < n; i++) {
        const size_t len = name(i, tmp, sizeof(tmp));
        gw_str(&w->kv, tmp, len);
    }
}

/* GGUF shape order: shape[0] is the innermost (row length, k). */
static void gw_tensor(struct gw *w, const char *name, uint32_t type, uint32_t n_dims, const uint64_t *shape,
                      const void *data, uint64_t bytes) {
    if (w->n_t == w->cap_t) {
        w->cap_t = w->cap_t ? 2 * w->cap_t : 64;
        struct gw_tensor *q = (struct gw_tensor *)realloc(w->t, (size_t)w->cap_t * sizeof(*q));
        if (!q) {
            fprintf(stderr, "gguf_write: out of memory\n");
            abort();
        }
        w->t = q;
    }
    struct gw_tensor *t = &w->t[w->n_t++];
    memset(t, 0, sizeof(*t));
    snprintf(t->name, sizeof(t->name), "%s", name);
    t->n_dims = n_dims;
    for (uint32_t d = 0; d < n_dims && d < 4; d++) t->shape[d] = shape[d];
    t->type = type;
    t->data = data;
    t->bytes = bytes;
}

static uint64_t gw_align(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

static int gw_pad(FILE *f, uint64_t n) {
    static const uint8_t zeros[256];
    while (n > 0) {
        const size_t c = n < sizeof(zeros) ? (size_t)n : sizeof(zeros);
        if (fwrite(zeros, 1, c, f) != c) return 0;
        n -= c;
    }
    return 1;
}

/* Returns 0 on success; the file holds header | kv | tensor infos | pad |
 * data. Writes the total byte count to *total when non-NULL. */
static int gw_write(struct gw *w, const char *path, uint64_t *total) {
    struct gw_buf h = {0};
    gw_u32(&h, 0x46554747u);                          /* "GGUF" */
    gw_u32(&h, 3);
    gw_u64(&h, w->n_t);
    gw_u64(&h, w->n_kv);
    gw_put(&h, w->kv.p, w->kv.n);
    uint64_t off = 0;
    for (uint64_t i = 0; i < w->n_t; i++) {
        struct gw_tensor *t = &w->t[i];
        t->offset = off;
        off = gw_align(off + t->bytes, w->alignment);
        gw_str(&h, t->name, strlen(t->name));
        gw_u32(&h, t->n_dims);
        for (uint32_t d = 0; d < t->n_dims; d++) gw_u64(&h, t->shape[d]);
        gw_u32(&h, t->type);
        gw_u64(&h, t->offset);
    }
    FILE *f = fopen(path, "wb");
    if (!f) {
        free(h.p);
        return -1;
    }
    int ok = fwrite(h.p, 1, h.n, f) == h.n;
    uint64_t pos = h.n;
    const uint64_t data_start = gw_align(pos, w->alignment);
    ok = ok && gw_pad(f, data_start - pos);
    pos = data_start;
    for (uint64_t i = 0; i < w->n_t && ok; i++) {
        const struct gw_tensor *t = &w->t[i];
        const uint64_t at = data_start + t->offset;
        ok = gw_pad(f, at - pos);
        ok = ok && fwrite(t->data, 1, (size_t)t->bytes, f) == t->bytes;
        pos = at + t->bytes;
    }
    ok = fclose(f) == 0 && ok;
    free(h.p);
    if (total) *total = pos;
    return ok ? 0 : -1;
}

#endif /* GGUF_WRITE_C */
