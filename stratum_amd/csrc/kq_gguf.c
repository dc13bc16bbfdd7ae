/*
 * kq_gguf.c -- GGUF v3 index with hostile-input guards, the type-42 file
 * conversion and the MoE pack byte check (host code, C11).
 *
 * The accept / reject rules and the descriptors follow gguf_open
 * (stratum_gguf.h:226-444) exactly, so that a file this index accepts is
 * one the reference accepts, with the same offsets and sizes; the code is
 * organised around a bounds-checked reader over the caller's mapping.
 */
#define _GNU_SOURCE
#include "../../include/kq_gguf.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int kq_fail(const char* fmt, ...);   /* kq_linear.c */

/* ------------------------------------------------------- type table */
/* elements and bytes per block by GGUF type id (stratum_gguf.h:57-79);
 * 43 and 44 are nominal entries (2 bytes per element) as there */
static const struct { uint16_t id, elems, bytes; } k_types[] = {
    {0, 1, 4},      {1, 1, 2},      {2, 32, 18},    {3, 32, 20},    {6, 32, 22},
    {7, 32, 24},    {8, 32, 34},    {9, 32, 40},    {10, 256, 84},  {11, 256, 110},
    {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 292}, {20, 32, 18},
    {23, 256, 136}, {30, 1, 2},     {42, 256, 148}, {43, 1, 2},     {44, 1, 2},
};

int kq_gguf_type_size(uint32_t type, int* elements_per_block) {
    for (size_t i = 0; i < sizeof k_types / sizeof k_types[0]; i++)
        if (k_types[i].id == type) {
            if (elements_per_block) *elements_per_block = k_types[i].elems;
            return k_types[i].bytes;
        }
    if (elements_per_block) *elements_per_block = 0;
    return 0;
}

/* ------------------------------------------------------------ reader */
typedef struct {
    const uint8_t* at;
    const uint8_t* end;
} rd_t;

static size_t rd_left(const rd_t* r) { return (size_t)(r->end - r->at); }

static int rd_bytes(rd_t* r, void* dst, size_t n) {
    if (rd_left(r) < n) return -1;
    memcpy(dst, r->at, n);
    r->at += n;
    return 0;
}

static int rd_skip(rd_t* r, uint64_t n) {
    if (n > rd_left(r)) return -1;
    r->at += n;
    return 0;
}

static int rd_u32(rd_t* r, uint32_t* v) { return rd_bytes(r, v, 4); }
static int rd_u64(rd_t* r, uint64_t* v) { return rd_bytes(r, v, 8); }

/* a length-prefixed string, copied and NUL-terminated */
static char* rd_string(rd_t* r) {
    uint64_t n;
    if (rd_u64(r, &n) || n >= (uint64_t)SIZE_MAX || n > rd_left(r)) return NULL;
    char* s = malloc((size_t)n + 1);
    if (!s) return NULL;
    memcpy(s, r->at, (size_t)n);
    s[n] = '\0';
    r->at += n;
    return s;
}

#define KQ_GGUF_MAX_DEPTH 16

/* skips one encoded value of type vt; arrays nest at most 16 deep */
static int rd_value(rd_t* r, uint32_t vt, int depth) {
    if (depth > KQ_GGUF_MAX_DEPTH) return -1;
    switch (vt) {
    case KQ_GGUF_U8: case KQ_GGUF_I8: case KQ_GGUF_BOOL: return rd_skip(r, 1);
    case KQ_GGUF_U16: case KQ_GGUF_I16: return rd_skip(r, 2);
    case KQ_GGUF_U32: case KQ_GGUF_I32: case KQ_GGUF_F32: return rd_skip(r, 4);
    case KQ_GGUF_U64: case KQ_GGUF_I64: case KQ_GGUF_F64: return rd_skip(r, 8);
    case KQ_GGUF_STRING: {
        uint64_t n;
        return rd_u64(r, &n) ? -1 : rd_skip(r, n);
    }
    case KQ_GGUF_ARRAY: {
        uint32_t et;
        uint64_t count;
        if (rd_u32(r, &et) || rd_u64(r, &count)) return -1;
        for (uint64_t i = 0; i < count; i++)
            if (rd_value(r, et, depth + 1)) return -1;
        return 0;
    }
    default: return -1;
    }
}

/* ------------------------------------------------------------- index */
void kq_gguf_close(kq_gguf* g) {
    if (!g) return;
    if (g->kv)
        for (uint64_t i = 0; i < g->n_kv; i++) free(g->kv[i].key);
    if (g->tensors)
        for (uint64_t i = 0; i < g->n_tensors; i++) free(g->tensors[i].name);
    free(g->kv);
    free(g->tensors);
    memset(g, 0, sizeof *g);
}

static int open_fail(kq_gguf* g, const char* what, ...) {
    char msg[256];
    va_list ap;
    va_start(ap, what);
    vsnprintf(msg, sizeof msg, what, ap);
    va_end(ap);
    kq_gguf_close(g);
    return kq_fail("kq_gguf_open: %s", msg);
}

/* one tensor-info record; the dims product and byte size checked as read */
static int read_tensor(rd_t* r, kq_tensor* t, kq_gguf* g) {
    t->name = rd_string(r);
    if (!t->name) return open_fail(g, "truncated tensor name");
    if (rd_u32(r, &t->n_dims)) return open_fail(g, "truncated tensor %s", t->name);
    if (t->n_dims > 8) return open_fail(g, "tensor %s has %u dims (max 8)", t->name, t->n_dims);
    int64_t ne = 1;
    int fits = 1;
    for (uint32_t d = 0; d < t->n_dims; d++) {
        if (rd_u64(r, &t->dims[d])) return open_fail(g, "truncated tensor %s", t->name);
        if (!fits) continue;
        if (t->dims[d] > (uint64_t)INT64_MAX) { fits = 0; continue; }
        const int64_t v = (int64_t)t->dims[d];
        if (v && ne > INT64_MAX / v) { fits = 0; continue; }
        ne *= v;
    }
    t->nelem = ne;
    if (rd_u32(r, &t->type) || rd_u64(r, &t->offset))
        return open_fail(g, "truncated tensor %s", t->name);
    if (!fits) return open_fail(g, "tensor %s dimension product does not fit in int64", t->name);
    int eb = 0;
    const int bb = kq_gguf_type_size(t->type, &eb);
    if (!bb) {
        t->nbytes = -1;           /* unknown type: size not computable */
        return 0;
    }
    if (t->nelem % eb) return open_fail(g, "tensor %s is not a whole number of blocks", t->name);
    const int64_t nblk = t->nelem / eb;
    if (nblk > INT64_MAX / bb) return open_fail(g, "tensor %s byte size overflows", t->name);
    t->nbytes = nblk * bb;
    return 0;
}

int kq_gguf_open(const uint8_t* base, size_t size, kq_gguf* g) {
    if (!g) return kq_fail("kq_gguf_open: NULL index");
    memset(g, 0, sizeof *g);
    if (!base) return kq_fail("kq_gguf_open: NULL mapping");
    g->base = base;
    g->size = size;
    rd_t r = {base, base + size};
    if (rd_left(&r) < 4 || memcmp(r.at, "GGUF", 4)) return open_fail(g, "bad magic");
    r.at += 4;
    if (rd_u32(&r, &g->version)) return open_fail(g, "truncated header");
    if (g->version != 3) return open_fail(g, "unsupported version %u (only v3)", g->version);
    if (rd_u64(&r, &g->n_tensors) || rd_u64(&r, &g->n_kv)) return open_fail(g, "truncated header");
    /* a record takes at least 24 (tensor) or 12 (kv) bytes of the file */
    if (g->n_tensors > (uint64_t)size / 24 || g->n_kv > (uint64_t)size / 12)
        return open_fail(g, "implausible counts (%llu tensors, %llu kv) for %zu bytes",
                         (unsigned long long)g->n_tensors, (unsigned long long)g->n_kv, size);
    g->kv = calloc(g->n_kv ? g->n_kv : 1, sizeof *g->kv);
    if (!g->kv) return open_fail(g, "out of memory");
    g->alignment = 32;
    for (uint64_t i = 0; i < g->n_kv; i++) {
        kq_gguf_kv* kv = &g->kv[i];
        kv->key = rd_string(&r);
        if (!kv->key || rd_u32(&r, &kv->vtype)) return open_fail(g, "truncated metadata");
        kv->bytes = r.at;
        if (rd_value(&r, kv->vtype, 0)) return open_fail(g, "bad metadata value for %s", kv->key);
        kv->bytes_len = (size_t)(r.at - kv->bytes);
        if (kv->vtype == KQ_GGUF_U32 && !strcmp(kv->key, "general.alignment")) {
            uint32_t a;
            memcpy(&a, kv->bytes, 4);
            if (a >= 16 && a <= 65536 && !(a & (a - 1))) g->alignment = a;
        }
    }
    g->tensors = calloc(g->n_tensors ? g->n_tensors : 1, sizeof *g->tensors);
    if (!g->tensors) return open_fail(g, "out of memory");
    for (uint64_t i = 0; i < g->n_tensors; i++)
        if (read_tensor(&r, &g->tensors[i], g)) return -1;
    const uint64_t idx_end = (uint64_t)(r.at - base);
    g->body_offset = (idx_end + g->alignment - 1) & ~(g->alignment - 1);
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        kq_tensor* t = &g->tensors[i];
        if (t->offset > UINT64_MAX - g->body_offset)
            return open_fail(g, "tensor %s offset overflows", t->name);
        t->offset += g->body_offset;
        if (t->offset > (uint64_t)size)
            return open_fail(g, "tensor %s offset %llu past the end (%zu)", t->name,
                             (unsigned long long)t->offset, size);
        if (t->nbytes >= 0 && (uint64_t)t->nbytes > (uint64_t)size - t->offset)
            return open_fail(g, "tensor %s [%llu + %lld) past the end (%zu)", t->name,
                             (unsigned long long)t->offset, (long long)t->nbytes, size);
    }
    return 0;
}

const kq_tensor* kq_gguf_find_tensor(const kq_gguf* g, const char* name) {
    for (uint64_t i = 0; g && name && i < g->n_tensors; i++)
        if (!strcmp(g->tensors[i].name, name)) return &g->tensors[i];
    return NULL;
}

const kq_gguf_kv* kq_gguf_find_kv(const kq_gguf* g, const char* key) {
    for (uint64_t i = 0; g && key && i < g->n_kv; i++)
        if (!strcmp(g->kv[i].key, key)) return &g->kv[i];
    return NULL;
}

static int is_int32(uint32_t t) { return t == KQ_GGUF_U32 || t == KQ_GGUF_I32; }
static int is_int64(uint32_t t) { return t == KQ_GGUF_U64 || t == KQ_GGUF_I64; }

int kq_gguf_get_u32(const kq_gguf* g, const char* key, uint32_t* out) {
    const kq_gguf_kv* kv = kq_gguf_find_kv(g, key);
    if (!kv || !out) return -1;
    if (is_int32(kv->vtype)) { memcpy(out, kv->bytes, 4); return 0; }
    if (is_int64(kv->vtype)) {
        uint64_t v;
        memcpy(&v, kv->bytes, 8);
        *out = (uint32_t)v;
        return 0;
    }
    return -1;
}

int kq_gguf_get_u64(const kq_gguf* g, const char* key, uint64_t* out) {
    const kq_gguf_kv* kv = kq_gguf_find_kv(g, key);
    if (!kv || !out) return -1;
    if (is_int64(kv->vtype)) { memcpy(out, kv->bytes, 8); return 0; }
    if (is_int32(kv->vtype)) {
        uint32_t v;
        memcpy(&v, kv->bytes, 4);
        *out = v;
        return 0;
    }
    return -1;
}

int kq_gguf_get_f32(const kq_gguf* g, const char* key, float* out) {
    const kq_gguf_kv* kv = kq_gguf_find_kv(g, key);
    if (!kv || !out || kv->vtype != KQ_GGUF_F32) return -1;
    memcpy(out, kv->bytes, 4);
    return 0;
}

char* kq_gguf_get_string_dup(const kq_gguf* g, const char* key) {
    const kq_gguf_kv* kv = kq_gguf_find_kv(g, key);
    if (!kv || kv->vtype != KQ_GGUF_STRING || kv->bytes_len < 8) return NULL;
    uint64_t n;
    memcpy(&n, kv->bytes, 8);
    if (n > kv->bytes_len - 8 || n >= (uint64_t)SIZE_MAX) return NULL;
    char* s = malloc((size_t)n + 1);
    if (!s) return NULL;
    memcpy(s, kv->bytes + 8, (size_t)n);
    s[n] = '\0';
    return s;
}

/* ------------------------------------------------ type-42 conversion */
/* Q2_K block (84 B: scales 16, qs 64, d, dmin) -> type 42 (148 B: scales
 * 16, nibbles 128, d, dmin).  Weight p of the block is the 2-bit field
 * (p % 128) / 32 of qs byte 32 (p / 128) + p % 32; type 42 keeps it in
 * byte 16 + 16 (p / 32) + p % 16, low nibble for p % 32 < 16, high
 * nibble otherwise (the converter's layout, tools_gguf_nib_convert.c:99-120). */
static void nib_block(const uint8_t* q, uint8_t* o) {
    memcpy(o, q, 16);
    memcpy(o + 144, q + 80, 4);
    for (int grp = 0; grp < 8; grp++) {             /* 32 weights p = 32 grp .. */
        const uint8_t* qs = q + 16 + 32 * (grp >> 2);
        const int sh = 2 * (grp & 3);
        uint8_t* dst = o + 16 + 16 * grp;
        for (int l = 0; l < 16; l++)
            dst[l] = (uint8_t)(((qs[l] >> sh) & 3) | (((qs[l + 16] >> sh) & 3) << 4));
    }
}

int64_t kq_gguf_nib_convert(const kq_gguf* g, uint8_t* out, uint64_t* out_size) {
    if (!g || !g->base || !out_size) return kq_fail("kq_gguf_nib_convert: NULL argument");
    /* the reference tool addresses its index by byte positions it re-derives
     * from the key and value lengths; the same walk here */
    uint64_t total = 0;
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        const kq_tensor* t = &g->tensors[i];
        if (t->nbytes < 0) return kq_fail("kq_gguf_nib_convert: tensor %s of unknown size", t->name);
        total += t->type == KQ_TYPE_Q2_K ? (uint64_t)(t->nelem / 256) * 148 : (uint64_t)t->nbytes;
    }
    *out_size = g->body_offset + total;
    if (!out) {
        int64_t n = 0;
        for (uint64_t i = 0; i < g->n_tensors; i++) n += g->tensors[i].type == KQ_TYPE_Q2_K;
        return n;
    }
    memcpy(out, g->base, g->body_offset);
    rd_t r = {g->base + 24, g->base + g->size};
    for (uint64_t i = 0; i < g->n_kv; i++) {
        uint64_t n;
        if (rd_u64(&r, &n) || rd_skip(&r, n) || rd_skip(&r, 4) || rd_skip(&r, g->kv[i].bytes_len))
            return kq_fail("kq_gguf_nib_convert: index walk failed");
    }
    uint64_t pos = 0;
    int64_t converted = 0;
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        const kq_tensor* t = &g->tensors[i];
        uint64_t n;
        uint32_t nd;
        if (rd_u64(&r, &n) || rd_skip(&r, n) || rd_u32(&r, &nd) || rd_skip(&r, 8ull * nd))
            return kq_fail("kq_gguf_nib_convert: index walk failed");
        const uint64_t type_at = (uint64_t)(r.at - g->base);
        if (rd_skip(&r, 12)) return kq_fail("kq_gguf_nib_convert: index walk failed");
        const uint8_t* src = g->base + t->offset;
        uint8_t* dst = out + g->body_offset + pos;
        uint64_t len;
        if (t->type == KQ_TYPE_Q2_K) {
            const uint32_t nt = KQ_TYPE_Q2K_NIB;
            memcpy(out + type_at, &nt, 4);
            const int64_t nb = t->nelem / 256;
            for (int64_t b = 0; b < nb; b++) nib_block(src + 84 * b, dst + 148 * b);
            len = (uint64_t)nb * 148;
            converted++;
        } else {
            len = (uint64_t)t->nbytes;
            memcpy(dst, src, len);
        }
        memcpy(out + type_at + 4, &pos, 8);
        pos += len;
    }
    return converted;
}

/* -------------------------------------------------- MoE pack check */
int kq_moe_pack_check(const kq_moe_pack* p, const uint8_t* model_base, int n_layers,
                      const kq_tensor* const* gate, const kq_tensor* const* up,
                      const kq_tensor* const* down, int n_embed, int n_ff, int full) {
    if (!p || !model_base || !gate || !up || !down || n_layers < 1 || n_layers > (int)p->n_layers)
        return kq_fail("kq_moe_pack_check: bad arguments");
    const int E = (int)p->n_experts;
    int checked = 0;
    for (int li = 0; li < n_layers; li++) {
        const kq_tensor* ts[3] = {gate[li], up[li], down[li]};
        const int64_t sl[3] = {kq_moe_slice_bytes(ts[0], n_embed, n_ff),
                               kq_moe_slice_bytes(ts[1], n_embed, n_ff),
                               kq_moe_slice_bytes(ts[2], n_ff, n_embed)};
        if (sl[0] != (int64_t)p->gate_slice || sl[1] != (int64_t)p->up_slice ||
            sl[2] != (int64_t)p->down_slice)
            return kq_fail("kq_moe_pack_check: layer %d slice sizes differ from the pack", li);
        for (int e = 0; e < E; e++) {
            if (!full && e != 0 && e != E / 2 && e != E - 1) continue;
            checked++;
            for (int w = 0; w < 3; w++) {
                const uint8_t* got = kq_moe_pack_which(p, li, e, w);
                const uint8_t* want = model_base + ts[w]->offset + (uint64_t)e * (uint64_t)sl[w];
                if (!got || memcmp(got, want, (size_t)sl[w]))
                    return kq_fail("kq_moe_pack_check: layer %d expert %d tensor %d differs", li,
                                   e, w);
            }
        }
    }
    return checked;
}
