/*
 * kq_gguf.h -- GGUF v3 index over a caller-mapped file, with the
 * reference's hostile-input guards, and the type-42 (Q2K_NIB) conversion.
 *
 * Replaces stratum_gguf.h's gguf_open / gguf_close / gguf_find_tensor /
 * gguf_find_kv / gguf_get_{u32,u64,f32,string_dup} (stratum_gguf.h:226-523)
 * for the GEMV path: the caller maps the file (mmap, or any buffer) and
 * passes [base, base + size); the index keeps pointers into it.  Tensor
 * descriptors are kq_tensor (== GgufTensor) with `offset` in bytes from
 * base, so they go straight to kq_linear_init(base, size) and
 * kq_linear_dispatch.
 */
#ifndef KQ_GGUF_H
#define KQ_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "kq_gemv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GgufValType (stratum_gguf.h:105-119) */
enum {
    KQ_GGUF_U8 = 0, KQ_GGUF_I8 = 1, KQ_GGUF_U16 = 2, KQ_GGUF_I16 = 3, KQ_GGUF_U32 = 4,
    KQ_GGUF_I32 = 5, KQ_GGUF_F32 = 6, KQ_GGUF_BOOL = 7, KQ_GGUF_STRING = 8,
    KQ_GGUF_ARRAY = 9, KQ_GGUF_U64 = 10, KQ_GGUF_I64 = 11, KQ_GGUF_F64 = 12,
};

/* One metadata entry: layout-compatible with GgufKV (stratum_gguf.h:121-127);
 * bytes / bytes_len is the encoded value inside the mapping. */
typedef struct kq_gguf_kv {
    char* key;
    uint32_t vtype;
    const uint8_t* bytes;
    size_t bytes_len;
} kq_gguf_kv;

typedef struct kq_gguf {
    const uint8_t* base;
    size_t size;
    uint32_t version;
    uint64_t n_tensors, n_kv;
    kq_gguf_kv* kv;
    kq_tensor* tensors;
    uint64_t body_offset, alignment;
} kq_gguf;

/* Parses the GGUF v3 index at [base, base + size) with gguf_open's checks
 * (stratum_gguf.h:226-444): magic and version 3; tensor and KV counts
 * bounded by what size could hold (24 and 12 bytes each); every read
 * bounds-checked; nested arrays at most 16 deep; general.alignment taken
 * when it is a UINT32 power of two in [16, 65536], else 32; at most 8
 * dims, their product within int64; known types need a whole number of
 * blocks and a byte size within int64 (unknown types get nbytes -1); the
 * body starts at the aligned end of the index; an offset must not wrap
 * when the body offset is added, must not pass the end of the mapping, and
 * a known size must fit after it.  The same files are accepted and
 * rejected as by gguf_open, with the same descriptors.  0, or -1 with
 * kq_last_error() set and *g zeroed. */
int kq_gguf_open(const uint8_t* base, size_t size, kq_gguf* g);

/* Frees the index (not the mapping). */
void kq_gguf_close(kq_gguf* g);

/* gguf_find_tensor / gguf_find_kv: the first entry with that name, or NULL. */
const kq_tensor* kq_gguf_find_tensor(const kq_gguf* g, const char* name);
const kq_gguf_kv* kq_gguf_find_kv(const kq_gguf* g, const char* key);

/* gguf_get_u32 / _u64 / _f32 (stratum_gguf.h:478-507): 0, or -1 when the
 * key is missing or its type does not convert (the reference's rules:
 * 32- and 64-bit integers convert both ways, F32 only from F32). */
int kq_gguf_get_u32(const kq_gguf* g, const char* key, uint32_t* out);
int kq_gguf_get_u64(const kq_gguf* g, const char* key, uint64_t* out);
int kq_gguf_get_f32(const kq_gguf* g, const char* key, float* out);

/* gguf_get_string_dup: a NUL-terminated copy (free() it), or NULL. */
char* kq_gguf_get_string_dup(const kq_gguf* g, const char* key);

/* Bytes per block and elements per block of a GGUF type id (the table of
 * stratum_gguf.h:57-79); 0 for an unknown id. */
int kq_gguf_type_size(uint32_t type, int* elements_per_block);

/* The type-42 file conversion of tools_gguf_nib_convert.c:17-131: every
 * Q2_K tensor's blocks re-laid as 148-byte Q2K_NIB blocks and its type id
 * set to 42, every other tensor copied; the index is copied with each
 * tensor's offset rewritten to the tensors laid back to back in index
 * order from the body offset (the reference tool's layout).  Writes
 * *out_size bytes to out when out != NULL (call with out == NULL first for
 * the size).  Returns the number of Q2_K tensors converted, or -1. */
int64_t kq_gguf_nib_convert(const kq_gguf* g, uint8_t* out, uint64_t* out_size);

/* The same block permutation on the device: nblocks Q2_K blocks (84 B) at
 * q2k to type-42 blocks (148 B) at nib.  No counterpart in the reference
 * (its converter is a host tool); for converting at upload time. */
int kq_q2k_to_nib_dev(const void* q2k, void* nib, int64_t nblocks, kq_stream stream);

/* The sampled byte comparison of moe_pack_load (stratum_arch_moe.inc.c:
 * 529-560, moe_pack_check_slice :452-457): for every layer li < n_layers,
 * the gate / up / down slices of experts 0, E/2 and E-1 (every expert when
 * full != 0) in the pack must equal the stacked tensors' slices in the
 * model mapping (model_base + tensor offset + e * slice).  gate[li] etc.
 * are each layer's stacked tensors; a layer whose slice sizes differ from
 * the pack's fails.  Returns the number of experts checked, or -1. */
int kq_moe_pack_check(const kq_moe_pack* p, const uint8_t* model_base, int n_layers,
                      const kq_tensor* const* gate, const kq_tensor* const* up,
                      const kq_tensor* const* down, int n_embed, int n_ff, int full);

#ifdef __cplusplus
}
#endif
#endif /* KQ_GGUF_H */
