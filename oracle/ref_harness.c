/*
 * ref_harness.c -- thin C-ABI around the reference's OWN scalar headers.
 *
 * TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile, only when
 * /root/reference is present, into oracle/_ref/libkqref.so with
 *   -I/root/reference/stratum/native -O2 -ffp-contract=off -fno-fast-math
 * No reference source is copied: the headers are #included where they
 * lie.  The library is used to (a) pin oracle/kq_oracle.c bit for bit and
 * to write the golden fixtures under tests/golden/, and (b) as the
 * "reference" CPU baseline in bench.py (kind "reference").
 *
 * Exported functions wrap, without changing any arithmetic:
 *   q4k_fp16_to_fp32, q4k_get_scale_min          (stratum_q4k.h:24-65)
 *   q{4,6,2}k_dequant_block_scalar               (stratum_q4k.h:67, q6k.h:17, q2k.h:16)
 *   q{4,6,2}k_dot_row_scalar                     (stratum_q4k.h:95, q6k.h:38, q2k.h:44)
 *   q{3,5}k_dequant_block_scalar / _dot_row_scalar (stratum_q3k.h:30, 58; q5k.h:18, 44)
 *   q8_0_dequant_block_scalar / _dot_row_scalar  (stratum_q8_0.h:14, 19)
 *   gguf_open / gguf_close                        (stratum_gguf.h:226-463)
 * plus a pthread row split with 64-row tickets, as ST_PAR_ROWS does
 * (stratum_linear.h:201-228) on a machine without NEON (stratum_linear.h:446-451).
 */
#define _GNU_SOURCE
#include "stratum_q4k.h"
#include "stratum_q6k.h"
#include "stratum_q2k.h"
#include "stratum_q3k.h"
#include "stratum_q5k.h"
#include "stratum_q8_0.h"
#include "stratum_gguf.h"

#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <string.h>

float kqref_fp16_to_fp32(uint16_t h) { return q4k_fp16_to_fp32(h); }

void kqref_scale_min(int j, const uint8_t* s, uint8_t* sc, uint8_t* m) {
    q4k_get_scale_min(j, s, sc, m);
}

/* q4k_get_scale_min for sub-block j over every value of the bytes idx[]
 * (the same enumeration as ko_q4k_scale_min_sweep, for an exhaustive
 * comparison) */
void kqref_scale_min_sweep(int j, const int* idx, int nidx, const uint8_t* bg, uint8_t* out) {
    uint8_t s[12];
    memcpy(s, bg, 12);
    const uint32_t n = 1u << (8 * nidx);
    for (uint32_t c = 0; c < n; c++) {
        for (int i = 0; i < nidx; i++) s[idx[i]] = (uint8_t)(c >> (8 * i));
        q4k_get_scale_min(j, s, &out[2 * (size_t)c], &out[2 * (size_t)c + 1]);
    }
}

/* bytes per 256 weights (Q8_0: eight of its 32-weight blocks) */
/* q3k_unpack_scales (stratum_q3k.h:17-28) group g over every value of the
 * bytes idx[] (the same enumeration as ko_q3k_scale_sweep); the unpacked
 * int8 is stored as its byte */
void kqref_q3k_scale_sweep(int g, const int* idx, int nidx, const uint8_t* bg, uint8_t* out) {
    uint8_t s[12];
    memcpy(s, bg, 12);
    const uint32_t n = 1u << (8 * nidx);
    for (uint32_t c = 0; c < n; c++) {
        for (int i = 0; i < nidx; i++) s[idx[i]] = (uint8_t)(c >> (8 * i));
        int8_t sc[16];
        q3k_unpack_scales(s, sc);
        out[c] = (uint8_t)sc[g];
    }
}

/* bytes per 256 weights (Q8_0: eight of its 32-weight blocks) */
int kqref_block_bytes(int type) {
    return type == 12 ? (int)sizeof(block_q4_K)
         : type == 14 ? (int)sizeof(block_q6_K)
         : type == 10 ? (int)sizeof(block_q2_K)
         : type == 11 ? (int)sizeof(block_q3_K)
         : type == 13 ? (int)sizeof(block_q5_K)
         : type == 8 ? 8 * (int)sizeof(block_q8_0) : 0;
}

int kqref_dequant_row(int type, const uint8_t* row, int K, float* y) {
    for (int b = 0; b < K / 256; b++) {
        switch (type) {
        case 12: q4k_dequant_block_scalar((const block_q4_K*)row + b, y + 256 * b); break;
        case 14: q6k_dequant_block_scalar((const block_q6_K*)row + b, y + 256 * b); break;
        case 10: q2k_dequant_block_scalar((const block_q2_K*)row + b, y + 256 * b); break;
        case 11: q3k_dequant_block_scalar((const block_q3_K*)row + b, y + 256 * b); break;
        case 13: q5k_dequant_block_scalar((const block_q5_K*)row + b, y + 256 * b); break;
        case 8:
            for (int q = 0; q < 8; q++)
                q8_0_dequant_block_scalar((const block_q8_0*)row + 8 * b + q, y + 256 * b + 32 * q);
            break;
        default: return -1;
        }
    }
    return 0;
}

float kqref_dot_row(int type, const uint8_t* row, int K, const float* x) {
    switch (type) {
    case 12: return q4k_dot_row_scalar((const block_q4_K*)row, K, x);
    case 14: return q6k_dot_row_scalar((const block_q6_K*)row, K, x);
    case 10: return q2k_dot_row_scalar((const block_q2_K*)row, K, x);
    case 11: return q3k_dot_row_scalar((const block_q3_K*)row, K, x);
    case 13: return q5k_dot_row_scalar((const block_q5_K*)row, K, x);
    case 8: return q8_0_dot_row_scalar((const block_q8_0*)row, K, x);
    default: return 0.0f;
    }
}

typedef struct {
    int type, N, K, B;
    size_t rb;
    const uint8_t* w;
    const float* x;
    float* y;
    atomic_int next;
} kqref_job;

static void* kqref_worker(void* a) {
    kqref_job* j = (kqref_job*)a;
    for (;;) {
        int s = atomic_fetch_add_explicit(&j->next, 64, memory_order_relaxed);
        if (s >= j->N) break;
        int e = s + 64 < j->N ? s + 64 : j->N;
        for (int r = s; r < e; r++)
            for (int b = 0; b < j->B; b++)
                j->y[(size_t)b * j->N + r] =
                    kqref_dot_row(j->type, j->w + (size_t)r * j->rb, j->K,
                                  j->x + (size_t)b * j->K);
    }
    return NULL;
}

/* ys[b*N + r] = row r . xs[b*K ...] for b < B, rows split over nthreads */
int kqref_gemv(int type, const uint8_t* w, const float* xs, float* ys,
               int B, int N, int K, int nthreads) {
    int bb = kqref_block_bytes(type);
    if (!bb || K % 256) return -1;
    kqref_job j;
    j.type = type; j.N = N; j.K = K; j.B = B;
    j.rb = (size_t)(K / 256) * (size_t)bb;
    j.w = w; j.x = xs; j.y = ys;
    atomic_store(&j.next, 0);
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    int started = 0;
    for (int t = 0; t < nthreads - 1; t++) {
        if (pthread_create(&th[t], NULL, kqref_worker, &j) != 0) break;
        started++;
    }
    kqref_worker(&j);
    for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
    return 0;
}

/* gguf_open on a file, its index copied out: 0 (opened) or -1 (refused).
 * Per tensor i < min(n_tensors, cap): type, n_dims, dims[8 i ..], offset
 * (absolute, as gguf_open leaves it), nelem, nbytes and the first 63
 * bytes of the name at names + 64 i. */
int kqref_gguf_open(const char* path, uint64_t* counts /* n_tensors, n_kv, body, align */,
                    int cap, uint32_t* types, uint32_t* ndims, uint64_t* dims, uint64_t* offsets,
                    int64_t* nelem, int64_t* nbytes, char* names) {
    Gguf g;
    if (gguf_open(path, &g) != 0) return -1;
    counts[0] = g.n_tensors; counts[1] = g.n_kv; counts[2] = g.body_offset; counts[3] = g.alignment;
    for (uint64_t i = 0; i < g.n_tensors && i < (uint64_t)cap; i++) {
        const GgufTensor* t = &g.tensors[i];
        types[i] = t->type; ndims[i] = t->n_dims;
        for (int d = 0; d < 8; d++) dims[8 * i + d] = t->dims[d];
        offsets[i] = t->offset; nelem[i] = t->nelem; nbytes[i] = t->nbytes;
        strncpy(names + 64 * i, t->name, 63);
        names[64 * i + 63] = 0;
    }
    gguf_close(&g);
    return 0;
}
