/*
 * kq_gemv.h -- C ABI of the MI355X (gfx950) k-quant GEMV library
 * (stratum_amd/libkqgemv.so).
 *
 * Drop-in boundary for stratum's quantized matvec layer (the L4/L5 seam of
 * /root/reference/stratum/native/stratum_linear.h).  Signatures, argument
 * order, tensor descriptor layout, GGML type ids and the -1 error convention
 * follow the reference; each entry point cites the function it replaces.
 * Plain C types only: no HIP or torch types appear in the signatures (a
 * stream is passed as an opaque pointer that is a hipStream_t).
 *
 * Numerics: every GEMV entry point computes, per row, the reference scalar
 * routine's binary32 sub-block arithmetic (stratum_q4k.h:95-131,
 * stratum_q6k.h:38-73, stratum_q2k.h:44-89) with the sub-block terms summed
 * in binary64; outputs match the scalar routine bit for bit except where a
 * binary64 re-association crosses a binary32 rounding boundary (at most
 * one ulp).  Dequantization is bit-exact.
 *
 * Threading: like the reference (single caller, non-reentrant global
 * state, stratum_linear.h:239-242), one host thread drives the library.
 */
#ifndef KQ_GEMV_H
#define KQ_GEMV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids the GEMV accepts (stratum_gguf.h:20-49).  Any other type
 * makes the dispatch return -1, as st_linear_dispatch does for types it
 * has no kernel for (stratum_linear.h:553-556). */
#define KQ_TYPE_Q2_K    10
#define KQ_TYPE_Q4_K    12
#define KQ_TYPE_Q6_K    14
#define KQ_TYPE_Q2K_NIB 42

/* Layout-compatible with GgufTensor (stratum_gguf.h:129-137): a caller may
 * pass its GgufTensor* cast to kq_tensor*.  `offset` is in bytes from the
 * weight base registered with kq_linear_init (the reference's
 * g_st.mmap_base + offset addressing, stratum_linear.h:169-188). */
typedef struct kq_tensor {
    char*    name;
    uint32_t n_dims;
    uint64_t dims[8];
    uint32_t type;
    uint64_t offset;
    int64_t  nelem;
    int64_t  nbytes;
} kq_tensor;

/* Opaque hipStream_t; NULL is the null (default) stream. */
typedef void* kq_stream;

/* ------------------------------------------------------------ set-up */

/* Replaces stratum_linear_init(mmap_base, mmap_size) (stratum_linear.h:90).
 * Selects the current HIP device, uploads [base, base+size) to HBM once and
 * makes it the region that kq_tensor offsets are resolved against.  May be
 * called again with a new base (the old upload is released).  0 or -1. */
int kq_linear_init(const uint8_t* base, size_t size);

/* Registers (uploads) an additional host mapping, e.g. the MoE expert pack
 * whose slices moe_bind_slice addresses as base + offset
 * (stratum_arch_moe.inc.c:327-337).  Offsets that land inside any
 * registered mapping resolve to its device copy.  0 or -1. */
int kq_register_region(const void* host, size_t size);

/* Device address of host byte range [host, host+nbytes) inside a registered
 * mapping, or NULL. */
const void* kq_device_ptr(const void* host, size_t nbytes);

/* Releases every upload and scratch buffer. */
void kq_linear_shutdown(void);

/* Message of the last failure (never NULL). */
const char* kq_last_error(void);

/* ------------------------------------------- host-pointer entry points
 * x/y/add are host buffers, exactly as in the reference; each call copies
 * the activations in, runs the kernel and copies y back (synchronous). */

/* y[0..N) = W . x.  Replaces st_linear_dispatch (stratum_linear.h:526).
 * Returns -1 for an unsupported type, K % 256 != 0, a weight range outside
 * the registered mappings, or a HIP error. */
int kq_linear_dispatch(const kq_tensor* w, const float* x, float* y, int N, int K);

/* y = add + W . x; add == NULL behaves as kq_linear_dispatch; add and y
 * must not alias.  Replaces st_linear_dispatch_add (stratum_linear.h:568). */
int kq_linear_dispatch_add(const kq_tensor* w, const float* x, const float* add,
                           float* y, int N, int K);

/* ys[s] = W . xs[s] for s < B with one weight pass; each stream's result
 * equals its single-stream result bit for bit.  Replaces st_linear_multix
 * (stratum_linear.h:715), which returns void; this returns 0 or -1. */
int kq_linear_multix(const kq_tensor* w, const float* const* xs, float* const* ys,
                     int B, int N, int K);

/* Same-input group: y0 = W0.x, y1 = W1.x and, when w2 != NULL, y2 = W2.x,
 * in one launch.  Replaces st_q4k_group (stratum_linear.h:1086-1121); any
 * mix of the supported types is accepted.  0 or -1. */
int kq_q4k_group(const float* x, int K,
                 const kq_tensor* w0, float* y0, int N0,
                 const kq_tensor* w1, float* y1, int N1,
                 const kq_tensor* w2, float* y2, int N2);

/* ----------------------------------------- device-pointer entry points
 * For a device-resident decode loop: all pointers are device pointers,
 * the call only enqueues work on `stream` (asynchronous).  x and xs must
 * be 16-byte aligned. */

/* y = W . x (+ add when add != NULL), W = N rows of K/256 blocks of `type`. */
int kq_gemv_dev(int type, const void* w, const float* x, const float* add, float* y,
                int N, int K, kq_stream stream);

/* Contiguous multix: ys[s*N + r] = row r . xs[s*K ...] for s < B. */
int kq_gemv_multix_dev(int type, const void* w, const float* xs, float* ys,
                       int B, int N, int K, kq_stream stream);

/* One segment of a batched launch: ngroups * rows_per_group rows of one
 * type and row length K.  Rows [g*rows_per_group, (g+1)*rows_per_group)
 * start at device address w[g] (separate bases: e.g. the selected MoE
 * expert slices, stratum_arch_moe.inc.c:327-337) and read x, or, when
 * x_stride != 0, x + g*x_stride.  y[i] (and add[i]) is segment row i. */
#define KQ_MAX_SEGMENTS 8
#define KQ_MAX_GROUPS 16
typedef struct kq_segment {
    int type;
    int K;
    int rows_per_group;
    int ngroups;
    const void* w[KQ_MAX_GROUPS];
    const float* x;
    int x_stride;
    const float* add;
    float* y;
} kq_segment;

/* Runs up to KQ_MAX_SEGMENTS segments in ONE launch, in order, each with
 * the numerics of kq_gemv_dev.  Consecutive segments that read the same x
 * (the same-input groups of st_q4k_group, stratum_linear.h:1086) stage it
 * once.  No counterpart in the reference, which issues one call per tensor;
 * it exists so a device-resident decode step pays one launch for several
 * matvecs (a layer's QKV, gate+up, or a set of MoE expert slices). */
int kq_gemv_segments_dev(const kq_segment* segs, int nseg, kq_stream stream);

/* Bit-exact dequantization of nblocks consecutive blocks into 256*nblocks
 * floats (q4k_dequant_row_scalar and peers, stratum_q4k.h:67-93,
 * stratum_q6k.h:17-36, stratum_q2k.h:16-42). */
int kq_dequant_dev(int type, const void* w, float* y, int64_t nblocks, kq_stream stream);

/* Bytes of one row of K weights of `type` (K/256 blocks), or -1. */
int64_t kq_row_bytes(int type, int K);

#ifdef __cplusplus
}
#endif
#endif /* KQ_GEMV_H */
