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
 * stratum_q6k.h:38-73, stratum_q2k.h:44-89, stratum_q5k.h:44-82,
 * stratum_q3k.h:58-99, stratum_q8_0.h:19-33) with the sub-block terms summed
 * in binary64; outputs match the scalar routine bit for bit except where a
 * binary64 re-association crosses a binary32 rounding boundary (at most
 * one ulp).  F16 and F32 rows are the binary64 sum of exact products,
 * rounded once (st_linear_f16 sums in element order; F32 goes to
 * cblas_sgemv in the reference, stratum_linear.h:491-512).  Dequantization
 * is bit-exact.
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

/* GGML type ids the GEMV accepts (stratum_gguf.h:20-49): every type of
 * st_linear_dispatch's switch (stratum_linear.h:533-541) except the Apple
 * W16 repacks (43, 44), plus type 42.  Any other type makes the dispatch
 * return -1, as st_linear_dispatch does for types it has no kernel for
 * (stratum_linear.h:553-556).  K must be a multiple of 256 for every type
 * (Q8_0 rows then hold K/32 blocks of 34 bytes). */
#define KQ_TYPE_F32     0
#define KQ_TYPE_F16     1
#define KQ_TYPE_Q8_0    8
#define KQ_TYPE_Q2_K    10
#define KQ_TYPE_Q3_K    11
#define KQ_TYPE_Q4_K    12
#define KQ_TYPE_Q5_K    13
#define KQ_TYPE_Q6_K    14
#define KQ_TYPE_Q2K_NIB 42

/* Int8-activation mode of Q4_K, Q6_K, Q5_K, Q3_K and Q8_0:
 * `type | KQ_INT8_ACT` on kq_gemv_dev, kq_gemv_multix_dev and
 * kq_gemv_segments_dev computes the reference's SDOT path (g_st.use_sdot,
 * stratum_linear.h:376-489, 581-603, 643-690): x quantized to int8 per 16
 * (Q6_K, q6k_quantize_x_q8_g16, stratum_q6k_neon.h:117-133) or per 32 (the
 * others, q4k_quantize_x_q8, stratum_q4k_neon.h:229-275), exact integer
 * dot products per sub-block, group or block, and the terms of
 * q4k_dot_row_sdot_f / q6k_dot_row_sdot_f / q5k_dot_row_sdot_f /
 * q3k_dot_row_sdot_f / q8_0_dot_row_sdot_f (stratum_q4k_neon.h:365-407,
 * q6k_neon.h:265-317, q5k_neon.h:158-204, q3k_neon.h:84-125,
 * stratum_q8_0.h:112-145): coefficient fl(fl(d*sc)*xscale) (Q8_0:
 * fl(d*xscale)) times the integer sum.  The quantized x, the integer parts
 * and the coefficients are bit-identical to the reference's; the terms are
 * summed in binary64 instead of the reference's four binary32 FMA lanes,
 * so y differs from q*_dot_row_sdot_f by at most 2^-22 * sum|term| (the
 * lanes' own rounding) and is independent of the launch shape.  The
 * weights are unchanged: kq_row_bytes is the base type's.  Batches take
 * the reference's batch arithmetic: kq_gemv_multix_dev at B >= 2 for Q4_K
 * and Q6_K the multix pack form (below), kq_moe_gemv_dev /
 * kq_moe_gemv_routed_dev / kq_moe_ffn_dev at B > 1 moe_forward_b's
 * tickets (at kq_moe_gemv_dev).  A segment list mixing Q4_K and Q6_K in
 * this mode runs as one launch (st_mixed_fused_sdot,
 * stratum_linear.h:1043-1085). */
#define KQ_INT8_ACT     0x100

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

/* Launch-shape overrides for tuning runs and tests: KQ_GRID (workgroups),
 * KQ_WG_THREADS (256, 512 or 1024 lanes), KQ_DEPTH (1 or 2 batches in
 * flight; 2 only with at most 512 lanes), KQ_MOE_GROUP_LAUNCH (MoE batches
 * grouped by a separate launch) and KQ_MOE_FFN_SPLIT (kq_moe_ffn_dev in its
 * six-launch form at batch 1, and without shared run tables at B > 1).  The environment is read once, at the first
 * call that touches the device; this re-reads it.  Results never depend on
 * these (the reduction order is fixed by the row length), only the launch
 * shape.  No counterpart in the reference.  Returns 0. */
int kq_tuning_reload(void);

/* g_st.use_sdot for the host-pointer entry points (kq_linear_dispatch*,
 * kq_linear_multix, kq_q4k_group): on != 0 routes Q4_K, Q6_K, Q5_K, Q3_K
 * and Q8_0 through the int8-activation mode (KQ_INT8_ACT), as
 * st_linear_q4k / _q6k / _q5k / _q3k / _q8_0 do when use_sdot is set
 * (stratum_linear.h:376-489).  Off at start-up: the
 * reference turns it on by default only where its NEON kernels exist
 * (stratum_linear.h:133-137).  Returns the previous setting. */
int kq_linear_set_sdot(int on);

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
 * be 16-byte aligned.  The MoE batch and matrix-core entries use scratch
 * buffers owned by the library, one set per stream, grown on demand: calls
 * on different streams may overlap in time, calls on one stream are
 * ordered.  The library keeps 16 sets; a seventeenth stream takes the least
 * recently used stream's set, freeing its buffers first (hipFree, which
 * waits for the device). */

/* The int8 quantizer of the int8-activation mode on its own: group 32 is
 * q4k_quantize_x_q8 (+ q4k_sum_i8_32 sums, stratum_q4k_neon.h:229-275,
 * 414-420), group 16 is q6k_quantize_x_q8_g16 (+ q6k_xsum16_i8,
 * stratum_q6k_neon.h:117-133, 261-264).  xq gets K bytes, xscale and xsum
 * (may be NULL) K/group entries.  Bit-identical to the reference. */
int kq_quantize_x_q8_dev(const float* x, int K, int group, int8_t* xq, float* xscale,
                         int32_t* xsum, kq_stream stream);

/* y = W . x (+ add when add != NULL), W = N rows of K/256 blocks of `type`. */
int kq_gemv_dev(int type, const void* w, const float* x, const float* add, float* y,
                int N, int K, kq_stream stream);

/* Contiguous multix: ys[s*N + r] = row r . xs[s*K ...] for s < B, one
 * weight pass; each stream equals its kq_gemv_dev result bit for bit.
 * Exception, as in the reference: Q4_K and Q6_K in the int8 mode at B >= 2
 * compute st_linear_multix's int8 arithmetic under use_sdot
 * (stratum_linear.h:732-907, q4k_dot_rows2_sdot_multix_pack /
 * q6k_dot_rows2_sdot_multix_pack, stratum_q4k_neon.h:870-948,
 * stratum_q6k_neon.h:627-700) bit for bit: one binary32 term per Q4_K
 * sub-block (binary64 per Q6_K 16-group) summed in binary64 in element
 * order, which differs from the single-stream SDOT form's rounding (the
 * reference's own quant_test.c holds the two within 1e-4).  That path
 * runs the integer dots on the matrix cores and uses the library's
 * matrix-core workspace of the call's stream (grown on demand, see
 * kq_reserve_mfma_workspace). */
int kq_gemv_multix_dev(int type, const void* w, const float* xs, float* ys,
                       int B, int N, int K, kq_stream stream);

/* The same product on the matrix cores, for many streams (B >= 16 is where
 * it pays): Q4_K and Q6_K only (-1 for other types).  Each super-block runs
 * as fp16 x fp16 -> fp32 MFMAs: the weights with their sub-block scales
 * folded in (exact fp16 integers), x as two fp16 planes (22 significant
 * bits, scaled per stream and super-block); the block scale, the Q4_K min
 * term and the sums across super-blocks are fp32.  The results are NOT
 * bit-identical to kq_gemv_multix_dev: every output is within
 * 2e-6 * sum_k |w_k x_k| of it (measured at most 6.6e-8 at the 27B shapes).
 * No counterpart in the reference, whose multix must equal the
 * single-stream result (stratum_linear.h:963-966); this is the opt-in
 * dense-contraction path for large B.  x must be finite.  The workspace is
 * the library's, one per stream, grown on the first call of a larger shape
 * on that stream (hipMalloc / hipFree, which synchronise the device) unless
 * reserved beforehand (kq_reserve_mfma_workspace); callers that cannot
 * allocate at all use kq_gemv_multix_mfma_noalloc_dev. */
int kq_gemv_multix_mfma_dev(int type, const void* w, const float* xs, float* ys,
                            int B, int N, int K, kq_stream stream);

/* Bytes of the library workspace kq_gemv_multix_mfma_dev uses for (type, B,
 * N, K), or -1.  No counterpart in the reference. */
int64_t kq_gemv_multix_mfma_workspace_bytes(int type, int B, int N, int K);

/* Grows the matrix-core workspace of the default stream (stream 0) and of
 * every stream the library has run device entries on to at least `bytes`
 * now (hipMalloc, which synchronises the device), so that later calls whose
 * workspace fits allocate nothing: for callers that set up once and then
 * enqueue only (graph capture of the calls, serving loops).  A stream first
 * used later gets at least `bytes` at its first call, so such a caller makes
 * one call on each of its streams before it stops allocating.  No workspace
 * is shrunk before kq_linear_shutdown.  No counterpart in the reference.
 * Returns 0, or -1 with a message. */
int kq_reserve_mfma_workspace(int64_t bytes);

/* Bytes of device scratch the library holds: the matrix-core workspace, the
 * MoE grouping records and the host-pointer entry points' staging buffers
 * (the uploads of kq_linear_init not included).  No counterpart in the
 * reference. */
int64_t kq_scratch_bytes(void);

/* kq_gemv_multix_mfma_dev without any allocation: the same kernels and the
 * same results bit for bit, with the workspace (x planes, x sums and
 * exponents, partial sums of shared row blocks) in a static device array of KQ_NOALLOC_SCRATCH_BYTES that
 * each GPU holds for the life of the process.  No counterpart in the
 * reference; it is for callers that cannot allocate device memory (code
 * under HIP graph capture, allocation-free serving loops).  Calls no
 * hipMalloc/hipFree and creates no stream; returns -1 with a message when
 * the workspace of (type, B, N, K) exceeds the array (the 27B MULTISEQ
 * shapes up to B = 64 fit).  Every call on one GPU shares that GPU's array:
 * calls that overlap in time on one GPU race (calls on one stream are
 * ordered). */
#define KQ_NOALLOC_SCRATCH_BYTES (32L << 20)
int kq_gemv_multix_mfma_noalloc_dev(int type, const void* w, const float* xs, float* ys,
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

/* ----------------------------------------------------------- MoE gather
 * Expert-stacked tensors (GGUF [K_in, N_out, E]: expert e's slice is bytes
 * [offset + e*slice, +slice)) and .moep packs (per layer and expert, the
 * gate|up|down slices contiguous), as addressed by
 * stratum_arch_moe.inc.c:220-337, and the routed expert GEMVs of
 * moe_forward_block / moe_forward_b (:605-755, :817-1267). */

#define KQ_MOE_MAX_EXPERTS 4096
#define KQ_MOE_MAX_TOKENS 64

/* Bytes of one expert slice of a stacked tensor.  Replaces moe_slice_bytes
 * (stratum_arch_moe.inc.c:220-238): nbytes / (nelem / (K_in * N_out)), the
 * block size formula when nbytes or nelem is unset, and the fixed formulas
 * of the W16 types 43 and 44.  -1 for an unknown type without sizes. */
int64_t kq_moe_slice_bytes(const kq_tensor* t, int K_in, int N_out);

/* Descriptor of one expert slice: *dst = *t with nelem = K_in * N_out,
 * nbytes = slice and offset moved to expert e's slice of the stacked
 * tensor or, when slice_host != NULL, to that host address (a pack slice)
 * relative to base.  Replaces moe_bind_slice (stratum_arch_moe.inc.c:327-337);
 * the result goes to kq_linear_dispatch like any tensor. */
void kq_moe_bind_slice(kq_tensor* dst, const kq_tensor* t, int e, int64_t slice, int N_out,
                       int K_in, const uint8_t* slice_host, const uint8_t* base);

/* The .moep header (MoePackHdr, stratum_arch_moe.inc.c:245-259): packed,
 * little-endian, 68 bytes. */
#pragma pack(push, 1)
typedef struct kq_moe_pack_hdr {
    char     magic[4];
    uint32_t version, n_layers, n_experts, n_embed, n_ff;
    uint32_t gate_type, up_type, down_type;
    uint64_t gate_slice, up_slice, down_slice, data_off;
} kq_moe_pack_hdr;
#pragma pack(pop)

/* A validated pack mapping. */
typedef struct kq_moe_pack {
    const uint8_t* base;
    size_t size;
    uint64_t data_off, gate_slice, up_slice, down_slice, stride;
    uint32_t n_layers, n_experts;
} kq_moe_pack;

/* Checks a pack mapped at [base, base+size) against the model, with the
 * header tests of moe_pack_load (stratum_arch_moe.inc.c:506-525: magic,
 * version, shape, types, slice sizes from the stacked tensors, data_off and
 * total size), and fills *out.  0, or -1 when the pack does not match.
 * The sampled byte comparison the reference then runs against the GGUF
 * (:535-560) is the caller's (it reads both host mappings). */
int kq_moe_pack_open(const uint8_t* base, size_t size, int n_layers, int n_experts, int n_embed,
                     int n_ff, const kq_tensor* gate, const kq_tensor* up,
                     const kq_tensor* down, kq_moe_pack* out);

/* Host address of layer li, expert e, tensor which (0 gate, 1 up, 2 down)
 * in the pack.  Replaces moe_pack_which (stratum_arch_moe.inc.c:307-313). */
const uint8_t* kq_moe_pack_which(const kq_moe_pack* p, int li, int e, int which);

/* Top-K experts of one token's router weights w[0..E): sel[s], selw[s] for
 * s < K in decreasing weight, equal weights in increasing expert id, slots
 * without an expert (w <= -1) left (-1, -1.0f).  Replaces moe_topk
 * (stratum_arch_moe.inc.c:368-385); host code, as in the reference. */
void kq_moe_topk(const float* w, int E, int K, int* sel, float* selw);

/* The same selection on the device for B tokens: probs is B x E (row per
 * token), sel and selw are B x k.  E <= KQ_MOE_MAX_EXPERTS.  0 or -1. */
int kq_moe_topk_dev(const float* probs, int B, int E, int k, int* sel, float* selw,
                    kq_stream stream);

/* One routed expert GEMV of a layer: for every member m = s*k + r (token s,
 * rank r) with expert e = sel[m] and every tensor t < ntensors,
 *   y[t][m*n_out .. +n_out) = W_t(e) . x[(m / x_div)*k_in .. +k_in)
 * where W_t(e) starts at w[t] + e * expert_stride (the stacked slice, or
 * the pack stride).  Gate and up (ntensors 2, x_div k: one x per token)
 * share one launch; down is ntensors 1, x_div 1 (one activation per
 * member).  Each member's y equals kq_gemv_dev on its slice bit for bit.
 * All pointers are device pointers; sel is read on the device (entries
 * outside [0, E) are clamped into it for B == 1 and skipped for B > 1;
 * their y is unspecified, as the reference skips sel < 0 ranks,
 * stratum_arch_moe.inc.c:722-725).  B == 1 runs the single-stream kernel
 * with the expert bases resolved on the device; B > 1 builds the distinct
 * experts' member lists on the device (moe_forward_b's grouping,
 * stratum_arch_moe.inc.c:1130-1205) and streams each selected slice once
 * for all of its tokens.  B <= KQ_MOE_MAX_TOKENS, k <= KQ_MAX_GROUPS.  No
 * counterpart as one call in the reference, which dispatches per slice
 * (moe_dispatch_slice / moe_multix_slice, :596-603, :808-815).
 * Int8 mode (type | KQ_INT8_ACT) at B > 1: moe_forward_b's tickets under
 * use_sdot (:1136-1201): each expert's members in increasing m, cut into
 * tickets of at most 8; for Q4_K / Q6_K a member of a ticket of two or more
 * equals kq_gemv_multix_dev over exactly that ticket's members (the multix
 * pack arithmetic), a member of a ticket of one equals kq_gemv_dev; for
 * Q5_K, Q3_K and Q8_0 (per-stream multix) every member equals kq_gemv_dev.
 * This path uses the library's matrix-core scratch (grown on first use). */
typedef struct kq_moe_op {
    int type, n_out, k_in;
    int ntensors;
    const void* w[2];
    int64_t expert_stride;
    const float* x;
    int x_div;
    float* y[2];
} kq_moe_op;
int kq_moe_gemv_dev(const kq_moe_op* op, const int* sel, int B, int k, int E, kq_stream stream);

/* Routed and gathered in one launch: the top-k of each token's router
 * weights probs[B][E] (E <= 1024; the rule of kq_moe_topk) is taken inside
 * the launch that runs op, written to sel[B*k] / selw[B*k] (device memory)
 * as kq_moe_topk_dev writes them, and used as kq_moe_gemv_dev(op, sel, B,
 * k, E) uses them -- the same outputs bit for bit, one launch fewer.  A
 * larger batch (B x E^2 above 2^16, E rounded up to 64: ranking in every
 * workgroup would cost more than the launch it saves) or one whose router
 * weights do not fit in the launch's LDS is routed by a separate top-k
 * launch first, with the same results.  The usual call is the gate+up op; the down
 * op then takes sel.  No counterpart in the reference, which routes on the
 * host (moe_topk, stratum_arch_moe.inc.c:368-385) before the per-slice
 * dispatch. */
int kq_moe_gemv_routed_dev(const kq_moe_op* op, const float* probs, int B, int k, int E, int* sel,
                           float* selw, kq_stream stream);

/* ---------------------------------------------------- MoE FFN step
 * The pieces around the gather that make it the whole expert FFN step of
 * the reference's MoE decode (stratum_arch_moe.inc.c:689-743 for one token,
 * 1107-1226 for a batch).  Device pointers, enqueue only. */

/* Softmax of B rows of E values in place: stratum_softmax_inplace
 * (stratum_engine.h:395-423, its scalar path): max by the sequential scan,
 * expf(x - max), the binary64 sum in index order, inv = (float)(1.0 / sum),
 * x * inv.  expf is the device's (within one ulp of correctly rounded
 * exp; the reference calls the host libm's), so probabilities agree with
 * the reference's to a few binary32 ulps, not bit for bit.  E <=
 * KQ_MOE_MAX_EXPERTS. */
int kq_softmax_dev(float* x, int B, int E, kq_stream stream);

/* SwiGLU y = (g / (1 + expf(-g))) * u over n values: stratum_swiglu
 * (stratum_engine.h:373-392, its scalar loop), binary32 with the device
 * expf (same caveat).  g, u, y 16-byte aligned. */
int kq_swiglu_dev(const float* g, const float* u, float* y, int64_t n, kq_stream stream);

/* Rank-ordered weighted accumulate plus the residual
 * (stratum_arch_moe.inc.c:728-743; batches :1213-1226): for token s < B,
 * x[s][i] = resid[s][i] + (((0 + selw[s][0] o[s*k][i]) + selw[s][1]
 * o[s*k+1][i]) + ...), ranks with sel < 0 skipped, every product and sum
 * rounded in binary32 -- bit-identical to the reference's loop.  o holds
 * B*k rows of H (member m = s*k + r), x may equal resid.  H % 4 == 0. */
int kq_moe_combine_dev(const float* o, const int* sel, const float* selw, const float* resid,
                       float* x, int B, int k, int H, kq_stream stream);

/* One MoE layer's expert tensors: the router (ffn_gate_inp, n_experts rows
 * of n_embed, any GEMV type; F32 in the usual GGUF) and expert 0's slice
 * of each stacked expert tensor with the byte stride between experts
 * (kq_moe_slice_bytes, or the pack stride). */
typedef struct kq_moe_ffn {
    int n_embed, n_ff, n_experts, k;
    int router_type;
    const void* router;
    int gate_type, up_type, down_type;
    const void* gate;
    const void* up;
    const void* down;
    int64_t gate_stride, up_stride, down_stride;
} kq_moe_ffn;

/* Bytes of device workspace kq_moe_ffn_dev needs for B tokens, or -1. */
int64_t kq_moe_ffn_workspace_bytes(const kq_moe_ffn* f, int B);

/* The expert FFN step for B tokens: router logits of xn (B x n_embed, the
 * normed hidden state), softmax, top-k (sel, selw: B x k, written), gate
 * and up of each selected slice, SwiGLU, down, and x = x + the rank-ordered
 * weighted sum (x: B x n_embed, the residual stream, updated in place).
 * The GEMVs follow the per-slice contract of kq_moe_gemv_dev; expf-based
 * steps as above.  No allocation: work is caller-provided device memory of
 * kq_moe_ffn_workspace_bytes.  B <= KQ_MOE_MAX_TOKENS, k <= KQ_MAX_GROUPS,
 * n_embed and n_ff multiples of 256.  Replaces the FFN half of
 * moe_forward_one_token / moe_forward_b after moe_rmsnorm.  At B = 1 (gate,
 * up and down of k-quant block types or Q8_0, exact or in the int8 mode;
 * gate and up of one type and stride, 2k <= KQ_MAX_GROUPS, n_experts <=
 * 256, n_embed and n_ff multiples of the CU count) the step runs in three
 * launches with the same results; the workspace then holds the
 * activations but not the probabilities or the gate, up and down outputs.
 * At B > 1 (block types of the multi-x kernel: every exact block type, and
 * Q5_K, Q3_K, Q8_0 in the int8 mode) the grouped gate+up launch stores
 * its expert-run tables in the workspace and the down launch loads them
 * instead of grouping the selection again, with the same results.  Where
 * a launch groups the selection in a launch of its own (run tables too
 * large for LDS, or KQ_MOE_GROUP_LAUNCH), the group records also go to the
 * workspace; so do, for int8 Q4_K / Q6_K experts (type | KQ_INT8_ACT) at
 * B > 1, the quantized rows and tickets of moe_forward_b's ticket batch
 * (kq_moe_gemv_dev): the step never touches the library's scratch. */
int kq_moe_ffn_dev(const kq_moe_ffn* f, const float* xn, float* x, int B, int* sel, float* selw,
                   void* work, int64_t work_bytes, kq_stream stream);

/* What the last kq_moe_ffn_dev call ran, as bits (0 after a failure):
 * KQ_FFN_FUSED_B1 the three-launch batch-1 form; KQ_FFN_RUNS_STORED the
 * gate+up launch stored its run tables; KQ_FFN_RUNS_LOADED a later launch
 * loaded them; KQ_FFN_GROUP_LAUNCH a separate grouping launch wrote its
 * records to the workspace.  No counterpart in the reference: for callers
 * and tests that check which form a layer shape takes. */
#define KQ_FFN_FUSED_B1 1
#define KQ_FFN_RUNS_STORED 2
#define KQ_FFN_RUNS_LOADED 4
#define KQ_FFN_GROUP_LAUNCH 8
int kq_moe_ffn_last_path(void);

#ifdef __cplusplus
}
#endif
#endif /* KQ_GEMV_H */
