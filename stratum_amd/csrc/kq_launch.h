/*
 * kq_launch.h -- the launchers of kq_kernels.hip as the host layer
 * (kq_linear.c) calls them.  Internal to the library (not installed);
 * included by both sides so that the two agree on every signature.
 */
#ifndef KQ_LAUNCH_H
#define KQ_LAUNCH_H

#include <hip/hip_runtime_api.h>

#include "../../include/kq_gemv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* launchers (kq_kernels.hip).  A launcher segment has nparts parts; part p
 * is rows[p] rows at w[p] writing y[p] (+ add[p]), reading x, or
 * x + p * x_stride when x_stride != 0. */
typedef struct {
    const void* w[KQ_MAX_GROUPS];
    float* y[KQ_MAX_GROUPS];
    const float* add[KQ_MAX_GROUPS];
    int rows[KQ_MAX_GROUPS];
    const float* x;
    int type, K, nparts, x_stride;
    const int* sel;          /* MoE gather: part p uses expert sel[p % ksel] */
    long estride;            /* bytes per expert */
    int ksel, emax;
    const float* probs;      /* routed in the launch: top-ksel of probs[0..emax), */
    int* sel_out;            /* written by workgroup 0 to sel_out / selw_out */
    float* selw_out;
    /* MoE FFN step pieces (first segment of a one-segment selection launch;
     * zero: unused) */
    int logits;              /* probs holds router logits: their softmax first */
    float* act;              /* parts = k gate then k up slices of one token:
                              * act[r][i] = SwiGLU(gate_r[i], up_r[i]) (no y written) */
    float* cx;               /* parts = one token's ranks: cx[i] += the sum over parts r
                              * with sel[r] >= 0, in order, of cw[r] * row i of part r */
    const float* cw;         /*   (no y written) */
} kqk_seg;
#define KQK_LIST_MAX 4   /* parts of unequal sizes one launcher segment takes */
long kqk_segs_lds(const kqk_seg* segs, int nseg, int grid, int* xs_off, int* terms_off,
                  int* scr_off);
int kqk_launch_segs(const kqk_seg* segs, int nseg, int grid, int threads, int depth,
                    long lds_bytes, int xs_off, int terms_off, int scr_off, hipStream_t st);
int kqk_launch_dequant(int type, const void* w, float* y, long nblocks, hipStream_t st);
/* dense F16 / F32 rows (types 1 / 0): y = W x (+ add) on `grid` workgroups */
int kqk_launch_dense(int type, const void* w, const float* x, const float* add, float* y, int N,
                     int K, int B, int grid, hipStream_t st);
/* Q2_K -> type-42 block permutation */
int kqk_launch_q2k_to_nib(const void* q2k, void* nib, long nblocks, hipStream_t st);
/* MoE FFN step pieces */
int kqk_launch_softmax(float* x, int B, int E, hipStream_t st);
int kqk_launch_swiglu(const float* g, const float* u, float* y, long n, hipStream_t st);
int kqk_launch_moe_combine(const float* o, const int* sel, const float* selw, const float* resid,
                           float* x, int B, int k, int H, hipStream_t st);
int kqk_dense_set_max_lds(int bytes);
/* x -> int8 per group (32 or 16), scales, integer sums (xsum may be NULL) */
int kqk_launch_quantize_q8(const float* x, int K, int group, int8_t* xq, float* xscale, int* xsum,
                           hipStream_t st);
int kqk_set_max_lds(int bytes);
/* multi-x launcher: plan[] = threads, S, RB, nblk, TC, sums bytes, x buffer
 * bytes, members staged together (kqk_mx_plan returns the LDS bytes, or
 * -1); gdev == NULL launches one inline group of M members (x_j = X + j
 * x_stride, y_j = Y + j y_stride) */
#define KQK_MX_PLAN 8
long kqk_mx_plan(int type, int N, int K, int mmax, int ngmax, int grid, int lds_max, int* plan,
                 const float* ngm);
int kqk_launch_mx(int type, const int* plan, long lds, int grid, const void* w, int M,
                  const void* gdev, const int* ngdev, const float* X, long x_stride, float* Y,
                  long y_stride, int N, int K, hipStream_t st);
int kqk_mx_set_max_lds(int bytes);
/* MoE: top-k per token; the expert groups (MxGroup records) of a selection */
int kqk_launch_moe_topk(const float* probs, int B, int E, int k, int* sel, float* selw,
                        hipStream_t st);
long kqk_mx_group_bytes(void);
long kqk_moe_runs_lds(int nm, int E, int ndmax, int B);
int kqk_launch_mx_moe(int type, const int* plan, long plan_lds, long lds, int grid, const int* sel,
                      int nm, int E, int nt, int x_div, const void* w0, const void* w1, float* y0,
                      float* y1, long estride, const float* X, int N, int K, const float* probs,
                      int B, int k, int* sel_out, float* selw_out, int* runs_out,
                      const int* runs_in, hipStream_t st);
/* ints of a stored run table (count first) for nm members, E experts and
 * at most ndmax runs */
long kqk_moe_runs_words(int nm, int E, int ndmax);
/* MFMA multi-x (Q4_K, Q6_K): workspace sizes for a launch over `grid`
 * workgroups, and the launch (the same grid) */
int kqk_mfma_workspace(int type, int B, int N, int K, int grid, long* planes, long* xs, long* part);
/* Bytes of the library's static device scratch (the public limit). */
#define KQK_NOALLOC_BYTES KQ_NOALLOC_SCRATCH_BYTES
/* Device address (on the current device) and size of the library's static
 * scratch array; the address is looked up once per device and cached. */
int kqk_noalloc_scratch(void** ptr, long* bytes);
int kqk_launch_mfma(int type, const float* x, const void* w, float* y, int B, int N, int K,
                    void* planes, float* xs, float* part, int grid, hipStream_t st);
/* int8 MULTISEQ on the matrix cores (Q4_K / Q6_K | KQ_INT8_ACT, B >= 2):
 * workspace bytes (*cf_off: offset of the coefficients), or -1; the
 * launch (prep + main kernel) with ws 256-byte aligned; ks: K-parts per
 * row block (1, 2, 4 or 8; anything else: kqk_mi8_parts(K), the rule the
 * library uses -- the grouping of the binary64 sums follows it) */
long kqk_mi8_workspace(int type, int B, int K, long* cf_off);
int kqk_mi8_parts(int K);
int kqk_launch_mi8(int type, const float* xs, long x_stride, const void* w, float* ys,
                   long y_stride, int B, int N, int K, void* ws, int ks, hipStream_t st);
long kqk_mi8_moe_workspace(int type, int nx, int K);
int kqk_launch_mi8_moe(int type, const int* sel, int nm, int E, int nt, int x_div,
                       const void* w0, const void* w1, float* y0, float* y1, long estride,
                       const float* x, int K, void* groups, int* ng, int ngmax, int N,
                       void* ws, int n_cu, hipStream_t st);
int kqk_launch_moe_group(const int* sel, int nm, int E, int nt, int x_div, int mch,
                         const void* w0, const void* w1, float* y0, float* y1, long estride,
                         void* groups, int* ng, hipStream_t st);

#ifdef __cplusplus
}
#endif
#endif /* KQ_LAUNCH_H */
