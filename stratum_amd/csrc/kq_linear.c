/*
 * kq_linear.c -- host side of the k-quant GEMV library (C11).
 *
 * Mirrors the reference's linear-dispatch layer (stratum_linear.h): one
 * global state, a weight base that tensor offsets resolve against, a
 * per-type dispatch that returns -1 for types it cannot run, and the
 * st_linear_dispatch / _add / multix / st_q4k_group entry points with the
 * reference's argument order.  Differences, all forced by the device:
 *   - the weight mapping is uploaded to HBM once (kq_linear_init) and
 *     offsets resolve to the device copy;
 *   - host-pointer calls copy x in and y out around the kernel;
 *   - device-pointer calls (kq_*_dev) only enqueue work on a stream.
 * The kernels themselves live in kq_kernels.hip behind kqk_* launchers.
 */
#define _GNU_SOURCE
#include "../../include/kq_gemv.h"
#include "../../include/kq_gguf.h"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kq_launch.h"

#define KQ_MAX_REGIONS 16
#define KQ_SCR_SLOTS 16    /* streams with their own device-entry scratch */

/* one stream's scratch: MoE group records + their count; the matrix-core
 * workspace (x planes, sums, partials; int8 rows and coefficients) */
typedef struct {
    hipStream_t st;
    int used;
    unsigned long long last;   /* the call count at its last use */
    float* moe; size_t cap_moe;
    uint8_t* mf; size_t cap_mf;
} kq_scr;

typedef struct {
    const uint8_t* host;
    size_t size;
    uint8_t* dev;
} kq_region;

typedef struct {
    int ready;             /* device queried */
    int device;
    int n_cu;
    int lds_max;           /* bytes of LDS one workgroup may use */
    hipStream_t stream;    /* library stream of the host-pointer ABI (default
                            * priority), created at its first use */
    int stream_ready;
    kq_region reg[KQ_MAX_REGIONS];
    int nreg;
    const uint8_t* base;   /* kq_linear_init base: offsets resolve here */
    /* staging for the host-pointer ABI */
    float* d_x; size_t cap_x;
    float* d_y; size_t cap_y;
    float* d_a; size_t cap_a;
    kq_scr scr[KQ_SCR_SLOTS];       /* the device entries' scratch, per stream */
    unsigned long long scr_calls;   /* scr_of calls, for the least recently used */
    size_t mf_reserve;              /* kq_reserve_mfma_workspace: least mf size */
    /* launch overrides from the environment (0: unset), read by kq_ready
     * and again only by kq_tuning_reload: the planner runs on every call */
    int env_grid, env_threads, env_depth, env_moe_group_launch, env_ffn_split;
    int use_sdot;          /* host-pointer ABI: Q4_K / Q6_K in the int8 mode */
    char err[512];
} kq_state;

static kq_state g_kq;


/* shared with kq_gguf.c; not exported */
__attribute__((visibility("hidden"))) int kq_fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_kq.err, sizeof g_kq.err, fmt, ap);
    va_end(ap);
    fprintf(stderr, "kq: %s\n", g_kq.err);
    return -1;
}

const char* kq_last_error(void) { return g_kq.err; }

/* The scratch of the device entries that stream `st` runs on: calls on
 * different streams get different buffers (they may overlap in time),
 * calls on one stream are ordered.  A stream first seen when all
 * KQ_SCR_SLOTS sets are taken gets the least recently used one, whose
 * buffers are freed first (hipFree waits for the device, so no launch
 * still reads them). */
static kq_scr* scr_of(hipStream_t st) {
    const unsigned long long now = ++g_kq.scr_calls;
    for (int i = 0; i < KQ_SCR_SLOTS; i++)
        if (g_kq.scr[i].used && g_kq.scr[i].st == st) {
            g_kq.scr[i].last = now;
            return &g_kq.scr[i];
        }
    int pick = -1;
    for (int i = 0; i < KQ_SCR_SLOTS && pick < 0; i++)
        if (!g_kq.scr[i].used) pick = i;
    if (pick < 0) {
        pick = 0;
        for (int i = 1; i < KQ_SCR_SLOTS; i++)
            if (g_kq.scr[i].last < g_kq.scr[pick].last) pick = i;
        kq_scr* v = &g_kq.scr[pick];
        if (v->moe) (void)hipFree(v->moe);
        if (v->mf) (void)hipFree(v->mf);
        memset(v, 0, sizeof *v);
    }
    g_kq.scr[pick].used = 1;
    g_kq.scr[pick].st = st;
    g_kq.scr[pick].last = now;
    return &g_kq.scr[pick];
}

/* the types with an int8-activation (SDOT) form: st_linear_q4k, _q6k,
 * _q5k, _q3k and _q8_0 under g_st.use_sdot (stratum_linear.h:369-489) */
static int has_sdot(int type) {
    return type == KQ_TYPE_Q4_K || type == KQ_TYPE_Q6_K || type == KQ_TYPE_Q5_K ||
           type == KQ_TYPE_Q3_K || type == KQ_TYPE_Q8_0;
}

/* bytes per 256 weights (stratum_gguf.h:57-79; Q8_0: eight 34-byte blocks);
 * the int8-activation mode (KQ_INT8_ACT) keeps the blocks */
static int block_bytes(int type) {
    if ((type & KQ_INT8_ACT) && has_sdot(type & ~KQ_INT8_ACT)) type &= ~KQ_INT8_ACT;
    switch (type) {
    case KQ_TYPE_F32: return 1024;
    case KQ_TYPE_F16: return 512;
    case KQ_TYPE_Q8_0: return 272;
    case KQ_TYPE_Q2_K: return 84;
    case KQ_TYPE_Q3_K: return 110;
    case KQ_TYPE_Q4_K: return 144;
    case KQ_TYPE_Q5_K: return 176;
    case KQ_TYPE_Q6_K: return 210;
    case KQ_TYPE_Q2K_NIB: return 148;
    default: return 0;
    }
}

/* dense rows (their own kernel) */
static int is_dense(int type) { return type == KQ_TYPE_F16 || type == KQ_TYPE_F32; }

/* Q4_K / Q6_K in the int8 mode: the types whose st_linear_multix under
 * use_sdot has its own (pack) arithmetic at B >= 2, and which share a
 * launch in a group (st_mixed_fused_sdot) */
static int is_i8mx(int type) {
    return type == (KQ_INT8_ACT | KQ_TYPE_Q4_K) || type == (KQ_INT8_ACT | KQ_TYPE_Q6_K);
}

/* the four types of the fused batch-1 MoE FFN step */
static int is_core(int type) {
    return type == KQ_TYPE_Q2_K || type == KQ_TYPE_Q4_K || type == KQ_TYPE_Q6_K ||
           type == KQ_TYPE_Q2K_NIB;
}

/* the types the batch-1 three-launch FFN step takes: every block type of
 * the gather kernel (the four above, Q5_K, Q3_K, Q8_0) and the int8 mode
 * of the five SDOT types (moe_forward_one_token's per-slice
 * st_linear_dispatch under use_sdot: the single-stream int8 forms, which
 * the gather kernel's int8 instantiations compute) */
static int is_ffn_b1(int type) {
    const int t = type & ~KQ_INT8_ACT;
    if (type & KQ_INT8_ACT) return has_sdot(t);
    return is_core(t) || t == KQ_TYPE_Q5_K || t == KQ_TYPE_Q3_K || t == KQ_TYPE_Q8_0;
}

/* the types the multi-x (MULTISEQ, MoE batch) kernel covers: every block
 * type, and the int8 mode of Q5_K, Q3_K and Q8_0 (whose batches are per
 * stream in the reference, so every member takes the single-stream int8
 * values); int8 Q4_K / Q6_K and the dense types have their own paths */
static int is_mx(int type) {
    const int t = type & ~KQ_INT8_ACT;
    if (type & KQ_INT8_ACT)
        return t == KQ_TYPE_Q5_K || t == KQ_TYPE_Q3_K || t == KQ_TYPE_Q8_0;
    return is_core(t) || t == KQ_TYPE_Q5_K || t == KQ_TYPE_Q3_K || t == KQ_TYPE_Q8_0;
}

int64_t kq_row_bytes(int type, int K) {
    int bb = block_bytes(type);
    if (!bb || K <= 0 || K % 256) return -1;
    return (int64_t)(K / 256) * bb;
}

static int hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return 0;
    return kq_fail("%s: %s", what, hipGetErrorString(e));
}

static int env_int(const char* name) {
    const char* e = getenv(name);
    return e ? atoi(e) : 0;
}

int kq_tuning_reload(void) {
    const int t = env_int("KQ_WG_THREADS"), d = env_int("KQ_DEPTH");
    g_kq.env_grid = env_int("KQ_GRID") > 0 ? env_int("KQ_GRID") : 0;
    g_kq.env_threads = t == 256 || t == 512 || t == 1024 ? t : 0;
    g_kq.env_depth = getenv("KQ_DEPTH") ? (d == 2 ? 2 : 1) : 0;
    g_kq.env_moe_group_launch = getenv("KQ_MOE_GROUP_LAUNCH") != NULL;
    g_kq.env_ffn_split = getenv("KQ_MOE_FFN_SPLIT") != NULL;
    return 0;
}

static int kq_ready(void) {
    if (g_kq.ready) return 0;
    kq_tuning_reload();
    int dev = 0, n = 0;
    if (hip_ok(hipGetDeviceCount(&n), "hipGetDeviceCount")) return -1;
    if (n < 1) return kq_fail("no HIP device");
    if (hip_ok(hipGetDevice(&dev), "hipGetDevice")) return -1;
    int ncu = 0, lds = 0;
    if (hip_ok(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev),
               "hipDeviceGetAttribute(CU count)")) return -1;
    if (hip_ok(hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev),
               "hipDeviceGetAttribute(LDS)")) return -1;
    g_kq.device = dev;
    g_kq.n_cu = ncu > 0 ? ncu : 1;
    g_kq.lds_max = lds > 0 ? lds : 65536;
    if (kqk_set_max_lds(g_kq.lds_max) != 0 || kqk_mx_set_max_lds(g_kq.lds_max) != 0 ||
        kqk_dense_set_max_lds(g_kq.lds_max) != 0)
        return kq_fail("cannot raise the LDS limit");
    /* the static scratch of the no-allocation entry point: its address on
     * this device, looked up once now (other devices at their first call) */
    void* scr = NULL;
    long scr_bytes = 0;
    const int e = kqk_noalloc_scratch(&scr, &scr_bytes);
    if (e) return kq_fail("static scratch: %s", hipGetErrorString((hipError_t)e));
    g_kq.ready = 1;
    return 0;
}

/* The library's own stream, used only by the host-pointer entry points
 * (created at their first call: the device-pointer entry points create
 * nothing).  A blocking stream at the default priority, so it orders with
 * the null stream. */
static int host_stream(void) {
    if (g_kq.stream_ready) return 0;
    if (hip_ok(hipStreamCreate(&g_kq.stream), "hipStreamCreate")) return -1;
    g_kq.stream_ready = 1;
    return 0;
}

/* ------------------------------------------------------------ regions */

static void drop_region(int i) {
    if (g_kq.reg[i].dev) (void)hipFree(g_kq.reg[i].dev);
    g_kq.reg[i] = g_kq.reg[--g_kq.nreg];
}

int kq_register_region(const void* host, size_t size) {
    if (!host || !size) return kq_fail("kq_register_region: empty mapping");
    if (kq_ready()) return -1;
    for (int i = 0; i < g_kq.nreg; i++)
        if (g_kq.reg[i].host == host && g_kq.reg[i].size == size) return 0;
    if (g_kq.nreg == KQ_MAX_REGIONS) return kq_fail("kq_register_region: too many mappings");
    uint8_t* dev = NULL;
    if (hip_ok(hipMalloc((void**)&dev, size), "hipMalloc(weights)")) return -1;
    if (hip_ok(hipMemcpy(dev, host, size, hipMemcpyHostToDevice), "upload weights")) {
        (void)hipFree(dev);
        return -1;
    }
    kq_region* r = &g_kq.reg[g_kq.nreg++];
    r->host = (const uint8_t*)host;
    r->size = size;
    r->dev = dev;
    return 0;
}

int kq_linear_init(const uint8_t* base, size_t size) {
    if (kq_ready()) return -1;
    if (g_kq.base) {
        for (int i = 0; i < g_kq.nreg; i++)
            if (g_kq.reg[i].host == g_kq.base) { drop_region(i); break; }
        g_kq.base = NULL;
    }
    if (kq_register_region(base, size)) return -1;
    g_kq.base = base;
    return 0;
}

const void* kq_device_ptr(const void* host, size_t nbytes) {
    const uint8_t* h = (const uint8_t*)host;
    for (int i = 0; i < g_kq.nreg; i++) {
        const kq_region* r = &g_kq.reg[i];
        if (h >= r->host && (size_t)(h - r->host) <= r->size &&
            nbytes <= r->size - (size_t)(h - r->host))
            return r->dev + (h - r->host);
    }
    return NULL;
}

void kq_linear_shutdown(void) {
    while (g_kq.nreg) drop_region(g_kq.nreg - 1);
    if (g_kq.d_x) (void)hipFree(g_kq.d_x);
    if (g_kq.d_y) (void)hipFree(g_kq.d_y);
    if (g_kq.d_a) (void)hipFree(g_kq.d_a);
    for (int i = 0; i < KQ_SCR_SLOTS; i++) {
        if (g_kq.scr[i].moe) (void)hipFree(g_kq.scr[i].moe);
        if (g_kq.scr[i].mf) (void)hipFree(g_kq.scr[i].mf);
    }
    if (g_kq.stream_ready) (void)hipStreamDestroy(g_kq.stream);
    memset(&g_kq, 0, sizeof g_kq);
}

static int grow(float** p, size_t* cap, size_t nfloats) {
    if (*cap >= nfloats) return 0;
    if (*p) (void)hipFree(*p);
    *p = NULL;
    *cap = 0;
    size_t n = nfloats < 4096 ? 4096 : nfloats;
    if (hip_ok(hipMalloc((void**)p, n * sizeof(float)), "hipMalloc(staging)")) return -1;
    *cap = n;
    return 0;
}

/* Device address of tensor w's rows: g_st.mmap_base + offset
 * (stratum_linear.h:169-188) resolved through the registered mappings. */
static const void* tensor_dev(const kq_tensor* w, int N, int K) {
    if (!w) { kq_fail("NULL tensor"); return NULL; }
    if (!g_kq.base) { kq_fail("kq_linear_init was not called"); return NULL; }
    int64_t rb = kq_row_bytes((int)w->type, K);
    if (rb < 0) { kq_fail("type %u / K %d not supported", w->type, K); return NULL; }
    const uint8_t* h = g_kq.base + w->offset;
    const void* d = kq_device_ptr(h, (size_t)rb * (size_t)N);
    if (!d) kq_fail("tensor %s: [offset %llu, +%lld) outside the registered weights",
                    w->name ? w->name : "?", (unsigned long long)w->offset,
                    (long long)rb * N);
    return d;
}

/* ----------------------------------------------------------- planning */
/* One persistent workgroup per CU (KQ_GRID overrides), one batch of loads
 * in flight per wave (KQ_DEPTH=2 overrides, for workgroups of at most 512
 * lanes).  The workgroup size follows the largest per-workgroup share of
 * 64-weight chunks over the segments: 1024 lanes above 512 chunks, else
 * 512 (KQ_WG_THREADS overrides: 256, 512 or 1024).  Measured in one
 * process over shares of 128-4096 chunks (K = 1024, 2048, 5120) against
 * 256 or 512 lanes with two batches in flight and two 512-lane workgroups
 * per CU: this rule was the fastest at every share measured, e.g. the
 * 27B Q/K/V group (2560 chunks) 10.1 -> 9.3 us, 1600 chunks 7.3 -> 6.7
 * us, 800 chunks 6.6 -> 5.6 us. */
static int plan_grid(void) {
    return g_kq.env_grid > 0 ? g_kq.env_grid : g_kq.n_cu;
}

static long max_share(const kqk_seg* segs, int nseg, int grid) {
    long chunks = 0;
    for (int i = 0; i < nseg; i++) {
        long n = 0;
        for (int p = 0; p < segs[i].nparts; p++) n += segs[i].rows[p];
        const long c = ((n + grid - 1) / grid) * (segs[i].K / 64);
        if (c > chunks) chunks = c;
    }
    return chunks;
}

static int plan_threads(const kqk_seg* segs, int nseg, int grid) {
    if (g_kq.env_threads) return g_kq.env_threads;
    return max_share(segs, nseg, grid) > 512 ? 1024 : 512;
}

static int plan_depth(void) {
    return g_kq.env_depth ? g_kq.env_depth : 1;
}

static int launch_segs_one(const kqk_seg* segs, int nseg, hipStream_t st);

/* Whether one kernel instantiation takes segments of types a and b
 * together: Q4_K and Q6_K (a Q4_K_M layer's mix), in the exact or the int8
 * mode (as st_mixed_fused_sdot, stratum_linear.h:1043-1085); else one
 * type. */
static int is_q46(int type) { return type == KQ_TYPE_Q4_K || type == KQ_TYPE_Q6_K; }

static int same_launch(int a, int b) {
    if (is_q46(a)) return is_q46(b);
    if (is_i8mx(a)) return is_i8mx(b);
    return a == b;
}

/* One launch per run of consecutive segments that one kernel instantiation
 * takes (same_launch).  The segments are independent, so splitting changes
 * no result. */
static int launch_segs(const kqk_seg* segs, int nseg, hipStream_t st) {
    int i = 0;
    while (i < nseg) {
        int j = i + 1;
        while (j < nseg && same_launch(segs[i].type, segs[j].type)) j++;
        if (launch_segs_one(segs + i, j - i, st)) return -1;
        i = j;
    }
    return 0;
}

static int launch_segs_one(const kqk_seg* segs, int nseg, hipStream_t st) {
    const int grid = plan_grid(), threads = plan_threads(segs, nseg, grid), depth = plan_depth();
    for (int i = 0; i < nseg; i++) {   /* the kernel's row arithmetic is 24-bit */
        long n = 0;
        for (int p = 0; p < segs[i].nparts; p++) n += segs[i].rows[p];
        if (n >= (1L << 24))
            return kq_fail("segment %d has %ld rows (at most 2^24 - 1 per launch): split the rows",
                           i, n);
    }
    int xs_off = 0, terms_off = 0, scr_off = 0;
    long lds = kqk_segs_lds(segs, nseg, grid, &xs_off, &terms_off, &scr_off);
    if (lds < 0) return kq_fail("invalid segment list");
    if (lds > g_kq.lds_max)
        return kq_fail("segments need %ld bytes of LDS (max %d): split the rows", lds,
                       g_kq.lds_max);
    int e = kqk_launch_segs(segs, nseg, grid, threads, depth, lds, xs_off, terms_off, scr_off, st);
    if (e) return kq_fail("gemv launch: %s", hipGetErrorString((hipError_t)e));
    return 0;
}

/* Largest row count one launch can give a single segment (LDS limit):
 * the x and xs regions are fixed, the term region grows with the rows per
 * workgroup. */
static int max_rows_per_launch(const kqk_seg* proto) {
    const int grid = plan_grid();
    kqk_seg t = *proto;
    t.nparts = 1;
    t.rows[0] = 1;
    int a, b2, c;
    const long fixed = kqk_segs_lds(&t, 1, grid, &a, &b2, &c) - (long)(t.K / 64) * 8;
    const long per_row = (long)(t.K / 64) * 8;
    long rows = (g_kq.lds_max - fixed) / per_row;      /* rows per workgroup */
    if (rows < 1) rows = 1;
    long n = rows * grid;
    return n > 0x40000000L ? 0x40000000 : (int)n;
}

static hipStream_t pick(kq_stream s) { return (hipStream_t)s; }

/* whether one segment fits one launch's LDS */
static int seg_fits(const kqk_seg* g) {
    int a, b, c;
    const long l = kqk_segs_lds(g, 1, plan_grid(), &a, &b, &c);
    return l > 0 && l <= g_kq.lds_max;
}

static int check_shape(int type, int N, int K) {
    if (!block_bytes(type)) return kq_fail("unsupported type %d", type);
    if (N <= 0 || K <= 0 || K % 256) return kq_fail("bad shape N=%d K=%d (K %% 256 must be 0)", N, K);
    return 0;
}

/* ------------------------------------------------- device-pointer ABI */

/* Dense F16 / F32 rows: their own kernel, one wave per row at a time; B
 * streams share each weight load (each stream's sum in the single-stream
 * order, so ys[s] equals the single call bit for bit). */
static int dense_gemv(int type, const void* w, const float* x, const float* add, float* y, int N,
                      int K, int B, hipStream_t st) {
    if ((uintptr_t)w & 15) return kq_fail("dense GEMV: weights must be 16-byte aligned");
    long g = ((long)N + 3) / 4;
    if (g > 8L * g_kq.n_cu) g = 8L * g_kq.n_cu;
    const int e = kqk_launch_dense(type, w, x, add, y, N, K, B, (int)g, st);
    if (e) return kq_fail("dense gemv launch: %s", hipGetErrorString((hipError_t)e));
    return 0;
}

int kq_gemv_dev(int type, const void* w, const float* x, const float* add, float* y,
                int N, int K, kq_stream stream) {
    if (check_shape(type, N, K) || kq_ready()) return -1;
    if (!w || !x || !y) return kq_fail("kq_gemv_dev: NULL pointer");
    if ((uintptr_t)x & 15) return kq_fail("kq_gemv_dev: x must be 16-byte aligned");
    if (is_dense(type)) return dense_gemv(type, w, x, add, y, N, K, 1, pick(stream));
    kqk_seg sg;
    memset(&sg, 0, sizeof sg);
    sg.type = type; sg.K = K; sg.nparts = 1; sg.x = x;
    const int maxr = max_rows_per_launch(&sg);
    const int64_t rb = kq_row_bytes(type, K);
    for (int r0 = 0; r0 < N; r0 += maxr) {       /* one launch unless LDS runs out */
        const int n = N - r0 < maxr ? N - r0 : maxr;
        sg.w[0] = (const uint8_t*)w + (size_t)r0 * (size_t)rb;
        sg.add[0] = add ? add + r0 : NULL;
        sg.y[0] = y + r0;
        sg.rows[0] = n;
        if (launch_segs(&sg, 1, pick(stream))) return -1;
    }
    return 0;
}

/* Consecutive single-group segments with the same type, K and x are merged
 * into one launcher segment of up to KQK_LIST_MAX parts (while the list
 * still fits the LDS): they are then one row space, swept and reduced
 * together -- one pass of the batch loop instead of one per tensor.  Each
 * row's arithmetic does not change. */
static int try_merge(kqk_seg* h, int nh, const kq_segment* s, int grid) {
    kqk_seg* prev = &h[nh - 1];
    if (s->ngroups != 1 || prev->type != s->type || prev->K != s->K || prev->x != s->x ||
        prev->x_stride != 0 || prev->nparts >= KQK_LIST_MAX)
        return 0;
    const kqk_seg keep = *prev;
    const int p = prev->nparts;
    prev->w[p] = s->w[0];
    prev->y[p] = s->y;
    prev->add[p] = s->add;
    prev->rows[p] = s->rows_per_group;
    prev->nparts = p + 1;
    int a, b, c;
    const long lds = kqk_segs_lds(h, nh, grid, &a, &b, &c);
    if (lds > 0 && lds <= g_kq.lds_max) return 1;
    *prev = keep;
    return 0;
}

int kq_gemv_segments_dev(const kq_segment* segs, int nseg, kq_stream stream) {
    if (nseg < 1 || nseg > KQ_MAX_SEGMENTS) return kq_fail("kq_gemv_segments_dev: nseg=%d", nseg);
    if (!segs || kq_ready()) return segs ? -1 : kq_fail("kq_gemv_segments_dev: NULL");
    kqk_seg h[KQ_MAX_SEGMENTS];
    memset(h, 0, sizeof h);
    int nh = 0;
    const int grid = plan_grid();
    for (int i = 0; i < nseg; i++) {
        const kq_segment* s = &segs[i];
        if (s->ngroups < 1 || s->ngroups > KQ_MAX_GROUPS)
            return kq_fail("segment %d: ngroups=%d", i, s->ngroups);
        if (check_shape(s->type, s->rows_per_group, s->K)) return -1;
        if (!s->x || !s->y) return kq_fail("segment %d: NULL x or y", i);
        if (((uintptr_t)s->x & 15) || (s->x_stride & 3))
            return kq_fail("segment %d: x must be 16-byte aligned", i);
        if ((int64_t)s->rows_per_group * s->ngroups > 0x7fffffff)
            return kq_fail("segment %d: too many rows", i);
        for (int g = 0; g < s->ngroups; g++)
            if (!s->w[g]) return kq_fail("segment %d: NULL weights for group %d", i, g);
        if (is_dense(s->type)) {               /* dense rows: one launch per group */
            for (int g = 0; g < s->ngroups; g++) {
                const float* xg = s->x + (s->ngroups > 1 ? (size_t)g * s->x_stride : 0);
                const size_t o = (size_t)g * s->rows_per_group;
                if (dense_gemv(s->type, s->w[g], xg, s->add ? s->add + o : NULL, s->y + o,
                               s->rows_per_group, s->K, 1, pick(stream)))
                    return -1;
            }
            continue;
        }
        if (nh > 0 && try_merge(h, nh, s, grid)) continue;
        kqk_seg* t = &h[nh++];
        for (int g = 0; g < s->ngroups; g++) {
            t->w[g] = s->w[g];
            t->y[g] = s->y + (size_t)g * s->rows_per_group;
            t->add[g] = s->add ? s->add + (size_t)g * s->rows_per_group : NULL;
            t->rows[g] = s->rows_per_group;
        }
        t->type = s->type; t->K = s->K; t->nparts = s->ngroups;
        t->x = s->x; t->x_stride = s->ngroups > 1 ? s->x_stride : 0;
    }
    return nh ? launch_segs(h, nh, pick(stream)) : 0;
}

/* Multi-x launch plans come from a cost model that scans every row-block
 * count, which costs more host time than a small launch takes on the GPU;
 * a decode loop asks for the same few shapes on every call, so the plans
 * are kept in a small table (replaced round robin).  moe[] is (B, k, E,
 * ntensors) for a MoE batch, zeros otherwise. */
typedef struct {
    int used, type, N, K, mmax, ngmax, grid, lds_max, moe[4];
    long lds;
    int plan[KQK_MX_PLAN];
} mx_plan_entry;
#define MX_PLAN_CACHE 32
static mx_plan_entry g_plans[MX_PLAN_CACHE];
static int g_plan_next;

static long mx_plan(int type, int N, int K, int mmax, int ngmax, int grid, const int moe[4],
                    int lds_max, int* plan) {
    for (int i = 0; i < MX_PLAN_CACHE; i++) {
        const mx_plan_entry* c = &g_plans[i];
        if (c->used && c->type == type && c->N == N && c->K == K && c->mmax == mmax &&
            c->ngmax == ngmax && c->grid == grid && c->lds_max == lds_max &&
            !memcmp(c->moe, moe, sizeof c->moe)) {
            memcpy(plan, c->plan, sizeof c->plan);
            return c->lds;
        }
    }
    long lds;
    if (moe[0] > 0) {
        /* MoE batch of B = moe[0] tokens, k = moe[1] of E = moe[2] experts:
         * under uniform routing an expert is chosen by a token with
         * probability p = k/E, so its member count c is Binomial(B, p); with
         * member lists cut into runs of at most m members the expected
         * number of groups is nt * E * sum_c P(c) ceil(c/m) */
        const int B = moe[0], k = moe[1], E = moe[2], nt = moe[3];
        const double pe = (double)k / E;
        double pc[KQ_MOE_MAX_TOKENS + 1];
        float ngm[17];
        pc[0] = pow(1.0 - pe, B);
        for (int c = 1; c <= B; c++)          /* P(c) from P(c-1): binomial recurrence */
            pc[c] = pe < 1.0 ? pc[c - 1] * (double)(B - c + 1) / c * pe / (1.0 - pe)
                             : (c == B ? 1.0 : 0.0);
        for (int m = 1; m <= 16; m++) {
            double runs = 0.0;
            for (int c = 1; c <= B; c++) runs += pc[c] * (double)((c + m - 1) / m);
            ngm[m] = (float)(nt * E * runs);
        }
        ngm[0] = ngm[1];
        lds = kqk_mx_plan(type, N, K, mmax, ngmax, grid, lds_max, plan, ngm);
    } else {
        lds = kqk_mx_plan(type, N, K, mmax, ngmax, grid, lds_max, plan, NULL);
    }
    mx_plan_entry* c = &g_plans[g_plan_next];
    g_plan_next = (g_plan_next + 1) % MX_PLAN_CACHE;
    c->used = 1; c->type = type; c->N = N; c->K = K; c->mmax = mmax; c->ngmax = ngmax;
    c->grid = grid; c->lds_max = lds_max;
    memcpy(c->moe, moe, sizeof c->moe);
    c->lds = lds;
    memcpy(c->plan, plan, sizeof c->plan);
    return lds;
}

static int mfma_reserve(kq_scr* sc, size_t need);

/* The int8 MULTISEQ of st_linear_multix under use_sdot (Q4_K / Q6_K, B >= 2,
 * stratum_linear.h:732-907): streams quantized into the library's
 * matrix-core workspace, then one weight pass on the matrix cores with the
 * reference's multix_pack arithmetic. */
static int mi8_multix(int type, const void* w, const float* xs, float* ys, int B, int N, int K,
                      hipStream_t st) {
    long cf_off = 0;
    const long need = kqk_mi8_workspace(type, B, K, &cf_off);
    if (need < 0) return kq_fail("int8 multix: bad shape B=%d K=%d", B, K);
    kq_scr* sc = scr_of(st);
    if (!sc || mfma_reserve(sc, (size_t)need)) return -1;
    const int e = kqk_launch_mi8(type, xs, K, w, ys, N, B, N, K, sc->mf, 0, st);
    if (e) return kq_fail("int8 multix launch: %s", hipGetErrorString((hipError_t)e));
    return 0;
}

/* B streams with one pass over the weights per group of up to 64 streams
 * (the multi-x kernel); each stream's y equals its single-stream result bit
 * for bit, except in the int8 mode of Q4_K / Q6_K (mi8_multix). */
int kq_gemv_multix_dev(int type, const void* w, const float* xs, float* ys,
                       int B, int N, int K, kq_stream stream) {
    if (B < 1) return kq_fail("kq_gemv_multix_dev: B=%d", B);
    if (check_shape(type, N, K) || kq_ready()) return -1;
    if (!w || !xs || !ys) return kq_fail("kq_gemv_multix_dev: NULL pointer");
    if ((uintptr_t)xs & 15) return kq_fail("kq_gemv_multix_dev: xs must be 16-byte aligned");
    if (is_dense(type) && B > 1) return dense_gemv(type, w, xs, NULL, ys, N, K, B, pick(stream));
    if (B > 1 && (type == (KQ_INT8_ACT | KQ_TYPE_Q4_K) || type == (KQ_INT8_ACT | KQ_TYPE_Q6_K)))
        return mi8_multix(type, w, xs, ys, B, N, K, pick(stream));
    if (B == 1 || !is_mx(type)) {     /* per-stream launches: the same bits as single calls */
        for (int s = 0; s < B; s++)
            if (kq_gemv_dev(type, w, xs + (size_t)s * K, NULL, ys + (size_t)s * N, N, K, stream))
                return -1;
        return 0;
    }
    const int grid = plan_grid();
    for (int s0 = 0; s0 < B; ) {
        const int nb = B - s0 < 64 ? B - s0 : 64;
        int plan[KQK_MX_PLAN];
        static const int no_moe[4] = {0, 0, 0, 0};
        const long lds = mx_plan(type, N, K, nb, 1, grid, no_moe, g_kq.lds_max, plan);
        if (lds < 0) {
            /* x too long to stage even in 8-chunk tiles: single-stream launches */
            for (int s = s0; s < s0 + nb; s++)
                if (kq_gemv_dev(type, w, xs + (size_t)s * K, NULL, ys + (size_t)s * N, N, K, stream))
                    return -1;
        } else {
            const int e = kqk_launch_mx(type, plan, lds, grid, w, nb, NULL, NULL,
                                        xs + (size_t)s0 * K, K, ys + (size_t)s0 * N, N, N, K,
                                        pick(stream));
            if (e) return kq_fail("multix launch: %s", hipGetErrorString((hipError_t)e));
        }
        s0 += nb;
    }
    return 0;
}

/* B streams on the matrix cores (Q4_K and Q6_K): the tolerance path.  Each
 * super-block's inner product runs as fp16 MFMAs over the weights with
 * their sub-block scales folded in and a two-plane (22-bit) split of x, so
 * results differ from the single-stream ones by a few binary32 ulps of the
 * terms' magnitude (not bit for bit). */
/* Checks an MFMA multi-x call and lays out its workspace (x planes, x
 * sums, K-part partials, each 256-byte aligned): *o_xs, *o_pt are the
 * offsets of the second and third parts, the return value the bytes
 * needed, or 0 after a failure (message set). */
static size_t mfma_prepare(const char* who, int type, const void* w, const float* xs, float* ys,
                           int B, int N, int K, size_t* o_xs, size_t* o_pt) {
    if (type != KQ_TYPE_Q4_K && type != KQ_TYPE_Q6_K) {
        kq_fail("%s: type %d has no MFMA path", who, type);
        return 0;
    }
    if (B < 1) { kq_fail("%s: B=%d", who, B); return 0; }
    if (check_shape(type, N, K) || kq_ready()) return 0;
    if (!w || !xs || !ys) { kq_fail("%s: NULL pointer", who); return 0; }
    if ((uintptr_t)xs & 15) { kq_fail("%s: xs must be 16-byte aligned", who); return 0; }
    long pl, xsb, pt;
    if (kqk_mfma_workspace(type, B, N, K, g_kq.n_cu, &pl, &xsb, &pt)) {
        kq_fail("%s: bad shape", who);
        return 0;
    }
    const size_t a = 256;
    *o_xs = (pl + a - 1) / a * a;
    *o_pt = *o_xs + (xsb + a - 1) / a * a;
    return *o_pt + (size_t)pt;
}

static int mfma_launch(int type, const void* w, const float* xs, float* ys, int B, int N, int K,
                       uint8_t* ws, size_t o_xs, size_t o_pt, kq_stream stream) {
    const int e = kqk_launch_mfma(type, xs, w, ys, B, N, K, ws, (float*)(ws + o_xs),
                                  (float*)(ws + o_pt), g_kq.n_cu, pick(stream));
    if (e) return kq_fail("mfma multix launch: %s", hipGetErrorString((hipError_t)e));
    return 0;
}

/* Grows a stream's matrix-core workspace to at least `need` bytes (and at
 * least what kq_reserve_mfma_workspace asked for). */
static int mfma_reserve(kq_scr* sc, size_t need) {
    if (need < g_kq.mf_reserve) need = g_kq.mf_reserve;
    if (sc->cap_mf >= need) return 0;
    if (sc->mf) (void)hipFree(sc->mf);
    sc->mf = NULL;
    sc->cap_mf = 0;
    if (hip_ok(hipMalloc((void**)&sc->mf, need), "hipMalloc(mfma workspace)")) return -1;
    sc->cap_mf = need;
    return 0;
}

int kq_gemv_multix_mfma_dev(int type, const void* w, const float* xs, float* ys,
                            int B, int N, int K, kq_stream stream) {
    size_t o_xs, o_pt;
    const size_t need = mfma_prepare("kq_gemv_multix_mfma_dev", type, w, xs, ys, B, N, K,
                                     &o_xs, &o_pt);
    if (!need) return -1;
    kq_scr* sc = scr_of(pick(stream));
    if (!sc || mfma_reserve(sc, need)) return -1;
    return mfma_launch(type, w, xs, ys, B, N, K, sc->mf, o_xs, o_pt, stream);
}

int64_t kq_gemv_multix_mfma_workspace_bytes(int type, int B, int N, int K) {
    static const float dummy[4];
    size_t o_xs, o_pt;
    const size_t need = mfma_prepare("kq_gemv_multix_mfma_workspace_bytes", type, dummy,
                                     dummy, (float*)dummy, B, N, K, &o_xs, &o_pt);
    return need ? (int64_t)need : -1;
}

int kq_reserve_mfma_workspace(int64_t bytes) {
    if (bytes < 0) return kq_fail("kq_reserve_mfma_workspace: bytes=%lld", (long long)bytes);
    if (kq_ready()) return -1;
    if ((size_t)bytes > g_kq.mf_reserve) g_kq.mf_reserve = (size_t)bytes;
    kq_scr* sc = scr_of(NULL);
    if (!sc) return -1;
    for (int i = 0; i < KQ_SCR_SLOTS; i++)     /* the default stream and every stream seen */
        if (g_kq.scr[i].used && mfma_reserve(&g_kq.scr[i], (size_t)bytes)) return -1;
    return 0;
}

int64_t kq_scratch_bytes(void) {
    size_t n = (g_kq.cap_x + g_kq.cap_y + g_kq.cap_a) * sizeof(float);
    for (int i = 0; i < KQ_SCR_SLOTS; i++)
        n += g_kq.scr[i].cap_mf + g_kq.scr[i].cap_moe * sizeof(float);
    return (int64_t)n;
}

/* The same launch with its workspace in the library's static device
 * scratch (kqk_noalloc_scratch): no allocation at all, for callers that
 * cannot allocate (graph capture, allocation-free serving loops). */
int kq_gemv_multix_mfma_noalloc_dev(int type, const void* w, const float* xs, float* ys,
                                    int B, int N, int K, kq_stream stream) {
    size_t o_xs, o_pt;
    const size_t need = mfma_prepare("kq_gemv_multix_mfma_noalloc_dev", type, w, xs, ys, B, N, K,
                                     &o_xs, &o_pt);
    if (!need) return -1;
    void* scr = NULL;
    long cap = 0;
    const int e = kqk_noalloc_scratch(&scr, &cap);
    if (e) return kq_fail("static scratch: %s", hipGetErrorString((hipError_t)e));
    if (need > (size_t)cap)
        return kq_fail("kq_gemv_multix_mfma_noalloc_dev: B=%d N=%d K=%d needs %zu bytes of "
                       "scratch, more than the static %ld (KQ_NOALLOC_SCRATCH_BYTES)",
                       B, N, K, need, cap);
    return mfma_launch(type, w, xs, ys, B, N, K, (uint8_t*)scr, o_xs, o_pt, stream);
}

int kq_dequant_dev(int type, const void* w, float* y, int64_t nblocks, kq_stream stream) {
    if (!block_bytes(type)) return kq_fail("unsupported type %d", type);
    if (kq_ready()) return -1;
    if (nblocks <= 0) return 0;
    int e = kqk_launch_dequant(type, w, y, (long)nblocks, pick(stream));
    if (e) return kq_fail("dequant launch: %s", hipGetErrorString((hipError_t)e));
    return 0;
}

/* --------------------------------------------------- host-pointer ABI */

/* st_linear_q4k, _q6k, _q5k, _q3k and _q8_0 take the SDOT
 * (int8-activation) path when g_st.use_sdot is set (stratum_linear.h:
 * 369-489): the same switch for the host-pointer entry points */
static int sdot_type(int type) {
    return g_kq.use_sdot && has_sdot(type) ? type | KQ_INT8_ACT : type;
}

int kq_linear_set_sdot(int on) {
    const int prev = g_kq.use_sdot;
    g_kq.use_sdot = on != 0;
    return prev;
}

int kq_quantize_x_q8_dev(const float* x, int K, int group, int8_t* xq, float* xscale,
                         int32_t* xsum, kq_stream stream) {
    if (kq_ready()) return -1;
    if (!x || !xq || !xscale) return kq_fail("kq_quantize_x_q8_dev: NULL pointer");
    if ((group != 32 && group != 16) || K <= 0 || K % group)
        return kq_fail("kq_quantize_x_q8_dev: group %d, K %d", group, K);
    if ((uintptr_t)x & 15) return kq_fail("kq_quantize_x_q8_dev: x must be 16-byte aligned");
    const int e = kqk_launch_quantize_q8(x, K, group, xq, xscale, (int*)xsum, pick(stream));
    if (e) return kq_fail("quantize launch: %s", hipGetErrorString((hipError_t)e));
    return 0;
}

static int h2d(float* d, const float* h, size_t n) {
    return hip_ok(hipMemcpyAsync(d, h, n * sizeof(float), hipMemcpyHostToDevice, g_kq.stream),
                  "copy x in");
}

static int finish_y(float* y, const float* d_y, size_t n) {
    if (hip_ok(hipMemcpyAsync(y, d_y, n * sizeof(float), hipMemcpyDeviceToHost, g_kq.stream),
               "copy y out")) return -1;
    return hip_ok(hipStreamSynchronize(g_kq.stream), "synchronize");
}

int kq_linear_dispatch_add(const kq_tensor* w, const float* x, const float* add,
                           float* y, int N, int K) {
    if (!w) return kq_fail("NULL tensor");
    if (check_shape((int)w->type, N, K) || kq_ready() || host_stream()) return -1;
    const void* dw = tensor_dev(w, N, K);
    if (!dw) return -1;
    if (grow(&g_kq.d_x, &g_kq.cap_x, (size_t)K) || grow(&g_kq.d_y, &g_kq.cap_y, (size_t)N))
        return -1;
    if (h2d(g_kq.d_x, x, (size_t)K)) return -1;
    const float* d_add = NULL;
    if (add) {
        if (grow(&g_kq.d_a, &g_kq.cap_a, (size_t)N) || h2d(g_kq.d_a, add, (size_t)N)) return -1;
        d_add = g_kq.d_a;
    }
    if (kq_gemv_dev(sdot_type((int)w->type), dw, g_kq.d_x, d_add, g_kq.d_y, N, K, g_kq.stream))
        return -1;
    return finish_y(y, g_kq.d_y, (size_t)N);
}

int kq_linear_dispatch(const kq_tensor* w, const float* x, float* y, int N, int K) {
    return kq_linear_dispatch_add(w, x, NULL, y, N, K);
}

int kq_linear_multix(const kq_tensor* w, const float* const* xs, float* const* ys,
                     int B, int N, int K) {
    if (!w) return kq_fail("NULL tensor");
    if (B < 1) return kq_fail("kq_linear_multix: B=%d", B);
    if (check_shape((int)w->type, N, K) || kq_ready() || host_stream()) return -1;
    const void* dw = tensor_dev(w, N, K);
    if (!dw) return -1;
    if (grow(&g_kq.d_x, &g_kq.cap_x, (size_t)B * K) ||
        grow(&g_kq.d_y, &g_kq.cap_y, (size_t)B * N)) return -1;
    for (int s = 0; s < B; s++)
        if (h2d(g_kq.d_x + (size_t)s * K, xs[s], (size_t)K)) return -1;
    if (kq_gemv_multix_dev(sdot_type((int)w->type), dw, g_kq.d_x, g_kq.d_y, B, N, K, g_kq.stream))
        return -1;
    for (int s = 0; s < B; s++)
        if (hip_ok(hipMemcpyAsync(ys[s], g_kq.d_y + (size_t)s * N, (size_t)N * sizeof(float),
                                  hipMemcpyDeviceToHost, g_kq.stream), "copy y out"))
            return -1;
    return hip_ok(hipStreamSynchronize(g_kq.stream), "synchronize");
}

int kq_q4k_group(const float* x, int K,
                 const kq_tensor* w0, float* y0, int N0,
                 const kq_tensor* w1, float* y1, int N1,
                 const kq_tensor* w2, float* y2, int N2) {
    const kq_tensor* ws[3] = {w0, w1, w2};
    float* ys[3] = {y0, y1, y2};
    const int Ns[3] = {N0, N1, N2};
    const int nw = w2 ? 3 : 2;
    if (kq_ready() || host_stream()) return -1;
    size_t ytot = 0;
    kq_segment sg[3];
    memset(sg, 0, sizeof sg);
    for (int i = 0; i < nw; i++) {
        if (!ws[i]) return kq_fail("kq_q4k_group: NULL tensor");
        if (check_shape((int)ws[i]->type, Ns[i], K)) return -1;
        const void* dw = tensor_dev(ws[i], Ns[i], K);
        if (!dw) return -1;
        sg[i].type = sdot_type((int)ws[i]->type); sg[i].K = K; sg[i].rows_per_group = Ns[i];
        sg[i].ngroups = 1; sg[i].w[0] = dw;
        ytot += (size_t)Ns[i];
    }
    if (grow(&g_kq.d_x, &g_kq.cap_x, (size_t)K) || grow(&g_kq.d_y, &g_kq.cap_y, ytot)) return -1;
    if (h2d(g_kq.d_x, x, (size_t)K)) return -1;
    size_t off = 0;
    for (int i = 0; i < nw; i++) {
        sg[i].x = g_kq.d_x;
        sg[i].y = g_kq.d_y + off;
        off += (size_t)Ns[i];
    }
    if (kq_gemv_segments_dev(sg, nw, g_kq.stream)) return -1;
    off = 0;
    for (int i = 0; i < nw; i++) {
        if (hip_ok(hipMemcpyAsync(ys[i], g_kq.d_y + off, (size_t)Ns[i] * sizeof(float),
                                  hipMemcpyDeviceToHost, g_kq.stream), "copy y out"))
            return -1;
        off += (size_t)Ns[i];
    }
    return hip_ok(hipStreamSynchronize(g_kq.stream), "synchronize");
}

/* ------------------------------------------------------------ MoE gather */

int64_t kq_moe_slice_bytes(const kq_tensor* t, int K_in, int N_out) {
    /* stratum_arch_moe.inc.c:220-238 */
    if (!t || K_in <= 0 || N_out <= 0) return -1;
    if (t->type == 43)   /* Q4K_W16: w16 + d/dm per 256 + m16 */
        return (int64_t)N_out * K_in * 2 + (int64_t)N_out * (K_in / 256) * 8 +
               (int64_t)N_out * (K_in / 32) * 2;
    if (t->type == 44)   /* Q6K_W16: the same without the m16 section */
        return (int64_t)N_out * K_in * 2 + (int64_t)N_out * (K_in / 256) * 8;
    const int64_t one = (int64_t)K_in * N_out;
    if (t->nbytes <= 0 || t->nelem <= 0) {
        const int bb = block_bytes((int)t->type);
        return bb ? one / 256 * bb : -1;
    }
    int64_t e_all = t->nelem / one;
    if (e_all < 1) e_all = 1;
    return t->nbytes / e_all;
}

void kq_moe_bind_slice(kq_tensor* dst, const kq_tensor* t, int e, int64_t slice, int N_out,
                       int K_in, const uint8_t* slice_host, const uint8_t* base) {
    /* stratum_arch_moe.inc.c:327-337 */
    *dst = *t;
    dst->nelem = (int64_t)K_in * N_out;
    dst->nbytes = slice;
    dst->offset = slice_host ? (uint64_t)(slice_host - base)
                             : t->offset + (uint64_t)e * (uint64_t)slice;
}

int kq_moe_pack_open(const uint8_t* base, size_t size, int n_layers, int n_experts, int n_embed,
                     int n_ff, const kq_tensor* gate, const kq_tensor* up, const kq_tensor* down,
                     kq_moe_pack* out) {
    /* the header checks of moe_pack_load (stratum_arch_moe.inc.c:506-525) */
    kq_moe_pack_hdr h;
    if (!base || !out || !gate || !up || !down) return kq_fail("kq_moe_pack_open: NULL argument");
    if (size < sizeof h) return kq_fail("MOE_PACK: not a pack file");
    memcpy(&h, base, sizeof h);
    const int64_t gsb = kq_moe_slice_bytes(gate, n_embed, n_ff);
    const int64_t usb = kq_moe_slice_bytes(up, n_embed, n_ff);
    const int64_t dsb = kq_moe_slice_bytes(down, n_ff, n_embed);
    int ok = memcmp(h.magic, "MOEP", 4) == 0 && h.version == 1 &&
             (int)h.n_layers == n_layers && (int)h.n_experts == n_experts &&
             (int)h.n_embed == n_embed && (int)h.n_ff == n_ff && h.gate_type == gate->type &&
             h.up_type == up->type && h.down_type == down->type &&
             h.gate_slice == (uint64_t)gsb && h.up_slice == (uint64_t)usb &&
             h.down_slice == (uint64_t)dsb && h.data_off >= sizeof h && h.data_off < size;
    const uint64_t stride = h.gate_slice + h.up_slice + h.down_slice;
    const uint64_t need = h.data_off + (uint64_t)n_layers * (uint64_t)n_experts * stride;
    if (ok && need > size) ok = 0;
    if (!ok) return kq_fail("MOE_PACK: the pack does not match this model");
    out->base = base;
    out->size = size;
    out->data_off = h.data_off;
    out->gate_slice = h.gate_slice;
    out->up_slice = h.up_slice;
    out->down_slice = h.down_slice;
    out->stride = stride;
    out->n_layers = h.n_layers;
    out->n_experts = h.n_experts;
    return 0;
}

const uint8_t* kq_moe_pack_which(const kq_moe_pack* p, int li, int e, int which) {
    /* stratum_arch_moe.inc.c:307-313 */
    uint64_t off = p->data_off + ((uint64_t)li * (uint64_t)p->n_experts + (uint64_t)e) * p->stride;
    if (which == 1) off += p->gate_slice;
    else if (which == 2) off += p->gate_slice + p->up_slice;
    return p->base + off;
}

void kq_moe_topk(const float* w, int E, int K, int* sel, float* selw) {
    /* stratum_arch_moe.inc.c:368-385: insertion on a strictly greater
     * weight, so equal weights keep the lower expert id first */
    for (int s = 0; s < K; s++) { sel[s] = -1; selw[s] = -1.0f; }
    for (int e = 0; e < E; e++) {
        const float ww = w[e];
        for (int s = 0; s < K; s++) {
            if (ww > selw[s]) {
                for (int t2 = K - 1; t2 > s; t2--) {
                    sel[t2] = sel[t2 - 1];
                    selw[t2] = selw[t2 - 1];
                }
                sel[s] = e;
                selw[s] = ww;
                break;
            }
        }
    }
}

int kq_moe_topk_dev(const float* probs, int B, int E, int k, int* sel, float* selw,
                    kq_stream stream) {
    if (kq_ready()) return -1;
    if (!probs || !sel || !selw) return kq_fail("kq_moe_topk_dev: NULL pointer");
    if (B < 1 || E < 1 || E > KQ_MOE_MAX_EXPERTS || k < 1 || k > E)
        return kq_fail("kq_moe_topk_dev: B=%d E=%d k=%d", B, E, k);
    const int e = kqk_launch_moe_topk(probs, B, E, k, sel, selw, pick(stream));
    if (e) return kq_fail("moe top-k launch: %s", hipGetErrorString((hipError_t)e));
    return 0;
}

/* One token: the single-stream kernel, part r of tensor t on expert sel[r]
 * read on the device, or (probs != NULL) routed in the launch itself: every
 * workgroup takes the top-k of probs and workgroup 0 writes it to sel and
 * selw. */
/* One token: its k selections as the parts of one launch.  The FFN step's
 * pieces (kq_moe_ffn_dev, batch 1), each instead of writing y: logits (probs
 * holds router logits, their softmax taken in the launch), act (gate and
 * up in one segment: act = SwiGLU(gate, up)), cx / cw (the ranks' outputs
 * combined into cx). */
static int moe_one_token_ffn(const kq_moe_op* op, const int* sel, int k, int E,
                             const float* probs, float* selw, int logits, float* act, float* cx,
                             const float* cw, hipStream_t st) {
    const int nt = op->ntensors;
    kqk_seg h[2];
    memset(h, 0, sizeof h);
    /* gate and up on one x: one row space of 2k parts (part p uses
     * sel[p % k]); else one segment per tensor */
    const int one = nt == 2 && op->x_div == k && 2 * k <= KQ_MAX_GROUPS;
    const int nh = one ? 1 : nt;
    for (int t = 0; t < nt; t++) {
        kqk_seg* g = &h[one ? 0 : t];
        const int p0 = one ? t * k : 0;
        for (int r = 0; r < k; r++) {
            g->w[p0 + r] = op->w[t];
            g->y[p0 + r] = op->y[t] + (size_t)r * op->n_out;
            g->rows[p0 + r] = op->n_out;
        }
        g->type = op->type; g->K = op->k_in; g->nparts = p0 + k;
        g->x = op->x;
        g->x_stride = op->x_div == 1 && k > 1 ? op->k_in : 0;
        g->sel = sel;
        g->estride = (long)op->expert_stride;
        g->ksel = k;
        g->emax = E;
        if (probs) {
            g->probs = probs;
            g->sel_out = (int*)sel;
            g->selw_out = selw;
            g->logits = logits;
        }
        g->act = act;
        g->cx = cx;
        g->cw = cw;
    }
    int fit = 1;
    for (int i = 0; i < nh; i++) fit = fit && seg_fits(&h[i]);
    if (fit || act || cx) return launch_segs(h, nh, st);   /* the fused forms: checked by the caller */
    /* A segment too large for LDS (k per-part x of a long row, or many
     * rows per workgroup): its parts go in several segments of m parts, m
     * a divisor of k, so each sub-segment's parts are consecutive ranks of
     * one tensor (part i uses sel[q0 + i]).  Routed in the launch, the
     * top-k is taken by a launch of its own first. */
    if (probs) {
        const int e = kqk_launch_moe_topk(probs, 1, E, k, (int*)sel, selw, st);
        if (e) return kq_fail("moe topk launch: %s", hipGetErrorString((hipError_t)e));
    }
    kqk_seg out[KQ_MAX_SEGMENTS];
    int no = 0;
    for (int i = 0; i < nh; i++) {
        kqk_seg g = h[i];
        g.probs = NULL; g.sel_out = NULL; g.selw_out = NULL; g.logits = 0;
        int m = k;
        for (; m > 1; m--) {
            if (k % m) continue;
            kqk_seg t = g;
            t.nparts = m;
            if (seg_fits(&t)) break;
        }
        for (int q0 = 0; q0 < g.nparts; q0 += m) {
            kqk_seg t;
            memset(&t, 0, sizeof t);
            for (int p = 0; p < m; p++) {
                t.w[p] = g.w[q0 + p];
                t.y[p] = g.y[q0 + p];
                t.rows[p] = g.rows[q0 + p];
            }
            t.type = g.type; t.K = g.K; t.nparts = m;
            t.x = g.x_stride ? g.x + (size_t)q0 * g.x_stride : g.x;
            t.x_stride = m > 1 ? g.x_stride : 0;
            t.sel = sel + q0 % k;
            t.estride = g.estride; t.ksel = m; t.emax = g.emax;
            out[no++] = t;
            if (no == KQ_MAX_SEGMENTS) {
                if (launch_segs(out, no, st)) return -1;
                no = 0;
            }
        }
    }
    return no ? launch_segs(out, no, st) : 0;
}

static int moe_one_token(const kq_moe_op* op, const int* sel, int k, int E, const float* probs,
                         float* selw, hipStream_t st) {
    return moe_one_token_ffn(op, sel, k, E, probs, selw, 0, NULL, NULL, NULL, st);
}

static int moe_check_op(const kq_moe_op* op, int k, int E, const char* who) {
    if (check_shape(op->type, op->n_out, op->k_in) || kq_ready()) return -1;
    if (is_dense(op->type)) return kq_fail("%s: dense (F16/F32) experts are not supported", who);
    if ((op->type & KQ_INT8_ACT) && !has_sdot(op->type & ~KQ_INT8_ACT))
        return kq_fail("%s: type %d has no int8-activation form", who, op->type & ~KQ_INT8_ACT);
    const int nt = op->ntensors;
    if (nt < 1 || nt > 2) return kq_fail("%s: ntensors=%d", who, nt);
    if (op->x_div != 1 && op->x_div != k) return kq_fail("%s: x_div must be 1 or k", who);
    if (!op->x || ((uintptr_t)op->x & 15)) return kq_fail("%s: x NULL or unaligned", who);
    const int64_t rb = kq_row_bytes(op->type, op->k_in);
    if (op->expert_stride < rb * op->n_out)
        return kq_fail("%s: expert_stride below the slice size", who);
    for (int t = 0; t < nt; t++)
        if (!op->w[t] || !op->y[t]) return kq_fail("%s: NULL w or y", who);
    (void)E;
    return 0;
}

/* Several tokens: expert groups built on the device, then one weight pass
 * per selected expert for all of its tokens.  The launch is planned for
 * uniform routing (mx_plan): the planner picks the run length, and with it
 * the item count, and the runs are cut accordingly.  The runs are built
 * inside the multi-x launch when their LDS fits beside the plan's (one
 * launch instead of two; the grouping launch is kept for the rest, and
 * under KQ_MOE_GROUP_LAUNCH=1).  probs != NULL: the top-k is taken in that
 * launch too, written to sel / selw; returns 1 (nothing launched) when it
 * does not fit or does not pay, for the caller to route separately.  Every
 * workgroup ranks all B x E weights itself, about B E^2 compares: at
 * B = 16, E = 128 that took longer (114 us per layer) than the separate
 * top-k launch (104 us), so the in-launch ranking is kept to B E^2 <= 2^16
 * (E padded to 64). */
/* Run tables of one selection shared by two grouped launches: out != NULL
 * has the launch store the runs it builds (stored = 1, mch = its run
 * length); in != NULL has a launch of the same run length load them
 * instead of building. */
typedef struct {
    int* out;
    const int* in;
    int mch, stored;
    /* where the grouping launch writes its records and their count (the
     * fallback when the runs are not built in the multi-x launch); NULL:
     * the library's scratch, grown on demand */
    void* grp;
    size_t grp_bytes;
    int grp_used;          /* set when the grouping launch ran */
    int runs_loaded;       /* set when a launch loaded the stored tables */
} moe_runs_io;

/* Bytes of the grouping launch's records and count for nt tensors, nm
 * members over E experts cut into runs of at most mch members. */
static size_t moe_group_bytes(int nt, int nm, int E, int mch) {
    const int dmax = E < nm ? E : nm;
    const long ngmax = (long)nt * (dmax + (nm + mch - 1) / mch);
    return (size_t)ngmax * (size_t)kqk_mx_group_bytes() + 64;
}

static int moe_batch(const kq_moe_op* op, int* sel, const float* probs, float* selw, int B, int k,
                     int E, moe_runs_io* io, hipStream_t st) {
    const long E64 = (E + 63) & ~63L;
    if (probs && (long)B * E64 * E64 > (1L << 16)) return 1;
    const int nt = op->ntensors;
    const int nm = B * k, dmax = E < nm ? E : nm;
    const int mmax = B < 16 ? B : 16;
    const int grid = plan_grid();
    int plan[KQK_MX_PLAN];
    const int moe[4] = {B, k, E, nt};
    const long rbytes = kqk_moe_runs_lds(nm, E, dmax + nm, probs ? B : 0);
    if (!g_kq.env_moe_group_launch && rbytes + 16 < g_kq.lds_max / 2) {
        const long pl = mx_plan(op->type, op->n_out, op->k_in, mmax, nt * dmax, grid, moe,
                                g_kq.lds_max - (int)rbytes - 16, plan);
        if (pl >= 0) {
            const long off = (pl + 15) & ~15L;
            const int* rin = io && io->in && !probs && io->mch == plan[7] ? io->in : NULL;
            int* rout = io && io->out && !rin ? io->out : NULL;
            const int e = kqk_launch_mx_moe(op->type, plan, off, off + rbytes, grid, sel, nm, E,
                                            nt, op->x_div, op->w[0], op->w[nt - 1], op->y[0],
                                            op->y[nt - 1], (long)op->expert_stride, op->x,
                                            op->n_out, op->k_in, probs, B, k, sel, selw, rout,
                                            rin, st);
            if (e) return kq_fail("moe gemv launch: %s", hipGetErrorString((hipError_t)e));
            if (rout) {
                io->stored = 1;
                io->mch = plan[7];
            }
            if (rin) io->runs_loaded = 1;
            return 0;
        }
    }
    if (probs) return 1;
    const long lds = mx_plan(op->type, op->n_out, op->k_in, mmax, nt * dmax, grid, moe,
                             g_kq.lds_max, plan);
    if (lds < 0) return kq_fail("kq_moe_gemv_dev: no launch plan for K=%d", op->k_in);
    const int mch = plan[7];
    const int ngmax = nt * (dmax + (nm + mch - 1) / mch);
    const size_t gbytes = (size_t)kqk_mx_group_bytes();
    const size_t need = moe_group_bytes(nt, nm, E, mch);
    uint8_t* gbase;
    if (io && io->grp) {           /* the caller's workspace: no allocation */
        if (need > io->grp_bytes)
            return kq_fail("moe grouping: %zu bytes of group records, %zu in the workspace", need,
                           io->grp_bytes);
        gbase = (uint8_t*)io->grp;
        io->grp_used = 1;
    } else {
        kq_scr* sc = scr_of(st);
        if (!sc || grow(&sc->moe, &sc->cap_moe, need / sizeof(float) + 1)) return -1;
        gbase = (uint8_t*)sc->moe;
    }
    void* groups = gbase;
    int* ng = (int*)(gbase + (size_t)ngmax * gbytes);
    int e = kqk_launch_moe_group(sel, nm, E, nt, op->x_div, mch, op->w[0], op->w[nt - 1], op->y[0],
                                 op->y[nt - 1], (long)op->expert_stride, groups, ng, st);
    if (e) return kq_fail("moe group launch: %s", hipGetErrorString((hipError_t)e));
    e = kqk_launch_mx(op->type, plan, lds, grid, NULL, 0, groups, ng, op->x, op->k_in, NULL,
                      op->n_out, op->n_out, op->k_in, st);
    if (e) return kq_fail("moe gemv launch: %s", hipGetErrorString((hipError_t)e));
    return 0;
}

/* Bytes of moe_i8_batch's workspace for nx x rows of K, nt tensors and nm
 * members over E experts: the quantized rows, their coefficients and the
 * zero page (kqk_mi8_moe_workspace), then the runs' group records; 0 for a
 * bad shape. */
static size_t moe_i8_bytes(int type, int nx, int K, int nt, int nm, int E) {
    const long xw = kqk_mi8_moe_workspace(type, nx, K);
    if (xw < 0) return 0;
    return (((size_t)xw + 255) & ~(size_t)255) + moe_group_bytes(nt, nm, E, 8);
}

/* Several tokens in the int8 mode, Q4_K / Q6_K.  moe_forward_b under
 * use_sdot (stratum_arch_moe.inc.c:1136-1201) runs each expert's members,
 * in increasing member order, in tickets of at most CH = 8 through
 * st_linear_multix: a ticket of two or more members takes the multix pack
 * arithmetic, a ticket of one the single-stream path.  Here the same runs
 * are cut on the device (kq_moe_group_kernel's rule, run length 8) in the
 * launch that quantizes every x row once, and one grouped matrix-core
 * launch computes all runs (kq_mi8_kernel, GR): each member equals
 * kq_gemv_multix_dev over its run (kq_gemv_dev for a run of one) bit for
 * bit.  (For Q5_K, Q3_K and Q8_0 st_linear_multix is per stream -- Q8_0's
 * pack equals its single-stream path, stratum_q8_0.h:145-149 -- so the
 * tickets do not matter: their batches run in the multi-x kernel, moe_batch.)
 * The workspace is io->grp when given (the FFN step's), else the library's
 * matrix-core scratch. */
static int moe_i8_batch(const kq_moe_op* op, const int* sel, int B, int k, int E,
                        moe_runs_io* io, hipStream_t st) {
    const int nm = B * k, nt = op->ntensors, nx = nm / op->x_div, K = op->k_in;
    const size_t need = moe_i8_bytes(op->type, nx, K, nt, nm, E);
    if (!need) return kq_fail("int8 moe batch: bad shape K=%d", K);
    uint8_t* base;
    if (io && io->grp) {
        if (need > io->grp_bytes)
            return kq_fail("int8 moe batch: %zu workspace bytes, %zu given", need, io->grp_bytes);
        base = (uint8_t*)io->grp;
        io->grp_used = 1;
    } else {
        kq_scr* sc = scr_of(st);
        if (!sc || mfma_reserve(sc, need)) return -1;
        base = sc->mf;
    }
    const size_t xwa = ((size_t)kqk_mi8_moe_workspace(op->type, nx, K) + 255) & ~(size_t)255;
    const int dmax = E < nm ? E : nm;
    const int ngmax = nt * (dmax + (nm + 7) / 8);
    void* groups = base + xwa;
    int* ng = (int*)(base + xwa + (size_t)ngmax * (size_t)kqk_mx_group_bytes());
    const int e = kqk_launch_mi8_moe(op->type, sel, nm, E, nt, op->x_div, op->w[0], op->w[nt - 1],
                                     op->y[0], op->y[nt - 1], (long)op->expert_stride, op->x, K,
                                     groups, ng, ngmax, op->n_out, base, g_kq.n_cu, st);
    if (e) return kq_fail("int8 moe launch: %s", hipGetErrorString((hipError_t)e));
    return 0;
}

/* B tokens of a type the multi-x kernel does not cover: one launch per
 * token, each with its k selections (the same bits as the batched path). */
static int moe_per_token(const kq_moe_op* op, const int* sel, int B, int k, int E, hipStream_t st) {
    for (int s = 0; s < B; s++) {
        kq_moe_op o = *op;
        o.x = op->x + (size_t)s * (op->x_div == k ? 1 : k) * op->k_in;
        for (int t = 0; t < op->ntensors; t++) o.y[t] = op->y[t] + (size_t)s * k * op->n_out;
        if (moe_one_token(&o, sel + (size_t)s * k, k, E, NULL, NULL, st)) return -1;
    }
    return 0;
}

/* kq_moe_gemv_routed_dev with the grouping records in io->grp when io is
 * given (the FFN step's workspace), else in the library's scratch */
static int moe_gemv_routed(const kq_moe_op* op, const float* probs, int B, int k, int E, int* sel,
                           float* selw, moe_runs_io* io, hipStream_t st) {
    if (!op || !probs || !sel || !selw) return kq_fail("kq_moe_gemv_routed_dev: NULL argument");
    if (B < 1 || B > KQ_MOE_MAX_TOKENS || k < 1 || k > KQ_MAX_GROUPS || E < 1 || E > 1024)
        return kq_fail("kq_moe_gemv_routed_dev: B=%d k=%d E=%d (E <= 1024)", B, k, E);
    if (moe_check_op(op, k, E, "kq_moe_gemv_routed_dev")) return -1;
    if (B == 1) return moe_one_token(op, sel, k, E, probs, selw, st);
    if (!is_mx(op->type)) {
        const int e = kqk_launch_moe_topk(probs, B, E, k, sel, selw, st);
        if (e) return kq_fail("moe topk launch: %s", hipGetErrorString((hipError_t)e));
        return is_i8mx(op->type) ? moe_i8_batch(op, sel, B, k, E, io, st)
                                 : moe_per_token(op, sel, B, k, E, st);
    }
    const int r = moe_batch(op, sel, probs, selw, B, k, E, io, st);
    if (r <= 0) return r;
    /* the router weights do not fit beside the plan: route separately */
    const int e = kqk_launch_moe_topk(probs, B, E, k, sel, selw, st);
    if (e) return kq_fail("moe topk launch: %s", hipGetErrorString((hipError_t)e));
    return moe_batch(op, sel, NULL, NULL, B, k, E, io, st);
}

int kq_moe_gemv_routed_dev(const kq_moe_op* op, const float* probs, int B, int k, int E, int* sel,
                           float* selw, kq_stream stream) {
    return moe_gemv_routed(op, probs, B, k, E, sel, selw, NULL, pick(stream));
}

/* kq_moe_gemv_dev with the grouping records in io->grp when io is given */
static int moe_gemv(const kq_moe_op* op, const int* sel, int B, int k, int E, moe_runs_io* io,
                    hipStream_t st) {
    if (!op || !sel) return kq_fail("kq_moe_gemv_dev: NULL argument");
    if (B < 1 || B > KQ_MOE_MAX_TOKENS || k < 1 || k > KQ_MAX_GROUPS || E < 1 ||
        E > KQ_MOE_MAX_EXPERTS)
        return kq_fail("kq_moe_gemv_dev: B=%d k=%d E=%d", B, k, E);
    if (moe_check_op(op, k, E, "kq_moe_gemv_dev")) return -1;
    if (B == 1) return moe_one_token(op, sel, k, E, NULL, NULL, st);
    if (is_i8mx(op->type)) return moe_i8_batch(op, sel, B, k, E, io, st);
    if (!is_mx(op->type)) return moe_per_token(op, sel, B, k, E, st);
    return moe_batch(op, (int*)sel, NULL, NULL, B, k, E, io, st);
}

int kq_moe_gemv_dev(const kq_moe_op* op, const int* sel, int B, int k, int E, kq_stream stream) {
    return moe_gemv(op, sel, B, k, E, NULL, pick(stream));
}

/* ------------------------------------------------------ MoE FFN step */

int kq_softmax_dev(float* x, int B, int E, kq_stream stream) {
    if (kq_ready()) return -1;
    if (!x) return kq_fail("kq_softmax_dev: NULL pointer");
    if (B < 1 || E < 1 || E > KQ_MOE_MAX_EXPERTS)
        return kq_fail("kq_softmax_dev: B=%d E=%d (E <= %d)", B, E, KQ_MOE_MAX_EXPERTS);
    const int e = kqk_launch_softmax(x, B, E, pick(stream));
    if (e) return kq_fail("softmax launch: %s", hipGetErrorString((hipError_t)e));
    return 0;
}

int kq_swiglu_dev(const float* g, const float* u, float* y, int64_t n, kq_stream stream) {
    if (kq_ready()) return -1;
    if (!g || !u || !y) return kq_fail("kq_swiglu_dev: NULL pointer");
    if (((uintptr_t)g | (uintptr_t)u | (uintptr_t)y) & 15)
        return kq_fail("kq_swiglu_dev: g, u and y must be 16-byte aligned");
    if (n < 1) return kq_fail("kq_swiglu_dev: n=%lld", (long long)n);
    const int e = kqk_launch_swiglu(g, u, y, (long)n, pick(stream));
    if (e) return kq_fail("swiglu launch: %s", hipGetErrorString((hipError_t)e));
    return 0;
}

int kq_moe_combine_dev(const float* o, const int* sel, const float* selw, const float* resid,
                       float* x, int B, int k, int H, kq_stream stream) {
    if (kq_ready()) return -1;
    if (!o || !sel || !selw || !resid || !x) return kq_fail("kq_moe_combine_dev: NULL pointer");
    if (((uintptr_t)o | (uintptr_t)resid | (uintptr_t)x) & 15)
        return kq_fail("kq_moe_combine_dev: o, resid and x must be 16-byte aligned");
    if (B < 1 || k < 1 || H < 4 || H % 4)
        return kq_fail("kq_moe_combine_dev: B=%d k=%d H=%d (H %% 4 must be 0)", B, k, H);
    const int e = kqk_launch_moe_combine(o, sel, selw, resid, x, B, k, H, pick(stream));
    if (e) return kq_fail("combine launch: %s", hipGetErrorString((hipError_t)e));
    return 0;
}

/* workspace of one step: probs B x E, g / u / act B*k x F, down outputs
 * B*k x H, the run tables of the batch launches, and the records of the
 * grouping launch (used when the runs cannot be built inside the multi-x
 * launch: sized for gate+up together and runs of one member, the most any
 * launch of the step needs), each 256-byte aligned */
#define FFN_REGIONS 7
static int64_t ffn_layout(const kq_moe_ffn* f, int B, int64_t off[FFN_REGIONS]) {
    const int64_t bk = (int64_t)B * f->k;
    const int dmax = f->n_experts < bk ? f->n_experts : (int)bk;
    /* the group records, or a batch's int8 workspace when larger */
    const int E = f->n_experts, pair = f->gate_type == f->up_type && f->gate_stride == f->up_stride;
    size_t g6 = moe_group_bytes(2, (int)bk, E, 1);
    if (B > 1) {
        const size_t i8[3] = {
            is_i8mx(f->gate_type) ? moe_i8_bytes(f->gate_type, B, f->n_embed, pair ? 2 : 1, (int)bk, E) : 0,
            is_i8mx(f->up_type) ? moe_i8_bytes(f->up_type, B, f->n_embed, 1, (int)bk, E) : 0,
            is_i8mx(f->down_type) ? moe_i8_bytes(f->down_type, (int)bk, f->n_ff, 1, (int)bk, E) : 0};
        for (int i = 0; i < 3; i++) g6 = i8[i] > g6 ? i8[i] : g6;
    }
    const int64_t sz[FFN_REGIONS] = {
        (int64_t)B * f->n_experts * 4, bk * f->n_ff * 4, bk * f->n_ff * 4, bk * f->n_ff * 4,
        bk * f->n_embed * 4, 4 * kqk_moe_runs_words((int)bk, f->n_experts, dmax + (int)bk),
        (int64_t)g6};
    int64_t t = 0;
    for (int i = 0; i < FFN_REGIONS; i++) {
        off[i] = t;
        t += (sz[i] + 255) & ~(int64_t)255;
    }
    return t;
}

static int ffn_check(const kq_moe_ffn* f, int B, const char* who) {
    if (!f) return kq_fail("%s: NULL descriptor", who);
    if (B < 1 || B > KQ_MOE_MAX_TOKENS) return kq_fail("%s: B=%d", who, B);
    if (f->k < 1 || f->k > KQ_MAX_GROUPS || f->n_experts < f->k ||
        f->n_experts > KQ_MOE_MAX_EXPERTS)
        return kq_fail("%s: k=%d E=%d", who, f->k, f->n_experts);
    if (f->n_embed <= 0 || f->n_embed % 256 || f->n_ff <= 0 || f->n_ff % 256)
        return kq_fail("%s: n_embed=%d n_ff=%d (multiples of 256)", who, f->n_embed, f->n_ff);
    if (!f->router || !f->gate || !f->up || !f->down) return kq_fail("%s: NULL tensor", who);
    return 0;
}

int64_t kq_moe_ffn_workspace_bytes(const kq_moe_ffn* f, int B) {
    if (ffn_check(f, B, "kq_moe_ffn_workspace_bytes")) return -1;
    int64_t off[FFN_REGIONS];
    return ffn_layout(f, B, off);
}

/* Whether the batch-1 three-launch form fits this layer: the launches'
 * LDS plans, and the conditions the fused epilogues put on them (each
 * workgroup's outputs of all parts fit the x region it no longer needs,
 * and the combine has a lane per output row of a part). */
static int ffn_fused_fits(const kq_moe_ffn* f) {
    const int grid = plan_grid(), H = f->n_embed, F = f->n_ff, k = f->k;
    if (F % grid || H % grid) return 0;
    static const float dummy[4];
    static int dsel[KQ_MAX_GROUPS];
    kqk_seg s;
    int xo, to, so;
    /* gate + up: 2k parts of F rows on one x of H, routed in the launch */
    memset(&s, 0, sizeof s);
    s.type = f->gate_type; s.K = H; s.nparts = 2 * k; s.x = dummy;
    for (int p = 0; p < 2 * k; p++) s.rows[p] = F;
    s.sel = dsel; s.ksel = k; s.emax = f->n_experts;
    s.probs = dummy; s.sel_out = dsel; s.selw_out = (float*)dummy;
    long l = kqk_segs_lds(&s, 1, grid, &xo, &to, &so);
    if (l < 0 || l > g_kq.lds_max || (long)2 * k * (F / grid) * 4 > xo) return 0;
    /* down: k parts of H rows, each on its own x of F */
    memset(&s, 0, sizeof s);
    s.type = f->down_type; s.K = F; s.nparts = k; s.x = dummy;
    s.x_stride = k > 1 ? F : 0;
    for (int p = 0; p < k; p++) s.rows[p] = H;
    s.sel = dsel; s.ksel = k; s.emax = f->n_experts;
    l = kqk_segs_lds(&s, 1, grid, &xo, &to, &so);
    if (l < 0 || l > g_kq.lds_max || (long)k * (H / grid) * 4 > xo ||
        H / grid > plan_threads(&s, 1, grid))
        return 0;
    return 1;
}

static int g_ffn_path;     /* what the last kq_moe_ffn_dev call did (KQ_FFN_* bits) */

int kq_moe_ffn_last_path(void) { return g_ffn_path; }

/* The expert FFN step of moe_forward_one_token / moe_forward_b
 * (stratum_arch_moe.inc.c:689-743, 1107-1226) after the norm: router GEMV,
 * softmax, top-k, gate and up of the selected slices, SwiGLU, down, and
 * the rank-ordered weighted accumulate plus the residual -- on one stream,
 * with every intermediate and every device-side table in the caller's
 * workspace (no allocation). */
int kq_moe_ffn_dev(const kq_moe_ffn* f, const float* xn, float* x, int B, int* sel, float* selw,
                   void* work, int64_t work_bytes, kq_stream stream) {
    static const char who[] = "kq_moe_ffn_dev";
    g_ffn_path = 0;
    if (ffn_check(f, B, who) || kq_ready()) return -1;
    if (!xn || !x || !sel || !selw || !work) return kq_fail("%s: NULL pointer", who);
    if (((uintptr_t)xn | (uintptr_t)x | (uintptr_t)work) & 15)
        return kq_fail("%s: xn, x and work must be 16-byte aligned", who);
    int64_t off[FFN_REGIONS];
    const int64_t need = ffn_layout(f, B, off);
    if (work_bytes < need)
        return kq_fail("%s: workspace of %lld bytes, %lld needed", who, (long long)work_bytes,
                       (long long)need);
    uint8_t* w8 = (uint8_t*)work;
    float* probs = (float*)(w8 + off[0]);
    float* g = (float*)(w8 + off[1]);
    float* u = (float*)(w8 + off[2]);
    float* act = (float*)(w8 + off[3]);
    float* ffo = (float*)(w8 + off[4]);
    void* grp = w8 + off[6];
    const size_t grp_bytes = (size_t)(need - off[6]);
    /* rio: the gate+up launch's run tables for the down launch; gio: group
     * records only (every other launch that may group) */
    moe_runs_io rio = {(int*)(w8 + off[5]), NULL, 0, 0, grp, grp_bytes, 0, 0};
    moe_runs_io gio = {NULL, NULL, 0, 0, grp, grp_bytes, 0, 0};
    const int H = f->n_embed, F = f->n_ff, E = f->n_experts, k = f->k;
    const int pair = f->gate_type == f->up_type && f->gate_stride == f->up_stride;
    hipStream_t st = pick(stream);

    /* One token in three launches: router logits; gate and up of the
     * selected slices with the softmax and top-k taken in that launch and
     * SwiGLU in its epilogue; down with the rank-ordered combine plus
     * residual in its epilogue.  The same arithmetic as the six-launch form
     * below (the tests hold the two bit-identical; KQ_MOE_FFN_SPLIT=1 forces
     * that form).  Needs one gate+up segment (2k <= KQ_MAX_GROUPS), E <= 256
     * (every logit in a lane), types of is_ffn_b1, n_ff and n_embed multiples
     * of the grid (a workgroup then holds a rank's gate and up row, and all
     * k ranks' down rows, of the same index), and the fused epilogues'
     * room (ffn_fused_fits). */
    if (B == 1 && pair && 2 * k <= KQ_MAX_GROUPS && E <= 256 && is_ffn_b1(f->gate_type) &&
        is_ffn_b1(f->down_type) && !g_kq.env_ffn_split && ffn_fused_fits(f)) {
        if (kq_gemv_dev(f->router_type, f->router, xn, NULL, probs, E, H, stream)) return -1;
        kq_moe_op gu;
        memset(&gu, 0, sizeof gu);
        gu.type = f->gate_type; gu.n_out = F; gu.k_in = H; gu.x = xn; gu.x_div = k;
        gu.ntensors = 2;
        gu.w[0] = f->gate; gu.y[0] = g;
        gu.w[1] = f->up; gu.y[1] = u;
        gu.expert_stride = f->gate_stride;
        if (moe_check_op(&gu, k, E, who)) return -1;
        if (moe_one_token_ffn(&gu, sel, k, E, probs, selw, 1, act, NULL, NULL, st)) return -1;
        kq_moe_op dn;
        memset(&dn, 0, sizeof dn);
        dn.type = f->down_type; dn.n_out = H; dn.k_in = F; dn.x = act; dn.x_div = 1;
        dn.ntensors = 1; dn.w[0] = f->down; dn.y[0] = ffo; dn.expert_stride = f->down_stride;
        if (moe_check_op(&dn, k, E, who)) return -1;
        g_ffn_path = KQ_FFN_FUSED_B1;
        return moe_one_token_ffn(&dn, sel, k, E, NULL, NULL, 0, NULL, x, selw, st);
    }

    /* router logits, softmax (stratum_arch_moe.inc.c:689-691, 1107-1121) */
    if (B == 1 ? kq_gemv_dev(f->router_type, f->router, xn, NULL, probs, E, H, stream)
               : kq_gemv_multix_dev(f->router_type, f->router, xn, probs, B, E, H, stream))
        return -1;
    if (kq_softmax_dev(probs, B, E, stream)) return -1;

    /* gate and up of the selected slices, routed in the launch when one op
     * holds both */
    kq_moe_op gu;
    memset(&gu, 0, sizeof gu);
    gu.type = f->gate_type; gu.n_out = F; gu.k_in = H; gu.x = xn; gu.x_div = k;
    gu.ntensors = pair ? 2 : 1;
    gu.w[0] = f->gate; gu.y[0] = g;
    gu.w[1] = pair ? f->up : NULL; gu.y[1] = pair ? u : NULL;
    gu.expert_stride = f->gate_stride;
    const int share = B > 1 && is_mx(f->gate_type) && is_mx(f->down_type) && E <= 1024 &&
                      !g_kq.env_ffn_split;
    if (share) {
        /* a batch: the grouped gate+up launch stores its run tables for the
         * down launch (routed inside it when that fits, else after a top-k
         * launch) */
        if (moe_check_op(&gu, k, E, who)) return -1;
        int r = moe_batch(&gu, sel, probs, selw, B, k, E, &rio, st);
        if (r == 1) {
            const int e = kqk_launch_moe_topk(probs, B, E, k, sel, selw, st);
            if (e) return kq_fail("moe topk launch: %s", hipGetErrorString((hipError_t)e));
            r = moe_batch(&gu, sel, NULL, NULL, B, k, E, &rio, st);
        }
        if (r < 0) return -1;
        if (r > 0 && moe_gemv(&gu, sel, B, k, E, &gio, st)) return -1;
    } else if (E <= 1024) {
        if (moe_gemv_routed(&gu, probs, B, k, E, sel, selw, &gio, st)) return -1;
    } else {
        if (kq_moe_topk_dev(probs, B, E, k, sel, selw, stream) ||
            moe_gemv(&gu, sel, B, k, E, &gio, st))
            return -1;
    }
    if (!pair) {
        kq_moe_op up;
        memset(&up, 0, sizeof up);
        up.type = f->up_type; up.n_out = F; up.k_in = H; up.x = xn; up.x_div = k;
        up.ntensors = 1; up.w[0] = f->up; up.y[0] = u; up.expert_stride = f->up_stride;
        if (moe_gemv(&up, sel, B, k, E, &gio, st)) return -1;
    }

    /* SwiGLU, down, weighted accumulate + residual */
    if (kq_swiglu_dev(g, u, act, (int64_t)B * k * F, stream)) return -1;
    kq_moe_op dn;
    memset(&dn, 0, sizeof dn);
    dn.type = f->down_type; dn.n_out = H; dn.k_in = F; dn.x = act; dn.x_div = 1;
    dn.ntensors = 1; dn.w[0] = f->down; dn.y[0] = ffo; dn.expert_stride = f->down_stride;
    if (share && rio.stored) {
        /* the gate+up launch's run tables, when the down plan cuts runs alike */
        rio.in = rio.out;
        rio.out = NULL;
        if (moe_check_op(&dn, k, E, who)) return -1;
        const int r = moe_batch(&dn, sel, NULL, NULL, B, k, E, &rio, st);
        if (r < 0) return -1;
        if (r > 0 && moe_gemv(&dn, sel, B, k, E, &gio, st)) return -1;
    } else if (moe_gemv(&dn, sel, B, k, E, &gio, st)) {
        return -1;
    }
    g_ffn_path = (rio.stored ? KQ_FFN_RUNS_STORED : 0) | (rio.runs_loaded ? KQ_FFN_RUNS_LOADED : 0) |
                 (rio.grp_used || gio.grp_used ? KQ_FFN_GROUP_LAUNCH : 0);
    return kq_moe_combine_dev(ffo, sel, selw, x, x, B, k, H, stream);
}

/* --------------------------------------------- type-42 on the device */
int kq_q2k_to_nib_dev(const void* q2k, void* nib, int64_t nblocks, kq_stream stream) {
    if (kq_ready()) return -1;
    if (!q2k || !nib) return kq_fail("kq_q2k_to_nib_dev: NULL pointer");
    if (((uintptr_t)q2k | (uintptr_t)nib) & 3)
        return kq_fail("kq_q2k_to_nib_dev: buffers must be 4-byte aligned");
    if (nblocks < 1 || nblocks > ((int64_t)1 << 40)) return kq_fail("kq_q2k_to_nib_dev: nblocks");
    const int e = kqk_launch_q2k_to_nib(q2k, nib, (long)nblocks, pick(stream));
    if (e) return kq_fail("q2k_to_nib launch: %s", hipGetErrorString((hipError_t)e));
    return 0;
}
