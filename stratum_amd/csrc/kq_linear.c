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

#include <hip/hip_runtime_api.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* launchers (kq_kernels.hip) */
long kqk_gemv_lds_bytes(int type, int K, int rows_per_wg);
int kqk_launch_gemv(int type, const void* w, const float* x, const float* add, float* y,
                    int N, int K, int rows_per_wg, int threads, int depth, hipStream_t st);
int kqk_launch_dequant(int type, const void* w, float* y, long nblocks, hipStream_t st);
int kqk_set_max_lds(int bytes);

#define KQ_MAX_REGIONS 16

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
    hipStream_t stream;    /* library stream (default priority) */
    kq_region reg[KQ_MAX_REGIONS];
    int nreg;
    const uint8_t* base;   /* kq_linear_init base: offsets resolve here */
    /* staging for the host-pointer ABI */
    float* d_x; size_t cap_x;
    float* d_y; size_t cap_y;
    float* d_a; size_t cap_a;
    char err[512];
} kq_state;

static kq_state g_kq;

static int kq_fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_kq.err, sizeof g_kq.err, fmt, ap);
    va_end(ap);
    fprintf(stderr, "kq: %s\n", g_kq.err);
    return -1;
}

const char* kq_last_error(void) { return g_kq.err; }

static int block_bytes(int type) {
    switch (type) {   /* stratum_gguf.h:57-79 */
    case KQ_TYPE_Q2_K: return 84;
    case KQ_TYPE_Q4_K: return 144;
    case KQ_TYPE_Q6_K: return 210;
    case KQ_TYPE_Q2K_NIB: return 148;
    default: return 0;
    }
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

static int kq_ready(void) {
    if (g_kq.ready) return 0;
    int dev = 0, n = 0;
    if (hip_ok(hipGetDeviceCount(&n), "hipGetDeviceCount")) return -1;
    if (n < 1) return kq_fail("no HIP device");
    if (hip_ok(hipGetDevice(&dev), "hipGetDevice")) return -1;
    int ncu = 0, lds = 0;
    if (hip_ok(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev),
               "hipDeviceGetAttribute(CU count)")) return -1;
    if (hip_ok(hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev),
               "hipDeviceGetAttribute(LDS)")) return -1;
    /* blocking stream, default priority: orders with the null stream */
    if (hip_ok(hipStreamCreate(&g_kq.stream), "hipStreamCreate")) return -1;
    g_kq.device = dev;
    g_kq.n_cu = ncu > 0 ? ncu : 1;
    g_kq.lds_max = lds > 0 ? lds : 65536;
    if (kqk_set_max_lds(g_kq.lds_max) != 0) return kq_fail("cannot raise the LDS limit");
    g_kq.ready = 1;
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
    if (g_kq.ready && g_kq.stream) (void)hipStreamDestroy(g_kq.stream);
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
/* One workgroup per CU, each owning ceil(N / n_cu) consecutive rows, as
 * long as x plus the per-chunk terms fit in LDS; workgroup size grows with
 * the chunks it owns.  KQ_ROWS_PER_WG / KQ_WG_THREADS / KQ_DEPTH override
 * (tuning). */
static int plan(int type, int N, int K, int* rows, int* threads, int* depth) {
    const int NC = K / 64;
    const long xb = kqk_gemv_lds_bytes(type, K, 0);
    if (xb < 0) return kq_fail("type %d has no GEMV kernel", type);
    const long cap = (long)g_kq.lds_max - 256;
    long rmax = (cap - xb) / ((long)NC * 8);
    if (rmax < 1) return kq_fail("K=%d needs %ld bytes of LDS for x (max %ld)", K, xb, cap);
    long R = (N + g_kq.n_cu - 1) / g_kq.n_cu;
    const char* er = getenv("KQ_ROWS_PER_WG");
    if (er && atoi(er) > 0) R = atoi(er);
    if (R > rmax) R = rmax;
    if (R < 1) R = 1;
    long chunks = R * NC;
    int T = chunks >= 4096 ? 1024 : chunks >= 1024 ? 512 : 256;

    const char* et = getenv("KQ_WG_THREADS");
    if (et) {
        int t = atoi(et);
        if (t == 256 || t == 512 || t == 1024) T = t;
    }
    int D = 2;
    const char* ed = getenv("KQ_DEPTH");
    if (ed && atoi(ed) >= 1 && atoi(ed) <= 6) D = atoi(ed);
    *rows = (int)R;
    *threads = T;
    *depth = D;
    return 0;
}

/* NULL is the null (default) stream, as in the HIP runtime itself. */
static hipStream_t pick(kq_stream s) { return (hipStream_t)s; }

static int check_shape(int type, int N, int K) {
    if (!block_bytes(type)) return kq_fail("unsupported type %d", type);
    if (N <= 0 || K <= 0 || K % 256) return kq_fail("bad shape N=%d K=%d (K %% 256 must be 0)", N, K);
    return 0;
}

/* ------------------------------------------------- device-pointer ABI */

int kq_gemv_dev(int type, const void* w, const float* x, const float* add, float* y,
                int N, int K, kq_stream stream) {
    if (check_shape(type, N, K) || kq_ready()) return -1;
    if (!w || !x || !y) return kq_fail("kq_gemv_dev: NULL pointer");
    if ((uintptr_t)x & 15) return kq_fail("kq_gemv_dev: x must be 16-byte aligned");
    int R = 1, T = 256, D = 2;
    if (plan(type, N, K, &R, &T, &D)) return -1;
    int e = kqk_launch_gemv(type, w, x, add, y, N, K, R, T, D, pick(stream));
    if (e) return kq_fail("gemv launch: %s", hipGetErrorString((hipError_t)e));
    return 0;
}

int kq_gemv_multix_dev(int type, const void* w, const float* xs, float* ys,
                       int B, int N, int K, kq_stream stream) {
    if (B < 1) return kq_fail("kq_gemv_multix_dev: B=%d", B);
    for (int s = 0; s < B; s++)
        if (kq_gemv_dev(type, w, xs + (size_t)s * K, NULL, ys + (size_t)s * N, N, K, stream))
            return -1;
    return 0;
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
    if (check_shape((int)w->type, N, K) || kq_ready()) return -1;
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
    if (kq_gemv_dev((int)w->type, dw, g_kq.d_x, d_add, g_kq.d_y, N, K, g_kq.stream)) return -1;
    return finish_y(y, g_kq.d_y, (size_t)N);
}

int kq_linear_dispatch(const kq_tensor* w, const float* x, float* y, int N, int K) {
    return kq_linear_dispatch_add(w, x, NULL, y, N, K);
}

int kq_linear_multix(const kq_tensor* w, const float* const* xs, float* const* ys,
                     int B, int N, int K) {
    if (!w) return kq_fail("NULL tensor");
    if (B < 1) return kq_fail("kq_linear_multix: B=%d", B);
    if (check_shape((int)w->type, N, K) || kq_ready()) return -1;
    const void* dw = tensor_dev(w, N, K);
    if (!dw) return -1;
    if (grow(&g_kq.d_x, &g_kq.cap_x, (size_t)B * K) ||
        grow(&g_kq.d_y, &g_kq.cap_y, (size_t)B * N)) return -1;
    for (int s = 0; s < B; s++)
        if (h2d(g_kq.d_x + (size_t)s * K, xs[s], (size_t)K)) return -1;
    if (kq_gemv_multix_dev((int)w->type, dw, g_kq.d_x, g_kq.d_y, B, N, K, g_kq.stream)) return -1;
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
    for (int i = 0; i < nw; i++)
        if (kq_linear_dispatch(ws[i], x, ys[i], Ns[i], K)) return -1;
    return 0;
}
