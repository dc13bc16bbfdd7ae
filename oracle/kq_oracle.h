/*
 * kq_oracle.h -- CPU restatement of stratum's scalar k-quant routines.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (stratum_amd/, include/)
 * links or calls this code; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and only as the checker or as the
 * timed CPU baseline.  It is compiled with strict IEEE binary32/binary64
 * semantics (-O2 -ffp-contract=off -fno-fast-math), so every product and
 * every sum is rounded exactly where the reference's C source rounds it.
 *
 * Reference functions restated here (paths under
 * /root/reference/stratum/native/):
 *   stratum_q4k.h:24-55   q4k_fp16_to_fp32        -> ko_fp16_to_fp32
 *   stratum_q4k.h:57-65   q4k_get_scale_min       -> ko_q4k_scale_min
 *   stratum_q4k.h:67-93   q4k_dequant_*_scalar    -> ko_dequant_row (Q4_K)
 *   stratum_q4k.h:95-131  q4k_dot_row_scalar      -> ko_dot_row (Q4_K)
 *   stratum_q6k.h:17-36   q6k_dequant_block_scalar-> ko_dequant_row (Q6_K)
 *   stratum_q6k.h:38-73   q6k_dot_row_scalar      -> ko_dot_row (Q6_K)
 *   stratum_q2k.h:16-42   q2k_dequant_block_scalar-> ko_dequant_row (Q2_K)
 *   stratum_q2k.h:44-89   q2k_dot_row_scalar      -> ko_dot_row (Q2_K)
 *   stratum_q5k.h:18-82   q5k_dequant/dot_row_scalar -> ko_dequant_row / ko_dot_row (Q5_K)
 *   stratum_q3k.h:17-99   q3k_unpack_scales, dequant/dot_row_scalar -> (Q3_K)
 *   stratum_q8_0.h:14-33  q8_0_dequant/dot_row_scalar -> (Q8_0, eight blocks per 256)
 *   stratum_linear.h:491-505 st_linear_f16 (binary64 element-order sum) -> (F16)
 *   stratum_linear.h:508-512 st_linear_f32 (cblas_sgemv; restated as the
 *                          binary64 sum of exact products: parity pinned
 *                          by closed forms only, not against the BLAS bits)
 *   stratum_q4k_neon.h:261-276 / stratum_q6k_neon.h:117-133 the int8
 *                          activation quantizers -> ko_quantize_x_q8
 *   stratum_q4k_neon.h:365-407 / stratum_q6k_neon.h:265-317 the int8 GEMV
 *                          (sdot_f) -> ko_gemv_i8(..., sdot_f = 1)
 *   tools_gguf_nib_convert.c:99-120  Q2_K -> type 42 byte permutation
 *                                     -> ko_q2k_to_nib / ko_nib_to_q2k
 *   stratum_linear.h:201-228 ST_PAR_ROWS 64-row tickets -> ko_gemv threads
 *   stratum_arch_moe.inc.c:368-385 moe_topk        -> ko_moe_topk
 *   stratum_engine.h:395-423 stratum_softmax_inplace -> ko_softmax
 *   stratum_engine.h:373-392 stratum_swiglu          -> ko_swiglu
 *   stratum_arch_moe.inc.c:689-743, 1213-1226 the FFN step's router,
 *                          accumulate and residual -> ko_moe_ffn, ko_moe_combine
 *                          (stratum_engine.h needs macOS headers and does not
 *                          build here: pinned by closed forms only)
 *
 * Pinning (what checks each function, see tests/test_oracle_*.py):
 *   - golden vectors in tests/golden/ written by the reference's own scalar
 *     headers compiled from /root/reference (oracle/_ref), bit-exact;
 *   - direct comparison against oracle/_ref when it is built;
 *   - closed forms: exhaustive fp16 vs numpy.float16, exhaustive scale
 *     decode, x = e_i gives the dequantized column, linearity checks, the
 *     type-42 permutation round trip and value identity.
 */
#ifndef KQ_ORACLE_H
#define KQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (stratum_gguf.h:20-49). */
enum {
    KO_F32 = 0,
    KO_F16 = 1,
    KO_Q8_0 = 8,
    KO_Q2_K = 10,
    KO_Q3_K = 11,
    KO_Q4_K = 12,
    KO_Q5_K = 13,
    KO_Q6_K = 14,
    KO_Q2K_NIB = 42,
};

/* bytes per 256-weight super-block for a type; 0 for unsupported types */
int ko_block_bytes(int type);

float ko_fp16_to_fp32(uint16_t h);
void ko_q4k_scale_min(int j, const uint8_t* scales, uint8_t* sc, uint8_t* m);
/* ko_q4k_scale_min over every value of the bytes idx[0..nidx) (nidx <= 3),
 * the other scale bytes fixed to bg[12]: out[2c], out[2c+1] = sc, m of
 * combination c = sum_i byte_i << 8i (an exhaustive-test helper) */
void ko_q4k_scale_min_sweep(int j, const int* idx, int nidx, const uint8_t* bg, uint8_t* out);

/* the Q3_K 6-bit scale of group g over every value of the bytes idx[]
 * (nidx <= 3), others fixed to bg[12] (an exhaustive-test helper) */
void ko_q3k_scale_sweep(int g, const int* idx, int nidx, const uint8_t* bg, uint8_t* out);

/* one row of K weights (K % 256 == 0) */
void ko_dequant_row(int type, const uint8_t* row, int K, float* y);
float ko_dot_row(int type, const uint8_t* row, int K, const float* x);
/* same sum, returned before the final (float) rounding */
double ko_dot_row_f64(int type, const uint8_t* row, int K, const float* x);

/* y[r] = dot(row r, x) for r < N; rows contiguous.  nthreads <= 1 runs on
 * the calling thread; otherwise 64-row atomic tickets over pthreads.
 * add != NULL gives y[r] = add[r] + dot (stratum_linear.h:568-632). */
int ko_gemv(int type, const uint8_t* w, const float* x, const float* add,
            float* y, int N, int K, int nthreads);

/* B streams over one weight: ys[s*N + r] = dot(row r, xs[s*K ...]) */
int ko_gemv_multix(int type, const uint8_t* w, const float* xs, float* ys,
                   int B, int N, int K, int nthreads);

/* int8 activations: q4k_quantize_x_q8 (G = 32) / q6k_quantize_x_q8_g16
 * (G = 16), and the GEMV of the int8 mode for Q4_K / Q6_K: sdot_f != 0 in
 * the reference's order (q4k_dot_row_sdot_f, q6k_dot_row_sdot_f), else the
 * GPU's (binary64 terms); mag, if not NULL, gets each row's sum |term| */
void ko_quantize_x_q8(const float* x, int K, int G, int8_t* xq, float* xscale);
int ko_gemv_i8(int type, const uint8_t* w, const float* x, const float* add, float* y,
               double* mag, int N, int K, int sdot_f);
/* int8 MULTISEQ (st_linear_multix under use_sdot, B >= 2; Q4_K / Q6_K):
 * ys[s * N + r], the reference's multix_pack arithmetic. 0, or -1. */
int ko_gemv_i8_multix(int type, const uint8_t* w, const float* xs, float* ys, int B, int N,
                      int K);

/* type-42 permutation (148-byte blocks) and its inverse */
void ko_q2k_to_nib(const uint8_t* q2k, uint8_t* nib, int64_t nblocks);
void ko_nib_to_q2k(const uint8_t* nib, uint8_t* q2k, int64_t nblocks);

/* top-k with strict '>' replacement: ties keep the lower expert id */
void ko_moe_topk(const float* w, int E, int K, int* sel, float* selw);

/* MoE FFN step pieces: softmax in place (libm expf, binary64 sum in
 * order), SwiGLU, rank-ordered combine + residual, and the whole step */
void ko_softmax(float* x, int N);
void ko_swiglu(const float* g, const float* u, float* y, int64_t n);
void ko_moe_combine(const float* o, const int* sel, const float* selw, const float* resid,
                    float* x, int B, int k, int H);
typedef struct ko_moe_ffn_desc {
    int n_embed, n_ff, n_experts, k;
    int router_type;
    const uint8_t* router;
    int gate_type, up_type, down_type;
    const uint8_t* gate;
    const uint8_t* up;
    const uint8_t* down;
    int64_t gate_stride, up_stride, down_stride;
} ko_moe_ffn_desc;
int ko_moe_ffn(const ko_moe_ffn_desc* f, const float* xn, float* x, int B, int* sel,
               float* selw, float* probs, float* g, float* u, float* act, float* ffo);

#ifdef __cplusplus
}
#endif
#endif
