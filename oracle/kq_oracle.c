/*
 * kq_oracle.c -- CPU restatement of stratum's scalar k-quant routines.
 *
 * TEST INFRASTRUCTURE ONLY (see kq_oracle.h).  Build with
 *   gcc -O2 -std=c11 -ffp-contract=off -fno-fast-math
 * so that every binary32 product and sum rounds where the reference's C
 * source rounds it (x86-64 without -mfma never contracts anyway).
 *
 * The arithmetic follows the reference statement by statement; the code
 * is organised by 32- or 16-weight sub-block rather than by the
 * reference's pointer walks.  Reference lines are cited per function.
 *
 * Pinning (tests/test_oracle*.py): every function is checked against the
 * reference build (oracle/_ref), golden vectors, closed forms or exact-input
 * identities.  One point is parity unpinned: in ko_gemv_i8_multix the
 * association of each Q4_K term's three binary32 products follows the
 * reference source as read, and no independent check separates it from
 * another association (the NEON source does not build here).
 */
#define _GNU_SOURCE
#include "kq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

int ko_block_bytes(int type) {
    switch (type) {   /* stratum_gguf.h:57-79, per 256 weights */
    case KO_Q2_K: return 84;
    case KO_Q3_K: return 110;
    case KO_Q4_K: return 144;
    case KO_Q5_K: return 176;
    case KO_Q6_K: return 210;
    case KO_Q8_0: return 8 * 34;     /* eight 32-weight blocks */
    case KO_F16: return 512;
    case KO_F32: return 1024;
    case KO_Q2K_NIB: return 148;
    default: return 0;
    }
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Exact IEEE binary16 -> binary32 widening (stratum_q4k.h:24-55):
 * zero, subnormal (renormalised), normal, inf and NaN (payload << 13). */
float ko_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    int e = (h >> 10) & 31;
    uint32_t frac = h & 0x3ffu;
    uint32_t bits;
    if (e == 31) {
        bits = sign | 0x7f800000u | (frac << 13);
    } else if (e != 0) {
        bits = sign | ((uint32_t)(e + 112) << 23) | (frac << 13);
    } else if (frac == 0) {
        bits = sign;
    } else {
        /* subnormal: shift the leading one up to bit 10 */
        int shift = 0;
        while (!(frac & 0x400u)) { frac <<= 1; shift++; }
        bits = sign | ((uint32_t)(113 - shift) << 23) | ((frac & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* 6-bit scale and min of Q4_K sub-block j (0..7) from the 12 packed bytes
 * (stratum_q4k.h:57-65).  Sub-blocks 0..3 keep their low six bits in bytes
 * 0..3 (scale) and 4..7 (min); sub-blocks 4..7 take a nibble from bytes
 * 8..11 and their top two bits from the high bits of bytes 0..7. */
void ko_q4k_scale_min(int j, const uint8_t* s, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = (uint8_t)(s[j] & 0x3f);
        *m = (uint8_t)(s[4 + j] & 0x3f);
    } else {
        int t = j - 4;
        *sc = (uint8_t)((s[8 + t] & 0x0f) | ((s[t] >> 6) << 4));
        *m = (uint8_t)((s[8 + t] >> 4) | ((s[4 + t] >> 6) << 4));
    }
}

/* Test sweep (no reference counterpart): ko_q4k_scale_min for sub-block j
 * on every value of the nidx bytes idx[] of the 12 scale bytes (the others
 * fixed to bg[]), combination c = sum_i byte_i << (8 i); out[2c] = sc,
 * out[2c + 1] = m.  2^(8 nidx) combinations, nidx <= 3. */
void ko_q4k_scale_min_sweep(int j, const int* idx, int nidx, const uint8_t* bg, uint8_t* out) {
    uint8_t s[12];
    memcpy(s, bg, 12);
    const uint32_t n = 1u << (8 * nidx);
    for (uint32_t c = 0; c < n; c++) {
        for (int i = 0; i < nidx; i++) s[idx[i]] = (uint8_t)(c >> (8 * i));
        ko_q4k_scale_min(j, s, &out[2 * (size_t)c], &out[2 * (size_t)c + 1]);
    }
}

/* ---------------------------------------------------------------- Q4_K */
/* block_q4_K (stratum_q4k.h:16-22): d@0, dmin@2, scales[12]@4, qs[128]@16.
 * Sub-block s (32 weights, positions 32s..32s+31) reads qs bytes
 * 32*(s/2) .. +31, low nibble for even s, high nibble for odd s. */
static inline int q4k_q(const uint8_t* blk, int s, int l) {
    uint8_t b = blk[16 + 32 * (s >> 1) + l];
    return (s & 1) ? (b >> 4) : (b & 0x0f);
}

static void q4k_dequant_block(const uint8_t* blk, float* y) {
    /* stratum_q4k.h:67-84: y = fl(fl(d*sc)*q) - fl(dmin*m) */
    const float d = ko_fp16_to_fp32(rd16(blk));
    const float dmin = ko_fp16_to_fp32(rd16(blk + 2));
    for (int s = 0; s < 8; s++) {
        uint8_t sc, m;
        ko_q4k_scale_min(s, blk + 4, &sc, &m);
        const float ds = d * (float)sc;
        const float dm = dmin * (float)m;
        for (int l = 0; l < 32; l++) y[32 * s + l] = ds * (float)q4k_q(blk, s, l) - dm;
    }
}

static double q4k_dot(const uint8_t* row, int K, const float* x) {
    /* stratum_q4k.h:95-131 */
    double dot = 0.0;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 144;
        const float* xb = x + (size_t)b * 256;
        const float d = ko_fp16_to_fp32(rd16(blk));
        const float dmin = ko_fp16_to_fp32(rd16(blk + 2));
        for (int s = 0; s < 8; s++) {
            uint8_t sc, m;
            ko_q4k_scale_min(s, blk + 4, &sc, &m);
            const float ds = d * (float)sc;
            const float dm = dmin * (float)m;
            float acc = 0.0f, xsum = 0.0f;
            for (int l = 0; l < 32; l++) {
                acc += (float)q4k_q(blk, s, l) * xb[32 * s + l];
                xsum += xb[32 * s + l];
            }
            dot += (double)(ds * acc - dm * xsum);
        }
    }
    return dot;
}

/* ---------------------------------------------------------------- Q6_K */
/* block_q6_K (stratum_q6k.h:9-15): ql[128]@0, qh[64]@128, int8
 * scales[16]@192, d@208.  Position p = 128h + 32t + l (h half, t 0..3,
 * l 0..31): low four bits from ql[64h + l + 32(t&1)] (nibble t>>1), high
 * two bits from qh[32h + l] bits 2t..2t+1, value minus 32; scale index
 * 8h + 2t + l/16. */
static inline int q6k_q(const uint8_t* blk, int h, int t, int l) {
    uint8_t lo = blk[64 * h + l + 32 * (t & 1)];
    uint8_t hi = blk[128 + 32 * h + l];
    int q = ((lo >> (4 * (t >> 1))) & 0x0f) | (((hi >> (2 * t)) & 3) << 4);
    return q - 32;
}

static void q6k_dequant_block(const uint8_t* blk, float* y) {
    /* stratum_q6k.h:17-36: y = fl(fl(d*s)*q) */
    const float d = ko_fp16_to_fp32(rd16(blk + 208));
    const int8_t* sc = (const int8_t*)(blk + 192);
    for (int h = 0; h < 2; h++)
        for (int t = 0; t < 4; t++)
            for (int l = 0; l < 32; l++)
                y[128 * h + 32 * t + l] =
                    d * (float)sc[8 * h + 2 * t + l / 16] * (float)q6k_q(blk, h, t, l);
}

static double q6k_dot(const uint8_t* row, int K, const float* x) {
    /* stratum_q6k.h:38-73: eight binary32 sums of 16 products per half,
     * then dot += ((double)d * (double)s) * (double)a in (is, t) order. */
    double dot = 0.0;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 210;
        const float* xb = x + (size_t)b * 256;
        const float d = ko_fp16_to_fp32(rd16(blk + 208));
        const int8_t* sc = (const int8_t*)(blk + 192);
        for (int h = 0; h < 2; h++) {
            float a[4][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}, {0.0f, 0.0f}, {0.0f, 0.0f}};
            for (int l = 0; l < 32; l++)
                for (int t = 0; t < 4; t++)
                    a[t][l / 16] += (float)q6k_q(blk, h, t, l) * xb[128 * h + 32 * t + l];
            for (int is = 0; is < 2; is++)
                for (int t = 0; t < 4; t++)
                    dot += (double)d * (double)sc[8 * h + is + 2 * t] * a[t][is];
        }
    }
    return dot;
}

/* ---------------------------------------------------------------- Q2_K */
/* block_q2_K (stratum_q2k.h:8-14): scales[16]@0, qs[64]@16, d@80,
 * dmin@82.  Group g = 8s + 2j + h (16 weights at 128s + 32j + 16h + l):
 * q = (qs[32s + 16h + l] >> 2j) & 3, scale byte scales[g] (low nibble
 * scale, high nibble min). */
static inline int q2k_q(const uint8_t* blk, int g, int l) {
    int s = g >> 3, j = (g >> 1) & 3, h = g & 1;
    return (blk[16 + 32 * s + 16 * h + l] >> (2 * j)) & 3;
}

/* type 42 (tools_gguf_nib_convert.c:99-120; stratum_q2k_neon.h:265-291):
 * scales[16]@0, nibbles[128]@16, d@144, dmin@146.  Position p lives in
 * byte 16 + 16*(p/32) + p%16, low nibble when p%32 < 16, else high. */
static inline int nib_q(const uint8_t* blk, int p) {
    uint8_t b = blk[16 + 16 * (p >> 5) + (p & 15)];
    return (p & 16) ? (b >> 4) : (b & 0x0f);
}

static inline int q2_pos(int g, int l) {
    return 128 * (g >> 3) + 32 * ((g >> 1) & 3) + 16 * (g & 1) + l;
}

static void q2_dequant_block(const uint8_t* blk, int nib, float* y) {
    /* stratum_q2k.h:16-42: y = fl(fl(d*sc)*q) - fl(dmin*m) */
    const int doff = nib ? 144 : 80;
    const float d = ko_fp16_to_fp32(rd16(blk + doff));
    const float dmin = ko_fp16_to_fp32(rd16(blk + doff + 2));
    for (int g = 0; g < 16; g++) {
        const uint8_t scb = blk[g];
        const float dl = d * (float)(scb & 0x0f);
        const float ml = dmin * (float)(scb >> 4);
        for (int l = 0; l < 16; l++) {
            int p = q2_pos(g, l);
            int q = nib ? nib_q(blk, p) : q2k_q(blk, g, l);
            y[p] = dl * (float)q - ml;
        }
    }
}

static double q2_dot(const uint8_t* row, int K, const float* x, int nib) {
    /* stratum_q2k.h:44-89, groups in (s, j, h) order */
    const int bb = nib ? 148 : 84, doff = nib ? 144 : 80;
    double dot = 0.0;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * bb;
        const float* xb = x + (size_t)b * 256;
        const float d = ko_fp16_to_fp32(rd16(blk + doff));
        const float dmin = ko_fp16_to_fp32(rd16(blk + doff + 2));
        for (int g = 0; g < 16; g++) {
            const uint8_t scb = blk[g];
            const float dl = d * (float)(scb & 0x0f);
            const float ml = dmin * (float)(scb >> 4);
            float qx = 0.0f, sx = 0.0f;
            for (int l = 0; l < 16; l++) {
                int p = q2_pos(g, l);
                int q = nib ? nib_q(blk, p) : q2k_q(blk, g, l);
                qx += (float)q * xb[p];
                sx += xb[p];
            }
            dot += (double)(dl * qx - ml * sx);
        }
    }
    return dot;
}

/* ---------------------------------------------------------------- Q5_K */
/* block_q5_K (stratum_q5k.h:9-16): d@0, dmin@2, scales[12]@4 (Q4_K's
 * 6-bit packing), qh[32]@16, qs[128]@48.  Chunk j (64 weights at 64j):
 * sub-block 2j takes the low nibbles of qs[32j + l] plus 16 when bit 2j of
 * qh[l] is set; sub-block 2j+1 the high nibbles plus bit 2j+1. */
static inline int q5k_q(const uint8_t* blk, int s, int l) {
    const int j = s >> 1;
    const uint8_t b = blk[48 + 32 * j + l];
    const int lo = (s & 1) ? (b >> 4) : (b & 0x0f);
    return lo + ((blk[16 + l] >> s) & 1) * 16;
}

static void q5k_dequant_block(const uint8_t* blk, float* y) {
    /* stratum_q5k.h:18-42: y = fl(fl(d*sc)*q) - fl(dmin*m) */
    const float d = ko_fp16_to_fp32(rd16(blk));
    const float dmin = ko_fp16_to_fp32(rd16(blk + 2));
    for (int s = 0; s < 8; s++) {
        uint8_t sc, m;
        ko_q4k_scale_min(s, blk + 4, &sc, &m);
        const float ds = d * (float)sc;
        const float dm = dmin * (float)m;
        for (int l = 0; l < 32; l++) y[32 * s + l] = ds * (float)q5k_q(blk, s, l) - dm;
    }
}

static double q5k_dot(const uint8_t* row, int K, const float* x) {
    /* stratum_q5k.h:44-82: per 64-weight chunk, one binary32 expression
     * ((d1*qx1 - m1*sx1) + d2*qx2) - m2*sx2, then widened and added */
    double dot = 0.0;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 176;
        const float* xb = x + (size_t)b * 256;
        const float d = ko_fp16_to_fp32(rd16(blk));
        const float dmin = ko_fp16_to_fp32(rd16(blk + 2));
        for (int j = 0; j < 4; j++) {
            uint8_t sc1, mn1, sc2, mn2;
            ko_q4k_scale_min(2 * j, blk + 4, &sc1, &mn1);
            ko_q4k_scale_min(2 * j + 1, blk + 4, &sc2, &mn2);
            const float d1 = d * (float)sc1, m1 = dmin * (float)mn1;
            const float d2 = d * (float)sc2, m2 = dmin * (float)mn2;
            float qx1 = 0.0f, sx1 = 0.0f, qx2 = 0.0f, sx2 = 0.0f;
            for (int l = 0; l < 32; l++) {
                qx1 += (float)q5k_q(blk, 2 * j, l) * xb[64 * j + l];
                sx1 += xb[64 * j + l];
            }
            for (int l = 0; l < 32; l++) {
                qx2 += (float)q5k_q(blk, 2 * j + 1, l) * xb[64 * j + 32 + l];
                sx2 += xb[64 * j + 32 + l];
            }
            dot += (double)(d1 * qx1 - m1 * sx1 + d2 * qx2 - m2 * sx2);
        }
    }
    return dot;
}

/* ---------------------------------------------------------------- Q3_K */
/* block_q3_K (stratum_q3k.h:8-14): hmask[32]@0, qs[64]@32, scales[12]@96,
 * d@108.  Group g = 8s + 2j + h (16 weights at 128s + 32j + 16h + l):
 * low two bits (qs[32s + 16h + l] >> 2j) & 3, minus 4 unless bit 4s + j
 * of hmask[16h + l] is set.  Scale g is 6 bits: the low nibble from byte
 * g%4 (g < 4, 8 <= g < 12: low nibble; otherwise high nibble) of bytes
 * 0..7, the top two bits from byte 8 + g%4 (stratum_q3k.h:17-28). */
static inline int q3k_scale(const uint8_t* sc12, int g) {
    const int w = g >> 2, bi = g & 3;
    const uint8_t lo = w == 0 ? (sc12[bi] & 0x0f) : w == 1 ? (sc12[4 + bi] & 0x0f)
                     : w == 2 ? (sc12[bi] >> 4) : (sc12[4 + bi] >> 4);
    const uint8_t hi = (sc12[8 + bi] >> (2 * w)) & 3;
    return (int)(lo | (hi << 4));
}

/* Test sweep (no reference counterpart): q3k_scale for group g on every
 * value of the nidx bytes idx[] of the 12 scale bytes (the others fixed to
 * bg[]); out[c] = the 6-bit scale of combination c = sum_i byte_i << 8i. */
void ko_q3k_scale_sweep(int g, const int* idx, int nidx, const uint8_t* bg, uint8_t* out) {
    uint8_t s[12];
    memcpy(s, bg, 12);
    const uint32_t n = 1u << (8 * nidx);
    for (uint32_t c = 0; c < n; c++) {
        for (int i = 0; i < nidx; i++) s[idx[i]] = (uint8_t)(c >> (8 * i));
        out[c] = (uint8_t)q3k_scale(s, g);
    }
}

static inline int q3k_q(const uint8_t* blk, int g, int l) {
    const int s = g >> 3, j = (g >> 1) & 3, h = g & 1;
    const int lo = (blk[32 + 32 * s + 16 * h + l] >> (2 * j)) & 3;
    const int hb = (blk[16 * h + l] >> (4 * s + j)) & 1;
    return lo - (hb ? 0 : 4);
}

static void q3k_dequant_block(const uint8_t* blk, float* y) {
    /* stratum_q3k.h:30-56: y = fl(fl(d*(sc-32))*q) */
    const float d = ko_fp16_to_fp32(rd16(blk + 108));
    for (int g = 0; g < 16; g++) {
        const float dl = d * (float)(q3k_scale(blk + 96, g) - 32);
        for (int l = 0; l < 16; l++) y[q2_pos(g, l)] = dl * (float)q3k_q(blk, g, l);
    }
}

static double q3k_dot(const uint8_t* row, int K, const float* x) {
    /* stratum_q3k.h:58-99, groups in (s, j, h) order:
     * dot += (double)fl(dl * acc), acc the binary32 sum of 16 products */
    double dot = 0.0;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 110;
        const float* xb = x + (size_t)b * 256;
        const float d = ko_fp16_to_fp32(rd16(blk + 108));
        for (int g = 0; g < 16; g++) {
            const float dl = d * (float)(q3k_scale(blk + 96, g) - 32);
            float acc = 0.0f;
            for (int l = 0; l < 16; l++) acc += (float)q3k_q(blk, g, l) * xb[q2_pos(g, l)];
            dot += (double)(dl * acc);
        }
    }
    return dot;
}

/* ---------------------------------------------------------------- Q8_0 */
/* block_q8_0 (stratum_q8_0.h:8-12): d@0, int8 qs[32]@2, 34 bytes per 32
 * weights. */
static void q8_0_dequant_block(const uint8_t* blk, float* y) {
    /* stratum_q8_0.h:14-17 */
    const float d = ko_fp16_to_fp32(rd16(blk));
    for (int k = 0; k < 32; k++) y[k] = d * (float)(int8_t)blk[2 + k];
}

static double q8_0_dot(const uint8_t* row, int K, const float* x) {
    /* stratum_q8_0.h:19-33: dot += (double)fl(d * acc) per 32 weights */
    double dot = 0.0;
    for (int b = 0; b < K / 32; b++) {
        const uint8_t* blk = row + (size_t)b * 34;
        const float d = ko_fp16_to_fp32(rd16(blk));
        float acc = 0.0f;
        for (int k = 0; k < 32; k++) acc += (float)(int8_t)blk[2 + k] * x[32 * b + k];
        dot += (double)(d * acc);
    }
    return dot;
}

/* ----------------------------------------------------------- F16 / F32 */
static double f16_dot(const uint8_t* row, int K, const float* x) {
    /* stratum_linear.h:491-505 (st_linear_f16): every product exact in
     * binary64, summed in binary64 in element order */
    double acc = 0.0;
    for (int c = 0; c < K; c++) acc += (double)ko_fp16_to_fp32(rd16(row + 2 * c)) * (double)x[c];
    return acc;
}

static double f32_dot(const uint8_t* row, int K, const float* x) {
    /* stratum_linear.h:508-512 hands F32 to cblas_sgemv, whose summation
     * order is the BLAS library's.  Restated as the binary64 sum of the
     * exact products in element order: the value every ordering
     * approximates, within K binary32 roundings of sum |w x|. */
    double acc = 0.0;
    for (int c = 0; c < K; c++) {
        float w;
        memcpy(&w, row + 4 * (size_t)c, 4);
        acc += (double)w * (double)x[c];
    }
    return acc;
}

/* -------------------------------------------------- int8 activations */
/* q4k_quantize_x_q8 (stratum_q4k_neon.h:230-277; its portable form
 * :261-276) with G = 32, and q6k_quantize_x_q8_g16 (stratum_q6k_neon.h:
 * 117-133) with G = 16: per group amax = max |x|, scale = fl(amax / 127),
 * inv = scale > 0 ? fl(1 / scale) : 0, q = clamp(rne(fl(x * inv)),
 * -128, 127) (lrintf in the default rounding mode; vcvtnq_s32_f32 on NEON
 * also rounds to nearest, ties to even). */
void ko_quantize_x_q8(const float* x, int K, int G, int8_t* xq, float* xscale) {
    for (int g = 0; g < K / G; g++) {
        const float* xp = x + (size_t)g * G;
        float amax = 0.0f;
        for (int i = 0; i < G; i++) {
            const float a = fabsf(xp[i]);
            if (a > amax) amax = a;
        }
        const float scale = amax / 127.0f;
        const float inv = (scale > 0.0f) ? (1.0f / scale) : 0.0f;
        xscale[g] = scale;
        for (int i = 0; i < G; i++) {
            int v = (int)lrintf(xp[i] * inv);
            if (v > 127) v = 127;
            if (v < -128) v = -128;
            xq[(size_t)g * G + i] = (int8_t)v;
        }
    }
}

/* integer sums of each group of G quantized values (q4k_sum_i8_32,
 * stratum_q4k_neon.h:414-420; q6k_xsum16_i8, stratum_q6k_neon.h:261-264) */
static void xsums(const int8_t* xq, int K, int G, int32_t* out) {
    for (int g = 0; g < K / G; g++) {
        int32_t t = 0;
        for (int i = 0; i < G; i++) t += xq[(size_t)g * G + i];
        out[g] = t;
    }
}

/* Q4_K with int8 activations in the reference's order, q4k_dot_row_sdot_f
 * (stratum_q4k_neon.h:365-407): per 64-weight chunk the exact integer dots
 * L, H of the two sub-blocks, coefficients fl(fl(d*sc)*xs) and
 * fl(fl(-dmin*m)*xs), four binary32 lanes each a fused multiply-add chain
 * over the chunks ([L, xsum_lo, H, xsum_hi] times the coefficients), then
 * (f0 + f1) + (f2 + f3) (vaddvq_f32's pairwise reduction).  *mag gets the
 * sum of |term| (for error bounds). */
static float q4k_sdot_f(const uint8_t* row, int K, const int8_t* xq, const float* xs,
                        const int32_t* xsum, double* mag) {
    float f[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    double m_ = 0.0;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 144;
        const float d = ko_fp16_to_fp32(rd16(blk)), dmin = ko_fp16_to_fp32(rd16(blk + 2));
        for (int j = 0; j < 4; j++) {
            const int g0 = 8 * b + 2 * j, g1 = g0 + 1;
            uint8_t sc1, mn1, sc2, mn2;
            ko_q4k_scale_min(2 * j, blk + 4, &sc1, &mn1);
            ko_q4k_scale_min(2 * j + 1, blk + 4, &sc2, &mn2);
            int32_t L = 0, H = 0;
            for (int l = 0; l < 32; l++) {
                L += (int32_t)(blk[16 + 32 * j + l] & 15) * xq[32 * g0 + l];
                H += (int32_t)(blk[16 + 32 * j + l] >> 4) * xq[32 * g1 + l];
            }
            const float c[4] = {d * (float)sc1 * xs[g0], -dmin * (float)mn1 * xs[g0],
                                d * (float)sc2 * xs[g1], -dmin * (float)mn2 * xs[g1]};
            const int32_t t[4] = {L, xsum[g0], H, xsum[g1]};
            for (int k = 0; k < 4; k++) {
                f[k] = fmaf((float)t[k], c[k], f[k]);
                m_ += fabs((double)t[k] * (double)c[k]);
            }
        }
    }
    if (mag) *mag = m_;
    return (f[0] + f[1]) + (f[2] + f[3]);
}

/* Q6_K with int8 activations per 16, q6k_dot_row_sdot_f
 * (stratum_q6k_neon.h:265-317): per (half, is) the four runs t hold the
 * unsigned 6-bit values (0..63); g4[t] = their exact dot with the run's 16
 * quantized values minus 32 * that group's x sum; coefficient
 * fl(fl(d * sc[g]) * xs[g]) for group g = 8 half + is + 2t; lane t of a
 * binary32 fused multiply-add chain; then (f0 + f1) + (f2 + f3). */
static float q6k_sdot_f(const uint8_t* row, int K, const int8_t* xq, const float* xs,
                        const int32_t* xsum, double* mag) {
    float f[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    double m_ = 0.0;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 210;
        const float d = ko_fp16_to_fp32(rd16(blk + 208));
        const int8_t* sc = (const int8_t*)(blk + 192);
        for (int h = 0; h < 2; h++)
            for (int is = 0; is < 2; is++) {
                for (int t = 0; t < 4; t++) {
                    const int g = 16 * b + 8 * h + is + 2 * t;
                    int32_t acc = 0;
                    for (int l = 0; l < 16; l++)
                        acc += (int32_t)(q6k_q(blk, h, t, 16 * is + l) + 32) * xq[16 * g + l];
                    acc -= 32 * xsum[g];
                    const float c = d * (float)sc[8 * h + is + 2 * t] * xs[g];
                    f[t] = fmaf((float)acc, c, f[t]);
                    m_ += fabs((double)acc * (double)c);
                }
            }
    }
    if (mag) *mag = m_;
    return (f[0] + f[1]) + (f[2] + f[3]);
}

/* The int8-activation GEMV as the GPU computes it: the same quantized x,
 * exact integer dots and coefficients as above, each sub-block term
 * (Q4_K: c1*L + c2*xsum; Q6_K: c*g4) formed exactly in binary64 and the
 * terms summed in binary64 (here in element order; the GPU's grouping of
 * that binary64 sum is its own, as for the exact path). */
static double q4k_i8_dot(const uint8_t* row, int K, const int8_t* xq, const float* xs,
                         const int32_t* xsum) {
    double dot = 0.0;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 144;
        const float d = ko_fp16_to_fp32(rd16(blk)), dmin = ko_fp16_to_fp32(rd16(blk + 2));
        for (int s = 0; s < 8; s++) {
            const int g = 8 * b + s;
            uint8_t sc, mn;
            ko_q4k_scale_min(s, blk + 4, &sc, &mn);
            int32_t L = 0;
            for (int l = 0; l < 32; l++) L += (int32_t)q4k_q(blk, s, l) * xq[32 * g + l];
            const float c1 = d * (float)sc * xs[g], c2 = -dmin * (float)mn * xs[g];
            dot += fma((double)c1, (double)L, (double)c2 * (double)xsum[g]);
        }
    }
    return dot;
}

static double q6k_i8_dot(const uint8_t* row, int K, const int8_t* xq, const float* xs,
                         const int32_t* xsum) {
    double dot = 0.0;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 210;
        const float d = ko_fp16_to_fp32(rd16(blk + 208));
        const int8_t* sc = (const int8_t*)(blk + 192);
        for (int h = 0; h < 2; h++)
            for (int is = 0; is < 2; is++)
                for (int t = 0; t < 4; t++) {
                    const int g = 16 * b + 8 * h + is + 2 * t;
                    int32_t acc = 0;
                    for (int l = 0; l < 16; l++)
                        acc += (int32_t)(q6k_q(blk, h, t, 16 * is + l) + 32) * xq[16 * g + l];
                    acc -= 32 * xsum[g];
                    const float c = d * (float)sc[8 * h + is + 2 * t] * xs[g];
                    dot += (double)c * (double)acc;
                }
    }
    return dot;
}

/* Q5_K with int8 activations per 32, q5k_dot_row_sdot_f
 * (stratum_q5k_neon.h:158-204): Q4_K's lanes with the 5-bit values
 * q5k_q (nibble plus 16 times the qh bit, 0..31) in the exact dots. */
static float q5k_sdot_f(const uint8_t* row, int K, const int8_t* xq, const float* xs,
                        const int32_t* xsum, double* mag) {
    float f[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    double m_ = 0.0;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 176;
        const float d = ko_fp16_to_fp32(rd16(blk)), dmin = ko_fp16_to_fp32(rd16(blk + 2));
        for (int j = 0; j < 4; j++) {
            const int g0 = 8 * b + 2 * j, g1 = g0 + 1;
            uint8_t sc1, mn1, sc2, mn2;
            ko_q4k_scale_min(2 * j, blk + 4, &sc1, &mn1);
            ko_q4k_scale_min(2 * j + 1, blk + 4, &sc2, &mn2);
            int32_t L = 0, H = 0;
            for (int l = 0; l < 32; l++) {
                L += (int32_t)q5k_q(blk, 2 * j, l) * xq[32 * g0 + l];
                H += (int32_t)q5k_q(blk, 2 * j + 1, l) * xq[32 * g1 + l];
            }
            const float c[4] = {d * (float)sc1 * xs[g0], -dmin * (float)mn1 * xs[g0],
                                d * (float)sc2 * xs[g1], -dmin * (float)mn2 * xs[g1]};
            const int32_t t[4] = {L, xsum[g0], H, xsum[g1]};
            for (int k = 0; k < 4; k++) {
                f[k] = fmaf((float)t[k], c[k], f[k]);
                m_ += fabs((double)t[k] * (double)c[k]);
            }
        }
    }
    if (mag) *mag = m_;
    return (f[0] + f[1]) + (f[2] + f[3]);
}

/* Q3_K with int8 activations per 32, q3k_dot_row_sdot_f
 * (stratum_q3k_neon.h:84-125): 16-weight group gg (positions 16 gg .. of
 * its block, q3k_q's signed values -4..3) dotted exactly with the
 * quantized x there; coefficient fl(fl(d * (sc - 32)) * xs) with the
 * scale of the 32-group holding it; four binary32 fused multiply-add
 * lanes t = gg % 4; then (f0 + f1) + (f2 + f3).  No min term. */
static float q3k_sdot_f(const uint8_t* row, int K, const int8_t* xq, const float* xs,
                        double* mag) {
    float f[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    double m_ = 0.0;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 110;
        const float d = ko_fp16_to_fp32(rd16(blk + 108));
        for (int gg = 0; gg < 16; gg++) {
            const int g = 16 * b + gg;
            int32_t acc = 0;
            for (int l = 0; l < 16; l++) acc += (int32_t)q3k_q(blk, gg, l) * xq[16 * g + l];
            const float c = d * (float)(q3k_scale(blk + 96, gg) - 32) * xs[g >> 1];
            f[gg & 3] = fmaf((float)acc, c, f[gg & 3]);
            m_ += fabs((double)acc * (double)c);
        }
    }
    if (mag) *mag = m_;
    return (f[0] + f[1]) + (f[2] + f[3]);
}

/* Q8_0 with int8 activations per 32 (one scale per block),
 * q8_0_dot_row_sdot_f (stratum_q8_0.h:112-145): block i's exact dot with
 * the quantized x, coefficient fl(d * xs[i]), lane i % 4 of four binary32
 * fused multiply-add chains (K % 256 == 0, so no tail), then
 * (f0 + f1) + (f2 + f3). */
static float q8_0_sdot_f(const uint8_t* row, int K, const int8_t* xq, const float* xs,
                         double* mag) {
    float f[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    double m_ = 0.0;
    for (int i = 0; i < K / 32; i++) {
        const uint8_t* blk = row + (size_t)i * 34;
        int32_t acc = 0;
        for (int l = 0; l < 32; l++) acc += (int32_t)(int8_t)blk[2 + l] * xq[32 * i + l];
        const float c = ko_fp16_to_fp32(rd16(blk)) * xs[i];
        f[i & 3] = fmaf((float)acc, c, f[i & 3]);
        m_ += fabs((double)acc * (double)c);
    }
    if (mag) *mag = m_;
    return (f[0] + f[1]) + (f[2] + f[3]);
}

/* The same three as the GPU computes them: the identical integer dots and
 * binary32 coefficients, each term formed in binary64 (Q5_K: c1*L + c2*xsum
 * with one rounding, as Q4_K; Q3_K, Q8_0: c * dot, exact) and summed in
 * binary64. */
static double q5k_i8_dot(const uint8_t* row, int K, const int8_t* xq, const float* xs,
                         const int32_t* xsum) {
    double dot = 0.0;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 176;
        const float d = ko_fp16_to_fp32(rd16(blk)), dmin = ko_fp16_to_fp32(rd16(blk + 2));
        for (int s = 0; s < 8; s++) {
            const int g = 8 * b + s;
            uint8_t sc, mn;
            ko_q4k_scale_min(s, blk + 4, &sc, &mn);
            int32_t L = 0;
            for (int l = 0; l < 32; l++) L += (int32_t)q5k_q(blk, s, l) * xq[32 * g + l];
            const float c1 = d * (float)sc * xs[g], c2 = -dmin * (float)mn * xs[g];
            dot += fma((double)c1, (double)L, (double)c2 * (double)xsum[g]);
        }
    }
    return dot;
}

static double q3k_i8_dot(const uint8_t* row, int K, const int8_t* xq, const float* xs) {
    double dot = 0.0;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 110;
        const float d = ko_fp16_to_fp32(rd16(blk + 108));
        for (int gg = 0; gg < 16; gg++) {
            const int g = 16 * b + gg;
            int32_t acc = 0;
            for (int l = 0; l < 16; l++) acc += (int32_t)q3k_q(blk, gg, l) * xq[16 * g + l];
            const float c = d * (float)(q3k_scale(blk + 96, gg) - 32) * xs[g >> 1];
            dot += (double)c * (double)acc;
        }
    }
    return dot;
}

static double q8_0_i8_dot(const uint8_t* row, int K, const int8_t* xq, const float* xs) {
    double dot = 0.0;
    for (int i = 0; i < K / 32; i++) {
        const uint8_t* blk = row + (size_t)i * 34;
        int32_t acc = 0;
        for (int l = 0; l < 32; l++) acc += (int32_t)(int8_t)blk[2 + l] * xq[32 * i + l];
        dot += (double)(ko_fp16_to_fp32(rd16(blk)) * xs[i]) * (double)acc;
    }
    return dot;
}

/* one row of the int8 mode: the reference's order (sdot_f) or the GPU's */
static float i8_row(int type, const uint8_t* row, int K, const int8_t* xq, const float* xs,
                    const int32_t* xsum, int sdot_f, double* mag) {
    switch (type) {
    case KO_Q4_K: return sdot_f ? q4k_sdot_f(row, K, xq, xs, xsum, mag)
                                : (float)q4k_i8_dot(row, K, xq, xs, xsum);
    case KO_Q6_K: return sdot_f ? q6k_sdot_f(row, K, xq, xs, xsum, mag)
                                : (float)q6k_i8_dot(row, K, xq, xs, xsum);
    case KO_Q5_K: return sdot_f ? q5k_sdot_f(row, K, xq, xs, xsum, mag)
                                : (float)q5k_i8_dot(row, K, xq, xs, xsum);
    case KO_Q3_K: return sdot_f ? q3k_sdot_f(row, K, xq, xs, mag)
                                : (float)q3k_i8_dot(row, K, xq, xs);
    default: return sdot_f ? q8_0_sdot_f(row, K, xq, xs, mag)
                           : (float)q8_0_i8_dot(row, K, xq, xs);
    }
}

/* y[r] (+ add[r]) for the int8-activation mode: x quantized once per call
 * (per 16 for Q6_K, per 32 for Q4_K, Q5_K, Q3_K and Q8_0), then each row
 * in the reference's order (sdot_f != 0) or the GPU's (binary64 terms).
 * mag (optional) receives each row's sum of |term|. */
int ko_gemv_i8(int type, const uint8_t* w, const float* x, const float* add, float* y,
               double* mag, int N, int K, int sdot_f) {
    if ((type != KO_Q4_K && type != KO_Q6_K && type != KO_Q5_K && type != KO_Q3_K &&
         type != KO_Q8_0) || K % 256)
        return -1;
    const int G = type == KO_Q6_K ? 16 : 32;
    int8_t* xq = malloc((size_t)K);
    float* xs = malloc((size_t)(K / G) * sizeof(float));
    int32_t* xsum = malloc((size_t)(K / G) * sizeof(int32_t));
    if (!xq || !xs || !xsum) { free(xq); free(xs); free(xsum); return -1; }
    ko_quantize_x_q8(x, K, G, xq, xs);
    xsums(xq, K, G, xsum);
    const size_t rb = (size_t)(K / 256) * (size_t)ko_block_bytes(type);
    for (int r = 0; r < N; r++) {
        const uint8_t* row = w + (size_t)r * rb;
        double m_ = 0.0;
        float v = i8_row(type, row, K, xq, xs, xsum, sdot_f, &m_);
        if (add) v = add[r] + v;
        y[r] = v;
        if (mag) {
            if (!sdot_f) (void)i8_row(type, row, K, xq, xs, xsum, 1, &m_);
            mag[r] = m_;
        }
    }
    free(xq); free(xs); free(xsum);
    return 0;
}

/* The int8 MULTISEQ of st_linear_multix under g_st.use_sdot, B >= 2
 * (stratum_linear.h:732-907): every stream quantized as the single-stream
 * form quantizes it (per 32, q4k_quantize_x_q8_1b, stratum_q4k_neon.h:
 * 185-226, the same rule as q4k_quantize_x_q8; per 16 for Q6_K,
 * q6k_quantize_x_q8_g16), then per (row, stream) a binary64 sum in element
 * order of one term per sub-block / 16-group:
 *   Q4_K (q4k_dot_rows2_sdot_multix_pack, stratum_q4k_neon.h:870-948):
 *     fl(fl(fl(d*sc) * fl(fl(L) * scl)) - fl(fl(dmin*m) * fl(fl(S) * scl)))
 *     with L the exact dot of the 4-bit values and S the group's int8 sum;
 *   Q6_K (q6k_dot_rows2_sdot_multix_pack, stratum_q6k_neon.h:627-700):
 *     (((double)d * sc) * (double)scl) * (double)A, binary64, with A the
 *     exact dot of the signed values q - 32.
 * The rows2 kernels take every row pair (the i8mm rows4 path keeps their
 * merge order, stratum_q4k_neon.h:1066-1071); the single-row multix_pack
 * form, used for an odd last row, is the same arithmetic except at B = 7,
 * where it takes a binary32-accumulating variant (q4k_dot_row_sdot_pack_b7)
 * that is not restated here.  Parity unpinned for the association of the
 * Q4_K term's products (see the header); indexing, signs, coefficients and
 * magnitude are pinned by exact inputs and quant_test.c's relation. */
int ko_gemv_i8_multix(int type, const uint8_t* w, const float* xs, float* ys, int B, int N,
                      int K) {
    if ((type != KO_Q4_K && type != KO_Q6_K) || K % 256 || B < 1) return -1;
    const int G = type == KO_Q4_K ? 32 : 16, ng = K / G;
    int8_t* xq = malloc((size_t)B * K);
    float* sc = malloc((size_t)B * ng * sizeof(float));
    int32_t* sm = malloc((size_t)B * ng * sizeof(int32_t));
    if (!xq || !sc || !sm) { free(xq); free(sc); free(sm); return -1; }
    for (int s = 0; s < B; s++) {
        ko_quantize_x_q8(xs + (size_t)s * K, K, G, xq + (size_t)s * K, sc + (size_t)s * ng);
        xsums(xq + (size_t)s * K, K, G, sm + (size_t)s * ng);
    }
    const size_t rb = (size_t)(K / 256) * (size_t)ko_block_bytes(type);
    for (int r = 0; r < N; r++) {
        const uint8_t* row = w + (size_t)r * rb;
        for (int s = 0; s < B; s++) {
            const int8_t* x8 = xq + (size_t)s * K;
            const float* scl = sc + (size_t)s * ng;
            const int32_t* S = sm + (size_t)s * ng;
            double dot = 0.0;
            for (int b = 0; b < K / 256; b++) {
                if (type == KO_Q4_K) {
                    const uint8_t* blk = row + (size_t)b * 144;
                    const float d = ko_fp16_to_fp32(rd16(blk)), dmin = ko_fp16_to_fp32(rd16(blk + 2));
                    for (int sb = 0; sb < 8; sb++) {
                        const int g = 8 * b + sb;
                        uint8_t scv, mn;
                        ko_q4k_scale_min(sb, blk + 4, &scv, &mn);
                        const float d_sc = d * (float)scv, dmin_m = dmin * (float)mn;
                        int32_t L = 0;
                        for (int l = 0; l < 32; l++) L += (int32_t)q4k_q(blk, sb, l) * x8[32 * g + l];
                        const float s_f = (float)S[g];
                        dot += (double)(d_sc * ((float)L * scl[g]) - dmin_m * (s_f * scl[g]));
                    }
                } else {
                    const uint8_t* blk = row + (size_t)b * 210;
                    const float d = ko_fp16_to_fp32(rd16(blk + 208));
                    const int8_t* sc8 = (const int8_t*)(blk + 192);
                    for (int h = 0; h < 2; h++)
                        for (int is = 0; is < 2; is++)
                            for (int t = 0; t < 4; t++) {
                                const int gl = 8 * h + is + 2 * t, g = 16 * b + gl;
                                int32_t acc = 0;
                                for (int l = 0; l < 16; l++)
                                    acc += (int32_t)q6k_q(blk, h, t, 16 * is + l) * x8[16 * g + l];
                                const double ds = (double)d * (double)sc8[gl];
                                dot += ds * (double)scl[g] * (double)acc;
                            }
                }
            }
            ys[(size_t)s * N + r] = (float)dot;
        }
    }
    free(xq); free(sc); free(sm);
    return 0;
}

/* ------------------------------------------------------------ dispatch */
void ko_dequant_row(int type, const uint8_t* row, int K, float* y) {
    const int bb = ko_block_bytes(type);
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * bb;
        float* yb = y + (size_t)b * 256;
        switch (type) {
        case KO_Q4_K: q4k_dequant_block(blk, yb); break;
        case KO_Q6_K: q6k_dequant_block(blk, yb); break;
        case KO_Q2_K: q2_dequant_block(blk, 0, yb); break;
        case KO_Q2K_NIB: q2_dequant_block(blk, 1, yb); break;
        case KO_Q5_K: q5k_dequant_block(blk, yb); break;
        case KO_Q3_K: q3k_dequant_block(blk, yb); break;
        case KO_Q8_0:
            for (int q = 0; q < 8; q++) q8_0_dequant_block(blk + 34 * q, yb + 32 * q);
            break;
        case KO_F16:
            for (int k = 0; k < 256; k++) yb[k] = ko_fp16_to_fp32(rd16(blk + 2 * k));
            break;
        case KO_F32: memcpy(yb, blk, 1024); break;
        default: return;
        }
    }
}

double ko_dot_row_f64(int type, const uint8_t* row, int K, const float* x) {
    switch (type) {
    case KO_Q4_K: return q4k_dot(row, K, x);
    case KO_Q6_K: return q6k_dot(row, K, x);
    case KO_Q2_K: return q2_dot(row, K, x, 0);
    case KO_Q2K_NIB: return q2_dot(row, K, x, 1);
    case KO_Q5_K: return q5k_dot(row, K, x);
    case KO_Q3_K: return q3k_dot(row, K, x);
    case KO_Q8_0: return q8_0_dot(row, K, x);
    case KO_F16: return f16_dot(row, K, x);
    case KO_F32: return f32_dot(row, K, x);
    default: return 0.0;
    }
}

float ko_dot_row(int type, const uint8_t* row, int K, const float* x) {
    return (float)ko_dot_row_f64(type, row, K, x);
}

/* --------------------------------------------------- threaded row split */
/* Mirrors ST_PAR_ROWS (stratum_linear.h:201-228): workers pull 64-row
 * tickets from an atomic counter; rows are independent, so the output does
 * not depend on the thread count. */
typedef struct {
    int type, N, K, B;
    size_t row_bytes;
    const uint8_t* w;
    const float* x;
    const float* add;
    float* y;
    atomic_int next;
} ko_job;

static void* ko_worker(void* arg) {
    ko_job* j = (ko_job*)arg;
    for (;;) {
        int s = atomic_fetch_add_explicit(&j->next, 64, memory_order_relaxed);
        if (s >= j->N) break;
        int e = s + 64 < j->N ? s + 64 : j->N;
        for (int r = s; r < e; r++) {
            const uint8_t* row = j->w + (size_t)r * j->row_bytes;
            for (int b = 0; b < j->B; b++) {
                float v = ko_dot_row(j->type, row, j->K, j->x + (size_t)b * j->K);
                if (j->add) v = j->add[(size_t)b * j->N + r] + v;
                j->y[(size_t)b * j->N + r] = v;
            }
        }
    }
    return NULL;
}

static int ko_run(ko_job* j, int nthreads) {
    if (ko_block_bytes(j->type) == 0 || j->K % 256 != 0 || j->N < 0 || j->K < 0) return -1;
    atomic_store(&j->next, 0);
    if (nthreads <= 1) {
        ko_worker(j);
        return 0;
    }
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    int started = 0;
    for (int t = 0; t < nthreads - 1; t++) {
        if (pthread_create(&th[t], NULL, ko_worker, j) != 0) break;
        started++;
    }
    ko_worker(j); /* the caller takes a share, as st_par_run does */
    for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
    return 0;
}

int ko_gemv(int type, const uint8_t* w, const float* x, const float* add,
            float* y, int N, int K, int nthreads) {
    ko_job j;
    j.type = type; j.N = N; j.K = K; j.B = 1;
    j.row_bytes = (size_t)(K / 256) * (size_t)ko_block_bytes(type);
    j.w = w; j.x = x; j.add = add; j.y = y;
    return ko_run(&j, nthreads);
}

int ko_gemv_multix(int type, const uint8_t* w, const float* xs, float* ys,
                   int B, int N, int K, int nthreads) {
    ko_job j;
    j.type = type; j.N = N; j.K = K; j.B = B;
    j.row_bytes = (size_t)(K / 256) * (size_t)ko_block_bytes(type);
    j.w = w; j.x = xs; j.add = NULL; j.y = ys;
    return ko_run(&j, nthreads);
}

/* ------------------------------------------------------ type-42 layout */
void ko_q2k_to_nib(const uint8_t* q2k, uint8_t* nib, int64_t nblocks) {
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t* src = q2k + b * 84;
        uint8_t* dst = nib + b * 148;
        memcpy(dst, src, 16);            /* scales unchanged */
        memset(dst + 16, 0, 128);
        memcpy(dst + 144, src + 80, 4);  /* d, dmin moved to the tail */
        for (int g = 0; g < 16; g++)
            for (int l = 0; l < 16; l++) {
                int p = q2_pos(g, l);
                int q = q2k_q(src, g, l);
                dst[16 + 16 * (p >> 5) + (p & 15)] |= (uint8_t)((p & 16) ? (q << 4) : q);
            }
    }
}

void ko_nib_to_q2k(const uint8_t* nib, uint8_t* q2k, int64_t nblocks) {
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t* src = nib + b * 148;
        uint8_t* dst = q2k + b * 84;
        memcpy(dst, src, 16);
        memset(dst + 16, 0, 64);
        memcpy(dst + 80, src + 144, 4);
        for (int g = 0; g < 16; g++)
            for (int l = 0; l < 16; l++) {
                int s = g >> 3, j = (g >> 1) & 3, h = g & 1;
                int q = nib_q(src, q2_pos(g, l)) & 3;
                dst[16 + 32 * s + 16 * h + l] |= (uint8_t)(q << (2 * j));
            }
    }
}

/* --------------------------------------------------------------- top-k */
void ko_moe_topk(const float* w, int E, int K, int* sel, float* selw) {
    /* stratum_arch_moe.inc.c:368-385: insertion into a descending list on
     * strictly greater weight; an equal weight never displaces an earlier
     * (lower-id) entry. */
    for (int s = 0; s < K; s++) { sel[s] = -1; selw[s] = -1.0f; }
    for (int e = 0; e < E; e++) {
        int pos = -1;
        for (int s = 0; s < K; s++)
            if (w[e] > selw[s]) { pos = s; break; }
        if (pos < 0) continue;
        for (int s = K - 1; s > pos; s--) { sel[s] = sel[s - 1]; selw[s] = selw[s - 1]; }
        sel[pos] = e;
        selw[pos] = w[e];
    }
}

/* ------------------------------------------------------ MoE FFN step */

/* stratum_softmax_inplace (stratum_engine.h:395-423) as its scalar path
 * runs it: the max by a sequential strictly-greater scan from x[0], libm
 * expf of each x - max, the binary64 sum in index order, one binary32
 * reciprocal of that sum, then a binary32 product per value. */
void ko_softmax(float* x, int N) {
    if (N <= 0) return;
    float top = x[0];
    for (int i = 1; i < N; i++)
        if (x[i] > top) top = x[i];
    double total = 0.0;
    for (int i = 0; i < N; i++) {
        x[i] = expf(x[i] - top);
    }
    for (int i = 0; i < N; i++) total += (double)x[i];
    const float r = (float)(1.0 / total);
    for (int i = 0; i < N; i++) x[i] = x[i] * r;
}

/* stratum_swiglu's scalar loop (stratum_engine.h:386-391) */
void ko_swiglu(const float* g, const float* u, float* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        const float gate = g[i];
        const float sig = gate / (1.0f + expf(-gate));
        y[i] = sig * u[i];
    }
}

/* Rank-ordered weighted accumulate and residual
 * (stratum_arch_moe.inc.c:728-743 and 1213-1226): o has B*k rows of H */
void ko_moe_combine(const float* o, const int* sel, const float* selw, const float* resid,
                    float* x, int B, int k, int H) {
    for (int s = 0; s < B; s++)
        for (int i = 0; i < H; i++) {
            float acc = 0.0f;
            for (int r = 0; r < k; r++) {
                if (sel[s * k + r] < 0) continue;
                const float t = selw[s * k + r] * o[((size_t)s * k + r) * H + i];
                acc = acc + t;
            }
            x[(size_t)s * H + i] = resid[(size_t)s * H + i] + acc;
        }
}

/* The whole expert FFN step for B tokens (stratum_arch_moe.inc.c:689-743):
 * router GEMV on each token's xn, softmax, top-k, then per selected rank
 * the gate, up (slices at e * stride), SwiGLU and down, and the combine.
 * The intermediate buffers are returned when their pointers are not NULL:
 * probs B x E, g / u / act B*k x F, ffo B*k x H. */
int ko_moe_ffn(const ko_moe_ffn_desc* f, const float* xn, float* x, int B, int* sel,
               float* selw, float* probs, float* g, float* u, float* act, float* ffo) {
    const int H = f->n_embed, F = f->n_ff, E = f->n_experts, k = f->k;
    const size_t bk = (size_t)B * k;
    float* P = malloc((size_t)B * E * sizeof(float));
    float* G = malloc(bk * F * sizeof(float));
    float* U = malloc(bk * F * sizeof(float));
    float* A = malloc(bk * F * sizeof(float));
    float* O = malloc(bk * H * sizeof(float));
    int rc = (P && G && U && A && O) ? 0 : -1;
    for (int s = 0; s < B && !rc; s++) {
        float* ps = P + (size_t)s * E;
        rc = ko_gemv(f->router_type, f->router, xn + (size_t)s * H, NULL, ps, E, H, 1);
        if (rc) break;
        ko_softmax(ps, E);
        ko_moe_topk(ps, E, k, sel + (size_t)s * k, selw + (size_t)s * k);
        for (int r = 0; r < k && !rc; r++) {
            const size_t m = (size_t)s * k + r;
            const int e = sel[m];
            if (e < 0) continue;
            rc = ko_gemv(f->gate_type, f->gate + (size_t)e * f->gate_stride, xn + (size_t)s * H,
                         NULL, G + m * F, F, H, 1) ||
                 ko_gemv(f->up_type, f->up + (size_t)e * f->up_stride, xn + (size_t)s * H, NULL,
                         U + m * F, F, H, 1);
            if (rc) break;
            ko_swiglu(G + m * F, U + m * F, A + m * F, F);
            rc = ko_gemv(f->down_type, f->down + (size_t)e * f->down_stride, A + m * F, NULL,
                         O + m * H, H, F, 1);
        }
    }
    if (!rc) {
        ko_moe_combine(O, sel, selw, x, x, B, k, H);
        if (probs) memcpy(probs, P, (size_t)B * E * sizeof(float));
        if (g) memcpy(g, G, bk * F * sizeof(float));
        if (u) memcpy(u, U, bk * F * sizeof(float));
        if (act) memcpy(act, A, bk * F * sizeof(float));
        if (ffo) memcpy(ffo, O, bk * H * sizeof(float));
    }
    free(P); free(G); free(U); free(A); free(O);
    return rc;
}
