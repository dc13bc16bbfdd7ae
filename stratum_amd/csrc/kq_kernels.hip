// kq_kernels.hip -- gfx950 (CDNA4) k-quant dequant-fused GEMV kernels.
//
// One hot path: y[N] = W[N x K] . x[K] with W in GGUF k-quant super-blocks
// (Q4_K 144 B, Q6_K 210 B, Q2_K 84 B, type-42 "Q2K_NIB" 148 B per 256
// weights), plus the B-stream form used by STRATUM_MULTISEQ and the MoE
// gather form.  Host code (kq_linear.c) plans launches and calls the
// extern "C" launchers at the bottom of this file.
//
// Numerical contract ("oracle order").  The kernels reproduce, for every
// sub-block, the exact binary32 operation sequence of the reference's
// scalar routines (stratum_q4k.h:95-131, stratum_q6k.h:38-73,
// stratum_q2k.h:44-89): each 32-weight (Q4_K) or 16-weight (Q6_K, Q2_K)
// partial is a sequential, uncontracted multiply-then-add chain in ONE lane,
// and the per-sub-block terms are summed in binary64.  Only the binary64
// summation order differs from the reference, so the binary32 result equals
// the reference's except when a binary64 rounding difference crosses a
// binary32 rounding boundary.  The file is compiled with
// -ffp-contract=off and carries the pragma below so no mul+add fuses.
//
// Exact integer-to-float tricks used on the hot loop:
//  * Q4_K / Q2_K / type-42 quants are converted with v_cvt_f32_ubyte{0..3}
//    straight from their packed bytes.  A quant that does not sit in the
//    low bits of its byte is masked in place, so the byte holds q * 2^s
//    (s = 4 for a high nibble, 2j for Q2_K's field j).  Since every
//    partial sum then equals 2^s times the reference's partial sum exactly
//    (power-of-two scaling commutes with binary32 rounding for these
//    magnitudes), the factor is removed exactly by scaling d*sc by 2^-s.
//  * Q6_K quants are assembled as the int8 byte 4*(q-32) and converted
//    with a sign-extending byte select; the partial sums are then exactly
//    4x the reference's, and the factor is folded into the exact binary64
//    scale product d*s/4.
// The scalings are exact for every finite input with |x| < 2^100.
//
// Work decomposition (all types).  A row of K weights is K/64 "chunks" of
// 64 weights; a chunk is one lane's work and always lies inside one
// super-block (4 chunks per block).  A workgroup owns R consecutive rows,
// i.e. a contiguous byte range of W, and its lanes sweep that range chunk
// by chunk (lane i takes chunks i, i+T, i+2T, ...), so each sweep step
// reads T/4 consecutive super-blocks: fully coalesced 128-bit loads.  x is
// staged once per workgroup in LDS in a padded chunk-major layout (17
// float4 per chunk: conflict-free for consecutive chunks).  Each chunk's
// binary64 term goes to LDS; after a barrier, 16 lanes per row reduce that
// row's terms in a fixed order.  Results therefore do not depend on the
// grid, the workgroup size or R.
#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma clang fp contract(off)

namespace {

constexpr int T_Q2K = 10;
constexpr int T_Q4K = 12;
constexpr int T_Q6K = 14;
constexpr int T_NIB = 42;

constexpr int XPAD = 17;  // float4 slots per 64-weight chunk in LDS (16 + 1 pad)

template <int TYPE> struct TypeInfo;
template <> struct TypeInfo<T_Q4K> { static constexpr int BB = 144; static constexpr bool LINEAR = true;  static constexpr int XS_PER_CHUNK = 2; };
template <> struct TypeInfo<T_Q6K> { static constexpr int BB = 210; static constexpr bool LINEAR = false; static constexpr int XS_PER_CHUNK = 0; };
template <> struct TypeInfo<T_Q2K> { static constexpr int BB = 84;  static constexpr bool LINEAR = false; static constexpr int XS_PER_CHUNK = 4; };
template <> struct TypeInfo<T_NIB> { static constexpr int BB = 148; static constexpr bool LINEAR = true;  static constexpr int XS_PER_CHUNK = 4; };

struct GemvArgs {
    const uint8_t* w;    // row 0 of the tensor (device)
    const float* x;      // [B][K] activations (device)
    const float* add;    // [B][N] residual or nullptr
    float* y;            // [B][N] output
    int N, K;
    int rows_per_wg;     // rows owned by one workgroup
    int B;               // streams (1 for the plain GEMV)
};

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
    return (float)v;  // v_cvt_f32_f16: exact widening incl. subnormals
}

// the four bytes of v as floats (v_cvt_f32_ubyte0..3).  The empty asm
// hides the masked value's known bits from the optimiser, which would
// otherwise re-extract every field with v_bfe before converting.
__device__ __forceinline__ void ubytes(uint32_t v, float& a, float& b, float& c, float& d) {
    asm volatile("" : "+v"(v));
    a = (float)(v & 0xffu);
    b = (float)((v >> 8) & 0xffu);
    c = (float)((v >> 16) & 0xffu);
    d = (float)(v >> 24);
}

__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t w) {
    return __builtin_amdgcn_ubfe(v, off, w);
}

// v of the lane selected by DPP control CTRL (both 32-bit halves moved).
// Used only with every lane of the 8-lane group active.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const int lo = __double2loint(v), hi = __double2hiint(v);
    const int l2 = __builtin_amdgcn_mov_dpp(lo, CTRL, 0xf, 0xf, false);
    const int h2 = __builtin_amdgcn_mov_dpp(hi, CTRL, 0xf, 0xf, false);
    return __hiloint2double(h2, l2);
}

// ------------------------------------------------------------------ LDS x
// Chunk index c and float4 slot g (0..15) of x position p (p % 4 == 0).
//  LINEAR  (Q4_K, type 42): chunk = 64 consecutive weights.
//  strided (Q6_K, Q2_K):    chunk = (block, half, 16-sub) = 4 runs of 16
//                           weights spaced 32 apart, slot g = 4*run + l/4.
template <bool LINEAR>
__device__ __forceinline__ void x_slot(int p, int& c, int& g) {
    if (LINEAR) {
        c = p >> 6;
        g = (p >> 2) & 15;
    } else {
        const int bi = p >> 8, pp = p & 255;
        const int h = pp >> 7, t = (pp >> 5) & 3, is = (pp >> 4) & 1, q = (pp >> 2) & 3;
        c = 4 * bi + 2 * h + is;
        g = 4 * t + q;
    }
}

// Staging of x (one stream) into LDS.
//   stage_dma  -- x goes straight from global memory into the padded LDS
//                 layout with global_load_lds_dwordx4 (lane i of a wave
//                 writes 16 bytes at base + 16 i).  No registers are
//                 involved, so every x load of the workgroup is issued back
//                 to back right after the weight prefetch and the whole
//                 staging costs about one memory latency;
//   stage_sums -- after a barrier, the per-sub-block plain sums the min
//                 terms need, read back from LDS (sequential binary32,
//                 exactly as the reference's xs1/xs2 and sx accumulators).

// global float4 index of LDS slot s (chunk c = s / XPAD, slot g = s % XPAD);
// the pad slot (g == 16) is filled with a copy of slot 0 and never read
template <bool LINEAR>
__device__ __forceinline__ int x_src_of_slot(int s) {
    const int c = s / XPAD;
    int g = s - c * XPAD;
    if (g == 16) g = 0;
    if (LINEAR) return 16 * c + g;
    // strided: chunk c = (block, half h, sub is); slot g = 4*run + l/4
    const int bi = c >> 2, h = (c >> 1) & 1, is = c & 1;
    return 64 * bi + 32 * h + 4 * is + 8 * (g >> 2) + (g & 3);
}

template <int TYPE>
__device__ __forceinline__ void stage_dma(const float* __restrict__ x, int K, int tid, int T,
                                          float4* xl) {
    const int total = (K >> 6) * XPAD;       // slots, pads included
    const int wbase = tid & ~63;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    for (int s0 = 0; s0 < total; s0 += T) {
        const int s = s0 + tid;
        if (s < total) {
            const float4* src = x4 + x_src_of_slot<TypeInfo<TYPE>::LINEAR>(s);
            __builtin_amdgcn_global_load_lds(
                src, (__attribute__((address_space(3))) void*)(xl + s0 + wbase), 16, 0, 0);
        }
    }
}

template <int TYPE>
__device__ __forceinline__ void stage_sums(int K, int tid, int T, const float4* xl, float* xs) {
    if (TYPE == T_Q4K) {
        // xs[sb] = sum of the 32 x of sub-block sb (stratum_q4k.h:115-122):
        // chunk sb/2, float4 slots 8*(sb&1) .. +7 of the linear layout
        for (int sb = tid; sb < (K >> 5); sb += T) {
            const float4* p = xl + (sb >> 1) * XPAD + 8 * (sb & 1);
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float4 v = p[k];
                s = s + v.x; s = s + v.y; s = s + v.z; s = s + v.w;
            }
            xs[sb] = s;
        }
    } else if (TYPE == T_Q2K || TYPE == T_NIB) {
        // sums over 16-weight groups (stratum_q2k.h:65-68), stored at the
        // chunk's slot: Q2_K chunk (block, s, h) holds groups j = 0..3 (its
        // float4 slots 4j..4j+3), type-42 chunk u holds groups 4u..4u+3.
        for (int gi = tid; gi < (K >> 4); gi += T) {
            int c, j;
            if (TYPE == T_NIB) {
                c = gi >> 2;
                j = gi & 3;
            } else {
                const int bi = gi >> 4, g16 = gi & 15;
                c = 4 * bi + 2 * (g16 >> 3) + (g16 & 1);
                j = (g16 >> 1) & 3;
            }
            const float4* p = xl + c * XPAD + 4 * j;
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float4 v = p[k];
                s = s + v.x; s = s + v.y; s = s + v.z; s = s + v.w;
            }
            xs[c * 4 + j] = s;
        }
    }
}

// ------------------------------------------------------------ raw loads
// 4-byte-aligned 128-bit vector: Q6_K/Q2_K/type-42 blocks are only dword
// aligned; global_load_dwordx4 needs dword alignment only.
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2a __attribute__((ext_vector_type(2), aligned(4)));

__device__ __forceinline__ uint4 ld16a4(const uint8_t* p) {
    const u32x4a v = *reinterpret_cast<const u32x4a*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

struct RawQ4 { uint4 hd, qa, qb; };
struct RawQ6 { uint32_t l[5], h[5], q[5], s[3], d; uint32_t sh; };
struct RawQ2 { uint4 q; uint2 s; uint32_t dd; };
struct RawNB { uint4 qa, qb; uint32_t s, dd; };

__device__ __forceinline__ RawQ4 load_q4k(const uint8_t* blk, int j) {
    RawQ4 r;
    r.hd = *reinterpret_cast<const uint4*>(blk);
    r.qa = *reinterpret_cast<const uint4*>(blk + 16 + 32 * j);
    r.qb = *reinterpret_cast<const uint4*>(blk + 32 + 32 * j);
    return r;
}

// Q6_K blocks are 210 B, so odd blocks start 2 bytes off a dword.  Loads
// are dword-aligned and realigned with v_alignbit (shift 0 or 16).
__device__ __forceinline__ void load5(const uint8_t* p, uint32_t* o) {
    const uint4 v = ld16a4(p);
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    o[4] = reinterpret_cast<const uint32_t*>(p)[4];
}

__device__ __forceinline__ RawQ6 load_q6k(const uint8_t* blk, int u) {
    RawQ6 r;
    const int h = u >> 1, is = u & 1;
    // realign by pointer arithmetic (not through an integer) so the
    // compiler keeps the global address space and emits global_load, not
    // flat_load (flat loads also count against lgkmcnt, so every LDS wait
    // would wait for the weight prefetch as well)
    const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(blk) & 3u;
    r.sh = mis * 8u;
    const uint8_t* b4 = blk - mis;
    load5(b4 + 64 * h + 16 * is, r.l);
    load5(b4 + 64 * h + 32 + 16 * is, r.h);
    load5(b4 + 128 + 32 * h + 16 * is, r.q);
    // scales: 8 bytes from 192 + 8h.  A third dword is needed only when the
    // block is 2 bytes off; when aligned, dword 1 is re-read instead so the
    // last block of a tensor never reads past its 210 bytes.
    const uint32_t* sp = reinterpret_cast<const uint32_t*>(b4 + 192 + 8 * h);
    r.s[0] = sp[0]; r.s[1] = sp[1]; r.s[2] = sp[r.sh ? 2 : 1];
    r.d = *reinterpret_cast<const uint16_t*>(blk + 208);
    return r;
}

__device__ __forceinline__ RawQ2 load_q2k(const uint8_t* blk, int u) {
    RawQ2 r;
    const int s = u >> 1, h = u & 1;
    r.q = ld16a4(blk + 16 + 32 * s + 16 * h);
    const u32x2a sv = *reinterpret_cast<const u32x2a*>(blk + 8 * s);
    r.s = make_uint2(sv.x, sv.y);
    r.dd = *reinterpret_cast<const uint32_t*>(blk + 80);
    return r;
}

__device__ __forceinline__ RawNB load_nib(const uint8_t* blk, int u) {
    RawNB r;
    r.qa = ld16a4(blk + 16 + 32 * u);
    r.qb = ld16a4(blk + 32 + 32 * u);
    r.s = *reinterpret_cast<const uint32_t*>(blk + 4 * u);
    r.dd = *reinterpret_cast<const uint32_t*>(blk + 144);
    return r;
}

// ---------------------------------------------------------- chunk terms
// Each returns the binary64 sum of the chunk's sub-block terms, computed in
// the reference's binary32 operation order.

__device__ __forceinline__ uint32_t dw_of(const uint4& v, int k) {
    return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}

// Q4_K chunk j of a block: sub-blocks 2j (low nibbles) and 2j+1 (high).
__device__ __forceinline__ double term_q4k(const RawQ4& r, int j, const float4* xc,
                                           float xs1, float xs2) {
    const float d = f16_bits_to_f32(r.hd.x & 0xffffu);
    const float dmin = f16_bits_to_f32(r.hd.x >> 16);
    // 6-bit scale/min decode (stratum_q4k.h:57-65) for sub-blocks 2j, 2j+1.
    // j < 2: sc = s[sb] & 63, m = s[sb+4] & 63.
    // j >= 2: sc = (s[sb+4] & 15) | (s[sb-4] >> 6) << 4,
    //         m  = (s[sb+4] >> 4) | (s[sb] >> 6) << 4.
    const uint32_t s0 = r.hd.y, s1 = r.hd.z, s2 = r.hd.w;
    const bool lo = j < 2;
    const uint32_t ob = (uint32_t)((2 * j) & 3) * 8u;   // bit offset of byte sb&3
    const uint32_t a_sc = lo ? s0 : s2;
    const uint32_t a_m = lo ? s1 : s2;
    const uint32_t w6 = lo ? 6u : 4u;
    const uint32_t om = lo ? 0u : 4u;
    const uint32_t wh = lo ? 0u : 2u;
    const uint32_t sc1 = bfe(a_sc, ob, w6) | (bfe(s0, ob + 6, wh) << 4);
    const uint32_t m1 = bfe(a_m, ob + om, w6) | (bfe(s1, ob + 6, wh) << 4);
    const uint32_t sc2 = bfe(a_sc, ob + 8, w6) | (bfe(s0, ob + 14, wh) << 4);
    const uint32_t m2 = bfe(a_m, ob + 8 + om, w6) | (bfe(s1, ob + 14, wh) << 4);
    const float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
    const float d2 = d * (float)sc2, mm2 = dmin * (float)m2;

    // high nibbles are converted in place (16 q), so a2 is 16x the
    // reference's partial sum and d2 is used divided by 16 (both exact)
    float a1 = 0.0f, a2 = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t v = k < 4 ? dw_of(r.qa, k) : dw_of(r.qb, k - 4);
        const uint32_t vl = v & 0x0f0f0f0fu, vh = v & 0xf0f0f0f0u;
        float l0, l1, l2, l3, h0, h1, h2, h3;
        ubytes(vl, l0, l1, l2, l3);
        ubytes(vh, h0, h1, h2, h3);
        const float4 xa = xc[k], xb = xc[8 + k];
        a1 = a1 + l0 * xa.x; a2 = a2 + h0 * xb.x;
        a1 = a1 + l1 * xa.y; a2 = a2 + h1 * xb.y;
        a1 = a1 + l2 * xa.z; a2 = a2 + h2 * xb.z;
        a1 = a1 + l3 * xa.w; a2 = a2 + h3 * xb.w;
    }
    const float t1 = d1 * a1 - mm1 * xs1;
    const float t2 = (d2 * 0.0625f) * a2 - mm2 * xs2;
    return (double)t1 + (double)t2;
}

__device__ __forceinline__ float i8f(uint32_t v, int e) {
    return (float)(int32_t)(int8_t)(uint8_t)(v >> (8 * e));
}

// Q6_K chunk (half h, sub is): four 16-weight sums a_t, t = 0..3.
__device__ __forceinline__ double term_q6k(const RawQ6& r, int u, const float4* xc) {
    const int is = u & 1;
    const uint32_t sh = r.sh;
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t L = __builtin_amdgcn_alignbit(r.l[k + 1], r.l[k], sh);
        const uint32_t H = __builtin_amdgcn_alignbit(r.h[k + 1], r.h[k], sh);
        const uint32_t Q = __builtin_amdgcn_alignbit(r.q[k + 1], r.q[k], sh) ^ 0xaaaaaaaau;
        // byte = ((q ^ 0x20) << 2) = int8 4*(q - 32), q = lo4 | hi2 << 4
        uint32_t y[4];
        y[0] = ((L << 2) & 0x3c3c3c3cu) | ((Q << 6) & 0xc0c0c0c0u);
        y[1] = ((H << 2) & 0x3c3c3c3cu) | ((Q << 4) & 0xc0c0c0c0u);
        y[2] = ((L >> 2) & 0x3c3c3c3cu) | ((Q << 2) & 0xc0c0c0c0u);
        y[3] = ((H >> 2) & 0x3c3c3c3cu) | (Q & 0xc0c0c0c0u);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float4 xv = xc[4 * t + k];
            a[t] = a[t] + i8f(y[t], 0) * xv.x;
            a[t] = a[t] + i8f(y[t], 1) * xv.y;
            a[t] = a[t] + i8f(y[t], 2) * xv.z;
            a[t] = a[t] + i8f(y[t], 3) * xv.w;
        }
    }
    // scales s[8h + is + 2t] sit at bytes is + 2t of the realigned pair
    const uint32_t S0 = __builtin_amdgcn_alignbit(r.s[1], r.s[0], sh);
    const uint32_t S1 = __builtin_amdgcn_alignbit(r.s[2], r.s[1], sh);
    const uint32_t dh = r.d;
    const double dq = (double)f16_bits_to_f32(dh) * 0.25;  // exact
    const uint32_t Sa = is ? (S0 >> 8) : S0;
    const uint32_t Sb = is ? (S1 >> 8) : S1;
    const double t0 = (dq * (double)(int8_t)(uint8_t)(Sa)) * (double)a[0];
    const double t1 = (dq * (double)(int8_t)(uint8_t)(Sa >> 16)) * (double)a[1];
    const double t2 = (dq * (double)(int8_t)(uint8_t)(Sb)) * (double)a[2];
    const double t3 = (dq * (double)(int8_t)(uint8_t)(Sb >> 16)) * (double)a[3];
    return (t0 + t1) + (t2 + t3);
}

// Q2_K chunk (half s, 16-sub h): groups j = 0..3, q = (qs >> 2j) & 3.
__device__ __forceinline__ double term_q2k(const RawQ2& r, int u, const float4* xc,
                                           const float4 xs4) {
    const int h = u & 1;
    const float d = f16_bits_to_f32(r.dd & 0xffffu);
    const float dmin = f16_bits_to_f32(r.dd >> 16);
    const uint32_t S0 = h ? (r.s.x >> 8) : r.s.x;   // bytes h, h+2
    const uint32_t S1 = h ? (r.s.y >> 8) : r.s.y;   // bytes h+4, h+6
    const uint32_t sc[4] = {S0 & 0xffu, (S0 >> 16) & 0xffu, S1 & 0xffu, (S1 >> 16) & 0xffu};
    const float sx[4] = {xs4.x, xs4.y, xs4.z, xs4.w};
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        // field j masked in place: bytes hold q * 4^j, so qx is 4^j times
        // the reference's sum and dl is used divided by 4^j (exact)
        const float dl = d * (float)(sc[j] & 15u);
        const float ml = dmin * (float)(sc[j] >> 4);
        const float inv = j == 0 ? 1.0f : j == 1 ? 0.25f : j == 2 ? 0.0625f : 0.015625f;
        float qx = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t v = dw_of(r.q, k) & (0x03030303u << (2 * j));
            float q0, q1, q2, q3;
            ubytes(v, q0, q1, q2, q3);
            const float4 xv = xc[4 * j + k];
            qx = qx + q0 * xv.x;
            qx = qx + q1 * xv.y;
            qx = qx + q2 * xv.z;
            qx = qx + q3 * xv.w;
        }
        const float t = (dl * inv) * qx - ml * sx[j];
        acc = acc + (double)t;
    }
    return acc;
}

// type-42 chunk u: 64 consecutive weights = groups 4u..4u+3; group g's
// 16 values are the low (g even) or high (g odd) nibbles of 16 bytes.
__device__ __forceinline__ double term_nib(const RawNB& r, const float4* xc, const float4 xs4) {
    const float d = f16_bits_to_f32(r.dd & 0xffffu);
    const float dmin = f16_bits_to_f32(r.dd >> 16);
    const float sx[4] = {xs4.x, xs4.y, xs4.z, xs4.w};
    double acc = 0.0;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const uint32_t scb = (r.s >> (8 * g)) & 0xffu;
        const float dl = d * (float)(scb & 15u);
        const float ml = dmin * (float)(scb >> 4);
        const uint4 src = (g < 2) ? r.qa : r.qb;
        // high-nibble groups are converted in place (16 q): scale dl by 1/16
        const float inv = (g & 1) ? 0.0625f : 1.0f;
        float qx = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t v = dw_of(src, k);
            v = (g & 1) ? (v & 0xf0f0f0f0u) : (v & 0x0f0f0f0fu);
            float q0, q1, q2, q3;
            ubytes(v, q0, q1, q2, q3);
            const float4 xv = xc[4 * g + k];
            qx = qx + q0 * xv.x;
            qx = qx + q1 * xv.y;
            qx = qx + q2 * xv.z;
            qx = qx + q3 * xv.w;
        }
        const float t = (dl * inv) * qx - ml * sx[g];
        acc = acc + (double)t;
    }
    return acc;
}

// ------------------------------------------------------ per-type dispatch
template <int TYPE> struct Chunk;

template <> struct Chunk<T_Q4K> {
    using Raw = RawQ4;
    static __device__ __forceinline__ Raw load(const uint8_t* blk, int u) { return load_q4k(blk, u); }
    static __device__ __forceinline__ double term(const Raw& r, int u, const float4* xc,
                                                  const float* xs, int c) {
        const float2 s = reinterpret_cast<const float2*>(xs)[c];
        return term_q4k(r, u, xc, s.x, s.y);
    }
};
template <> struct Chunk<T_Q6K> {
    using Raw = RawQ6;
    static __device__ __forceinline__ Raw load(const uint8_t* blk, int u) { return load_q6k(blk, u); }
    static __device__ __forceinline__ double term(const Raw& r, int u, const float4* xc,
                                                  const float*, int) {
        return term_q6k(r, u, xc);
    }
};
template <> struct Chunk<T_Q2K> {
    using Raw = RawQ2;
    static __device__ __forceinline__ Raw load(const uint8_t* blk, int u) { return load_q2k(blk, u); }
    static __device__ __forceinline__ double term(const Raw& r, int u, const float4* xc,
                                                  const float* xs, int c) {
        return term_q2k(r, u, xc, reinterpret_cast<const float4*>(xs)[c]);
    }
};
template <> struct Chunk<T_NIB> {
    using Raw = RawNB;
    static __device__ __forceinline__ Raw load(const uint8_t* blk, int u) { return load_nib(blk, u); }
    static __device__ __forceinline__ double term(const Raw& r, int, const float4* xc,
                                                  const float* xs, int c) {
        return term_nib(r, xc, reinterpret_cast<const float4*>(xs)[c]);
    }
};

template <int TYPE>
__host__ __device__ constexpr int xs_floats_per_chunk() { return TypeInfo<TYPE>::XS_PER_CHUNK; }

// LDS bytes for x staging of one stream
template <int TYPE>
__host__ __device__ inline int x_lds_bytes(int K) {
    const int NC = K >> 6;
    return NC * XPAD * 16 + NC * xs_floats_per_chunk<TYPE>() * 4;
}

// ------------------------------------------------------------- the GEMV
// One workgroup = R consecutive rows; see the header comment.  Each lane
// keeps DEPTH chunks in flight: the first DEPTH loads are issued before x
// is staged (their latency overlaps the staging), then every computed
// chunk's registers are refilled with the chunk DEPTH*T further on.
// T (blockDim.x) is a multiple of 64, so a lane's chunk index modulo 4 --
// its sub-block position inside the super-block -- never changes.
template <int TYPE, int DEPTH>
__global__ __launch_bounds__(1024) void kq_gemv_kernel(GemvArgs a) {
    using TI = TypeInfo<TYPE>;
    using C = Chunk<TYPE>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, T = blockDim.x;
    const int K = a.K, NC = K >> 6;
    const int r0 = blockIdx.x * a.rows_per_wg;
    const int R = min(a.rows_per_wg, a.N - r0);
    if (R <= 0) return;

    float4* xl = reinterpret_cast<float4*>(smem);
    float* xs = reinterpret_cast<float*>(smem + NC * XPAD * 16);
    double* terms = reinterpret_cast<double*>(smem + x_lds_bytes<TYPE>(K));

    const int nch = R * NC;
    const uint8_t* wb = a.w + (size_t)r0 * (size_t)(K >> 8) * TI::BB;
    const int u = tid & 3;

    // Dynamic distribution: each wave grabs the next batch of 64
    // consecutive chunks from an LDS counter, keeping DEPTH batches in
    // flight.  Waves are not served fairly by the issue arbiter (the oldest
    // wins), so a static split leaves a long tail with few waves, and so
    // little memory parallelism, at the end; with batches the waves finish
    // together.  A chunk's term does not depend on which wave computes it,
    // so the result stays deterministic.  Loads are issued unconditionally
    // (indices past the end are clamped to the last chunk) so the compiler
    // can count outstanding loads exactly.
    const int last = nch - 1;
    const int lane = tid & 63;
    int* next = reinterpret_cast<int*>(terms + nch);
    if (tid == 0) *next = 64 * DEPTH * (T >> 6);
    int base[DEPTH];
    typename C::Raw buf[DEPTH];
#pragma unroll
    for (int k = 0; k < DEPTH; k++) {
        base[k] = (k * (T >> 6) + (tid >> 6)) * 64;     // first batches: static
        const int fk = min(base[k] + lane, last);
        buf[k] = C::load(wb + (size_t)(fk >> 2) * TI::BB, u);
    }

    stage_dma<TYPE>(a.x, K, tid, T, xl);
    __syncthreads();
    if (TI::XS_PER_CHUNK) {
        stage_sums<TYPE>(K, tid, T, xl, xs);
        __syncthreads();
    }

    while (base[0] < nch) {
#pragma unroll
        for (int k = 0; k < DEPTH; k++) {
            int nb = 0;
            if (lane == 0) nb = atomicAdd(next, 64);
            const int f = base[k] + lane;
            if (base[k] < nch) {
                const int c = f % NC;
                const double t = C::term(buf[k], u, xl + c * XPAD, xs, c);
                if (f < nch) terms[f] = t;
            }
            base[k] = __builtin_amdgcn_readfirstlane(nb);
            const int fn = min(base[k] + lane, last);
            buf[k] = C::load(wb + (size_t)(fn >> 2) * TI::BB, u);
        }
    }
    __syncthreads();

    // Row reduction: L lanes per row (L = 8..64, as many as T allows), lane
    // p sums terms p, p+L, ... in two interleaved partial sums, then a
    // butterfly over the L lanes.  The order depends only on NC and L.
    int L = 8;
    while (L < 64 && 2 * L * R <= T) L *= 2;
    for (int task = tid; task < R * L; task += T) {
        const int rho = task / L, p = task & (L - 1);
        const double* tr = terms + rho * NC;
        double s0 = 0.0, s1 = 0.0;
        int i = p;
        for (; i + L < NC; i += 2 * L) {
            s0 = s0 + tr[i];
            s1 = s1 + tr[i + L];
        }
        if (i < NC) s0 = s0 + tr[i];
        double s = s0 + s1;
        s = s + dpp_f64<0xB1>(s);    // quad_perm [1,0,3,2]: lane ^ 1
        s = s + dpp_f64<0x4E>(s);    // quad_perm [2,3,0,1]: lane ^ 2
        s = s + dpp_f64<0x141>(s);   // row_half_mirror: lane i <-> 7 - i (8 lanes)
        if (L >= 16) s = s + dpp_f64<0x140>(s);   // row_mirror (16 lanes)
        if (L >= 32) s = s + __shfl_xor(s, 16, 64);
        if (L >= 64) s = s + __shfl_xor(s, 32, 64);
        if (p == 0) {
            float v = (float)s;
            if (a.add) v = a.add[r0 + rho] + v;
            a.y[r0 + rho] = v;
        }
    }
}

// --------------------------------------------------------------- dequant
// Bit-exact dequantization, one lane per 64-weight chunk (64 floats out).
template <int TYPE>
__global__ __launch_bounds__(256) void kq_dequant_kernel(const uint8_t* __restrict__ w,
                                                         float* __restrict__ y, long nchunks) {
    using TI = TypeInfo<TYPE>;
    const long f = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= nchunks) return;
    const uint8_t* blk = w + (size_t)(f >> 2) * TI::BB;
    const int u = (int)(f & 3);
    float* yb = y + (size_t)(f >> 2) * 256;
    if (TYPE == T_Q4K) {
        const RawQ4 r = load_q4k(blk, u);
        const float d = f16_bits_to_f32(r.hd.x & 0xffffu);
        const float dmin = f16_bits_to_f32(r.hd.x >> 16);
        const uint8_t* s = blk + 4;
#pragma unroll
        for (int half = 0; half < 2; half++) {
            const int sb = 2 * u + half;
            uint32_t sc, m;
            if (sb < 4) { sc = s[sb] & 63u; m = s[sb + 4] & 63u; }
            else { sc = (s[sb + 4] & 15u) | ((uint32_t)(s[sb - 4] >> 6) << 4);
                   m = ((uint32_t)s[sb + 4] >> 4) | ((uint32_t)(s[sb] >> 6) << 4); }
            const float ds = d * (float)sc, dm = dmin * (float)m;
            for (int l = 0; l < 32; l++) {
                const uint32_t v = blk[16 + 32 * u + l];
                const uint32_t q = half ? (v >> 4) : (v & 15u);
                yb[32 * sb + l] = ds * (float)q - dm;
            }
        }
    } else if (TYPE == T_Q6K) {
        const int h = u >> 1, is = u & 1;
        const float d = f16_bits_to_f32((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
        for (int t = 0; t < 4; t++) {
            const float ds = d * (float)(int8_t)blk[192 + 8 * h + is + 2 * t];
            for (int l2 = 0; l2 < 16; l2++) {
                const int l = 16 * is + l2;
                const uint32_t lo = blk[64 * h + l + 32 * (t & 1)];
                const uint32_t hi = blk[128 + 32 * h + l];
                const int q = (int)(((lo >> (4 * (t >> 1))) & 15u) | (((hi >> (2 * t)) & 3u) << 4)) - 32;
                yb[128 * h + 32 * t + l] = ds * (float)q;
            }
        }
    } else {
        const bool nib = TYPE == T_NIB;
        const int doff = nib ? 144 : 80;
        const float d = f16_bits_to_f32((uint32_t)blk[doff] | ((uint32_t)blk[doff + 1] << 8));
        const float dmin = f16_bits_to_f32((uint32_t)blk[doff + 2] | ((uint32_t)blk[doff + 3] << 8));
        for (int j4 = 0; j4 < 4; j4++) {
            // chunk u covers: Q2_K groups (s = u>>1, j = j4, h = u&1);
            //                 type 42 groups 4u + j4
            int gi, pos0;
            if (nib) { gi = 4 * u + j4; pos0 = 16 * gi; }
            else { const int s = u >> 1, h = u & 1; gi = 8 * s + 2 * j4 + h; pos0 = 128 * s + 32 * j4 + 16 * h; }
            const uint32_t scb = blk[gi];
            const float dl = d * (float)(scb & 15u), ml = dmin * (float)(scb >> 4);
            for (int l = 0; l < 16; l++) {
                const int p = pos0 + l;
                uint32_t q;
                if (nib) {
                    const uint32_t v = blk[16 + 16 * (p >> 5) + (p & 15)];
                    q = (p & 16) ? (v >> 4) : (v & 15u);
                } else {
                    const int s = u >> 1, h = u & 1;
                    q = ((uint32_t)blk[16 + 32 * s + 16 * h + l] >> (2 * j4)) & 3u;
                }
                yb[p] = dl * (float)q - ml;
            }
        }
    }
}

template <int TYPE>
int launch_gemv(const GemvArgs& a, int grid, int threads, int depth, hipStream_t st) {
    const int NC = a.K >> 6;
    const size_t lds = (size_t)x_lds_bytes<TYPE>(a.K) + (size_t)a.rows_per_wg * NC * 8 + 16;
    switch (depth) {
    case 1: hipLaunchKernelGGL((kq_gemv_kernel<TYPE, 1>), dim3(grid), dim3(threads), lds, st, a); break;
    case 2: hipLaunchKernelGGL((kq_gemv_kernel<TYPE, 2>), dim3(grid), dim3(threads), lds, st, a); break;
    case 3: hipLaunchKernelGGL((kq_gemv_kernel<TYPE, 3>), dim3(grid), dim3(threads), lds, st, a); break;
    case 4: hipLaunchKernelGGL((kq_gemv_kernel<TYPE, 4>), dim3(grid), dim3(threads), lds, st, a); break;
    default: hipLaunchKernelGGL((kq_gemv_kernel<TYPE, 6>), dim3(grid), dim3(threads), lds, st, a); break;
    }
    return (int)hipGetLastError();
}

template <int TYPE, int D>
int set_lds1(int bytes) {
    return (int)hipFuncSetAttribute(reinterpret_cast<const void*>(&kq_gemv_kernel<TYPE, D>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

template <int TYPE>
int set_lds(int bytes) {
    int e = set_lds1<TYPE, 1>(bytes);
    if (!e) e = set_lds1<TYPE, 2>(bytes);
    if (!e) e = set_lds1<TYPE, 3>(bytes);
    if (!e) e = set_lds1<TYPE, 4>(bytes);
    if (!e) e = set_lds1<TYPE, 6>(bytes);
    return e;
}

template <int TYPE>
int launch_dequant(const uint8_t* w, float* y, long nblocks, hipStream_t st) {
    const long nch = nblocks * 4;
    const long grid = (nch + 255) / 256;
    hipLaunchKernelGGL(kq_dequant_kernel<TYPE>, dim3((unsigned)grid), dim3(256), 0, st, w, y, nch);
    return (int)hipGetLastError();
}

}  // namespace

// ------------------------------------------------------------ C launchers
extern "C" {

// LDS bytes the GEMV kernel needs for a given type, K and rows per group.
long kqk_gemv_lds_bytes(int type, int K, int rows_per_wg) {
    const long NC = K >> 6;
    long x;
    switch (type) {
    case T_Q4K: x = x_lds_bytes<T_Q4K>(K); break;
    case T_Q6K: x = x_lds_bytes<T_Q6K>(K); break;
    case T_Q2K: x = x_lds_bytes<T_Q2K>(K); break;
    case T_NIB: x = x_lds_bytes<T_NIB>(K); break;
    default: return -1;
    }
    return x + (long)rows_per_wg * NC * 8 + 16;
}

// Allows dynamic LDS up to `bytes` for every GEMV instantiation.
int kqk_set_max_lds(int bytes) {
    int e = set_lds<T_Q4K>(bytes);
    if (!e) e = set_lds<T_Q6K>(bytes);
    if (!e) e = set_lds<T_Q2K>(bytes);
    if (!e) e = set_lds<T_NIB>(bytes);
    return e;
}

// threads must be 256, 512 or 1024; rows_per_wg * (K/64) * 8 plus the x
// staging must fit the LDS limit set above (checked by the caller); depth
// (1..3) is the number of chunks each lane keeps in flight.
int kqk_launch_gemv(int type, const void* w, const float* x, const float* add, float* y,
                    int N, int K, int rows_per_wg, int threads, int depth, hipStream_t st) {
    GemvArgs a;
    a.w = static_cast<const uint8_t*>(w);
    a.x = x; a.add = add; a.y = y;
    a.N = N; a.K = K; a.rows_per_wg = rows_per_wg; a.B = 1;
    const int grid = (N + rows_per_wg - 1) / rows_per_wg;
    switch (type) {
    case T_Q4K: return launch_gemv<T_Q4K>(a, grid, threads, depth, st);
    case T_Q6K: return launch_gemv<T_Q6K>(a, grid, threads, depth, st);
    case T_Q2K: return launch_gemv<T_Q2K>(a, grid, threads, depth, st);
    case T_NIB: return launch_gemv<T_NIB>(a, grid, threads, depth, st);
    default: return -1;
    }
}

int kqk_launch_dequant(int type, const void* w, float* y, long nblocks, hipStream_t st) {
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    switch (type) {
    case T_Q4K: return launch_dequant<T_Q4K>(wb, y, nblocks, st);
    case T_Q6K: return launch_dequant<T_Q6K>(wb, y, nblocks, st);
    case T_Q2K: return launch_dequant<T_Q2K>(wb, y, nblocks, st);
    case T_NIB: return launch_dequant<T_NIB>(wb, y, nblocks, st);
    default: return -1;
    }
}

}  // extern "C"
