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

#include <type_traits>

#include "kq_launch.h"


#pragma clang fp contract(off)

namespace {

constexpr int T_Q80 = 8;
constexpr int T_Q2K = 10;
constexpr int T_Q3K = 11;
constexpr int T_Q4K = 12;
constexpr int T_Q5K = 13;
constexpr int T_Q6K = 14;
constexpr int T_NIB = 42;
// the int8-activation mode (the reference's SDOT path) of Q4_K, Q6_K,
// Q5_K, Q3_K and Q8_0: the type id with this bit set
constexpr int T_I8 = 0x100;
constexpr int T_Q4K_I8 = T_I8 | T_Q4K;
constexpr int T_Q6K_I8 = T_I8 | T_Q6K;
constexpr int T_Q5K_I8 = T_I8 | T_Q5K;
constexpr int T_Q3K_I8 = T_I8 | T_Q3K;
constexpr int T_Q80_I8 = T_I8 | T_Q80;
// float4 slots per chunk in the int8 x layout: 64 bytes padded to 80
// (chunk c at byte 80c; 16-byte reads by consecutive chunks hit distinct
// banks)
constexpr int XPAD_I8 = 5;

constexpr int XPAD = 17;  // float4 slots per 64-weight chunk in LDS (16 + 1 pad)

typedef float f32x4 __attribute__((ext_vector_type(4)));

// BB: bytes per 256 weights; LINEAR: a chunk is 64 consecutive x values
// (else 4 runs of 16, spaced 32 apart); XS_PER_CHUNK: x sums per chunk for
// min terms; SCALED: products by the byte-select multiply on x staged as
// x * 2^KSC (the other types read x as staged and fold the factor into
// their scale).
// I8: the int8-activation mode (x quantized per group, XSTRIDE float4
// slots per chunk of int8 x; XS_PER_CHUNK floats hold each group's scale
// and integer sum).
template <int TYPE> struct TypeInfo;
template <> struct TypeInfo<T_Q4K> { static constexpr int BB = 144; static constexpr bool LINEAR = true;  static constexpr int XS_PER_CHUNK = 2; static constexpr bool SCALED = true; };
template <> struct TypeInfo<T_Q4K_I8> { static constexpr int BB = 144; static constexpr bool LINEAR = true;  static constexpr int XS_PER_CHUNK = 4; static constexpr bool SCALED = false; };
template <> struct TypeInfo<T_Q6K_I8> { static constexpr int BB = 210; static constexpr bool LINEAR = false; static constexpr int XS_PER_CHUNK = 8; static constexpr bool SCALED = false; };
template <> struct TypeInfo<T_Q5K_I8> { static constexpr int BB = 176; static constexpr bool LINEAR = true;  static constexpr int XS_PER_CHUNK = 4; static constexpr bool SCALED = false; };
template <> struct TypeInfo<T_Q80_I8> { static constexpr int BB = 272; static constexpr bool LINEAR = true;  static constexpr int XS_PER_CHUNK = 4; static constexpr bool SCALED = false; };
template <> struct TypeInfo<T_Q3K_I8> { static constexpr int BB = 110; static constexpr bool LINEAR = false; static constexpr int XS_PER_CHUNK = 8; static constexpr bool SCALED = false; };
template <> struct TypeInfo<T_Q6K> { static constexpr int BB = 210; static constexpr bool LINEAR = false; static constexpr int XS_PER_CHUNK = 0; static constexpr bool SCALED = false; };
template <> struct TypeInfo<T_Q2K> { static constexpr int BB = 84;  static constexpr bool LINEAR = false; static constexpr int XS_PER_CHUNK = 4; static constexpr bool SCALED = true; };
template <> struct TypeInfo<T_NIB> { static constexpr int BB = 148; static constexpr bool LINEAR = true;  static constexpr int XS_PER_CHUNK = 4; static constexpr bool SCALED = true; };
template <> struct TypeInfo<T_Q5K> { static constexpr int BB = 176; static constexpr bool LINEAR = true;  static constexpr int XS_PER_CHUNK = 2; static constexpr bool SCALED = true; };
template <> struct TypeInfo<T_Q3K> { static constexpr int BB = 110; static constexpr bool LINEAR = false; static constexpr int XS_PER_CHUNK = 0; static constexpr bool SCALED = false; };
template <> struct TypeInfo<T_Q80> { static constexpr int BB = 272; static constexpr bool LINEAR = true;  static constexpr int XS_PER_CHUNK = 0; static constexpr bool SCALED = false; };


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

// fl(b * x) * 2^-149 for byte SEL (= b) of v: v_mul_f32 with an SDWA byte
// select reads the zero-extended byte b as the binary32 bit pattern b,
// i.e. the denormal b * 2^-149, and multiplies it exactly (fp32 denormals
// are enabled).  With x pre-scaled so that every nonzero product lands in
// the normal range, the rounded product is the reference's fl(b * x)
// times a power of two -- one instruction instead of convert + multiply.
template <int SEL>
__device__ __forceinline__ float bmul(uint32_t v, float x) {
    float r;
    if (SEL == 0)
        asm("v_mul_f32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0 src1_sel:DWORD"
            : "=v"(r) : "v"(v), "v"(x));
    else if (SEL == 1)
        asm("v_mul_f32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1 src1_sel:DWORD"
            : "=v"(r) : "v"(v), "v"(x));
    else if (SEL == 2)
        asm("v_mul_f32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2 src1_sel:DWORD"
            : "=v"(r) : "v"(v), "v"(x));
    else
        asm("v_mul_f32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3 src1_sel:DWORD"
            : "=v"(r) : "v"(v), "v"(x));
    return r;
}

// The products of the four bytes of v with x.x .. x.w: exact conversion +
// multiply (SC = false), or the scaled single-instruction form above.
// x4 is read as one 128-bit LDS load (f32x4, a native vector type, keeps
// the compiler from splitting it into 32-bit reads).

template <bool SC>
__device__ __forceinline__ void bmul4(uint32_t v, const float4* x4, float& p0, float& p1,
                                      float& p2, float& p3) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(x4);
    if (SC) {
        p0 = bmul<0>(v, x.x); p1 = bmul<1>(v, x.y); p2 = bmul<2>(v, x.z); p3 = bmul<3>(v, x.w);
    } else {
        float a, b, c, d;
        ubytes(v, a, b, c, d);
        p0 = a * x.x; p1 = b * x.y; p2 = c * x.z; p3 = d * x.w;
    }
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

// The row reduction's phase count: a row's chunk terms are summed as G
// partials (partial p: chunks p, p+G, ... in order, binary64 from 0),
// combined by the pairwise tree below.  G depends on the row length only
// (8, or 32 for rows longer than 128 chunks, whose long chains would
// otherwise leave few lanes per row busy), so every kernel reproduces it.
__host__ __device__ __forceinline__ int kq_phases(int NC) { return NC > 128 ? 32 : 8; }

// v of lane ^ 16 (both halves)
__device__ __forceinline__ double xor16_f64(double v) {
    const int lo = __shfl_xor(__double2loint(v), 16);
    const int hi = __shfl_xor(__double2hiint(v), 16);
    return __hiloint2double(hi, lo);
}

// Pairwise tree over the G = 8 or 32 partials held by consecutive lanes
// (every lane of the group active):
//   8: ((P0 + P1) + (P2 + P3)) + ((P4 + P5) + (P6 + P7))
//  32: ((S0 + S1) + (S2 + S3)) over the 8-lane sums S0..S3.
// A butterfly: each addition is commutative, so every lane of the group
// ends with the same bits.
__device__ __forceinline__ double phase_tree(double s, int G) {
    s = s + dpp_f64<0xB1>(s);    // quad_perm [1,0,3,2]: lane ^ 1
    s = s + dpp_f64<0x4E>(s);    // quad_perm [2,3,0,1]: lane ^ 2
    s = s + dpp_f64<0x141>(s);   // row_half_mirror: lane i <-> 7 - i (8 lanes)
    if (G == 32) {
        s = s + dpp_f64<0x140>(s);   // row_mirror: 8-lane halves of a 16-lane row
        s = s + xor16_f64(s);        // 16-lane rows 0 <-> 1, 2 <-> 3
    }
    return s;
}

// ------------------------------------------------------------------ LDS x
// x is staged once per workgroup in LDS, in a padded chunk-major layout:
// chunk c (the 64 x values one lane's weights meet) occupies float4 slots
// c*XPAD .. c*XPAD+15.
//  LINEAR  (Q4_K, type 42): chunk = 64 consecutive x values.
//  strided (Q6_K, Q2_K):    chunk = (block, half, 16-sub) = 4 runs of 16
//                           values spaced 32 apart, slot g = 4*run + l/4.
//
// Staging goes through registers in "sum groups": runs of consecutive x
// that one lane loads (128-bit loads), sums in the reference's sequential
// binary32 order when the type has min terms (Q4_K: 32 values per
// sub-block, stratum_q4k.h:115-122; Q2_K / type 42: 16 values,
// stratum_q2k.h:65-68), scales, and writes to its LDS slots.  The first
// weight batches are issued once the first round of x has arrived, so the
// weight stream does not queue ahead of x; their latency overlaps the LDS
// stores and the barrier.
//
// Scaled mode (Q4_K, Q2_K, type 42).  The byte-select multiply (bmul) needs
// every nonzero product q * x' (q >= 1) in the binary32 normal range, so x
// is staged as x' = x * 2^KSC.  Every product and partial sum is then the
// reference's times the same power of two -- exactly, as long as nothing
// overflows or lands below the normal range -- and the factor is folded into
// the block scale at the end (d * sc * 2^(149-KSC) < 2^128).  That holds when
// every finite nonzero x has 2^(23-KSC) <= |x| < 2^(116-KSC), which also
// keeps Q6_K's 16-term sums of int8 * x' below 2^127 (so a Q6_K segment can
// read a scaled x).  When some x falls outside (subnormal, or beyond 2^52),
// the workgroup restages x unscaled and uses the convert-and-multiply path.
constexpr int KSC = 64;
// window test on frexp exponents (|v| in [2^(e-1), 2^e)): allowed
// e in [24 - KSC, 117 - KSC); frexp gives 0 for zero, inf and NaN, which are
// allowed too.  out_of_window(v) = (e - (24 - KSC)) as unsigned >= KSC_SPAN.
constexpr int KSC_ELO = 24 - KSC;
constexpr uint32_t KSC_SPAN = 117 - 24;

template <int TYPE> struct XGroup {
    // float4 per group: 32 values for the types with 32-weight sub-blocks
    // (and the int8 mode's per-32 quantization), else 16
    static constexpr int G4 = (TYPE == T_Q4K || TYPE == T_Q5K || TYPE == T_Q80 ||
                               TYPE == T_Q4K_I8 || TYPE == T_Q5K_I8 || TYPE == T_Q80_I8 ||
                               TYPE == T_Q3K_I8) ? 8 : 4;
    static constexpr bool SUMS = TypeInfo<TYPE>::XS_PER_CHUNK != 0;
    static constexpr bool I8 = (TYPE & T_I8) != 0;
    static constexpr int XSTRIDE = I8 ? XPAD_I8 : XPAD;   // float4 slots per chunk
};

// (e - KSC_ELO) as unsigned: >= KSC_SPAN when v is finite, nonzero and
// outside the scaled-mode window (v_frexp_exp_i32_f32 returns 0 for zero,
// infinities and NaN)
__device__ __forceinline__ uint32_t window_dist(float v) {
    return (uint32_t)(__builtin_amdgcn_frexp_expf(v) - KSC_ELO);
}

// LDS slot (within one x) of float4 q of group gi, and the xs index (within
// one x) of the group's sum.
template <int TYPE>
__device__ __forceinline__ void group_place(int gi, int& slot0, int& xsi) {
    if (XGroup<TYPE>::G4 == 8) {       // 32 values gi: chunk gi/2, slots 8*(gi&1)..
        slot0 = (gi >> 1) * XPAD + 8 * (gi & 1);
        xsi = gi;
    } else if (TYPE == T_NIB) {        // 16-group gi: chunk gi/4, slots 4*(gi&3)..
        slot0 = (gi >> 2) * XPAD + 4 * (gi & 3);
        xsi = gi;                      // == 4 * chunk + (gi & 3)
    } else {                           // strided: x positions 16 gi .. 16 gi + 15
        const int p = 16 * gi, bi = p >> 8, pp = p & 255;
        const int h = pp >> 7, t = (pp >> 5) & 3, is = (pp >> 4) & 1;
        const int c = 4 * bi + 2 * h + is;
        slot0 = c * XPAD + 4 * t;
        xsi = 4 * c + t;
    }
}

// SwiGLU (stratum_swiglu, stratum_engine.h:373-392): g / (1 + expf(-g)) * u,
// binary32 -- kq_swiglu_kernel's expression, so the gather launch's fused
// SwiGLU writes the activations that kernel writes.
__device__ __forceinline__ float swiglu1(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

template <int TYPE>
struct XStage {
    static constexpr int G4 = XGroup<TYPE>::G4;
    const float* x;
    int x_stride, per, total;          // groups per x, groups over all staged x
    int NC;

    __device__ __forceinline__ void load(int gidx, f32x4* v) const {
        const int gc = min(gidx, total - 1);           // branch-free: clamped
        const int gx = per == total ? 0 : gc / per;
        const f32x4* src = reinterpret_cast<const f32x4*>(x + (size_t)gx * x_stride) +
                           (size_t)(gc - gx * per) * G4;
#pragma unroll
        for (int q = 0; q < G4; q++) v[q] = src[q];
    }

    // writes group gidx (if it exists); returns "out of window" for it
    __device__ __forceinline__ bool store(int gidx, const f32x4* v, bool scale, bool sums,
                                          float4* xl, float* xs) const {
        if (gidx >= total) return false;
        const int gx = per == total ? 0 : gidx / per;
        const int gi = gidx - gx * per;
        int slot0, xsi;
        group_place<TYPE>(gi, slot0, xsi);
        f32x4* dst = reinterpret_cast<f32x4*>(xl) + gx * NC * XPAD + slot0;
        uint32_t dist = 0;
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < G4; q++) {
            const f32x4 w = v[q];
            acc = acc + w.x; acc = acc + w.y; acc = acc + w.z; acc = acc + w.w;
            dist = max(max(dist, window_dist(w.x)), window_dist(w.y));
            dist = max(max(dist, window_dist(w.z)), window_dist(w.w));
            f32x4 o = w;
            if (scale) {
                o.x = ldexpf(w.x, KSC); o.y = ldexpf(w.y, KSC);
                o.z = ldexpf(w.z, KSC); o.w = ldexpf(w.w, KSC);
            }
            dst[q] = o;
        }
        if (XGroup<TYPE>::SUMS && sums) xs[gx * per + xsi] = acc;
        return dist >= KSC_SPAN;
    }
};

// Recomputes the per-group sums from an x already in LDS (for a segment
// whose type needs sums laid out differently from the staging type's).
// When the staged x is scaled by 2^ks, the sum of the scaled values is
// scaled back: power-of-two scaling commutes with each binary32 addition
// here (no overflow, and a sum below the normal range is exact), so the
// result equals the unscaled sum.
template <int TYPE>
__device__ __forceinline__ void resum(int K, int ngx, int tid, int T, const float4* xl,
                                      float* xs, int ks) {
    constexpr int G4 = XGroup<TYPE>::G4;
    const int per = K / (4 * G4), NC = K >> 6;
    for (int t = tid; t < ngx * per; t += T) {
        const int gx = t / per, gi = t - gx * per;
        int slot0, xsi;
        group_place<TYPE>(gi, slot0, xsi);
        const f32x4* p = reinterpret_cast<const f32x4*>(xl) + gx * NC * XPAD + slot0;
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < G4; q++) {
            const f32x4 v = p[q];
            acc = acc + v.x; acc = acc + v.y; acc = acc + v.z; acc = acc + v.w;
        }
        xs[gx * per + xsi] = ks ? ldexpf(acc, -ks) : acc;
    }
}

// int8 staging (q4k_quantize_x_q8, stratum_q4k_neon.h:230-277, per 32;
// q6k_quantize_x_q8_g16, stratum_q6k_neon.h:117-133, per 16): a lane
// quantizes the group it loaded -- amax = max |x|, scale = fl(amax / 127),
// inv = scale > 0 ? fl(1 / scale) : 0, q = clamp(rne(fl(x * inv)), -128,
// 127) -- and writes the int8 values to the chunk's slot and {scale, sum}
// to the group's two floats:
//  Q4_K, Q5_K, Q8_0 (linear chunks, per 32): group gi at byte 80(gi/2) +
//    32(gi&1), floats 4 per chunk;
//  Q6_K (strided chunks, per 16): the 16-group at positions 16gi is run t
//    of chunk (block, half, is), at byte 80c + 16t, floats 8 per chunk;
//  Q3_K (strided chunks, per 32): the group's first 16 values are run j of
//    chunk (block, s, 0), its last 16 run j of chunk (block, s, 1) (the
//    group covers positions 128s + 32j ..), and both chunks get its
//    {scale, sum} in their run-j floats.
// x must be finite.
template <int TYPE>
__device__ __forceinline__ void store_i8(int gidx, int per, int NC, const f32x4* v, uint8_t* xq,
                                         float* xs) {
    constexpr int G4 = XGroup<TYPE>::G4;
    const int gx = gidx / per, gi = gidx - gx * per;
    float amax = 0.0f;
#pragma unroll
    for (int q = 0; q < G4; q++)
        amax = fmaxf(fmaxf(fmaxf(amax, fabsf(v[q].x)), fmaxf(fabsf(v[q].y), fabsf(v[q].z))),
                     fabsf(v[q].w));
    const float scale = __fdiv_rn(amax, 127.0f);
    const float inv = scale > 0.0f ? __fdiv_rn(1.0f, scale) : 0.0f;
    int sum = 0;
    uint32_t packed[G4];
#pragma unroll
    for (int q = 0; q < G4; q++) {
        const float e[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int iv = min(127, max(-128, __float2int_rn(e[i] * inv)));
            sum += iv;
            w |= ((uint32_t)iv & 0xffu) << (8 * i);
        }
        packed[q] = w;
    }
    constexpr int XPC = TypeInfo<TYPE>::XS_PER_CHUNK;
    float* xsx = xs + (size_t)gx * NC * XPC;
    if (TYPE == T_Q3K_I8) {
        const int bi = gi >> 3, s = (gi >> 2) & 1, j = gi & 3, c0 = 4 * bi + 2 * s;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint4* dst = reinterpret_cast<uint4*>(xq + (size_t)(gx * NC + c0 + h) * 80 + 16 * j);
            *dst = make_uint4(packed[4 * h], packed[4 * h + 1], packed[4 * h + 2],
                              packed[4 * h + 3]);
            *reinterpret_cast<float2*>(xsx + XPC * (c0 + h) + 2 * j) =
                make_float2(scale, (float)sum);
        }
        return;
    }
    int c, off, slot;
    if (TYPE == T_Q6K_I8) {
        const int p = 16 * gi, bi = p >> 8, h = (p >> 7) & 1, t = (p >> 5) & 3, is = (p >> 4) & 1;
        c = 4 * bi + 2 * h + is; off = 16 * t; slot = 8 * c + 2 * t;
    } else {
        c = gi >> 1; off = 32 * (gi & 1); slot = 2 * gi;
    }
    uint4* dst = reinterpret_cast<uint4*>(xq + (size_t)(gx * NC + c) * 80 + off);
#pragma unroll
    for (int q = 0; q < G4; q += 4)
        dst[q / 4] = make_uint4(packed[q], packed[q + 1], packed[q + 2], packed[q + 3]);
    *reinterpret_cast<float2*>(xsx + slot) = make_float2(scale, (float)sum);
}

// ------------------------------------------------------------ raw loads
// Weight bytes are read through explicit global-address-space pointers.
// A generic pointer (e.g. one read back from the LDS weight-base table)
// would make the compiler emit FLAT loads, which count against lgkmcnt as
// well as vmcnt: every LDS wait in the loop would then also wait for the
// whole weight prefetch.
#define KQ_GLOBAL __attribute__((address_space(1)))
typedef const uint8_t KQ_GLOBAL* wptr;

__device__ __forceinline__ wptr to_global(const uint8_t* p) { return (wptr)p; }

// 128-bit vectors: 16-byte aligned (Q4_K blocks are 144 B) and 4-byte
// aligned (Q6_K/Q2_K/type-42 blocks are only dword aligned;
// global_load_dwordx4 needs dword alignment only).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2a __attribute__((ext_vector_type(2), aligned(4)));

// Weight loads use the default cache policy.  The nontemporal policy
// (global_load ... nt) lifts a plain read stream on this GPU from about 6.4
// to 7.1 TB/s, but here neighbouring lanes read one cache line through
// different load instructions (a block's header and the two quant vectors
// of a 64-weight chunk), and with nt each of them fetches the line again:
// measured 2x slower for Q6_K, 1.2x for Q4_K.
template <typename V>
__device__ __forceinline__ V wload(wptr p) {
    return *reinterpret_cast<const KQ_GLOBAL V*>(p);
}

__device__ __forceinline__ uint4 ld16(wptr p) {
    const u32x4 v = wload<u32x4>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 ld16a4(wptr p) {
    const u32x4a v = wload<u32x4a>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld8a4(wptr p) {
    const u32x2a v = wload<u32x2a>(p);
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ld4(wptr p) {
    return wload<uint32_t>(p);
}
__device__ __forceinline__ uint32_t ld2(wptr p) {
    return wload<uint16_t>(p);
}

struct RawQ4 { uint4 hd, qa, qb; };
struct RawQ6 { uint32_t l[5], h[5], q[5], s[3], d; uint32_t sh; };
struct RawQ2 { uint4 q; uint2 s; uint32_t dd; };
struct RawNB { uint4 qa, qb; uint32_t s, dd; };
struct RawQ5 { uint4 hd, h0, h1, qa, qb; };
struct RawQ3 { uint32_t q[5], m[5], s[4]; uint32_t d, sh; };
struct RawQ8 { uint32_t w[17]; };

__device__ __forceinline__ RawQ4 load_q4k(wptr blk, int j) {
    RawQ4 r;
    r.hd = ld16(blk);
    r.qa = ld16(blk + 16 + 32 * j);
    r.qb = ld16(blk + 32 + 32 * j);
    return r;
}

// Q6_K blocks are 210 B, so odd blocks start 2 bytes off a dword.  Loads
// are dword-aligned and realigned with v_alignbit (shift 0 or 16).
__device__ __forceinline__ void load5(wptr p, uint32_t* o) {
    const uint4 v = ld16a4(p);
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    o[4] = ld4(p + 16);
}

__device__ __forceinline__ RawQ6 load_q6k(wptr blk, int u) {
    RawQ6 r;
    const int h = u >> 1, is = u & 1;
    // realign by pointer arithmetic, which keeps the global address space
    const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(blk) & 3u;
    r.sh = mis * 8u;
    const wptr b4 = blk - mis;
    load5(b4 + 64 * h + 16 * is, r.l);
    load5(b4 + 64 * h + 32 + 16 * is, r.h);
    load5(b4 + 128 + 32 * h + 16 * is, r.q);
    // scales: 8 bytes from 192 + 8h.  A third dword is needed only when the
    // block is 2 bytes off; when aligned, dword 1 is re-read instead so the
    // last block of a tensor never reads past its 210 bytes.
    const wptr sp = b4 + 192 + 8 * h;
    r.s[0] = ld4(sp); r.s[1] = ld4(sp + 4); r.s[2] = ld4(sp + (r.sh ? 8 : 4));
    r.d = ld2(blk + 208);
    return r;
}

__device__ __forceinline__ RawQ2 load_q2k(wptr blk, int u) {
    RawQ2 r;
    const int s = u >> 1, h = u & 1;
    r.q = ld16a4(blk + 16 + 32 * s + 16 * h);
    r.s = ld8a4(blk + 8 * s);
    r.dd = ld4(blk + 80);
    return r;
}

// Q5_K (176 B, 16-byte aligned): header (d, dmin, scales), all of qh, and
// the 32 qs bytes of chunk j
__device__ __forceinline__ RawQ5 load_q5k(wptr blk, int j) {
    RawQ5 r;
    r.hd = ld16(blk);
    r.h0 = ld16(blk + 16);
    r.h1 = ld16(blk + 32);
    r.qa = ld16(blk + 48 + 32 * j);
    r.qb = ld16(blk + 64 + 32 * j);
    return r;
}

// Q3_K (110 B, blocks 2-byte aligned): chunk u = (s, h) reads 16 qs bytes
// at 32 + 32s + 16h, 16 hmask bytes at 16h, the 12 scale bytes at 96 and d
// at 108.  Dword-aligned loads realigned by v_alignbit; the fourth scale
// dword is needed only when the block is 2 bytes off (else dword 2 is read
// again), so the last block of a tensor is never read past its end.
__device__ __forceinline__ RawQ3 load_q3k(wptr blk, int u) {
    RawQ3 r;
    const int s = u >> 1, h = u & 1;
    const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(blk) & 3u;
    r.sh = mis * 8u;
    const wptr b4 = blk - mis;
    load5(b4 + 32 + 32 * s + 16 * h, r.q);
    load5(b4 + 16 * h, r.m);
    r.s[0] = ld4(b4 + 96); r.s[1] = ld4(b4 + 100); r.s[2] = ld4(b4 + 104);
    r.s[3] = ld4(b4 + (mis ? 108 : 104));
    r.d = ld2(blk + 108);
    return r;
}

// Q8_0: a 256-weight unit is eight 34-byte blocks (272 B, 16-byte aligned);
// chunk u is blocks 2u, 2u+1: 68 bytes from the dword-aligned offset 68u
__device__ __forceinline__ RawQ8 load_q80(wptr blk, int u) {
    RawQ8 r;
    const wptr p = blk + 68 * u;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint4 v = ld16a4(p + 16 * k);
        r.w[4 * k] = v.x; r.w[4 * k + 1] = v.y; r.w[4 * k + 2] = v.z; r.w[4 * k + 3] = v.w;
    }
    r.w[16] = ld4(p + 64);
    return r;
}

__device__ __forceinline__ RawNB load_nib(wptr blk, int u) {
    RawNB r;
    r.qa = ld16a4(blk + 16 + 32 * u);
    r.qb = ld16a4(blk + 32 + 32 * u);
    r.s = ld4(blk + 4 * u);
    r.dd = ld4(blk + 144);
    return r;
}

// ---------------------------------------------------------- chunk terms
// Each returns the binary64 sum of the chunk's sub-block terms, computed in
// the reference's binary32 operation order.

__device__ __forceinline__ uint32_t dw_of(const uint4& v, int k) {
    return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}

// Q4_K chunk j of a block: sub-blocks 2j (low nibbles) and 2j+1 (high).
// SC: x is scaled by 2^k and f = 2^(149-k) (see bmul); otherwise f = 1.
// LOWREG: a fence every few steps (the partial sums pinned in registers,
// then a scheduling barrier) keeps the x reads and products from being
// hoisted all at once (the multi-x kernel's register budget).
template <bool SC, bool LOWREG = false>
__device__ __forceinline__ double term_q4k(const RawQ4& r, int j, const float4* xc,
                                           float xs1, float xs2, float f) {
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

    // high nibbles are used in place (16 q), so a2 is 16x the reference's
    // partial sum and d2 is used divided by 16 (both exact)
    float a1 = 0.0f, a2 = 0.0f;
    if (SC) {
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t v = k < 4 ? dw_of(r.qa, k) : dw_of(r.qb, k - 4);
            const uint32_t vl = v & 0x0f0f0f0fu, vh = v & 0xf0f0f0f0u;
            float l0, l1, l2, l3, h0, h1, h2, h3;
            bmul4<true>(vl, xc + k, l0, l1, l2, l3);
            bmul4<true>(vh, xc + 8 + k, h0, h1, h2, h3);
            a1 = a1 + l0; a2 = a2 + h0;
            a1 = a1 + l1; a2 = a2 + h1;
            a1 = a1 + l2; a2 = a2 + h2;
            a1 = a1 + l3; a2 = a2 + h3;
            if (LOWREG && (k & 1)) {
                asm volatile("" : "+v"(a1), "+v"(a2));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else {
        // exact convert path for x outside the window (rare): a rolled loop,
        // the packed words rotating through q0, so that its registers do not
        // raise the register count of the whole kernel
        uint32_t q0 = r.qa.x, q1 = r.qa.y, q2 = r.qa.z, q3 = r.qa.w;
        uint32_t q4 = r.qb.x, q5 = r.qb.y, q6 = r.qb.z, q7 = r.qb.w;
#pragma unroll 1
        for (int k = 0; k < 8; k++) {
            const uint32_t v = q0;
            q0 = q1; q1 = q2; q2 = q3; q3 = q4; q4 = q5; q5 = q6; q6 = q7; q7 = v;
            float l0, l1, l2, l3, h0, h1, h2, h3;
            bmul4<false>(v & 0x0f0f0f0fu, xc + k, l0, l1, l2, l3);
            bmul4<false>(v & 0xf0f0f0f0u, xc + 8 + k, h0, h1, h2, h3);
            a1 = a1 + l0; a2 = a2 + h0;
            a1 = a1 + l1; a2 = a2 + h1;
            a1 = a1 + l2; a2 = a2 + h2;
            a1 = a1 + l3; a2 = a2 + h3;
        }
    }
    const float d1s = SC ? d1 * f : d1;
    const float d2s = d2 * (SC ? f * 0.0625f : 0.0625f);
    const float t1 = d1s * a1 - mm1 * xs1;
    const float t2 = d2s * a2 - mm2 * xs2;
    return (double)t1 + (double)t2;
}

__device__ __forceinline__ float i8f(uint32_t v, int e) {
    return (float)(int32_t)(int8_t)(uint8_t)(v >> (8 * e));
}

// Q6_K chunk (half h, sub is): four 16-weight sums a_t, t = 0..3.
// f6 = 2^(-2-k) when x is scaled by 2^k (k = 0: unscaled).
// The four words of step k (16 weights of each of the 4 runs of the chunk):
// byte = ((q ^ 0x20) << 2) = int8 4*(q - 32), q = lo4 | hi2 << 4.
__device__ __forceinline__ void q6k_words(const RawQ6& r, int k, uint32_t (&y)[4]) {
    const uint32_t sh = r.sh;
    const uint32_t L = __builtin_amdgcn_alignbit(r.l[k + 1], r.l[k], sh);
    const uint32_t H = __builtin_amdgcn_alignbit(r.h[k + 1], r.h[k], sh);
    const uint32_t Q = __builtin_amdgcn_alignbit(r.q[k + 1], r.q[k], sh) ^ 0xaaaaaaaau;
    y[0] = ((L << 2) & 0x3c3c3c3cu) | ((Q << 6) & 0xc0c0c0c0u);
    y[1] = ((H << 2) & 0x3c3c3c3cu) | ((Q << 4) & 0xc0c0c0c0u);
    y[2] = ((L >> 2) & 0x3c3c3c3cu) | ((Q << 2) & 0xc0c0c0c0u);
    y[3] = ((H >> 2) & 0x3c3c3c3cu) | (Q & 0xc0c0c0c0u);
}

// The chunk term from the four 16-weight sums: d * s[t] * a_t in binary64.
__device__ __forceinline__ double q6k_combine(const RawQ6& r, int u, const float (&a)[4],
                                              double f6) {
    const int is = u & 1;
    const uint32_t sh = r.sh;
    // scales s[8h + is + 2t] sit at bytes is + 2t of the realigned pair
    const uint32_t S0 = __builtin_amdgcn_alignbit(r.s[1], r.s[0], sh);
    const uint32_t S1 = __builtin_amdgcn_alignbit(r.s[2], r.s[1], sh);
    const uint32_t dh = r.d;
    const double dq = (double)f16_bits_to_f32(dh) * f6;  // exact
    const uint32_t Sa = is ? (S0 >> 8) : S0;
    const uint32_t Sb = is ? (S1 >> 8) : S1;
    const double t0 = (dq * (double)(int8_t)(uint8_t)(Sa)) * (double)a[0];
    const double t1 = (dq * (double)(int8_t)(uint8_t)(Sa >> 16)) * (double)a[1];
    const double t2 = (dq * (double)(int8_t)(uint8_t)(Sb)) * (double)a[2];
    const double t3 = (dq * (double)(int8_t)(uint8_t)(Sb >> 16)) * (double)a[3];
    return (t0 + t1) + (t2 + t3);
}

// Q6_K chunk (half h, sub is): four 16-weight sums a_t, t = 0..3.
// f6 = 2^(-2-k) when x is scaled by 2^k (k = 0: unscaled).
template <bool LOWREG = false>
__device__ __forceinline__ double term_q6k(const RawQ6& r, int u, const float4* xc, double f6) {
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t y[4];
        q6k_words(r, k, y);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float4 xv = xc[4 * t + k];
            a[t] = a[t] + i8f(y[t], 0) * xv.x;
            a[t] = a[t] + i8f(y[t], 1) * xv.y;
            a[t] = a[t] + i8f(y[t], 2) * xv.z;
            a[t] = a[t] + i8f(y[t], 3) * xv.w;
        }
        if (LOWREG) {
            asm volatile("" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    return q6k_combine(r, u, a, f6);
}

// The Q6_K chunk terms of S members at once (the multi-x kernel): each
// step's 16 conversions are shared by the members, and fences bound the
// live ranges (converted quants, x, partial sums).  Member s's term is
// term_q6k's for xc[s], operation for operation; members with !ok[s] are
// skipped.
template <int S>
__device__ __forceinline__ void mx_term_q6k(const RawQ6& r, int u, const float4* const (&xc)[S],
                                            const bool (&ok)[S], double f6, double (&part)[S]) {
    float a[S][4];
#pragma unroll
    for (int s = 0; s < S; s++) a[s][0] = a[s][1] = a[s][2] = a[s][3] = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t y[4];
        q6k_words(r, k, y);
        float q[16];
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int e = 0; e < 4; e++) q[4 * t + e] = i8f(y[t], e);
        asm volatile("" : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(q[4]),
                     "+v"(q[5]), "+v"(q[6]), "+v"(q[7]), "+v"(q[8]), "+v"(q[9]), "+v"(q[10]),
                     "+v"(q[11]), "+v"(q[12]), "+v"(q[13]), "+v"(q[14]), "+v"(q[15]));
#pragma unroll
        for (int s = 0; s < S; s++) {
            if (ok[s]) {
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const float4 xv = xc[s][4 * t + k];
                    a[s][t] = a[s][t] + q[4 * t + 0] * xv.x;
                    a[s][t] = a[s][t] + q[4 * t + 1] * xv.y;
                    a[s][t] = a[s][t] + q[4 * t + 2] * xv.z;
                    a[s][t] = a[s][t] + q[4 * t + 3] * xv.w;
                }
                asm volatile("" : "+v"(a[s][0]), "+v"(a[s][1]), "+v"(a[s][2]), "+v"(a[s][3]));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
#pragma unroll
    for (int s = 0; s < S; s++)
        if (ok[s]) part[s] = part[s] + q6k_combine(r, u, a[s], f6);
}

// Q2_K chunk (half s, 16-sub h): groups j = 0..3, q = (qs >> 2j) & 3.
template <bool SC, bool LOWREG = false>
__device__ __forceinline__ double term_q2k(const RawQ2& r, int u, const float4* xc,
                                           const float4 xs4, float f) {
    const int h = u & 1;
    const float d = f16_bits_to_f32(r.dd & 0xffffu);
    const float dmin = f16_bits_to_f32(r.dd >> 16);
    const uint32_t S0 = h ? (r.s.x >> 8) : r.s.x;   // bytes h, h+2
    const uint32_t S1 = h ? (r.s.y >> 8) : r.s.y;   // bytes h+4, h+6
    double acc = 0.0;
    if (SC) {
        const uint32_t sc[4] = {S0 & 0xffu, (S0 >> 16) & 0xffu, S1 & 0xffu, (S1 >> 16) & 0xffu};
        const float sx[4] = {xs4.x, xs4.y, xs4.z, xs4.w};
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
                float p0, p1, p2, p3;
                bmul4<true>(v, xc + 4 * j + k, p0, p1, p2, p3);
                qx = qx + p0;
                qx = qx + p1;
                qx = qx + p2;
                qx = qx + p3;
            }
            const float t = (dl * (inv * f)) * qx - ml * sx[j];
            acc = acc + (double)t;
            if (LOWREG) {
                asm volatile("" : "+v"(acc));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else {
        // exact convert path (x outside the window): rolled over j, with
        // the scale bytes, x sums and 1/4^j rotating through the first slot
        uint32_t s0 = S0 & 0xffu, s1 = (S0 >> 16) & 0xffu, s2 = S1 & 0xffu, s3 = (S1 >> 16) & 0xffu;
        float x0 = xs4.x, x1 = xs4.y, x2 = xs4.z, x3 = xs4.w;
        float inv = 1.0f;
#pragma unroll 1
        for (int j = 0; j < 4; j++) {
            const float dl = d * (float)(s0 & 15u);
            const float ml = dmin * (float)(s0 >> 4);
            const uint32_t m = 0x03030303u << (2 * j);
            float qx = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float p0, p1, p2, p3;
                bmul4<false>(dw_of(r.q, k) & m, xc + 4 * j + k, p0, p1, p2, p3);
                qx = qx + p0;
                qx = qx + p1;
                qx = qx + p2;
                qx = qx + p3;
            }
            const float t = (dl * inv) * qx - ml * x0;
            acc = acc + (double)t;
            s0 = s1; s1 = s2; s2 = s3;
            x0 = x1; x1 = x2; x2 = x3;
            inv = inv * 0.25f;
        }
    }
    return acc;
}

// type-42 chunk u: 64 consecutive weights = groups 4u..4u+3; group g's
// 16 values are the low (g even) or high (g odd) nibbles of 16 bytes.
template <bool SC, bool LOWREG = false>
__device__ __forceinline__ double term_nib(const RawNB& r, const float4* xc, const float4 xs4,
                                           float f) {
    const float d = f16_bits_to_f32(r.dd & 0xffffu);
    const float dmin = f16_bits_to_f32(r.dd >> 16);
    double acc = 0.0;
    if (SC) {
        const float sx[4] = {xs4.x, xs4.y, xs4.z, xs4.w};
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const uint32_t scb = (r.s >> (8 * g)) & 0xffu;
            const float dl = d * (float)(scb & 15u);
            const float ml = dmin * (float)(scb >> 4);
            const uint4 src = (g < 2) ? r.qa : r.qb;
            // high-nibble groups are used in place (16 q): scale dl by 1/16
            const float inv = (g & 1) ? 0.0625f : 1.0f;
            float qx = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                uint32_t v = dw_of(src, k);
                v = (g & 1) ? (v & 0xf0f0f0f0u) : (v & 0x0f0f0f0fu);
                float p0, p1, p2, p3;
                bmul4<true>(v, xc + 4 * g + k, p0, p1, p2, p3);
                qx = qx + p0;
                qx = qx + p1;
                qx = qx + p2;
                qx = qx + p3;
            }
            const float t = (dl * (inv * f)) * qx - ml * sx[g];
            acc = acc + (double)t;
            if (LOWREG) {
                asm volatile("" : "+v"(acc));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else {
        // exact convert path (x outside the window): rolled over g, with the
        // packed words and x sums rotating through the first slots
        uint32_t w0 = r.qa.x, w1 = r.qa.y, w2 = r.qa.z, w3 = r.qa.w;
        uint32_t w4 = r.qb.x, w5 = r.qb.y, w6 = r.qb.z, w7 = r.qb.w;
        float x0 = xs4.x, x1 = xs4.y, x2 = xs4.z, x3 = xs4.w;
        uint32_t sc = r.s;
#pragma unroll 1
        for (int g = 0; g < 4; g++) {
            const float dl = d * (float)(sc & 15u);
            const float ml = dmin * (float)((sc >> 4) & 15u);
            const bool hi = g & 1;
            const uint32_t m = hi ? 0xf0f0f0f0u : 0x0f0f0f0fu;
            float qx = 0.0f;
            const uint32_t v4[4] = {w0, w1, w2, w3};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float p0, p1, p2, p3;
                bmul4<false>(v4[k] & m, xc + 4 * g + k, p0, p1, p2, p3);
                qx = qx + p0;
                qx = qx + p1;
                qx = qx + p2;
                qx = qx + p3;
            }
            const float t = (dl * (hi ? 0.0625f : 1.0f)) * qx - ml * x0;
            acc = acc + (double)t;
            if (hi) {                    // next pair of groups reads qb
                w0 = w4; w1 = w5; w2 = w6; w3 = w7;
            }
            sc >>= 8;
            x0 = x1; x1 = x2; x2 = x3;
        }
    }
    return acc;
}

// Q4_K / Q5_K 6-bit scale and min of sub-blocks 2j, 2j+1 from the 12
// scale bytes in words s0..s2 (stratum_q4k.h:57-65)
__device__ __forceinline__ void scale_min_pair(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                               uint32_t& sc1, uint32_t& m1, uint32_t& sc2,
                                               uint32_t& m2) {
    const bool lo = j < 2;
    const uint32_t ob = (uint32_t)((2 * j) & 3) * 8u;
    const uint32_t a_sc = lo ? s0 : s2;
    const uint32_t a_m = lo ? s1 : s2;
    const uint32_t w6 = lo ? 6u : 4u;
    const uint32_t om = lo ? 0u : 4u;
    const uint32_t wh = lo ? 0u : 2u;
    sc1 = bfe(a_sc, ob, w6) | (bfe(s0, ob + 6, wh) << 4);
    m1 = bfe(a_m, ob + om, w6) | (bfe(s1, ob + 6, wh) << 4);
    sc2 = bfe(a_sc, ob + 8, w6) | (bfe(s0, ob + 14, wh) << 4);
    m2 = bfe(a_m, ob + 8 + om, w6) | (bfe(s1, ob + 14, wh) << 4);
}

// Q5_K chunk j (stratum_q5k.h:44-82): sub-blocks 2j and 2j+1 with the
// fifth bit from qh bits 2j / 2j+1; the chunk's term is ONE binary32
// expression ((d1*qx1 - m1*sx1) + d2*qx2) - m2*sx2.  Bytes hold q (0..31),
// so the scaled byte-select products apply as for Q4_K.
template <bool SC>
__device__ __forceinline__ double term_q5k(const RawQ5& r, int j, const float4* xc, float xs1,
                                           float xs2, float f) {
    const float d = f16_bits_to_f32(r.hd.x & 0xffffu);
    const float dmin = f16_bits_to_f32(r.hd.x >> 16);
    uint32_t sc1, mn1, sc2, mn2;
    scale_min_pair(r.hd.y, r.hd.z, r.hd.w, j, sc1, mn1, sc2, mn2);
    const float d1 = d * (float)sc1, m1 = dmin * (float)mn1;
    const float d2 = d * (float)sc2, m2 = dmin * (float)mn2;
    const uint32_t b1 = 2u * (uint32_t)j;
    float a1 = 0.0f, a2 = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t v = k < 4 ? dw_of(r.qa, k) : dw_of(r.qb, k - 4);
        const uint32_t h = k < 4 ? dw_of(r.h0, k) : dw_of(r.h1, k - 4);
        const uint32_t vl = (v & 0x0f0f0f0fu) | (((h >> b1) & 0x01010101u) << 4);
        const uint32_t vh = ((v >> 4) & 0x0f0f0f0fu) | (((h >> (b1 + 1)) & 0x01010101u) << 4);
        float l0, l1, l2, l3, h0, h1, h2, h3;
        bmul4<SC>(vl, xc + k, l0, l1, l2, l3);
        bmul4<SC>(vh, xc + 8 + k, h0, h1, h2, h3);
        a1 = a1 + l0; a2 = a2 + h0;
        a1 = a1 + l1; a2 = a2 + h1;
        a1 = a1 + l2; a2 = a2 + h2;
        a1 = a1 + l3; a2 = a2 + h3;
        // fence every two steps: without it the x reads of all eight are
        // hoisted and, with qh held too, the kernel spills at 128 VGPRs
        if (k & 1) {
            asm volatile("" : "+v"(a1), "+v"(a2));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const float d1s = SC ? d1 * f : d1;
    const float d2s = SC ? d2 * f : d2;
    const float t = ((d1s * a1 - m1 * xs1) + d2s * a2) - m2 * xs2;
    return (double)t;
}

// Q3_K chunk u = (s, h): groups j = 0..3 of 16 weights at 128s + 32j + 16h
// (stratum_q3k.h:58-99).  q3 = ((qs >> 2j) & 3) - 4 unless bit 4s + j of
// hmask is set; each byte is built as the int8 32*q3 (the three bits of the
// two's-complement q3 in bits 5..7) and converted exactly, so every partial
// sum is 32x the reference's; that factor and the staging scale 2^k are
// folded into the group's scale (fk = 2^-k).
__device__ __forceinline__ double term_q3k(const RawQ3& r, int u, const float4* xc, double fk) {
    const int s = u >> 1, h = u & 1;
    const uint32_t sh = r.sh;
    const float d = f16_bits_to_f32(r.d);
    const float fs = (float)(fk * 0.03125);
    const uint32_t S0 = __builtin_amdgcn_alignbit(r.s[1], r.s[0], sh);
    const uint32_t S1 = __builtin_amdgcn_alignbit(r.s[2], r.s[1], sh);
    const uint32_t S2 = __builtin_amdgcn_alignbit(r.s[3], r.s[2], sh);
    uint32_t Q[4], M[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        Q[k] = __builtin_amdgcn_alignbit(r.q[k + 1], r.q[k], sh);
        M[k] = __builtin_amdgcn_alignbit(r.m[k + 1], r.m[k], sh);
    }
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        // 6-bit scale of group g = 8s + 2j + h: word 2s + (j >> 1), byte
        // bi = 2(j & 1) + h (stratum_q3k.h:17-28)
        const uint32_t bi = 8u * (uint32_t)(2 * (j & 1) + h);
        const uint32_t w = (uint32_t)(2 * s + (j >> 1));
        const uint32_t nib = bfe((w & 1u) ? S1 : S0, bi + ((w & 2u) ? 4u : 0u), 4);
        const uint32_t hi2 = bfe(S2, bi + 2u * w, 2);
        const float dl = d * (float)((int)(nib | (hi2 << 4)) - 32);
        float a = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t lo2 = (Q[k] >> (2 * j)) & 0x03030303u;
            const uint32_t neg = ((~M[k] >> (4 * s + j)) & 0x01010101u) << 2;
            const uint32_t y = (lo2 | neg) << 5;              // int8 32 * q3 per byte
            const float4 xv = xc[4 * j + k];
            a = a + i8f(y, 0) * xv.x;
            a = a + i8f(y, 1) * xv.y;
            a = a + i8f(y, 2) * xv.z;
            a = a + i8f(y, 3) * xv.w;
        }
        acc = acc + (double)((dl * fs) * a);
    }
    return acc;
}

// Q8_0 chunk u: blocks 2u and 2u+1 (stratum_q8_0.h:19-33): per block the
// binary32 sum of 32 products int8 q * x, then fl(d * acc); fk = 2^-k for
// x staged as x * 2^k.
__device__ __forceinline__ double term_q80(const RawQ8& r, const float4* xc, double fk) {
    const float f = (float)fk;
    double acc = 0.0;
#pragma unroll
    for (int half = 0; half < 2; half++) {
        const float d = f16_bits_to_f32(half ? (r.w[8] >> 16) : (r.w[0] & 0xffffu));
        float a = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            // block 0's quants start 2 bytes into dword 0; block 1's at dword 9
            const uint32_t v = half ? r.w[9 + k] : __builtin_amdgcn_alignbit(r.w[k + 1], r.w[k], 16);
            const float4 xv = xc[8 * half + k];
            a = a + i8f(v, 0) * xv.x;
            a = a + i8f(v, 1) * xv.y;
            a = a + i8f(v, 2) * xv.z;
            a = a + i8f(v, 3) * xv.w;
        }
        acc = acc + (double)((d * f) * a);
    }
    return acc;
}

// Q4_K chunk j with int8 activations: exact integer dots L, H of the two
// sub-blocks (v_dot4), coefficients as q4k_dot_row_sdot_f forms them
// (stratum_q4k_neon.h:389-392: fl(fl(d*sc)*xs), fl(fl(-dmin*m)*xs)), and
// each sub-block's term c1*L + c2*xsum formed exactly in binary64 (the
// products are exact; one rounding).  xq: the chunk's 16 dwords; xs4 =
// {scale, sum} of the two sub-blocks.
__device__ __forceinline__ double term_q4k_i8(const RawQ4& r, int j, const uint32_t* xq,
                                              float4 xs4) {
    const float d = f16_bits_to_f32(r.hd.x & 0xffffu);
    const float dmin = f16_bits_to_f32(r.hd.x >> 16);
    uint32_t sc1, mn1, sc2, mn2;
    scale_min_pair(r.hd.y, r.hd.z, r.hd.w, j, sc1, mn1, sc2, mn2);
    const uint4 xa = reinterpret_cast<const uint4*>(xq)[0], xb = reinterpret_cast<const uint4*>(xq)[1];
    const uint4 xc = reinterpret_cast<const uint4*>(xq)[2], xd = reinterpret_cast<const uint4*>(xq)[3];
    const uint32_t lo_x[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    const uint32_t hi_x[8] = {xc.x, xc.y, xc.z, xc.w, xd.x, xd.y, xd.z, xd.w};
    int L = 0, H = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t v = k < 4 ? dw_of(r.qa, k) : dw_of(r.qb, k - 4);
        L = __builtin_amdgcn_sdot4((int)(v & 0x0f0f0f0fu), (int)lo_x[k], L, false);
        H = __builtin_amdgcn_sdot4((int)((v >> 4) & 0x0f0f0f0fu), (int)hi_x[k], H, false);
    }
    const float c1 = d * (float)sc1 * xs4.x, c2 = -dmin * (float)mn1 * xs4.x;
    const float c3 = d * (float)sc2 * xs4.z, c4 = -dmin * (float)mn2 * xs4.z;
    const double t1 = fma((double)c1, (double)L, (double)c2 * (double)xs4.y);
    const double t2 = fma((double)c3, (double)H, (double)c4 * (double)xs4.w);
    return t1 + t2;
}

// Q6_K chunk (half h, sub is) with int8 activations per 16
// (q6k_dot_row_sdot_f, stratum_q6k_neon.h:265-317): run t holds the
// unsigned 6-bit values; g4 = their exact dot with the run's 16 quantized
// values minus 32 * the group's x sum; the coefficient fl(fl(d*sc)*xs);
// term c * g4 exact in binary64, summed over t in order.  xs8 = {scale,
// sum} of the four groups.
__device__ __forceinline__ double term_q6k_i8(const RawQ6& r, int u, const uint32_t* xq,
                                              const float* xs8) {
    int acc[4] = {0, 0, 0, 0};
    const uint32_t sh = r.sh;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t L = __builtin_amdgcn_alignbit(r.l[k + 1], r.l[k], sh);
        const uint32_t H = __builtin_amdgcn_alignbit(r.h[k + 1], r.h[k], sh);
        const uint32_t Q = __builtin_amdgcn_alignbit(r.q[k + 1], r.q[k], sh);
        const uint32_t y[4] = {(L & 0x0f0f0f0fu) | ((Q & 0x03030303u) << 4),
                               (H & 0x0f0f0f0fu) | (((Q >> 2) & 0x03030303u) << 4),
                               ((L >> 4) & 0x0f0f0f0fu) | (((Q >> 4) & 0x03030303u) << 4),
                               ((H >> 4) & 0x0f0f0f0fu) | (((Q >> 6) & 0x03030303u) << 4)};
#pragma unroll
        for (int t = 0; t < 4; t++) acc[t] = __builtin_amdgcn_sdot4((int)y[t], (int)xq[4 * t + k], acc[t], false);
    }
    const int is = u & 1;
    const uint32_t S0 = __builtin_amdgcn_alignbit(r.s[1], r.s[0], sh);
    const uint32_t S1 = __builtin_amdgcn_alignbit(r.s[2], r.s[1], sh);
    const uint32_t Sa = is ? (S0 >> 8) : S0, Sb = is ? (S1 >> 8) : S1;
    const int scv[4] = {(int8_t)(uint8_t)Sa, (int8_t)(uint8_t)(Sa >> 16), (int8_t)(uint8_t)Sb,
                        (int8_t)(uint8_t)(Sb >> 16)};
    const float d = f16_bits_to_f32(r.d);
    double t = 0.0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float c = d * (float)scv[q] * xs8[2 * q];
        const int g4 = acc[q] - 32 * (int)xs8[2 * q + 1];
        t = t + (double)c * (double)g4;
    }
    return t;
}

// Q5_K chunk j with int8 activations (q5k_dot_row_sdot_f,
// stratum_q5k_neon.h:158-204): Q4_K's form with the 5-bit values (nibble
// plus 16 times the qh bit, 0..31) in the exact dots.
__device__ __forceinline__ double term_q5k_i8(const RawQ5& r, int j, const uint32_t* xq,
                                              float4 xs4) {
    const float d = f16_bits_to_f32(r.hd.x & 0xffffu);
    const float dmin = f16_bits_to_f32(r.hd.x >> 16);
    uint32_t sc1, mn1, sc2, mn2;
    scale_min_pair(r.hd.y, r.hd.z, r.hd.w, j, sc1, mn1, sc2, mn2);
    const uint4 xa = reinterpret_cast<const uint4*>(xq)[0], xb = reinterpret_cast<const uint4*>(xq)[1];
    const uint4 xc = reinterpret_cast<const uint4*>(xq)[2], xd = reinterpret_cast<const uint4*>(xq)[3];
    const uint32_t lo_x[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    const uint32_t hi_x[8] = {xc.x, xc.y, xc.z, xc.w, xd.x, xd.y, xd.z, xd.w};
    const uint32_t b1 = 2u * (uint32_t)j;
    int L = 0, H = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t v = k < 4 ? dw_of(r.qa, k) : dw_of(r.qb, k - 4);
        const uint32_t h = k < 4 ? dw_of(r.h0, k) : dw_of(r.h1, k - 4);
        const uint32_t vl = (v & 0x0f0f0f0fu) | (((h >> b1) & 0x01010101u) << 4);
        const uint32_t vh = ((v >> 4) & 0x0f0f0f0fu) | (((h >> (b1 + 1)) & 0x01010101u) << 4);
        L = __builtin_amdgcn_sdot4((int)vl, (int)lo_x[k], L, false);
        H = __builtin_amdgcn_sdot4((int)vh, (int)hi_x[k], H, false);
    }
    const float c1 = d * (float)sc1 * xs4.x, c2 = -dmin * (float)mn1 * xs4.x;
    const float c3 = d * (float)sc2 * xs4.z, c4 = -dmin * (float)mn2 * xs4.z;
    const double t1 = fma((double)c1, (double)L, (double)c2 * (double)xs4.y);
    const double t2 = fma((double)c3, (double)H, (double)c4 * (double)xs4.w);
    return t1 + t2;
}

// Q3_K chunk u = (s, h) with int8 activations per 32 (q3k_dot_row_sdot_f,
// stratum_q3k_neon.h:84-125): group j's 16 signed 3-bit values, built as
// the int8 32 q3 (term_q3k's bytes) so v_dot4 gives 32 times the exact dot,
// which an arithmetic shift undoes; coefficient fl(fl(d (sc - 32)) xs) with
// the scale of the 32-group holding the run (xs8[2j]); term c * dot exact
// in binary64, summed over j in order.  No min term.
__device__ __forceinline__ double term_q3k_i8(const RawQ3& r, int u, const uint32_t* xq,
                                              const float* xs8) {
    const int s = u >> 1, h = u & 1;
    const uint32_t sh = r.sh;
    const float d = f16_bits_to_f32(r.d);
    const uint32_t S0 = __builtin_amdgcn_alignbit(r.s[1], r.s[0], sh);
    const uint32_t S1 = __builtin_amdgcn_alignbit(r.s[2], r.s[1], sh);
    const uint32_t S2 = __builtin_amdgcn_alignbit(r.s[3], r.s[2], sh);
    uint32_t Q[4], M[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        Q[k] = __builtin_amdgcn_alignbit(r.q[k + 1], r.q[k], sh);
        M[k] = __builtin_amdgcn_alignbit(r.m[k + 1], r.m[k], sh);
    }
    double t = 0.0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t bi = 8u * (uint32_t)(2 * (j & 1) + h);
        const uint32_t w = (uint32_t)(2 * s + (j >> 1));
        const uint32_t nib = bfe((w & 1u) ? S1 : S0, bi + ((w & 2u) ? 4u : 0u), 4);
        const uint32_t hi2 = bfe(S2, bi + 2u * w, 2);
        const float c = d * (float)((int)(nib | (hi2 << 4)) - 32) * xs8[2 * j];
        int acc = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t lo2 = (Q[k] >> (2 * j)) & 0x03030303u;
            const uint32_t neg = ((~M[k] >> (4 * s + j)) & 0x01010101u) << 2;
            acc = __builtin_amdgcn_sdot4((int)((lo2 | neg) << 5), (int)xq[4 * j + k], acc, false);
        }
        t = t + (double)c * (double)(acc >> 5);
    }
    return t;
}

// Q8_0 chunk u (blocks 2u, 2u+1) with int8 activations per 32
// (q8_0_dot_row_sdot_f, stratum_q8_0.h:112-145): per block the exact dot
// of its int8 quants with the block's quantized x, coefficient fl(d * xs),
// term c * dot exact in binary64; the chunk's two terms added.
__device__ __forceinline__ double term_q80_i8(const RawQ8& r, const uint32_t* xq, float4 xs4) {
    double t = 0.0;
#pragma unroll
    for (int half = 0; half < 2; half++) {
        const float d = f16_bits_to_f32(half ? (r.w[8] >> 16) : (r.w[0] & 0xffffu));
        int acc = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t v = half ? r.w[9 + k] : __builtin_amdgcn_alignbit(r.w[k + 1], r.w[k], 16);
            acc = __builtin_amdgcn_sdot4((int)v, (int)xq[8 * half + k], acc, false);
        }
        const float c = d * (half ? xs4.z : xs4.x);
        t = t + (double)c * (double)acc;
    }
    return t;
}

// ------------------------------------------------------ per-type dispatch
template <int TYPE> struct Chunk;
template <> struct Chunk<T_Q5K_I8> {
    using Raw = RawQ5;
    static __device__ __forceinline__ Raw load(wptr blk, int u) { return load_q5k(blk, u); }
    static __device__ __forceinline__ void drain(const Raw& r) {
        asm volatile("" ::"v"(r.hd.x), "v"(r.h0.x), "v"(r.h1.x), "v"(r.qa.x), "v"(r.qb.x));
    }
    template <bool SC, bool LOWREG = false>
    static __device__ __forceinline__ double term(const Raw& r, int u, const float4* xc,
                                                  const float* xs, int c, float, double) {
        return term_q5k_i8(r, u, reinterpret_cast<const uint32_t*>(xc),
                           reinterpret_cast<const float4*>(xs)[c]);
    }
};
template <> struct Chunk<T_Q3K_I8> {
    using Raw = RawQ3;
    static __device__ __forceinline__ Raw load(wptr blk, int u) { return load_q3k(blk, u); }
    static __device__ __forceinline__ void drain(const Raw& r) {
        asm volatile("" ::"v"(r.q[0]), "v"(r.q[4]), "v"(r.m[0]), "v"(r.m[4]), "v"(r.s[0]),
                     "v"(r.s[3]), "v"(r.d));
    }
    template <bool SC, bool LOWREG = false>
    static __device__ __forceinline__ double term(const Raw& r, int u, const float4* xc,
                                                  const float* xs, int c, float, double) {
        return term_q3k_i8(r, u, reinterpret_cast<const uint32_t*>(xc), xs + 8 * c);
    }
};
template <> struct Chunk<T_Q80_I8> {
    using Raw = RawQ8;
    static __device__ __forceinline__ Raw load(wptr blk, int u) { return load_q80(blk, u); }
    static __device__ __forceinline__ void drain(const Raw& r) {
        asm volatile("" ::"v"(r.w[0]), "v"(r.w[12]), "v"(r.w[16]));
    }
    template <bool SC, bool LOWREG = false>
    static __device__ __forceinline__ double term(const Raw& r, int, const float4* xc,
                                                  const float* xs, int c, float, double) {
        return term_q80_i8(r, reinterpret_cast<const uint32_t*>(xc),
                           reinterpret_cast<const float4*>(xs)[c]);
    }
};
template <> struct Chunk<T_Q4K_I8> {
    using Raw = RawQ4;
    static __device__ __forceinline__ Raw load(wptr blk, int u) { return load_q4k(blk, u); }
    static __device__ __forceinline__ void drain(const Raw& r) {
        asm volatile("" ::"v"(r.hd.x), "v"(r.qa.x), "v"(r.qb.x));
    }
    template <bool SC, bool LOWREG = false>
    static __device__ __forceinline__ double term(const Raw& r, int u, const float4* xc,
                                                  const float* xs, int c, float, double) {
        return term_q4k_i8(r, u, reinterpret_cast<const uint32_t*>(xc),
                           reinterpret_cast<const float4*>(xs)[c]);
    }
};
template <> struct Chunk<T_Q6K_I8> {
    using Raw = RawQ6;
    static __device__ __forceinline__ Raw load(wptr blk, int u) { return load_q6k(blk, u); }
    static __device__ __forceinline__ void drain(const Raw& r) {
        asm volatile("" ::"v"(r.l[0]), "v"(r.l[4]), "v"(r.h[0]), "v"(r.h[4]), "v"(r.q[0]),
                     "v"(r.q[4]), "v"(r.s[0]), "v"(r.s[1]), "v"(r.s[2]), "v"(r.d));
    }
    template <bool SC, bool LOWREG = false>
    static __device__ __forceinline__ double term(const Raw& r, int u, const float4* xc,
                                                  const float* xs, int c, float, double) {
        return term_q6k_i8(r, u, reinterpret_cast<const uint32_t*>(xc), xs + 8 * c);
    }
};

template <> struct Chunk<T_Q4K> {
    using Raw = RawQ4;
    static __device__ __forceinline__ Raw load(wptr blk, int u) { return load_q4k(blk, u); }
    static __device__ __forceinline__ void drain(const Raw& r) {
        asm volatile("" ::"v"(r.hd.x), "v"(r.qa.x), "v"(r.qb.x));
    }
    template <bool SC, bool LOWREG = false>
    static __device__ __forceinline__ double term(const Raw& r, int u, const float4* xc,
                                                  const float* xs, int c, float f, double) {
        const float2 s = reinterpret_cast<const float2*>(xs)[c];
        return term_q4k<SC, LOWREG>(r, u, xc, s.x, s.y, f);
    }
};
template <> struct Chunk<T_Q6K> {
    using Raw = RawQ6;
    static __device__ __forceinline__ Raw load(wptr blk, int u) { return load_q6k(blk, u); }
    static __device__ __forceinline__ void drain(const Raw& r) {
        asm volatile("" ::"v"(r.l[0]), "v"(r.l[4]), "v"(r.h[0]), "v"(r.h[4]), "v"(r.q[0]),
                     "v"(r.q[4]), "v"(r.s[0]), "v"(r.s[1]), "v"(r.s[2]), "v"(r.d));
    }
    template <bool SC, bool LOWREG = false>
    static __device__ __forceinline__ double term(const Raw& r, int u, const float4* xc,
                                                  const float*, int, float, double f6) {
        return term_q6k<LOWREG>(r, u, xc, f6);
    }
};
template <> struct Chunk<T_Q2K> {
    using Raw = RawQ2;
    static __device__ __forceinline__ Raw load(wptr blk, int u) { return load_q2k(blk, u); }
    static __device__ __forceinline__ void drain(const Raw& r) {
        asm volatile("" ::"v"(r.q.x), "v"(r.s.x), "v"(r.dd));
    }
    template <bool SC, bool LOWREG = false>
    static __device__ __forceinline__ double term(const Raw& r, int u, const float4* xc,
                                                  const float* xs, int c, float f, double) {
        return term_q2k<SC, LOWREG>(r, u, xc, reinterpret_cast<const float4*>(xs)[c], f);
    }
};
template <> struct Chunk<T_Q5K> {
    using Raw = RawQ5;
    static __device__ __forceinline__ Raw load(wptr blk, int u) { return load_q5k(blk, u); }
    static __device__ __forceinline__ void drain(const Raw& r) {
        asm volatile("" ::"v"(r.hd.x), "v"(r.h0.x), "v"(r.h1.x), "v"(r.qa.x), "v"(r.qb.x));
    }
    template <bool SC, bool LOWREG = false>
    static __device__ __forceinline__ double term(const Raw& r, int u, const float4* xc,
                                                  const float* xs, int c, float f, double) {
        const float2 sx = reinterpret_cast<const float2*>(xs)[c];
        return term_q5k<SC>(r, u, xc, sx.x, sx.y, f);
    }
};
template <> struct Chunk<T_Q3K> {
    using Raw = RawQ3;
    static __device__ __forceinline__ Raw load(wptr blk, int u) { return load_q3k(blk, u); }
    static __device__ __forceinline__ void drain(const Raw& r) {
        asm volatile("" ::"v"(r.q[0]), "v"(r.q[4]), "v"(r.m[0]), "v"(r.m[4]), "v"(r.s[0]),
                     "v"(r.s[3]), "v"(r.d));
    }
    template <bool SC, bool LOWREG = false>
    static __device__ __forceinline__ double term(const Raw& r, int u, const float4* xc,
                                                  const float*, int, float, double f6) {
        return term_q3k(r, u, xc, 4.0 * f6);
    }
};
template <> struct Chunk<T_Q80> {
    using Raw = RawQ8;
    static __device__ __forceinline__ Raw load(wptr blk, int u) { return load_q80(blk, u); }
    static __device__ __forceinline__ void drain(const Raw& r) {
        asm volatile("" ::"v"(r.w[0]), "v"(r.w[12]), "v"(r.w[16]));
    }
    template <bool SC, bool LOWREG = false>
    static __device__ __forceinline__ double term(const Raw& r, int, const float4* xc,
                                                  const float*, int, float, double f6) {
        return term_q80(r, xc, 4.0 * f6);
    }
};
template <> struct Chunk<T_NIB> {
    using Raw = RawNB;
    static __device__ __forceinline__ Raw load(wptr blk, int u) { return load_nib(blk, u); }
    static __device__ __forceinline__ void drain(const Raw& r) {
        asm volatile("" ::"v"(r.qa.x), "v"(r.qb.x), "v"(r.s), "v"(r.dd));
    }
    template <bool SC, bool LOWREG = false>
    static __device__ __forceinline__ double term(const Raw& r, int, const float4* xc,
                                                  const float* xs, int c, float f, double) {
        return term_nib<SC, LOWREG>(r, xc, reinterpret_cast<const float4*>(xs)[c], f);
    }
};

// ------------------------------------------------------------- the GEMV
// One persistent launch runs a list of segments.  A segment is a tensor of
// N = ngroups * Ng rows of one type and row length K; rows of group g live
// at w[g] + row * row_bytes (separate weight bases: the MoE expert slices),
// and use the shared x or, when x_stride != 0, their own x at x + g *
// x_stride.  y and add are indexed by the segment row g * Ng + row.
//
// Workgroup b of G owns rows b, b + G, b + 2G, ... of every segment, so at
// any moment all workgroups stream neighbouring rows (DRAM locality).  Its
// R rows are R * NC chunks of 64 weights; the waves take batches of 64
// consecutive chunks (first batch static, then from an LDS counter: the
// issue arbiter favours old waves, and a static split would leave a long,
// poorly overlapped tail).  Each chunk's binary64 term goes to LDS; after
// a barrier, L lanes per row reduce that row's terms in a fixed order, so
// the result depends on nothing but the inputs.
//
// x is staged once per segment, or not at all when the segment uses the
// same x (same pointer, K and layout) as the previous one: the same-input
// groups (QKV, gate+up).
constexpr int MAXSEG = 8;
constexpr int MAXG = 16;
constexpr int LIST_MAX = 4;   // parts of a same-input group of any sizes

// A segment: N rows of one type and row length K, made of nparts parts.
// Part p holds rows [start[p], start[p+1]) at weight base w[p], writes
// y[p][row - start[p]] (plus add[p][...] when add[p] != nullptr) and reads
// x, or x + p * x_stride when x_stride != 0.  One part is a plain tensor;
// several parts are the matvecs of a same-input group (Q/K/V, gate/up)
// merged into one row space, or the selected experts of an MoE layer.
// The fields a segment needs first come first (one scalar load).
struct Seg {
    const float* x;
    // MoE gather (nullptr: unused): part p's weights are w[p] plus
    // sel[p % ksel] expert strides, the expert index read on the device
    // (clamped to [0, emax)).  Read with the leading fields: the part mode
    // depends on it.
    const int* sel;
    int type, K, N, nparts, x_stride;
    int pn;            // rows per part when every part has the same count, else 0
    uint32_t pn_m;     // magic multiplier for division by pn (0: pn <= 1)
    int pn_l;          // its shift
    uint32_t nc_m;     // the same for division by NC = K / 64
    int nc_l;
    // the fields the first weight address needs sit ahead of the pointer
    // tables, in the kernel's first round of scalar loads
    int start[LIST_MAX];
    long estride;      // MoE gather: bytes per expert,
    int ksel, emax;    // the selection period and the expert count
    const uint8_t* w[MAXG];
    float* y[MAXG];
    const float* add[MAXG];
    // routed in the launch (nullptr: sel is an input): every workgroup
    // takes the top-ksel of the emax router weights probs[] itself, and
    // workgroup 0 writes them to sel_out / selw_out
    const float* probs;
    int* sel_out;
    float* selw_out;
};

// Issues the scalar loads of a segment's leading fields together and waits
// for them once: used as they are needed, the fields would be fetched in
// several dependent round trips to the kernel-argument memory.  (The
// launch-wide fields are loaded in the same round by the kernel's entry.)
__device__ __forceinline__ void prefetch_seg(const Seg& S) {
    asm volatile("" ::"s"(S.x), "s"(S.sel), "s"(S.type), "s"(S.K), "s"(S.N), "s"(S.nparts),
                 "s"(S.x_stride), "s"(S.pn), "s"(S.pn_m), "s"(S.pn_l), "s"(S.nc_m), "s"(S.nc_l),
                 "s"(S.start[1]), "s"(S.start[2]), "s"(S.start[3]), "s"(S.w[0]), "s"(S.y[0]),
                 "s"(S.add[0]));
}

struct SegsArg {
    Seg s[MAXSEG];
    int nseg;
    int threads;       // blockDim.x and gridDim.x, passed as plain arguments:
    int grid;          // the built-ins are read through a dependent load chain
    uint32_t grid_m;   // magic multiplier and shift for division by grid
    int grid_l;
    int xs_off;        // LDS byte offsets of the xs, terms and scratch regions
    int terms_off;
    int scr_off;
    // MoE FFN step pieces folded into a one-segment MoE gather launch
    // (segment 0, selection kernels only; null / 0: unused), each instead
    // of writing y (see run_segment's epilogue):
    float* act;        // parts k gate then k up slices: act = SwiGLU(gate, up)
    float* cx;         // parts = ranks: cx += the rank-ordered weighted sum,
    const float* cw;   //   weights cw[part]
    int logits;        // the routing input holds router logits: softmax first
};

// n / d for the divisor encoded by (m, l): the invariant-integer division
// of Granlund and Montgomery (1994), valid for every 32-bit n.
__device__ __forceinline__ uint32_t div_magic(uint32_t n, uint32_t m, int l) {
    if (m == 0) return n;
    const uint32_t t = __umulhi(m, n);
    return (t + ((n - t) >> 1)) >> (l - 1);
}

// What the LDS x region currently holds: x (pointer, K, groups, the
// stride between the groups' x, layout),
// which type's per-group sums are in the xs region (0: none), the scale
// exponent of the staged values (0 or KSC) and whether some x fell outside
// the scaled-mode window.
struct Staged {
    const float* x;
    int K, layout, ngx, xst, sums, k;
    bool bad;
};

// LDS scratch: per-segment batch counters, per-wave flags, part tables,
// and the experts chosen when a segment is routed in the launch (kept here
// rather than beside the routing's work arrays in the terms region: the
// part tables read them after the routing's last barrier, and a segment
// that reuses the staged x has no barrier before its sweep writes terms)
constexpr int SCR_FLAGS = 4 * MAXSEG;
constexpr int SCR_TABS = SCR_FLAGS + 4 * 16;
constexpr int SCR_RSEL = SCR_TABS + 3 * 8 * MAXG;
constexpr int SCR_CMB = SCR_RSEL + 8 * MAXG;     // combine: weight per part (<0 skip flag)
constexpr int SCR_BYTES = SCR_CMB + 8 * MAXG;

// Part layout of a segment: one part; up to 4 parts of any sizes (a merged
// same-input group: the part of a row by comparing with the part starts,
// its base by selection); or up to 16 equal parts (MoE experts: the part of
// a row by division, its base from an LDS table).
// PM_SEL: PM_EQUAL whose part bases are moved by a device-side expert
// selection (the MoE gather kernels only).
constexpr int PM_ONE = 0, PM_LIST = 1, PM_EQUAL = 2, PM_SEL = 3;

template <typename V>
__device__ __forceinline__ V pick4(uint32_t g, V v0, V v1, V v2, V v3) {
    return g == 0 ? v0 : g == 1 ? v1 : g == 2 ? v2 : v3;
}

// Part g and part-local row rg of segment row r.
template <int PM>
__device__ __forceinline__ uint32_t part_of(const Seg& S, uint32_t r, uint32_t& rg) {
    if (PM == PM_ONE) {
        rg = r;
        return 0;
    }
    uint32_t g;
    if (PM >= PM_EQUAL) {
        g = div_magic(r, S.pn_m, S.pn_l);
        rg = r - __umul24(g, (uint32_t)S.pn);   // g <= 16, rows < 2^24
        return g;
    }
    g = 0;
#pragma unroll
    for (int i = 1; i < LIST_MAX; i++) g += (i < S.nparts && r >= (uint32_t)S.start[i]) ? 1u : 0u;
    rg = r - (uint32_t)pick4(g, S.start[0], S.start[1], S.start[2], S.start[3]);
    return g;
}

// weight base of part g (the LDS table holds the PM_EQUAL bases)
template <int PM>
__device__ __forceinline__ const uint8_t* part_w(const Seg& S, uint32_t g,
                                                 const uint8_t* const* wtab) {
    if (PM == PM_ONE) return S.w[0];
    if (PM == PM_LIST) return pick4(g, S.w[0], S.w[1], S.w[2], S.w[3]);
    return wtab[g];
}

// Where chunk f = base + lane of a workgroup's range lives: its staged-x
// chunk cx and weight address (past the last chunk, the row is clamped to
// the last row: an in-bounds load whose term is never stored).  Branch-free,
// so the loads that follow are unconditional and the compiler can count the
// outstanding ones exactly.
//
// base is the same in every lane of a wave, so its row and column are
// scalar work; a lane adds its fixed offset (lane / NC rows, lane % NC
// columns, set once per segment) with one carry.  Rows, row bytes and
// chunk counts stay below 2^24 (the host rejects larger segments), so every
// product is a full-rate 24-bit multiply rather than a 32-bit one.
template <int TYPE, int PM>
struct Walk {
    const Seg* S;
    const uint8_t* const* wtab;
    int NC, b, G, lane;
    uint32_t rbytes;
    uint32_t lq, lr;      // lane / NC, lane % NC
    uint32_t rho_max;     // the workgroup's last row (R - 1)

    __device__ __forceinline__ wptr locate(int base, int& cx) const {
        const uint32_t ub = (uint32_t)__builtin_amdgcn_readfirstlane(base);
        const uint32_t rho0 = div_magic(ub, S->nc_m, S->nc_l);
        const uint32_t c0 = ub - rho0 * (uint32_t)NC;
        uint32_t c = c0 + lr, rho = rho0 + lq;
        if (c >= (uint32_t)NC) {
            c -= (uint32_t)NC;
            rho += 1u;
        }
        rho = min(rho, rho_max);
        __builtin_assume(rho < (1u << 24));
        const uint32_t r = (uint32_t)b + __umul24((uint32_t)G, rho);
        uint32_t rg;
        const uint32_t g = part_of<PM>(*S, r, rg);
        __builtin_assume(rg < (1u << 24));
        __builtin_assume(rbytes < (1u << 24));
        __builtin_assume(c < (1u << 24));
        cx = (PM != PM_ONE && S->x_stride ? (int)__umul24(g, (uint32_t)NC) : 0) + (int)c;
        return to_global(part_w<PM>(*S, g, wtab)) + (uint64_t)rg * rbytes +
               __umul24(c >> 2, (uint32_t)TypeInfo<TYPE>::BB);
    }
};

// The batch loop.  Each wave keeps DEPTH batches in flight: a computed
// batch's registers are refilled at once with the next batch from the
// counter.  Batches are handed out in increasing order, so base[0] <
// base[1] < ...; the first DEPTH batches are static (set by the caller).
template <int TYPE, int DEPTH, int PM, bool SC>
__device__ __forceinline__ void sweep(const Walk<TYPE, PM>& W, int nch, int u, int* next,
                                      const float4* xl, const float* xs, double* terms, float f,
                                      double f6, int* base, int* cx,
                                      typename Chunk<TYPE>::Raw* buf) {
    using C = Chunk<TYPE>;
    while (base[0] < nch) {
#pragma unroll
        for (int k = 0; k < DEPTH; k++) {
            int nb = 0;
            if (W.lane == 0) nb = atomicAdd(next, 64);
            if (base[k] < nch) {                 // uniform over the wave
                const int fi = base[k] + W.lane;
                __builtin_assume(cx[k] >= 0 && cx[k] < (1 << 24));   // 24-bit multiply
                const double t = C::template term<SC>(buf[k], u,
                                                      xl + cx[k] * XGroup<TYPE>::XSTRIDE, xs,
                                                      cx[k], f, f6);
                if (fi < nch) terms[fi] = t;
            }
            base[k] = __builtin_amdgcn_readfirstlane(nb);
            buf[k] = C::load(W.locate(base[k], cx[k]), u);
        }
    }
    // the last refill is past the end: wait for it here, so no load is
    // outstanding into the next segment (the compiler would otherwise wait
    // for all loads where the next segment reuses the registers, including
    // that segment's x loads)
#pragma unroll
    for (int k = 0; k < DEPTH; k++) C::drain(buf[k]);
}

// A workgroup barrier for LDS traffic only: waits for this wave's LDS
// operations (lgkmcnt), not for its global loads (vmcnt), which
// __syncthreads() would also wait for.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0); vmcnt, expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Top-k of one token's router weights, E <= 1024, computed by the whole
// workgroup (T lanes) with the rule of kq_moe_topk_rank_kernel: slot r of
// rsel gets the expert with r eligible experts beating it (a larger weight,
// or an equal weight and a lower id; weights <= -1 and NaN are not
// eligible); slots without an expert stay -1.  Lane (p, e) counts the
// experts of part p (of P) that beat e.  pv holds w[tid] (lanes tid < E64,
// -1 past E), loaded by the caller ahead of its other loads; where E64 > T
// the lanes load the rest here.  Work arrays: ROUTE_BYTES of LDS at
// work, free again on return; the result goes to rsel / rselw (MAXG
// entries each, elsewhere in LDS).  Only LDS barriers: global loads the
// caller issued stay in flight.
constexpr int ROUTE_BYTES = 1024 * 4 + 1024 * 4;
__device__ void wg_topk(const float* w, float pv, int E, int k, int T, uint8_t* work,
                        int* rsel, float* rselw) {
    float* wl = reinterpret_cast<float*>(work);
    int* part = reinterpret_cast<int*>(work + 4096);
    const int tid = threadIdx.x, E64 = (E + 63) & ~63;
    int P = 1;
    while (2 * P * E64 <= T && (E64 / (2 * P)) % 4 == 0) P *= 2;
    const int L = E64 / P;
    if (tid < E64) wl[tid] = pv;
    if (E64 > T)                          // uniform: its wait covers every load in flight
        for (int i = tid + T; i < E64; i += T) wl[i] = i < E ? w[i] : -1.0f;
    if (tid < MAXG) { rsel[tid] = -1; rselw[tid] = -1.0f; }
    lds_barrier();
    for (int idx = tid; idx < P * E64; idx += T) {
        const int e = idx % E64, p = idx / E64;
        const float v = wl[e];
        int r = 0;
        for (int q = p * L; q < (p + 1) * L; q += 4) {
            const float4 o = *reinterpret_cast<const float4*>(&wl[q]);
            const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float x = ov[j];
                const int beat = (x > v) | ((x == v) & (q + j < e));
                r += (x > -1.0f) & beat;
            }
        }
        part[idx] = r;
    }
    lds_barrier();
    for (int e = tid; e < E; e += T) {
        int rank = 0;
        for (int i = 0; i < P; i++) rank += part[i * E64 + e];
        const float v = wl[e];
        if (v > -1.0f && rank < k) { rsel[rank] = e; rselw[rank] = v; }
    }
    lds_barrier();
}

// Softmax of one token's E <= T router logits, computed by the whole
// workgroup with kq_softmax_kernel's arithmetic (stratum_engine.h:395-423):
// the NaN-ignoring maximum (NaN when logit 0 is NaN), expf(v - max), their
// binary64 sum in index order by one lane, inv = (float)(1 / sum), p = e *
// inv.  v: lane tid's logit (tid < E); returns its probability, -1 past E.
// Work: E + 17 floats of LDS at sm, free again on return.
__device__ float wg_softmax(float v, int E, int T, float* sm) {
    const int tid = threadIdx.x;
    float* wm = sm + 1024;                     // per-wave maxima, then inv
    float m = tid < E ? v : -INFINITY;
    if (tid < E) sm[tid] = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((tid & 63) == 0) wm[tid >> 6] = m;
    lds_barrier();
    float maxv = wm[0];
    for (int w = 1; w < (T >> 6); w++) maxv = fmaxf(maxv, wm[w]);
    if (isnan(sm[0])) maxv = sm[0];
    lds_barrier();
    const float e = tid < E ? expf(v - maxv) : 0.0f;
    if (tid < E) sm[tid] = e;
    lds_barrier();
    if (tid == 0) {                            // 16 values per LDS round trip
        double sum = 0.0;
        int i = 0;
        for (; i + 16 <= E; i += 16) {
            float4 q[4];
#pragma unroll
            for (int j = 0; j < 4; j++) q[j] = *reinterpret_cast<const float4*>(sm + i + 4 * j);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                sum = sum + (double)q[j].x; sum = sum + (double)q[j].y;
                sum = sum + (double)q[j].z; sum = sum + (double)q[j].w;
            }
        }
        for (; i < E; i++) sum = sum + (double)sm[i];
        wm[16] = (float)(1.0 / sum);
    }
    lds_barrier();
    const float pr = e * wm[16];
    lds_barrier();                             // sm is the caller's again
    return tid < E ? pr : -1.0f;
}

template <int TYPE, int DEPTH, int PM>
__device__ void run_segment(const Seg& S, const SegsArg& A, int seg, Staged& st, uint8_t* smem,
                            bool last_seg) {
    using TI = TypeInfo<TYPE>;
    using C = Chunk<TYPE>;
    const int tid = threadIdx.x, T = A.threads, lane = tid & 63, wave = tid >> 6;
    const int G = A.grid;
    // logical workgroup index, XCD-major (dispatch is round robin over the 8
    // XCDs, each with its own L2): neighbouring rows, which share the cache
    // line at their boundary, are then read on one XCD
    const int b = (G & 7) ? (int)blockIdx.x
                          : (int)(blockIdx.x & 7) * (G >> 3) + (int)(blockIdx.x >> 3);
    const int K = S.K, NC = K >> 6, N = S.N;
    const int R = N > b ? (int)div_magic((uint32_t)(N - b + G - 1), A.grid_m, A.grid_l) : 0;
    if (R == 0) return;                       // uniform over the workgroup
    const int nch = R * NC;
    const int u = tid & 3;
    const uint32_t rbytes = (uint32_t)(K >> 8) * TI::BB;
    float4* xl = reinterpret_cast<float4*>(smem);
    float* xs = reinterpret_cast<float*>(smem + A.xs_off);
    double* terms = reinterpret_cast<double*>(smem + A.terms_off);
    int* next = reinterpret_cast<int*>(smem + A.scr_off) + seg;
    int* flags = reinterpret_cast<int*>(smem + A.scr_off + SCR_FLAGS);
    const uint8_t** wtab = reinterpret_cast<const uint8_t**>(smem + A.scr_off + SCR_TABS);
    float** ytab = reinterpret_cast<float**>(smem + A.scr_off + SCR_TABS + 8 * MAXG);
    const float** atab = reinterpret_cast<const float**>(smem + A.scr_off + SCR_TABS + 16 * MAXG);
    const int ngx = (PM != PM_ONE && S.x_stride) ? S.nparts : 1;

    // x staging decision: SC types stage x scaled, Q6_K unscaled; a Q6_K
    // segment can read a scaled x, an SC type restages an unscaled one
    // unless the window already failed for it.
    constexpr bool SCTYPE = TI::SCALED;
    const int xst = ngx > 1 ? S.x_stride : 0;
    // x layouts: 0 strided fp32, 1 linear fp32, 2 / 3 int8 per 32 / per 16
    // (the int8 layouts: 2 linear chunks per 32, 3 strided per 16, 4 strided per 32)
    constexpr int LAYOUT = !XGroup<TYPE>::I8 ? (int)TI::LINEAR
                         : TYPE == T_Q6K_I8 ? 3 : TYPE == T_Q3K_I8 ? 4 : 2;
    // the MoE FFN step pieces of a one-segment gather launch (segment 0)
    const bool cmb = PM == PM_SEL && seg == 0 && A.cx != nullptr;   // uniform
    const bool swe = PM == PM_SEL && seg == 0 && A.act != nullptr;  // uniform
    const bool same_x = st.x == S.x && st.K == K && st.layout == LAYOUT && st.ngx == ngx &&
                        st.xst == xst;
    const bool restage = !same_x || (SCTYPE && st.k == 0 && !st.bad);
    constexpr int G4 = XGroup<TYPE>::G4;
    const XStage<TYPE> xg = {S.x, S.x_stride, K / (4 * G4), ngx * (K / (4 * G4)), NC};
    // routed in the launch: the router weights go out first, so the routing
    // can wait for them while the x loads behind them are still in flight
    const bool route = PM == PM_SEL && S.probs;   // uniform
    float pv = -1.0f;
    if (PM == PM_SEL && route && tid < S.emax) pv = S.probs[tid];
    // equal parts: lane g reads part g's pointers itself (vector loads from
    // the argument block, issued at once and ahead of x, rather than a
    // second round of scalar loads of all 48 pointers)
    const int gl = lane & (MAXG - 1);
    const uint8_t* wv = nullptr;
    float* yv = nullptr;
    const float* av = nullptr;
    if (PM >= PM_EQUAL) {
        wv = S.w[gl];
        yv = S.y[gl];
        av = S.add[gl];
    }
    // combine: part lane's weight, and the residual of output row b + tid G
    // for the first pn / G lanes, loaded now so the epilogue waits for none
    float cwl = 0.0f, cres = 0.0f;
    if (PM == PM_SEL && cmb) {
        if (lane < S.nparts) cwl = A.cw[lane];
        if (tid < S.pn / G) cres = A.cx[b + tid * G];
    }
    f32x4 xv[G4];
    // first round of x, ahead of the weights (and of the routing, which
    // does not depend on it)
    // (only the lanes that own a group: the clamped loads of the others
    // would queue ahead of the weights in the address units, e.g. 864 of
    // 1024 lanes at Q4_K, K = 5120; measured over lane- and wave-granular
    // guards, the lane form gave the best layer set: 63.2 -> 62.1 us)
    if (restage && tid < xg.total) xg.load(tid, xv);
    // A second round (x longer than one round of the workgroup, e.g. Q6_K
    // at K = 17408 with 1024 lanes) is loaded together with the first, so
    // its latency is not paid after the first round's stores.  Types with
    // 16-float groups only: their registers allow it (Q4_K needs a second
    // round only beyond K = 32768).
    constexpr bool PRE2 = G4 == 4;
    const bool two = PRE2 && restage && xg.total > T;   // uniform
    f32x4 xv2[PRE2 ? G4 : 1];
    if (PRE2 && two && tid + T < xg.total) xg.load(tid + T, xv2);

    const int* rsel = nullptr;
    if (PM == PM_SEL && route) {
        // work arrays in the terms region (written only by the sweep, after
        // the routing's last barrier); the result in the scratch region
        int* rs = reinterpret_cast<int*>(smem + A.scr_off + SCR_RSEL);
        float* rw = reinterpret_cast<float*>(rs + MAXG);
        // router logits: their softmax first (the host allows it for emax <= 256,
        // so wg_topk reads no weight beyond its lanes' pv)
        if (A.logits) pv = wg_softmax(pv, S.emax, T, reinterpret_cast<float*>(smem + A.terms_off));
        wg_topk(S.probs, pv, S.emax, S.ksel, T, smem + A.terms_off, rs, rw);
        rsel = rs;
        if (b == 0 && tid < S.ksel) {
            S.sel_out[tid] = rs[tid];
            S.selw_out[tid] = rw[tid];
        }
    }
    if (PM >= PM_EQUAL) {
        // each wave writes the part tables itself (identical values), so its
        // own reads need no barrier
        if (lane < S.nparts) {
            int se = 0;
            if (PM == PM_SEL) {                   // the expert chosen on the device
                se = rsel ? rsel[lane % S.ksel] : S.sel[lane % S.ksel];
                const int e = min(max(se, 0), S.emax - 1);
                wv += (size_t)e * S.estride;
            }
            wtab[lane] = wv;
            ytab[lane] = yv;
            atab[lane] = av;
            if (PM == PM_SEL && cmb) {       // the combine's weight and skip flag (empty slot)
                reinterpret_cast<float*>(smem + A.scr_off + SCR_CMB)[lane] = cwl;
                reinterpret_cast<int*>(smem + A.scr_off + SCR_CMB + 4 * MAXG)[lane] = se < 0;
            }
        }
    }
    const uint32_t lq = div_magic((uint32_t)lane, S.nc_m, S.nc_l);
    const Walk<TYPE, PM> W = {&S, wtab, NC, b, G, lane, rbytes,
                              lq, (uint32_t)lane - lq * (uint32_t)NC, (uint32_t)(R - 1)};


    // first DEPTH batches: static (wave w takes chunks 64w .., then
    // 64(W + w) ..).  A segment that stages x issues them once its x has
    // arrived (the wait below, after the first x stores are computed): all
    // 256 workgroups' first batches together are about 13 MB, and issued
    // ahead of the x arrival they queue in front of it in the memory system
    // (x staged about 2 us after issue).  Measured on the 27B layer set in
    // one process, against issuing them before the staging: 58.22 -> 57.07
    // us ([down] 18.56 -> 18.09, [Q,K,V] 8.59 -> 8.45 us).
    int base[DEPTH], cx[DEPTH];
    typename C::Raw buf[DEPTH];
    auto first_batches = [&]() {
        if (restage) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
        for (int k = 0; k < DEPTH; k++) {
            base[k] = (k * (T >> 6) + wave) * 64;
            buf[k] = C::load(W.locate(base[k], cx[k]), u);
        }
    };
    if (!restage) first_batches();

    if (XGroup<TYPE>::I8 && restage) {
        uint8_t* xq = reinterpret_cast<uint8_t*>(xl);
        const int per = xg.per;
        if (tid < xg.total) store_i8<TYPE>(tid, per, NC, xv, xq, xs);
        first_batches();
        int gi0 = tid + T;
        if (PRE2 && two) {
            if (gi0 < xg.total) store_i8<TYPE>(gi0, per, NC, xv2, xq, xs);
            gi0 += T;
        }
        for (int gi = gi0; gi < xg.total; gi += T) {
            xg.load(gi, xv);
            store_i8<TYPE>(gi, per, NC, xv, xq, xs);
        }
        __syncthreads();
        st.x = S.x; st.K = K; st.layout = LAYOUT; st.ngx = ngx; st.xst = xst;
        st.sums = TYPE;
        st.k = 0;
        st.bad = false;
    } else if (restage) {
        bool bad = xg.store(tid, xv, SCTYPE, true, xl, xs);
        first_batches();
        int gi0 = tid + T;
        if (PRE2 && two) {
            bad |= xg.store(gi0, xv2, SCTYPE, true, xl, xs);
            gi0 += T;
        }
        for (int gi = gi0; gi < xg.total; gi += T) {
            xg.load(gi, xv);
            bad |= xg.store(gi, xv, SCTYPE, true, xl, xs);
        }
        const bool wave_bad = __ballot(bad) != 0ull;   // with every lane active
        if (lane == 0) flags[wave] = wave_bad;
        __syncthreads();
        int any = 0;
        for (int i = 0; i < (T >> 6); i++) any |= flags[i];
        st.x = S.x; st.K = K; st.layout = LAYOUT; st.ngx = ngx; st.xst = xst;
        st.sums = TI::XS_PER_CHUNK ? TYPE : 0;
        st.k = SCTYPE ? KSC : 0;
        st.bad = SCTYPE && any;
        if (st.bad) {                         // the same in every workgroup
            for (int gi = tid; gi < xg.total; gi += T) {
                xg.load(gi, xv);
                xg.store(gi, xv, false, false, xl, xs);
            }
            __syncthreads();
            st.k = 0;
        }
    } else if (!XGroup<TYPE>::I8 && TI::XS_PER_CHUNK && st.sums != TYPE) {   // sums per type
        resum<TYPE>(K, ngx, tid, T, xl, xs, st.k);
        __syncthreads();
        st.sums = TYPE;
    }
    const float f = st.k ? ldexpf(1.0f, 149 - st.k) : 1.0f;
    const double f6 = ldexp(0.25, -st.k);

    if (SCTYPE && st.k > 0)
        sweep<TYPE, DEPTH, PM, true>(W, nch, u, next, xl, xs, terms, f, f6, base, cx, buf);
    else
        sweep<TYPE, DEPTH, PM, false>(W, nch, u, next, xl, xs, terms, f, f6, base, cx, buf);
    __syncthreads();

    // Row reduction, in one fixed order that depends on NC only (so the
    // result does not depend on the grid, the workgroup size or how rows
    // are batched, and the multi-x kernel reproduces it): GP = kq_phases(NC)
    // lanes per row, lane p sums the terms of chunks p, p+GP, ... in
    // increasing order (binary64, from 0), then phase_tree.  GP divides 64
    // and R * GP is a multiple of GP, so each lane group is entirely active.
    const int GP = kq_phases(NC), lgp = GP == 32 ? 5 : 3;
    for (int task = tid; task < R * GP; task += T) {
        const int rho = task >> lgp, p = task & (GP - 1);
        const double* tr = terms + rho * NC;
        // four terms are read ahead of their additions (one LDS round trip
        // per four adds, not per add); the adds stay in order
        double s = 0.0;
        int i = p;
        for (; i + 3 * GP < NC; i += 4 * GP) {
            const double t0 = tr[i], t1 = tr[i + GP], t2 = tr[i + 2 * GP], t3 = tr[i + 3 * GP];
            s = s + t0;
            s = s + t1;
            s = s + t2;
            s = s + t3;
        }
        for (; i < NC; i += GP) s = s + tr[i];
        s = phase_tree(s, GP);
        if (p == 0) {
            uint32_t rg;
            const uint32_t g = part_of<PM>(S, (uint32_t)(b + G * rho), rg);
            float* y;
            const float* add;
            if (PM == PM_ONE) {
                y = S.y[0];
                add = S.add[0];
            } else if (PM == PM_LIST) {
                y = pick4(g, S.y[0], S.y[1], S.y[2], S.y[3]);
                add = pick4(g, S.add[0], S.add[1], S.add[2], S.add[3]);
            } else {
                y = ytab[g];
                add = atab[g];
            }
            float v = (float)s;
            if (add) v = add[rg] + v;
            if (PM == PM_SEL && (cmb || swe))
                reinterpret_cast<float*>(smem)[rho] = v;   // the x region is free now
            else
                y[rg] = v;
        }
    }
    if (PM == PM_SEL && swe) {
        // SwiGLU of one token's selections (stratum_engine.h:373-392, as
        // kq_swiglu_kernel): parts 0..k-1 are the k ranks' gate slices,
        // k..2k-1 their up slices; with the rows per part a multiple of G
        // (the host checks) the workgroup holds rank r's gate and up row
        // i = b + jG as its rows r * m + j and (k + r) * m + j.
        __syncthreads();
        const float* ov = reinterpret_cast<const float*>(smem);
        const int m = S.pn / G, kr = S.nparts >> 1;
        for (int t = tid; t < kr * m; t += T) {
            const int r = t / m, j = t - r * m;
            A.act[(size_t)r * S.pn + b + j * G] = swiglu1(ov[r * m + j], ov[(kr + r) * m + j]);
        }
    }
    if (PM == PM_SEL && cmb) {
        // The weighted accumulate in rank order plus the residual
        // (stratum_arch_moe.inc.c:728-743; kq_moe_combine_kernel's
        // arithmetic): part r is rank r of one token, and with the rows per
        // part a multiple of G (the host checks) the workgroup holds every
        // part's row i = b + jG as its row r * (pn / G) + j.
        __syncthreads();
        const float* ov = reinterpret_cast<const float*>(smem);
        const float* cwt = reinterpret_cast<const float*>(smem + A.scr_off + SCR_CMB);
        const int* skip = reinterpret_cast<const int*>(smem + A.scr_off + SCR_CMB + 4 * MAXG);
        const int m = S.pn / G;                  // <= T (the host checks)
        if (tid < m) {
            float acc = 0.0f;
            for (int r = 0; r < S.nparts; r++) {
                if (skip[r]) continue;
                acc = acc + cwt[r] * ov[r * m + tid];
            }
            A.cx[b + tid * G] = cres + acc;
        }
    }
    if (last_seg) return;
    // Before the next segment: wait for the y stores here (a store keeps its
    // data registers busy until it completes, and the next segment's first
    // writes to those registers would otherwise wait for every outstanding
    // load -- its x), and let every wave finish with the LDS.
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
    __syncthreads();
}

// TYPES is a bit set of the types the launch contains (bit 0 Q4_K, 1 Q6_K,
// 2 Q2_K, 3 type 42, 5 Q5_K, 6 Q3_K, 7 Q8_0): the host launches the
// instantiation with only the types present, so a single-type launch
// carries one type's code and the register allocation is not constrained
// by the others.  Launches that mix Q4_K and Q6_K run the TB_Q46 kernel;
// the host gives every other type launches of its own.  (One kernel for all
// four core types took 4 KB of scratch per lane and ran a Q4_K+Q6_K list
// 16 times slower than the two single-type launches.)
constexpr int TB_Q4K = 1, TB_Q6K = 2, TB_Q2K = 4, TB_NIB = 8, TB_Q46 = TB_Q4K | TB_Q6K;
constexpr int TB_Q5K = 32, TB_Q3K = 64, TB_Q80 = 128, TB_Q4K_I8 = 256, TB_Q6K_I8 = 512;
constexpr int TB_Q5K_I8 = 1024, TB_Q3K_I8 = 2048, TB_Q80_I8 = 4096;
// Q4_K and Q6_K in the int8 mode mixed in one launch (st_mixed_fused_sdot,
// stratum_linear.h:1043-1085: one dispatch for a group whose tensors have
// either type, e.g. Q, K, V with a Q6_K V)
constexpr int TB_I8MIX = TB_Q4K_I8 | TB_Q6K_I8;
// TB_SEL: the MoE gather instantiations (every segment has a selection)
constexpr int TB_SEL = 16;

// MULTI = false: the launch has exactly one segment (no segment loop, so
// no state flows between segments and the compiler's wait analysis stays
// exact; most launches are this).
template <int DEPTH, int TYPES, bool MULTI>
__global__ __launch_bounds__(1024) void kq_segs_kernel(SegsArg A) {
    extern __shared__ __align__(16) uint8_t smem[];
    // one round of scalar loads for the launch-wide and first-segment fields
    // (two asm statements would wait between them)
    {
        const Seg& S = A.s[0];
        asm volatile("" ::"s"(A.nseg), "s"(A.threads), "s"(A.grid), "s"(A.grid_m),
                     "s"(A.grid_l), "s"(A.xs_off), "s"(A.terms_off), "s"(A.scr_off), "s"(S.x),
                     "s"(S.sel), "s"(S.type), "s"(S.K), "s"(S.N), "s"(S.nparts), "s"(S.x_stride),
                     "s"(S.pn), "s"(S.pn_m), "s"(S.pn_l), "s"(S.nc_m), "s"(S.nc_l),
                     "s"(S.start[1]), "s"(S.start[2]), "s"(S.start[3]), "s"(S.w[0]),
                     "s"(S.y[0]), "s"(S.add[0]));
    }
    const int nseg = MULTI ? A.nseg : 1;
    // batch counters of every segment (the first segment that runs stages
    // x, and its barrier orders these writes before any batch is taken)
    if (threadIdx.x < (unsigned)nseg)
        reinterpret_cast<int*>(smem + A.scr_off)[threadIdx.x] = 64 * DEPTH * (A.threads >> 6);
    Staged st = {nullptr, 0, -1, 0, 0, 0, 0, false};
    // a single-type instantiation does not read the segment types (the host
    // launches it only for segment lists of that type)
    constexpr bool SELK = (TYPES & TB_SEL) != 0;    // MoE gather: every segment has sel
    constexpr int TYB = TYPES & ~TB_SEL;
    constexpr bool SINGLE = TYB == TB_Q4K || TYB == TB_Q6K || TYB == TB_Q2K || TYB == TB_NIB ||
                            TYB == TB_Q5K || TYB == TB_Q3K || TYB == TB_Q80 ||
                            TYB == TB_Q4K_I8 || TYB == TB_Q6K_I8 || TYB == TB_Q5K_I8 ||
                            TYB == TB_Q3K_I8 || TYB == TB_Q80_I8;
    for (int i = 0; i < nseg; i++) {
        const Seg& S = A.s[i];
        if (i) prefetch_seg(S);
        const int pm = S.nparts == 1 ? PM_ONE : S.nparts <= LIST_MAX ? PM_LIST : PM_EQUAL;
        const bool last = i == nseg - 1;
#define KQ_RUN(T_)                                                                   \
        if (SELK) run_segment<T_, DEPTH, PM_SEL>(S, A, i, st, smem, last);           \
        else if (pm == PM_ONE) run_segment<T_, DEPTH, PM_ONE>(S, A, i, st, smem, last); \
        else if (pm == PM_LIST) run_segment<T_, DEPTH, PM_LIST>(S, A, i, st, smem, last); \
        else run_segment<T_, DEPTH, PM_EQUAL>(S, A, i, st, smem, last);
        if (SINGLE) {
            constexpr int TY = TYB == TB_Q4K ? T_Q4K : TYB == TB_Q6K ? T_Q6K
                             : TYB == TB_Q2K ? T_Q2K : TYB == TB_NIB ? T_NIB
                             : TYB == TB_Q5K ? T_Q5K : TYB == TB_Q3K ? T_Q3K
                             : TYB == TB_Q80 ? T_Q80 : TYB == TB_Q4K_I8 ? T_Q4K_I8
                             : TYB == TB_Q6K_I8 ? T_Q6K_I8 : TYB == TB_Q5K_I8 ? T_Q5K_I8
                             : TYB == TB_Q3K_I8 ? T_Q3K_I8 : T_Q80_I8;
            KQ_RUN(TY)
        } else {
            switch (S.type) {
            case T_Q4K: if (TYPES & TB_Q4K) { KQ_RUN(T_Q4K) } break;
            case T_Q6K: if (TYPES & TB_Q6K) { KQ_RUN(T_Q6K) } break;
            case T_Q4K_I8: if (TYB == TB_I8MIX) { KQ_RUN(T_Q4K_I8) } break;
            case T_Q6K_I8: if (TYB == TB_I8MIX) { KQ_RUN(T_Q6K_I8) } break;
            default: break;
            }
        }
#undef KQ_RUN
        // leave straight from the last segment: its y stores may still be
        // in flight, and only the other paths return to the loop head
        if (last) break;
    }
}

// ------------------------------------------------------------- multi-x
// y_j = W_g . x_j for the members j of each group g, with one pass over the
// group's weight rows: STRATUM_MULTISEQ (one group, B members) and the MoE
// gather (one group per selected expert, its routed tokens as members).
// Each member's result is bit-identical to the single-stream kernel's for
// the same row and x: the same chunk terms (same arithmetic, same x scaling
// rule) and the same reduction (GP = kq_phases(K/64) partial sums over
// chunks p, p+GP, ... in order, combined by phase_tree).
//
// Work.  A group's rows are cut into items of RB rows; workgroup b takes
// items b, b+G, ...  Within an item a task is (group of 64/GP rows,
// subgroup of S members): a wave's 64 lanes are the rows x GP chunk phases
// (lane p takes chunks p, p+GP, ... of its row, like the single-stream
// reduction), and each weight load serves the S members.  Tasks go
// round-robin over the waves (task t to wave t % W, at most MX_TW per
// wave), so the four SIMDs of a CU carry equal task counts whatever the row
// count.  Per wave the (step, task) sequence runs with the next unit's
// weights in flight.
// x.  The members' x is staged in LDS in the single-stream kernel's
// chunk-major layout, whole when it fits, else in double-buffered tiles of
// TC chunks (a multiple of GP) staged while the previous tile is consumed.
// A prologue pass over x gives the per-sub-block sums (min terms) and the
// scaled-mode window vote.  Members are staged mch (<= MX_MC) at a time;
// each such member chunk is one more pass over the item's rows (from L2).
constexpr int MX_MAXM = 64;   // members per group
constexpr int MX_MC = 16;     // members staged together, at most
constexpr int MX_TW = 4;      // tasks per wave, at most

struct MxGroup {
    const uint8_t* w;         // row r at w + r * row_bytes
    float* y;                 // member j writes y + yi[j] * y_stride
    int M;                    // members, 1..MX_MAXM
    int pad_;
    int xi[MX_MAXM];          // member j reads x = X + xi[j] * x_stride
    int yi[MX_MAXM];
};

struct MxArg {
    const uint8_t* w;         // inline group (gdev == nullptr): weights and
    int M;                    // members j = 0..M-1 (xi = yi = j)
    int N, K;
    const MxGroup* gdev;      // else groups in device memory, *ngdev of them
    const int* ngdev;
    const float* X;
    float* Y;
    long x_stride, y_stride;  // floats
    int RB, nblk;             // rows per item, items per group
    int threads, grid;
    int mch;                  // members staged together
    int TC;                   // chunks per x tile; >= K/64: x staged whole
    int sums_bytes;           // LDS bytes of the sums of mch members
    int xt_bytes;             // LDS bytes of one x buffer
    // MoE batch grouped in the launch (sel != nullptr): every workgroup
    // builds the expert runs of the selection itself (MoeRuns), in LDS at
    // byte offset grp_off, instead of reading groups made by a separate
    // launch.  Group g = t * nd + run, as kq_moe_group_kernel numbers them.
    const int* sel;
    int nm, E, nt, x_div, grp_off;
    const uint8_t* wt[2];
    float* yt[2];
    long estride;
    // routed in the launch (probs != nullptr, sel unused): every workgroup
    // also takes the top-k of each token's router weights probs[B][E] (the
    // rule of kq_moe_topk_rank_kernel), and workgroup 0 writes them to
    // sel_out / selw_out
    const float* probs;
    int B, k;
    int* sel_out;
    float* selw_out;
    // the runs as built (cnt, gid, ms, pl, rexp; [0] the run count):
    // runs_out != nullptr: workgroup 0 stores them; runs_in != nullptr:
    // every workgroup loads them instead of building (a later launch of the
    // same selection, E, nm and run length)
    int* runs_out;
    const int* runs_in;
};

// LDS slot of the float4 at tile-relative x position pos (a multiple of 4;
// tiles start on super-block boundaries)
template <bool LINEAR>
__device__ __forceinline__ int tile_slot(int pos) {
    if (LINEAR) return (pos >> 6) * XPAD + ((pos >> 2) & 15);
    const int bi = pos >> 8, pp = pos & 255;
    const int h = pp >> 7, t = (pp >> 5) & 3, is = (pp >> 4) & 1, qq = (pp >> 2) & 3;
    return (4 * bi + 2 * h + is) * XPAD + 4 * t + qq;
}

// One wave's tasks (wave-uniform: scalar registers).  Task k covers rows
// r0 + RPT grp[k] .. + RPT-1 (the lane's row: lane >> lgp) and members
// sg[k]*S .. +S-1.
struct MxTasks {
    int grp[MX_TW];
    int sg[MX_TW];
    int ntw;                  // tasks of this wave
    int r0, rows;             // the item's rows
    int GP, lgp, RPT;         // phases, log2, rows per task
};

// The step/task sweep of one member chunk: tiles, steps, tasks.  SC: x is
// staged scaled (byte-select products); else unscaled (exact convert path).
template <int TYPE, int S, bool WHOLE, bool SC>
__device__ __forceinline__ void mx_sweep(const MxArg& A, const MxTasks& tk, wptr gw,
                                         double (&part)[MX_TW][S], int MC, int mc0,
                                         const int* d_xi, const float* sums, float4* xb0,
                                         float4* xb1, int TC, int ntile,
                                         typename Chunk<TYPE>::Raw first) {
    using TI = TypeInfo<TYPE>;
    using C = Chunk<TYPE>;
    const int tid = threadIdx.x, T = A.threads, GP = tk.GP;
    const int p = tid & (GP - 1), u = p & 3, lrow = (tid & 63) >> tk.lgp;
    const int K = A.K, NC = K >> 6, nstep = (NC + GP - 1) >> tk.lgp, nsub = TC >> tk.lgp;
    constexpr int XS = XGroup<TYPE>::XSTRIDE;     // float4 slots per chunk
    const int xmem = TC * XS;                     // float4 per member in a buffer
    // floats of sums per member: one per group, or (int8) the chunks' {scale, sum} pairs
    const int per2 = XGroup<TYPE>::I8 ? TC * TI::XS_PER_CHUNK : K / (4 * XGroup<TYPE>::G4);
    const int tq = MC * TC * 16;                  // float4 per tile
    const float f = SC ? ldexpf(1.0f, 149 - KSC) : 1.0f;
    const double f6 = 0.25;                       // Q6_K x is never scaled here
    const size_t rbytes = (size_t)(K >> 8) * TI::BB;

    auto tile_load = [&](int ti, f32x4* v) {
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int q = min(tid + r * T, tq - 1);
            const int j = q / (TC * 16), w4 = q - j * (TC * 16);
            // positions past K (a last tile of fewer chunks) read the
            // member's last float4 instead: those slots are never used
            const int pos = min(ti * TC * 64 + 4 * w4, K - 4);
            v[r] = *reinterpret_cast<const f32x4*>(A.X + (size_t)d_xi[mc0 + j] * A.x_stride + pos);
        }
    };
    auto tile_store = [&](const f32x4* v, float4* xb) {
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int q = tid + r * T;
            if (q < tq) {
                const int j = q / (TC * 16), w4 = q - j * (TC * 16);
                f32x4 o = v[r];
                if (SC) {
                    o.x = ldexpf(o.x, KSC); o.y = ldexpf(o.y, KSC);
                    o.z = ldexpf(o.z, KSC); o.w = ldexpf(o.w, KSC);
                }
                reinterpret_cast<f32x4*>(xb)[j * xmem + tile_slot<TI::LINEAR>(4 * w4)] = o;
            }
        }
    };
    // the lane's row of task k (clamped into the item) and its weights
    auto wrow = [&](int k) {
        return gw + (size_t)(tk.r0 + min(tk.RPT * tk.grp[k] + lrow, tk.rows - 1)) * rbytes;
    };

    f32x4 xv[2];
    if (!WHOLE) {                                 // tile 0, synchronously
        tile_load(0, xv);
        tile_store(xv, xb0);
        __syncthreads();
    }
    typename C::Raw nxt = first;                  // issued before the x staging
    for (int ti = 0; ti < ntile; ti++) {
        const float4* xcur = (ti & 1) ? xb1 : xb0;
        const bool more = !WHOLE && ti + 1 < ntile;
        if (more) tile_load(ti + 1, xv);
        for (int j = 0; j < nsub; j++) {
            const int st = ti * nsub + j;
            if (st >= nstep) break;
            const int c = GP * st + p, cl = GP * j + p;
            // The loads are unconditional (a wave with fewer than MX_TW tasks
            // re-reads its next step's first unit): a load under a branch
            // would join with the old value and force a copy that waits for
            // it, serializing the prefetch.
#pragma unroll
            for (int k = 0; k < MX_TW; k++) {
                const typename C::Raw cur = nxt;
                // the next unit: task k+1 of this step, or task 0 of the next
                const bool wrap = k + 1 >= tk.ntw;
                const wptr wn = wrow(wrap ? 0 : (k + 1 < MX_TW ? k + 1 : 0));
                const int cn = min(GP * (st + (wrap ? 1 : 0)) + p, NC - 1);
                nxt = C::load(wn + (size_t)(cn >> 2) * TI::BB, u);
                if (k < tk.ntw && tk.RPT * tk.grp[k] + lrow < tk.rows && c < NC) {
                    if constexpr (TYPE == T_Q6K) {
                        const float4* xc[S];
                        bool ok[S];
#pragma unroll
                        for (int s = 0; s < S; s++) {
                            const int m = tk.sg[k] * S + s;
                            ok[s] = m < MC;
                            xc[s] = xcur + min(m, MC - 1) * xmem + cl * XS;
                        }
                        mx_term_q6k<S>(cur, u, xc, ok, f6, part[k]);
                    } else {
#pragma unroll
                        for (int s = 0; s < S; s++) {
                            const int m = tk.sg[k] * S + s;
                            if (m < MC) {
                                const float4* xc = xcur + m * xmem + cl * XS;
                                const float* xs = sums + m * per2;
                                part[k][s] = part[k][s] +
                                             C::template term<SC, true>(cur, u, xc, xs, c, f, f6);
                            }
                        }
                    }
                }
            }
        }
        if (more) {
            tile_store(xv, (ti & 1) ? xb0 : xb1);
            __syncthreads();                      // next tile in; this tile's reads done
        }
    }
    C::drain(nxt);
}

// The expert runs of a MoE selection, built in LDS by one workgroup: the
// same runs and member order as kq_moe_group_kernel writes to memory.
//  cnt[e]  members of expert e;  gid[e]  its first run (exclusive scan of
//  ceil(cnt / mch));  ms[m]  member m's expert (-1: none);  pl[m]  its place
//  among its expert's members (increasing m);  rexp[run]  the run's expert.
// Returns nd, the number of runs.  Every thread of the workgroup calls it.
struct MoeRuns {
    int* cnt;
    int* gid;
    int* ms;
    int* pl;
    int* rexp;

    // LDS at base: [routed: B x E64 router weights, 4 ceil(nm/4) selected
    // weights], cnt[E], gid[E] (16-byte padded), ms[4 ceil(nm/4)], pl[nm],
    // rexp[runs]
    __device__ int build(const MxArg& A, int* wsum, uint8_t* base) {
        const int tid = threadIdx.x, T = A.threads, lane = tid & 63, wave = tid >> 6;
        const int nm4 = (A.nm + 3) >> 2, E64 = (A.E + 63) & ~63;
        const bool routed = A.probs != nullptr;                 // uniform
        float* pw = reinterpret_cast<float*>(base);
        float* msw = pw + (routed ? A.B * E64 : 0);
        cnt = reinterpret_cast<int*>(msw + (routed ? 4 * nm4 : 0));
        gid = cnt + A.E;
        ms = cnt + ((2 * A.E + 3) & ~3);
        pl = ms + 4 * nm4;
        rexp = pl + A.nm;
        for (int e = tid; e < A.E; e += T) cnt[e] = 0;
        if (routed) {
            for (int i = tid; i < A.B * E64; i += T) {
                const int t = i / E64, e = i - t * E64;
                pw[i] = e < A.E ? A.probs[(size_t)t * A.E + e] : -1.0f;   // -1: never eligible
            }
            for (int m = tid; m < 4 * nm4; m += T) ms[m] = -1;
            __syncthreads();
            // expert e of token t takes slot rank = the eligible experts that
            // beat it (larger weight, or equal and lower id) when rank < k
            for (int i = tid; i < A.B * E64; i += T) {
                const int t = i / E64, e = i - t * E64;
                const float* row = pw + t * E64;
                const float v = row[e];
                int r = 0;
                for (int q = 0; q < E64; q += 4) {
                    const float4 o = *reinterpret_cast<const float4*>(row + q);
                    const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float x = ov[j];
                        const int beat = (x > v) | ((x == v) & (q + j < e));
                        r += (x > -1.0f) & beat;
                    }
                }
                if (v > -1.0f && r < A.k) {
                    ms[t * A.k + r] = e;
                    msw[t * A.k + r] = v;
                }
            }
            __syncthreads();
            if (blockIdx.x == 0)
                for (int m = tid; m < A.nm; m += T) {
                    A.sel_out[m] = ms[m];
                    A.selw_out[m] = ms[m] >= 0 ? msw[m] : -1.0f;
                }
            for (int m = tid; m < A.nm; m += T)
                if (ms[m] >= 0) atomicAdd(&cnt[ms[m]], 1);
        } else {
            __syncthreads();
            for (int m = tid; m < 4 * nm4; m += T) {
                const int e = m < A.nm ? A.sel[m] : -1;
                const int ok = e >= 0 && e < A.E;
                ms[m] = ok ? e : -1;
                if (ok) atomicAdd(&cnt[e], 1);
            }
        }
        __syncthreads();
        const int run = (A.E + T - 1) / T, e0 = tid * run, e1 = min(A.E, e0 + run);
        int local = 0;
        for (int e = e0; e < e1; e++) local += (cnt[e] + A.mch - 1) / A.mch;
        int incl = local;
        for (int off = 1; off < 64; off <<= 1) {
            const int o = __shfl_up(incl, off);
            if (lane >= off) incl += o;
        }
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        int before = incl - local;
        for (int i = 0; i < wave; i++) before += wsum[i];
        for (int e = e0; e < e1; e++) {
            const int nr = (cnt[e] + A.mch - 1) / A.mch;
            gid[e] = before;
            for (int r = 0; r < nr; r++) rexp[before + r] = e;
            before += nr;
        }
        int nd = 0;
        for (int i = 0; i < (T >> 6); i++) nd += wsum[i];
        for (int m = tid; m < A.nm; m += T) {
            const int e = ms[m];
            int j = 0;
            for (int q = 0; q < nm4; q++) {            // broadcast reads, 4 entries each
                const int4 v = reinterpret_cast<const int4*>(ms)[q];
                const int b = 4 * q;
                j += (b + 0 < m) & (v.x == e);
                j += (b + 1 < m) & (v.y == e);
                j += (b + 2 < m) & (v.z == e);
                j += (b + 3 < m) & (v.w == e);
            }
            pl[m] = j;
        }
        __syncthreads();
        return nd;
    }

    // ints of the tables from cnt on, for nd runs
    __device__ static int words(const MxArg& A, int nd) {
        return ((2 * A.E + 3) & ~3) + 4 * ((A.nm + 3) >> 2) + A.nm + nd;
    }
    // workgroup 0, after build: the tables to runs_out (after their count)
    __device__ void store(const MxArg& A, int nd) const {
        const int n = words(A, nd);
        for (int i = threadIdx.x; i < n; i += A.threads) A.runs_out[1 + i] = cnt[i];
        if (threadIdx.x == 0) A.runs_out[0] = nd;
    }
    // instead of build: the tables a previous launch stored (no probs here)
    __device__ int load(const MxArg& A, uint8_t* base) {
        const int nm4 = (A.nm + 3) >> 2;
        cnt = reinterpret_cast<int*>(base);
        gid = cnt + A.E;
        ms = cnt + ((2 * A.E + 3) & ~3);
        pl = ms + 4 * nm4;
        rexp = pl + A.nm;
        const int nd = A.runs_in[0];
        const int n = words(A, nd);
        for (int i = threadIdx.x; i < n; i += A.threads) cnt[i] = A.runs_in[1 + i];
        __syncthreads();
        return nd;
    }
};

// Workgroup size: 1024 lanes (128 VGPRs); Q5_K, Q3_K and Q8_0 (exact and
// int8), whose weight registers and terms do not fit 128 VGPRs with the
// next unit in flight (40-400 bytes of spill per lane), take 512 (256
// VGPRs, no spill).
template <int TYPE> constexpr int mx_threads() {
    return TYPE == T_Q5K || TYPE == T_Q3K || TYPE == T_Q80 || TYPE == T_Q5K_I8 ||
                   TYPE == T_Q3K_I8 || TYPE == T_Q80_I8
               ? 512
               : 1024;
}

template <int TYPE, int S, bool WHOLE>
__global__ __launch_bounds__(mx_threads<TYPE>()) void kq_mx_kernel(MxArg A) {
    using TI = TypeInfo<TYPE>;
    constexpr int G4 = XGroup<TYPE>::G4;
    constexpr bool SCTYPE = TI::SCALED;           // the single-stream kernel's staging rule
    constexpr bool SUMS = XGroup<TYPE>::SUMS;
    // the int8 mode of the types whose batches are per stream (Q5_K, Q3_K,
    // Q8_0): x quantized per member as the single-stream kernel does
    // (store_i8), staged whole (the host plans no tiles for them)
    constexpr bool I8 = XGroup<TYPE>::I8;
    static_assert(!I8 || WHOLE, "int8 members are staged whole");
    extern __shared__ __align__(16) uint8_t smem[];
    // the wave index in a scalar register: task choice and the task loop's
    // branches are then scalar (no exec masking around the weight loads)
    const int tid = threadIdx.x, T = A.threads, lane = tid & 63, W = T >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = A.K, NC = K >> 6, N = A.N;
    const int per = K / (4 * G4);
    const int GP = kq_phases(NC), lgp = GP == 32 ? 5 : 3, RPT = 64 / GP;
    const int TC = WHOLE ? (NC + GP - 1) & -GP : A.TC;
    const int ntile = WHOLE ? 1 : (NC + TC - 1) / TC;
    const int xmem = TC * XGroup<TYPE>::XSTRIDE;

    // LDS: member tables, flags, sums [mch][per], x buffer(s)
    int* d_xi = reinterpret_cast<int*>(smem);
    int* d_yi = d_xi + MX_MAXM;
    int* flags = d_yi + MX_MAXM;
    float* sums = reinterpret_cast<float*>(flags + 16);
    float4* xb0 = reinterpret_cast<float4*>(smem + 8 * MX_MAXM + 64 + A.sums_bytes);
    float4* xb1 = reinterpret_cast<float4*>(reinterpret_cast<uint8_t*>(xb0) + A.xt_bytes);

    MoeRuns mr;
    int nd = 1;
    const bool moe = A.nm > 0;                    // uniform: MoE runs built here
    if (moe && A.runs_in) {
        nd = mr.load(A, smem + A.grp_off);
    } else if (moe) {
        nd = mr.build(A, flags, smem + A.grp_off);
        if (A.runs_out && blockIdx.x == 0) mr.store(A, nd);
    }
    const int ng = moe ? A.nt * nd : A.gdev ? *A.ngdev : 1;
    const int nitems = ng * A.nblk;
    // Workgroups are dispatched round robin over the 8 XCDs (each with its
    // own L2): workgroup b takes the item sequence of logical index
    // (b % 8) * (grid / 8) + b / 8, so neighbouring items -- the runs of
    // one expert, which stream the same slice -- run on one XCD and share
    // its L2.  (grid a multiple of 8; otherwise the plain order.)
    const int lb = (A.grid & 7) ? (int)blockIdx.x
                                : (int)(blockIdx.x & 7) * (A.grid >> 3) + (int)(blockIdx.x >> 3);
    for (int item = lb; item < nitems; item += A.grid) {
        const int g = item / A.nblk, blk = item - g * A.nblk;
        const int r0 = blk * A.RB, rows = min(A.RB, N - r0);
        const uint8_t* gw;
        float* Yb;
        int M;
        __syncthreads();                          // the previous item's table reads are done
        if (moe) {
            const int t = g >= nd ? 1 : 0, rn = g - t * nd;
            const int e = mr.rexp[rn], r = rn - mr.gid[e];
            gw = A.wt[t] + (size_t)e * A.estride;
            Yb = A.yt[t];
            M = min(mr.cnt[e] - r * A.mch, A.mch);
            for (int m = tid; m < A.nm; m += T) {
                const int j = mr.pl[m];
                if (mr.ms[m] == e && j / A.mch == r) {
                    const int slot = j - r * A.mch;
                    d_xi[slot] = m / A.x_div;
                    d_yi[slot] = m;
                }
            }
        } else if (A.gdev) {
            const MxGroup* Gd = A.gdev + g;
            gw = Gd->w;
            Yb = Gd->y;
            M = min(Gd->M, MX_MAXM);
            for (int j = tid; j < M; j += T) { d_xi[j] = Gd->xi[j]; d_yi[j] = Gd->yi[j]; }
        } else {
            gw = A.w;
            Yb = A.Y;
            M = A.M;
            for (int j = tid; j < M; j += T) { d_xi[j] = j; d_yi[j] = j; }
        }
        for (int mc0 = 0; mc0 < M; mc0 += A.mch) {
            const int MC = min(A.mch, M - mc0);
            __syncthreads();                      // tables in; the previous chunk's LDS reads done

            // this wave's tasks t = wave + k * W
            const int nsg = (MC + S - 1) / S;
            const int ntask = ((rows + RPT - 1) / RPT) * nsg;
            MxTasks tk;
            tk.ntw = wave < ntask ? min(MX_TW, (ntask - wave + W - 1) / W) : 0;
            tk.r0 = r0;
            tk.rows = rows;
            tk.GP = GP;
            tk.lgp = lgp;
            tk.RPT = RPT;
#pragma unroll
            for (int k = 0; k < MX_TW; k++) {
                const int t = wave + k * W;
                tk.grp[k] = t / nsg;
                tk.sg[k] = t - tk.grp[k] * nsg;
            }
            // the first weights go out now, so their latency overlaps the x
            // staging
            const typename Chunk<TYPE>::Raw first = Chunk<TYPE>::load(
                to_global(gw) + (size_t)(r0 + min(RPT * tk.grp[0] + (lane >> lgp), rows - 1)) *
                                    ((size_t)(K >> 8) * TI::BB) +
                    (size_t)(min(lane & (GP - 1), NC - 1) >> 2) * TI::BB,
                lane & 3);

            // prologue: sums, window vote, and x itself when staged whole
            uint32_t dist = 0;
            if constexpr (I8) {
                // member j's chunks at xb0 + j * xmem and its {scale, sum}
                // floats at sums + j * TC * XS_PER_CHUNK (store_i8 with TC
                // as the chunk stride)
                for (int q = tid; q < MC * per; q += T) {
                    const int j = q / per, gi = q - j * per;
                    const f32x4* src = reinterpret_cast<const f32x4*>(
                                           A.X + (size_t)d_xi[mc0 + j] * A.x_stride) +
                                       (size_t)gi * G4;
                    f32x4 v[G4];
#pragma unroll
                    for (int k = 0; k < G4; k++) v[k] = src[k];
                    store_i8<TYPE>(q, per, TC, v, reinterpret_cast<uint8_t*>(xb0), sums);
                }
            } else if (SUMS || WHOLE) {
                for (int q = tid; q < MC * per; q += T) {
                    const int j = q / per, gi = q - j * per;
                    const f32x4* src = reinterpret_cast<const f32x4*>(
                                           A.X + (size_t)d_xi[mc0 + j] * A.x_stride) +
                                       (size_t)gi * G4;
                    f32x4 v[G4];
#pragma unroll
                    for (int k = 0; k < G4; k++) v[k] = src[k];
                    float acc = 0.0f;
#pragma unroll
                    for (int k = 0; k < G4; k++) {
                        acc = acc + v[k].x; acc = acc + v[k].y; acc = acc + v[k].z; acc = acc + v[k].w;
                        dist = max(max(dist, window_dist(v[k].x)), window_dist(v[k].y));
                        dist = max(max(dist, window_dist(v[k].z)), window_dist(v[k].w));
                    }
                    int slot0, xsi;
                    group_place<TYPE>(gi, slot0, xsi);
                    if (SUMS) sums[j * per + xsi] = acc;
                    if (WHOLE) {
                        f32x4* dst = reinterpret_cast<f32x4*>(xb0) + j * xmem + slot0;
#pragma unroll
                        for (int k = 0; k < G4; k++) {
                            f32x4 o = v[k];
                            if (SCTYPE) {
                                o.x = ldexpf(o.x, KSC); o.y = ldexpf(o.y, KSC);
                                o.z = ldexpf(o.z, KSC); o.w = ldexpf(o.w, KSC);
                            }
                            dst[k] = o;
                        }
                    }
                }
            }
            bool sc = false;
            if (SCTYPE) {
                const bool wave_bad = __ballot(dist >= KSC_SPAN) != 0ull;
                if (lane == 0) flags[wave] = wave_bad;
                __syncthreads();
                int any = 0;
                for (int i = 0; i < W; i++) any |= flags[i];
                sc = !any;                        // uniform over the workgroup
                if (WHOLE && any) {               // restage unscaled
                    for (int q = tid; q < MC * per; q += T) {
                        const int j = q / per, gi = q - j * per;
                        const f32x4* src = reinterpret_cast<const f32x4*>(
                                               A.X + (size_t)d_xi[mc0 + j] * A.x_stride) +
                                           (size_t)gi * G4;
                        int slot0, xsi;
                        group_place<TYPE>(gi, slot0, xsi);
                        f32x4* dst = reinterpret_cast<f32x4*>(xb0) + j * xmem + slot0;
#pragma unroll
                        for (int k = 0; k < G4; k++) dst[k] = src[k];
                    }
                    __syncthreads();
                }
            } else {
                __syncthreads();
            }

            double part[MX_TW][S];
#pragma unroll
            for (int k = 0; k < MX_TW; k++)
#pragma unroll
                for (int s = 0; s < S; s++) part[k][s] = 0.0;

            if (sc)
                mx_sweep<TYPE, S, WHOLE, SCTYPE>(A, tk, to_global(gw), part, MC, mc0, d_xi, sums,
                                                 xb0, xb1, TC, ntile, first);
            else
                mx_sweep<TYPE, S, WHOLE, false>(A, tk, to_global(gw), part, MC, mc0, d_xi, sums,
                                                xb0, xb1, TC, ntile, first);

            // phase_tree per member (every lane of the wave takes part)
#pragma unroll
            for (int k = 0; k < MX_TW; k++) {
                if (k < tk.ntw) {
#pragma unroll
                    for (int s = 0; s < S; s++) {
                        const double v = phase_tree(part[k][s], GP);
                        const int m = tk.sg[k] * S + s;
                        const int rr = RPT * tk.grp[k] + (lane >> lgp);
                        if (rr < rows && (lane & (GP - 1)) == 0 && m < MC)
                            Yb[(size_t)d_yi[mc0 + m] * A.y_stride + r0 + rr] = (float)v;
                    }
                }
            }
        }
    }
}

template <int TYPE>
int launch_mx_t(const MxArg& a, int s, bool whole, long lds, hipStream_t st) {
#define KQ_MX_GO(S_, W_) \
    hipLaunchKernelGGL((kq_mx_kernel<TYPE, S_, W_>), dim3(a.grid), dim3(a.threads), (size_t)lds, st, a)
    if (whole) {
        if (s == 1) KQ_MX_GO(1, true); else KQ_MX_GO(2, true);
    } else if constexpr (!XGroup<TYPE>::I8) {
        if (s == 1) KQ_MX_GO(1, false); else KQ_MX_GO(2, false);
    } else {
        return (int)hipErrorInvalidValue;     // int8 members are staged whole
    }
#undef KQ_MX_GO
    return (int)hipGetLastError();
}

// ------------------------------------------------------------ MoE routing
// Top-k per token (moe_topk, stratum_arch_moe.inc.c:368-385): slots start
// at (sel -1, weight -1.0f) and expert e, in increasing e, displaces the
// first slot whose weight it beats strictly.  The result is the k largest
// weights in decreasing order, equal weights in increasing expert order,
// counting only weights > -1 (NaN never beats anything); missing slots
// stay (-1, -1.0f).  One wave per token: k rounds of a wave argmax over the
// eligible experts (ties to the lower index).
__global__ __launch_bounds__(256) void kq_moe_topk_kernel(const float* probs, int B, int E, int k,
                                                         int* sel, float* selw) {
    const int lane = threadIdx.x & 63;
    const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (tok >= B) return;                      // uniform over the wave
    const float* w = probs + (size_t)tok * E;
    uint64_t taken = 0;                        // experts lane + 64 i already chosen, bit i
    for (int r = 0; r < k; r++) {
        float bv = -1.0f;
        int be = 0x7fffffff;
        for (int i = 0, e = lane; e < E; i++, e += 64) {
            const float v = w[e];
            const bool free_ = !((taken >> i) & 1);     // E <= 4096: i < 64
            if (free_ && v > bv) { bv = v; be = e; }   // first (lowest) e wins ties in a lane
        }
        // wave argmax: larger weight, then lower expert
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oe = __shfl_xor(be, off);
            if (ov > bv || (ov == bv && oe < be)) { bv = ov; be = oe; }
        }
        const bool found = be != 0x7fffffff;
        if (lane == 0) {
            sel[(size_t)tok * k + r] = found ? be : -1;
            selw[(size_t)tok * k + r] = found ? bv : -1.0f;
        }
        if (found && (be & 63) == lane) taken |= 1ull << (be >> 6);
    }
}

// The same selection for E <= 1024 by ranks: expert e's slot is the number
// of eligible experts that beat it (a larger weight, or an equal weight and
// a lower id).  One 1024-lane workgroup per token: the weights go to LDS,
// lane (p, e) counts the experts of part p (of P) that beat e, and the P
// partial counts are added.  (One wave per token, scanning all E experts,
// was a serial chain of ~E x 15 dependent instructions: 8 us at E = 128.)
__global__ __launch_bounds__(1024) void kq_moe_topk_rank_kernel(const float* probs, int B, int E,
                                                              int k, int* sel, float* selw) {
    __shared__ __align__(16) float wl[1024];
    __shared__ int part[1024];
    __shared__ int nel;
    const int tid = threadIdx.x, tok = blockIdx.x;
    const int E64 = (E + 63) & ~63;                  // experts, padded: <= 1024
    // parts: a power of two P with P * E64 <= 1024 and E64 / P a multiple of 4
    int P = 1;
    while (2 * P * E64 <= 1024 && (E64 / (2 * P)) % 4 == 0) P *= 2;
    const int L = E64 / P;                           // experts per part
    const float* w = probs + (size_t)tok * E;
    if (tid < E64) wl[tid] = tid < E ? w[tid] : -1.0f;   // -1: never eligible
    if (tid == 0) nel = 0;
    __syncthreads();
    const int e = tid % E64, p = tid / E64;
    if (p < P) {
        const float v = wl[e];
        int r = 0;
        const int q0 = p * L;
        for (int q = q0; q < q0 + L; q += 4) {
            const float4 o = *reinterpret_cast<const float4*>(&wl[q]);
            const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float x = ov[j];
                // bitwise, not short-circuit: straight-line compares
                const int beat = (x > v) | ((x == v) & (q + j < e));
                r += (x > -1.0f) & beat;             // NaN is not eligible either
            }
        }
        part[tid] = r;
        if (p == 0 && e < E && v > -1.0f) atomicAdd(&nel, 1);
    }
    __syncthreads();
    if (tid < E) {
        int rank = 0;
        for (int i = 0; i < P; i++) rank += part[i * E64 + tid];
        const float v = wl[tid];
        if (v > -1.0f && rank < k) {
            sel[(size_t)tok * k + rank] = tid;
            selw[(size_t)tok * k + rank] = v;
        }
    }
    for (int r = nel + tid; r < k; r += 1024) {     // slots without an expert
        sel[(size_t)tok * k + r] = -1;
        selw[(size_t)tok * k + r] = -1.0f;
    }
}

// Expert groups of the selected (token, rank) members, in increasing expert
// order (moe_forward_b's member lists, stratum_arch_moe.inc.c:1130-1140):
// for each distinct expert e, the members m (in increasing m) that chose e,
// cut into runs of at most mch (the reference's chunked tickets, :1158-1170,
// here so that every work item carries about the same load), and one
// MxGroup per run and tensor t: weights w[t] + e * estride, x row m / x_div,
// output row m of y[t].  One workgroup; *ng = nt * runs.
struct MoeGroupArg {
    const int* sel;
    int nm, E, nt, x_div, mch;     // members (B * k), experts, tensors, x divisor, run
    const uint8_t* w[2];
    float* y[2];
    long estride;
    MxGroup* groups;
    int* ng;
};

// (the body, for one workgroup of 1024 lanes with the dynamic LDS lds_i)
__device__ void moe_group_body(const MoeGroupArg& a, int* lds_i) {
    int* cnt = lds_i;                 // [E]
    int* gid = cnt + a.E;             // [E] group index of expert e
    // [4 ceil(nm/4)] the members' experts (-1: none), 16-byte aligned, the
    // tail past nm filled with -1 (it is read in whole int4s)
    int* ms = lds_i + ((2 * a.E + 3) & ~3);
    const int nm4 = (a.nm + 3) >> 2;
    __shared__ int wsum[16];
    const int tid = threadIdx.x, T = blockDim.x, lane = tid & 63, wave = tid >> 6;
    for (int e = tid; e < a.E; e += T) cnt[e] = 0;
    __syncthreads();
    for (int m = tid; m < 4 * nm4; m += T) {
        const int e = m < a.nm ? a.sel[m] : -1;
        const int ok = e >= 0 && e < a.E;
        ms[m] = ok ? e : -1;
        if (ok) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // exclusive scan of the run counts ceil(cnt[e] / mch) over e: each
    // thread a range of experts
    const int run = (a.E + T - 1) / T, e0 = tid * run, e1 = min(a.E, e0 + run);
    int local = 0;
    for (int e = e0; e < e1; e++) local += (cnt[e] + a.mch - 1) / a.mch;
    int incl = local;
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(incl, off);
        if (lane >= off) incl += o;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int before = incl - local;
    for (int i = 0; i < wave; i++) before += wsum[i];
    for (int e = e0; e < e1; e++) {
        gid[e] = before;
        before += (cnt[e] + a.mch - 1) / a.mch;
    }
    int nd = 0;
    for (int i = 0; i < (T >> 6); i++) nd += wsum[i];
    __syncthreads();
    if (tid == 0) *a.ng = a.nt * nd;
    // One thread per member: its place j among the members of its expert
    // (the members before it with the same expert, so places follow
    // increasing m), then its slot j % mch of run j / mch; the first member
    // of a run writes the run's header.  The scan reads ms[] at the same
    // index in every lane (broadcast), four entries per LDS read and four
    // reads in flight.
    const int4* ms4 = reinterpret_cast<const int4*>(ms);
    auto count4 = [](int4 v, int b, int m, int e) {
        return ((b + 0 < m) & (v.x == e)) + ((b + 1 < m) & (v.y == e)) +
               ((b + 2 < m) & (v.z == e)) + ((b + 3 < m) & (v.w == e));
    };
    for (int m0 = 0; m0 < a.nm; m0 += T) {
        const int m = m0 + tid;
        const int e = m < a.nm ? ms[m] : -1;
        int j = 0;
        const int lim = min(a.nm, m0 + T);               // uniform bound of the scan
        const int nq = min(nm4, (lim + 3) >> 2);
        int q = 0;
        for (; q + 4 <= nq; q += 4) {
            const int4 v0 = ms4[q], v1 = ms4[q + 1], v2 = ms4[q + 2], v3 = ms4[q + 3];
            j += count4(v0, 4 * q, m, e) + count4(v1, 4 * q + 4, m, e) +
                 count4(v2, 4 * q + 8, m, e) + count4(v3, 4 * q + 12, m, e);
        }
        for (; q < nq; q++) j += count4(ms4[q], 4 * q, m, e);
        if (e >= 0) {
            const int r = j / a.mch, slot = j - r * a.mch;
            for (int t = 0; t < a.nt; t++) {
                MxGroup* G = a.groups + (size_t)t * nd + gid[e] + r;
                G->xi[slot] = m / a.x_div;
                G->yi[slot] = m;
                if (slot == 0) {
                    G->w = a.w[t] + (size_t)e * a.estride;
                    G->y = a.y[t];
                    G->M = min(cnt[e] - j, a.mch);
                    G->pad_ = 0;
                }
            }
        }
    }
}

__global__ __launch_bounds__(1024) void kq_moe_group_kernel(MoeGroupArg a) {
    extern __shared__ __align__(16) int lds_i[];
    moe_group_body(a, lds_i);
}

// ------------------------------------------------------- MFMA multi-x
// Tolerance path for many streams (B >= 16), Q4_K and Q6_K, on the matrix
// cores.  The weights enter with their sub-block scales folded in, as exact
// fp16 integers: Q4_K w = sc*q (sc <= 63, q <= 15: at most 945), Q6_K
// w = sc*(q - 32) (|w| <= 4096) split exactly into 16*sh*(q - 32) and
// sl*(q - 32), sc = 16 sh + sl.  x enters as two fp16 planes, hi = fp16(x') and
// mid = fp16(x' - hi), of x' = x*2^(15-E), E the binary exponent of the
// largest |x| of the (stream, super-block): the planes cannot overflow, each
// x keeps 22 significant bits (|x - (hi + mid) 2^(E-15)| <= 2^-21 |x| +
// 2^-39 max|x|), and every product w*plane is exact in fp32.  A super-block
// (256 weights) accumulates in one MFMA accumulator
// (mfma_f32_16x16x32_f16) and joins the row's running sum as
// fma(d*2^(E-15), acc, sum); the Q4_K min term -sum_j dmin*m_j*xsum_j
// (xsum_j the sequential binary32 sum of sub-block j's 32 x) runs on the
// fp32 matrix cores (mfma_f32_16x16x4_f32) into the same sum.  Differences
// from the reference: x rounded to 22 bits, the fp32 order of the sums, and
// the block scale applied to the super-block sum instead of each
// sub-block's.
//
// Operands: D[stream][row] = sum_k A[stream][k] B[k][row], A = an x plane,
// B = the weights.  In the 16x16x32 MFMAs lane l holds B[k][row = l % 16]
// for k = 8*(l/16) + v and receives D[4*(l/16) + v][l % 16]; in the
// 16x16x4 fp32 MFMA lane l holds A[l % 16][l / 16] and B[l / 16][l % 16].
// A lane's weight row is its output row, so each lane decodes only its own
// row.
//  * kq_mf_split_kernel: one workgroup per (super-block, 16-stream group)
//    writes the two planes in A-operand order, the x sums and E;
//  * kq_mf_kernel: 8 waves; a wave owns MfShape::TILES 16-row tiles (Q4_K 2,
//    Q6_K 1: Q6_K's two weight parts already use each A operand twice), so a
//    workgroup sweeps a block of 256 (Q4_K) or 128 (Q6_K) rows.  The
//    (row block, super-block) iterations are split into one contiguous range
//    per workgroup (whole row blocks when there are at least two per
//    workgroup); a super-block's planes for all stream groups are staged in
//    LDS (double-buffered) while the previous super-block is consumed, and
//    each weight step is decoded once for every stream group;
//  * kq_mf_reduce_kernel adds, in workgroup order, the partial sums of the
//    row blocks that several workgroups share (a fixed order: the result
//    does not depend on timing).
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
constexpr int MF_NW = 8;                         // waves per workgroup
constexpr int MF_GROUP_U4 = 8 * 2 * 64;          // uint4 of planes per (super-block, group)
constexpr int MF_SIDE_U4 = (8 * 16 + 16) / 4;    // x sums (8 x 16 floats), then E (16 ints)

template <int TYPE> struct MfShape {
    static constexpr int TILES = TYPE == T_Q4K ? 2 : 1;
    static constexpr int ROWS = 16 * TILES * MF_NW;                    // rows per row block
};

// uint4 of one super-block's LDS stage for nsg stream groups
__host__ __device__ constexpr int mf_stage_u4(int nsg) { return nsg * (MF_GROUP_U4 + MF_SIDE_U4); }

// How the (row block, super-block) iterations go to the workgroups: whole
// row blocks per workgroup when there are at least two per workgroup, else
// an even split of all nrb * NSB iterations (G <= T).
struct MfPlan {
    int rows, nrb, G, whole;
    long T;
    long part_floats;        // partial sums (0 when every row block has one owner)
};

__host__ __device__ inline MfPlan mf_plan(int type, int NSG, int N, int K, int grid) {
    MfPlan p;
    p.rows = type == T_Q4K ? MfShape<T_Q4K>::ROWS : MfShape<T_Q6K>::ROWS;
    p.nrb = (N + p.rows - 1) / p.rows;
    p.T = (long)p.nrb * (K >> 8);
    p.whole = p.nrb >= 2 * grid;
    p.G = p.whole ? grid : (int)(p.T < grid ? p.T : grid);
    p.part_floats = p.whole ? 0 : (long)(p.G + p.nrb) * 16 * NSG * p.rows;
    return p;
}

// the workgroup whose range holds iteration a (uneven split of T over G)
__device__ __forceinline__ long mf_owner(long a, long T, int G) { return ((a + 1) * G - 1) / T; }

struct MfSplitArg {
    const float* x;          // B x K
    uint4* planes;           // NSB x NSG x 8 steps x 2 planes x 64 lanes (8 fp16 each)
    uint4* side;             // NSB x NSG x (8 x 16 sums of 32, 16 E)
    int B, K, NSG;
};

__device__ __forceinline__ uint32_t pack_h2(_Float16 a, _Float16 b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// One workgroup per (super-block, 16-stream group): thread t = 16 si + p
// takes stream si's 16 x at 16 p (sub-block p / 2, k-groups 2 (p & 1) and
// 2 (p & 1) + 1 of step p / 2); E is the exponent of the stream's largest
// |x| in the super-block (a 16-lane max).  Padding streams write zeros.
__global__ __launch_bounds__(256) void kq_mf_split_kernel(MfSplitArg a) {
    const int sb = blockIdx.x / a.NSG, g = blockIdx.x - sb * a.NSG;
    const int t = threadIdx.x, si = t >> 4, p = t & 15;
    const int s = 16 * g + si;
    const bool live = s < a.B;
    float v[16];
    const float4* src = reinterpret_cast<const float4*>(a.x + (size_t)(live ? s : 0) * a.K + 256 * sb + 16 * p);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float4 f = live ? src[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) mx = fmaxf(mx, fabsf(v[i]));
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));   // the stream's 16 lanes
    const int E = __builtin_amdgcn_frexp_expf(mx);        // mx = m 2^E, m in [0.5, 1); 0 for 0
    uint32_t hw[8], mw[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        _Float16 h2[2], m2[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const float xv = ldexpf(v[2 * e + i], 15 - E);
            h2[i] = (_Float16)xv;
            m2[i] = (_Float16)(xv - (float)h2[i]);
        }
        hw[e] = pack_h2(h2[0], h2[1]);
        mw[e] = pack_h2(m2[0], m2[1]);
    }
    const size_t pair = (size_t)sb * a.NSG + g;
    uint4* dst = a.planes + (pair * 8 + (p >> 1)) * 128 + 16 * (2 * (p & 1)) + si;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        dst[16 * h] = make_uint4(hw[4 * h], hw[4 * h + 1], hw[4 * h + 2], hw[4 * h + 3]);
        dst[64 + 16 * h] = make_uint4(mw[4 * h], mw[4 * h + 1], mw[4 * h + 2], mw[4 * h + 3]);
    }
    float* side = reinterpret_cast<float*>(a.side + pair * MF_SIDE_U4);
    if (p == 0) reinterpret_cast<int*>(side)[128 + si] = E;
    // sequential binary32 sum of the 32 values of sub-block p / 2: the even
    // lane sums its 16, the odd lane continues from it
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) acc = acc + v[i];
    const float first = __shfl(acc, (t & 63) - (p & 1));
    if (p & 1) {
        acc = first;
#pragma unroll
        for (int i = 0; i < 16; i++) acc = acc + v[i];
        side[(p >> 1) * 16 + si] = acc;
    }
}

struct MfArg {
    const uint8_t* w;
    const uint4* planes;
    const uint4* side;
    float* y;                // B x N
    float* part;             // (G + nrb) slots x 16 NSG x rows: partial sums
    int B, N, K, NSG, nrb, G, whole;
    long T;
};

__device__ __forceinline__ uint32_t byte_of(const uint4& v, int i) {
    const uint32_t w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return (w >> (8 * (i & 3))) & 0xffu;
}

// One super-block of one row as one lane needs it (k-group kg).
struct MfRawQ4 { uint4 hd; uint2 q[4]; };
struct MfRawQ6 { uint32_t ql[4][3], qh[2][3], sc[5]; uint32_t d, sh; };
template <int TYPE> struct MfRaw;
template <> struct MfRaw<T_Q4K> { using T = MfRawQ4; };
template <> struct MfRaw<T_Q6K> { using T = MfRawQ6; };

// Q4_K: chunk c's 8 bytes for this lane: low nibbles are sub-block 2c at
// positions 64c + 8kg + v, high nibbles sub-block 2c + 1 at 64c + 32 + 8kg + v
__device__ __forceinline__ MfRawQ4 mf_load_q4k(wptr blk, int kg) {
    MfRawQ4 r;
    r.hd = ld16(blk);
#pragma unroll
    for (int c = 0; c < 4; c++) r.q[c] = ld8a4(blk + 16 + 32 * c + 8 * kg);
    return r;
}

// Q6_K: positions 32 st + 8 kg + v (step st = 4h + t) are bytes
// 64h + 32(t&1) + 16(kg>>1) + 8(kg&1) + v of ql (nibble t >> 1) and
// 128 + 32h + 16(kg>>1) + 8(kg&1) + v of qh (bits 2t): four ql fields and
// two qh fields of 8 bytes, each read as three dwords of the 4-aligned
// block and realigned (the third repeats the second when the block is
// aligned, so no read passes the block's 210 bytes); the lane's sub-block
// scales are bytes 192 + 2 st + (kg >> 1).
__device__ __forceinline__ MfRawQ6 mf_load_q6k(wptr blk, int kg) {
    MfRawQ6 r;
    const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(blk) & 3u;
    r.sh = mis * 8u;
    const wptr b4 = blk - mis;
    const int nx = mis ? 4 : 0;
    const int o = 16 * (kg >> 1) + 8 * (kg & 1);
#pragma unroll
    for (int f = 0; f < 4; f++) {
        const int off = 64 * (f >> 1) + 32 * (f & 1) + o;
        r.ql[f][0] = ld4(b4 + off);
        r.ql[f][1] = ld4(b4 + off + 4);
        r.ql[f][2] = ld4(b4 + off + 4 + nx);
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int off = 128 + 32 * h + o;
        r.qh[h][0] = ld4(b4 + off);
        r.qh[h][1] = ld4(b4 + off + 4);
        r.qh[h][2] = ld4(b4 + off + 4 + nx);
    }
    const uint4 sv = ld16a4(b4 + 192);
    r.sc[0] = sv.x; r.sc[1] = sv.y; r.sc[2] = sv.z; r.sc[3] = sv.w;
    r.sc[4] = ld4(b4 + 192 + 12 + nx);
    r.d = ld2(blk + 208);
    return r;
}

template <int TYPE>
__device__ __forceinline__ typename MfRaw<TYPE>::T mf_load(wptr blk, int kg) {
    if constexpr (TYPE == T_Q4K) return mf_load_q4k(blk, kg);
    else return mf_load_q6k(blk, kg);
}

// fp16 of sc * q for the 4 nibble bytes of nib (each < 16), sc <= 63: the
// bytes become 1024 + q (fp16 0x6400 | q), and fma((1024 + q), sc,
// -1024 sc) = sc q exactly (every value is an integer below 2048)
__device__ __forceinline__ void q4_scaled(uint32_t nib, half2v sc2, half2v off2, uint32_t& w01,
                                          uint32_t& w23) {
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, nib, 0x05010400u);   // q0, q1
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, nib, 0x05030402u);   // q2, q3
    w01 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2v, a), sc2, off2));
    w23 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2v, b), sc2, off2));
}

// fp16 of the two parts of w = sc * (q - 32) for the four q bytes of q4
// (each < 64), sc = 16 sh + sl: the bytes 4 q become halves 0x6C00 | 4q =
// 4096 + 16 q, and fma(4096 + 16 q, sh, -4608 sh) = 16 sh (q - 32),
// fma(4096 + 16 q, sl / 16, -288 sl) = sl (q - 32): exact integers (every
// intermediate below 65504, the results of at most 9 significant bits), and
// their sum is w.  m1, a1, m2, a2 = sh, -4608 sh, sl / 16, -288 sl.
__device__ __forceinline__ void q6_split(uint32_t q4, _Float16 m1, _Float16 a1, _Float16 m2,
                                         _Float16 a2, uint32_t& h01, uint32_t& h23, uint32_t& l01,
                                         uint32_t& l23) {
    const uint32_t s4 = q4 << 2;                                               // 4 q per byte
    const half2v p01 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x6c6c6c6cu, s4, 0x05010400u));
    const half2v p23 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x6c6c6c6cu, s4, 0x05030402u));
    const half2v M1 = {m1, m1}, A1 = {a1, a1}, M2 = {m2, m2}, A2 = {a2, a2};
    h01 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(p01, M1, A1));
    h23 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(p23, M1, A1));
    l01 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(p01, M2, A2));
    l23 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(p23, M2, A2));
}

// Per-super-block constants of one lane's row.  Q4_K: d, and the B operands
// of the min term, -dmin*m_kg and -dmin*m_(4+kg) (6-bit mins,
// stratum_q4k.h:57-65).  Q6_K: d, and the lane's scale bytes realigned.
template <int TYPE> struct MfSb;
template <> struct MfSb<T_Q4K> { float d, nm0, nm1; };
template <> struct MfSb<T_Q6K> { float d; uint32_t scw[4]; };

__device__ __forceinline__ MfSb<T_Q4K> mf_sb(const MfRawQ4& r, int kg) {
    MfSb<T_Q4K> c;
    c.d = f16_bits_to_f32(r.hd.x & 0xffffu);
    const float dmin = f16_bits_to_f32(r.hd.x >> 16);
    const uint32_t sh = 8u * (uint32_t)kg;
    const uint32_t b4 = (r.hd.z >> sh) & 0xffu;           // scale byte 4 + kg
    const uint32_t b8 = (r.hd.w >> sh) & 0xffu;           // scale byte 8 + kg
    c.nm0 = -(dmin * (float)(b4 & 63u));
    c.nm1 = -(dmin * (float)((b8 >> 4) | ((b4 >> 6) << 4)));
    return c;
}

__device__ __forceinline__ MfSb<T_Q6K> mf_sb(const MfRawQ6& r, int) {
    MfSb<T_Q6K> c;
    c.d = f16_bits_to_f32(r.d);
#pragma unroll
    for (int k = 0; k < 4; k++) c.scw[k] = __builtin_amdgcn_alignbit(r.sc[k + 1], r.sc[k], r.sh);
    return c;
}

// Q4_K step j (sub-block j): the lane's 8 weights sc_j * q
__device__ __forceinline__ half8 mf_step_q4k(const MfRawQ4& r, int j) {
    const uint4 sc = make_uint4(r.hd.y, r.hd.z, r.hd.w, 0u);
    const uint32_t s_ = j < 4 ? byte_of(sc, j) & 63u
                              : (byte_of(sc, j + 4) & 15u) | ((byte_of(sc, j - 4) >> 6) << 4);
    const _Float16 sh = (_Float16)(float)s_;
    const half2v sc2 = {sh, sh};
    const _Float16 of = (_Float16)(-1024.0f * (float)s_);
    const half2v off2 = {of, of};
    const uint2 q = r.q[j >> 1];
    const uint32_t n0 = (j & 1) ? (q.x >> 4) & 0x0f0f0f0fu : q.x & 0x0f0f0f0fu;
    const uint32_t n1 = (j & 1) ? (q.y >> 4) & 0x0f0f0f0fu : q.y & 0x0f0f0f0fu;
    uint32_t w0, w1, w2, w3;
    q4_scaled(n0, sc2, off2, w0, w1);
    q4_scaled(n1, sc2, off2, w2, w3);
    return __builtin_bit_cast(half8, make_uint4(w0, w1, w2, w3));
}

// Q6_K step st: the lane's 8 weights sc * (q - 32) as its two parts 16 sh (q - 32) and sl (q - 32)
__device__ __forceinline__ void mf_step_q6k(const MfRawQ6& r, const MfSb<T_Q6K>& c, int kg, int st,
                                            half8& wh, half8& wl) {
    const uint32_t sh = r.sh;
    const int h = st >> 2, t = st & 3;
    const int f = 2 * h + (t & 1);
    const uint32_t L0 = __builtin_amdgcn_alignbit(r.ql[f][1], r.ql[f][0], sh);
    const uint32_t L1 = __builtin_amdgcn_alignbit(r.ql[f][2], r.ql[f][1], sh);
    const uint32_t H0 = __builtin_amdgcn_alignbit(r.qh[h][1], r.qh[h][0], sh);
    const uint32_t H1 = __builtin_amdgcn_alignbit(r.qh[h][2], r.qh[h][1], sh);
    const uint32_t q0 = ((L0 >> (4 * (t >> 1))) & 0x0f0f0f0fu) | (((H0 >> (2 * t)) & 0x03030303u) << 4);
    const uint32_t q1 = ((L1 >> (4 * (t >> 1))) & 0x0f0f0f0fu) | (((H1 >> (2 * t)) & 0x03030303u) << 4);
    // the lane's scale: byte 2 st + (kg >> 1), split as sc = 16 sh + sl
    // (sh = sc >> 4 in [-8, 7], sl = sc & 15)
    const int b = 2 * st + (kg >> 1);
    const int sc = (int)(int8_t)(uint8_t)(c.scw[b >> 2] >> (8 * (b & 3)));
    const int shi = sc >> 4, slo = sc & 15;
    const _Float16 m1 = (_Float16)(short)shi, a1 = (_Float16)(float)(-4608 * shi);   // |a1| <= 36864
    const _Float16 m2 = (_Float16)(short)slo * (_Float16)0.0625f, a2 = (_Float16)(short)(-288 * slo);
    uint32_t h4[4], l4[4];
    q6_split(q0, m1, a1, m2, a2, h4[0], h4[1], l4[0], l4[1]);
    q6_split(q1, m1, a1, m2, a2, h4[2], h4[3], l4[2], l4[3]);
    wh = __builtin_bit_cast(half8, make_uint4(h4[0], h4[1], h4[2], h4[3]));
    wl = __builtin_bit_cast(half8, make_uint4(l4[0], l4[1], l4[2], l4[3]));
}

template <int TYPE, int NSG>
__global__ __launch_bounds__(64 * MF_NW) void kq_mf_kernel(MfArg A) {
    using TI = TypeInfo<TYPE>;
    using SH = MfShape<TYPE>;
    constexpr int TL = SH::TILES, R = SH::ROWS, NT = 64 * MF_NW;
    constexpr int PU = NSG * MF_GROUP_U4, NX = NSG * MF_SIDE_U4, SU = PU + NX;   // uint4 per stage
    constexpr int NP = PU / NT;                                        // plane uint4 per thread
    constexpr int NH = NP / 2 + 1;                                     // per staging half
    static_assert(NP * NT == PU && NP % 2 == 0 && NX <= NT, "stage split");
    extern __shared__ __align__(16) uint8_t smem[];
    u32x4* lds = reinterpret_cast<u32x4*>(smem);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, kg = lane >> 4;
    const int NSB = A.K >> 8;
    const size_t rbytes = (size_t)NSB * TI::BB;
    const int wg = blockIdx.x;
    int it0, it1;
    if (A.whole) {
        it0 = (int)((long)wg * A.nrb / A.G) * NSB;
        it1 = (int)((long)(wg + 1) * A.nrb / A.G) * NSB;
    } else {
        it0 = (int)((long)wg * A.T / A.G);
        it1 = (int)((long)(wg + 1) * A.T / A.G);
    }
    if (it0 >= it1) return;                 // the whole workgroup: no barrier is left waiting
    auto wrow = [&](int rb, int t) {
        const int row = rb * R + 16 * (TL * wave + t) + (lane & 15);
        return to_global(A.w) + (size_t)min(row, A.N - 1) * rbytes;
    };
    // staging of super-block sb in two halves (the planes' first half; the
    // second half, the x sums and E); the loads are branch-free (clamped), so
    // the compiler counts outstanding loads exactly
    auto sload = [&](int h, int sb, u32x4 (&v)[NH]) {
        const u32x4* pp = reinterpret_cast<const u32x4*>(A.planes) + (size_t)sb * PU + tid + NT * (NP / 2) * h;
#pragma unroll
        for (int k = 0; k < NP / 2; k++) v[k] = pp[NT * k];
        if (h) v[NP / 2] = reinterpret_cast<const u32x4*>(A.side)[(size_t)sb * NX + min(tid, NX - 1)];
    };
    auto sstore = [&](int h, int buf, const u32x4 (&v)[NH]) {
#pragma unroll
        for (int k = 0; k < NP / 2; k++) lds[buf * SU + tid + NT * (k + (NP / 2) * h)] = v[k];
        if (h && tid < NX) lds[buf * SU + PU + tid] = v[NP / 2];
    };
    int rb = it0 / NSB, sb = it0 - rb * NSB;
    typename MfRaw<TYPE>::T raw[TL];
    {
        u32x4 v0[NH], v1[NH];
        sload(0, sb, v0);
        sload(1, sb, v1);
#pragma unroll
        for (int t = 0; t < TL; t++) raw[t] = mf_load<TYPE>(wrow(rb, t) + (size_t)sb * TI::BB, kg);
        sstore(0, 0, v0);
        sstore(1, 0, v1);
    }
    __syncthreads();
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc[TL][NSG];
#pragma unroll
    for (int t = 0; t < TL; t++)
#pragma unroll
        for (int g = 0; g < NSG; g++) acc[t][g] = zero;
    for (int it = it0; it < it1; it++) {
        const int buf = (it - it0) & 1;
        const bool more = it + 1 < it1;
        const int sbn = sb + 1 == NSB ? 0 : sb + 1, rbn = sb + 1 == NSB ? rb + 1 : rb;
        const int sbl = more ? sbn : sb, rbl = more ? rbn : rb;   // the last iteration reloads its own
        typename MfRaw<TYPE>::T rc[TL];
        MfSb<TYPE> cs[TL];
#pragma unroll
        for (int t = 0; t < TL; t++) {
            rc[t] = raw[t];
            cs[t] = mf_sb(rc[t], kg);
        }
        u32x4 sv[NH];
        sload(0, sbl, sv);                  // the next stage's first half, then the next weights
#pragma unroll
        for (int t = 0; t < TL; t++) raw[t] = mf_load<TYPE>(wrow(rbl, t) + (size_t)sbl * TI::BB, kg);
        f32x4 C[TL][NSG], D[TL][NSG];       // D: the Q6_K sl parts
#pragma unroll
        for (int t = 0; t < TL; t++)
#pragma unroll
            for (int g = 0; g < NSG; g++) C[t][g] = D[t][g] = zero;
        const u32x4* sp = lds + buf * SU + lane;
        // step j + 1's plane reads and weight decode are issued while step
        // j's MFMAs run
        half8 x0[2][NSG], x1[2][NSG], wa[2][TL], wb[2][TL];
        auto fetch = [&](int j, int c) {
#pragma unroll
            for (int g = 0; g < NSG; g++) {
                x0[c][g] = __builtin_bit_cast(half8, sp[(g * 8 + j) * 128]);
                x1[c][g] = __builtin_bit_cast(half8, sp[(g * 8 + j) * 128 + 64]);
            }
#pragma unroll
            for (int t = 0; t < TL; t++) {
                if constexpr (TYPE == T_Q4K) wa[c][t] = mf_step_q4k(rc[t], j);
                else mf_step_q6k(rc[t], cs[t], kg, j, wa[c][t], wb[c][t]);
            }
        };
        fetch(0, 0);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int c = j & 1;
            if (j < 7) fetch(j + 1, c ^ 1);
            // every accumulator once per pass, so dependent MFMAs are
            // TL * NSG instructions apart
#pragma unroll
            for (int pass = 0; pass < 2; pass++) {
#pragma unroll
                for (int g = 0; g < NSG; g++)
#pragma unroll
                    for (int t = 0; t < TL; t++) {
                        const half8 xa = pass ? x1[c][g] : x0[c][g];
                        C[t][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, wa[c][t], C[t][g], 0, 0, 0);
                        if constexpr (TYPE == T_Q6K)
                            D[t][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, wb[c][t], D[t][g], 0, 0, 0);
                    }
            }
            if (j == 3) {                   // the first half is in: store it, fetch the second
                sstore(0, buf ^ 1, sv);
                sload(1, sbl, sv);
            }
            // keeps the compiler from hoisting later steps' reads (registers)
            __builtin_amdgcn_sched_barrier(0);
        }
        // the running sums: sum = fma(d 2^(E-15), C, sum), then (Q4_K) the
        // min term
#pragma unroll
        for (int g = 0; g < NSG; g++) {
            const u32x4* sd = lds + buf * SU + PU + MF_SIDE_U4 * g;
            const float a0 = reinterpret_cast<const float*>(sd)[lane];
            const float a1 = reinterpret_cast<const float*>(sd)[64 + lane];
            const u32x4 e4 = sd[32 + kg];         // E of streams 4 kg + v
#pragma unroll
            for (int t = 0; t < TL; t++) {
                const float f0 = ldexpf(cs[t].d, (int)e4.x - 15), f1 = ldexpf(cs[t].d, (int)e4.y - 15);
                const float f2 = ldexpf(cs[t].d, (int)e4.z - 15), f3 = ldexpf(cs[t].d, (int)e4.w - 15);
                f32x4 s = acc[t][g];
                s.x = fmaf(f0, C[t][g].x, s.x);
                s.y = fmaf(f1, C[t][g].y, s.y);
                s.z = fmaf(f2, C[t][g].z, s.z);
                s.w = fmaf(f3, C[t][g].w, s.w);
                if constexpr (TYPE == T_Q6K) {
                    s.x = fmaf(f0, D[t][g].x, s.x);
                    s.y = fmaf(f1, D[t][g].y, s.y);
                    s.z = fmaf(f2, D[t][g].z, s.z);
                    s.w = fmaf(f3, D[t][g].w, s.w);
                } else {
                    s = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, cs[t].nm0, s, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, cs[t].nm1, s, 0, 0, 0);
                }
                acc[t][g] = s;
            }
        }
        sstore(1, buf ^ 1, sv);             // unused after the last iteration
        if (sb == NSB - 1 || !more) {       // the row block's sums: y, or a partial
            const long a0 = (long)rb * NSB;
            const bool own = A.whole || mf_owner(a0, A.T, A.G) == mf_owner(a0 + NSB - 1, A.T, A.G);
#pragma unroll
            for (int g = 0; g < NSG; g++) {
                const int s0 = 16 * g + 4 * kg;
#pragma unroll
                for (int t = 0; t < TL; t++) {
                    const int rr = 16 * (TL * wave + t) + (lane & 15);
                    const int row = rb * R + rr;
                    const float v4[4] = {acc[t][g].x, acc[t][g].y, acc[t][g].z, acc[t][g].w};
                    if (row < A.N) {
#pragma unroll
                        for (int v = 0; v < 4; v++) {
                            if (s0 + v >= A.B) continue;
                            if (own) A.y[(size_t)(s0 + v) * A.N + row] = v4[v];
                            else A.part[((size_t)(wg + rb) * 16 * NSG + s0 + v) * R + rr] = v4[v];
                        }
                    }
                    acc[t][g] = zero;
                }
            }
        }
        rb = rbn;
        sb = sbn;
        __syncthreads();
    }
}

// y of the row blocks that several workgroups share: their partial sums
// added in workgroup order (slot wg + rb, written by kq_mf_kernel).  One
// workgroup per (row block, 4 streams); a lane takes 4 consecutive rows and
// loads up to 8 partials at a time.
__global__ __launch_bounds__(256) void kq_mf_reduce_kernel(const float* part, float* y, int B, int N,
                                                          int NSG, int R, int NSB, long T, int G) {
    const int rb = blockIdx.x, s = 4 * blockIdx.y + (threadIdx.x >> 6), r = 4 * (threadIdx.x & 63);
    const long w0 = mf_owner((long)rb * NSB, T, G), w1 = mf_owner((long)rb * NSB + NSB - 1, T, G);
    if (w0 == w1 || s >= B || r >= R) return;
    const size_t stride = (size_t)16 * NSG * R;           // floats between slots
    const float4* p = reinterpret_cast<const float4*>(part + ((size_t)(w0 + rb) * 16 * NSG + s) * R + r);
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (long w = w0; w <= w1; w += 8) {
        float4 q[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
            q[i] = w + i <= w1 ? p[(size_t)(w - w0 + i) * (stride / 4)] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (w + i <= w1) {
                v.x = v.x + q[i].x; v.y = v.y + q[i].y; v.z = v.z + q[i].z; v.w = v.w + q[i].w;
            }
    }
    const float vv[4] = {v.x, v.y, v.z, v.w};
    const int row = rb * R + r;
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (row + i < N) y[(size_t)s * N + row + i] = vv[i];
}

template <int TYPE>
int launch_mfma_t(const float* x, const void* w, float* y, int B, int N, int K, void* planes,
                  float* xs, float* part, int grid, hipStream_t st) {
    const int NSG = (B + 15) / 16, NSB = K >> 8;
    if (NSG > 4 || grid < 1) return (int)hipErrorInvalidValue;
    MfSplitArg s;
    s.x = x; s.planes = static_cast<uint4*>(planes);
    s.side = reinterpret_cast<uint4*>(xs);
    s.B = B; s.K = K; s.NSG = NSG;
    hipLaunchKernelGGL(kq_mf_split_kernel, dim3((unsigned)(NSB * NSG)), dim3(256), 0, st, s);
    const MfPlan p = mf_plan(TYPE, NSG, N, K, grid);
    MfArg a;
    a.w = static_cast<const uint8_t*>(w);
    a.planes = static_cast<const uint4*>(planes);
    a.side = s.side; a.y = y; a.part = part;
    a.B = B; a.N = N; a.K = K; a.NSG = NSG;
    a.nrb = p.nrb; a.G = p.G; a.whole = p.whole; a.T = p.T;
    const size_t lds = (size_t)2 * mf_stage_u4(NSG) * 16;
    typedef void (*mf_fn)(MfArg);
    const mf_fn fn[4] = {&kq_mf_kernel<TYPE, 1>, &kq_mf_kernel<TYPE, 2>, &kq_mf_kernel<TYPE, 3>,
                         &kq_mf_kernel<TYPE, 4>};
    hipLaunchKernelGGL(fn[NSG - 1], dim3((unsigned)p.G), dim3(64 * MF_NW), lds, st, a);
    if (!p.whole)
        hipLaunchKernelGGL(kq_mf_reduce_kernel, dim3((unsigned)p.nrb, (unsigned)((B + 3) / 4)), dim3(256), 0,
                           st, (const float*)part, y, B, N, NSG, p.rows, NSB, p.T, p.G);
    return (int)hipGetLastError();
}

// --------------------------------------------------------------- dequant
// ------------------------------------------------- int8 MULTISEQ (MFMA)
// st_linear_multix under g_st.use_sdot for Q4_K / Q6_K, B >= 2
// (stratum_linear.h:732-907): every stream's x quantized as the
// single-stream int8 mode quantizes it (kq_mi8_prep_kernel), then per
// (row, stream) the reference's multix_pack arithmetic, bit for bit:
//  Q4_K (q4k_dot_rows2_sdot_multix_pack, stratum_q4k_neon.h:870-948): per
//    sub-block the binary32 term fl(fl(fl(d*sc) * fl(fl(L) * scl)) -
//    fl(fl(dmin*m) * fl(fl(S) * scl))), added to a binary64 sum in element
//    order (L the exact dot of the 4-bit values, S the group's int8 sum);
//  Q6_K (q6k_dot_rows2_sdot_multix_pack, stratum_q6k_neon.h:627-700): per
//    16-group ((double)d * sc * (double)scl) * (double)A in binary64, A the
//    exact dot of q - 32.
// The integer dots run on the matrix cores (v_mfma_i32_16x16x64_i8, exact
// in int32), the terms and the sequential binary64 sums on the VALU.
//
// Operands.  One MFMA: A = 16 rows of x operands (i), B = 16 weight rows
// (j), 64 k-values: lane l gives A[l % 16][16 (l/16) .. +15] and
// B[..][l % 16] for the same 16 k-values, so any assignment of the chunk's
// positions to (l / 16, byte) is summed correctly as long as A and B use the
// same one: here byte b of lane group q is chunk position 16q + b.
//  Q4_K: A row i = (stream i/2, sub-block i&1) holds that stream's x only
//    at the sub-block's positions (q >> 1 == i & 1), zero elsewhere, so
//    D[i][j] is the sub-block's dot: 8 streams x both sub-blocks per MFMA.
//  Q6_K: A row i = (stream i/4, run i&3) holds x only at run i&3's 16
//    positions (q == i & 3): 4 streams x the chunk's 4 runs per MFMA.
// D[i][j] lands in lane j + 16 (i/4), register i % 4: a lane holds its
// weight row's dots for 2 streams x 2 sub-blocks (Q4_K) or 1 stream x 4
// runs (Q6_K), in the order its binary64 sums need them.
//
// Work.  A wave owns 16 rows and SW streams for the whole row (the sums are
// sequential in k); a workgroup's 4 waves take 4 neighbouring row blocks
// with the same streams, whose quantized x and coefficients for one
// super-block are staged in LDS (double-buffered, one barrier per
// super-block) and read by all four.  Weights and staging data are loaded
// P super-blocks ahead into registers: the x, coefficient and weight loads
// of a super-block are issued together, so the in-order wait for one never
// waits on data needed later.
typedef int i32x4 __attribute__((ext_vector_type(4)));

struct Mi8Arg {
    const uint8_t* w;         // N rows of K weights (Q4_K / Q6_K blocks)
    const int8_t* xq;         // [B][K] quantized streams
    const uint8_t* zp;        // 64 zero bytes
    const uint8_t* cf;        // per (stream, group) coefficients: Q4_K float2
                              // {scl, fl(fl(S) * scl)} [B][K/32]; Q6_K double
                              // scl [B][K/16]
    float* y;                 // y[s * y_stride + r]
    long y_stride;
    int N, K, B;
    // grouped launches (the int8 MoE batch): blockIdx.y is group g < *ng of
    // the kq_moe_group_kernel records (runs of at most 8 members of one
    // expert); member slot j reads quantized row xi[j] and writes row
    // yi[j] of the group's y (stride y_stride); slots past M read row zrow
    // (all zero).  w and y above are unused.
    const MxGroup* groups;
    const int* ng;
    int zrow;
    int rbw;                  // 16-row blocks per workgroup (1 unless KS = 1)
    const float2* sm;         // grouped: {scale, sum} per (row, group)
    int pack2;                // grouped Q4_K: runs of two members on the VALU
};

// x -> int8 per group (the single-stream rule, kq_quantize_kernel's) and
// the coefficients the main kernel needs, one thread per (stream, group).
// Streams B .. bpad - 1 (the padding up to the main kernel's stream
// count) get zero values and coefficients, so their terms are 0.
// It also zeroes the 256-byte zero page zp.
template <int G>
__device__ __forceinline__ void mi8_prep_one(long gid, const float* x, long x_stride, int K,
                                             int B, int bpad, int8_t* xq, uint8_t* cf,
                                             uint8_t* zp, float2* sm) {
    const int ng = K / G;
    if (gid < 16) reinterpret_cast<uint4*>(zp)[gid] = make_uint4(0, 0, 0, 0);
    if (gid >= (long)ng * bpad) return;
    const int s = (int)(gid / ng), g = (int)(gid - (long)s * ng);
    const f32x4* src =
        reinterpret_cast<const f32x4*>(x + (size_t)min(s, B - 1) * x_stride) + (size_t)g * (G / 4);
    f32x4 v[G / 4];
#pragma unroll
    for (int k = 0; k < G / 4; k++) v[k] = s < B ? src[k] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < G / 4; k++)
        amax = fmaxf(fmaxf(fmaxf(amax, fabsf(v[k].x)), fmaxf(fabsf(v[k].y), fabsf(v[k].z))),
                     fabsf(v[k].w));
    const float scale = __fdiv_rn(amax, 127.0f);
    const float inv = scale > 0.0f ? __fdiv_rn(1.0f, scale) : 0.0f;
    int sum = 0;
    uint32_t* dst = reinterpret_cast<uint32_t*>(xq + (size_t)s * K + (size_t)g * G);
#pragma unroll
    for (int k = 0; k < G / 4; k++) {
        const float e[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int iv = min(127, max(-128, __float2int_rn(e[i] * inv)));
            sum += iv;
            w |= ((uint32_t)iv & 0xffu) << (8 * i);
        }
        dst[k] = w;
    }
    if (G == 32)
        reinterpret_cast<float2*>(cf)[gid] = make_float2(scale, (float)sum * scale);
    else
        reinterpret_cast<double*>(cf)[gid] = (double)scale;
    if (sm) sm[gid] = make_float2(scale, (float)sum);   // the single-stream form's {scale, sum}
}

template <int G>
__global__ __launch_bounds__(256) void kq_mi8_prep_kernel(const float* x, long x_stride, int K,
                                                          int B, int bpad, int8_t* xq,
                                                          uint8_t* cf, uint8_t* zp, float2* sm) {
    mi8_prep_one<G>((long)blockIdx.x * 256 + threadIdx.x, x, x_stride, K, B, bpad, xq, cf, zp, sm);
}

// The int8 MoE batch's set-up in one launch: workgroup 0 cuts the runs
// (moe_group_body, as kq_moe_group_kernel), the others quantize the x rows
// (256 groups each, as kq_mi8_prep_kernel).  256-lane workgroups: the
// quantizing is about 300 VALU instructions per group, so 1024-lane
// workgroups (four waves per SIMD on a few CUs) made it the longer part.
template <int G>
__global__ __launch_bounds__(256) void kq_mi8_moe_prep_kernel(MoeGroupArg ga, const float* x,
                                                               int K, int B, int bpad, int8_t* xq,
                                                               uint8_t* cf, uint8_t* zp,
                                                               float2* sm) {
    extern __shared__ __align__(16) int lds_i[];
    if (blockIdx.x == 0) {
        moe_group_body(ga, lds_i);
        return;
    }
    mi8_prep_one<G>((long)(blockIdx.x - 1) * 256 + threadIdx.x, x, (long)K, K, B, bpad, xq, cf,
                    zp, sm);
}

// A run of one member in a grouped launch (st_linear_multix at B = 1 is
// st_linear_dispatch): the single-stream int8 kernel's arithmetic, so the
// member equals kq_gemv_dev(type | KQ_INT8_ACT) bit for bit.  The T lanes
// take the 64-weight chunks of rows r0 .. r0 + 16 nrw - 1 in row-major
// order (neighbouring lanes read neighbouring chunks of a row), each chunk
// term exactly as kq_segs_kernel forms it (term_q4k_i8 / term_q6k_i8, x
// and {scale, sum} read from the quantized row xi), kept in LDS
// ([row][K/64] doubles), then that kernel's row reduction: GP =
// kq_phases(K/64) lanes per row, lane p sums chunks p, p+GP, ... in order
// from 0, then phase_tree.  Output y[r] (y: the member's row).
template <int TYPE>
__device__ __forceinline__ void mi8_single(const Mi8Arg& A, const uint8_t* w, int xi, float* y,
                                           int rb0, int nrw, double* terms, int tid, int T) {
    using C = Chunk<TYPE>;
    constexpr bool Q4 = TYPE == T_Q4K_I8;
    constexpr int BB = Q4 ? 144 : 210;
    const int N = A.N, K = A.K, NCH = K >> 6, nb = K >> 8;
    const int r0 = rb0 * 16, nr = min(16 * nrw, N - r0), nchk = nr * NCH;
    const uint8_t* xr = reinterpret_cast<const uint8_t*>(A.xq) + (size_t)xi * K;
    const float2* sr = A.sm + (size_t)xi * (Q4 ? K >> 5 : K >> 4);
    struct In { typename C::Raw r; uint4 x[4]; float s[8]; };
    auto ld = [&](int f, In& in) {
        const int fc = min(f, nchk - 1), rr = fc / NCH, c = fc - rr * NCH;
        const wptr blk = to_global(w) + (size_t)(r0 + rr) * nb * BB + (size_t)(c >> 2) * BB;
        in.r = C::load(blk, c & 3);
        if constexpr (Q4) {
            // chunk c: x[64c .. 64c+63], groups 2c, 2c+1
#pragma unroll
            for (int k = 0; k < 4; k++) in.x[k] = *reinterpret_cast<const uint4*>(xr + 64 * c + 16 * k);
            const float4 s4 = *reinterpret_cast<const float4*>(sr + 2 * c);
            in.s[0] = s4.x; in.s[1] = s4.y; in.s[2] = s4.z; in.s[3] = s4.w;
        } else {
            // chunk c = (block bi, half h, is): run t at 256 bi + 128 h + 32 t + 16 is
            const int bi = c >> 2, h = (c >> 1) & 1, is = c & 1;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int pos = 256 * bi + 128 * h + 32 * t + 16 * is;
                in.x[t] = *reinterpret_cast<const uint4*>(xr + pos);
                const float2 v = sr[pos >> 4];
                in.s[2 * t] = v.x; in.s[2 * t + 1] = v.y;
            }
        }
    };
    auto term = [&](int f, const In& in) {
        const int fc = min(f, nchk - 1), rr = fc / NCH, c = fc - rr * NCH;
        double t;
        if constexpr (Q4)
            t = term_q4k_i8(in.r, c & 3, reinterpret_cast<const uint32_t*>(in.x),
                            make_float4(in.s[0], in.s[1], in.s[2], in.s[3]));
        else
            t = term_q6k_i8(in.r, c & 3, reinterpret_cast<const uint32_t*>(in.x), in.s);
        if (f < nchk) terms[rr * NCH + c] = t;
    };
    // two batches in flight: the next one's loads go out before this one's term
    const int nit = (nchk + T - 1) / T;
    In a, b;
    ld(tid, a);
    for (int it = 0; it < nit; it += 2) {
        ld(tid + (it + 1) * T, b);
        term(tid + it * T, a);
        ld(tid + (it + 2) * T, a);
        if (it + 1 < nit) term(tid + (it + 1) * T, b);
    }
    __syncthreads();
    const int GP = kq_phases(NCH), lgp = GP == 32 ? 5 : 3;
    for (int task = tid; task < 16 * nrw * GP; task += T) {   // whole waves
        const int rho = task >> lgp, p = task & (GP - 1);
        const double* tr = terms + rho * NCH;
        double v = 0.0;
        for (int i = p; i < NCH; i += GP) v = v + tr[i];
        v = phase_tree(v, GP);
        if (p == 0 && rho < nr) y[r0 + rho] = (float)v;
    }
}

// A Q4_K run of two members in a grouped launch (KS = 1): the same values as
// the matrix-core form below (st_linear_multix's pack arithmetic), on the
// VALU.  Each lane takes one (row, member) of rows r0 .. r0 + 16 nrw - 1
// and walks the row's 64-weight chunks in order: the exact 4-bit x int8
// dots of the two sub-blocks (sdot4), then per sub-block the binary32 term
// fl(fl(d*sc) * fl(fl(L) * scl)) - fl(fl(dmin*m) * fl(fl(S)*scl)) added to
// the lane's binary64 sum, in element order.  The matrix-core form leaves
// three of its four lane groups on empty member slots for two members
// (their epilogue instructions run anyway); here every lane's term is a
// member's.  The two members' quantized rows and coefficients are staged in
// LDS (2.5 K bytes), read by the lanes as broadcasts.
__device__ __forceinline__ void mi8_pack2_q4k(const Mi8Arg& A, const MxGroup* gp, int rb0,
                                              int nrw, uint8_t* lds, int tid) {
    const int N = A.N, K = A.K, nb = K >> 8, ng = K >> 5;
    const int xr[2] = {gp->xi[0], gp->xi[1]};
    uint4* xs = reinterpret_cast<uint4*>(lds);                     // [2][K] int8
    float4* cs = reinterpret_cast<float4*>(lds + 2 * (size_t)K);   // [2][K/64] {c0, c1}
    const int s = tid & 1, rl = tid >> 1;
    const int r = rb0 * 16 + rl;
    const bool live = rl < 16 * nrw && r < N;
    const wptr row = to_global(gp->w) + (size_t)min(r, N - 1) * (size_t)nb * 144;
    // half a super-block per step (its header and 64 quant bytes: two
    // chunks), the next half's loads issued before this one's terms
    struct In { uint4 hd, q[4]; };
    auto ld = [&](int hs, In& in) {
        const int h = min(hs, 2 * nb - 1);
        const wptr blk = row + (size_t)(h >> 1) * 144;
        in.hd = ld16(blk);
#pragma unroll
        for (int i = 0; i < 4; i++) in.q[i] = ld16(blk + 16 + 64 * (h & 1) + 16 * i);
    };
    // the first half super-block's weights go out before the x staging,
    // which does not hold them up
    In a, b;
    ld(0, a);
    const int xq16 = K >> 4, nc2 = ng >> 1;
    for (int i = tid; i < 2 * xq16; i += 64) {
        const int m = i >= xq16, o = i - m * xq16;
        xs[i] = reinterpret_cast<const uint4*>(A.xq + (size_t)xr[m] * K)[o];
    }
    for (int i = tid; i < 2 * nc2; i += 64) {
        const int m = i >= nc2, o = i - m * nc2;
        cs[i] = reinterpret_cast<const float4*>(A.cf + (size_t)xr[m] * ng * 8)[o];
    }
    __syncthreads();
    const uint4* xm = xs + (size_t)s * xq16;
    const float4* cm = cs + (size_t)s * nc2;
    double acc = 0.0;
    auto step = [&](int hs, const In& in) {
        const float d = f16_bits_to_f32(in.hd.x & 0xffffu);
        const float dmin = f16_bits_to_f32(in.hd.x >> 16);
#pragma unroll
        for (int jj = 0; jj < 2; jj++) {
            const int j = 2 * (hs & 1) + jj, c = 2 * hs + jj;
            uint32_t sc1, mn1, sc2, mn2;
            scale_min_pair(in.hd.y, in.hd.z, in.hd.w, j, sc1, mn1, sc2, mn2);
            const float4 dm = make_float4(d * (float)sc1, dmin * (float)mn1, d * (float)sc2,
                                          dmin * (float)mn2);
            const uint4 q0 = in.q[2 * jj], q1 = in.q[2 * jj + 1];
            const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            const uint4 x0 = xm[4 * c], x1 = xm[4 * c + 1], x2 = xm[4 * c + 2], x3 = xm[4 * c + 3];
            const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            const uint32_t xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
            int L = 0, H = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                L = __builtin_amdgcn_sdot4((int)(q[k] & 0x0f0f0f0fu), (int)xl[k], L, false);
                H = __builtin_amdgcn_sdot4((int)((q[k] >> 4) & 0x0f0f0f0fu), (int)xh[k], H, false);
            }
            const float4 cf = cm[c];
            const float tl = dm.x * ((float)L * cf.x) - dm.y * cf.y;
            acc = acc + (double)tl;
            const float th = dm.z * ((float)H * cf.z) - dm.w * cf.w;
            acc = acc + (double)th;
        }
    };
    for (int hs = 0; hs < 2 * nb; hs += 2) {
        ld(hs + 1, b);
        step(hs, a);
        ld(hs + 2, a);
        step(hs + 1, b);
    }
    if (live) gp->y[(size_t)gp->yi[s] * A.y_stride + r] = (float)acc;
}

// Weight registers of one super-block of one lane's row.
//  Q4_K: the header and, of each chunk's 32 quant bytes, the half lane
//    group q reads (16 (q & 1) ..).
//  Q6_K (lane group q = run t): for each chunk u = (half h, is) the 16 ql
//    bytes run t takes its nibbles from (64h + 16is + 32 (t & 1)) and the
//    16 qh bytes (128 + 32h + 16is), each as 5 dwords from the dword-aligned
//    address below (realigned by sh: 210-byte blocks are only 2-byte
//    aligned); the 16 scale bytes and d.
struct Mi8W4 { uint4 hd, qv[4]; };
struct Mi8W6 { uint32_t l[4][5], h[4][5], s[5]; uint32_t d, sh; };

// Shape of one launch: SW streams per wave (8 streams x 2 sub-blocks per
// Q4_K MFMA, 4 streams x 4 runs per Q6_K MFMA), P super-blocks of loads in
// flight, and a workgroup of KS waves on one 16-row block, one K-part each.
// A wave needs no other wave until the end: its weights, its A operands
// (loaded per lane straight from the quantized streams; lanes whose A row
// is zero at their positions read the workspace's zero page) and its
// coefficients all come through its own register ring, and it stages the
// coefficients in its own LDS region (LDS operations of one wave complete
// in order, so no barrier).  The KS partial sums of a row are added in LDS
// in K-part order at the end: the binary64 sum is grouped by K-part -- a
// fixed order, like the single-stream kernel's phases (the result equals
// the reference's strictly sequential sum unless a binary64 re-association
// crosses a binary32 rounding boundary).
//
// GR (the int8 MoE batch, moe_forward_b under use_sdot,
// stratum_arch_moe.inc.c:1158-1201): one workgroup per (16-row block, run of
// one expert's members).  A run of two or more members takes
// st_linear_multix's pack arithmetic above, exactly as a kq_gemv_multix_dev
// call on that expert's slice would.  A run of one member takes the
// single-stream path (mi8_single): the member equals its
// kq_gemv_dev(type | KQ_INT8_ACT) result bit for bit.
// (Q4_K: four waves per SIMD asked of the register allocator, which the
// 16-stream forms reach with the A operands and coefficients out of the ring;
// Q6_K reaches three by itself, and asking for them makes it spill)
template <int TYPE, int SW, int P, int KS, bool GR>
__global__ __launch_bounds__(64 * KS) __attribute__((amdgpu_waves_per_eu(TYPE == T_Q4K_I8 ? 4 : 1)))
void kq_mi8_kernel(Mi8Arg A) {
    constexpr bool Q4 = TYPE == T_Q4K_I8;
    constexpr int NM = Q4 ? SW / 8 : SW / 4;        // MFMAs per chunk
    constexpr int NACC = Q4 ? 2 * NM : NM;          // binary64 sums per lane
    constexpr int CB = Q4 ? 64 : 128;               // coefficient bytes per stream and super-block
    constexpr int CU = SW * CB / 16, CPT = (CU + 63) / 64;
    constexpr int DEC = Q4 ? 16 * 4 * 16 : 0;       // Q4_K: decoded d*sc, dmin*m per (chunk, row)
    constexpr int WL = SW * CB + DEC;               // LDS bytes per wave
    constexpr int STAGE = KS * WL, COMB = KS * 64 * NACC * 8;
    __shared__ __align__(16) uint8_t lds[STAGE > COMB ? STAGE : COMB];
    using W = typename std::conditional<Q4, Mi8W4, Mi8W6>::type;

    const int tid = threadIdx.x, lane = tid & 63, kp = tid >> 6;
    const int q = lane >> 4, jr = lane & 15;
    const int N = A.N, K = A.K, nb = K >> 8;
    const int ng = Q4 ? K >> 5 : K >> 4;            // coefficient groups per stream
    const int s0 = GR ? 0 : blockIdx.y * SW;
    // row blocks rb0 .. rb0 + nrw - 1 (one after the other; KS = 1 only)
    const int rbw = KS == 1 ? A.rbw : 1;
    const int rb0 = blockIdx.x * rbw, nrw = min(rbw, (N + 15) / 16 - rb0);
    constexpr int BB = Q4 ? 144 : 210;
    const MxGroup* gp = nullptr;
    int M = SW;
    const uint8_t* wbase = A.w;
    if constexpr (GR) {
        gp = A.groups + blockIdx.y;               // read with the count (in bounds)
        const int ngv = *A.ng;
        M = gp->M;
        wbase = gp->w;
        if ((int)blockIdx.y >= ngv) return;       // uniform over the workgroup
    }
    // quantized row of member slot j (0 .. SW-1)
    auto xrow = [&](int j) -> long {
        if constexpr (GR) return j < M ? gp->xi[j] : A.zrow;
        return s0 + j;
    };
    if (GR && M == 1) {                           // uniform
        extern __shared__ __align__(16) double mi8_terms[];
        mi8_single<TYPE>(A, wbase, gp->xi[0], gp->y + (size_t)gp->yi[0] * A.y_stride, rb0, nrw,
                         mi8_terms, tid, 64 * KS);
        return;
    }
    if constexpr (GR && Q4 && KS == 1) {
        if (M == 2 && A.pack2) {                  // uniform
            extern __shared__ __align__(16) double mi8_terms[];
            mi8_pack2_q4k(A, gp, rb0, nrw, reinterpret_cast<uint8_t*>(mi8_terms), tid);
            return;
        }
    }
    // this lane's weight row in row block rb0 + i
    auto wrow = [&](int i) -> wptr {
        return to_global(wbase) + (size_t)min((rb0 + i) * 16 + jr, N - 1) * (size_t)nb * BB;
    };
    const int nbp = (nb + KS - 1) / KS;             // super-blocks per K-part
    const int kb0 = kp * nbp, kb1 = min(nb, kb0 + nbp);
    uint8_t* wl = lds + kp * WL;                    // this wave's LDS
    // (xq and cf hold a multiple of 16 streams: streams past B are zero;
    // zp is 64 zero bytes)
    const uint8_t* cf = A.cf;
    // this lane's A row holds x at its positions: Q4_K row (stream jr/2,
    // sub-block jr&1) at lane groups q >> 1 == jr & 1; Q6_K row (stream
    // jr/4, run jr&3) at lane group q == jr & 3.  Its x: stream sa + NS m,
    // chunk position offset qo; else the zero page.
    const bool on = Q4 ? (q >> 1) == (jr & 1) : q == (jr & 3);
    const int sa = Q4 ? jr >> 1 : jr >> 2, NS = Q4 ? 8 : 4;
    const uint8_t* xa[NM];
#pragma unroll
    for (int m = 0; m < NM; m++)
        xa[m] = reinterpret_cast<const uint8_t*>(A.xq) + (size_t)xrow(sa + NS * m) * K;
    const uint8_t* zp = A.zp;
    constexpr int CPS = CB / 16;                    // uint4 of coefficients per stream
    long crow[CPT];                                 // coefficient row of this lane's pieces
#pragma unroll
    for (int k = 0; k < CPT; k++) crow[k] = xrow(min(lane + 64 * k, CU - 1) / CPS);

    struct Slot { W w; };
    // the A operands (this lane's x bytes, or the zero page) and the
    // coefficients of super-block b: loaded at the step that uses them, not
    // through the ring (they come from L2, and keeping them out of the
    // ring's slots saves 2 x (4 x 4 NM + 4 CPT) registers a lane)
    auto loada = [&](int b, i32x4 (&av)[4][NM], uint4 (&cv)[CPT]) {
        const int bb = min(b, nb - 1);
#pragma unroll
        for (int k = 0; k < CPT; k++) {
            const int v = min(lane + 64 * k, CU - 1);
            cv[k] = *reinterpret_cast<const uint4*>(
                cf + ((size_t)crow[k] * ng + (size_t)bb * (CB / 8)) * 8 + 16 * (v % CPS));
        }
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int m = 0; m < NM; m++) {
                // chunk j's positions of this lane: Q4_K 64j + 16q; Q6_K run
                // q of chunk (h, is) at 128h + 32q + 16is
                const int qo = Q4 ? 64 * j + 16 * q : 128 * (j >> 1) + 32 * q + 16 * (j & 1);
                const uint8_t* src = on ? xa[m] + 256 * (size_t)bb + qo : zp;
                av[j][m] = *reinterpret_cast<const i32x4*>(src);
            }
    };
    auto load = [&](int i, int b, Slot& sl) {
        const wptr blk = wrow(i) + (size_t)b * BB;
        if constexpr (Q4) {
            sl.w.hd = ld16(blk);
#pragma unroll
            for (int j = 0; j < 4; j++) sl.w.qv[j] = ld16(blk + 16 + 32 * j + 16 * (q & 1));
        } else {
            const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(blk) & 3u;
            sl.w.sh = mis * 8u;
            const wptr b4 = blk - mis;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int h = u >> 1, is = u & 1;
                load5(b4 + 64 * h + 16 * is + 32 * (q & 1), sl.w.l[u]);
                load5(b4 + 128 + 32 * h + 16 * is, sl.w.h[u]);
            }
            // the scales' fifth dword only when 2 bytes off (else dword 3
            // again: the last block is never read past its 210 bytes)
            sl.w.s[0] = ld4(b4 + 192); sl.w.s[1] = ld4(b4 + 196);
            sl.w.s[2] = ld4(b4 + 200); sl.w.s[3] = ld4(b4 + 204);
            sl.w.s[4] = ld4(b4 + (mis ? 208 : 204));
            sl.w.d = ld2(blk + 208);
        }
    };
    double acc[NACC];
#pragma unroll
    for (int a = 0; a < NACC; a++) acc[a] = 0.0;
    const i32x4 zero = {0, 0, 0, 0};
    // A row block's end (KS = 1): its outputs, then the sums start again.
    auto finish = [&](int ib) {
        const int r = (rb0 + ib) * 16 + jr;
#pragma unroll
        for (int a = 0; a < NACC; a++) {
            const int so = Q4 ? 8 * (a >> 1) + 2 * q + (a & 1) : 4 * a + q;   // member slot
            if (r < N) {
                if constexpr (GR) {
                    if (so < M) gp->y[(size_t)gp->yi[so] * A.y_stride + r] = (float)acc[a];
                } else if (s0 + so < A.B) {
                    A.y[(size_t)(s0 + so) * A.y_stride + r] = (float)acc[a];
                }
            }
            acc[a] = 0.0;
        }
    };
    // A ring of R = P + 1 register slots: step t computes slot t % R and
    // reloads slot (t + P) % R, which step t - 1 finished with, for step
    // t + P.  Step t is row block t / nbp, super-block kb0 + t % nbp.  The
    // loop body is R steps with no exit (the steps past the end only
    // reload), so every slot keeps its registers around the loop and no
    // load in flight is waited for early to move one.
    constexpr int R = P + 1;
    const int nst = nrw * nbp;
    int ci = 0, cb = kb0;                           // this step's row block, super-block
    int li = 0, lb = kb0;                           // those of the step P ahead
    Slot ring[R];
#pragma unroll
    for (int p = 0; p < P; p++) {
        load(min(li, nrw - 1), min(lb, nb - 1), ring[p]);
        if (++lb == kb0 + nbp) { lb = kb0; li++; }
    }
    const int nit = (nst + R - 1) / R * R;
    for (int i0 = 0; i0 < nit; i0 += R) {
#pragma unroll
        for (int p = 0; p < R; p++) {
            const int b = cb, ib = ci;
            const Slot& cur = ring[p];
            const bool go = i0 + p < nst && b < kb1;               // uniform
            const bool last = KS == 1 && go && b == nb - 1;        // a row block's end
            if (++cb == kb0 + nbp) { cb = kb0; ci++; }
            // this step's A operands, then the next slot's loads: waiting
            // for this step's data then leaves the latter in flight
            i32x4 av[4][NM];
            uint4 cv[CPT];
            loada(b, av, cv);
            load(min(li, nrw - 1), min(lb, nb - 1), ring[(p + P) % R]);
            if (++lb == kb0 + nbp) { lb = kb0; li++; }
            if (go) {
                // the coefficients into this wave's LDS (unconditional
                // stores: a lane past the last piece stores it again)
                constexpr int CPS = CB / 16;
#pragma unroll
                for (int k = 0; k < CPT; k++) {
                    const int v = min(lane + 64 * k, CU - 1);
                    *reinterpret_cast<uint4*>(wl + CB * (v / CPS) + 16 * (v % CPS)) = cv[k];
                }
                if constexpr (Q4) {
                    // lane group q decodes chunk q of its row: d*sc, dmin*m of
                    // sub-blocks 2q, 2q+1 (shared with the other groups)
                    const float d = f16_bits_to_f32(cur.w.hd.x & 0xffffu);
                    const float dmin = f16_bits_to_f32(cur.w.hd.x >> 16);
                    uint32_t sc1, mn1, sc2, mn2;
                    scale_min_pair(cur.w.hd.y, cur.w.hd.z, cur.w.hd.w, q, sc1, mn1, sc2, mn2);
                    *reinterpret_cast<float4*>(wl + SW * CB + 16 * (16 * q + jr)) =
                        make_float4(d * (float)sc1, dmin * (float)mn1, d * (float)sc2,
                                    dmin * (float)mn2);
                }
            }
            if (!go) continue;
            if constexpr (Q4) {
                const uint32_t sh = 4u * (uint32_t)(q >> 1);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float4 dm = *reinterpret_cast<const float4*>(wl + SW * CB + 16 * (16 * j + jr));
                    const uint4 qv = cur.w.qv[j];
                    const i32x4 bop = {(int)((qv.x >> sh) & 0x0f0f0f0fu),
                                       (int)((qv.y >> sh) & 0x0f0f0f0fu),
                                       (int)((qv.z >> sh) & 0x0f0f0f0fu),
                                       (int)((qv.w >> sh) & 0x0f0f0f0fu)};
#pragma unroll
                    for (int m = 0; m < NM; m++) {
                        const i32x4 D = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[j][m], bop, zero,
                                                                              0, 0, 0);
                        // D[2e + sb]: stream 8m + 2q + e, sub-block sb
#pragma unroll
                        for (int e = 0; e < 2; e++) {
                            const float4 c = *reinterpret_cast<const float4*>(
                                wl + 64 * (8 * m + 2 * q + e) + 16 * j);
                            const float tl = dm.x * ((float)D[2 * e] * c.x) - dm.y * c.y;
                            acc[2 * m + e] = acc[2 * m + e] + (double)tl;
                            const float th = dm.z * ((float)D[2 * e + 1] * c.z) - dm.w * c.w;
                            acc[2 * m + e] = acc[2 * m + e] + (double)th;
                        }
                    }
                    // one chunk at a time: hoisting the next chunk's LDS
                    // reads over this one only costs registers
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
                const double d = (double)f16_bits_to_f32(cur.w.d);
                uint32_t S[4];
#pragma unroll
                for (int k = 0; k < 4; k++)
                    S[k] = __builtin_amdgcn_alignbit(cur.w.s[k + 1], cur.w.s[k], cur.w.sh);
                const uint32_t tsh = 4u * (uint32_t)(q >> 1), hsh = 2u * (uint32_t)q;
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int h = u >> 1, is = u & 1;
                    // this row's d * sc for the chunk's four runs (scale 8h + is + 2t)
                    double ds[4];
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const int g = 8 * h + is + 2 * t;
                        ds[t] = d * (double)(int8_t)(uint8_t)(S[g >> 2] >> (8 * (g & 3)));
                    }
                    uint32_t bw[4];
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const uint32_t L = __builtin_amdgcn_alignbit(cur.w.l[u][k + 1], cur.w.l[u][k], cur.w.sh);
                        const uint32_t H = __builtin_amdgcn_alignbit(cur.w.h[u][k + 1], cur.w.h[u][k], cur.w.sh);
                        const uint32_t v = ((L >> tsh) & 0x0f0f0f0fu) | (((H >> hsh) & 0x03030303u) << 4);
                        bw[k] = ((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u;   // bytes v - 32
                    }
                    const i32x4 bop = {(int)bw[0], (int)bw[1], (int)bw[2], (int)bw[3]};
#pragma unroll
                    for (int m = 0; m < NM; m++) {
                        const i32x4 D = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[u][m], bop, zero,
                                                                              0, 0, 0);
                        // D[t]: stream 4m + q, run t
                        const double* cs = reinterpret_cast<const double*>(wl + 128 * (4 * m + q));
#pragma unroll
                        for (int t = 0; t < 4; t++)
                            acc[m] = acc[m] + ds[t] * cs[8 * h + is + 2 * t] * (double)D[t];
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            if (last) finish(ib);
        }
    }
    if (KS == 1) return;
    // KS > 1: one row block (rb0)
    // the K-parts' partial sums, added in K-part order
    double* part = reinterpret_cast<double*>(lds);
    if (KS > 1) {
        __syncthreads();
#pragma unroll
        for (int a = 0; a < NACC; a++) part[(kp * 64 + lane) * NACC + a] = acc[a];
        __syncthreads();
        if (kp != 0) return;
#pragma unroll
        for (int a = 0; a < NACC; a++) {
            double v = part[lane * NACC + a];
#pragma unroll
            for (int k = 1; k < KS; k++) v = v + part[(k * 64 + lane) * NACC + a];
            acc[a] = v;
        }
    }
    finish(0);
}

// Bit-exact dequantization, one lane per 64-weight chunk (64 floats out).
template <int TYPE>
__global__ __launch_bounds__(256) void kq_dequant_kernel(const uint8_t* __restrict__ w,
                                                         float* __restrict__ y, long nchunks) {
    using TI = TypeInfo<TYPE>;
    const long f = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= nchunks) return;
    const wptr blk = to_global(w) + (size_t)(f >> 2) * TI::BB;
    const int u = (int)(f & 3);
    float* yb = y + (size_t)(f >> 2) * 256;
    if (TYPE == T_Q4K) {
        const RawQ4 r = load_q4k(blk, u);
        const float d = f16_bits_to_f32(r.hd.x & 0xffffu);
        const float dmin = f16_bits_to_f32(r.hd.x >> 16);
        const wptr s = blk + 4;
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
    } else if (TYPE == T_Q5K) {
        // stratum_q5k.h:18-42: y = fl(fl(d*sc)*q) - fl(dmin*m), q 5 bits
        const float d = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        const float dmin = f16_bits_to_f32((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
        const wptr s = blk + 4;
#pragma unroll
        for (int half = 0; half < 2; half++) {
            const int sb = 2 * u + half;
            uint32_t sc, m;
            if (sb < 4) { sc = s[sb] & 63u; m = s[sb + 4] & 63u; }
            else { sc = (s[sb + 4] & 15u) | ((uint32_t)(s[sb - 4] >> 6) << 4);
                   m = ((uint32_t)s[sb + 4] >> 4) | ((uint32_t)(s[sb] >> 6) << 4); }
            const float ds = d * (float)sc, dm = dmin * (float)m;
            for (int l = 0; l < 32; l++) {
                const uint32_t v = blk[48 + 32 * u + l];
                const uint32_t q = (half ? (v >> 4) : (v & 15u)) + (((uint32_t)blk[16 + l] >> sb) & 1u) * 16u;
                yb[32 * sb + l] = ds * (float)q - dm;
            }
        }
    } else if (TYPE == T_Q3K) {
        // stratum_q3k.h:30-56: y = fl(fl(d*(sc-32))*q3), chunk u = (s, h)
        const float d = f16_bits_to_f32((uint32_t)blk[108] | ((uint32_t)blk[109] << 8));
        const int s = u >> 1, h = u & 1;
        for (int j = 0; j < 4; j++) {
            const int g = 8 * s + 2 * j + h, w = g >> 2, bi = g & 3;
            const uint32_t lo = (w & 1) ? blk[100 + bi] : blk[96 + bi];
            const uint32_t nib = (w & 2) ? (lo >> 4) : (lo & 15u);
            const uint32_t hi2 = ((uint32_t)blk[104 + bi] >> (2 * w)) & 3u;
            const float dl = d * (float)((int)(nib | (hi2 << 4)) - 32);
            for (int l = 0; l < 16; l++) {
                const int q = (int)(((uint32_t)blk[32 + 32 * s + 16 * h + l] >> (2 * j)) & 3u) -
                              ((((uint32_t)blk[16 * h + l] >> (4 * s + j)) & 1u) ? 0 : 4);
                yb[128 * s + 32 * j + 16 * h + l] = dl * (float)q;
            }
        }
    } else if (TYPE == T_Q80) {
        // stratum_q8_0.h:14-17, blocks 2u and 2u+1 of the 256-weight unit
        for (int half = 0; half < 2; half++) {
            const wptr bp = blk + 68 * u + 34 * half;
            const float d = f16_bits_to_f32((uint32_t)bp[0] | ((uint32_t)bp[1] << 8));
            for (int k = 0; k < 32; k++)
                yb[64 * u + 32 * half + k] = d * (float)(int8_t)bp[2 + k];
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

// --------------------------------------------------------- dense rows
// F16 and F32 tensors (st_linear_f16 / st_linear_f32, stratum_linear.h:
// 491-512).  Every product w * x is exact in binary64 (11 or 24 bits times
// 24), so y is the binary64 sum of exact products rounded once; the
// reference sums F16 rows in element order (a different binary64 grouping,
// at most one binary32 ulp apart after the final rounding) and hands F32
// to cblas_sgemv.  A wave takes a row; lane i takes elements
// [E i + 64 E m, +E) of step m (E = 4 for F32, 8 for F16: one 16-byte load,
// a wave reads 1 KB of the row per step), summed in increasing m, and the
// 64 lane sums are combined by a fixed butterfly: the order depends on K
// only.  Rows go to waves w, w + 4G, ... of G workgroups of 256 lanes
// (G at most N / 4, rounded up).
constexpr int T_F32 = 0, T_F16 = 1;
constexpr int DENSE_XLDS_MAX = 16384;   // x staged in LDS up to this K

struct DenseArg {
    const uint8_t* w;
    const float* x;
    const float* add;
    float* y;
    long row_bytes;
    int N, K;
    int B;               // streams: x is B x K, y is B x N (add only for B == 1)
};

// streams per workgroup pass of the dense multi-stream kernel
constexpr int DENSE_SB = 8;

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int lo = __shfl_xor(__double2loint(v), off);
        const int hi = __shfl_xor(__double2hiint(v), off);
        v = v + __hiloint2double(hi, lo);
    }
    return v;
}

// One wave per row; lane l takes elements E*l + 64*E*i in order, the 64
// partial sums meet in a fixed butterfly, so the result does not depend on
// the grid.  SB streams (blockIdx.y selects the group of SB) share each
// weight load; every stream's sum runs in the single-stream order.
template <int TYPE, bool XLDS, int SB>
__global__ __launch_bounds__(256) void kq_dense_kernel(DenseArg a) {
    extern __shared__ __align__(16) float xl[];
    constexpr int E = TYPE == T_F32 ? 4 : 8;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = a.K;
    const int s0 = blockIdx.y * SB;
    const int nb = min(SB, a.B - s0);
    const float* xg = a.x + (size_t)s0 * K;
    if (XLDS) {
        // eight loads in flight per lane before their stores; the index is
        // clamped so the loads need no branch
        const int n4 = nb * K / 4;
        const float4* xg4 = reinterpret_cast<const float4*>(xg);
        float4* xl4 = reinterpret_cast<float4*>(xl);
        for (int i0 = tid; i0 < n4; i0 += 256 * 8) {
            float4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = xg4[min(i0 + 256 * j, n4 - 1)];
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (i0 + 256 * j < n4) xl4[i0 + 256 * j] = v[j];
        }
        __syncthreads();
    }
    const float* xs = XLDS ? xl : xg;
    for (int r = blockIdx.x * 4 + wave; r < a.N; r += gridDim.x * 4) {
        const wptr row = to_global(a.w) + (size_t)r * a.row_bytes;
        double acc[SB];
#pragma unroll
        for (int s = 0; s < SB; s++) acc[s] = 0.0;
        for (int m = 0; m < K; m += 64 * E) {
            const int e0 = m + E * lane;
            if (e0 < K) {                       // F16 rows of K % 512 == 256 end half-way
                const uint4 v = ld16(row + (size_t)e0 * (TYPE == T_F32 ? 4 : 2));
                const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int q = 0; q < E / 4; q++) {
                    float wf[4];
                    if (TYPE == T_F32) {
                        wf[0] = __uint_as_float(wv[0]); wf[1] = __uint_as_float(wv[1]);
                        wf[2] = __uint_as_float(wv[2]); wf[3] = __uint_as_float(wv[3]);
                    } else {
                        wf[0] = f16_bits_to_f32(wv[2 * q] & 0xffffu);
                        wf[1] = f16_bits_to_f32(wv[2 * q] >> 16);
                        wf[2] = f16_bits_to_f32(wv[2 * q + 1] & 0xffffu);
                        wf[3] = f16_bits_to_f32(wv[2 * q + 1] >> 16);
                    }
#pragma unroll
                    for (int s = 0; s < SB; s++) {
                        if (s < nb) {
                            const float4 xv =
                                *reinterpret_cast<const float4*>(xs + (size_t)s * K + e0 + 4 * q);
                            acc[s] = fma((double)wf[0], (double)xv.x, acc[s]);   // exact product
                            acc[s] = fma((double)wf[1], (double)xv.y, acc[s]);
                            acc[s] = fma((double)wf[2], (double)xv.z, acc[s]);
                            acc[s] = fma((double)wf[3], (double)xv.w, acc[s]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int s = 0; s < SB; s++) {
            if (s < nb) {
                const double t = wave_sum_f64(acc[s]);
                if (lane == 0) {
                    float v = (float)t;
                    if (SB == 1 && a.add) v = a.add[r] + v;
                    a.y[(size_t)(s0 + s) * a.N + r] = v;
                }
            }
        }
    }
}

// dense dequant: F16 widened, F32 copied (4 values per lane)
__global__ __launch_bounds__(256) void kq_dense_dequant_kernel(const uint8_t* w, float* y, long n,
                                                               int type) {
    const long i = 4 * ((long)blockIdx.x * 256 + threadIdx.x);
    if (i >= n) return;
    const wptr p = to_global(w);
    if (type == T_F32) {
        const uint4 v = ld16(p + 4 * i);
        y[i] = __uint_as_float(v.x); y[i + 1] = __uint_as_float(v.y);
        y[i + 2] = __uint_as_float(v.z); y[i + 3] = __uint_as_float(v.w);
    } else {
        const uint2 v = ld8a4(p + 2 * i);
        y[i] = f16_bits_to_f32(v.x & 0xffffu); y[i + 1] = f16_bits_to_f32(v.x >> 16);
        y[i + 2] = f16_bits_to_f32(v.y & 0xffffu); y[i + 3] = f16_bits_to_f32(v.y >> 16);
    }
}

// ------------------------------------------------------ MoE FFN step
// Softmax of one row of E values per workgroup (stratum_softmax_inplace,
// stratum_engine.h:395-423): max as the sequential scan takes it (a NaN
// first value stays the max; later NaNs never replace it), e = expf(x -
// max) per value, the binary64 sum in index order by one lane (the
// reference's order), inv = (float)(1.0 / sum), x = e * inv.  expf is the
// device's (within 1 ulp of a correctly rounded exp).
__global__ __launch_bounds__(256) void kq_softmax_kernel(float* x, int E) {
    extern __shared__ __align__(16) float sm[];          // E values + 64 for the max
    float* row = x + (size_t)blockIdx.x * E;
    const int tid = threadIdx.x;
    float m = -INFINITY;
    for (int i = tid; i < E; i += 256) {
        const float v = row[i];
        sm[i] = v;
        m = fmaxf(m, v);                                 // NaN-ignoring
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
    float* wm = sm + ((E + 3) & ~3);
    if ((tid & 63) == 0) wm[tid >> 6] = m;
    __syncthreads();
    float maxv = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    if (isnan(sm[0])) maxv = sm[0];
    __syncthreads();
    for (int i = tid; i < E; i += 256) sm[i] = expf(sm[i] - maxv);
    __syncthreads();
    if (tid == 0) {
        double sum = 0.0;
        int i = 0;
        for (; i + 4 <= E; i += 4) {
            const float4 v = *reinterpret_cast<const float4*>(sm + i);
            sum = sum + (double)v.x; sum = sum + (double)v.y;
            sum = sum + (double)v.z; sum = sum + (double)v.w;
        }
        for (; i < E; i++) sum = sum + (double)sm[i];
        wm[0] = (float)(1.0 / sum);
    }
    __syncthreads();
    const float inv = wm[0];
    for (int i = tid; i < E; i += 256) row[i] = sm[i] * inv;
}

// SwiGLU (stratum_swiglu, stratum_engine.h:373-392, the scalar loop):
// y = (g / (1 + expf(-g))) * u, binary32 throughout, 4 values per lane.
__global__ __launch_bounds__(256) void kq_swiglu_kernel(const float* g, const float* u, float* y,
                                                        long n) {
    const long i = 4 * ((long)blockIdx.x * 256 + threadIdx.x);
    if (i + 4 <= n) {
        const float4 gv = *reinterpret_cast<const float4*>(g + i);
        const float4 uv = *reinterpret_cast<const float4*>(u + i);
        float4 o;
        o.x = (gv.x / (1.0f + expf(-gv.x))) * uv.x;
        o.y = (gv.y / (1.0f + expf(-gv.y))) * uv.y;
        o.z = (gv.z / (1.0f + expf(-gv.z))) * uv.z;
        o.w = (gv.w / (1.0f + expf(-gv.w))) * uv.w;
        *reinterpret_cast<float4*>(y + i) = o;
    } else {
        for (long j = i; j < n; j++) y[j] = (g[j] / (1.0f + expf(-g[j]))) * u[j];
    }
}

// Weighted accumulate in rank order plus the residual (batch 1:
// stratum_arch_moe.inc.c:728-743; batches: :1213-1226): for token s and
// element i, acc = 0; for r < k with sel >= 0: acc = acc + selw[r] * o[r][i]
// (product and sum rounded separately); x = resid + acc.  o is the down
// output of member s*k + r (B*k rows of H).
__global__ __launch_bounds__(256) void kq_moe_combine_kernel(const float* o, const int* sel,
                                                             const float* selw,
                                                             const float* resid, float* x, int k,
                                                             int H) {
    const int s = blockIdx.y;
    const int i = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (i >= H) return;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int r = 0; r < k; r++) {
        if (sel[s * k + r] < 0) continue;
        const float w = selw[s * k + r];
        const float4 v = *reinterpret_cast<const float4*>(o + ((size_t)s * k + r) * H + i);
        acc.x = acc.x + w * v.x; acc.y = acc.y + w * v.y;
        acc.z = acc.z + w * v.z; acc.w = acc.w + w * v.w;
    }
    const float4 rv = *reinterpret_cast<const float4*>(resid + (size_t)s * H + i);
    *reinterpret_cast<float4*>(x + (size_t)s * H + i) =
        make_float4(rv.x + acc.x, rv.y + acc.y, rv.z + acc.z, rv.w + acc.w);
}

// Q2_K (84 B) -> type 42 (148 B), one lane per output dword: dwords 0-3
// the scales, 4-35 the nibbles (weight p of the block, the 2-bit field
// (p % 128) / 32 of qs byte 32 (p / 128) + p % 32, goes to byte
// 16 + 16 (p / 32) + p % 16, low nibble for p % 32 < 16), 36 d and dmin
// (tools_gguf_nib_convert.c:99-120).
__global__ __launch_bounds__(256) void kq_q2k_to_nib_kernel(const uint32_t* q, uint32_t* o,
                                                            long nblocks) {
    const long t = (long)blockIdx.x * 256 + threadIdx.x;
    if (t >= nblocks * 37) return;
    const long b = t / 37;
    const int w = (int)(t - b * 37);
    const uint32_t* src = q + b * 21;
    uint32_t v;
    if (w < 4) {
        v = src[w];
    } else if (w == 36) {
        v = src[20];
    } else {
        const int grp = (w - 4) >> 2, l0 = 4 * ((w - 4) & 3), sh = 2 * (grp & 3);
        const uint32_t lo = src[4 + 8 * (grp >> 2) + (l0 >> 2)];       // qs bytes l0 .. l0+3
        const uint32_t hi = src[4 + 8 * (grp >> 2) + 4 + (l0 >> 2)];   // qs bytes l0+16 ..
        v = ((lo >> sh) & 0x03030303u) | (((hi >> sh) & 0x03030303u) << 4);
    }
    o[b * 37 + w] = v;
}

// x -> int8 per group of G (32: q4k_quantize_x_q8 + q4k_sum_i8_32; 16:
// q6k_quantize_x_q8_g16 + q6k_xsum16_i8), the arithmetic of store_i8: one
// lane per group.
template <int G>
__global__ __launch_bounds__(256) void kq_quantize_kernel(const float* x, int ngroups, int8_t* xq,
                                                          float* xscale, int* xsum) {
    const int g = blockIdx.x * 256 + threadIdx.x;
    if (g >= ngroups) return;
    const f32x4* src = reinterpret_cast<const f32x4*>(x) + (size_t)g * (G / 4);
    f32x4 v[G / 4];
#pragma unroll
    for (int q = 0; q < G / 4; q++) v[q] = src[q];
    float amax = 0.0f;
#pragma unroll
    for (int q = 0; q < G / 4; q++)
        amax = fmaxf(fmaxf(fmaxf(amax, fabsf(v[q].x)), fmaxf(fabsf(v[q].y), fabsf(v[q].z))),
                     fabsf(v[q].w));
    const float scale = __fdiv_rn(amax, 127.0f);
    const float inv = scale > 0.0f ? __fdiv_rn(1.0f, scale) : 0.0f;
    int sum = 0;
    uint32_t* dst = reinterpret_cast<uint32_t*>(xq + (size_t)g * G);
#pragma unroll
    for (int q = 0; q < G / 4; q++) {
        const float e[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int iv = min(127, max(-128, __float2int_rn(e[i] * inv)));
            sum += iv;
            w |= ((uint32_t)iv & 0xffu) << (8 * i);
        }
        dst[q] = w;
    }
    xscale[g] = scale;
    if (xsum) xsum[g] = sum;
}

template <int TYPE>
int launch_dequant(const uint8_t* w, float* y, long nblocks, hipStream_t st) {
    const long nch = nblocks * 4;
    const long grid = (nch + 255) / 256;
    hipLaunchKernelGGL(kq_dequant_kernel<TYPE>, dim3((unsigned)grid), dim3(256), 0, st, w, y, nch);
    return (int)hipGetLastError();
}

}  // namespace

// ------------------------------------------------------ static scratch
// Device memory for the entry point that allocates nothing
// (kq_gemv_multix_mfma_noalloc_dev): its workspace -- x planes, x sums and
// K-part partials -- lives in this array instead of a library allocation.
// Every GPU the library runs on holds its own copy, at its own address,
// until the process ends.  Host code never passes `scratch` itself (in host
// code the name is a host-side stand-in, not a device address): it uses the
// address hipGetSymbolAddress returns for the current device, looked up
// once per device and kept in scratch_dev[].  Calls that overlap on one GPU
// share the array and race; every byte a launch reads is written by that
// launch first, so nothing needs clearing between calls.
static __device__ __align__(256) uint8_t scratch[KQK_NOALLOC_BYTES];

namespace {
constexpr int SCRATCH_MAX_DEVICES = 64;
void* scratch_dev[SCRATCH_MAX_DEVICES];
}  // namespace

// ------------------------------------------------------------ C launchers
extern "C" {

int kqk_noalloc_scratch(void** ptr, long* bytes) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= SCRATCH_MAX_DEVICES) return (int)hipErrorInvalidDevice;
    if (!scratch_dev[dev]) {                  // first use on this device (it is current)
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p) return (int)hipErrorInvalidSymbol;
        scratch_dev[dev] = p;
    }
    *ptr = scratch_dev[dev];
    *bytes = (long)KQK_NOALLOC_BYTES;
    return 0;
}

// Host view of one segment (plain C layout, mirrored in kq_linear.c):
// nparts parts, part p = rows [start[p], start[p] + rows[p]) at w[p],
// writing y[p] (+ add[p]); x, or x + p * x_stride when x_stride != 0.

static long seg_rows(const kqk_seg& g) {
    long n = 0;
    for (int p = 0; p < g.nparts; p++) n += g.rows[p];
    return n;
}

static int xs_per_chunk(int type) {
    switch (type) {
    case T_Q4K: return TypeInfo<T_Q4K>::XS_PER_CHUNK;
    case T_Q6K: return TypeInfo<T_Q6K>::XS_PER_CHUNK;
    case T_Q2K: return TypeInfo<T_Q2K>::XS_PER_CHUNK;
    case T_NIB: return TypeInfo<T_NIB>::XS_PER_CHUNK;
    case T_Q5K: return TypeInfo<T_Q5K>::XS_PER_CHUNK;
    case T_Q3K: return TypeInfo<T_Q3K>::XS_PER_CHUNK;
    case T_Q80: return TypeInfo<T_Q80>::XS_PER_CHUNK;
    case T_Q4K_I8: return TypeInfo<T_Q4K_I8>::XS_PER_CHUNK;
    case T_Q6K_I8: return TypeInfo<T_Q6K_I8>::XS_PER_CHUNK;
    case T_Q5K_I8: return TypeInfo<T_Q5K_I8>::XS_PER_CHUNK;
    case T_Q3K_I8: return TypeInfo<T_Q3K_I8>::XS_PER_CHUNK;
    case T_Q80_I8: return TypeInfo<T_Q80_I8>::XS_PER_CHUNK;
    default: return -1;
    }
}

static int block_bytes_of(int type) {
    switch (type) {
    case T_Q4K: return TypeInfo<T_Q4K>::BB;
    case T_Q6K: return TypeInfo<T_Q6K>::BB;
    case T_Q2K: return TypeInfo<T_Q2K>::BB;
    case T_NIB: return TypeInfo<T_NIB>::BB;
    case T_Q5K: return TypeInfo<T_Q5K>::BB;
    case T_Q3K: return TypeInfo<T_Q3K>::BB;
    case T_Q80: return TypeInfo<T_Q80>::BB;
    case T_Q4K_I8: return TypeInfo<T_Q4K_I8>::BB;
    case T_Q6K_I8: return TypeInfo<T_Q6K_I8>::BB;
    case T_Q5K_I8: return TypeInfo<T_Q5K_I8>::BB;
    case T_Q3K_I8: return TypeInfo<T_Q3K_I8>::BB;
    case T_Q80_I8: return TypeInfo<T_Q80_I8>::BB;
    default: return 0;
    }
}

// index of a type's single-type instantiations (k_segs, k_segs_sel), or -1
static int type_slot(int type) {
    switch (type) {
    case T_Q4K: return 0;
    case T_Q6K: return 1;
    case T_Q2K: return 2;
    case T_NIB: return 3;
    case T_Q5K: return 5;
    case T_Q3K: return 6;
    case T_Q80: return 7;
    case T_Q4K_I8: return 8;
    case T_Q6K_I8: return 9;
    case T_Q5K_I8: return 10;
    case T_Q3K_I8: return 11;
    case T_Q80_I8: return 12;
    default: return -1;
    }
}

static void magic_for(uint32_t d, uint32_t& m, int& l) {
    if (d <= 1) { m = 0; l = 0; return; }
    l = 0;
    while ((1ull << l) < d) l++;
    m = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
}

// LDS plan of a segment list for `grid` workgroups: x region, xs region and
// term region sized for the largest segment.  Returns total bytes or -1.
long kqk_segs_lds(const kqk_seg* segs, int nseg, int grid, int* xs_off, int* terms_off,
                  int* scr_off) {
    long xl = 0, xsb = 0, tb = 0;
    for (int i = 0; i < nseg; i++) {
        const kqk_seg& g = segs[i];
        const int xpc = xs_per_chunk(g.type);
        if (xpc < 0 || g.K <= 0 || (g.K & 255) || g.nparts < 1 || g.nparts > MAXG)
            return -1;
        bool equal = true;
        for (int p = 0; p < g.nparts; p++) {
            if (g.rows[p] < 1) return -1;
            equal = equal && g.rows[p] == g.rows[0];
        }
        if (g.nparts > LIST_MAX && !equal) return -1;   // many parts must be equal
        const long N = seg_rows(g);
        if (N > 0x7fffffffL) return -1;
        const long NC = g.K >> 6;
        const long ngx = g.x_stride && g.nparts > 1 ? g.nparts : 1;
        const long xb = ngx * NC * ((g.type & T_I8) ? XPAD_I8 : XPAD) * 16;   // int8: 80 B/chunk
        xl = xl > xb ? xl : xb;
        xsb = xsb > ngx * NC * xpc * 4 ? xsb : ngx * NC * xpc * 4;
        const long R = (N + grid - 1) / grid;
        tb = tb > R * NC * 8 ? tb : R * NC * 8;
        if (g.probs) {                       // routing scratch (wg_topk) in the terms region
            if (!g.sel_out || g.emax < 1 || g.emax > 1024 || g.ksel < 1 || g.ksel > MAXG) return -1;
            tb = tb > ROUTE_BYTES ? tb : ROUTE_BYTES;
        }
    }
    xsb = (xsb + 15) & ~15L;
    *xs_off = (int)xl;
    *terms_off = (int)(xl + xsb);
    *scr_off = (int)(xl + xsb + tb);
    return xl + xsb + tb + SCR_BYTES;
}

// Every instantiation, indexed by [multi][depth - 1][slot]: slots 0..3 and
// 5..7 single types (type_slot), 4 Q4_K and Q6_K mixed, 8..12 the int8
// mode of Q4_K, Q6_K, Q5_K, Q3_K and Q8_0, 13 int8 Q4_K and Q6_K mixed.
constexpr int NSLOT = 14;
#define KQ_SEGS_ROW(D, M)                                                       \
    {&kq_segs_kernel<D, TB_Q4K, M>, &kq_segs_kernel<D, TB_Q6K, M>,              \
     &kq_segs_kernel<D, TB_Q2K, M>, &kq_segs_kernel<D, TB_NIB, M>,              \
     &kq_segs_kernel<1, TB_Q46, M>, &kq_segs_kernel<D, TB_Q5K, M>,              \
     &kq_segs_kernel<D, TB_Q3K, M>, &kq_segs_kernel<D, TB_Q80, M>,              \
     &kq_segs_kernel<D, TB_Q4K_I8, M>, &kq_segs_kernel<D, TB_Q6K_I8, M>,        \
     &kq_segs_kernel<D, TB_Q5K_I8, M>, &kq_segs_kernel<D, TB_Q3K_I8, M>,        \
     &kq_segs_kernel<D, TB_Q80_I8, M>, &kq_segs_kernel<1, TB_I8MIX, M>}
typedef void (*segs_fn)(SegsArg);
static const segs_fn k_segs[2][2][NSLOT] = {{KQ_SEGS_ROW(1, false), KQ_SEGS_ROW(2, false)},
                                           {KQ_SEGS_ROW(1, true), KQ_SEGS_ROW(2, true)}};
#undef KQ_SEGS_ROW
// the MoE gather (TB_SEL) instantiations, single type only (slots 4 and
// 13 unused: the mixed kernels have no gather form; the int8 mode's at
// depth 1)
#define KQ_SEL_ROW(D, M)                                                                  \
    {&kq_segs_kernel<D, TB_Q4K | TB_SEL, M>, &kq_segs_kernel<D, TB_Q6K | TB_SEL, M>,       \
     &kq_segs_kernel<D, TB_Q2K | TB_SEL, M>, &kq_segs_kernel<D, TB_NIB | TB_SEL, M>,       \
     &kq_segs_kernel<D, TB_Q4K | TB_SEL, M>, &kq_segs_kernel<D, TB_Q5K | TB_SEL, M>,       \
     &kq_segs_kernel<D, TB_Q3K | TB_SEL, M>, &kq_segs_kernel<D, TB_Q80 | TB_SEL, M>,       \
     &kq_segs_kernel<1, TB_Q4K_I8 | TB_SEL, M>, &kq_segs_kernel<1, TB_Q6K_I8 | TB_SEL, M>, \
     &kq_segs_kernel<1, TB_Q5K_I8 | TB_SEL, M>, &kq_segs_kernel<1, TB_Q3K_I8 | TB_SEL, M>, \
     &kq_segs_kernel<1, TB_Q80_I8 | TB_SEL, M>, &kq_segs_kernel<1, TB_Q4K_I8 | TB_SEL, M>}
static const segs_fn k_segs_sel[2][2][NSLOT] = {{KQ_SEL_ROW(1, false), KQ_SEL_ROW(2, false)},
                                               {KQ_SEL_ROW(1, true), KQ_SEL_ROW(2, true)}};
#undef KQ_SEL_ROW

int kqk_set_max_lds(int bytes) {
    for (int m = 0; m < 2; m++)
        for (int d = 0; d < 2; d++)
            for (int t = 0; t < 2 * NSLOT; t++) {
                const segs_fn f = t < NSLOT ? k_segs[m][d][t] : k_segs_sel[m][d][t - NSLOT];
                const hipError_t e =
                    hipFuncSetAttribute(reinterpret_cast<const void*>(f),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
                if (e != hipSuccess) return (int)e;
            }
    return 0;
}

// One launch over nseg (<= 8) segments; grid workgroups of `threads`
// (a multiple of 64, at most 1024), `depth` (1 or 2) batches in flight per
// wave (a third would not fit the 128 VGPRs a 1024-lane workgroup allows).
int kqk_launch_segs(const kqk_seg* segs, int nseg, int grid, int threads, int depth,
                    long lds_bytes, int xs_off, int terms_off, int scr_off, hipStream_t st) {
    if (nseg < 1 || nseg > MAXSEG || threads < 64 || threads > 1024 || (threads & 63) ||
        depth < 1 || depth > 2)
        return (int)hipErrorInvalidValue;
    SegsArg A;
    A.nseg = nseg;
    A.act = segs[0].act;
    A.cx = segs[0].cx;
    A.cw = segs[0].cw;
    A.logits = segs[0].logits;
    A.xs_off = xs_off;
    A.terms_off = terms_off;
    A.scr_off = scr_off;
    A.threads = threads;
    A.grid = grid;
    magic_for((uint32_t)grid, A.grid_m, A.grid_l);
    int set = 0;
    for (int i = 0; i < nseg; i++) {
        Seg& d = A.s[i];
        const kqk_seg& h = segs[i];
        int start = 0;
        bool equal = true;
        for (int g = 0; g < MAXG; g++) {
            const int q = g < h.nparts ? g : 0;      // unused slots repeat part 0
            d.w[g] = static_cast<const uint8_t*>(h.w[q]);
            d.y[g] = h.y[q];
            d.add[g] = h.add[q];
            if (g < LIST_MAX) d.start[g] = g < h.nparts ? start : 0;
            if (g < h.nparts) {
                start += h.rows[g];
                equal = equal && h.rows[g] == h.rows[0];
            }
        }
        d.x = h.x;
        d.sel = h.sel;
        d.probs = h.probs;
        d.sel_out = h.sel_out;
        d.selw_out = h.selw_out;
        d.estride = h.estride;
        d.ksel = h.ksel > 0 ? h.ksel : 1;
        d.emax = h.emax > 0 ? h.emax : 1;
        if (start >= (1 << 24) || (long)(h.K >> 8) * block_bytes_of(h.type) >= (1L << 24) ||
            type_slot(h.type) < 0)                                    // 24-bit addressing
            return (int)hipErrorInvalidValue;
        d.type = h.type; d.K = h.K; d.N = start; d.nparts = h.nparts;
        d.x_stride = h.nparts > 1 ? h.x_stride : 0;
        d.pn = equal ? h.rows[0] : 0;
        magic_for((uint32_t)(equal ? h.rows[0] : 1), d.pn_m, d.pn_l);
        magic_for((uint32_t)(h.K >> 6), d.nc_m, d.nc_l);
        set |= h.type == T_Q4K ? TB_Q4K : h.type == T_Q6K ? TB_Q6K : h.type == T_Q2K ? TB_Q2K
             : h.type == T_NIB ? TB_NIB : h.type == T_Q5K ? TB_Q5K : h.type == T_Q3K ? TB_Q3K
             : h.type == T_Q80 ? TB_Q80 : h.type == T_Q4K_I8 ? TB_Q4K_I8
             : h.type == T_Q6K_I8 ? TB_Q6K_I8 : h.type == T_Q5K_I8 ? TB_Q5K_I8
             : h.type == T_Q3K_I8 ? TB_Q3K_I8 : TB_Q80_I8;
    }
    const int t = set == TB_Q4K ? 0 : set == TB_Q6K ? 1 : set == TB_Q2K ? 2 : set == TB_NIB ? 3
                : set == TB_Q5K ? 5 : set == TB_Q3K ? 6 : set == TB_Q80 ? 7
                : set == TB_Q4K_I8 ? 8 : set == TB_Q6K_I8 ? 9 : set == TB_Q5K_I8 ? 10
                : set == TB_Q3K_I8 ? 11 : set == TB_Q80_I8 ? 12 : set == TB_I8MIX ? 13
                : set == TB_Q46 ? 4 : -1;
    if (t < 0) return (int)hipErrorInvalidValue;   // other types are never mixed in a launch
    if (t == 4 || t == 13) depth = 1;   // the mixed kernels fit 128 VGPRs at depth 1 only
    int nsel = 0;
    for (int i = 0; i < nseg; i++) nsel += segs[i].sel != nullptr;
    if (nsel && (nsel != nseg || t == 4 || t == 13)) return (int)hipErrorInvalidValue;
    // the MoE FFN step pieces: one selection segment; the combine needs
    // equal parts whose rows are a multiple of the grid and its outputs in
    // the x region; in-launch softmax needs every logit in a lane
    const kqk_seg& h0 = segs[0];
    if (h0.act || h0.cx || h0.logits) {
        if (nseg != 1 || !h0.sel || t == 4 || t == 13 || (h0.act && h0.cx))
            return (int)hipErrorInvalidValue;
        if (h0.act || h0.cx) {   // equal parts, rows a multiple of the grid, outputs in the x region
            const int pn = h0.rows[0];
            bool ok = pn % grid == 0 && (long)h0.nparts * (pn / grid) * 4 <= xs_off;
            for (int p = 1; p < h0.nparts; p++) ok = ok && h0.rows[p] == pn;
            if (h0.cx) ok = ok && h0.cw && pn / grid <= threads;
            if (h0.act) ok = ok && !(h0.nparts & 1);
            if (!ok) return (int)hipErrorInvalidValue;
        }
        if (h0.logits && (!h0.probs || ((h0.emax + 63) & ~63) > threads))
            return (int)hipErrorInvalidValue;
    }
    const segs_fn f = nsel ? k_segs_sel[nseg > 1][depth - 1][t] : k_segs[nseg > 1][depth - 1][t];
    hipLaunchKernelGGL(f, dim3(grid), dim3(threads), (size_t)lds_bytes, st, A);
    return (int)hipGetLastError();
}

// Multi-x launch plan for groups of N x K rows with at most mmax members
// and at most ngmax groups.  plan[]: 0 threads, 1 S (members per weight
// load), 2 RB (rows per item), 3 nblk (items per group), 4 TC (chunks per x
// tile), 5 sums bytes, 6 x buffer bytes, 7 mch (members staged together).
// Returns the LDS bytes, or -1.  ngm (MoE batches, else null): ngm[m] is
// the expected number of groups when member lists are cut into runs of at
// most m members (m = 1..MX_MC); the item count then follows the chosen
// run length, as the grouping kernel will cut them.
//
// The choice comes from a small cost model, in instruction issues of the
// busiest SIMD: item rounds x member chunks x (steps x task-step cost +
// per-item and per-tile overheads).  Tasks t go to SIMD t % 4; a task-step
// costs c0 (shared by the S members) + S c1 (per member) issues, per-type
// counts from the generated code; a SIMD with fewer than 3 tasks is
// latency-bound and taken as 3.
long kqk_mx_plan(int type, int N, int K, int mmax, int ngmax, int grid, int lds_max, int* plan,
                 const float* ngm) {
    const int xpc = xs_per_chunk(type);
    if (xpc < 0 || mmax < 1 || mmax > MX_MAXM || ngmax < 1 || N < 1 || K <= 0 || (K & 255) ||
        grid < 1)
        return -1;
    const bool i8 = type == T_Q5K_I8 || type == T_Q3K_I8 || type == T_Q80_I8;
    const int T = type == T_Q5K || type == T_Q3K || type == T_Q80 || i8 ? 512 : 1024;   // mx_threads
    const int W = T / 64;
    const int NC = K >> 6, GP = kq_phases(NC), RPT = 64 / GP;
    const int NCg = (NC + GP - 1) / GP * GP, nstep = NCg / GP;
    const int G4 = type == T_Q4K || type == T_Q5K || type == T_Q80 || i8 ? 8 : 4;
    const long per = K / (4 * G4);
    const long head = 8L * MX_MAXM + 64;
    const long rbytes = (long)(K >> 8) * block_bytes_of(type);
    // (Q5_K, Q3_K, Q8_0: estimated from their decode next to Q4_K's)
    const double c0 = type == T_Q4K ? 45 : type == T_Q6K ? 170 : type == T_Q2K ? 30
                    : type == T_Q5K ? 55 : type == T_Q3K ? 70 : type == T_Q80 ? 25 : i8 ? 50 : 35;
    const double c1 = type == T_Q6K ? 140 : i8 ? 60 : 150;
    // per-pass and per-tile overheads, fitted to timings of the 27B gate
    // and down shapes (a pass stages x and ramps the weight stream up)
    const double item_cost = 20000, tile_cost = 500;
    double best = 1e300;
    long best_lds = -1;
    const int m0 = mmax < MX_MC ? mmax : MX_MC;
    for (int mch = m0; mch >= 1; mch = mch > 1 ? (mch + 1) / 2 : 0) {
        // int8 members: chunks of XPAD_I8 slots and XS_PER_CHUNK floats
        const long sums = i8 ? ((long)mch * NCg * xpc * 4 + 15) & ~15L
                        : xpc ? ((long)mch * per * 4 + 15) & ~15L : 0;
        const long whole = (long)mch * NCg * (i8 ? XPAD_I8 : XPAD) * 16;
        long xt, lds;
        int TC;
        if (head + sums + whole <= lds_max) {
            TC = NCg;
            xt = whole;
            lds = head + sums + xt;
        } else if (i8) {
            continue;                           // int8 members are staged whole
        } else {
            TC = 0;
            for (int tc = GP; tc < NCg; tc += GP) {
                if (head + sums + 2L * mch * tc * XPAD * 16 > lds_max || mch * tc * 16 > 2 * T) break;
                TC = tc;
            }
            if (TC == 0) continue;
            xt = (long)mch * TC * XPAD * 16;
            lds = head + sums + 2 * xt;
        }
        const int ntile = (NC + TC - 1) / TC;
        // MoE runs are cut at mch members: one member chunk each, and
        // ngm[mch] groups expected
        const int nmc = ngm ? 1 : (mmax + mch - 1) / mch;
        for (int S = 1; S <= 2; S++) {
            if (S > 1 && S > mch) break;
            const int nsg = (mch + S - 1) / S;
            const int maxgrp = W * MX_TW / nsg;
            if (maxgrp < 1) continue;
            const int nblk0 = (N + RPT * maxgrp - 1) / (RPT * maxgrp);
            for (int nblk = nblk0; nblk <= N && nblk <= 4096; nblk++) {
                const int RB = (N + nblk - 1) / nblk;
                if (nblk > nblk0 && (N + RB - 1) / RB != nblk) continue;
                const int ntask = ((RB + RPT - 1) / RPT) * nsg;
                if (ntask > W * MX_TW) continue;
                const long items = ngm ? (long)ceil((double)ngm[mch] * nblk) : (long)ngmax * nblk;
                const long rounds = (items + grid - 1) / grid;
                const int simd = (ntask + 3) / 4;
                const double step = (simd < 3 ? 3 : simd) * (c0 + S * c1);
                // weight streaming: a CU's share of HBM is ~33 B per issue;
                // a pass needs about 32 tasks (two per wave) in flight to
                // draw it, and later member chunks re-read from L2
                const double stream = (double)RB * rbytes / 33.0 / (ntask < 32 ? ntask / 32.0 : 1.0);
                const double cost =
                    (double)rounds * ((step * nstep > stream ? step * nstep : stream) * nmc +
                                      nmc * (item_cost + (ntile - 1) * tile_cost));
                if (cost <= best) {             // ties: the later (more items, or fewer
                    best = cost;                // members per load) choice
                    best_lds = lds;
                    plan[0] = T; plan[1] = S; plan[2] = RB; plan[3] = nblk; plan[4] = TC;
                    plan[5] = (int)sums; plan[6] = (int)xt; plan[7] = mch;
                }
            }
        }
    }
    return best_lds;
}

int kqk_mx_set_max_lds(int bytes) {
#define KQ_MX_ATTR(T_)                                                                  \
    {&kq_mx_kernel<T_, 1, true>, &kq_mx_kernel<T_, 2, true>, &kq_mx_kernel<T_, 1, false>, \
     &kq_mx_kernel<T_, 2, false>}
    typedef void (*mx_fn)(MxArg);
#define KQ_MX_ATTR8(T_)                                                                 \
    {&kq_mx_kernel<T_, 1, true>, &kq_mx_kernel<T_, 2, true>, &kq_mx_kernel<T_, 1, true>,  \
     &kq_mx_kernel<T_, 2, true>}
    const mx_fn fns[10][4] = {KQ_MX_ATTR(T_Q4K), KQ_MX_ATTR(T_Q6K), KQ_MX_ATTR(T_Q2K),
                              KQ_MX_ATTR(T_NIB), KQ_MX_ATTR(T_Q5K), KQ_MX_ATTR(T_Q3K),
                              KQ_MX_ATTR(T_Q80), KQ_MX_ATTR8(T_Q5K_I8), KQ_MX_ATTR8(T_Q3K_I8),
                              KQ_MX_ATTR8(T_Q80_I8)};
#undef KQ_MX_ATTR
#undef KQ_MX_ATTR8
    for (int t = 0; t < 10; t++)
        for (int i = 0; i < 4; i++) {
            const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fns[t][i]),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
            if (e != hipSuccess) return (int)e;
        }
    // the matrix-core sweep stages up to 2 x 66 KB
    typedef void (*mf_fn)(MfArg);
    const mf_fn mfs[8] = {&kq_mf_kernel<T_Q4K, 1>, &kq_mf_kernel<T_Q4K, 2>, &kq_mf_kernel<T_Q4K, 3>,
                          &kq_mf_kernel<T_Q4K, 4>, &kq_mf_kernel<T_Q6K, 1>, &kq_mf_kernel<T_Q6K, 2>,
                          &kq_mf_kernel<T_Q6K, 3>, &kq_mf_kernel<T_Q6K, 4>};
    for (int i = 0; i < 8; i++) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(mfs[i]),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        if (e != hipSuccess) return (int)e;
    }
    return 0;
}

// One multi-x launch.  Inline group (gdev == NULL): weights w, members
// j = 0..M-1 with x_j = X + j * x_stride and y_j = Y + j * y_stride.  Else
// *ngdev groups of MxGroup layout at gdev (device memory).
int kqk_launch_mx(int type, const int* plan, long lds, int grid, const void* w, int M,
                  const void* gdev, const int* ngdev, const float* X, long x_stride, float* Y,
                  long y_stride, int N, int K, hipStream_t st) {
    MxArg a;
    a.w = static_cast<const uint8_t*>(w);
    a.M = M;
    a.N = N; a.K = K;
    a.gdev = static_cast<const MxGroup*>(gdev);
    a.ngdev = ngdev;
    a.X = X; a.Y = Y;
    a.runs_out = nullptr; a.runs_in = nullptr;
    a.x_stride = x_stride; a.y_stride = y_stride;
    a.RB = plan[2]; a.nblk = plan[3];
    a.threads = plan[0]; a.grid = grid;
    a.TC = plan[4]; a.sums_bytes = plan[5]; a.xt_bytes = plan[6]; a.mch = plan[7];
    a.sel = nullptr;
    a.nm = a.E = a.nt = a.x_div = a.grp_off = 0;
    a.wt[0] = a.wt[1] = nullptr;
    a.yt[0] = a.yt[1] = nullptr;
    a.estride = 0;
    a.probs = nullptr;
    a.B = a.k = 0;
    a.sel_out = nullptr;
    a.selw_out = nullptr;
    const bool whole = a.TC >= (K >> 6);
    switch (type) {
    case T_Q4K: return launch_mx_t<T_Q4K>(a, plan[1], whole, lds, st);
    case T_Q6K: return launch_mx_t<T_Q6K>(a, plan[1], whole, lds, st);
    case T_Q2K: return launch_mx_t<T_Q2K>(a, plan[1], whole, lds, st);
    case T_NIB: return launch_mx_t<T_NIB>(a, plan[1], whole, lds, st);
    case T_Q5K: return launch_mx_t<T_Q5K>(a, plan[1], whole, lds, st);
    case T_Q3K: return launch_mx_t<T_Q3K>(a, plan[1], whole, lds, st);
    case T_Q80: return launch_mx_t<T_Q80>(a, plan[1], whole, lds, st);
    case T_Q5K_I8: return launch_mx_t<T_Q5K_I8>(a, plan[1], whole, lds, st);
    case T_Q3K_I8: return launch_mx_t<T_Q3K_I8>(a, plan[1], whole, lds, st);
    case T_Q80_I8: return launch_mx_t<T_Q80_I8>(a, plan[1], whole, lds, st);
    default: return (int)hipErrorInvalidValue;
    }
}

// MoE: top-k per token (E <= 4096), and the expert groups of a selection
int kqk_launch_moe_topk(const float* probs, int B, int E, int k, int* sel, float* selw,
                        hipStream_t st) {
    if (B < 1 || E < 1 || E > 4096 || k < 1) return (int)hipErrorInvalidValue;
    if (E <= 1024)
        hipLaunchKernelGGL(kq_moe_topk_rank_kernel, dim3(B), dim3(1024), 0, st, probs, B, E, k, sel,
                           selw);
    else
        hipLaunchKernelGGL(kq_moe_topk_kernel, dim3((B + 3) / 4), dim3(256), 0, st, probs, B, E,
                           k, sel, selw);
    return (int)hipGetLastError();
}

long kqk_mx_group_bytes(void) { return (long)sizeof(MxGroup); }

// LDS bytes of the in-launch MoE runs (MoeRuns) for nm members, E experts
// and at most ndmax runs; B > 0: routed in the launch for B tokens
long kqk_moe_runs_words(int nm, int E, int ndmax) {
    return 1 + ((2L * E + 3) & ~3L) + 4L * ((nm + 3) / 4) + nm + ndmax;
}

long kqk_moe_runs_lds(int nm, int E, int ndmax, int B) {
    const long E64 = (E + 63) & ~63L, nm4 = (nm + 3) / 4;
    return 4L * ((B > 0 ? B * E64 + 4 * nm4 : 0) + ((2L * E + 3) & ~3L) + 4 * nm4 + nm + ndmax);
}

// A MoE batch in one multi-x launch that groups the selection itself: the
// groups kq_moe_group_kernel would write, built in every workgroup's LDS
// at byte offset plan_lds (lds = plan_lds + kqk_moe_runs_lds(...)).
int kqk_launch_mx_moe(int type, const int* plan, long plan_lds, long lds, int grid, const int* sel,
                      int nm, int E, int nt, int x_div, const void* w0, const void* w1, float* y0,
                      float* y1, long estride, const float* X, int N, int K, const float* probs,
                      int B, int k, int* sel_out, float* selw_out, int* runs_out,
                      const int* runs_in, hipStream_t st) {
    if (nm < 1 || E < 1 || E > 4096 || nt < 1 || nt > 2 || x_div < 1 || plan[7] < 1 ||
        plan[7] > MX_MAXM || plan_lds < 0 || (plan_lds & 15) || (runs_in && probs) ||
        (probs && (B < 1 || k < 1 || B * k != nm || !sel_out || !selw_out)) || (!probs && !sel))
        return (int)hipErrorInvalidValue;
    MxArg a;
    a.w = nullptr;
    a.M = 0;
    a.N = N; a.K = K;
    a.gdev = nullptr;
    a.ngdev = nullptr;
    a.X = X; a.Y = nullptr;
    a.runs_out = runs_out; a.runs_in = runs_in;
    a.x_stride = K; a.y_stride = N;
    a.RB = plan[2]; a.nblk = plan[3];
    a.threads = plan[0]; a.grid = grid;
    a.TC = plan[4]; a.sums_bytes = plan[5]; a.xt_bytes = plan[6]; a.mch = plan[7];
    a.sel = sel;
    a.nm = nm; a.E = E; a.nt = nt; a.x_div = x_div; a.grp_off = (int)plan_lds;
    a.wt[0] = static_cast<const uint8_t*>(w0);
    a.wt[1] = static_cast<const uint8_t*>(nt > 1 ? w1 : w0);
    a.yt[0] = y0;
    a.yt[1] = nt > 1 ? y1 : y0;
    a.estride = estride;
    a.probs = probs;
    a.B = probs ? B : 0;
    a.k = probs ? k : 0;
    a.sel_out = sel_out;
    a.selw_out = selw_out;
    const bool whole = a.TC >= (K >> 6);
    switch (type) {
    case T_Q4K: return launch_mx_t<T_Q4K>(a, plan[1], whole, lds, st);
    case T_Q6K: return launch_mx_t<T_Q6K>(a, plan[1], whole, lds, st);
    case T_Q2K: return launch_mx_t<T_Q2K>(a, plan[1], whole, lds, st);
    case T_NIB: return launch_mx_t<T_NIB>(a, plan[1], whole, lds, st);
    case T_Q5K: return launch_mx_t<T_Q5K>(a, plan[1], whole, lds, st);
    case T_Q3K: return launch_mx_t<T_Q3K>(a, plan[1], whole, lds, st);
    case T_Q80: return launch_mx_t<T_Q80>(a, plan[1], whole, lds, st);
    case T_Q5K_I8: return launch_mx_t<T_Q5K_I8>(a, plan[1], whole, lds, st);
    case T_Q3K_I8: return launch_mx_t<T_Q3K_I8>(a, plan[1], whole, lds, st);
    case T_Q80_I8: return launch_mx_t<T_Q80_I8>(a, plan[1], whole, lds, st);
    default: return (int)hipErrorInvalidValue;
    }
}

int kqk_launch_moe_group(const int* sel, int nm, int E, int nt, int x_div, int mch,
                         const void* w0, const void* w1, float* y0, float* y1, long estride,
                         void* groups, int* ng, hipStream_t st) {
    if (nm < 1 || E < 1 || E > 4096 || nt < 1 || nt > 2 || x_div < 1 || mch < 1 || mch > MX_MAXM)
        return (int)hipErrorInvalidValue;
    MoeGroupArg a;
    a.sel = sel; a.nm = nm; a.E = E; a.nt = nt; a.x_div = x_div; a.mch = mch;
    a.w[0] = static_cast<const uint8_t*>(w0);
    a.w[1] = static_cast<const uint8_t*>(nt > 1 ? w1 : w0);
    a.y[0] = y0;
    a.y[1] = nt > 1 ? y1 : y0;
    a.estride = estride;
    a.groups = static_cast<MxGroup*>(groups);
    a.ng = ng;
    const size_t lds = (size_t)(((2 * E + 3) & ~3) + 4 * ((nm + 3) / 4)) * sizeof(int);
    hipLaunchKernelGGL(kq_moe_group_kernel, dim3(1), dim3(1024), lds, st, a);
    return (int)hipGetLastError();
}

// MFMA multi-x (Q4_K, Q6_K): workspace sizes for B streams of N x K, and the
// launch (x split into planes, the matrix-core sweep over `grid`
// workgroups, and the sum of shared row blocks' partials).
// Workspace of one launch of up to 64 streams (larger B runs in chunks of
// 64 on the same workspace): the planes, then the x sums and the exponents
// (one region), then the partial sums.
int kqk_mfma_workspace(int type, int B, int N, int K, int grid, long* planes, long* xs, long* part) {
    if ((type != T_Q4K && type != T_Q6K) || B < 1 || N < 1 || K <= 0 || (K & 255) || grid < 1)
        return -1;
    const int NSG = B >= 64 ? 4 : (B + 15) / 16;
    const long NSB = K >> 8;
    *planes = NSB * NSG * MF_GROUP_U4 * 16;
    *xs = NSB * NSG * MF_SIDE_U4 * 16;
    *part = mf_plan(type, NSG, N, K, grid).part_floats * 4;
    return 0;
}

int kqk_launch_mfma(int type, const float* x, const void* w, float* y, int B, int N, int K,
                    void* planes, float* xs, float* part, int grid, hipStream_t st) {
    if (type != T_Q4K && type != T_Q6K) return (int)hipErrorInvalidValue;
    for (int s0 = 0; s0 < B; s0 += 64) {
        const int nb = B - s0 < 64 ? B - s0 : 64;
        const float* xc = x + (size_t)s0 * K;
        float* yc = y + (size_t)s0 * N;
        const int e = type == T_Q4K
                          ? launch_mfma_t<T_Q4K>(xc, w, yc, nb, N, K, planes, xs, part, grid, st)
                          : launch_mfma_t<T_Q6K>(xc, w, yc, nb, N, K, planes, xs, part, grid, st);
        if (e) return e;
    }
    return 0;
}

int kqk_launch_dequant(int type, const void* w, float* y, long nblocks, hipStream_t st) {
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    switch (type) {
    case T_Q4K: return launch_dequant<T_Q4K>(wb, y, nblocks, st);
    case T_Q6K: return launch_dequant<T_Q6K>(wb, y, nblocks, st);
    case T_Q2K: return launch_dequant<T_Q2K>(wb, y, nblocks, st);
    case T_NIB: return launch_dequant<T_NIB>(wb, y, nblocks, st);
    case T_Q5K: return launch_dequant<T_Q5K>(wb, y, nblocks, st);
    case T_Q3K: return launch_dequant<T_Q3K>(wb, y, nblocks, st);
    case T_Q80: return launch_dequant<T_Q80>(wb, y, nblocks, st);
    case T_F16: case T_F32: {
        const long n = nblocks * 256;
        hipLaunchKernelGGL(kq_dense_dequant_kernel, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256),
                           0, st, wb, y, n, type);
        return (int)hipGetLastError();
    }
    default: return -1;
    }
}

int kqk_launch_q2k_to_nib(const void* q2k, void* nib, long nblocks, hipStream_t st) {
    if (nblocks < 1) return (int)hipErrorInvalidValue;
    const long n = nblocks * 37;
    hipLaunchKernelGGL(kq_q2k_to_nib_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       static_cast<const uint32_t*>(q2k), static_cast<uint32_t*>(nib), nblocks);
    return (int)hipGetLastError();
}

int kqk_launch_softmax(float* x, int B, int E, hipStream_t st) {
    if (B < 1 || E < 1 || E > KQ_MOE_MAX_EXPERTS) return (int)hipErrorInvalidValue;
    const size_t shm = (size_t)(((E + 3) & ~3) + 64) * sizeof(float);
    hipLaunchKernelGGL(kq_softmax_kernel, dim3(B), dim3(256), shm, st, x, E);
    return (int)hipGetLastError();
}

int kqk_launch_swiglu(const float* g, const float* u, float* y, long n, hipStream_t st) {
    if (n < 1) return (int)hipErrorInvalidValue;
    const long lanes = (n + 3) / 4;
    hipLaunchKernelGGL(kq_swiglu_kernel, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, st, g,
                       u, y, n);
    return (int)hipGetLastError();
}

int kqk_launch_moe_combine(const float* o, const int* sel, const float* selw, const float* resid,
                           float* x, int B, int k, int H, hipStream_t st) {
    if (B < 1 || k < 1 || H < 4 || (H & 3)) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(kq_moe_combine_kernel, dim3((H / 4 + 255) / 256, B), dim3(256), 0, st, o, sel,
                       selw, resid, x, k, H);
    return (int)hipGetLastError();
}

int kqk_launch_quantize_q8(const float* x, int K, int group, int8_t* xq, float* xscale, int* xsum,
                           hipStream_t st) {
    if ((group != 32 && group != 16) || K < group || K % group) return (int)hipErrorInvalidValue;
    const int ng = K / group;
    if (group == 32)
        hipLaunchKernelGGL(kq_quantize_kernel<32>, dim3((ng + 255) / 256), dim3(256), 0, st, x, ng, xq,
                           xscale, xsum);
    else
        hipLaunchKernelGGL(kq_quantize_kernel<16>, dim3((ng + 255) / 256), dim3(256), 0, st, x, ng, xq,
                           xscale, xsum);
    return (int)hipGetLastError();
}

// Dense rows (F16, F32): x staged in LDS when K <= DENSE_XLDS_MAX
int kqk_launch_dense(int type, const void* w, const float* x, const float* add, float* y, int N,
                     int K, int B, int grid, hipStream_t st) {
    if ((type != T_F16 && type != T_F32) || N < 1 || K < 256 || (K & 255) || grid < 1 || B < 1 ||
        (B > 1 && add))
        return (int)hipErrorInvalidValue;
    DenseArg a;
    a.w = static_cast<const uint8_t*>(w);
    a.x = x; a.add = add; a.y = y; a.N = N; a.K = K; a.B = B;
    a.row_bytes = (long)K * (type == T_F32 ? 4 : 2);
    // DENSE_SB streams per wave share its weight loads, unless that leaves
    // fewer than 8 waves per CU (a 128-row MoE router at B = 16: 256 waves
    // of long serial chains); then one stream per wave
    const long w8 = (long)N * ((B + DENSE_SB - 1) / DENSE_SB);
    const int sb = B == 1 || w8 < 8L * 256 ? 1 : DENSE_SB;
    const bool lds = (long)sb * K <= DENSE_XLDS_MAX;
    const size_t shm = lds ? (size_t)sb * K * 4 : 0;
    // a wave per row: no more workgroups than rows / 4 (each would stage x
    // for nothing)
    const dim3 g(grid < (N + 3) / 4 ? grid : (N + 3) / 4, (B + sb - 1) / sb);
#define KQ_DENSE_GO(T_, L_, S_) hipLaunchKernelGGL((kq_dense_kernel<T_, L_, S_>), g, dim3(256), shm, st, a)
#define KQ_DENSE_SB(S_)                                                              \
    if (type == T_F32) { if (lds) KQ_DENSE_GO(T_F32, true, S_); else KQ_DENSE_GO(T_F32, false, S_); } \
    else { if (lds) KQ_DENSE_GO(T_F16, true, S_); else KQ_DENSE_GO(T_F16, false, S_); }
    if (sb == 1) { KQ_DENSE_SB(1) } else { KQ_DENSE_SB(DENSE_SB) }
#undef KQ_DENSE_SB
#undef KQ_DENSE_GO
    return (int)hipGetLastError();
}

// int8 MULTISEQ on the matrix cores: workspace bytes (quantized streams,
// then their coefficients, 256-byte aligned), and the launches (prep, main).
int kqk_mi8_parts(int K) {
    // measured over 1, 2, 4 and 8 parts at B = 8, 16, 64: the 27B gate
    // (20 super-blocks) is fastest with 2 (1 at B = 8 by 10 %), the down
    // projection (68) with 4 (2 at B = 16 by 9 %); 8 was never fastest
    const int nb = K >> 8;
    return nb >= 48 ? 4 : nb >= 12 ? 2 : 1;
}

// (streams padded to a multiple of 16, the widest wave's stream count)
long kqk_mi8_workspace(int type, int B, int K, long* cf_off) {
    if ((type != T_Q4K_I8 && type != T_Q6K_I8) || B < 1 || K < 256 || (K & 255)) return -1;
    const long bp = (B + 15) & ~15L;
    const long xb = (bp * K + 255) & ~255L;
    const long cb = bp * (type == T_Q4K_I8 ? K / 32 : K / 16) * 8;
    *cf_off = xb;
    return xb + ((cb + 255) & ~255L) + 256;     // + the zero page
}

int kqk_launch_mi8(int type, const float* xs, long x_stride, const void* w, float* ys,
                   long y_stride, int B, int N, int K, void* ws, int ks, hipStream_t st) {
    long cf_off = 0;
    const long wsb = kqk_mi8_workspace(type, B, K, &cf_off);
    if (wsb < 0 || N < 1 || B < 2 || (x_stride & 3) || x_stride < K || y_stride < N ||
        ((uintptr_t)xs & 15) || ((uintptr_t)ws & 255))
        return (int)hipErrorInvalidValue;
    int8_t* xq = static_cast<int8_t*>(ws);
    uint8_t* cf = static_cast<uint8_t*>(ws) + cf_off;
    uint8_t* zp = static_cast<uint8_t*>(ws) + wsb - 256;   // zeroed by the prep kernel
    const int G = type == T_Q4K_I8 ? 32 : 16;
    const int bpad = (B + 15) & ~15;
    const long groups = (long)bpad * (K / G);
    if (G == 32)
        hipLaunchKernelGGL(kq_mi8_prep_kernel<32>, dim3((unsigned)((groups + 255) / 256)), dim3(256),
                           0, st, xs, x_stride, K, B, bpad, xq, cf, zp, nullptr);
    else
        hipLaunchKernelGGL(kq_mi8_prep_kernel<16>, dim3((unsigned)((groups + 255) / 256)), dim3(256),
                           0, st, xs, x_stride, K, B, bpad, xq, cf, zp, nullptr);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    Mi8Arg a;
    a.w = static_cast<const uint8_t*>(w);
    a.xq = xq;
    a.zp = zp;
    a.cf = cf;
    a.y = ys;
    a.y_stride = y_stride;
    a.N = N; a.K = K; a.B = B;
    a.groups = nullptr; a.ng = nullptr; a.zrow = 0; a.rbw = 1; a.sm = nullptr; a.pack2 = 0;
    // Q4_K: 8 or 16 streams per wave; Q6_K: 8 (its A operands take
    // 16 registers per MFMA and super-block)
    // (8 streams per wave up to B = 8, one super-block in flight; measured
    // at the 27B gate, B = 8 .. 64, against 8 streams at every B and two
    // super-blocks in flight)
#ifndef KQ_MI8_SWB
#define KQ_MI8_SWB 8
#endif
#ifndef KQ_MI8_P8
#define KQ_MI8_P8 1
#endif
    const int SW = type == T_Q6K_I8 || B <= KQ_MI8_SWB ? 8 : 16;
    const int nset = (B + SW - 1) / SW, nrb = (N + 15) / 16;
    // K-parts: a function of the row length only (kqk_mi8_parts), so the
    // binary64 grouping -- and with it the result -- does not depend on the
    // batch or the row count
    if (ks != 1 && ks != 2 && ks != 4 && ks != 8) ks = kqk_mi8_parts(K);
#define KQ_MI8_GO(T_, S_, P_, K_)                                                            \
    hipLaunchKernelGGL((kq_mi8_kernel<T_, S_, P_, K_, false>), dim3((unsigned)nrb,           \
                       (unsigned)nset), dim3(64 * K_), 0, st, a)
#define KQ_MI8_KS(T_, S_, P_)                                                                \
    if (ks == 1) KQ_MI8_GO(T_, S_, P_, 1);                                                   \
    else if (ks == 2) KQ_MI8_GO(T_, S_, P_, 2);                                              \
    else if (ks == 4) KQ_MI8_GO(T_, S_, P_, 4);                                              \
    else KQ_MI8_GO(T_, S_, P_, 8);
    if (type == T_Q4K_I8) {
        if (SW == 8) { KQ_MI8_KS(T_Q4K_I8, 8, KQ_MI8_P8) } else { KQ_MI8_KS(T_Q4K_I8, 16, 1) }
    } else {
        KQ_MI8_KS(T_Q6K_I8, 8, 1)
    }
#undef KQ_MI8_KS
#undef KQ_MI8_GO
    return (int)hipGetLastError();
}

// The int8 MoE batch: workspace bytes for nx quantized x rows (plus the
// zero row: the MULTISEQ workspace of nx + 1 streams, then the rows'
// {scale, sum} pairs) and the launches: the runs of at most 8 members of
// one expert (kq_moe_group_kernel's rule; records in groups, their count
// in *ng, at most ngmax) together with the quantized x rows (nx = nm /
// x_div of them), then the grouped main kernel.  K-parts as kqk_launch_mi8
// takes them, so a run's members equal a kq_gemv_multix_dev call over them.
#ifndef KQ_MI8_RBW
#define KQ_MI8_RBW 2
#endif
// (Q4_K super-blocks in flight per wave: 1 keeps the wave at 114 VGPRs,
// four waves per SIMD; measured at configs[4] B = 4 / 16 / 64 against 2
// and 3, and against 1 and 4 row blocks per workgroup)
#ifndef KQ_MI8G_P
#define KQ_MI8G_P 1
#endif
static long mi8_moe_layout(int type, int nx, int K, long* cf_off, long* sm_off, long* zp_off) {
    const long base = nx < 1 ? -1 : kqk_mi8_workspace(type, nx + 1, K, cf_off);
    if (base < 0) return -1;
    const long bpad = (nx + 1 + 15) & ~15L;
    *zp_off = base - 256;
    *sm_off = base;
    return base + ((bpad * (K / (type == T_Q4K_I8 ? 32 : 16)) * 8 + 255) & ~255L);
}

long kqk_mi8_moe_workspace(int type, int nx, int K) {
    long a, b, c;
    return mi8_moe_layout(type, nx, K, &a, &b, &c);
}

int kqk_launch_mi8_moe(int type, const int* sel, int nm, int E, int nt, int x_div,
                       const void* w0, const void* w1, float* y0, float* y1, long estride,
                       const float* x, int K, void* groups, int* ng, int ngmax, int N,
                       void* ws, int n_cu, hipStream_t st) {
    const int nx = x_div > 0 ? nm / x_div : 0;
    const long y_stride = N;
    if (nm < 1 || E < 1 || E > 4096 || nt < 1 || nt > 2 || x_div < 1 || nm % x_div)
        return (int)hipErrorInvalidValue;
    long cf_off = 0, sm_off = 0, zp_off = 0;
    const long wsb = mi8_moe_layout(type, nx, K, &cf_off, &sm_off, &zp_off);
    const int ks = kqk_mi8_parts(K);
    // several row blocks per workgroup when the row is one K-part and the
    // runs' workgroups outnumber what the GPU holds at once (one wave each,
    // four per SIMD): a workgroup then streams one weight sequence instead
    // of paying a launch-to-first-load latency per 16 rows.  When they all
    // fit (few members), the launch lasts one wave's chain of super-blocks,
    // and one row block per workgroup halves it.
    const long fit = (long)nt * (E < nm ? E : nm) * ((N + 15) / 16);
    const int rbw = ks != 1 ? 1 : fit <= 16L * (n_cu > 0 ? n_cu : 256) ? 1 : KQ_MI8_RBW;
    // runs of two Q4_K members on the VALU (mi8_pack2_q4k) when a workgroup
    // has two row blocks, so that its 64 lanes are 32 rows x 2 members (with
    // one row block half of them would idle: slower than the matrix-core
    // form at configs[4] B = 4)
    const int pack2 = type == T_Q4K_I8 && ks == 1 && rbw == 2;
    // a single member's chunk terms; with pack2 also a run of two members'
    // quantized rows and coefficients
    long tl = 16L * rbw * (K >> 6) * 8;
    if (pack2 && tl < 2L * K + K / 2) tl = 2L * K + K / 2;
    if (wsb < 0 || nx < 1 || N < 1 || ngmax < 1 || ngmax > 65535 || y_stride < N || !groups ||
        !ng || ((uintptr_t)x & 15) || ((uintptr_t)ws & 15) || tl > 65536)
        return (int)hipErrorInvalidValue;
    int8_t* xq = static_cast<int8_t*>(ws);
    uint8_t* cf = static_cast<uint8_t*>(ws) + cf_off;
    uint8_t* zp = static_cast<uint8_t*>(ws) + zp_off;
    float2* sm = reinterpret_cast<float2*>(static_cast<uint8_t*>(ws) + sm_off);
    const int G = type == T_Q6K_I8 ? 16 : 32;
    const int bpad = (nx + 1 + 15) & ~15;        // rows nx .. bpad-1 zero
    const long gq = (long)bpad * (K / G);
    // the runs (workgroup 0, kq_moe_group_kernel's rule with run length 8)
    // and the quantized rows (the other workgroups) in one launch
    MoeGroupArg ga;
    ga.sel = sel; ga.nm = nm; ga.E = E; ga.nt = nt; ga.x_div = x_div; ga.mch = 8;
    ga.w[0] = static_cast<const uint8_t*>(w0);
    ga.w[1] = static_cast<const uint8_t*>(nt > 1 ? w1 : w0);
    ga.y[0] = y0;
    ga.y[1] = nt > 1 ? y1 : y0;
    ga.estride = estride;
    ga.groups = static_cast<MxGroup*>(groups);
    ga.ng = ng;
    const size_t glds = (size_t)(((2 * E + 3) & ~3) + 4 * ((nm + 3) / 4)) * sizeof(int);
    const dim3 pg((unsigned)(1 + (gq + 255) / 256));
    if (G == 32)
        hipLaunchKernelGGL(kq_mi8_moe_prep_kernel<32>, pg, dim3(256), glds, st, ga, x, K, nx, bpad,
                           xq, cf, zp, sm);
    else
        hipLaunchKernelGGL(kq_mi8_moe_prep_kernel<16>, pg, dim3(256), glds, st, ga, x, K, nx, bpad,
                           xq, cf, zp, sm);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    Mi8Arg a;
    a.w = nullptr;
    a.xq = xq; a.zp = zp; a.cf = cf;
    a.y = nullptr;
    a.y_stride = y_stride;
    a.N = N; a.K = K; a.B = 8;
    a.groups = static_cast<const MxGroup*>(groups);
    a.ng = ng;
    a.zrow = nx;
    a.rbw = rbw;
    a.sm = sm;
    a.pack2 = pack2;
    const int nrb = ((N + 15) / 16 + rbw - 1) / rbw;
#define KQ_MI8G_GO(T_, P_, K_)                                                               \
    hipLaunchKernelGGL((kq_mi8_kernel<T_, 8, P_, K_, true>), dim3((unsigned)nrb,             \
                       (unsigned)ngmax), dim3(64 * K_), (size_t)tl, st, a)
#define KQ_MI8G_KS(T_, P_)                                                                   \
    if (ks == 1) KQ_MI8G_GO(T_, P_, 1);                                                      \
    else if (ks == 2) KQ_MI8G_GO(T_, P_, 2);                                                 \
    else KQ_MI8G_GO(T_, P_, 4);
    if (type == T_Q4K_I8) { KQ_MI8G_KS(T_Q4K_I8, KQ_MI8G_P) } else { KQ_MI8G_KS(T_Q6K_I8, 1) }
#undef KQ_MI8G_KS
#undef KQ_MI8G_GO
    return (int)hipGetLastError();
}

int kqk_dense_set_max_lds(int bytes) {
    const void* fns[4] = {reinterpret_cast<const void*>(&kq_dense_kernel<T_F32, true, 1>),
                          reinterpret_cast<const void*>(&kq_dense_kernel<T_F16, true, 1>),
                          reinterpret_cast<const void*>(&kq_dense_kernel<T_F32, true, DENSE_SB>),
                          reinterpret_cast<const void*>(&kq_dense_kernel<T_F16, true, DENSE_SB>)};
    for (int i = 0; i < 4; i++) {
        const hipError_t e = hipFuncSetAttribute(fns[i], hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 bytes < DENSE_XLDS_MAX * 4 ? bytes : DENSE_XLDS_MAX * 4);
        if (e != hipSuccess) return (int)e;
    }
    return 0;
}

}  // extern "C"
