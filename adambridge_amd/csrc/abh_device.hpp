// abh_device.hpp -- per-element arithmetic of the fused optimizer update on gfx950.
//
// Every function reproduces the reference's host kernel (adambridge/csrc/
// adambridge_kernels.c) bit for bit on finite inputs; the line numbers cited
// are that file's.  Rules this relies on, all gfx950 / HIP defaults plus the
// build flags in adambridge_amd/build.py:
//   - FP32 '/' and sqrtf are correctly rounded (v_div_scale/fmas/fixup and the
//     refined v_sqrt sequence), denormals are kept;
//   - -ffp-contract=off: a product and a sum are rounded separately unless
//     written as __builtin_fmaf, which is exactly where the reference's vector
//     bodies use an FMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace abh {

enum : int { DT_NONE = 0, DT_F32 = 1, DT_BF16 = 2, DT_FP8 = 3, DT_F24 = 4, DT_PACKED = 5, DT_PACKED8 = 6,
             DT_PACKED_LION = 7, DT_PACKED_F32 = 8, DT_PACKED_F24 = 9,
             DT_PACKED_LION_F24 = 10, DT_PACKED8_F24 = 11, DT_PACKED_LION_F32 = 12,
             DT_PACKED8_LION = 13, DT_PACKED_F24_F32 = 14, DT_PACKED_LION_F24_F32 = 15,
             DT_PACKED8_LION_F24 = 16 };
enum : int { ALGO_ADAMW = 0, ALGO_LION = 1 };
constexpr int kFp8Block = 128;

struct Coef {
    float b1, b2, omb1, omb2, decay, step, isbc2, eps;
};

__device__ __forceinline__ uint32_t fbits(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float bitsf(uint32_t u) { return __uint_as_float(u); }

// lowbias32 counter hash, kernels.c:100-106.  The rounding bits of element i of
// a parameter are hash32(uint32(offset + i) ^ stream).
__device__ __forceinline__ uint32_t hash32(uint32_t x)
{
    x = (x ^ (x >> 16)) * 0x7feb352du;
    x = (x ^ (x >> 15)) * 0x846ca68bu;
    return x ^ (x >> 16);
}

// hash32 split after its first xor-shift: hash32(x) == hash32_tail(hash32_head(x)).  The head
// commutes with xor by any k < 2^16 (x >> 16 does not see those bits), so for an index a with
// a % 8 == 0 the streams of a .. a + 7 are hash32_tail(hash32_head(a ^ stream) ^ k), k < 8:
// one head per group of 8.
__device__ __forceinline__ uint32_t hash32_head(uint32_t x) { return x ^ (x >> 16); }
// hash32_tail after its first multiplication: hash32_tail(x) == hash32_tail_mul(x * 0x7feb352d).
__device__ __forceinline__ uint32_t hash32_tail_mul(uint32_t x)
{
    x = (x ^ (x >> 15)) * 0x846ca68bu;
    return x ^ (x >> 16);
}
__device__ __forceinline__ uint32_t hash32_tail(uint32_t x) { return hash32_tail_mul(x * 0x7feb352du); }

// Whether a wavefront's lanes agree in bits 16-18 of their rounding index, and those bits (see hash8).
struct Wave8 {
    uint32_t mixed;   // 0 where the wavefront's indices agree in bits 16-18 (a scalar)
    uint32_t hi3;
};

// The rounding bits of the 8 elements idx .. idx + 7 (idx % 8 == 0) in stream `seed` are
// hash32((idx + k) ^ seed).  idx + k == idx ^ k, so the 8 share one head h (hash32_head commutes
// with xor by k < 2^16) and the tails start from (h ^ k) * 0x7feb352d: hash8_mul gives those 8
// products.  Where the wavefront's indices agree in bits 16-18 (w), h's low 3 bits are the
// wavefront's c = (seed ^ seed >> 16 ^ bits 16-18) & 7 (the index's own low 3 bits are 0), so
// h ^ k = (h & ~7) + (c ^ k), and the 8 products are (h & ~7) * 0x7feb352d plus the
// wavefront-uniform (c ^ k) * 0x7feb352d: a scalar product and one vector add each, in place of a
// vector xor and a vector multiply.
__device__ __forceinline__ void hash8_mul(uint32_t idx, uint32_t seed, const Wave8& w, uint32_t (&x)[8])
{
    constexpr uint32_t kMul = 0x7feb352du;
    const uint32_t head = hash32_head(idx ^ seed);
    // the flag as an opaque scalar at each call: one test shared by the calls would be kept as a
    // lane mask and negated through a vector register
    uint32_t mixed = w.mixed;
    asm volatile("" : "+s"(mixed));
    if (mixed == 0u) {
        const uint32_t c = (seed ^ (seed >> 16) ^ w.hi3) & 7u;
        const uint32_t a = (head & ~7u) * kMul;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            // the uniform product as an opaque scalar: otherwise a + b * kMul is folded back into
            // ((head & ~7) + b) * kMul, one vector multiply per element again
            uint32_t b = (c ^ (uint32_t)k) * kMul;
            asm volatile("" : "+s"(b));
            x[k] = a + b;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = (head ^ (uint32_t)k) * kMul;
    }
}

// r[k] = hash32((idx + k) ^ seed), k < 8.
__device__ __forceinline__ void hash8(uint32_t idx, uint32_t seed, const Wave8& w, uint32_t (&r)[8])
{
    uint32_t x[8];
    hash8_mul(idx, seed, w, x);
#pragma unroll
    for (int k = 0; k < 8; ++k) r[k] = hash32_tail_mul(x[k]);
}

// The low byte of hash32's last step, (y ^ (y >> 16)) & 0xff, in one v_xor_b32 with sub-dword
// operands (the upper half of y as the second source, the result's byte 0 kept and the rest zero).
__device__ __forceinline__ uint32_t hash_low8(uint32_t y)
{
    uint32_t r;
    asm("v_xor_b32_sdwa %0, %1, %1 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_1"
        : "=v"(r) : "v"(y));
    return r;
}

// r[k] = hash32((idx + k) ^ seed) & 0xff, k < 8: the FP24 master's rounding bits.
__device__ __forceinline__ void hash8_low8(uint32_t idx, uint32_t seed, const Wave8& w, uint32_t (&r)[8])
{
    uint32_t x[8];
    hash8_mul(idx, seed, w, x);
#pragma unroll
    for (int k = 0; k < 8; ++k) r[k] = hash_low8((x[k] ^ (x[k] >> 15)) * 0x846ca68bu);
}

// Wave8 of this lane's index (the first active lane's bits stand for the wavefront's).
__device__ __forceinline__ Wave8 wave8_of(uint32_t idx)
{
    const uint32_t hi3 = (idx >> 16) & 7u;
    const uint32_t first = __builtin_amdgcn_readfirstlane(hi3);
    // the lanes that differ, as an integer (the two halves of the ballot or'ed): a bool made here
    // would be kept as a lane mask and turned into an integer through vector registers
    const uint64_t differ = __builtin_amdgcn_ballot_w64(hi3 != first);
    return Wave8{(uint32_t)differ | (uint32_t)(differ >> 32), first};
}

// BF16 bits of x, nearest-even, NaN quietened (kernels.c:108-112), in the low half: the rule
// written out in integer steps.  The kernels use gfx950's conversion instruction instead (below);
// this form is what adambridge_check_conversions compares that instruction with.
__device__ __forceinline__ uint32_t bf16_rne_soft(float x)
{
    const uint32_t b = fbits(x);
    const uint32_t r = b + 0x7fffu + ((b >> 16) & 1u);
    return ((x != x) ? (b | 0x00400000u) : r) >> 16;
}

// BF16 bits of x0 (low half) and x1 (high half), one v_cvt_pk_bf16_f32.  The instruction rounds
// to nearest-even and turns a NaN into its top 16 bits with the quiet bit set: the same bits as
// bf16_rne_soft for every FP32 input, NaN and infinity included (compared over all 2^32 bit
// patterns by adambridge_check_conversions).
__device__ __forceinline__ uint32_t bf16x2_rne(float x0, float x1)
{
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x0, x1}, bf16x2));
}

__device__ __forceinline__ uint32_t bf16_rne(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }

// A moment stored as BF16: stochastic (bits + low 16 bits of r, no NaN special
// case) or nearest-even, kernels.c:120-126.  Result in the low half.  The
// rounding mode is a template parameter so the per-element code is straight-line.
template <bool SR>
__device__ __forceinline__ uint32_t bf16_store(float x, uint32_t r)
{
    if constexpr (SR) return (fbits(x) + (r & 0xffffu)) >> 16;
    else return bf16_rne(x);
}

// FP24 master round (kernels.c:145-150): the FP32 bits kept in the top 24.
template <bool SR>
__device__ __forceinline__ uint32_t f24_round(float x, uint32_t r)
{
    const uint32_t b = fbits(x);
    const uint32_t t = (SR ? b + (r & 0xffu) : b + 0x7fu + ((b >> 8) & 1u)) & ~0xffu;
    return (x != x) ? (b | 0x00400000u) : t;
}

// ----------------------------------------------------------------- FP8 codec

// Code -> value (kernels.c:826-843) with gfx950's conversion instructions, which implement the
// OCP E4M3FN (m) and E5M2 (sqrt v) formats the reference decodes: every finite code converts
// exactly (checked against the reference's tables for all 256 codes of both formats).  For a NaN
// code the hardware returns one fixed NaN; the code's own sign is copied in, which gives the
// reference's quiet NaN with that sign.  SEL: which byte of `word` holds the code.
template <int SEL>
__device__ __forceinline__ float e4m3_decode(uint32_t word)
{
    const float a = __builtin_amdgcn_cvt_f32_fp8((int)word, SEL);
    const uint32_t sign = (word << (24 - 8 * SEL)) & 0x80000000u;
    return bitsf((fbits(a) & 0x7fffffffu) | sign);
}

template <int SEL>
__device__ __forceinline__ float e5m2_decode(uint32_t word)
{
    const float a = __builtin_amdgcn_cvt_f32_bf8((int)word, SEL);
    const uint32_t sign = (word << (24 - 8 * SEL)) & 0x80000000u;
    return bitsf((fbits(a) & 0x7fffffffu) | sign);
}

// Codes in bytes 2H and 2H + 1 of `word` as FP32, one v_cvt_pk_f32_fp8 / v_cvt_pk_f32_bf8:
// the reference's value for every code but NaN, whose sign the instruction drops (the kernels
// then restore it with the decoders above; adambridge_check_conversions, check 6).
template <bool E5M2, bool H>
__device__ __forceinline__ void fp8_decode2(uint32_t word, float& x0, float& x1)
{
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    f32x2 d;
    if constexpr (E5M2) d = __builtin_amdgcn_cvt_pk_f32_bf8((int)word, H);
    else d = __builtin_amdgcn_cvt_pk_f32_fp8((int)word, H);
    x0 = d.x;
    x1 = d.y;
}

// The value of an FP8 code from the format's definition (OCP E4M3FN / E5M2), for the self-check.
template <bool E5M2>
__device__ __forceinline__ float fp8_value_soft(uint32_t code)
{
    constexpr int kM = E5M2 ? 2 : 3, kBias = E5M2 ? 15 : 7, kEmax = E5M2 ? 31 : 15;
    const int e = (int)((code >> kM) & (uint32_t)kEmax);
    const uint32_t f = code & ((1u << kM) - 1u);
    float mag;
    if (E5M2 && e == kEmax) mag = f ? __builtin_nanf("") : __builtin_inff();
    else if (!E5M2 && e == kEmax && f == 7u) mag = __builtin_nanf("");
    else if (e == 0) mag = ldexpf((float)f, 1 - kBias - kM);
    else mag = ldexpf((float)(f + (1u << kM)), e - kBias - kM);
    return (code & 0x80u) ? -mag : mag;
}

// Value -> code, the steps of kernels.c:857-876: optional stochastic truncation
// of the FP32 bits to the format's mantissa width, saturation at the format's
// maximum, nearest-even for normals, nearest-even for subnormals, the sign
// re-attached and NaN mapped to the format's NaN code.  Written on the
// magnitude's bit pattern: for non-negative floats (infinity included) integer
// order is float order, so the saturation is one unsigned min and the
// normal/subnormal choice one unsigned compare; a NaN magnitude goes through
// either and is replaced at the end.
template <int MBITS, int BIAS, bool SR>
__device__ __forceinline__ uint32_t fp8_encode(float x, uint32_t r)
{
    constexpr unsigned kCut = 23 - MBITS;                               // FP32 mantissa bits dropped
    constexpr uint32_t kBelow = (1u << kCut) - 1u;
    constexpr uint32_t kMaxBits = MBITS == 3 ? 0x43e00000u : 0x47600000u;   // 448, 57344
    constexpr uint32_t kMinNormalBits = (uint32_t)(128 - BIAS) << 23;       // 2^(1-bias)
    constexpr uint32_t kRebias = (uint32_t)(127 - BIAS) << MBITS;
    constexpr uint32_t kNanCode = MBITS == 3 ? 0x7fu : 0x7eu;
    const uint32_t in = fbits(x);
    const uint32_t kept = SR ? (in + (r & kBelow)) & ~kBelow : in;
    const uint32_t mag = __builtin_elementwise_min(kept & 0x7fffffffu, kMaxBits);
    uint32_t code;
    if (mag >= kMinNormalBits) {
        // exponent and kept mantissa are adjacent above bit kCut: a carry out of the
        // mantissa moves to the next binade, and re-biasing is one subtraction
        const uint32_t rounded = SR ? mag : mag + (kBelow >> 1) + ((mag >> kCut) & 1u);
        code = (rounded >> kCut) - kRebias;
    } else {
        // |x| * 2^(bias+mbits-1) is exact (a power-of-two scaling); adding 2^23 leaves
        // the nearest-even integer in the low mantissa bits
        const float scaled = __builtin_fmaf(bitsf(mag), bitsf((uint32_t)(127 + BIAS + MBITS - 1) << 23), 0x1p23f);
        code = fbits(scaled) & 0xffu;
    }
    return ((in >> 24) & 0x80u) | ((x != x) ? kNanCode : code);
}

template <bool SR>
__device__ __forceinline__ uint32_t e4m3_encode(float x, uint32_t r) { return fp8_encode<3, 7, SR>(x, r); }
template <bool SR>
__device__ __forceinline__ uint32_t e5m2_encode(float x, uint32_t r) { return fp8_encode<2, 15, SR>(x, r); }

// gfx950's FP8 conversion instructions against fp8_encode, over every FP32 bit pattern
// (adambridge_check_conversions), with the input first clamped to [-max, max] (one v_med3_f32;
// the reference saturates there too):
//   - nearest-even, v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32: the same code for every x but NaN,
//     subnormal results and zeros included;
//   - stochastic, v_cvt_sr_fp8_f32 / v_cvt_sr_bf8_f32: the same code for every x but NaN with
//     |x| >= the smallest normal, when the instruction's 32-bit random operand carries the
//     reference's random bits r & (2^(23-mbits) - 1) at its top, i.e. r << (9 + mbits).  Below
//     the smallest normal the instruction rounds at the subnormal spacing, where the reference
//     truncates at the normal mantissa width first.
// fp8_hw_range(x) tells whether x is in the range where the instruction is used:
// fp8_hw_offset(x) <= fp8_hw_span, so that several values are tested at once by the unsigned
// maximum of their offsets.
template <bool E5M2, bool SR>
constexpr uint32_t fp8_hw_min = SR ? (E5M2 ? 0x38800000u : 0x3c800000u) : 0u;   // 2^-14, 2^-6

template <bool E5M2, bool SR>
constexpr uint32_t fp8_hw_span = (0x7f800000u - fp8_hw_min<E5M2, SR>) << 1;

// The magnitude's bits shifted out of the sign, less the range's start: below it (zero
// included) wraps above the span, NaN lies above it.
template <bool E5M2, bool SR>
__device__ __forceinline__ uint32_t fp8_hw_offset(float x)
{
    return (fbits(x) << 1) - (fp8_hw_min<E5M2, SR> << 1);
}

template <bool E5M2, bool SR>
__device__ __forceinline__ bool fp8_hw_range(float x)
{
    return fp8_hw_offset<E5M2, SR>(x) <= fp8_hw_span<E5M2, SR>;
}

template <bool E5M2>
__device__ __forceinline__ float fp8_saturate(float x)
{
    constexpr float kMax = E5M2 ? 57344.0f : 448.0f;
    return __builtin_amdgcn_fmed3f(x, -kMax, kMax);
}

// Stochastic code of x into byte B of `word` (the other bytes kept).
template <bool E5M2, int B>
__device__ __forceinline__ uint32_t fp8_hw_sr(float x, uint32_t r, uint32_t word)
{
    const float c = fp8_saturate<E5M2>(x);
    if constexpr (E5M2) return (uint32_t)__builtin_amdgcn_cvt_sr_bf8_f32(c, (int)(r << 11), (int)word, B);
    else return (uint32_t)__builtin_amdgcn_cvt_sr_fp8_f32(c, (int)(r << 12), (int)word, B);
}

// Nearest-even codes of x0, x1 into bytes 2H, 2H + 1 of `word` (the other half kept).
template <bool E5M2, bool H>
__device__ __forceinline__ uint32_t fp8_hw_rne2(float x0, float x1, uint32_t word)
{
    const float c0 = fp8_saturate<E5M2>(x0), c1 = fp8_saturate<E5M2>(x1);
    if constexpr (E5M2) return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(c0, c1, (int)word, H);
    else return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c0, c1, (int)word, H);
}

// ----------------------------------------------------------- element steps

// AdamW, kernels.c:447-455 (FUSED: the AVX-512/AVX2 bodies) and 171-176 (the
// scalar path: every product and sum rounded on its own).  m and v are
// updated in place; sq receives sqrt(new v); returns the new master before
// storage rounding.
template <bool FUSED>
__device__ __forceinline__ float adamw(float p, float g, float& m, float& v, const Coef& c, float& sq)
{
    const float pd = p * c.decay;
    if (FUSED) {
        m = __builtin_fmaf(c.b1, m, c.omb1 * g);
        v = __builtin_fmaf(c.b2, v, c.omb2 * (g * g));
        sq = __builtin_sqrtf(v);
        const float den = __builtin_fmaf(sq, c.isbc2, c.eps);
        return __builtin_fmaf(-c.step, m / den, pd);
    }
    const float m1 = c.b1 * m;
    const float m2 = c.omb1 * g;
    m = m1 + m2;
    const float gg = g * g;
    const float v1 = c.b2 * v;
    const float v2 = c.omb2 * gg;
    v = v1 + v2;
    sq = __builtin_sqrtf(v);
    const float sb = sq * c.isbc2;
    const float den = sb + c.eps;
    const float u = c.step * (m / den);
    return pd - u;
}

template <bool FUSED>
__device__ __forceinline__ float adamw(float p, float g, float& m, float& v, const Coef& c)
{
    float sq;
    return adamw<FUSED>(p, g, m, v, c, sq);
}

// Correctly rounded square root for 2^-100 <= x < 2^100 in 5 instructions, one of them a
// transcendental (the general sqrtf also scales denormals and handles 0, infinity and NaN): from
// y = rsq(x), the root g = x y and one Newton correction g + (x - g^2) y / 2.  g is within a few
// ulp of the root there, so the residual x - g^2 is a float and one fused multiply-add gives it
// exactly.  The result is the nearest root for every x in the range, decided in exact integer
// arithmetic by adambridge_check_conversions (check 5).  (An earlier form corrected v_sqrt_f32's
// root with the same step -- two transcendentals, also exact; the correction with v_rcp_f32(s) / 2
// in place of rsq(x) / 2 misses the nearest root for 100 inputs of the range.)
constexpr uint32_t kSqrtMidLo = 0x0d800000u, kSqrtMidSpan = 0x71800000u - 0x0d800000u;

__device__ __forceinline__ bool sqrt_mid_range(float x) { return fbits(x) - kSqrtMidLo < kSqrtMidSpan; }

__device__ __forceinline__ float sqrt_mid(float x)
{
    const float y = __builtin_amdgcn_rsqf(x);
    const float g = x * y;
    const float r = __builtin_fmaf(-g, g, x);
    return __builtin_fmaf(r, y * 0.5f, g);
}

// The fused AdamW step of two elements (the pair kernel's body): the same operations as
// adamw<true> on each, with the square roots of the new second moments taken by sqrt_mid when
// every one of the wavefront lies in its range (2^-100 <= v < 2^100, a uniform branch), where it
// equals the correctly rounded root; outside it, sqrtf.  Saves ~12 instructions per element.
__device__ __forceinline__ void adamw_pair_fused(float& p0, float& p1, float g0, float g1, float& m0, float& m1,
                                                 float& v0, float& v1, const Coef& c)
{
    m0 = __builtin_fmaf(c.b1, m0, c.omb1 * g0);
    m1 = __builtin_fmaf(c.b1, m1, c.omb1 * g1);
    v0 = __builtin_fmaf(c.b2, v0, c.omb2 * (g0 * g0));
    v1 = __builtin_fmaf(c.b2, v1, c.omb2 * (g1 * g1));
    const uint32_t worst = __builtin_elementwise_max(fbits(v0) - kSqrtMidLo, fbits(v1) - kSqrtMidLo);
    float s0, s1;
    if (__all(worst < kSqrtMidSpan)) {
        s0 = sqrt_mid(v0);
        s1 = sqrt_mid(v1);
    } else {
        s0 = __builtin_sqrtf(v0);
        s1 = __builtin_sqrtf(v1);
    }
    const float d0 = __builtin_fmaf(s0, c.isbc2, c.eps), d1 = __builtin_fmaf(s1, c.isbc2, c.eps);
    p0 = __builtin_fmaf(-c.step, m0 / d0, p0 * c.decay);
    p1 = __builtin_fmaf(-c.step, m1 / d1, p1 * c.decay);
}

__device__ __forceinline__ float adamw_sel(float p, float g, float& m, float& v, const Coef& c, bool fused,
                                           float& sq)
{
    return fused ? adamw<true>(p, g, m, v, c, sq) : adamw<false>(p, g, m, v, c, sq);
}

__device__ __forceinline__ float adamw_sel(float p, float g, float& m, float& v, const Coef& c, bool fused)
{
    float sq;
    return adamw_sel(p, g, m, v, c, fused, sq);
}

// x / s, correctly rounded, for every element x of one FP8 block divided by the block's scale s
// (kernels.c:1049-1057), at a fraction of the cost of a division each: y = 1/s once per block,
// then per element q = x*y and one residual correction q + (x - q*s)*y with fused multiply-adds
// (Markstein's theorem: with y within half an ulp of 1/s and q within one ulp of x/s, the
// corrected quotient is the correctly rounded one, provided x - q*s is exact).  Blocks whose
// absmax is below 2^-40 are first scaled by 2^100, exactly, so the residual stays exact for
// every element whose quotient reaches the FP8 formats (>= 2^-18); smaller quotients may differ
// in their last bit and encode to the same signed zero code either way.  Checked on 4e9 random
// and edge-case blocks against division and the encoders.  A zero or infinite scale takes the
// division.
struct BlockDiv {
    float s, s2, y, pre;
    bool fast;
};

// 1 / s correctly rounded, for s in [2^-126, 2^126) (normal, with a normal reciprocal): the
// hardware reciprocal (within one ulp) refined by one Newton step in fused multiply-adds,
// e = 1 - s y0 (exact), y = y0 + e y0.  That this is the float nearest to 1/s was checked for
// every s of that range against the exact quotient (adambridge_check_conversions).
constexpr uint32_t kRecipLo = 0x00800000u, kRecipSpan = 0x7e800000u - 0x00800000u;

__device__ __forceinline__ bool recip_range(float s) { return fbits(s) - kRecipLo < kRecipSpan; }

__device__ __forceinline__ float recip_nearest(float s)
{
    const float y0 = __builtin_amdgcn_rcpf(s);
    const float e = __builtin_fmaf(-s, y0, 1.0f);
    return __builtin_fmaf(e, y0, y0);
}

// The AdamW step's m / den, correctly rounded, in 6 instructions instead of the general
// division's 11, where every operand is in range: y = 1/den correctly rounded (recip_nearest),
// q = m y, and one residual correction q + (m - q den) y (Markstein's theorem, as for the FP8 block
// quotients).  The range: 2^-60 <= |m| <= 2^60 (quot_m_offset <= kQuotMSpan, for a single value;
// adamw8_fused_q tests a lane's largest and smallest |m|), and 2^-50 <= den < 2^61, which holds
// when every v is in sqrt_mid's range (so sqrt(v) lies in [2^-50, 2^50)) and the step's
// 1 <= inv_sqrt_bc2 <= 2^10 and 0 <= eps <= 2^30 (checked on the host: the segment flag of
// adamw8_fused_q's caller).  Then y, q and the quotient are normal
// (|m / den| in [2^-121, 2^110]) and m - q den, about |m| 2^-24 >= 2^-84, is exact, which the
// theorem needs.  Zero m lies outside the range: its wavefront divides.
constexpr uint32_t kQuotMLo = 0x21800000u, kQuotMSpan = (0x5d800000u - 0x21800000u) << 1;   // 2^-60, 2^60

__device__ __forceinline__ uint32_t quot_m_offset(float m) { return (fbits(m) << 1) - (kQuotMLo << 1); }

__device__ __forceinline__ float quot_fast(float m, float den)
{
    const float y = recip_nearest(den);
    const float q = m * y;
    return __builtin_fmaf(__builtin_fmaf(-q, den, m), y, q);
}

// The fused form of adamw for a lane's 8 elements, up to the quotients q = m / den (the master's
// update follows in adamw8_fused).  The square roots take sqrt_mid when every new v
// of the wavefront lies in its range (one uniform branch), sqrtf otherwise; with ``fastdiv`` (the
// step's coefficients are in quot_fast's range) and every m of the wavefront in range as well, the
// quotients m / den take quot_fast.  Returns whether sqrt_mid was taken, i.e. whether every v, and
// so every sq, of the wavefront is positive and finite; m_plain receives whether quot_fast was
// taken, i.e. whether every new m of the wavefront is finite with 2^-60 <= |m| <= 2^60, and m_low
// then the smallest |m| of the lane.
//
// The range tests take each lane's extremes: the v's as unsigned bits (a negative v, -0 and NaN
// lie above the range's end, +0 below its start), the |m| by gfx950's three-operand maximum and
// minimum that keep NaN (v_maximum3_f32, v_minimum3_f32: a NaN fails the test).
__device__ __forceinline__ bool adamw8_fused_q(const float (&g)[8], float (&m)[8], float (&v)[8], const Coef& c,
                                               float (&sq)[8], bool fastdiv, bool& m_plain, float& m_low,
                                               float (&q)[8])
{
    uint32_t v_hi = 0u, v_lo = 0xffffffffu;   // the largest and smallest bits of the new v's
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        m[k] = __builtin_fmaf(c.b1, m[k], c.omb1 * g[k]);
        v[k] = __builtin_fmaf(c.b2, v[k], c.omb2 * (g[k] * g[k]));
        v_hi = __builtin_elementwise_max(v_hi, fbits(v[k]));
        v_lo = __builtin_elementwise_min(v_lo, fbits(v[k]));
    }
    const bool mid = __all(v_lo >= kSqrtMidLo) && __all(v_hi < kSqrtMidLo + kSqrtMidSpan);
    if (mid) {
#pragma unroll
        for (int k = 0; k < 8; ++k) sq[k] = sqrt_mid(v[k]);
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) sq[k] = __builtin_sqrtf(v[k]);
    }
    bool fast = false;
    float m_min = 0.0f;
    if (mid && fastdiv) {
        float m_max = fabsf(m[0]);
        m_min = fabsf(m[0]);
#pragma unroll
        for (int k = 1; k < 8; ++k) {
            m_max = __builtin_elementwise_maximum(m_max, fabsf(m[k]));
            m_min = __builtin_elementwise_minimum(m_min, fabsf(m[k]));
        }
        fast = __all(m_max <= 0x1p60f) && __all(m_min >= 0x1p-60f);
    }
    if (fast) {
#pragma unroll
        for (int k = 0; k < 8; ++k) q[k] = quot_fast(m[k], __builtin_fmaf(sq[k], c.isbc2, c.eps));
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) q[k] = m[k] / __builtin_fmaf(sq[k], c.isbc2, c.eps);
    }
    m_plain = fast;
    m_low = m_min;
    return mid;
}

// adamw8_fused_q, then the masters: p = p decay - step q (one fused multiply-add each).
__device__ __forceinline__ bool adamw8_fused(float (&p)[8], const float (&g)[8], float (&m)[8], float (&v)[8],
                                             const Coef& c, float (&sq)[8], bool fastdiv, bool& m_plain,
                                             float& m_low)
{
    float q[8];
    const bool mid = adamw8_fused_q(g, m, v, c, sq, fastdiv, m_plain, m_low, q);
#pragma unroll
    for (int k = 0; k < 8; ++k) p[k] = __builtin_fmaf(-c.step, q[k], p[k] * c.decay);
    return mid;
}

__device__ __forceinline__ BlockDiv block_div(float s, float absmax)
{
    BlockDiv d;
    d.s = s;
    d.fast = s > 0.0f && s <= 3.40282347e38f;
    d.pre = absmax < 0x1p-40f ? 0x1p100f : 1.0f;
    d.s2 = s * d.pre;
    d.y = recip_range(d.s2) ? recip_nearest(d.s2) : 1.0f / d.s2;
    return d;
}

// SCALED: the block was scaled by d.pre (absmax < 2^-40).  PLAIN: x is never -0, and a NaN x
// needs no sign (the sqrt-domain v, whose NaNs the encoder replaces by 0; m wherever the AdamW
// step took quot_fast, i.e. every m of the wavefront is finite and nonzero), so the corrected
// quotient needs no care for signs: it is the correctly rounded quotient, with x's sign, for every
// other x; only -0 would come out as +0 (q + 0*y), and a NaN without x's sign.  Otherwise x's sign
// bit is copied into the result, which is exact for every other x (the quotient has x's sign) and
// gives -0 / NaN the sign the reference's division gives them.
template <bool SCALED, bool PLAIN>
__device__ __forceinline__ float block_quot_fast(float x, const BlockDiv& d)
{
    const float xs = SCALED ? x * d.pre : x;
    const float q = xs * d.y;
    const float r = __builtin_fmaf(-q, d.s2, xs);
    const float qc = __builtin_fmaf(r, d.y, q);
    if constexpr (PLAIN) return qc;
    return bitsf(fbits(qc) | (fbits(x) & 0x80000000u));
}

// Lion, kernels.c:1107-1124: c = b1 m + (1-b1) g (fused), p = p*decay - lr*sign(c)
// (fused, sign(0) = sign(NaN) = 0), m = b2 m + (1-b2) g (fused).  Identical on
// every reference path, so there is no tail form.
__device__ __forceinline__ float lion(float p, float g, float& m, const Coef& c)
{
    const float cc = __builtin_fmaf(c.b1, m, c.omb1 * g);
    const float u = cc > 0.0f ? c.step : (cc < 0.0f ? -c.step : 0.0f);
    const float pn = __builtin_fmaf(p, c.decay, -u);
    m = __builtin_fmaf(c.b2, m, c.omb2 * g);
    return pn;
}

}  // namespace abh
