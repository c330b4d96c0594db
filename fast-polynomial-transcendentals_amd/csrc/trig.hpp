// trig.hpp -- paired sin/cos programs and the fixed-point RoPE phase.
//
// Half-turn programs (angles in radians, FP32):
//   k = round(angle / pi) with the 1.5*2^23 shifter (one FMA, round to
//   nearest; Muller, "Elementary Functions", ch. 11), r = angle - k*pi with a
//   one-term FP32 pi, sign = parity(k).  r in [-pi/2, pi/2] is rounded to the
//   16-bit format, sq = r*r, sin = r * S(sq), cos = C(sq) (Horner in sq, one
//   rounding per step), and both results take the sign bit of parity(k).
// RoPE programs (phase in turns, Q0.32): phase = position * increment
//   (uint32 wrap), the top 17 bits give a signed Q15 quarter-turn residual r
//   in [-1, 1) and a sign; sin/cos of r*pi/2 come from S(sq) / C(sq) with
//   coefficients that absorb pi/2.
// Coefficients: autonumerics_zero/spline_ops/sincos_kernels.cu (each table
// row cites its evaluator).
#pragma once

#include "programs.hpp"

namespace pt {

struct SinCosProg {
    int ns;         // sin coefficients (highest power of sq first)
    float s[4];
    int nc;         // cos coefficients (highest power of sq first)
    float c[4];
};

enum SinCosId : int {
    kBf16HalfD3D4 = 0,   // PolynomialD3D4HalfTurnBF16, sincos_kernels.cu:681-718
    kBf16HalfD5D6 = 1,   // PolynomialD5D6HalfTurnBF16, :874-920
    kF16HalfD3D4 = 2,    // PolynomialD3D4HalfTurnFP16, :644-679
    kF16HalfD5D4 = 3,    // evaluate_half_turn_d5_d4_fp16, :720-761
    kF16HalfD5D6 = 4,    // PolynomialD5D6HalfTurnFP16, :820-860
    kF16HalfD7D6 = 5,    // PolynomialD7D6HalfTurnFP16, :773-818
    kF16RopeQ15D5D6 = 6, // evaluate_half_turn_q15_d5_d6_fp16, :1289-1328
};

constexpr SinCosProg kSinCos[7] = {
    {2, {-0.1455078125f, 0.98828125f}, 3, {0.037109375f, -0.49609375f, 1.0f}},
    {3, {0.007598876953125f, -0.166015625f, 1.0f}, 4,
     {-0.00125885009765625f, 0.04150390625f, -0.5f, 1.0f}},
    {2, {-0.14501953125f, 0.98876953125f}, 3,
     {0.037200927734375f, -0.496337890625f, 0.99951171875f}},
    {3, {0.0074920654296875f, -0.16552734375f, 0.99951171875f}, 3,
     {0.036773681640625f, -0.49560546875f, 0.99951171875f}},
    {3, {0.0074920654296875f, -0.16552734375f, 0.99951171875f}, 4,
     {-0.0012674331665039062f, 0.041412353515625f, -0.499755859375f, 1.0f}},
    {4, {-0.00018227100372314453f, 0.00829315185546875f, -0.1666259765625f, 1.0f}, 4,
     {-0.0012674331665039062f, 0.041412353515625f, -0.499755859375f, 1.0f}},
    {3, {0.072021484375f, -0.64208984375f, 1.5703125f}, 4,
     {-0.0190887451171875f, 0.25244140625f, -1.2333984375f, 1.0f}},
};

// FP32 reduction to a half turn.  1/pi and pi are the FP32 roundings of the
// constants; the shifter 1.5*2^23 makes the FMA round k to an integer.
constexpr float kInvPi = 0.318309886183790671538f;
constexpr float kPiF32 = 3.14159265358979323846f;
constexpr float kShifter = 12582912.0f;

__device__ __forceinline__ void reduce_half_turn(float angle, float& r, uint32_t& sign) {
    const float biased = __builtin_fmaf(angle, kInvPi, kShifter);
    const float k = biased - kShifter;
    r = __builtin_fmaf(k, -kPiF32, angle);
    sign = (as_u32(biased) & 1u) << 31;
}

// FP16 packed program on two lanes of reduced arguments `r` (h2) with
// combined sign bits `signs` (bit 15 low lane, bit 31 high lane).
template <int P>
__device__ __forceinline__ void f16_sincos_reduced(h2_t r, uint32_t signs, uint32_t& cos2,
                                                   uint32_t& sin2) {
    constexpr SinCosProg Q = kSinCos[P];
    const h2_t sq = r * r;
    h2_t sp = __builtin_elementwise_fma(as_h2(f16_pair_bits(Q.s[0])), sq, as_h2(f16_pair_bits(Q.s[1])));
#pragma unroll
    for (int i = 2; i < Q.ns; ++i) sp = __builtin_elementwise_fma(sp, sq, as_h2(f16_pair_bits(Q.s[i])));
    const h2_t sr = r * sp;
    h2_t cp = __builtin_elementwise_fma(as_h2(f16_pair_bits(Q.c[0])), sq, as_h2(f16_pair_bits(Q.c[1])));
#pragma unroll
    for (int i = 2; i < Q.nc; ++i) cp = __builtin_elementwise_fma(cp, sq, as_h2(f16_pair_bits(Q.c[i])));
    sin2 = as_u32(sr) ^ signs;
    cos2 = as_u32(cp) ^ signs;
}

// FP16 half-turn program on two FP32 angles.
template <int P>
__device__ __forceinline__ void f16_sincos(float a_lo, float a_hi, uint32_t& cos2, uint32_t& sin2) {
    float r_lo, r_hi;
    uint32_t s_lo, s_hi;
    reduce_half_turn(a_lo, r_lo, s_lo);
    reduce_half_turn(a_hi, r_hi, s_hi);
    const h2_t r = {(_Float16)r_lo, (_Float16)r_hi};
    f16_sincos_reduced<P>(r, (s_lo >> 16) | s_hi, cos2, sin2);
}

// Horner in sq over n BF16 coefficients (highest power first), every step
// rounded to BF16 except the last, which is returned before its rounding.
__device__ __forceinline__ float bf16_horner_open(const float (&k)[4], int n, float sq) {
    float h = bf16_value(k[0]);
#pragma unroll
    for (int i = 1; i < n - 1; ++i) h = bfma(h, sq, bf16_value(k[i]));
    return __builtin_fmaf(h, sq, bf16_value(k[n - 1]));
}

// BF16 half-turn program on one FP32 angle; results are the FP32 values of
// the last steps (signs applied) before their final rounding, which the
// caller's pack to BF16 performs: RNE is odd-symmetric, so rounding after the
// sign is applied gives the same bits.
template <int P>
__device__ __forceinline__ void bf16_sincos_lane(float angle, float& c, float& s) {
    constexpr SinCosProg Q = kSinCos[P];
    float r;
    uint32_t sign;
    reduce_half_turn(angle, r, sign);
    r = rbf(r);
    const float sq = rbf(r * r);
    const float sp = rbf(bf16_horner_open(Q.s, Q.ns, sq));
    s = as_f32(as_u32(r * sp) ^ sign);
    c = as_f32(as_u32(bf16_horner_open(Q.c, Q.nc, sq)) ^ sign);
}

// ---------------------------------------------------------------------------
// quarter-turn reduction and quadrant restore
// ---------------------------------------------------------------------------
//
// k = round(angle * 2/pi), r = angle - k*pi/2, quadrant = k mod 4; then
// sin(angle) = +-{sin r | cos r} and cos(angle) = +-{cos r | sin r}: odd
// quadrants swap the two, quadrants 2-3 negate sin and 1-2 negate cos.

constexpr float kInvHalfPi = 0.63661977236758134308f;
constexpr float kHalfPiF32 = 1.57079637050628662109375f;       // FP32(pi/2)
constexpr float kHalfPiHi = 1.57079625129699707031f;           // Cody-Waite split
constexpr float kHalfPiLo = 7.54978941586159635335e-08f;
constexpr float kPiHi = 3.141592502593994140625f;
constexpr float kPiLo = 1.50995788317231927067e-07f;

// Cody-Waite with an explicit round-to-nearest-even conversion
// (reduce_to_quarter_turn, sincos_kernels.cu:24-37).  The conversion
// saturates and maps NaN to 0 like cvt.rni.s32.f32.
__device__ __forceinline__ void reduce_quarter_cw(float angle, float& r, uint32_t& quadrant) {
    const float kf_raw = __builtin_rintf(angle * kInvHalfPi);
    int q;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(q) : "v"(kf_raw));
    const float kf = (float)q;
    r = __builtin_fmaf(kf, -kHalfPiHi, angle);
    r = __builtin_fmaf(kf, -kHalfPiLo, r);
    quadrant = (uint32_t)q;
}

// Shifter rounding: the FMA with 1.5*2^23 leaves k in the low mantissa bits
// of `biased`, so the quadrant is read from its bits with no conversion
// (reduce_to_quarter_turn_magic_bias{,_fast}, sincos_kernels.cu:39-70).
template <bool TwoTerm>
__device__ __forceinline__ void reduce_quarter_shift(float angle, float& r, uint32_t& quadrant) {
    const float biased = __builtin_fmaf(angle, kInvHalfPi, kShifter);
    const float k = biased - kShifter;
    if constexpr (TwoTerm) {
        r = __builtin_fmaf(k, -kHalfPiHi, angle);
        r = __builtin_fmaf(k, -kHalfPiLo, r);
    } else {
        r = __builtin_fmaf(k, -kHalfPiF32, angle);
    }
    quadrant = as_u32(biased);
}

// Half turn with a two-term pi (reduce_to_half_turn_magic_bias, :72-86).
__device__ __forceinline__ void reduce_half_turn_two_term(float angle, float& r, uint32_t& sign) {
    const float biased = __builtin_fmaf(angle, kInvPi, kShifter);
    const float k = biased - kShifter;
    r = __builtin_fmaf(k, -kPiHi, angle);
    r = __builtin_fmaf(k, -kPiLo, r);
    sign = (as_u32(biased) & 1u) << 31;
}

// FP32 quadrant restore (restore_quadrant, :104-118).
__device__ __forceinline__ void restore_quadrant_f32(float sr, float cr, uint32_t q, float& s,
                                                     float& c) {
    const bool swap = (q & 1u) != 0;
    const float sm = swap ? cr : sr;
    const float cm = swap ? sr : cr;
    s = as_f32(as_u32(sm) ^ ((q & 2u) << 30));
    c = as_f32(as_u32(cm) ^ (((q + 1u) & 2u) << 30));
}

// Packed 16-bit quadrant restore on two lanes (restore_quadrant_packed16,
// :424-443): swap masks select per lane, signs land in bits 15 and 31.
__device__ __forceinline__ void restore_quadrant_pair(uint32_t sr, uint32_t cr, uint32_t q_lo,
                                                      uint32_t q_hi, uint32_t& s, uint32_t& c) {
    const uint32_t swap = ((0u - (q_lo & 1u)) & 0x0000ffffu) | ((0u - (q_hi & 1u)) & 0xffff0000u);
    const uint32_t x = (sr ^ cr) & swap;
    const uint32_t ss = ((q_lo & 2u) << 14) | ((q_hi & 2u) << 30);
    const uint32_t cs = (((q_lo + 1u) & 2u) << 14) | (((q_hi + 1u) & 2u) << 30);
    s = sr ^ x ^ ss;
    c = cr ^ x ^ cs;
}

// ---------------------------------------------------------------------------
// FP32 paired programs (sincos_kernels.cu:120-406)
// ---------------------------------------------------------------------------

enum F32SinCosId : int {
    kF32D3D4 = 0,          // PolynomialD3D4, :129-160 (Cody-Waite quarter turn)
    kF32D3D4Shift = 1,     // PolynomialD3D4MagicBias, :207-237
    kF32D5D4 = 2,          // PolynomialD5D4, :331-365
    kF32D7D6 = 3,          // PolynomialD7D6, :367-406
    kF32HalfD5D4Ls = 4,    // PolynomialD5D4HalfTurnLS, :263-279
    kF32HalfD5D4Sollya = 5,     // PolynomialD5D4HalfTurnSollya, :281-297
    kF32HalfD5D4SollyaFast = 6, // PolynomialD5D4HalfTurnSollyaFast, :299-329
};

enum Reduction : int { kQuarterCw = 0, kQuarterShift2 = 1, kHalfShift2 = 2, kHalfShift1 = 3 };

struct F32SinCosProg {
    int red;
    SinCosProg p;
};

constexpr F32SinCosProg kF32SinCos[7] = {
    {kQuarterCw, {2, {-0.16034401953220367431640625f, 0.99903142452239990234375f}, 3,
                  {0.0403986163437366485595703125f, -0.4997082054615020751953125f,
                   0.999990046024322509765625f}}},
    {kQuarterShift2, {2, {-0.16034401953220367431640625f, 0.99903142452239990234375f}, 3,
                      {0.0403986163437366485595703125f, -0.4997082054615020751953125f,
                       0.999990046024322509765625f}}},
    {kQuarterCw, {3, {0.008137642405927181f, -0.16661198437213898f, 0.9999962449073792f}, 3,
                  {0.04051213711500168f, -0.499763548374176f, 0.999993085861206f}}},
    {kQuarterCw, {4, {-0.00019484198128338903f, 0.00833179522305727f, -0.1666664183139801f, 1.0f}, 4,
                  {-0.0013605882413685322f, 0.041656624525785446f, -0.49999886751174927f, 1.0f}}},
    {kHalfShift2, {3, {0.00757423602044582366943359375f, -0.16582702100276947021484375f,
                       0.999771416187286376953125f}, 3,
                   {0.0372092612087726593017578125f, -0.4963922202587127685546875f,
                    0.999579489231109619140625f}}},
    {kHalfShift2, {3, {0.0075143859721720218658447265625f, -0.1656731069087982177734375f,
                       0.999696791172027587890625f}, 3,
                   {0.03679168224334716796875f, -0.495580852031707763671875f,
                    0.9994032382965087890625f}}},
    {kHalfShift1, {3, {0.0075143859721720218658447265625f, -0.1656731069087982177734375f,
                       0.999696791172027587890625f}, 3,
                   {0.03679168224334716796875f, -0.495580852031707763671875f,
                    0.9994032382965087890625f}}},
};

template <int P>
__device__ __forceinline__ void f32_sincos(float angle, float& c, float& s) {
    constexpr F32SinCosProg Q = kF32SinCos[P];
    float r;
    uint32_t q;
    if constexpr (Q.red == kQuarterCw) reduce_quarter_cw(angle, r, q);
    else if constexpr (Q.red == kQuarterShift2) reduce_quarter_shift<true>(angle, r, q);
    else if constexpr (Q.red == kHalfShift2) reduce_half_turn_two_term(angle, r, q);
    else reduce_half_turn(angle, r, q);
    const float sq = r * r;
    float sp = __builtin_fmaf(Q.p.s[0], sq, Q.p.s[1]);
#pragma unroll
    for (int i = 2; i < Q.p.ns; ++i) sp = __builtin_fmaf(sp, sq, Q.p.s[i]);
    const float sr = r * sp;
    float cp = __builtin_fmaf(Q.p.c[0], sq, Q.p.c[1]);
#pragma unroll
    for (int i = 2; i < Q.p.nc; ++i) cp = __builtin_fmaf(cp, sq, Q.p.c[i]);
    if constexpr (Q.red == kQuarterCw || Q.red == kQuarterShift2) {
        restore_quadrant_f32(sr, cp, q, s, c);
    } else {
        s = as_f32(as_u32(sr) ^ q);
        c = as_f32(as_u32(cp) ^ q);
    }
}

// PolynomialD3D4Cycle (:162-205): reduce in turns and fold into [0, 1/8]
// by the sin/cos symmetries; coefficients absorb 2*pi.
__device__ __forceinline__ void f32_sincos_cycle(float angle, float& c, float& s) {
    constexpr float kInvTwoPi = 0.15915494309189533577f;
    const float cycles = angle * kInvTwoPi;
    const float wrapped = cycles - __builtin_rintf(cycles);
    const uint32_t sin_sign = as_u32(wrapped) & 0x80000000u;
    float r = __builtin_fabsf(wrapped);
    const bool outer = r > 0.25f;
    r = outer ? 0.5f - r : r;
    const bool swap = r > 0.125f;
    r = swap ? 0.25f - r : r;
    const float sq = r * r;
    const float sr = r * __builtin_fmaf(-39.77336883544921875f, sq, 6.277099609375f);
    float cr = __builtin_fmaf(62.96308135986328125f, sq, -19.7276897430419921875f);
    cr = __builtin_fmaf(cr, sq, 0.999990046024322509765625f);
    const float sm = swap ? cr : sr;
    const float cm = swap ? sr : cr;
    s = as_f32(as_u32(sm) ^ sin_sign);
    c = as_f32(as_u32(cm) ^ ((uint32_t)outer << 31));
}

// ---------------------------------------------------------------------------
// 16-bit quarter-turn programs (sincos_kernels.cu:544-642, 940-978)
// ---------------------------------------------------------------------------

// Coefficients, highest power of sq first.
constexpr SinCosProg kF16QuarterD3D4 = {  // evaluate_quarter_turn_d3_d4_fp16, :544-571
    2, {-0.1602783203125f, 0.9990234375f}, 3, {0.040435791015625f, -0.499755859375f, 1.0f}};
constexpr SinCosProg kBf16QuarterD3D4 = {  // PolynomialD3D4QuarterTurnBF16, :597-642
    2, {-0.162109375f, 1.0f}, 3, {0.041015625f, -0.5f, 1.0f}};
constexpr SinCosProg kBf16CwD3D4 = {  // PolynomialD3D4BF16, :940-978 (FP32 Sollya set)
    2, {-0.16034401953220367431640625f, 0.99903142452239990234375f}, 3,
    {0.0403986163437366485595703125f, -0.4997082054615020751953125f, 0.999990046024322509765625f}};
constexpr SinCosProg kF16RopeQuarterD3D4 = {  // evaluate_quarter_turn_q15_d3_d4_fp16, :1254-1287
    2, {-0.07763671875f, 0.78466796875f}, 3, {0.01538848876953125f, -0.308349609375f, 1.0f}};

// Packed FP16 polynomial on a reduced pair r (sin = r*S(r^2), cos = C(r^2)),
// no sign handling.
__device__ __forceinline__ void f16_poly_pair(const SinCosProg& Q, h2_t r, uint32_t& cr,
                                              uint32_t& sr) {
    const h2_t sq = r * r;
    h2_t sp = __builtin_elementwise_fma(as_h2(f16_pair_bits(Q.s[0])), sq, as_h2(f16_pair_bits(Q.s[1])));
    for (int i = 2; i < Q.ns; ++i) sp = __builtin_elementwise_fma(sp, sq, as_h2(f16_pair_bits(Q.s[i])));
    h2_t cp = __builtin_elementwise_fma(as_h2(f16_pair_bits(Q.c[0])), sq, as_h2(f16_pair_bits(Q.c[1])));
    for (int i = 2; i < Q.nc; ++i) cp = __builtin_elementwise_fma(cp, sq, as_h2(f16_pair_bits(Q.c[i])));
    sr = as_u32(r * sp);
    cr = as_u32(cp);
}

// BF16 polynomial on one reduced lane (FP32 value holding a BF16 value);
// results are the last steps' FP32 values before their final rounding, which
// the caller's pack to BF16 performs.
__device__ __forceinline__ void bf16_poly_lane(const SinCosProg& Q, float r, float& cr, float& sr) {
    const float sq = rbf(r * r);
    sr = r * rbf(bf16_horner_open(Q.s, Q.ns, sq));
    cr = bf16_horner_open(Q.c, Q.nc, sq);
}

// FP16 quarter-turn D3/D4 on two FP32 angles (PolynomialD3D4QuarterTurnFP16, :573-595).
__device__ __forceinline__ void f16_sincos_quarter(float a_lo, float a_hi, uint32_t& cos2,
                                                   uint32_t& sin2) {
    float r_lo, r_hi;
    uint32_t q_lo, q_hi;
    reduce_quarter_shift<false>(a_lo, r_lo, q_lo);
    reduce_quarter_shift<false>(a_hi, r_hi, q_hi);
    uint32_t cr, sr;
    f16_poly_pair(kF16QuarterD3D4, (h2_t){(_Float16)r_lo, (_Float16)r_hi}, cr, sr);
    restore_quadrant_pair(sr, cr, q_lo, q_hi, sin2, cos2);
}

// BF16 quarter-turn programs on two FP32 angles: shifter reduction with a
// one-term pi/2 (PolynomialD3D4QuarterTurnBF16) or Cody-Waite with a
// converted quadrant (PolynomialD3D4BF16).
template <bool CodyWaite>
__device__ __forceinline__ void bf16_sincos_quarter(float a_lo, float a_hi, uint32_t& cos2,
                                                    uint32_t& sin2) {
    constexpr SinCosProg Q = CodyWaite ? kBf16CwD3D4 : kBf16QuarterD3D4;
    float r_lo, r_hi;
    uint32_t q_lo, q_hi;
    if constexpr (CodyWaite) {
        reduce_quarter_cw(a_lo, r_lo, q_lo);
        reduce_quarter_cw(a_hi, r_hi, q_hi);
    } else {
        reduce_quarter_shift<false>(a_lo, r_lo, q_lo);
        reduce_quarter_shift<false>(a_hi, r_hi, q_hi);
    }
    float c_lo, s_lo, c_hi, s_hi;
    bf16_poly_lane(Q, rbf(r_lo), c_lo, s_lo);
    bf16_poly_lane(Q, rbf(r_hi), c_hi, s_hi);
    restore_quadrant_pair(pack_bf(s_lo, s_hi), pack_bf(c_lo, c_hi), q_lo, q_hi, sin2, cos2);
}

// RoPE fixed-point phase, quarter turn (reduce_rope_phase_to_quarter_turn_q15
// and evaluate_quarter_turn_q15_d3_d4_fp16, :1242-1287): the quadrant is the
// phase rounded to quarter turns, the residual keeps 16 bits below it as
// signed Q15 of a quarter turn.
__device__ __forceinline__ void rope_q15_quarter_sincos(uint32_t position, uint32_t inc_lo,
                                                        uint32_t inc_hi, uint32_t& cos2,
                                                        uint32_t& sin2) {
    const uint32_t ph_lo = position * inc_lo, ph_hi = position * inc_hi;
    const uint32_t q_lo = (ph_lo + 0x20000000u) >> 30, q_hi = (ph_hi + 0x20000000u) >> 30;
    const int16_t r_lo = (int16_t)((int32_t)(ph_lo - (q_lo << 30)) >> 14);
    const int16_t r_hi = (int16_t)((int32_t)(ph_hi - (q_hi << 30)) >> 14);
    const h2_t r = (h2_t){(_Float16)r_lo, (_Float16)r_hi} * as_h2(f16_pair_bits(0x1p-15f));
    uint32_t cr, sr;
    f16_poly_pair(kF16RopeQuarterD3D4, r, cr, sr);
    restore_quadrant_pair(sr, cr, q_lo, q_hi, sin2, cos2);
}

// RoPE phase through a 128-entry table and a first-order correction
// (evaluate_rope_phase_lut_fp16, :1350-1385).  table[i] holds FP16
// (sin, cos) of the table phase i/128 turn (sin in the low half); the
// residual phase delta (|delta| <= pi/128 rad) gives sin = fma(delta, cos_i,
// sin_i), cos = fma(-delta, sin_i, cos_i) in packed FP16.
__device__ __forceinline__ void rope_lut_sincos(uint32_t position, uint32_t inc_lo, uint32_t inc_hi,
                                                const uint32_t* __restrict__ table, uint32_t& cos2,
                                                uint32_t& sin2) {
    constexpr float kRadPerUnit = 0x1.921fb6p-30f;  // 2*pi / 2^32
    const uint32_t ph_lo = position * inc_lo, ph_hi = position * inc_hi;
    const uint32_t i_lo = ((ph_lo + (1u << 24)) >> 25) & 127u;
    const uint32_t i_hi = ((ph_hi + (1u << 24)) >> 25) & 127u;
    const int32_t d_lo = (int32_t)(ph_lo - (i_lo << 25));
    const int32_t d_hi = (int32_t)(ph_hi - (i_hi << 25));
    const h2_t delta = {(_Float16)((float)d_lo * kRadPerUnit), (_Float16)((float)d_hi * kRadPerUnit)};
    const uint32_t b_lo = table[i_lo], b_hi = table[i_hi];
    const h2_t sb = as_h2(__builtin_amdgcn_perm(b_hi, b_lo, 0x05040100u));
    const h2_t cb = as_h2(__builtin_amdgcn_perm(b_hi, b_lo, 0x07060302u));
    sin2 = as_u32(__builtin_elementwise_fma(delta, cb, sb));
    cos2 = as_u32(__builtin_elementwise_fma(as_h2(as_u32(delta) ^ 0x80008000u), sb, cb));
}

__device__ __forceinline__ void rope_q15_sincos(uint32_t position, uint32_t inc_lo, uint32_t inc_hi,
                                                uint32_t& cos2, uint32_t& sin2) {
    const uint32_t ph_lo = position * inc_lo;
    const uint32_t ph_hi = position * inc_hi;
    const int16_t q_lo = (int16_t)(ph_lo >> 15);
    const int16_t q_hi = (int16_t)(ph_hi >> 15);
    const h2_t r = (h2_t){(_Float16)q_lo, (_Float16)q_hi} * as_h2(f16_pair_bits(0x1p-15f));
    // sign = bit31 ^ bit30 of each phase, in bit 15 / bit 31 of the pair
    const uint32_t upper = (ph_lo >> 16) | (ph_hi & 0xffff0000u);
    const uint32_t signs = (upper ^ (upper << 1)) & 0x80008000u;
    f16_sincos_reduced<kF16RopeQ15D5D6>(r, signs, cos2, sin2);
}


// ---------------------------------------------------------------------------
// table evaluators
// 16-bit: eval(a0, a1, cos pair, sin pair) on two FP32 angles.
// FP32:   eval(a, cos, sin).
// ---------------------------------------------------------------------------

template <int P>
struct F16HalfTurn {
    __device__ __forceinline__ static void eval(float a0, float a1, uint32_t& c, uint32_t& s) {
        f16_sincos<P>(a0, a1, c, s);
    }
};

// FP16 evaluation, BF16 output (PolynomialD5D4HalfTurnFP16BF16, sincos_kernels.cu:922-938).
template <int P>
struct F16HalfTurnToBF16 {
    __device__ __forceinline__ static void eval(float a0, float a1, uint32_t& c, uint32_t& s) {
        uint32_t ch, sh;
        f16_sincos<P>(a0, a1, ch, sh);
        const h2_t cc = as_h2(ch), ss = as_h2(sh);
        c = pack_bf((float)cc.x, (float)cc.y);
        s = pack_bf((float)ss.x, (float)ss.y);
    }
};

template <int P>
struct BF16HalfTurn {
    __device__ __forceinline__ static void eval(float a0, float a1, uint32_t& c, uint32_t& s) {
        float c0, s0, c1, s1;
        bf16_sincos_lane<P>(a0, c0, s0);
        bf16_sincos_lane<P>(a1, c1, s1);
        c = pack_bf(c0, c1);  // the programs' final roundings
        s = pack_bf(s0, s1);
    }
};

struct F16Quarter {
    __device__ __forceinline__ static void eval(float a0, float a1, uint32_t& c, uint32_t& s) {
        f16_sincos_quarter(a0, a1, c, s);
    }
};

template <bool CodyWaite>
struct BF16Quarter {
    __device__ __forceinline__ static void eval(float a0, float a1, uint32_t& c, uint32_t& s) {
        bf16_sincos_quarter<CodyWaite>(a0, a1, c, s);
    }
};

// Hardware transcendentals: __sinf/__cosf lower to v_sin_f32/v_cos_f32.
template <bool BF>
struct NativeSinCos {
    __device__ __forceinline__ static void eval(float a0, float a1, uint32_t& c, uint32_t& s) {
        const float c0 = __cosf(a0), s0 = __sinf(a0), c1 = __cosf(a1), s1 = __sinf(a1);
        if constexpr (BF) {
            c = pack_bf(c0, c1);
            s = pack_bf(s0, s1);
        } else {
            c = as_u32((h2_t){(_Float16)c0, (_Float16)c1});
            s = as_u32((h2_t){(_Float16)s0, (_Float16)s1});
        }
    }
};

template <int P>
struct F32Prog {
    __device__ __forceinline__ static void eval(float a, float& c, float& s) { f32_sincos<P>(a, c, s); }
};

struct F32Cycle {
    __device__ __forceinline__ static void eval(float a, float& c, float& s) { f32_sincos_cycle(a, c, s); }
};

struct F32Native {
    __device__ __forceinline__ static void eval(float a, float& c, float& s) {
        c = __cosf(a);
        s = __sinf(a);
    }
};

}  // namespace pt
