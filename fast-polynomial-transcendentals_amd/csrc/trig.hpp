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

// BF16 half-turn program on one FP32 angle; results are FP32 values that hold
// BF16 values (signs applied).
template <int P>
__device__ __forceinline__ void bf16_sincos_lane(float angle, float& c, float& s) {
    constexpr SinCosProg Q = kSinCos[P];
    float r;
    uint32_t sign;
    reduce_half_turn(angle, r, sign);
    r = rbf(r);
    const float sq = rbf(r * r);
    float sp = bfma(bf16_value(Q.s[0]), sq, bf16_value(Q.s[1]));
#pragma unroll
    for (int i = 2; i < Q.ns; ++i) sp = bfma(sp, sq, bf16_value(Q.s[i]));
    const float sr = rbf(r * sp);
    float cp = bfma(bf16_value(Q.c[0]), sq, bf16_value(Q.c[1]));
#pragma unroll
    for (int i = 2; i < Q.nc; ++i) cp = bfma(cp, sq, bf16_value(Q.c[i]));
    s = as_f32(as_u32(sr) ^ sign);
    c = as_f32(as_u32(cp) ^ sign);
}

// RoPE fixed-point phase for two frequencies at one position
// (evaluate_rope_half_turn_q15_d5_d6_fp16, sincos_kernels.cu:1330-1348).
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

}  // namespace pt
