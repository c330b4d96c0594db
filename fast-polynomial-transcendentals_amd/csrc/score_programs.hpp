// score_programs.hpp -- the attention-side lane programs, shared by the
// elementwise score kernels (attention.hip) and the fused flash-attention
// kernel (flash_attn.hip):
//  * B3: the deployed sigmoid-attention program (direct D3 probability +
//    factored D4 derivative) and the B3-D2 exp2 form;
//  * B2: constants of the D4 BF16 tanh softcap and its derivative;
//  * B5: fractional exp2 with FP32 range reduction (D2 "safe", FA4 D3,
//    v_exp_f32).
#pragma once

#include "programs.hpp"

namespace pt {

// ---------------------------------------------------------------------------
// B3: deployed direct-D3 probability and factored-D4 derivative
// (scripts/audit_b3_deployed_fit.py:341-366; PTX main.tex:1072-1117).
// ---------------------------------------------------------------------------

struct B3Consts {
    // Manifest rows (tests/test_audit_b3_deployed_fit.py:30-37) scaled by
    // 1/4096 and rounded to BF16 (DirectB3Spec.deployed_forward_rows).
    static constexpr float r0[4] = {bf16_value(1.0f / 4096), bf16_value(1.0546875f / 4096),
                                    bf16_value(0.53515625f / 4096), bf16_value(0.11328125f / 4096)};
    static constexpr float r1[4] = {bf16_value(-8.5625f / 4096), bf16_value(17.5f / 4096),
                                    bf16_value(-9.0625f / 4096), bf16_value(2.140625f / 4096)};
    // (intercept, slope) of the factored derivative.
    static constexpr float g0[2] = {bf16_value(1.0f), bf16_value(-0.0087890625f)};
    static constexpr float g1[2] = {bf16_value(1.0078125f), bf16_value(-0.0028076171875f)};
    static constexpr float split = bf16_value(1.25f);
    static constexpr float clamp = bf16_value(6.0f);
};

// The six coefficients of each row as FP16 pairs, two to a word: every
// coefficient of the deployed rows is exactly an FP16 value (the smallest,
// 0.11328125 / 4096 = 29 * 2^-20, an FP16 subnormal), so one 32-bit select
// per word picks two of the lane's row coefficients and v_fma_mix_f32 reads
// each half as the exact FP32 operand of its FMA: three selects per score
// where one per coefficient took six, with the same FMAs and roundings.
constexpr bool f16_exact(float c) { return (float)(_Float16)c == c; }
constexpr uint32_t f16_word(float hi, float lo) {
    return ((uint32_t)f16_bits_rne(hi) << 16) | f16_bits_rne(lo);
}
struct B3Pairs {
    using C = B3Consts;
    // [c3 : c2], [c1 : c0] and the derivative's [slope : intercept], row 0 / 1
    static constexpr uint32_t c32_0 = f16_word(C::r0[3], C::r0[2]), c32_1 = f16_word(C::r1[3], C::r1[2]);
    static constexpr uint32_t c10_0 = f16_word(C::r0[1], C::r0[0]), c10_1 = f16_word(C::r1[1], C::r1[0]);
    static constexpr uint32_t g10_0 = f16_word(C::g0[1], C::g0[0]), g10_1 = f16_word(C::g1[1], C::g1[0]);
};
static_assert(f16_exact(B3Consts::r0[0]) && f16_exact(B3Consts::r0[1]) && f16_exact(B3Consts::r0[2]) &&
              f16_exact(B3Consts::r0[3]) && f16_exact(B3Consts::r1[0]) && f16_exact(B3Consts::r1[1]) &&
              f16_exact(B3Consts::r1[2]) && f16_exact(B3Consts::r1[3]) && f16_exact(B3Consts::g0[0]) &&
              f16_exact(B3Consts::g0[1]) && f16_exact(B3Consts::g1[0]) && f16_exact(B3Consts::g1[1]),
              "a B3 coefficient is not an FP16 value");

// The row's pair word, kept opaque so that the compiler selects the packed
// word (one v_cndmask_b32) instead of folding the FP16 widening back into
// two selects of FP32 constants.
__device__ __forceinline__ h2_t b3_row_pair(bool row, uint32_t w0, uint32_t w1) {
    uint32_t r = row ? w1 : w0;
    asm("" : "+v"(r));
    return as_h2(r);
}

// One lane on a BF16 value held in FP32.  NaN follows the audit's Python
// semantics: the clamp keeps NaN, max(0, NaN) gives 0, the derivative is NaN.
// OPEN_Y (probability only) returns y before its final rounding, for callers
// whose conversion to BF16 is that rounding: RNE of an already rounded value
// is the same value, so the converted bits are unchanged.
template <bool WITH_GRAD, bool OPEN_Y = false>
__device__ __forceinline__ void b3_lane(float x, float& y, float& dy) {
    static_assert(!(WITH_GRAD && OPEN_Y), "the derivative multiplies the rounded probability");
    using C = B3Consts;
    using P = B3Pairs;
    const bool row = x >= C::split;
    const float xc = __builtin_elementwise_minimum(
        __builtin_elementwise_maximum(x, -C::clamp), C::clamp);
    const h2_t c32 = b3_row_pair(row, P::c32_0, P::c32_1);
    const h2_t c10 = b3_row_pair(row, P::c10_0, P::c10_1);
    float f = bfma(xc, (float)c32.y, (float)c32.x);
    f = bfma(xc, f, (float)c10.y);
    // y = max(0, bf16(v)) taken as bf16(max(0, v)): RNE is monotone and maps
    // 0 to +0, so both give +0 for v <= 0 (and for NaN) and bf16(v) for v > 0.
    // The maximum then reads the FMA's own result, which needs no NaN
    // quieting, instead of the bits of the packed rounding.
    const float v = __builtin_fmaf(xc, f, (float)c10.x);
    y = OPEN_Y ? (v > 0.0f ? v : 0.0f) : rbf(v > 0.0f ? v : 0.0f);
    if constexpr (WITH_GRAD) {
        const h2_t g = b3_row_pair(row, P::g10_0, P::g10_1);
        const float fac = bfma(xc, (float)g.y, (float)g.x);
        dy = y * fac;  // rounded once by the final pack
    }
}

// ---------------------------------------------------------------------------
// B3-D2: FlashSigmoid probability via a range-reduced degree-2 exp2
// (model autonumerics_zero/evolution/fit_flash_sigmoid_exp2_d2.py:55-77;
// FA4 selects it for sigmoid_degree == 2, src/sfu_repro/fa4.py:469-476).
// t = clamp(s * log2(e), -200, 200) (FP32; beyond the clamp the result is
// 0 or inf either way, NaN scores give 0), n = floor(t), f = t - n,
// m = c0 + f (c1 + f c2), p = m * 2^(n - 12)  (1/4096 folded into the
// exponent), y = bf16(p), dy = bf16(p (1 - p)) with one FMA.
// Coefficients: the fitter's FP32 output for n = 4096 (seed 1234).
// ---------------------------------------------------------------------------

struct B3D2Consts {
    static constexpr float c0 = 1.0018835067749023f;   // 0x3F803DB8
    static constexpr float c1 = 0.6557925939559937f;   // 0x3F27E206
    static constexpr float c2 = 0.33421099185943604f;  // 0x3EAB1DB4
    static constexpr float log2e = 1.44269504088896340736f;
};

__device__ __forceinline__ void b3_d2_lane(float s, float& y, float& dy) {
    using C = B3D2Consts;
    const float t = __builtin_fminf(__builtin_fmaxf(s * C::log2e, -200.0f), 200.0f);
    const float fl = __builtin_floorf(t);
    const float f = t - fl;
    const float m = __builtin_fmaf(__builtin_fmaf(f, C::c2, C::c1), f, C::c0);
    const float p = __builtin_ldexpf(m, (int)fl - 12);
    y = p;
    dy = __builtin_fmaf(-p, p, p);
}

// ---------------------------------------------------------------------------
// B2: tanh softcap.  u = bf16(s * (1/cap)) (FP32 product, one RNE rounding),
// T = TANH_FWD_D4_ODD_BF16(u) (spline_structs_odd_bf16.cuh:153-179),
// y = bf16(T * cap).  The derivative d y / d s = T'(u) (the scale cancels,
// extras/paper/manuscript/main.tex:443-449) evaluates the derivative of the
// D4 odd polynomial, D(t) = c1 + 2 c2 t + 3 c3 t^2 + 4 c4 t^3 with BF16
// coefficients k*c_k and BF16 Horner steps, at t = |u|; D = 0 once t reaches
// 2.609375, the first BF16 magnitude at which the forward program saturates
// at 1 (and above the 2.75 clamp).
// ---------------------------------------------------------------------------

struct SoftcapConsts {
    using T = BF16Prog<kTanh, kFwd, 4>;
    static constexpr float d0 = bf16_value(T::P.c[1]);
    static constexpr float d1 = bf16_value(2.0f * bf16_value(T::P.c[2]));
    static constexpr float d2 = bf16_value(3.0f * bf16_value(T::P.c[3]));
    static constexpr float d3 = bf16_value(4.0f * bf16_value(T::P.c[4]));
    static constexpr float t_sat = 2.609375f;

    // D(t) at t = |u| (a BF16 magnitude); NaN magnitudes fail t < t_sat.
    __device__ __forceinline__ static float deriv(float t) {
        float r = bfma(t, d3, d2);
        r = bfma(t, r, d1);
        r = bfma(t, r, d0);
        return t < t_sat ? r : 0.0f;
    }

    // |u| = bf16(|s| * (1/cap)) for a score s (FP32 holding a BF16 value):
    // RNE is odd-symmetric, so this is the magnitude of u = bf16(s * (1/cap)).
    __device__ __forceinline__ static float abs_u(float s, float inv_cap) {
        return rbf(__builtin_fabsf(s) * inv_cap);
    }

    // The forward program on the magnitude, before its last rounding:
    // |y| = bf16(cap * bf16(min(t * H(t), 1))), t = min(|u|, Lc).  Equal to
    // the signed program sign(s) * bf16(cap * bf16(clamp(ts * H(t), -1, 1)))
    // because every step is odd-symmetric and t * H(t) >= 0 on [0, Lc]; the
    // caller restores the sign of s on the packed result.  The clamp is an
    // unsigned minimum on the FP32 bits of |u| (low half zero): integer order
    // is numeric order for non-negative patterns, and a NaN magnitude selects
    // Lc, the rule of the signed program's packed 16-bit minimum.
    __device__ __forceinline__ static float mag_open(float s, float inv_cap, float cap) {
        const uint32_t tb = as_u32(abs_u(s, inv_cap));
        const uint32_t lc = as_u32(bf16_value(T::P.lc));
        const float t = as_f32(tb < lc ? tb : lc);
        return rbf(__builtin_fminf(t * T::odd_horner(t), 1.0f)) * cap;
    }
};

// ---------------------------------------------------------------------------
// B5: exp2 with FP32 range reduction (autonumerics_zero/cuda_benchmarks/
// utils_exp2_cuda.cuh:13-74): x = max(x, -127); n = floor(x); f = x - n;
// p = polynomial 2^f on [0, 1); result bits = (n << 23) + bits(p).
// D2 "safe" fraction p = 1 + a f + (1 - a) f^2, a = 0.6602339719
// (extras/paper/manuscript/appendix_exp2.tex:29-32; sampled-minimax fit),
// keeps p(0) = 1 and p(1) = 2.  D3 is FA4's e2e_asm2 fraction.  PWL2 is
// the continuous two-piece FP32 fraction of the full-range benchmark
// (autonumerics_zero/cuda_benchmarks/benchmark_exp2_pwl2.cu:126-170):
// p = 0.98946118 + 0.82085252 f + 0.34246066 max(f - 0.5, 0).
// PWL2 "safe" is the endpoint-constrained hinge p = 1 + a f + c max(f - 1/2, 0)
// with c = 2 (1 - a) (appendix_exp2.tex:22-27): p(0) = 1 and p(1) = 2, so
// p >= 1 and the -127 clamp cannot wrap the exponent field.  FP32
// (pwl2_safe): the sampled-minimax a = 0.7980513010317143, c =
// 0.4038973979365714 (evidence/report-data/b5_exp2_softmax_constrained_fits.json,
// two_piece_linear.sampled_minimax) rounded to FP32.  Packed FP16
// (pwl2_safe_f16): a = 0.7978515625, c = 0.40380859375, the FP16 coefficients
// of appendix_exp2.tex:72-76, on f rounded to FP16 (RNE); both endpoints stay
// exact after FP16 rounding.  The FP16 core evaluates two lanes per
// instruction: f16 = rne16(f); h = max(f16 - 1/2, 0) (v_pk_add_f16,
// v_pk_max_f16); b = fma(f16, a, 1); p = fma(h, c, b) (v_pk_fma_f16, one
// rounding each); p is widened to FP32 exactly for the exponent add.  FA4's
// own 16-bit instruction sequence is not in the reference tree; this order is
// the FP32 hinge's (fma(f, a, 1), then fma(hinge, c, .)).
// Defined for x < 128 (softmax exponents are <= 0); -inf and NaN give +0
// (D2, D3, the PWL2 safe programs) or the value at the clamp (PWL2).
//
// The PWL2 fraction starts below one (p(0) = 0.98946), so at n = -127 the
// exponent field of (n << 23) + bits(p) wraps below zero and the bits are a
// NaN for x < -126.987: the reference's hinge clamps at -127 too
// (benchmark_exp2_pwl2.cu:161-162), harmlessly on its benchmark domain
// [-16, 0].  A softmax exponent takes any negative value (a key far below
// the row maximum, or s - lse in the backward), so PWL2 is clamped at -126
// here: from there on the result is positive and at most 2^-126, as 2^x is.
// The programs agree with the reference's bit for bit on x >= -126.
// ---------------------------------------------------------------------------

enum Exp2Kind : int {
    kExp2D2 = 0,             // d2_safe
    kExp2D3 = 1,             // d3
    kExp2Native = 2,         // v_exp_f32
    kExp2Pwl2 = 3,           // pwl2 (FP32 least-squares hinge)
    kExp2Pwl2Safe = 4,       // pwl2_safe
    kExp2Pwl2SafeF16 = 5,    // pwl2_safe_f16
    kExp2Pwl1Safe = 6,       // pwl1_safe
    kExp2Pwl1SafeF16 = 7,    // pwl1_safe_f16
    kExp2Pwl2SafeBF16 = 8,   // pwl2_safe_bf16
    kExp2D2NoClamp = 9,      // d2_safe_noclamp
    kExp2D2SafeF16 = 10,     // d2_safe_f16
    kExp2D2SafeBF16 = 11,    // d2_safe_bf16
    kExp2Pwl2F16 = 12,       // pwl2_f16
    kExp2Kinds = 13
};

// Programs whose fraction runs in packed FP16 (two lanes per instruction).
constexpr bool exp2_is_f16(int kind) {
    return kind == kExp2Pwl2SafeF16 || kind == kExp2Pwl1SafeF16 || kind == kExp2D2SafeF16 || kind == kExp2Pwl2F16;
}
// The lower clamp of the exponent: FA4's -127, or -126 for the hinges whose
// fraction starts below one (there -127 would wrap the exponent field into
// NaN bits); d2_safe_noclamp has none.
constexpr float exp2_clamp(int kind) { return kind == kExp2Pwl2 || kind == kExp2Pwl2F16 ? -126.0f : -127.0f; }

struct Pwl2SafeConsts {
    static constexpr float a = 0.7980513010317143f;
    static constexpr float c = 0.4038973979365714f;
    static constexpr float a16 = 0.7978515625f;   // 0x3A62
    static constexpr float c16 = 0.40380859375f;  // 0x3676
    static constexpr float abf = 0.796875f;       // 0x3F4C, bf16(a)
    static constexpr float cbf = 0.404296875f;    // 0x3ECF, bf16(c)
};

// D2 "safe" fraction with 16-bit coefficients: c1 = 0.6602339719 and
// c2 = 1 - c1 rounded to FP16 / BF16; both roundings give 0.66015625 and
// 0.33984375, whose sum is exactly one, so p(1) = 2 survives the rounding.
struct D2SafeConsts {
    static constexpr float c1 = 0.6602339719000094f;
    static constexpr float c2 = 0.33976602809999057f;
    static constexpr float c1_16 = 0.66015625f;   // FP16 0x3948, BF16 0x3F29
    static constexpr float c2_16 = 0.33984375f;   // FP16 0x3570, BF16 0x3EAE
};

// The reference's FP16 hinge (FractionalPwl2Hinge,
// autonumerics_zero/cuda_benchmarks/benchmark_exp2_pwl2.cu:84-99): offset
// 0x3BEA, slope 0x3A91, slope change 0x357B at f = 1/2.
struct Pwl2F16Consts {
    static constexpr float offset = 0.9892578125f;
    static constexpr float slope = 0.82080078125f;
    static constexpr float delta = 0.342529296875f;
};

// The fraction program on f in [0, 1) for the FP32 and BF16 programs.
// BF16 steps are an FP32 FMA of BF16 values rounded once to BF16 (RNE);
// the hinge max(bf16(f) - 1/2, 0) is exact in BF16.
template <int KIND>
__device__ __forceinline__ float exp2_frac(float f) {
    if constexpr (KIND == kExp2D2 || KIND == kExp2D2NoClamp) {
        return __builtin_fmaf(__builtin_fmaf(f, D2SafeConsts::c2, D2SafeConsts::c1), f, 1.0f);
    } else if constexpr (KIND == kExp2Pwl2) {
        const float p = __builtin_fmaf(f, 0.820852518081665f, 0.9894611835479736f);
        return __builtin_fmaf(__builtin_fmaxf(f - 0.5f, 0.0f), 0.34246066212654114f, p);
    } else if constexpr (KIND == kExp2Pwl2Safe) {
        const float p = __builtin_fmaf(f, Pwl2SafeConsts::a, 1.0f);
        return __builtin_fmaf(__builtin_fmaxf(f - 0.5f, 0.0f), Pwl2SafeConsts::c, p);
    } else if constexpr (KIND == kExp2Pwl1Safe) {
        return f + 1.0f;
    } else if constexpr (KIND == kExp2Pwl2SafeBF16) {
        const float fb = rbf(f);
        const float b = rbf(__builtin_fmaf(fb, Pwl2SafeConsts::abf, 1.0f));
        return rbf(__builtin_fmaf(__builtin_fmaxf(fb - 0.5f, 0.0f), Pwl2SafeConsts::cbf, b));
    } else if constexpr (KIND == kExp2D2SafeBF16) {
        const float fb = rbf(f);
        return rbf(__builtin_fmaf(rbf(__builtin_fmaf(fb, D2SafeConsts::c2_16, D2SafeConsts::c1_16)), fb, 1.0f));
    } else {
        static_assert(KIND == kExp2D3, "FP16 programs run in pairs (exp2_pair)");
        float p = __builtin_fmaf(f, 0.077119089663028717041015625f, 0.227564394474029541015625f);
        p = __builtin_fmaf(p, f, 0.695146143436431884765625f);
        return __builtin_fmaf(p, f, 1.0f);
    }
}

// The packed FP16 fraction of two lanes (f rounded to FP16 by the caller),
// one instruction per step, each step one FP16 rounding.
template <int KIND>
__device__ __forceinline__ h2_t exp2_frac_f16(h2_t f) {
    const h2_t one = {(_Float16)1.0f, (_Float16)1.0f};
    if constexpr (KIND == kExp2Pwl1SafeF16) {
        return f + one;
    } else if constexpr (KIND == kExp2D2SafeF16) {
        const h2_t c1 = {(_Float16)D2SafeConsts::c1_16, (_Float16)D2SafeConsts::c1_16};
        const h2_t c2 = {(_Float16)D2SafeConsts::c2_16, (_Float16)D2SafeConsts::c2_16};
        return __builtin_elementwise_fma(__builtin_elementwise_fma(f, c2, c1), f, one);
    } else {
        static_assert(KIND == kExp2Pwl2SafeF16 || KIND == kExp2Pwl2F16, "not an FP16 hinge");
        constexpr float a = KIND == kExp2Pwl2F16 ? Pwl2F16Consts::slope : Pwl2SafeConsts::a16;
        constexpr float c = KIND == kExp2Pwl2F16 ? Pwl2F16Consts::delta : Pwl2SafeConsts::c16;
        constexpr float b = KIND == kExp2Pwl2F16 ? Pwl2F16Consts::offset : 1.0f;
        const h2_t half = {(_Float16)0.5f, (_Float16)0.5f};
        const h2_t zero = {(_Float16)0.0f, (_Float16)0.0f};
        const h2_t av = {(_Float16)a, (_Float16)a}, cv = {(_Float16)c, (_Float16)c}, bv = {(_Float16)b, (_Float16)b};
        const h2_t hinge = __builtin_elementwise_max(f - half, zero);
        return __builtin_elementwise_fma(hinge, cv, __builtin_elementwise_fma(f, av, bv));
    }
}

template <int KIND>
__device__ __forceinline__ float exp2_lane(float x) {
    static_assert(!exp2_is_f16(KIND), "FP16 programs run in pairs (exp2_pair)");
    if constexpr (KIND == kExp2Native) {
        return __builtin_amdgcn_exp2f(x);
    } else {
        if constexpr (KIND != kExp2D2NoClamp) x = __builtin_fmaxf(x, exp2_clamp(KIND));
        const float fl = __builtin_floorf(x);
        const float p = exp2_frac<KIND>(x - fl);
        const int n = (int)fl;  // v_cvt_i32_f32 (saturating)
        return as_f32(((uint32_t)n << 23) + as_u32(p));
    }
}

// Two lanes of one program.  The packed FP16 programs evaluate both
// fractions with one instruction per step (f rounded to FP16 by
// v_cvt_pk_f16_f32, RNE; p widened to FP32 exactly for the exponent add);
// every other program is exp2_lane per lane.
template <int KIND>
__device__ __forceinline__ void exp2_pair(float x0, float x1, float& y0, float& y1) {
    if constexpr (exp2_is_f16(KIND)) {
        x0 = __builtin_fmaxf(x0, exp2_clamp(KIND));
        x1 = __builtin_fmaxf(x1, exp2_clamp(KIND));
        const float fl0 = __builtin_floorf(x0), fl1 = __builtin_floorf(x1);
        const h2_t f = {(_Float16)(x0 - fl0), (_Float16)(x1 - fl1)};
        const h2_t p = exp2_frac_f16<KIND>(f);
        y0 = as_f32(((uint32_t)(int)fl0 << 23) + as_u32((float)p.x));
        y1 = as_f32(((uint32_t)(int)fl1 << 23) + as_u32((float)p.y));
    } else {
        y0 = exp2_lane<KIND>(x0);
        y1 = exp2_lane<KIND>(x1);
    }
}

}  // namespace pt
