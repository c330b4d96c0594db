// attention.hip -- score-side programs of the attention path:
//  * B3: the deployed sigmoid-attention program (direct D3 probability +
//    factored D4 derivative);
//  * B2: tanh softcap cap*tanh(s/cap) with the D4 BF16 tanh program, and its
//    derivative from the differentiated D4 coefficients;
//  * B5: fractional exp2 with FP32 range reduction (D2 "safe" fraction, FA4's
//    D3 fraction, and the v_exp_f32 baseline), FP32 in, BF16 or FP32 out.
#include <hip/hip_runtime.h>

#include "ops.hpp"
#include "score_programs.hpp"
#include "spline_ops_hip.h"

namespace pt {

struct B3Op {
    static constexpr int NIN = 1, NOUT = 2;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[1], uint32_t (&b)[2]) {
        float y0, y1, d0, d1;
        b3_lane<true>(bf_lo(a[0]), y0, d0);
        b3_lane<true>(bf_hi(a[0]), y1, d1);
        b[0] = pack_exact_bf(y0, y1);
        b[1] = pack_bf(d0, d1);
    }
};

struct B3FwdOp {
    static constexpr int NIN = 1, NOUT = 1;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[1], uint32_t (&b)[1]) {
        float y0, y1, d;
        b3_lane<false, true>(bf_lo(a[0]), y0, d);
        b3_lane<false, true>(bf_hi(a[0]), y1, d);
        b[0] = pack_bf(y0, y1);  // the probability's final rounding
    }
};

// Hardware control of B3 (FA4's sigmoid_variant="sfu", the "native" B3
// component config, src/sfu_repro/fa4.py:687-693): p = sigmoid(x - ln 4096)
// = 1 / (1 + 2^(12 - x log2 e)) in FP32 with v_exp_f32 / v_rcp_f32,
// dy = p (1 - p), each rounded once to BF16.
struct B3NativeOp {
    static constexpr int NIN = 1, NOUT = 2;
    __device__ __forceinline__ static void lane(float x, float& y, float& dy) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(-x, 1.44269504088896340736f, 12.0f));
        y = __builtin_amdgcn_rcpf(1.0f + e);
        dy = __builtin_fmaf(-y, y, y);
    }
    __device__ __forceinline__ static void pair(const uint32_t (&a)[1], uint32_t (&b)[2]) {
        float y0, y1, d0, d1;
        lane(bf_lo(a[0]), y0, d0);
        lane(bf_hi(a[0]), y1, d1);
        b[0] = pack_bf(y0, y1);
        b[1] = pack_bf(d0, d1);
    }
};

struct B3D2Op {
    static constexpr int NIN = 1, NOUT = 2;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[1], uint32_t (&b)[2]) {
        float y0, y1, d0, d1;
        b3_d2_lane(bf_lo(a[0]), y0, d0);
        b3_d2_lane(bf_hi(a[0]), y1, d1);
        b[0] = pack_bf(y0, y1);
        b[1] = pack_bf(d0, d1);
    }
};

// FP32 scores: 8 scores (32 B) per thread-iteration, two 16-byte loads.
template <bool LNT, bool SNT>
__global__ void __launch_bounds__(kBlock)
b3_f32_kernel(const float* __restrict__ s, uint16_t* __restrict__ y, uint16_t* __restrict__ dy,
              int64_t n, int vec_ok) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const int64_t n8 = vec_ok ? (n >> 3) : 0;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n8; i += stride) {
        const Vec4 a = ld16<LNT>(s, 2 * i);
        const Vec4 c = ld16<LNT>(s, 2 * i + 1);
        const uint32_t w[8] = {a.w[0], a.w[1], a.w[2], a.w[3], c.w[0], c.w[1], c.w[2], c.w[3]};
        Vec4 oy, od;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float y0, y1, d0, d1;
            b3_lane<true>(rbf(as_f32(w[2 * k])), y0, d0);
            b3_lane<true>(rbf(as_f32(w[2 * k + 1])), y1, d1);
            oy.w[k] = pack_exact_bf(y0, y1);
            od.w[k] = pack_bf(d0, d1);
        }
        st16<SNT>(y, i, oy);
        st16<SNT>(dy, i, od);
    }
    for (int64_t e = (n8 << 3) + (int64_t)blockIdx.x * kBlock + threadIdx.x; e < n; e += stride) {
        float yy, dd;
        b3_lane<true>(rbf(s[e]), yy, dd);
        y[e] = (uint16_t)(pack_exact_bf(yy, yy) & 0xffffu);
        dy[e] = (uint16_t)(pack_bf(dd, dd) & 0xffffu);
    }
}

// Forward on the magnitudes (SoftcapConsts::mag_open), the scores' sign bits
// written into the packed result (whose sign bits are zero).  Measured on
// MI355X at [4,32,2048,2048]: 323 us against 335 us for the same program
// with the sign carried through the lanes (the packed 16-bit clamp, sign
// merge and unpack of the signed form cost 10 VALU per pair against 8).
struct SoftcapFwdOp {
    static constexpr int NIN = 1, NOUT = 1;
    static constexpr bool kParams = true;  // prm[0] = cap, prm[1] = 1/cap (FP32)
    __device__ __forceinline__ static void pair(const uint32_t (&a)[1], uint32_t (&b)[1],
                                                const float (&prm)[2]) {
        const uint32_t m = pack_bf(SoftcapConsts::mag_open(bf_lo(a[0]), prm[1], prm[0]),
                                   SoftcapConsts::mag_open(bf_hi(a[0]), prm[1], prm[0]));
        b[0] = (a[0] & 0x80008000u) | m;
    }
};

// Native baseline: cap * tanh(s / cap) in FP32 with hardware exp/rcp,
// tanh(u) = 1 - 2 / (exp(2u) + 1), one RNE rounding to BF16.
struct SoftcapNativeOp {
    static constexpr int NIN = 1, NOUT = 1;
    static constexpr bool kParams = true;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[1], uint32_t (&b)[1],
                                                const float (&prm)[2]) {
        const float y0 = prm[0] * native_lane<kTanh, kFwd>(bf_lo(a[0]) * prm[1]);
        const float y1 = prm[0] * native_lane<kTanh, kFwd>(bf_hi(a[0]) * prm[1]);
        b[0] = pack_bf(y0, y1);
    }
};

// Native backward baseline (FA4's softcap_backward_mode 'native',
// src/sfu_repro/fa4.py:306-311): grad_out * (1 - tanh^2(s / cap)) in FP32
// with the hardware tanh of SoftcapNativeOp, one RNE rounding to BF16.
struct SoftcapNativeBwdOp {
    static constexpr int NIN = 2, NOUT = 1;  // (grad_out, scores) -> grad_scores
    static constexpr bool kParams = true;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[2], uint32_t (&b)[1],
                                                const float (&prm)[2]) {
        const float d0 = native_lane<kTanh, kBwd>(bf_lo(a[1]) * prm[1]);
        const float d1 = native_lane<kTanh, kBwd>(bf_hi(a[1]) * prm[1]);
        b[0] = pack_bf(bf_lo(a[0]) * d0, bf_hi(a[0]) * d1);
    }
};

struct SoftcapBwdOp {
    static constexpr int NIN = 2, NOUT = 1;  // (grad_out, scores) -> grad_scores
    static constexpr bool kParams = true;
    __device__ __forceinline__ static float deriv(float t) { return SoftcapConsts::deriv(t); }
    __device__ __forceinline__ static void pair(const uint32_t (&a)[2], uint32_t (&b)[1],
                                                const float (&prm)[2]) {
        // |u| per lane; NaN magnitudes fail t < t_sat
        const float t0 = SoftcapConsts::abs_u(bf_lo(a[1]), prm[1]);
        const float t1 = SoftcapConsts::abs_u(bf_hi(a[1]), prm[1]);
        b[0] = pack_bf(bf_lo(a[0]) * deriv(t0), bf_hi(a[0]) * deriv(t1));
    }
};

// FP32 -> BF16: 8 values (two 16-byte loads) per thread-iteration.
template <int KIND, bool LNT, bool SNT>
__global__ void __launch_bounds__(kBlock)
exp2_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y, int64_t n, int vec_ok) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const int64_t n8 = vec_ok ? (n >> 3) : 0;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n8; i += stride) {
        const Vec4 a = ld16<LNT>(x, 2 * i);
        const Vec4 c = ld16<LNT>(x, 2 * i + 1);
        const uint32_t w[8] = {a.w[0], a.w[1], a.w[2], a.w[3], c.w[0], c.w[1], c.w[2], c.w[3]};
        Vec4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float r0, r1;
            exp2_pair<KIND>(as_f32(w[2 * k]), as_f32(w[2 * k + 1]), r0, r1);
            o.w[k] = pack_bf(r0, r1);
        }
        st16<SNT>(y, i, o);
    }
    for (int64_t e = (n8 << 3) + (int64_t)blockIdx.x * kBlock + threadIdx.x; e < n; e += stride) {
        float r, unused;
        exp2_pair<KIND>(x[e], x[e], r, unused);
        y[e] = (uint16_t)(pack_bf(r, r) & 0xffffu);
    }
}

// FP32 -> FP32: 4 values per thread-iteration.
template <int KIND, bool LNT, bool SNT>
__global__ void __launch_bounds__(kBlock)
exp2_f32_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n, int vec_ok) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const int64_t n4 = vec_ok ? (n >> 2) : 0;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride) {
        const Vec4 a = ld16<LNT>(x, i);
        Vec4 o;
#pragma unroll
        for (int k = 0; k < 4; k += 2) {
            float r0, r1;
            exp2_pair<KIND>(as_f32(a.w[k]), as_f32(a.w[k + 1]), r0, r1);
            o.w[k] = as_u32(r0);
            o.w[k + 1] = as_u32(r1);
        }
        st16<SNT>(y, i, o);
    }
    for (int64_t e = (n4 << 2) + (int64_t)blockIdx.x * kBlock + threadIdx.x; e < n; e += stride) {
        float r, unused;
        exp2_pair<KIND>(x[e], x[e], r, unused);
        y[e] = r;
    }
}

template <int KIND, bool BF_OUT>
int launch_exp2(void* y, const void* x, int64_t n, void* stream) {
    if (bad_args(n, {y, x})) return hipErrorInvalidValue;
    if (n == 0) return hipSuccess;
    const int vec_ok = aligned16(y) && aligned16(x);
    const int per = BF_OUT ? 8 : 4;
    const int64_t grid = grid_one_pass(vec_ok ? n / per : n);
    const int mode = nt_mode(4 * n, (BF_OUT ? 2 : 4) * n);
#define PT_EXP2_LAUNCH(LNT, SNT)                                                                  \
    if constexpr (BF_OUT)                                                                         \
        hipLaunchKernelGGL((exp2_bf16_kernel<KIND, LNT, SNT>), dim3((unsigned)grid), dim3(kBlock), \
                           0, hs(stream), (const float*)x, (uint16_t*)y, n, vec_ok);              \
    else                                                                                          \
        hipLaunchKernelGGL((exp2_f32_kernel<KIND, LNT, SNT>), dim3((unsigned)grid), dim3(kBlock),  \
                           0, hs(stream), (const float*)x, (float*)y, n, vec_ok);
    if (mode == kNtBoth) {
        PT_EXP2_LAUNCH(true, true)
    } else if (mode == kNtStore) {
        PT_EXP2_LAUNCH(false, true)
    } else {
        PT_EXP2_LAUNCH(false, false)
    }
#undef PT_EXP2_LAUNCH
    return hipGetLastError();
}

}  // namespace pt

using namespace pt;

extern "C" int launch_flash_sigmoid_direct_d3_d4_bf16(void* y, void* dy, const void* scores,
                                                      int64_t size, void* stream) {
    if (bad_args(size, {y, dy, scores})) return hipErrorInvalidValue;
    Streams<1, 2> s{{scores}, {y, dy}};
    return launch_pairwise<B3Op>(s, size, hs(stream));
}

extern "C" int launch_flash_sigmoid_direct_d3_bf16(void* y, const void* scores, int64_t size,
                                                   void* stream) {
    return run1<B3FwdOp>(y, scores, size, stream);
}

extern "C" int launch_flash_sigmoid_native_bf16(void* y, void* dy, const void* scores,
                                                int64_t size, void* stream) {
    if (bad_args(size, {y, dy, scores})) return hipErrorInvalidValue;
    Streams<1, 2> s{{scores}, {y, dy}};
    return launch_pairwise<B3NativeOp>(s, size, hs(stream));
}

extern "C" int launch_flash_sigmoid_direct_d3_d4_f32_bf16(void* y, void* dy, const void* scores,
                                                          int64_t size, void* stream) {
    if (bad_args(size, {y, dy, scores})) return hipErrorInvalidValue;
    if (size == 0) return hipSuccess;
    const int vec_ok = aligned16(y) && aligned16(dy) && aligned16(scores);
    const int64_t grid = grid_one_pass(vec_ok ? (size >> 3) : size);
    // 4 bytes read and 4 bytes written per score.
    switch (nt_mode(4 * size, 4 * size)) {
    case kNtBoth:
        hipLaunchKernelGGL((b3_f32_kernel<true, true>), dim3((unsigned)grid), dim3(kBlock), 0,
                           hs(stream), (const float*)scores, (uint16_t*)y, (uint16_t*)dy, size,
                           vec_ok);
        break;
    case kNtStore:
        hipLaunchKernelGGL((b3_f32_kernel<false, true>), dim3((unsigned)grid), dim3(kBlock), 0,
                           hs(stream), (const float*)scores, (uint16_t*)y, (uint16_t*)dy, size,
                           vec_ok);
        break;
    default:
        hipLaunchKernelGGL((b3_f32_kernel<false, false>), dim3((unsigned)grid), dim3(kBlock), 0,
                           hs(stream), (const float*)scores, (uint16_t*)y, (uint16_t*)dy, size,
                           vec_ok);
    }
    return hipGetLastError();
}


// ---- B2 softcap ---------------------------------------------------------------

extern "C" int launch_softcap_tanh_d4_bf16(void* out, const void* scores, int64_t size, float cap,
                                           void* stream) {
    if (bad_args(size, {out, scores}) || !(cap > 0.0f && cap <= __FLT_MAX__)) return hipErrorInvalidValue;
    Streams<1, 1> s{{scores}, {out}, {cap, 1.0f / cap}};
    return launch_pairwise<SoftcapFwdOp>(s, size, hs(stream));
}

extern "C" int launch_softcap_tanh_native_bf16(void* out, const void* scores, int64_t size,
                                               float cap, void* stream) {
    if (bad_args(size, {out, scores}) || !(cap > 0.0f && cap <= __FLT_MAX__)) return hipErrorInvalidValue;
    Streams<1, 1> s{{scores}, {out}, {cap, 1.0f / cap}};
    return launch_pairwise<SoftcapNativeOp>(s, size, hs(stream));
}

extern "C" int launch_softcap_tanh_d4_bwd_bf16(void* grad_scores, const void* grad_out,
                                               const void* scores, int64_t size, float cap,
                                               void* stream) {
    if (bad_args(size, {grad_scores, grad_out, scores}) || !(cap > 0.0f && cap <= __FLT_MAX__))
        return hipErrorInvalidValue;
    Streams<2, 1> s{{grad_out, scores}, {grad_scores}, {cap, 1.0f / cap}};
    return launch_pairwise<SoftcapBwdOp>(s, size, hs(stream));
}

extern "C" int launch_softcap_tanh_native_bwd_bf16(void* grad_scores, const void* grad_out,
                                                   const void* scores, int64_t size, float cap,
                                                   void* stream) {
    if (bad_args(size, {grad_scores, grad_out, scores}) || !(cap > 0.0f && cap <= __FLT_MAX__))
        return hipErrorInvalidValue;
    Streams<2, 1> s{{grad_out, scores}, {grad_scores}, {cap, 1.0f / cap}};
    return launch_pairwise<SoftcapNativeBwdOp>(s, size, hs(stream));
}

// ---- B5 exp2 ------------------------------------------------------------------

extern "C" int launch_exp2_d2_f32_bf16(void* y, const void* x, int64_t size, void* stream) {
    return launch_exp2<kExp2D2, true>(y, x, size, stream);
}
extern "C" int launch_exp2_d3_f32_bf16(void* y, const void* x, int64_t size, void* stream) {
    return launch_exp2<kExp2D3, true>(y, x, size, stream);
}
extern "C" int launch_exp2_native_f32_bf16(void* y, const void* x, int64_t size, void* stream) {
    return launch_exp2<kExp2Native, true>(y, x, size, stream);
}
extern "C" int launch_exp2_d2_f32(void* y, const void* x, int64_t size, void* stream) {
    return launch_exp2<kExp2D2, false>(y, x, size, stream);
}
extern "C" int launch_exp2_d3_f32(void* y, const void* x, int64_t size, void* stream) {
    return launch_exp2<kExp2D3, false>(y, x, size, stream);
}
extern "C" int launch_exp2_native_f32(void* y, const void* x, int64_t size, void* stream) {
    return launch_exp2<kExp2Native, false>(y, x, size, stream);
}
extern "C" int launch_exp2_pwl2_safe_f32_bf16(void* y, const void* x, int64_t size, void* stream) {
    return launch_exp2<kExp2Pwl2Safe, true>(y, x, size, stream);
}
extern "C" int launch_exp2_pwl2_safe_f32(void* y, const void* x, int64_t size, void* stream) {
    return launch_exp2<kExp2Pwl2Safe, false>(y, x, size, stream);
}
extern "C" int launch_exp2_pwl2_safe_f16_f32_bf16(void* y, const void* x, int64_t size, void* stream) {
    return launch_exp2<kExp2Pwl2SafeF16, true>(y, x, size, stream);
}
extern "C" int launch_exp2_pwl2_safe_f16_f32(void* y, const void* x, int64_t size, void* stream) {
    return launch_exp2<kExp2Pwl2SafeF16, false>(y, x, size, stream);
}

// The remaining FA4 exp2 backends (src/sfu_repro/fa4.py:33-46).
#define PT_EXP2_ENTRY(NAME, KIND)                                                                   \
    extern "C" int launch_exp2_##NAME##_f32_bf16(void* y, const void* x, int64_t size, void* stream) { \
        return launch_exp2<KIND, true>(y, x, size, stream);                                        \
    }                                                                                              \
    extern "C" int launch_exp2_##NAME##_f32(void* y, const void* x, int64_t size, void* stream) {      \
        return launch_exp2<KIND, false>(y, x, size, stream);                                       \
    }
PT_EXP2_ENTRY(pwl2, kExp2Pwl2)
PT_EXP2_ENTRY(pwl1_safe, kExp2Pwl1Safe)
PT_EXP2_ENTRY(pwl1_safe_f16, kExp2Pwl1SafeF16)
PT_EXP2_ENTRY(pwl2_safe_bf16, kExp2Pwl2SafeBF16)
PT_EXP2_ENTRY(d2_safe_noclamp, kExp2D2NoClamp)
PT_EXP2_ENTRY(d2_safe_f16, kExp2D2SafeF16)
PT_EXP2_ENTRY(d2_safe_bf16, kExp2D2SafeBF16)
PT_EXP2_ENTRY(pwl2_f16, kExp2Pwl2F16)
#undef PT_EXP2_ENTRY

// ---- B3-D2 ----------------------------------------------------------------------

extern "C" int launch_flash_sigmoid_exp2_d2_bf16(void* y, void* dy, const void* scores,
                                                 int64_t size, void* stream) {
    if (bad_args(size, {y, dy, scores})) return hipErrorInvalidValue;
    Streams<1, 2> s{{scores}, {y, dy}};
    return launch_pairwise<B3D2Op>(s, size, hs(stream));
}
