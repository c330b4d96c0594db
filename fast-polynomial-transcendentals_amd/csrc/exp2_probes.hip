// exp2_probes.hip -- the isolated exp2 measurements of the reference's
// harness (autonumerics_zero/cuda_benchmarks/benchmark_exp2_pwl2.cu:24-36,
// 55-266), on gfx950:
//  * the fractional FP16 programs (f in [0, 1] -> 2^f, two lanes per 32-bit
//    pair): v_exp_f16, the historical two-segment fit and the PWL2 hinge,
//    streamed through L2 or HBM with the pairwise driver;
//  * the compute probes: 65,536 threads, each chaining eight register-resident
//    pairs through an exp2 program and a feedback FMA that maps the result
//    back into the program's domain, for the FP16 fractional programs and the
//    full FP32 programs (v_exp_f32, FA4's D3, the PWL2 hinge).
// The full FP32 programs' L2 / HBM streams are the launch_exp2_*_f32 entry
// points of attention.hip.
#include <hip/hip_runtime.h>

#include "ops.hpp"
#include "score_programs.hpp"
#include "spline_ops_hip.h"

namespace pt {

enum Exp2FracVariant : int { kFracNative = 0, kFracPwl2Historical = 1, kFracPwl2Hinge = 2 };
enum Exp2FullVariant : int { kFullNative = 0, kFullDegree3 = 1, kFullPwl2Hinge = 2 };

// The historical two-segment fit (benchmark_exp2_pwl2.cu:60-82): the
// fraction clamped to [0, 0x3BFE] (one ULP below the largest FP16 value under
// one, so that fp16(f + 1) stays below 2), the segment taken from the top
// mantissa bit of fp16(f + 1) -- set when the rounded sum reaches 1.5 -- and
// p = fma(f, slope, offset) with (slope, offset) = (0x3A91, 0x3BEA) below,
// (0x3CA7, 0x3A8C) above.  The per-lane selection is one bitfield insert per
// constant under a mask built from the two lanes' segment bits.
struct Pwl2HistoricalF16 {
    static constexpr uint32_t kSlope0 = 0x3A913A91u, kSlope1 = 0x3CA73CA7u;
    static constexpr uint32_t kOffset0 = 0x3BEA3BEAu, kOffset1 = 0x3A8C3A8Cu;
    static constexpr uint32_t kTop = 0x3BFE3BFEu, kOne = 0x3C003C00u;
};

template <int V>
__device__ __forceinline__ h2_t exp2_fraction_f16(h2_t f) {
    if constexpr (V == kFracNative) {
        return __builtin_elementwise_exp2(f);  // v_exp_f16 per lane
    } else if constexpr (V == kFracPwl2Hinge) {
        return exp2_frac_f16<kExp2Pwl2F16>(f);
    } else {
        using C = Pwl2HistoricalF16;
        const h2_t zero = {(_Float16)0.0f, (_Float16)0.0f};
        const h2_t c = __builtin_elementwise_min(__builtin_elementwise_max(f, zero), as_h2(C::kTop));
        const uint32_t sum = as_u32(c + as_h2(C::kOne));
        const uint32_t mask = ((sum >> 9) & 0x00010001u) * 0xFFFFu;  // 0xFFFF per lane above 1.5
        const uint32_t slope = (C::kSlope1 & mask) | (C::kSlope0 & ~mask);
        const uint32_t offset = (C::kOffset1 & mask) | (C::kOffset0 & ~mask);
        return __builtin_elementwise_fma(c, as_h2(slope), as_h2(offset));
    }
}

template <int V>
__device__ __forceinline__ float exp2_full_f32(float x) {
    if constexpr (V == kFullNative) return __builtin_amdgcn_exp2f(x);
    else if constexpr (V == kFullDegree3) return exp2_lane<kExp2D3>(x);
    else return exp2_lane<kExp2Pwl2>(x);
}

template <int V>
struct Exp2FractionOp {
    static constexpr int NIN = 1, NOUT = 1;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[1], uint32_t (&b)[1]) {
        b[0] = as_u32(exp2_fraction_f16<V>(as_h2(a[0])));
    }
};

// ---- compute probes ---------------------------------------------------------
// The reference's protocol: `threads` threads (65,536 there) in blocks of 256,
// each with kProbeChains independent pairs read once and `iterations` rounds
// of x <- feedback(program(x)); one pair per thread is stored (chain
// thread % 8) so that no evaluation is dead.  65,536 threads are one wave per
// SIMD on MI355X, where the chains' dependency latency sets the time; eight
// times that many fill every SIMD with eight waves and measure issue rate.  FP16 feedback (chains 0-3 / 4-7):
// fma(v, 1/2, -1/2) maps [1, 2] to [0, 1/2], fma(v, -1/2, 3/2) to [1/2, 1];
// FP32: fma(v, 8, -16) and -8 v, keeping x in [-16, 0].

constexpr int kProbeChains = 8;
constexpr int kProbeBlock = 256;

template <int V>
__global__ void __launch_bounds__(kProbeBlock)
    exp2_compute_f16x2_kernel(const uint32_t* __restrict__ in, uint32_t* __restrict__ out, int threads,
                              int iterations) {
    const int i = blockIdx.x * kProbeBlock + threadIdx.x;
    h2_t x[kProbeChains];
#pragma unroll
    for (int c = 0; c < kProbeChains; ++c) x[c] = as_h2(in[i + c * threads]);
    const h2_t lo_scale = {(_Float16)0.5f, (_Float16)0.5f}, lo_bias = {(_Float16)-0.5f, (_Float16)-0.5f};
    const h2_t hi_scale = {(_Float16)-0.5f, (_Float16)-0.5f}, hi_bias = {(_Float16)1.5f, (_Float16)1.5f};
    for (int it = 0; it < iterations; ++it) {
#pragma unroll
        for (int c = 0; c < kProbeChains; ++c) {
            const h2_t v = exp2_fraction_f16<V>(x[c]);
            x[c] = c < kProbeChains / 2 ? __builtin_elementwise_fma(v, lo_scale, lo_bias)
                                        : __builtin_elementwise_fma(v, hi_scale, hi_bias);
        }
    }
    uint32_t r = 0;
#pragma unroll
    for (int c = 0; c < kProbeChains; ++c)
        if ((i & (kProbeChains - 1)) == c) r = as_u32(x[c]);
    out[i] = r;
}

template <int V>
__global__ void __launch_bounds__(kProbeBlock)
    exp2_compute_f32x2_kernel(const float2* __restrict__ in, float2* __restrict__ out, int threads, int iterations) {
    const int i = blockIdx.x * kProbeBlock + threadIdx.x;
    float x[kProbeChains][2];
#pragma unroll
    for (int c = 0; c < kProbeChains; ++c) {
        const float2 v = in[i + c * threads];
        x[c][0] = v.x;
        x[c][1] = v.y;
    }
    for (int it = 0; it < iterations; ++it) {
#pragma unroll
        for (int c = 0; c < kProbeChains; ++c)
#pragma unroll
            for (int l = 0; l < 2; ++l) {
                const float v = exp2_full_f32<V>(x[c][l]);
                x[c][l] = c < kProbeChains / 2 ? __builtin_fmaf(v, 8.0f, -16.0f) : -8.0f * v;
            }
    }
    float2 r = {0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < kProbeChains; ++c)
        if ((i & (kProbeChains - 1)) == c) r = {x[c][0], x[c][1]};
    out[i] = r;
}

extern "C" int launch_exp2_fraction_native_f16(void* y, const void* x, int64_t size, void* stream) {
    return run1<Exp2FractionOp<kFracNative>>(y, x, size, stream);
}
extern "C" int launch_exp2_fraction_pwl2_historical_f16(void* y, const void* x, int64_t size, void* stream) {
    return run1<Exp2FractionOp<kFracPwl2Historical>>(y, x, size, stream);
}
extern "C" int launch_exp2_fraction_pwl2_hinge_f16(void* y, const void* x, int64_t size, void* stream) {
    return run1<Exp2FractionOp<kFracPwl2Hinge>>(y, x, size, stream);
}

// threads: a positive multiple of 256, at most 2^24 (the grid is threads / 256
// blocks and the input's 8 * threads pairs are indexed in int).
inline bool probe_shape_ok(const void* out, const void* in, int64_t threads, int iterations) {
    return out && in && iterations >= 0 && threads > 0 && threads % kProbeBlock == 0 && threads <= (1 << 24);
}

extern "C" int launch_exp2_compute_f16x2(int variant, void* out, const void* in, int64_t threads, int iterations,
                                         void* stream) {
    if (!probe_shape_ok(out, in, threads, iterations)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)(threads / kProbeBlock)), block(kProbeBlock);
    const uint32_t* src = static_cast<const uint32_t*>(in);
    uint32_t* dst = static_cast<uint32_t*>(out);
    const int t = (int)threads;
    switch (variant) {
        case kFracNative:
            hipLaunchKernelGGL(exp2_compute_f16x2_kernel<kFracNative>, grid, block, 0, hs(stream), src, dst, t,
                               iterations);
            break;
        case kFracPwl2Historical:
            hipLaunchKernelGGL(exp2_compute_f16x2_kernel<kFracPwl2Historical>, grid, block, 0, hs(stream), src, dst,
                               t, iterations);
            break;
        case kFracPwl2Hinge:
            hipLaunchKernelGGL(exp2_compute_f16x2_kernel<kFracPwl2Hinge>, grid, block, 0, hs(stream), src, dst, t,
                               iterations);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

extern "C" int launch_exp2_compute_f32x2(int variant, void* out, const void* in, int64_t threads, int iterations,
                                         void* stream) {
    if (!probe_shape_ok(out, in, threads, iterations)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)(threads / kProbeBlock)), block(kProbeBlock);
    const float2* src = static_cast<const float2*>(in);
    float2* dst = static_cast<float2*>(out);
    const int t = (int)threads;
    switch (variant) {
        case kFullNative:
            hipLaunchKernelGGL(exp2_compute_f32x2_kernel<kFullNative>, grid, block, 0, hs(stream), src, dst, t,
                               iterations);
            break;
        case kFullDegree3:
            hipLaunchKernelGGL(exp2_compute_f32x2_kernel<kFullDegree3>, grid, block, 0, hs(stream), src, dst, t,
                               iterations);
            break;
        case kFullPwl2Hinge:
            hipLaunchKernelGGL(exp2_compute_f32x2_kernel<kFullPwl2Hinge>, grid, block, 0, hs(stream), src, dst, t,
                               iterations);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace pt
