// sincos.hip -- paired sin/cos tables and their repeated-evaluation
// ("compute") probes for gfx950, with their C ABI.
//
// Tables: FP32 angles [n] -> [2, n] (plane 0 cos, plane 1 sin).
//  * 16-bit outputs: a thread reads 8 angles (two 16-byte loads) and writes
//    one 16-byte vector to each plane.
//  * FP32 outputs: a thread reads 4 angles and writes 16 bytes to each plane.
// Elements past the last full vector, or every element when a pointer is not
// 16-byte aligned, take an element path with identical results (the programs
// are lane-independent).
//
// Compute probes (sincos_compute_*_kernel, sincos_kernels.cu:1014-1240):
// each element evaluates its program `iterations` times on a probe angle
// that steps by p <- fma(p, 0.99999994, 2^-13) and writes the running sums
// (FP32 adds, or packed 16-bit adds for the 16-bit programs).  The loads and
// stores are negligible next to the evaluations, so these time the
// instruction issue of a program rather than the memory system.
#include <hip/hip_runtime.h>

#include "ops.hpp"
#include "spline_ops_hip.h"
#include "trig.hpp"

namespace pt {

constexpr float kProbeScale = 0.999999940395355224609375f;
constexpr float kProbeOffset = 0.0001220703125f;

__device__ __forceinline__ float probe_step(float p) { return __builtin_fmaf(p, kProbeScale, kProbeOffset); }

// Packed 16-bit add of two pairs (__hadd2).  For BF16 the FP32 sum of two
// BF16 values rounded once to BF16 is the correctly rounded BF16 sum: when
// the exponents differ by more than 16 the FP32 rounding error is far below
// the BF16 half-ulp distance to any tie.
template <bool BF>
__device__ __forceinline__ uint32_t add_pair(uint32_t a, uint32_t b) {
    if constexpr (BF) return pack_bf(bf_lo(a) + bf_lo(b), bf_hi(a) + bf_hi(b));
    else return as_u32(as_h2(a) + as_h2(b));
}

// ---------------------------------------------------------------------------
// 16-bit tables and probes
// ---------------------------------------------------------------------------

template <class E>
__global__ void __launch_bounds__(kBlock)
sincos_table_kernel(const float* __restrict__ angles, uint16_t* __restrict__ out, int64_t n,
                    int vec_ok) {
    uint16_t* cos_plane = out;
    uint16_t* sin_plane = out + n;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const int64_t n8 = vec_ok ? (n >> 3) : 0;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n8; i += stride) {
        const Vec4 a = ld16<false>(angles, 2 * i);
        const Vec4 b = ld16<false>(angles, 2 * i + 1);
        const uint32_t w[8] = {a.w[0], a.w[1], a.w[2], a.w[3], b.w[0], b.w[1], b.w[2], b.w[3]};
        Vec4 oc, os;
#pragma unroll
        for (int k = 0; k < 4; ++k) E::eval(as_f32(w[2 * k]), as_f32(w[2 * k + 1]), oc.w[k], os.w[k]);
        st16<false>(cos_plane, i, oc);
        st16<false>(sin_plane, i, os);
    }
    for (int64_t e = (n8 << 3) + (int64_t)blockIdx.x * kBlock + threadIdx.x; e < n; e += stride) {
        uint32_t c, s;
        E::eval(angles[e], angles[e], c, s);
        cos_plane[e] = (uint16_t)(c & 0xffffu);
        sin_plane[e] = (uint16_t)(s & 0xffffu);
    }
}

template <class E, bool BF>
__global__ void __launch_bounds__(kBlock)
sincos_compute_kernel(const float* __restrict__ angles, uint16_t* __restrict__ out, int64_t n,
                      int vec_ok, int iterations) {
    uint16_t* cos_plane = out;
    uint16_t* sin_plane = out + n;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const int64_t n8 = vec_ok ? (n >> 3) : 0;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n8; i += stride) {
        const Vec4 a = ld16<false>(angles, 2 * i);
        const Vec4 b = ld16<false>(angles, 2 * i + 1);
        float p[8] = {as_f32(a.w[0]), as_f32(a.w[1]), as_f32(a.w[2]), as_f32(a.w[3]),
                      as_f32(b.w[0]), as_f32(b.w[1]), as_f32(b.w[2]), as_f32(b.w[3])};
        Vec4 oc{{0u, 0u, 0u, 0u}}, os{{0u, 0u, 0u, 0u}};
#pragma unroll 1
        for (int it = 0; it < iterations; ++it) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint32_t c, s;
                E::eval(p[2 * k], p[2 * k + 1], c, s);
                oc.w[k] = add_pair<BF>(oc.w[k], c);
                os.w[k] = add_pair<BF>(os.w[k], s);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) p[k] = probe_step(p[k]);
        }
        st16<false>(cos_plane, i, oc);
        st16<false>(sin_plane, i, os);
    }
    for (int64_t e = (n8 << 3) + (int64_t)blockIdx.x * kBlock + threadIdx.x; e < n; e += stride) {
        float p = angles[e];
        uint32_t cs = 0u, ss = 0u;
        for (int it = 0; it < iterations; ++it) {
            uint32_t c, s;
            E::eval(p, p, c, s);
            cs = add_pair<BF>(cs, c);
            ss = add_pair<BF>(ss, s);
            p = probe_step(p);
        }
        cos_plane[e] = (uint16_t)(cs & 0xffffu);
        sin_plane[e] = (uint16_t)(ss & 0xffffu);
    }
}

template <class E>
int launch_sincos_table(void* out, const void* angles, int64_t n, void* stream) {
    if (bad_args(n, {out, angles})) return hipErrorInvalidValue;
    if (n == 0) return hipSuccess;
    // Both planes are 16-byte aligned only when n is a multiple of 8.
    const int vec_ok = aligned16(out) && aligned16(angles) && (n % 8 == 0);
    const int64_t grid = grid_one_pass(vec_ok ? (n >> 3) : n);
    hipLaunchKernelGGL((sincos_table_kernel<E>), dim3((unsigned)grid), dim3(kBlock), 0, hs(stream),
                       (const float*)angles, (uint16_t*)out, n, vec_ok);
    return hipGetLastError();
}

template <class E, bool BF>
int launch_sincos_compute(void* out, const void* angles, int64_t n, int64_t iterations,
                          void* stream) {
    if (bad_args(n, {out, angles}) || iterations <= 0 || iterations > 0x7fffffff)
        return hipErrorInvalidValue;
    if (n == 0) return hipSuccess;
    const int vec_ok = aligned16(out) && aligned16(angles) && (n % 8 == 0);
    const int64_t grid = grid_one_pass(vec_ok ? (n >> 3) : n);
    hipLaunchKernelGGL((sincos_compute_kernel<E, BF>), dim3((unsigned)grid), dim3(kBlock), 0,
                       hs(stream), (const float*)angles, (uint16_t*)out, n, vec_ok,
                       (int)iterations);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// FP32 tables and probes
// ---------------------------------------------------------------------------

template <class E>
__global__ void __launch_bounds__(kBlock)
sincos_f32_kernel(const float* __restrict__ angles, float* __restrict__ out, int64_t n, int vec_ok,
                  int iterations) {
    float* cos_plane = out;
    float* sin_plane = out + n;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const int64_t n4 = vec_ok ? (n >> 2) : 0;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride) {
        const Vec4 a = ld16<false>(angles, i);
        Vec4 oc, os;
        if (iterations == 0) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float c, s;
                E::eval(as_f32(a.w[k]), c, s);
                oc.w[k] = as_u32(c);
                os.w[k] = as_u32(s);
            }
        } else {
            float p[4], cs[4] = {0.f, 0.f, 0.f, 0.f}, ss[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 4; ++k) p[k] = as_f32(a.w[k]);
#pragma unroll 1
            for (int it = 0; it < iterations; ++it) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    float c, s;
                    E::eval(p[k], c, s);
                    cs[k] += c;
                    ss[k] += s;
                    p[k] = probe_step(p[k]);
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                oc.w[k] = as_u32(cs[k]);
                os.w[k] = as_u32(ss[k]);
            }
        }
        st16<false>(cos_plane, i, oc);
        st16<false>(sin_plane, i, os);
    }
    for (int64_t e = (n4 << 2) + (int64_t)blockIdx.x * kBlock + threadIdx.x; e < n; e += stride) {
        float c, s;
        if (iterations == 0) {
            E::eval(angles[e], c, s);
        } else {
            float p = angles[e];
            c = 0.f;
            s = 0.f;
            for (int it = 0; it < iterations; ++it) {
                float ci, si;
                E::eval(p, ci, si);
                c += ci;
                s += si;
                p = probe_step(p);
            }
        }
        cos_plane[e] = c;
        sin_plane[e] = s;
    }
}

// iterations == 0: table; > 0: compute probe.
template <class E>
int launch_sincos_f32(void* out, const void* angles, int64_t n, int64_t iterations, void* stream) {
    if (bad_args(n, {out, angles}) || iterations < 0 || iterations > 0x7fffffff)
        return hipErrorInvalidValue;
    if (n == 0) return hipSuccess;
    const int vec_ok = aligned16(out) && aligned16(angles) && (n % 4 == 0);
    const int64_t grid = grid_one_pass(vec_ok ? (n >> 2) : n);
    hipLaunchKernelGGL((sincos_f32_kernel<E>), dim3((unsigned)grid), dim3(kBlock), 0, hs(stream),
                       (const float*)angles, (float*)out, n, vec_ok, (int)iterations);
    return hipGetLastError();
}

}  // namespace pt

using namespace pt;

// ---- 16-bit tables -------------------------------------------------------------

#define PT_SINCOS(name, EVAL)                                                         \
    extern "C" int name(void* out, const void* angles, int64_t size, void* stream) {  \
        return launch_sincos_table<PT_STRIP EVAL>(out, angles, size, stream);         \
    }
#define PT_SINCOS_COMPUTE(name, EVAL, BF)                                                     \
    extern "C" int name(void* out, const void* angles, int64_t size, int64_t iterations,      \
                        void* stream) {                                                       \
        return launch_sincos_compute<PT_STRIP EVAL, BF>(out, angles, size, iterations, stream); \
    }

PT_SINCOS(launch_sincos_native_bf16, (NativeSinCos<true>))
PT_SINCOS(launch_sincos_d3_d4_bf16, (BF16Quarter<true>))
PT_SINCOS(launch_sincos_d3_d4_quarter_turn_bf16, (BF16Quarter<false>))
PT_SINCOS(launch_sincos_d3_d4_half_turn_bf16, (BF16HalfTurn<kBf16HalfD3D4>))
PT_SINCOS(launch_sincos_d5_d6_half_turn_bf16, (BF16HalfTurn<kBf16HalfD5D6>))
PT_SINCOS(launch_sincos_d5_d4_half_turn_fp16_bf16, (F16HalfTurnToBF16<kF16HalfD5D4>))
PT_SINCOS(launch_sincos_native_fp16, (NativeSinCos<false>))
PT_SINCOS(launch_sincos_d3_d4_quarter_turn_fp16, (F16Quarter))
PT_SINCOS(launch_sincos_d3_d4_half_turn_fp16, (F16HalfTurn<kF16HalfD3D4>))
PT_SINCOS(launch_sincos_d5_d4_half_turn_fp16, (F16HalfTurn<kF16HalfD5D4>))
PT_SINCOS(launch_sincos_d5_d6_half_turn_fp16, (F16HalfTurn<kF16HalfD5D6>))
PT_SINCOS(launch_sincos_d7_d6_half_turn_fp16, (F16HalfTurn<kF16HalfD7D6>))

PT_SINCOS_COMPUTE(launch_sincos_native_bf16_compute, (NativeSinCos<true>), true)
PT_SINCOS_COMPUTE(launch_sincos_d3_d4_bf16_compute, (BF16Quarter<true>), true)
PT_SINCOS_COMPUTE(launch_sincos_d3_d4_quarter_turn_bf16_compute, (BF16Quarter<false>), true)
PT_SINCOS_COMPUTE(launch_sincos_d3_d4_half_turn_bf16_compute, (BF16HalfTurn<kBf16HalfD3D4>), true)
PT_SINCOS_COMPUTE(launch_sincos_d5_d6_half_turn_bf16_compute, (BF16HalfTurn<kBf16HalfD5D6>), true)
PT_SINCOS_COMPUTE(launch_sincos_d5_d4_half_turn_fp16_bf16_compute, (F16HalfTurnToBF16<kF16HalfD5D4>), true)
PT_SINCOS_COMPUTE(launch_sincos_native_fp16_compute, (NativeSinCos<false>), false)
PT_SINCOS_COMPUTE(launch_sincos_d3_d4_quarter_turn_fp16_compute, (F16Quarter), false)
PT_SINCOS_COMPUTE(launch_sincos_d3_d4_half_turn_fp16_compute, (F16HalfTurn<kF16HalfD3D4>), false)
PT_SINCOS_COMPUTE(launch_sincos_d5_d4_half_turn_fp16_compute, (F16HalfTurn<kF16HalfD5D4>), false)
PT_SINCOS_COMPUTE(launch_sincos_d5_d6_half_turn_fp16_compute, (F16HalfTurn<kF16HalfD5D6>), false)
PT_SINCOS_COMPUTE(launch_sincos_d7_d6_half_turn_fp16_compute, (F16HalfTurn<kF16HalfD7D6>), false)

// ---- FP32 ------------------------------------------------------------------------

#define PT_SINCOS_F32(base, EVAL)                                                              \
    extern "C" int launch_sincos_##base##_f32(void* out, const void* angles, int64_t size,     \
                                              void* stream) {                                  \
        return launch_sincos_f32<PT_STRIP EVAL>(out, angles, size, 0, stream);                 \
    }                                                                                          \
    extern "C" int launch_sincos_##base##_compute_f32(void* out, const void* angles,           \
                                                      int64_t size, int64_t iterations,        \
                                                      void* stream) {                          \
        if (iterations <= 0) return hipErrorInvalidValue;                                      \
        return launch_sincos_f32<PT_STRIP EVAL>(out, angles, size, iterations, stream);        \
    }

PT_SINCOS_F32(native, (F32Native))
PT_SINCOS_F32(d3_d4, (F32Prog<kF32D3D4>))
PT_SINCOS_F32(d3_d4_cycle, (F32Cycle))
PT_SINCOS_F32(d3_d4_magic_bias, (F32Prog<kF32D3D4Shift>))
PT_SINCOS_F32(d5_d4_half_turn_ls, (F32Prog<kF32HalfD5D4Ls>))
PT_SINCOS_F32(d5_d4_half_turn_sollya, (F32Prog<kF32HalfD5D4Sollya>))
PT_SINCOS_F32(d5_d4_half_turn_sollya_fast, (F32Prog<kF32HalfD5D4SollyaFast>))
PT_SINCOS_F32(d5_d4, (F32Prog<kF32D5D4>))
PT_SINCOS_F32(d7_d6, (F32Prog<kF32D7D6>))

// ---------------------------------------------------------------------------
// RoPE reference evaluator (src/sfu_repro/rope/polynomial_sincos.py:85-165):
// quarter-turn reduction in FP64 ("accurate", for cached tables) or FP32
// Cody-Waite ("fast"), then sin = r * S(r^2), cos = C(r^2) with Horner steps
// that round the product and the sum separately (value * x + c, as the
// reference's tensor arithmetic does), then the quadrant swap and signs.
// Coefficients arrive by value, lowest power first.
// ---------------------------------------------------------------------------

namespace pt {

constexpr int kMaxRefCoeffs = 8;

struct RefPoly {
    int ns, nc;
    float s[kMaxRefCoeffs], c[kMaxRefCoeffs];
};

__device__ __forceinline__ float ref_horner(float x, const float* c, int n) {
    float v = c[n - 1];
    for (int i = n - 2; i >= 0; --i) v = v * x + c[i];  // two roundings per step
    return v;
}

// float -> int64 conversion with the host's conventions for NaN and
// out-of-range values (INT64_MIN), so quadrant = q & 3 is defined for all.
template <class T>
__device__ __forceinline__ int64_t ref_to_i64(T q) {
    const T lim = (T)9223372036854775808.0;
    return (q < lim && q > -lim) ? (int64_t)q : INT64_MIN;
}

__device__ __forceinline__ void ref_reduce(const void* angles, int f64, int64_t i, int accurate,
                                           float& r, int64_t& quadrant) {
    if (accurate) {
        const double w = f64 ? ((const double*)angles)[i] : (double)((const float*)angles)[i];
        const double q = __builtin_rint(w * 0.6366197723675814);
        r = (float)(w - q * 1.5707963267948966);
        quadrant = ref_to_i64(q) & 3;
    } else {
        const float w = f64 ? (float)((const double*)angles)[i] : ((const float*)angles)[i];
        const float q = __builtin_rintf(w * 0.63661977236758134f);
        r = (w - q * 1.570796251296997f) - q * 7.549789415861596e-08f;
        quadrant = ref_to_i64(q) & 3;
    }
}

// mode 0: (cos, sin) of angles; 1: (reduced, quadrant); 2: (sin, cos) of
// reduced arguments (evaluate_reduced_sincos).
__global__ void __launch_bounds__(kBlock)
ref_sincos_kernel(const void* __restrict__ in, int in_f64, void* __restrict__ out0,
                  void* __restrict__ out1, int64_t n, int mode, int accurate, RefPoly p) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        float r;
        int64_t q = 0;
        if (mode == 2) {
            r = in_f64 ? (float)((const double*)in)[i] : ((const float*)in)[i];
        } else {
            ref_reduce(in, in_f64, i, accurate, r, q);
            if (mode == 1) {
                ((float*)out0)[i] = r;
                ((int64_t*)out1)[i] = q;
                continue;
            }
        }
        const float sq = r * r;
        const float sr = r * ref_horner(sq, p.s, p.ns);
        const float cr = ref_horner(sq, p.c, p.nc);
        if (mode == 2) {
            ((float*)out0)[i] = sr;
            ((float*)out1)[i] = cr;
            continue;
        }
        const bool swap = (q & 1) != 0;
        const float sm = swap ? cr : sr;
        const float cm = swap ? sr : cr;
        ((float*)out0)[i] = ((q + 1) & 2) ? -cm : cm;  // cos < 0 in quadrants 1, 2
        ((float*)out1)[i] = (q & 2) ? -sm : sm;         // sin < 0 in quadrants 2, 3
    }
}

}  // namespace pt

// Returns hipErrorInvalidValue for more than 8 coefficients per polynomial or
// none at all.
static int launch_ref_sincos(const void* in, int in_f64, void* out0, void* out1, int64_t n, int mode,
                             int accurate, const float* s, int ns, const float* c, int nc,
                             void* stream) {
    if (bad_args(n, {in, out0, out1})) return hipErrorInvalidValue;
    RefPoly p{};
    if (mode != 1) {
        if (!s || !c || ns < 1 || nc < 1 || ns > kMaxRefCoeffs || nc > kMaxRefCoeffs)
            return hipErrorInvalidValue;
        p.ns = ns;
        p.nc = nc;
        for (int k = 0; k < ns; ++k) p.s[k] = s[k];
        for (int k = 0; k < nc; ++k) p.c[k] = c[k];
    }
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(ref_sincos_kernel, dim3((unsigned)grid_one_pass(n)), dim3(kBlock), 0,
                       hs(stream), in, in_f64, out0, out1, n, mode, accurate, p);
    return hipGetLastError();
}

extern "C" int launch_polynomial_sincos_f32(void* cos_out, void* sin_out, const void* angles,
                                            int angles_f64, int64_t size, int accurate,
                                            const float* sin_coeffs, int n_sin,
                                            const float* cos_coeffs, int n_cos, void* stream) {
    // mode 0 writes cos then sin (the kernel's out0 is the cosine)
    return launch_ref_sincos(angles, angles_f64, cos_out, sin_out, size, 0, accurate, sin_coeffs,
                             n_sin, cos_coeffs, n_cos, stream);
}

extern "C" int launch_reduce_to_quarter_turn(void* reduced_out, void* quadrant_out,
                                             const void* angles, int angles_f64, int64_t size,
                                             int accurate, void* stream) {
    return launch_ref_sincos(angles, angles_f64, reduced_out, quadrant_out, size, 1, accurate,
                             nullptr, 0, nullptr, 0, stream);
}

extern "C" int launch_evaluate_reduced_sincos(void* sin_out, void* cos_out, const void* reduced,
                                              int reduced_f64, int64_t size,
                                              const float* sin_coeffs, int n_sin,
                                              const float* cos_coeffs, int n_cos, void* stream) {
    return launch_ref_sincos(reduced, reduced_f64, sin_out, cos_out, size, 2, 1, sin_coeffs, n_sin,
                             cos_coeffs, n_cos, stream);
}
