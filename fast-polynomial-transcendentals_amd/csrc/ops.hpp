// ops.hpp -- pairwise operations (one 32-bit pair of each input stream ->
// one pair of each output stream) and the small helpers shared by the C-ABI
// translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <initializer_list>

#include "elementwise.hpp"
#include "programs.hpp"

namespace pt {

// out = P(x)
template <class P>
struct UnaryOp {
    static constexpr int NIN = 1, NOUT = 1;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[1], uint32_t (&b)[1]) {
        b[0] = P::eval(a[0]);
    }
};

// FP16: gi = go * P(x)   (binary_vec_kernel, spline_kernels.cu:66-89)
template <class P>
struct F16MulOp {
    static constexpr int NIN = 2, NOUT = 1;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[2], uint32_t (&b)[1]) {
        b[0] = as_u32(as_h2(a[0]) * as_h2(P::eval(a[1])));
    }
};

// BF16: gi = go * P(x)   (binary_vec_kernel_bf16, spline_kernels_bf16.cu:74-95).
// The product of two BF16 values is exact in FP32, so one RNE pack is the
// single rounding of __hmul2.
template <class P>
struct BF16MulOp {
    static constexpr int NIN = 2, NOUT = 1;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[2], uint32_t (&b)[1]) {
        float d_lo, d_hi;
        P::eval2(a[1], d_lo, d_hi);
        b[0] = pack_bf(bf_lo(a[0]) * d_lo, bf_hi(a[0]) * d_hi);
    }
};

// FP16: out = F(gate) * up   (swish_mul_vec_kernel, spline_kernels.cu:137-158)
template <class P>
struct F16SwishMulOp {
    static constexpr int NIN = 2, NOUT = 1;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[2], uint32_t (&b)[1]) {
        b[0] = as_u32(as_h2(P::eval(a[0])) * as_h2(a[1]));
    }
};

// BF16: out = F(gate) * up   (swish_mul_vec_kernel_bf16, spline_kernels_bf16.cu:143-164)
template <class P>
struct BF16SwishMulOp {
    static constexpr int NIN = 2, NOUT = 1;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[2], uint32_t (&b)[1]) {
        float s_lo, s_hi;
        P::eval2(a[0], s_lo, s_hi);
        b[0] = pack_bf(s_lo * bf_lo(a[1]), s_hi * bf_hi(a[1]));
    }
};

// SwiGLU backward, inputs (go, gate, up), outputs (grad_gate, grad_up):
// grad_gate = (go*up) * B(gate), grad_up = go * F(gate)
// (swish_mul_bwd_vec_kernel, spline_kernels.cu:160-214,
//  spline_kernels_bf16.cu:208-253).
template <class PF, class PB>
struct F16SwishMulBwdOp {
    static constexpr int NIN = 3, NOUT = 2;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[3], uint32_t (&b)[2]) {
        const h2_t go = as_h2(a[0]);
        b[0] = as_u32((go * as_h2(a[2])) * as_h2(PB::eval(a[1])));
        b[1] = as_u32(go * as_h2(PF::eval(a[1])));
    }
};

template <class PF, class PB>
struct BF16SwishMulBwdOp {
    static constexpr int NIN = 3, NOUT = 2;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[3], uint32_t (&b)[2]) {
        float s_lo, s_hi, d_lo, d_hi;
        PF::eval2(a[1], s_lo, s_hi);
        PB::eval2(a[1], d_lo, d_hi);
        const float gu_lo = rbf(bf_lo(a[0]) * bf_lo(a[2]));
        const float gu_hi = rbf(bf_hi(a[0]) * bf_hi(a[2]));
        b[0] = pack_bf(gu_lo * d_lo, gu_hi * d_hi);
        b[1] = pack_bf(bf_lo(a[0]) * s_lo, bf_hi(a[0]) * s_hi);
    }
};

// BF16 degree-3 SwiGLU backward with the algebraic derivative
// (swish_d3_fwd_bwd_alg_bf16, spline_kernels_bf16.cu:255-265):
// s = sigmoid_d3(x); swish = x*s; d = fma(swish, 1 - s, s).
struct BF16SwishMulBwdD3AlgOp {
    static constexpr int NIN = 3, NOUT = 2;
    __device__ __forceinline__ static void lane(float go, float x, float up, float sig,
                                                float& gg, float& gu) {
        const float swish = rbf(x * sig);
        const float d = bfma(swish, rbf(1.0f - sig), sig);
        gg = rbf(go * up) * d;
        gu = go * swish;
    }
    __device__ __forceinline__ static void pair(const uint32_t (&a)[3], uint32_t (&b)[2]) {
        float s_lo, s_hi;
        BF16Prog<kSigmoid, kFwd, 3>::eval2(a[1], s_lo, s_hi);
        float gg_lo, gu_lo, gg_hi, gu_hi;
        lane(bf_lo(a[0]), bf_lo(a[1]), bf_lo(a[2]), s_lo, gg_lo, gu_lo);
        lane(bf_hi(a[0]), bf_hi(a[1]), bf_hi(a[2]), s_hi, gg_hi, gu_hi);
        b[0] = pack_bf(gg_lo, gg_hi);
        b[1] = pack_bf(gu_lo, gu_hi);
    }
};

// Native SwiGLU backward on separate tensors (swish_mul_bwd_vec_kernel with
// SWISH_{FWD,BWD}_NATIVE): both factors are rounded to 16 bits first.
template <bool BF>
struct NativeSwishMulBwdOp {
    static constexpr int NIN = 3, NOUT = 2;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[3], uint32_t (&b)[2]) {
        if constexpr (BF) {
            BF16SwishMulBwdOp<BF16Native<kSwishFam, kFwd>, BF16Native<kSwishFam, kBwd>>::pair(a, b);
        } else {
            F16SwishMulBwdOp<F16Native<kSwishFam, kFwd>, F16Native<kSwishFam, kBwd>>::pair(a, b);
        }
    }
};

// Native SwiGLU backward of the packed layout (the specialisation
// swish_mul_packed_grads<SWISH_FWD_NATIVE, SWISH_BWD_NATIVE>,
// spline_kernels.cu:397-416, spline_kernels_bf16.cu:397-419):
// dy = go*up rounded to 16 bits, grad_gate = dy * s * (1 + x(1-s)) in FP32
// with one rounding, grad_up = go * native_swish(gate).
template <bool BF>
struct PackedNativeSwishMulBwdOp {
    static constexpr int NIN = 3, NOUT = 2;
    __device__ __forceinline__ static float gg_lane(float dy, float x) {
        const float s = nat_sigmoid(x);
        return dy * s * (1.0f + x * (1.0f - s));
    }
    __device__ __forceinline__ static void pair(const uint32_t (&a)[3], uint32_t (&b)[2]) {
        if constexpr (BF) {
            const float dy_lo = rbf(bf_lo(a[0]) * bf_lo(a[2]));
            const float dy_hi = rbf(bf_hi(a[0]) * bf_hi(a[2]));
            b[0] = pack_bf(gg_lane(dy_lo, bf_lo(a[1])), gg_lane(dy_hi, bf_hi(a[1])));
            float s_lo, s_hi;
            BF16Native<kSwishFam, kFwd>::eval2(a[1], s_lo, s_hi);
            b[1] = pack_bf(bf_lo(a[0]) * s_lo, bf_hi(a[0]) * s_hi);
        } else {
            const h2_t dy = as_h2(a[0]) * as_h2(a[2]);
            const h2_t x = as_h2(a[1]);
            const h2_t gg = {(_Float16)gg_lane((float)dy.x, (float)x.x),
                             (_Float16)gg_lane((float)dy.y, (float)x.y)};
            b[0] = as_u32(gg);
            b[1] = as_u32(as_h2(a[0]) * as_h2(F16Native<kSwishFam, kFwd>::eval(a[1])));
        }
    }
};

// ---------------------------------------------------------------------------
// C-ABI helpers
// ---------------------------------------------------------------------------

inline hipStream_t hs(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool bad_args(int64_t n, std::initializer_list<const void*> ptrs) {
    if (n < 0) return true;
    if (n == 0) return false;
    for (const void* p : ptrs)
        if (p == nullptr) return true;
    return false;
}

template <class Op>
int run1(void* out, const void* in, int64_t n, void* stream) {
    if (bad_args(n, {out, in})) return hipErrorInvalidValue;
    Streams<Op::NIN, Op::NOUT> s{{in}, {out}};
    return launch_pairwise<Op>(s, n, hs(stream));
}

template <class Op>
int run2(void* out, const void* a, const void* b, int64_t n, void* stream) {
    if (bad_args(n, {out, a, b})) return hipErrorInvalidValue;
    Streams<Op::NIN, Op::NOUT> s{{a, b}, {out}};
    return launch_pairwise<Op>(s, n, hs(stream));
}

template <class Op>
int run_bwd3(void* gg, void* gu, const void* go, const void* gate, const void* up, int64_t n,
             void* stream) {
    if (bad_args(n, {gg, gu, go, gate, up})) return hipErrorInvalidValue;
    Streams<3, 2> s{{go, gate, up}, {gg, gu}};
    return launch_pairwise<Op>(s, n, hs(stream));
}

}  // namespace pt

// Macro arguments that contain commas are parenthesised; PT_STRIP removes
// the parentheses.
#define PT_STRIP(...) __VA_ARGS__
