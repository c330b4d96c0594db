// experiments.hip -- the reference's FP16 experiment kernels for gfx950, with
// their C ABI: hybrid transcendental/polynomial programs, fused forward +
// backward, forward-with-derivative pairs and the elementwise multiply
// (autonumerics_zero/spline_ops/spline_kernels.cu:776-1168, 1394-1480).
//
// Every op runs through the one-pass 16-byte streaming driver of
// elementwise.hpp.  Semantics follow the reference's vector path for every
// size; where its small-size fallbacks compute something else (fwd_deriv_alg
// returns y * y' there, swish_fwd_deriv switches programs, multiply drops the
// tail) this build keeps the vector-path result, so outputs do not depend on
// the tensor size.
#include <hip/hip_runtime.h>

#include "ops.hpp"
#include "spline_ops_hip.h"

namespace pt {

// ---------------------------------------------------------------------------
// hybrid: the first pair of every 16-byte vector through the hardware
// transcendental unit, the other three through the polynomial
// (hybrid_vec_kernel / hybrid_bwd_vec_kernel, spline_kernels.cu:816-862).
// The transcendental lanes use the native programs (v_exp_f32 / v_rcp_f32,
// rounded to FP16): gfx950 issues its FP32 and FP16 transcendentals at the
// same rate, and the FP32 form is the more accurate one.
// ---------------------------------------------------------------------------

template <int F, class Poly>
struct HybridFwdOp {
    static constexpr int NIN = 1, NOUT = 1;
    static constexpr bool kPositional = true;
    template <int W>
    __device__ __forceinline__ static void pair_at(const uint32_t (&a)[1], uint32_t (&b)[1]) {
        if constexpr (W == 0) b[0] = F16Native<F, kFwd>::eval(a[0]);
        else b[0] = Poly::eval(a[0]);
    }
    __device__ __forceinline__ static void pair(const uint32_t (&a)[1], uint32_t (&b)[1]) {
        b[0] = Poly::eval(a[0]);
    }
};

template <int F, class Poly>
struct HybridBwdOp {  // inputs (grad_out, x)
    static constexpr int NIN = 2, NOUT = 1;
    static constexpr bool kPositional = true;
    template <int W>
    __device__ __forceinline__ static void pair_at(const uint32_t (&a)[2], uint32_t (&b)[1]) {
        const uint32_t d = W == 0 ? F16Native<F, kBwd>::eval(a[1]) : Poly::eval(a[1]);
        b[0] = as_u32(as_h2(a[0]) * as_h2(d));
    }
    __device__ __forceinline__ static void pair(const uint32_t (&a)[2], uint32_t (&b)[1]) {
        b[0] = as_u32(as_h2(a[0]) * as_h2(Poly::eval(a[1])));
    }
};

// The hybrid split exists only on the reference's vector path (at least 4096
// pairs, a multiple of 4 pairs); smaller or ragged tensors are all
// polynomial (launch_hybrid_unary / launch_hybrid_binary, :1127-1168).
inline bool hybrid_split(int64_t n) { return n >= 8192 && n % 8 == 0; }

template <int F, class Poly>
int run_hybrid_fwd(void* out, const void* in, int64_t n, void* stream) {
    if (bad_args(n, {out, in})) return hipErrorInvalidValue;
    Streams<1, 1> s{{in}, {out}};
    if (hybrid_split(n)) return launch_pairwise<HybridFwdOp<F, Poly>>(s, n, hs(stream));
    return launch_pairwise<UnaryOp<Poly>>(s, n, hs(stream));
}

template <int F, class Poly>
int run_hybrid_bwd(void* gi, const void* go, const void* x, int64_t n, void* stream) {
    if (bad_args(n, {gi, go, x})) return hipErrorInvalidValue;
    Streams<2, 1> s{{go, x}, {gi}};
    if (hybrid_split(n)) return launch_pairwise<HybridBwdOp<F, Poly>>(s, n, hs(stream));
    return launch_pairwise<F16MulOp<Poly>>(s, n, hs(stream));
}

// ---------------------------------------------------------------------------
// fused forward + backward, inputs (x, grad_out), outputs (y, grad_in)
// (fused_fwd_bwd_kernel, :868-896; swish: launch_swish_fused_kernel, :1428-1443)
// ---------------------------------------------------------------------------

template <int F>
struct FusedAlgOp {  // y = D3(x), gi = go * alg(y)
    static constexpr int NIN = 2, NOUT = 2;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[2], uint32_t (&b)[2]) {
        const uint32_t y = F16Prog<F, kFwd, 3>::eval(a[0]);
        b[0] = y;
        b[1] = as_u32(as_h2(a[1]) * as_h2(F16Alg<F>::eval(y)));
    }
};

struct FusedSwishOp {  // y = SWISH_FWD_D3(x), gi = go * SWISH_BWD_D4(x)
    static constexpr int NIN = 2, NOUT = 2;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[2], uint32_t (&b)[2]) {
        b[0] = F16Prog<kSwishFam, kFwd, 3>::eval(a[0]);
        b[1] = as_u32(as_h2(a[1]) * as_h2(F16Prog<kSwishFam, kBwd, 4>::eval(a[0])));
    }
};

// ---------------------------------------------------------------------------
// forward with derivative, input x, outputs (y, f'(x))
// (fwd_deriv_{alg,poly,swish}_kernel, :903-1010)
// ---------------------------------------------------------------------------

template <int F>
struct FwdDerivAlgOp {  // y = D3(x), dy = alg(y)
    static constexpr int NIN = 1, NOUT = 2;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[1], uint32_t (&b)[2]) {
        const uint32_t y = F16Prog<F, kFwd, 3>::eval(a[0]);
        b[0] = y;
        b[1] = F16Alg<F>::eval(y);
    }
};

template <int F>
struct FwdDerivPolyOp {  // y = D3(x), dy = D4 derivative program of x
    static constexpr int NIN = 1, NOUT = 2;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[1], uint32_t (&b)[2]) {
        b[0] = F16Prog<F, kFwd, 3>::eval(a[0]);
        b[1] = F16Prog<F, kBwd, 4>::eval(a[0]);
    }
};

struct FwdDerivSwishOp {  // s = SIGMOID_FWD_D3(x): y = x*s, dy = s * fma(x, 1 - s, 1)
    static constexpr int NIN = 1, NOUT = 2;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[1], uint32_t (&b)[2]) {
        const h2_t x = as_h2(a[0]);
        const h2_t s = as_h2(F16Prog<kSigmoid, kFwd, 3>::eval(a[0]));
        const h2_t one = as_h2(f16_pair_bits(1.0f));
        b[0] = as_u32(x * s);
        b[1] = as_u32(s * __builtin_elementwise_fma(x, one - s, one));
    }
};

// out = a * b (multiply_vec_kernel, :1012-1030); BF16 rounds the exact FP32
// product once.
template <bool BF>
struct MultiplyOp {
    static constexpr int NIN = 2, NOUT = 1;
    __device__ __forceinline__ static void pair(const uint32_t (&a)[2], uint32_t (&b)[1]) {
        if constexpr (BF) b[0] = pack_bf(bf_lo(a[0]) * bf_lo(a[1]), bf_hi(a[0]) * bf_hi(a[1]));
        else b[0] = as_u32(as_h2(a[0]) * as_h2(a[1]));
    }
};

template <class Op>
int run_1in2out(void* o0, void* o1, const void* in, int64_t n, void* stream) {
    if (bad_args(n, {o0, o1, in})) return hipErrorInvalidValue;
    Streams<1, 2> s{{in}, {o0, o1}};
    return launch_pairwise<Op>(s, n, hs(stream));
}

template <class Op>
int run_2in2out(void* o0, void* o1, const void* i0, const void* i1, int64_t n, void* stream) {
    if (bad_args(n, {o0, o1, i0, i1})) return hipErrorInvalidValue;
    Streams<2, 2> s{{i0, i1}, {o0, o1}};
    return launch_pairwise<Op>(s, n, hs(stream));
}

}  // namespace pt

using namespace pt;

// ---- hybrid -----------------------------------------------------------------------

extern "C" int launch_sigmoid_fwd_hybrid_kernel(void* out, const void* in, int64_t size, void* stream) {
    return run_hybrid_fwd<kSigmoid, F16Prog<kSigmoid, kFwd, 3>>(out, in, size, stream);
}
extern "C" int launch_tanh_fwd_hybrid_kernel(void* out, const void* in, int64_t size, void* stream) {
    return run_hybrid_fwd<kTanh, F16Prog<kTanh, kFwd, 3>>(out, in, size, stream);
}
extern "C" int launch_swish_fwd_hybrid_kernel(void* out, const void* in, int64_t size, void* stream) {
    return run_hybrid_fwd<kSwishFam, F16Prog<kSwishFam, kFwd, 3>>(out, in, size, stream);
}
extern "C" int launch_sigmoid_bwd_hybrid_kernel(void* gi, const void* go, const void* in, int64_t size,
                                                void* stream) {
    return run_hybrid_bwd<kSigmoid, F16Prog<kSigmoid, kBwd, 4>>(gi, go, in, size, stream);
}
extern "C" int launch_tanh_bwd_hybrid_kernel(void* gi, const void* go, const void* in, int64_t size,
                                             void* stream) {
    return run_hybrid_bwd<kTanh, F16Prog<kTanh, kBwd, 4>>(gi, go, in, size, stream);
}
extern "C" int launch_swish_bwd_hybrid_kernel(void* gi, const void* go, const void* in, int64_t size,
                                              void* stream) {
    return run_hybrid_bwd<kSwishFam, F16Prog<kSwishFam, kBwd, 4>>(gi, go, in, size, stream);
}

// ---- fused forward + backward ---------------------------------------------------------

extern "C" int launch_sigmoid_fused_kernel(void* y, void* gi, const void* x, const void* go,
                                           int64_t size, void* stream) {
    return run_2in2out<FusedAlgOp<kSigmoid>>(y, gi, x, go, size, stream);
}
extern "C" int launch_tanh_fused_kernel(void* y, void* gi, const void* x, const void* go,
                                        int64_t size, void* stream) {
    return run_2in2out<FusedAlgOp<kTanh>>(y, gi, x, go, size, stream);
}
extern "C" int launch_swish_fused_kernel(void* y, void* gi, const void* x, const void* go,
                                         int64_t size, void* stream) {
    return run_2in2out<FusedSwishOp>(y, gi, x, go, size, stream);
}

// ---- forward with derivative ------------------------------------------------------------

extern "C" int launch_sigmoid_fwd_deriv_alg_kernel(void* y, void* dy, const void* x, int64_t size,
                                                   void* stream) {
    return run_1in2out<FwdDerivAlgOp<kSigmoid>>(y, dy, x, size, stream);
}
extern "C" int launch_sigmoid_fwd_deriv_poly_kernel(void* y, void* dy, const void* x, int64_t size,
                                                    void* stream) {
    return run_1in2out<FwdDerivPolyOp<kSigmoid>>(y, dy, x, size, stream);
}
extern "C" int launch_tanh_fwd_deriv_alg_kernel(void* y, void* dy, const void* x, int64_t size,
                                                void* stream) {
    return run_1in2out<FwdDerivAlgOp<kTanh>>(y, dy, x, size, stream);
}
extern "C" int launch_tanh_fwd_deriv_poly_kernel(void* y, void* dy, const void* x, int64_t size,
                                                 void* stream) {
    return run_1in2out<FwdDerivPolyOp<kTanh>>(y, dy, x, size, stream);
}
extern "C" int launch_swish_fwd_deriv_kernel(void* y, void* dy, const void* x, int64_t size,
                                             void* stream) {
    return run_1in2out<FwdDerivSwishOp>(y, dy, x, size, stream);
}
extern "C" int launch_swish_fwd_deriv_poly_kernel(void* y, void* dy, const void* x, int64_t size,
                                                  void* stream) {
    return run_1in2out<FwdDerivPolyOp<kSwishFam>>(y, dy, x, size, stream);
}

// ---- multiply --------------------------------------------------------------------------

extern "C" int launch_multiply_kernel(void* out, const void* a, const void* b, int64_t size,
                                      void* stream) {
    return run2<MultiplyOp<false>>(out, a, b, size, stream);
}
extern "C" int launch_multiply_kernel_bf16(void* out, const void* a, const void* b, int64_t size,
                                           void* stream) {
    return run2<MultiplyOp<true>>(out, a, b, size, stream);
}
