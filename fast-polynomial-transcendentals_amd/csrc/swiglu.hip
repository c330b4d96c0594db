// swiglu.hip -- SwiGLU activation kernels: separate gate/up tensors (B4
// routed experts) and the packed [rows, 2H] = [gate | up] layout that a fused
// gate+up projection produces (B1 dense MLP), forward and backward.
#include <hip/hip_runtime.h>

#include "ops.hpp"
#include "spline_ops_hip.h"

namespace pt {

// Unsigned division by a launch-constant divisor d for numerators below
// 2^31 (Granlund & Montgomery, "Division by invariant integers using
// multiplication", 1994, Fig. 4.1 with the add that cannot overflow here).
struct FastDiv {
    uint32_t m;
    uint32_t l;
};

inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    const uint64_t m = ((((uint64_t)1 << 32) * (((uint64_t)1 << l) - d)) / d) + 1;
    return FastDiv{(uint32_t)m, l};
}

__device__ __forceinline__ uint32_t fast_div(uint32_t n, FastDiv f) {
    return (__umulhi(n, f.m) + n) >> f.l;
}

// Packed forward: vector v of the output row-major [rows, H] maps to
// gate vector r*2*hv + c and up vector r*2*hv + hv + c (hv = H/8 vectors).
template <class Op, bool LNT, bool SNT>
__global__ void __launch_bounds__(kBlock)
packed_fwd_kernel(const void* __restrict__ packed, void* __restrict__ out, uint32_t n_vec,
                  uint32_t hv, FastDiv div_hv) {
    static_assert(Op::NIN == 2 && Op::NOUT == 1, "packed forward op shape");
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t v = blockIdx.x * kBlock + threadIdx.x; v < n_vec; v += stride) {
        const uint32_t r = fast_div(v, div_hv);
        const int64_t g = (int64_t)r * hv + v;  // = r*2*hv + c
        const Vec4 gate = ld16<LNT>(packed, g);
        const Vec4 up = ld16<LNT>(packed, g + hv);
        Vec4 o;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t a[2] = {gate.w[w], up.w[w]}, b[1];
            Op::pair(a, b);
            o.w[w] = b[0];
        }
        st16<SNT>(out, v, o);
    }
}

// Packed backward: grad_out is [rows, H]; grad_packed mirrors packed.
template <class Op, bool LNT, bool SNT>
__global__ void __launch_bounds__(kBlock)
packed_bwd_kernel(const void* __restrict__ grad_out, const void* __restrict__ packed,
                  void* __restrict__ grad_packed, uint32_t n_vec, uint32_t hv, FastDiv div_hv) {
    static_assert(Op::NIN == 3 && Op::NOUT == 2, "packed backward op shape");
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t v = blockIdx.x * kBlock + threadIdx.x; v < n_vec; v += stride) {
        const uint32_t r = fast_div(v, div_hv);
        const int64_t g = (int64_t)r * hv + v;
        const Vec4 go = ld16<LNT>(grad_out, v);
        const Vec4 gate = ld16<LNT>(packed, g);
        const Vec4 up = ld16<LNT>(packed, g + hv);
        Vec4 gg, gu;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t a[3] = {go.w[w], gate.w[w], up.w[w]}, b[2];
            Op::pair(a, b);
            gg.w[w] = b[0];
            gu.w[w] = b[1];
        }
        st16<SNT>(grad_packed, g, gg);
        st16<SNT>(grad_packed, g + hv, gu);
    }
}

// Element path (H not a multiple of 8, unaligned storage or > 2^31 vectors).
template <class Op, bool BWD>
__global__ void __launch_bounds__(kBlock)
packed_element_kernel(const void* __restrict__ grad_out, const void* __restrict__ packed,
                      void* __restrict__ out, int64_t rows, int64_t h) {
    const int64_t n = rows * h;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const uint16_t* p = reinterpret_cast<const uint16_t*>(packed);
    for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < n; e += stride) {
        const int64_t r = e / h;
        const int64_t c = e - r * h;
        const int64_t g = r * 2 * h + c;
        const uint32_t gate = p[g], up = p[g + h];
        if constexpr (!BWD) {
            uint32_t a[2] = {gate | (gate << 16), up | (up << 16)}, b[1];
            Op::pair(a, b);
            reinterpret_cast<uint16_t*>(out)[e] = (uint16_t)(b[0] & 0xffffu);
        } else {
            const uint32_t go = reinterpret_cast<const uint16_t*>(grad_out)[e];
            uint32_t a[3] = {go | (go << 16), gate | (gate << 16), up | (up << 16)}, b[2];
            Op::pair(a, b);
            reinterpret_cast<uint16_t*>(out)[g] = (uint16_t)(b[0] & 0xffffu);
            reinterpret_cast<uint16_t*>(out)[g + h] = (uint16_t)(b[1] & 0xffffu);
        }
    }
}

template <class Op, bool BWD>
int launch_packed(void* out, const void* grad_out, const void* packed, int64_t rows, int64_t h,
                  void* stream) {
    if (rows < 0 || h < 0) return hipErrorInvalidValue;
    const int64_t n = rows * h;
    if (n == 0) return hipSuccess;
    if (!out || !packed || (BWD && !grad_out)) return hipErrorInvalidValue;
    const int64_t n_vec = n / 8;
    const bool vec = (h % 8 == 0) && aligned16(out) && aligned16(packed) &&
                     (!BWD || aligned16(grad_out)) && n_vec < (int64_t(1) << 31);
    if (!vec) {
        const int64_t grid = grid_one_pass(n);
        hipLaunchKernelGGL((packed_element_kernel<Op, BWD>), dim3((unsigned)grid), dim3(kBlock), 0,
                           hs(stream), grad_out, packed, out, rows, h);
        return hipGetLastError();
    }
    const uint32_t hv = (uint32_t)(h / 8);
    const FastDiv div = make_fastdiv(hv);
    const int64_t grid = grid_one_pass(n_vec);
    // bytes: forward reads gate+up (4n) and writes 2n; backward reads
    // grad_out+gate+up (6n) and writes 4n.
    const int mode = BWD ? nt_mode(6 * n, 4 * n) : nt_mode(4 * n, 2 * n);
#define PT_PACKED_LAUNCH(LNT, SNT)                                                              \
    if constexpr (BWD)                                                                         \
        hipLaunchKernelGGL((packed_bwd_kernel<Op, LNT, SNT>), dim3((unsigned)grid), dim3(kBlock), \
                           0, hs(stream), grad_out, packed, out, (uint32_t)n_vec, hv, div);     \
    else                                                                                       \
        hipLaunchKernelGGL((packed_fwd_kernel<Op, LNT, SNT>), dim3((unsigned)grid), dim3(kBlock), \
                           0, hs(stream), packed, out, (uint32_t)n_vec, hv, div);
    if (mode == kNtBoth) {
        PT_PACKED_LAUNCH(true, true)
    } else if (mode == kNtStore) {
        PT_PACKED_LAUNCH(false, true)
    } else {
        PT_PACKED_LAUNCH(false, false)
    }
#undef PT_PACKED_LAUNCH
    return hipGetLastError();
}

}  // namespace pt

using namespace pt;

// ---- separate gate / up tensors ------------------------------------------

#define PT_SWISH_MUL(name, OP)                                                     \
    extern "C" int name(void* out, const void* gate, const void* up, int64_t size, \
                        void* stream) {                                            \
        return run2<PT_STRIP OP>(out, gate, up, size, stream);                     \
    }

#define PT_F16_SM(G) (F16SwishMulOp<F16Prog<kSwishFam, kFwd, G>>)
#define PT_BF16_SM(G) (BF16SwishMulOp<BF16Prog<kSwishFam, kFwd, G>>)
#define PT_F16_SM_NATIVE (F16SwishMulOp<F16Native<kSwishFam, kFwd>>)
#define PT_BF16_SM_NATIVE (BF16SwishMulOp<BF16Native<kSwishFam, kFwd>>)

PT_SWISH_MUL(launch_swish_mul_fwd_native_kernel, PT_F16_SM_NATIVE)
PT_SWISH_MUL(launch_swish_mul_fwd_d3_kernel, PT_F16_SM(3))
PT_SWISH_MUL(launch_swish_mul_fwd_d4_kernel, PT_F16_SM(4))
PT_SWISH_MUL(launch_swish_mul_fwd_d5_kernel, PT_F16_SM(5))
PT_SWISH_MUL(launch_swish_mul_fwd_d6_kernel, PT_F16_SM(6))
PT_SWISH_MUL(launch_swish_mul_fwd_native_kernel_bf16, PT_BF16_SM_NATIVE)
PT_SWISH_MUL(launch_swish_mul_fwd_d3_kernel_bf16, PT_BF16_SM(3))
PT_SWISH_MUL(launch_swish_mul_fwd_d4_kernel_bf16, PT_BF16_SM(4))
PT_SWISH_MUL(launch_swish_mul_fwd_d5_kernel_bf16, PT_BF16_SM(5))
PT_SWISH_MUL(launch_swish_mul_fwd_d6_kernel_bf16, PT_BF16_SM(6))

// BF16 Sollya coefficient set (spline_kernels_bf16.cu:1174-1199)
#define PT_BF16_SM_S(G) (BF16SwishMulOp<BF16Prog<kSwishFam, kFwd, G, kSollya>>)
PT_SWISH_MUL(launch_swish_mul_fwd_d3_kernel_bf16_sollya, PT_BF16_SM_S(3))
PT_SWISH_MUL(launch_swish_mul_fwd_d4_kernel_bf16_sollya, PT_BF16_SM_S(4))
PT_SWISH_MUL(launch_swish_mul_fwd_d5_kernel_bf16_sollya, PT_BF16_SM_S(5))
PT_SWISH_MUL(launch_swish_mul_fwd_d6_kernel_bf16_sollya, PT_BF16_SM_S(6))

#define PT_SWISH_MUL_BWD(name, OP)                                                          \
    extern "C" int name(void* grad_gate, void* grad_up, const void* grad_out,               \
                        const void* gate, const void* up, int64_t size, void* stream) {     \
        return run_bwd3<PT_STRIP OP>(grad_gate, grad_up, grad_out, gate, up, size, stream); \
    }

#define PT_F16_SMB(G) (F16SwishMulBwdOp<F16Prog<kSwishFam, kFwd, G>, F16Prog<kSwishFam, kBwd, G>>)
#define PT_BF16_SMB(G) \
    (BF16SwishMulBwdOp<BF16Prog<kSwishFam, kFwd, G>, BF16Prog<kSwishFam, kBwd, G>>)

PT_SWISH_MUL_BWD(launch_swish_mul_bwd_native_kernel, (NativeSwishMulBwdOp<false>))
PT_SWISH_MUL_BWD(launch_swish_mul_bwd_d3_kernel, PT_F16_SMB(3))
PT_SWISH_MUL_BWD(launch_swish_mul_bwd_d4_kernel, PT_F16_SMB(4))
PT_SWISH_MUL_BWD(launch_swish_mul_bwd_d5_kernel, PT_F16_SMB(5))
PT_SWISH_MUL_BWD(launch_swish_mul_bwd_d6_kernel, PT_F16_SMB(6))
PT_SWISH_MUL_BWD(launch_swish_mul_bwd_native_kernel_bf16, (NativeSwishMulBwdOp<true>))
PT_SWISH_MUL_BWD(launch_swish_mul_bwd_d3_kernel_bf16, (BF16SwishMulBwdD3AlgOp))
PT_SWISH_MUL_BWD(launch_swish_mul_bwd_d4_kernel_bf16, PT_BF16_SMB(4))
PT_SWISH_MUL_BWD(launch_swish_mul_bwd_d5_kernel_bf16, PT_BF16_SMB(5))
PT_SWISH_MUL_BWD(launch_swish_mul_bwd_d6_kernel_bf16, PT_BF16_SMB(6))

// Sollya: the generic forward/backward program pair at every degree,
// D3 included (spline_kernels_bf16.cu:1187-1198).
#define PT_BF16_SMB_S(G)                                            \
    (BF16SwishMulBwdOp<BF16Prog<kSwishFam, kFwd, G, kSollya>,       \
                       BF16Prog<kSwishFam, kBwd, G, kSollya>>)
PT_SWISH_MUL_BWD(launch_swish_mul_bwd_d3_kernel_bf16_sollya, PT_BF16_SMB_S(3))
PT_SWISH_MUL_BWD(launch_swish_mul_bwd_d4_kernel_bf16_sollya, PT_BF16_SMB_S(4))
PT_SWISH_MUL_BWD(launch_swish_mul_bwd_d5_kernel_bf16_sollya, PT_BF16_SMB_S(5))
PT_SWISH_MUL_BWD(launch_swish_mul_bwd_d6_kernel_bf16_sollya, PT_BF16_SMB_S(6))

// ---- packed [rows, 2H] layout ---------------------------------------------

#define PT_PACKED_FWD(name, OP)                                                            \
    extern "C" int name(void* out, const void* packed, int64_t rows, int64_t hidden_size,  \
                        void* stream) {                                                    \
        return launch_packed<PT_STRIP OP, false>(out, nullptr, packed, rows, hidden_size,  \
                                                 stream);                                  \
    }

PT_PACKED_FWD(launch_swish_mul_packed_fwd_native_kernel, PT_F16_SM_NATIVE)
PT_PACKED_FWD(launch_swish_mul_packed_fwd_d3_kernel, PT_F16_SM(3))
PT_PACKED_FWD(launch_swish_mul_packed_fwd_d4_kernel, PT_F16_SM(4))
PT_PACKED_FWD(launch_swish_mul_packed_fwd_d5_kernel, PT_F16_SM(5))
PT_PACKED_FWD(launch_swish_mul_packed_fwd_d6_kernel, PT_F16_SM(6))
PT_PACKED_FWD(launch_swish_mul_packed_fwd_native_kernel_bf16, PT_BF16_SM_NATIVE)
PT_PACKED_FWD(launch_swish_mul_packed_fwd_d3_kernel_bf16, PT_BF16_SM(3))
PT_PACKED_FWD(launch_swish_mul_packed_fwd_d4_kernel_bf16, PT_BF16_SM(4))
PT_PACKED_FWD(launch_swish_mul_packed_fwd_d5_kernel_bf16, PT_BF16_SM(5))
PT_PACKED_FWD(launch_swish_mul_packed_fwd_d6_kernel_bf16, PT_BF16_SM(6))
PT_PACKED_FWD(launch_swish_mul_packed_fwd_d3_kernel_bf16_sollya, PT_BF16_SM_S(3))
PT_PACKED_FWD(launch_swish_mul_packed_fwd_d4_kernel_bf16_sollya, PT_BF16_SM_S(4))
PT_PACKED_FWD(launch_swish_mul_packed_fwd_d5_kernel_bf16_sollya, PT_BF16_SM_S(5))
PT_PACKED_FWD(launch_swish_mul_packed_fwd_d6_kernel_bf16_sollya, PT_BF16_SM_S(6))

#define PT_PACKED_BWD(name, OP)                                                               \
    extern "C" int name(void* grad_packed, const void* grad_out, const void* packed,          \
                        int64_t rows, int64_t hidden_size, void* stream) {                    \
        return launch_packed<PT_STRIP OP, true>(grad_packed, grad_out, packed, rows,          \
                                                hidden_size, stream);                         \
    }

PT_PACKED_BWD(launch_swish_mul_packed_bwd_native_kernel, (PackedNativeSwishMulBwdOp<false>))
PT_PACKED_BWD(launch_swish_mul_packed_bwd_d3_kernel, PT_F16_SMB(3))
PT_PACKED_BWD(launch_swish_mul_packed_bwd_d4_kernel, PT_F16_SMB(4))
PT_PACKED_BWD(launch_swish_mul_packed_bwd_d5_kernel, PT_F16_SMB(5))
PT_PACKED_BWD(launch_swish_mul_packed_bwd_d6_kernel, PT_F16_SMB(6))
PT_PACKED_BWD(launch_swish_mul_packed_bwd_native_kernel_bf16, (PackedNativeSwishMulBwdOp<true>))
PT_PACKED_BWD(launch_swish_mul_packed_bwd_d3_kernel_bf16, (BF16SwishMulBwdD3AlgOp))
PT_PACKED_BWD(launch_swish_mul_packed_bwd_d4_kernel_bf16, PT_BF16_SMB(4))
PT_PACKED_BWD(launch_swish_mul_packed_bwd_d5_kernel_bf16, PT_BF16_SMB(5))
PT_PACKED_BWD(launch_swish_mul_packed_bwd_d6_kernel_bf16, PT_BF16_SMB(6))
PT_PACKED_BWD(launch_swish_mul_packed_bwd_d3_kernel_bf16_sollya, PT_BF16_SMB_S(3))
PT_PACKED_BWD(launch_swish_mul_packed_bwd_d4_kernel_bf16_sollya, PT_BF16_SMB_S(4))
PT_PACKED_BWD(launch_swish_mul_packed_bwd_d5_kernel_bf16_sollya, PT_BF16_SMB_S(5))
PT_PACKED_BWD(launch_swish_mul_packed_bwd_d6_kernel_bf16_sollya, PT_BF16_SMB_S(6))
