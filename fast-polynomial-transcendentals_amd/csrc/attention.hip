// attention.hip -- score-side programs of the attention path: the deployed B3
// sigmoid-attention program (direct D3 probability + factored D4 derivative).
#include <hip/hip_runtime.h>

#include "ops.hpp"
#include "spline_ops_hip.h"

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

// One lane on a BF16 value held in FP32.  NaN follows the audit's Python
// semantics: the clamp keeps NaN, max(0, NaN) gives 0, the derivative is NaN.
template <bool WITH_GRAD>
__device__ __forceinline__ void b3_lane(float x, float& y, float& dy) {
    using C = B3Consts;
    const bool row = x >= C::split;
    const float xc = __builtin_elementwise_minimum(
        __builtin_elementwise_maximum(x, -C::clamp), C::clamp);
    float f = bfma(xc, row ? C::r1[3] : C::r0[3], row ? C::r1[2] : C::r0[2]);
    f = bfma(xc, f, row ? C::r1[1] : C::r0[1]);
    f = bfma(xc, f, row ? C::r1[0] : C::r0[0]);
    y = f > 0.0f ? f : 0.0f;
    if constexpr (WITH_GRAD) {
        const float fac = bfma(xc, row ? C::g1[1] : C::g0[1], row ? C::g1[0] : C::g0[0]);
        dy = y * fac;  // rounded once by the final pack
    }
}

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
        b3_lane<false>(bf_lo(a[0]), y0, d);
        b3_lane<false>(bf_hi(a[0]), y1, d);
        b[0] = pack_exact_bf(y0, y1);
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

