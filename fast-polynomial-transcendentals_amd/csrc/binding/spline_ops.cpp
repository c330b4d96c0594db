// spline_ops.cpp -- PyTorch-ROCm binding of the MI355X polynomial kernels.
//
// Mirrors the reference extension's Python surface
// (autonumerics_zero/spline_ops/spline_ops.cpp:2212-2452): the pybind
// functions keep their names, argument order, defaults and error messages,
// and TORCH_LIBRARY(spline_ops) registers the same schemas with the same
// AutogradCUDA / CUDA split (on ROCm the HIP device uses the CUDA dispatch
// keys).  All compute goes through the C ABI of libspline_hip.so
// (include/spline_ops_hip.h); nothing here computes on the host.
#include <torch/extension.h>
#include <torch/library.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>

#include <cstdlib>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "spline_ops_hip.h"

namespace {

// ---------------------------------------------------------------------------
// checks (spline_ops.cpp:293-323)
// ---------------------------------------------------------------------------

#define CHECK_CUDA(x) TORCH_CHECK(x.is_cuda(), #x " must be a CUDA tensor")
#define CHECK_CONTIGUOUS(x) TORCH_CHECK(x.is_contiguous(), #x " must be contiguous")
#define CHECK_HALF_OR_BF16(x)                                              \
    TORCH_CHECK(x.scalar_type() == at::kHalf || x.scalar_type() == at::kBFloat16, \
                #x " must be float16 or bfloat16")
#define CHECK_INPUT(x) \
    CHECK_CUDA(x);     \
    CHECK_CONTIGUOUS(x); \
    CHECK_HALF_OR_BF16(x)

bool spline_env_flag(const char* name) {
    const char* v = std::getenv(name);
    if (v == nullptr || v[0] == '\0') return false;
    for (const char* on : {"1", "true", "TRUE", "yes", "YES", "on", "ON"})
        if (std::strcmp(v, on) == 0) return true;
    return false;
}

void* current_stream(const at::Tensor& t) {
    return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

// Launch-status check; with SPLINE_OPS_SYNC_DEBUG set, also synchronise the
// stream unless it is being captured into a graph.
void check_launch(int rc, void* stream) {
    TORCH_CHECK(rc == 0, "spline_ops HIP launch failed: ",
                hipGetErrorString(static_cast<hipError_t>(rc)));
    if (spline_env_flag("SPLINE_OPS_SYNC_DEBUG")) {
        auto s = reinterpret_cast<hipStream_t>(stream);
        hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
        TORCH_CHECK(hipStreamIsCapturing(s, &status) == hipSuccess, "hipStreamIsCapturing failed");
        if (status == hipStreamCaptureStatusNone) {
            const hipError_t err = hipStreamSynchronize(s);
            TORCH_CHECK(err == hipSuccess, "spline_ops kernel failed: ", hipGetErrorString(err));
        }
    }
}

// ---------------------------------------------------------------------------
// launcher tables
// ---------------------------------------------------------------------------

using Unary = int (*)(void*, const void*, int64_t, void*);
using Binary = int (*)(void*, const void*, const void*, int64_t, void*);
using SwishMulBwd = int (*)(void*, void*, const void*, const void*, const void*, int64_t, void*);
using PackedFwd = int (*)(void*, const void*, int64_t, int64_t, void*);
using PackedBwd = int (*)(void*, const void*, const void*, int64_t, int64_t, void*);

enum Fam { SIGMOID = 0, TANH = 1, SWISH = 2, GELU = 3 };
const char* kFamName[] = {"sigmoid", "tanh", "swish", "GeLU"};

// Columns of every table: 0 = FP16, 1 = BF16 (coeff_source current),
// 2 = BF16 Sollya coefficient set.  Rows: degree, 0 = native.
#define PT_POLY(n, sfx)                                                        \
    nullptr, nullptr, launch_##n##_d3_kernel##sfx, launch_##n##_d4_kernel##sfx, \
        launch_##n##_d5_kernel##sfx, launch_##n##_d6_kernel##sfx
#define PT_ROW(n, sfx) {nullptr, PT_POLY(n, sfx)}
#define PT_ROW_NATIVE(n, sfx) {launch_##n##_native_kernel##sfx, PT_POLY(n, sfx)}
#define PT_NONE {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr}

// [family][column][degree]
Unary kFwd[4][3][7] = {
    {PT_ROW_NATIVE(sigmoid_fwd, ), PT_ROW_NATIVE(sigmoid_fwd, _bf16), PT_ROW(sigmoid_fwd, _bf16_sollya)},
    {PT_ROW_NATIVE(tanh_fwd, ), PT_ROW_NATIVE(tanh_fwd, _bf16), PT_NONE},
    {PT_ROW_NATIVE(swish_fwd, ), PT_ROW_NATIVE(swish_fwd, _bf16), PT_ROW(swish_fwd, _bf16_sollya)},
    {PT_ROW(gelu_fwd, ), PT_ROW(gelu_fwd, _bf16), PT_ROW(gelu_fwd, _bf16_sollya)},
};

Binary kBwd[4][3][7] = {
    {PT_ROW(sigmoid_bwd, ), PT_ROW(sigmoid_bwd, _bf16), PT_ROW(sigmoid_bwd, _bf16_sollya)},
    {PT_ROW(tanh_bwd, ), PT_ROW(tanh_bwd, _bf16), PT_NONE},
    {PT_ROW_NATIVE(swish_bwd, ), PT_ROW_NATIVE(swish_bwd, _bf16), PT_ROW(swish_bwd, _bf16_sollya)},
    {PT_ROW(gelu_bwd, ), PT_ROW(gelu_bwd, _bf16), PT_ROW(gelu_bwd, _bf16_sollya)},
};

Binary kSwishMul[3][7] = {PT_ROW_NATIVE(swish_mul_fwd, ), PT_ROW_NATIVE(swish_mul_fwd, _bf16),
                          PT_ROW(swish_mul_fwd, _bf16_sollya)};
SwishMulBwd kSwishMulBwd[3][7] = {PT_ROW_NATIVE(swish_mul_bwd, ),
                                  PT_ROW_NATIVE(swish_mul_bwd, _bf16),
                                  PT_ROW(swish_mul_bwd, _bf16_sollya)};
PackedFwd kPackedFwd[3][7] = {PT_ROW_NATIVE(swish_mul_packed_fwd, ),
                              PT_ROW_NATIVE(swish_mul_packed_fwd, _bf16),
                              PT_ROW(swish_mul_packed_fwd, _bf16_sollya)};
PackedBwd kPackedBwd[3][7] = {PT_ROW_NATIVE(swish_mul_packed_bwd, ),
                              PT_ROW_NATIVE(swish_mul_packed_bwd, _bf16),
                              PT_ROW(swish_mul_packed_bwd, _bf16_sollya)};
#undef PT_POLY
#undef PT_ROW
#undef PT_ROW_NATIVE
#undef PT_NONE

// spline_ops.cpp:1179-1185
int normalize_coeff_source_id(int64_t coeff_source_id) {
    TORCH_CHECK(coeff_source_id == 0 || coeff_source_id == 1,
                "coeff_source_id must be 0 (current) or 1 (sollya)");
    return static_cast<int>(coeff_source_id);
}

// Resolution rules of resolve_*_launcher (spline_ops.cpp:1187-1502): FP16
// accepts only the current coefficient source; BF16 takes the current or the
// Sollya set; degree 0 (native) exists for the SiLU family's current set only.
template <class T>
T resolve(T (&table)[3][7], at::ScalarType dtype, int64_t degree, int coeff_source,
          const char* what, bool allow_native) {
    const bool bf = dtype == at::kBFloat16;
    if (!bf) {
        TORCH_CHECK(coeff_source == 0, "FP16 spline kernels only support coeff_source=current");
    }
    const int col = bf ? 1 + coeff_source : 0;
    bool any = false;
    for (T fn : table[col]) any = any || fn != nullptr;
    TORCH_CHECK(any, "coeff_source=sollya has no ", what, " programs");
    const bool ok = (degree >= 3 && degree <= 6) || (degree == 0 && allow_native);
    TORCH_CHECK(ok && table[col][degree] != nullptr, "Unsupported ", what, " degree: ", degree);
    return table[col][degree];
}

at::ScalarType check_same(const at::Tensor& a, const at::Tensor& b, const char* msg_dtype,
                          const char* msg_numel) {
    TORCH_CHECK(a.scalar_type() == b.scalar_type(), msg_dtype);
    TORCH_CHECK(a.numel() == b.numel(), msg_numel);
    return a.scalar_type();
}

// ---------------------------------------------------------------------------
// unary / binary entry points
// ---------------------------------------------------------------------------

at::Tensor run_unary(const at::Tensor& x, Unary fn) {
    c10::OptionalDeviceGuard guard(x.device());
    at::Tensor out = at::empty_like(x);
    void* s = current_stream(x);
    check_launch(fn(out.data_ptr(), x.data_ptr(), x.numel(), s), s);
    return out;
}

at::Tensor run_binary(const at::Tensor& go, const at::Tensor& x, Binary fn) {
    c10::OptionalDeviceGuard guard(x.device());
    at::Tensor gi = at::empty_like(x);
    void* s = current_stream(x);
    check_launch(fn(gi.data_ptr(), go.data_ptr(), x.data_ptr(), x.numel(), s), s);
    return gi;
}

at::Tensor fwd_fixed(at::Tensor x, int fam, int degree) {
    CHECK_INPUT(x);
    return run_unary(x, kFwd[fam][x.scalar_type() == at::kBFloat16][degree]);
}

at::Tensor bwd_fixed(at::Tensor grad_out, at::Tensor x, int fam, int degree) {
    CHECK_INPUT(grad_out);
    CHECK_INPUT(x);
    check_same(grad_out, x, "grad_out and x must have the same dtype",
               "grad_out and x must have the same number of elements");
    return run_binary(grad_out, x, kBwd[fam][x.scalar_type() == at::kBFloat16][degree]);
}

at::Tensor fwd_variant(at::Tensor x, int64_t degree, int64_t coeff_source_id, int fam) {
    CHECK_INPUT(x);
    std::string what = std::string(kFamName[fam]) + " forward";
    Unary fn = resolve(kFwd[fam], x.scalar_type(), degree,
                       normalize_coeff_source_id(coeff_source_id), what.c_str(), fam == SWISH);
    return run_unary(x, fn);
}

at::Tensor bwd_variant(at::Tensor grad_out, at::Tensor x, int64_t degree, int64_t coeff_source_id,
                       int fam) {
    CHECK_INPUT(grad_out);
    CHECK_INPUT(x);
    check_same(grad_out, x, "grad_out and x must have the same dtype",
               "grad_out and x must have the same number of elements");
    std::string what = std::string(kFamName[fam]) + " backward";
    Binary fn = resolve(kBwd[fam], x.scalar_type(), degree,
                        normalize_coeff_source_id(coeff_source_id), what.c_str(), fam == SWISH);
    return run_binary(grad_out, x, fn);
}

at::Tensor bwd_alg(at::Tensor grad_out, at::Tensor y, int fam) {
    CHECK_INPUT(grad_out);
    CHECK_INPUT(y);
    check_same(grad_out, y, "grad_out and y must have the same dtype",
               "grad_out and y must have the same number of elements");
    const bool bf = y.scalar_type() == at::kBFloat16;
    Binary fn = fam == SIGMOID ? (bf ? launch_sigmoid_bwd_alg_kernel_bf16 : launch_sigmoid_bwd_alg_kernel)
                               : (bf ? launch_tanh_bwd_alg_kernel_bf16 : launch_tanh_bwd_alg_kernel);
    return run_binary(grad_out, y, fn);
}

// ---------------------------------------------------------------------------
// SwiGLU entry points (spline_ops.cpp:1645-1828)
// ---------------------------------------------------------------------------

at::Tensor swish_mul_fwd_variant(at::Tensor gate, at::Tensor up, int64_t degree,
                                 int64_t coeff_source_id) {
    CHECK_INPUT(gate);
    CHECK_INPUT(up);
    TORCH_CHECK(gate.scalar_type() == up.scalar_type(), "gate and up must have the same dtype");
    TORCH_CHECK(gate.numel() == up.numel(), "gate and up must have the same number of elements");
    Binary fn = resolve(kSwishMul, gate.scalar_type(), degree,
                        normalize_coeff_source_id(coeff_source_id), "swish_mul forward", true);
    c10::OptionalDeviceGuard guard(gate.device());
    at::Tensor out = at::empty_like(up);
    void* s = current_stream(gate);
    check_launch(fn(out.data_ptr(), gate.data_ptr(), up.data_ptr(), gate.numel(), s), s);
    return out;
}

std::vector<at::Tensor> swish_mul_bwd_variant(at::Tensor grad_out, at::Tensor gate, at::Tensor up,
                                              int64_t degree, int64_t coeff_source_id) {
    CHECK_INPUT(grad_out);
    CHECK_INPUT(gate);
    CHECK_INPUT(up);
    TORCH_CHECK(gate.scalar_type() == up.scalar_type(), "gate and up must have the same dtype");
    TORCH_CHECK(grad_out.scalar_type() == gate.scalar_type(),
                "grad_out and gate must have the same dtype");
    TORCH_CHECK(gate.numel() == up.numel(), "gate and up must have the same number of elements");
    TORCH_CHECK(grad_out.numel() == gate.numel(),
                "grad_out and gate must have the same number of elements");
    SwishMulBwd fn = resolve(kSwishMulBwd, gate.scalar_type(), degree,
                             normalize_coeff_source_id(coeff_source_id), "swish_mul backward", true);
    c10::OptionalDeviceGuard guard(gate.device());
    at::Tensor grad_gate = at::empty_like(gate);
    at::Tensor grad_up = at::empty_like(up);
    void* s = current_stream(gate);
    check_launch(fn(grad_gate.data_ptr(), grad_up.data_ptr(), grad_out.data_ptr(), gate.data_ptr(),
                    up.data_ptr(), gate.numel(), s),
                 s);
    return {grad_gate, grad_up};
}

at::Tensor swish_mul_packed_fwd_variant(at::Tensor packed, int64_t degree,
                                        int64_t coeff_source_id) {
    CHECK_INPUT(packed);
    TORCH_CHECK(packed.dim() >= 1, "packed gate/up tensor must have at least one dimension");
    const int64_t packed_hidden_size = packed.size(-1);
    TORCH_CHECK((packed_hidden_size % 2) == 0, "packed gate/up last dimension must be even");
    const int64_t hidden_size = packed_hidden_size / 2;
    TORCH_CHECK((hidden_size % 2) == 0, "packed SwiGLU hidden size must be even");
    std::vector<int64_t> out_sizes(packed.sizes().begin(), packed.sizes().end());
    out_sizes.back() = hidden_size;
    c10::OptionalDeviceGuard guard(packed.device());
    at::Tensor out = at::empty(out_sizes, packed.options());
    if (packed.numel() == 0) return out;
    const int64_t rows = packed.numel() / packed_hidden_size;
    PackedFwd fn = resolve(kPackedFwd, packed.scalar_type(), degree,
                           normalize_coeff_source_id(coeff_source_id), "swish_mul_packed forward",
                           true);
    void* s = current_stream(packed);
    check_launch(fn(out.data_ptr(), packed.data_ptr(), rows, hidden_size, s), s);
    return out;
}

at::Tensor swish_mul_packed_bwd_variant(at::Tensor grad_out, at::Tensor packed, int64_t degree,
                                        int64_t coeff_source_id) {
    CHECK_INPUT(grad_out);
    CHECK_INPUT(packed);
    TORCH_CHECK(packed.dim() >= 1, "packed gate/up tensor must have at least one dimension");
    TORCH_CHECK(grad_out.dim() == packed.dim(), "grad_out and packed must have the same rank");
    TORCH_CHECK(grad_out.scalar_type() == packed.scalar_type(),
                "grad_out and packed must have the same dtype");
    const int64_t packed_hidden_size = packed.size(-1);
    TORCH_CHECK((packed_hidden_size % 2) == 0, "packed gate/up last dimension must be even");
    const int64_t hidden_size = packed_hidden_size / 2;
    TORCH_CHECK((hidden_size % 2) == 0, "packed SwiGLU hidden size must be even");
    TORCH_CHECK(grad_out.size(-1) == hidden_size,
                "grad_out last dimension must be half the packed last dimension");
    for (int64_t d = 0; d + 1 < packed.dim(); ++d)
        TORCH_CHECK(grad_out.size(d) == packed.size(d),
                    "grad_out and packed leading dimensions must match");
    c10::OptionalDeviceGuard guard(packed.device());
    at::Tensor grad_packed = at::empty_like(packed);
    if (packed.numel() == 0) return grad_packed;
    const int64_t rows = packed.numel() / packed_hidden_size;
    PackedBwd fn = resolve(kPackedBwd, packed.scalar_type(), degree,
                           normalize_coeff_source_id(coeff_source_id), "swish_mul_packed backward",
                           true);
    void* s = current_stream(packed);
    check_launch(fn(grad_packed.data_ptr(), grad_out.data_ptr(), packed.data_ptr(), rows,
                    hidden_size, s),
                 s);
    return grad_packed;
}

// ---------------------------------------------------------------------------
// B3 deployed direct-D3 / factored-D4 program
// ---------------------------------------------------------------------------

std::vector<at::Tensor> flash_sigmoid_direct_d3_d4(at::Tensor scores) {
    CHECK_CUDA(scores);
    CHECK_CONTIGUOUS(scores);
    TORCH_CHECK(scores.scalar_type() == at::kBFloat16 || scores.scalar_type() == at::kFloat,
                "scores must be bfloat16 or float32");
    c10::OptionalDeviceGuard guard(scores.device());
    auto opts = scores.options().dtype(at::kBFloat16);
    at::Tensor y = at::empty(scores.sizes(), opts);
    at::Tensor dy = at::empty(scores.sizes(), opts);
    void* s = current_stream(scores);
    const int rc = scores.scalar_type() == at::kBFloat16
                       ? launch_flash_sigmoid_direct_d3_d4_bf16(y.data_ptr(), dy.data_ptr(),
                                                                scores.data_ptr(), scores.numel(), s)
                       : launch_flash_sigmoid_direct_d3_d4_f32_bf16(
                             y.data_ptr(), dy.data_ptr(), scores.data_ptr(), scores.numel(), s);
    check_launch(rc, s);
    return {y, dy};
}

using B3PairLauncher = int (*)(void*, void*, const void*, int64_t, void*);

std::vector<at::Tensor> flash_sigmoid_pair(at::Tensor scores, B3PairLauncher fn) {
    CHECK_CUDA(scores);
    CHECK_CONTIGUOUS(scores);
    TORCH_CHECK(scores.scalar_type() == at::kBFloat16, "scores must be bfloat16");
    c10::OptionalDeviceGuard guard(scores.device());
    at::Tensor y = at::empty_like(scores);
    at::Tensor dy = at::empty_like(scores);
    void* s = current_stream(scores);
    check_launch(fn(y.data_ptr(), dy.data_ptr(), scores.data_ptr(), scores.numel(), s), s);
    return {y, dy};
}

std::vector<at::Tensor> flash_sigmoid_exp2_d2(at::Tensor scores) {
    return flash_sigmoid_pair(scores, launch_flash_sigmoid_exp2_d2_bf16);
}

std::vector<at::Tensor> flash_sigmoid_native(at::Tensor scores) {
    return flash_sigmoid_pair(scores, launch_flash_sigmoid_native_bf16);
}

at::Tensor flash_sigmoid_direct_d3(at::Tensor scores) {
    CHECK_CUDA(scores);
    CHECK_CONTIGUOUS(scores);
    TORCH_CHECK(scores.scalar_type() == at::kBFloat16, "scores must be bfloat16");
    c10::OptionalDeviceGuard guard(scores.device());
    at::Tensor y = at::empty_like(scores);
    void* s = current_stream(scores);
    check_launch(launch_flash_sigmoid_direct_d3_bf16(y.data_ptr(), scores.data_ptr(), scores.numel(), s),
                 s);
    return y;
}

// ---------------------------------------------------------------------------
// B2 softcap and B5 exp2
// ---------------------------------------------------------------------------

using SoftcapLauncher = int (*)(void*, const void*, int64_t, float, void*);

at::Tensor softcap_fwd(at::Tensor scores, double cap, SoftcapLauncher fn) {
    CHECK_CUDA(scores);
    CHECK_CONTIGUOUS(scores);
    TORCH_CHECK(scores.scalar_type() == at::kBFloat16, "scores must be bfloat16");
    TORCH_CHECK(cap > 0.0, "cap must be positive");
    c10::OptionalDeviceGuard guard(scores.device());
    at::Tensor out = at::empty_like(scores);
    void* s = current_stream(scores);
    check_launch(fn(out.data_ptr(), scores.data_ptr(), scores.numel(), static_cast<float>(cap), s), s);
    return out;
}

at::Tensor softcap_tanh_fwd_bf16(at::Tensor scores, double cap) {
    return softcap_fwd(scores, cap, launch_softcap_tanh_d4_bf16);
}

at::Tensor softcap_tanh_native_bf16(at::Tensor scores, double cap) {
    return softcap_fwd(scores, cap, launch_softcap_tanh_native_bf16);
}

using SoftcapBwdLauncher = int (*)(void*, const void*, const void*, int64_t, float, void*);

at::Tensor softcap_bwd(at::Tensor grad_out, at::Tensor scores, double cap, SoftcapBwdLauncher fn) {
    CHECK_CUDA(grad_out);
    CHECK_CUDA(scores);
    CHECK_CONTIGUOUS(grad_out);
    CHECK_CONTIGUOUS(scores);
    TORCH_CHECK(scores.scalar_type() == at::kBFloat16, "scores must be bfloat16");
    TORCH_CHECK(grad_out.scalar_type() == at::kBFloat16, "grad_out must be bfloat16");
    TORCH_CHECK(grad_out.numel() == scores.numel(),
                "grad_out and scores must have the same number of elements");
    TORCH_CHECK(cap > 0.0, "cap must be positive");
    c10::OptionalDeviceGuard guard(scores.device());
    at::Tensor g = at::empty_like(scores);
    void* s = current_stream(scores);
    check_launch(fn(g.data_ptr(), grad_out.data_ptr(), scores.data_ptr(), scores.numel(),
                    static_cast<float>(cap), s),
                 s);
    return g;
}

at::Tensor softcap_tanh_bwd_bf16(at::Tensor grad_out, at::Tensor scores, double cap) {
    return softcap_bwd(grad_out, scores, cap, launch_softcap_tanh_d4_bwd_bf16);
}

at::Tensor softcap_tanh_native_bwd_bf16(at::Tensor grad_out, at::Tensor scores, double cap) {
    return softcap_bwd(grad_out, scores, cap, launch_softcap_tanh_native_bwd_bf16);
}

using Exp2Launcher = int (*)(void*, const void*, int64_t, void*);

at::Tensor exp2_f32_to(at::Tensor x, Exp2Launcher fn, at::ScalarType out_type) {
    CHECK_CUDA(x);
    CHECK_CONTIGUOUS(x);
    TORCH_CHECK(x.scalar_type() == at::kFloat, "x must be float32");
    c10::OptionalDeviceGuard guard(x.device());
    at::Tensor y = at::empty(x.sizes(), x.options().dtype(out_type));
    void* s = current_stream(x);
    check_launch(fn(y.data_ptr(), x.data_ptr(), x.numel(), s), s);
    return y;
}

// ---------------------------------------------------------------------------
// sin/cos tables and RoPE (spline_ops.cpp:326-918)
// ---------------------------------------------------------------------------

using SincosLauncher = int (*)(void*, const void*, int64_t, void*);
using SincosComputeLauncher = int (*)(void*, const void*, int64_t, int64_t, void*);

// sincos_f32 / sincos_bf16 / sincos_fp16 and their compute forms
// (spline_ops.cpp:326-580, 980-1100): FP32 angles -> [2, *angles.shape].
// The 16-bit tables need an even element count and the 16-bit probes a
// multiple of four, as in the reference.
at::Tensor sincos_out(const at::Tensor& angles, at::ScalarType out_type, int64_t multiple,
                      int64_t iterations) {
    CHECK_CUDA(angles);
    CHECK_CONTIGUOUS(angles);
    TORCH_CHECK(angles.scalar_type() == at::kFloat, "angles must be float32");
    if (multiple == 2)
        TORCH_CHECK((angles.numel() % 2) == 0, "angles must contain an even number of elements");
    if (multiple == 4)
        TORCH_CHECK((angles.numel() % 4) == 0, "angles must contain a multiple of four elements");
    if (iterations >= 0) {
        TORCH_CHECK(iterations > 0, "iterations must be positive");
        TORCH_CHECK(iterations <= std::numeric_limits<int>::max(),
                    "iterations is too large for the CUDA launcher");
    }
    std::vector<int64_t> sizes = angles.sizes().vec();
    sizes.insert(sizes.begin(), 2);
    return at::empty(sizes, angles.options().dtype(out_type));
}

at::Tensor sincos_table(at::Tensor angles, SincosLauncher fn, at::ScalarType out_type) {
    c10::OptionalDeviceGuard guard(angles.device());
    at::Tensor out = sincos_out(angles, out_type, out_type == at::kFloat ? 1 : 2, -1);
    void* s = current_stream(angles);
    check_launch(fn(out.data_ptr(), angles.data_ptr(), angles.numel(), s), s);
    return out;
}

at::Tensor sincos_compute(at::Tensor angles, int64_t iterations, SincosComputeLauncher fn,
                          at::ScalarType out_type) {
    c10::OptionalDeviceGuard guard(angles.device());
    at::Tensor out = sincos_out(angles, out_type, out_type == at::kFloat ? 1 : 4, iterations);
    void* s = current_stream(angles);
    check_launch(fn(out.data_ptr(), angles.data_ptr(), angles.numel(), iterations, s), s);
    return out;
}

// allocate_rope_sincos_fp16_output + rope_sincos_fp16 / _compute
// (spline_ops.cpp:585-760): parameters [F] (int32 increments or FP32
// frequencies) -> [2, S, F] FP16.
at::Tensor rope_table_out(const at::Tensor& params, int64_t sequence_length,
                          at::ScalarType param_type, const char* param_name, int64_t multiple) {
    CHECK_CUDA(params);
    CHECK_CONTIGUOUS(params);
    TORCH_CHECK(params.dim() == 1, param_name, " must be one-dimensional");
    TORCH_CHECK(params.scalar_type() == param_type, param_name, " has the wrong dtype");
    if (multiple == 4)
        TORCH_CHECK((params.numel() % 4) == 0, param_name, " must contain a multiple of four elements");
    TORCH_CHECK((params.numel() % 2) == 0, param_name, " must contain an even number of elements");
    TORCH_CHECK(sequence_length >= 0, "sequence_length must be non-negative");
    return at::empty({2, sequence_length, params.numel()}, params.options().dtype(at::kHalf));
}

using RopeTableLauncher = int (*)(void*, const void*, int64_t, int64_t, void*);
using RopeTableComputeLauncher = int (*)(void*, const void*, int64_t, int64_t, int64_t, void*);

at::Tensor rope_table(at::Tensor params, int64_t sequence_length, at::ScalarType param_type,
                      const char* param_name, int64_t multiple, RopeTableLauncher fn) {
    c10::OptionalDeviceGuard guard(params.device());
    at::Tensor out = rope_table_out(params, sequence_length, param_type, param_name, multiple);
    void* s = current_stream(params);
    check_launch(fn(out.data_ptr(), params.data_ptr(), sequence_length, params.numel(), s), s);
    return out;
}

at::Tensor rope_table_compute(at::Tensor params, int64_t sequence_length, int64_t iterations,
                              at::ScalarType param_type, const char* param_name, int64_t multiple,
                              RopeTableComputeLauncher fn) {
    c10::OptionalDeviceGuard guard(params.device());
    at::Tensor out = rope_table_out(params, sequence_length, param_type, param_name, multiple);
    TORCH_CHECK(iterations > 0, "iterations must be positive");
    TORCH_CHECK(iterations <= std::numeric_limits<int>::max(),
                "iterations is too large for the CUDA launcher");
    void* s = current_stream(params);
    check_launch(fn(out.data_ptr(), params.data_ptr(), sequence_length, params.numel(), iterations,
                    s),
                 s);
    return out;
}

// check_rope_phase_table (spline_ops.cpp:675-691)
void check_rope_phase_table(const at::Tensor& phase_increments, const at::Tensor& phase_table) {
    CHECK_CUDA(phase_table);
    CHECK_CONTIGUOUS(phase_table);
    TORCH_CHECK(phase_table.scalar_type() == at::kHalf, "phase_table must be float16");
    TORCH_CHECK(phase_table.dim() == 2 && phase_table.size(0) == 128 && phase_table.size(1) == 2,
                "phase_table must have shape [128, 2]");
    TORCH_CHECK(phase_table.get_device() == phase_increments.get_device(),
                "phase_table and phase_increments must be on the same CUDA device");
}

at::Tensor rope_sincos_fixed_lut_fp16(at::Tensor phase_increments, at::Tensor phase_table,
                                      int64_t sequence_length, int64_t iterations) {
    c10::OptionalDeviceGuard guard(phase_increments.device());
    at::Tensor out =
        rope_table_out(phase_increments, sequence_length, at::kInt, "phase_increments", 2);
    check_rope_phase_table(phase_increments, phase_table);
    void* s = current_stream(phase_increments);
    if (iterations < 0) {
        check_launch(launch_rope_sincos_fixed_lut_fp16(out.data_ptr(), phase_increments.data_ptr(),
                                                       phase_table.data_ptr(), sequence_length,
                                                       phase_increments.numel(), s),
                     s);
    } else {
        TORCH_CHECK(iterations > 0, "iterations must be positive");
        TORCH_CHECK(iterations <= std::numeric_limits<int>::max(),
                    "iterations is too large for the CUDA launcher");
        check_launch(launch_rope_sincos_fixed_lut_fp16_compute(
                         out.data_ptr(), phase_increments.data_ptr(), phase_table.data_ptr(),
                         sequence_length, phase_increments.numel(), iterations, s),
                     s);
    }
    return out;
}

using RopeLauncher = int (*)(void*, void*, const void*, const void*, const void*, int64_t,
                             int64_t, int64_t, int64_t, int64_t, void*);

// check_rope_apply_fp16_inputs + rope_apply_parameter_fp16 (spline_ops.cpp:831-918)
std::vector<at::Tensor> rope_apply(at::Tensor q, at::Tensor k, at::Tensor parameters,
                                   at::ScalarType dtype, at::ScalarType parameter_type,
                                   const char* parameter_name, RopeLauncher fn) {
    const char* dname = dtype == at::kHalf ? "float16" : "bfloat16";
    CHECK_CUDA(q);
    CHECK_CUDA(k);
    CHECK_CONTIGUOUS(q);
    CHECK_CONTIGUOUS(k);
    TORCH_CHECK(q.scalar_type() == dtype, "q must be ", dname);
    TORCH_CHECK(k.scalar_type() == dtype, "k must be ", dname);
    TORCH_CHECK(q.dim() == 4, "q must have shape [batch, sequence, heads, head_dim]");
    TORCH_CHECK(k.dim() == 4, "k must have shape [batch, sequence, heads, head_dim]");
    TORCH_CHECK(q.get_device() == k.get_device(), "q and k must be on the same CUDA device");
    TORCH_CHECK(q.size(0) == k.size(0), "q and k batch sizes must match");
    TORCH_CHECK(q.size(1) == k.size(1), "q and k sequence lengths must match");
    TORCH_CHECK(q.size(3) == k.size(3), "q and k head dimensions must match");
    TORCH_CHECK(q.size(2) > 0 && k.size(2) > 0, "q and k must contain at least one head");
    TORCH_CHECK(q.size(3) > 0 && (q.size(3) % 8) == 0,
                "head_dim must be a positive multiple of eight");
    // CHECK_CUDA / CHECK_CONTIGUOUS name the argument: `parameters` in
    // rope_apply_parameter_fp16, `rope_table` in rope_apply_cached_fp16.
    const bool cached = std::strcmp(parameter_name, "rope_table") == 0;
    const char* arg = cached ? "rope_table" : "parameters";
    TORCH_CHECK(parameters.is_cuda(), arg, " must be a CUDA tensor");
    TORCH_CHECK(parameters.is_contiguous(), arg, " must be contiguous");
    if (cached) {
        // rope_apply_cached_fp16 (spline_ops.cpp:920-953)
        TORCH_CHECK(parameters.scalar_type() == at::kHalf, "rope_table must be float16");
        TORCH_CHECK(parameters.get_device() == q.get_device(),
                    "rope_table must be on the same CUDA device as q and k");
        TORCH_CHECK(parameters.dim() == 3 && parameters.size(0) == 2 &&
                        parameters.size(1) == q.size(1) && parameters.size(2) == q.size(3) / 2,
                    "rope_table must have shape [2, sequence_length, head_dim / 2]");
    } else {
        TORCH_CHECK(parameters.dim() == 1, parameter_name, " must be one-dimensional");
        TORCH_CHECK(parameters.scalar_type() == parameter_type, parameter_name,
                    " has the wrong dtype");
        TORCH_CHECK(parameters.get_device() == q.get_device(), parameter_name,
                    " must be on the same CUDA device as q and k");
        TORCH_CHECK(parameters.numel() == q.size(3) / 2, parameter_name,
                    " must contain head_dim / 2 elements");
    }
    c10::OptionalDeviceGuard guard(q.device());
    const int64_t b = q.size(0), sl = q.size(1), hq = q.size(2), hk = k.size(2), d = q.size(3);
    at::Tensor q_out = at::empty({b, hq, sl, d}, q.options());
    at::Tensor k_out = at::empty({b, hk, sl, d}, k.options());
    void* s = current_stream(q);
    check_launch(fn(q_out.data_ptr(), k_out.data_ptr(), q.data_ptr(), k.data_ptr(),
                    parameters.data_ptr(), b, sl, hq, hk, d, s),
                 s);
    return {q_out, k_out};
}

// ---------------------------------------------------------------------------
// RoPE reference evaluator (src/sfu_repro/rope/polynomial_sincos.py:85-165)
// ---------------------------------------------------------------------------

// FP32 or FP64 storage the kernel reads directly; 16-bit angles are widened
// exactly to FP32 first.
at::Tensor ref_angles(const at::Tensor& angles, const char* name) {
    TORCH_CHECK(at::isFloatingType(angles.scalar_type()), name, " must be a floating-point tensor");
    CHECK_CUDA(angles);
    at::Tensor a = angles.contiguous();
    if (a.scalar_type() != at::kFloat && a.scalar_type() != at::kDouble) a = a.to(at::kFloat);
    return a;
}

void check_coeffs(const std::vector<double>& c, const char* name) {
    TORCH_CHECK(!c.empty() && c.size() <= 8, name, " must hold 1 to 8 coefficients");
}

std::vector<float> to_f32(const std::vector<double>& c) {
    return std::vector<float>(c.begin(), c.end());  // each rounded to FP32 (RNE)
}

std::vector<at::Tensor> polynomial_sincos_f32(at::Tensor angles, std::vector<double> sin_coeffs,
                                              std::vector<double> cos_coeffs, bool accurate) {
    at::Tensor a = ref_angles(angles, "angles");
    check_coeffs(sin_coeffs, "sin_coefficients");
    check_coeffs(cos_coeffs, "cos_coefficients");
    const std::vector<float> sc = to_f32(sin_coeffs), cc = to_f32(cos_coeffs);
    c10::OptionalDeviceGuard guard(a.device());
    at::Tensor c = at::empty(a.sizes(), a.options().dtype(at::kFloat));
    at::Tensor sn = at::empty_like(c);
    void* s = current_stream(a);
    check_launch(launch_polynomial_sincos_f32(c.data_ptr(), sn.data_ptr(), a.data_ptr(),
                                              a.scalar_type() == at::kDouble, a.numel(), accurate,
                                              sc.data(), (int)sc.size(), cc.data(), (int)cc.size(), s),
                 s);
    return {c, sn};
}

// ---------------------------------------------------------------------------
// fused attention (the runtime behind sfu_repro.fa4; FA4's flash_attn_fwd,
// src/sfu_repro/fa4.py:356-428): q [B, S, Hq, 128], k and v [B, S, Hkv, 128]
// BF16 with a contiguous head dimension -> out [B, S, Hq, 128], lse [B, Hq, S]
// ---------------------------------------------------------------------------

void check_attn_operand(const at::Tensor& t, const char* name) {
    TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
    TORCH_CHECK(t.scalar_type() == at::kBFloat16, name, " must be bfloat16");
    TORCH_CHECK(t.dim() == 4, name, " must have shape [batch, seqlen, heads, head_dim]");
    TORCH_CHECK(t.stride(3) == 1, name, " must be contiguous in head_dim");
}

std::vector<at::Tensor> flash_attn_fwd_bf16(at::Tensor q, at::Tensor k, at::Tensor v, int64_t mode,
                                            int64_t exp2_route, bool causal, double softmax_scale,
                                            double softcap, double sigmoid_bias, int64_t valid_keys) {
    check_attn_operand(q, "q");
    check_attn_operand(k, "k");
    check_attn_operand(v, "v");
    TORCH_CHECK(k.sizes() == v.sizes(), "k and v must have the same shape");
    TORCH_CHECK(q.size(0) == k.size(0) && q.size(1) == k.size(1) && q.size(3) == k.size(3),
                "q, k and v must agree in batch, seqlen and head_dim");
    TORCH_CHECK(q.size(3) == 64 || q.size(3) == 128, "head_dim must be 64 or 128, got ", q.size(3));
    TORCH_CHECK(q.size(2) % k.size(2) == 0, "q heads (", q.size(2),
                ") must be a multiple of kv heads (", k.size(2), ")");
    c10::OptionalDeviceGuard guard(q.device());
    const int64_t b = q.size(0), sq = q.size(1), hq = q.size(2), hkv = k.size(2);
    const int64_t d = q.size(3);
    at::Tensor out = at::empty({b, sq, hq, d}, q.options());
    // the softmax and softcap modes write every lse row; the sigmoid modes
    // (5..11) have no partition function and leave it untouched, so only
    // they need it cleared
    const bool sigmoid_mode = mode >= 5 && mode <= 11;
    at::Tensor lse = sigmoid_mode ? at::zeros({b, hq, sq}, q.options().dtype(at::kFloat))
                                  : at::empty({b, hq, sq}, q.options().dtype(at::kFloat));
    const int64_t strides[12] = {q.stride(0), q.stride(2), q.stride(1), k.stride(0), k.stride(2),
                                 k.stride(1), v.stride(0), v.stride(2), v.stride(1), out.stride(0),
                                 out.stride(2), out.stride(1)};
    void* s = current_stream(q);
    TORCH_CHECK(valid_keys < 0 || (valid_keys >= 1 && valid_keys <= sq),
                "valid_keys must be in [1, seqlen] (or negative for all), got ", valid_keys);
    check_launch(launch_flash_attention_fwd_strided_keys_bf16(
                     out.data_ptr(), lse.data_ptr<float>(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                     b, hq, hkv, sq, valid_keys < 0 ? sq : valid_keys, d, strides, (int)mode,
                     (int)exp2_route, causal ? 1 : 0, (float)softmax_scale, (float)softcap,
                     (float)sigmoid_bias, s),
                 s);
    return {out, lse};
}

// Largest dS workspace the attention backward allocates: the environment's
// SPLINE_ATTN_DS_MAX_BYTES (bytes, 0 turns the dS-keeping backward off),
// 8 GiB by default.
int64_t attn_ds_max_bytes() {
    const char* e = std::getenv("SPLINE_ATTN_DS_MAX_BYTES");
    if (e == nullptr || *e == '\0') return int64_t(8) << 30;
    char* end = nullptr;
    const long long v = std::strtoll(e, &end, 10);
    TORCH_CHECK(end != e && *end == '\0' && v >= 0, "SPLINE_ATTN_DS_MAX_BYTES must be a byte count, got '", e, "'");
    return (int64_t)v;
}

std::vector<at::Tensor> flash_attn_bwd_bf16(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor out,
                                            at::Tensor dout, at::Tensor lse, int64_t mode, int64_t grad,
                                            int64_t exp2_route, bool causal, double softmax_scale,
                                            double softcap, double sigmoid_bias) {
    check_attn_operand(q, "q");
    check_attn_operand(k, "k");
    check_attn_operand(v, "v");
    check_attn_operand(out, "out");
    check_attn_operand(dout, "dout");
    TORCH_CHECK(k.sizes() == v.sizes(), "k and v must have the same shape");
    TORCH_CHECK(out.sizes() == q.sizes() && dout.sizes() == q.sizes(), "out and dout must have q's shape");
    TORCH_CHECK(q.size(0) == k.size(0) && q.size(1) == k.size(1) && q.size(3) == k.size(3),
                "q, k and v must agree in batch, seqlen and head_dim");
    TORCH_CHECK(q.size(3) == 64 || q.size(3) == 128, "head_dim must be 64 or 128, got ", q.size(3));
    TORCH_CHECK(q.size(2) % k.size(2) == 0, "q heads must be a multiple of kv heads");
    const int64_t b = q.size(0), sq = q.size(1), hq = q.size(2), hkv = k.size(2);
    TORCH_CHECK(lse.is_cuda() && lse.scalar_type() == at::kFloat && lse.is_contiguous() &&
                    lse.dim() == 3 && lse.size(0) == b && lse.size(1) == hq && lse.size(2) == sq,
                "lse must be a contiguous float32 CUDA tensor [batch, heads, seqlen]");
    c10::OptionalDeviceGuard guard(q.device());
    const int64_t d = q.size(3);
    at::Tensor dq = at::empty({b, sq, hq, d}, q.options());
    at::Tensor dk = at::empty({b, sq, hkv, d}, q.options());
    at::Tensor dv = at::empty({b, sq, hkv, d}, q.options());
    at::Tensor delta = at::empty({b, hq, sq}, q.options().dtype(at::kFloat));
    at::Tensor dkv_ws = hq != hkv ? at::empty({2, b, hq, sq, d}, q.options().dtype(at::kFloat))
                                  : at::Tensor();
    const int64_t strides[24] = {q.stride(0),    q.stride(2),    q.stride(1),    k.stride(0),
                                 k.stride(2),    k.stride(1),    v.stride(0),    v.stride(2),
                                 v.stride(1),    out.stride(0),  out.stride(2),  out.stride(1),
                                 dout.stride(0), dout.stride(2), dout.stride(1), dq.stride(0),
                                 dq.stride(2),   dq.stride(1),   dk.stride(0),   dk.stride(2),
                                 dk.stride(1),   dv.stride(0),   dv.stride(2),   dv.stride(1)};
    // dS workspace of the dS-keeping backward (B * Hq * S^2 BF16 where it
    // applies), up to SPLINE_ATTN_DS_MAX_BYTES (default 8 GiB; 0 turns it
    // off), from the caching allocator
    const int64_t ds_bytes = spline_hip_attn_bwd_ds_bytes(b, hq, sq, d, (int)mode);
    at::Tensor ds_ws = ds_bytes > 0 && ds_bytes <= attn_ds_max_bytes()
                           ? at::empty({ds_bytes / 2}, q.options())
                           : at::Tensor();
    void* s = current_stream(q);
    check_launch(launch_flash_attention_bwd_strided_ds_bf16(
                     dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), delta.data_ptr<float>(),
                     hq != hkv ? dkv_ws.data_ptr<float>() : nullptr, ds_ws.defined() ? ds_ws.data_ptr() : nullptr,
                     q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), dout.data_ptr(),
                     lse.data_ptr<float>(), b, hq, hkv, sq, d, strides, (int)mode, (int)grad,
                     (int)exp2_route, causal ? 1 : 0, (float)softmax_scale, (float)softcap,
                     (float)sigmoid_bias, s),
                 s);
    return {dq, dk, dv};
}

std::vector<at::Tensor> reduce_to_quarter_turn_f32(at::Tensor angles, bool accurate) {
    at::Tensor a = ref_angles(angles, "angles");
    c10::OptionalDeviceGuard guard(a.device());
    at::Tensor r = at::empty(a.sizes(), a.options().dtype(at::kFloat));
    at::Tensor q = at::empty(a.sizes(), a.options().dtype(at::kLong));
    void* s = current_stream(a);
    check_launch(launch_reduce_to_quarter_turn(r.data_ptr(), q.data_ptr(), a.data_ptr(),
                                               a.scalar_type() == at::kDouble, a.numel(), accurate, s),
                 s);
    return {r, q};
}

std::vector<at::Tensor> evaluate_reduced_sincos_f32(at::Tensor reduced, std::vector<double> sin_coeffs,
                                                    std::vector<double> cos_coeffs) {
    at::Tensor r = ref_angles(reduced, "reduced");
    check_coeffs(sin_coeffs, "sin_coefficients");
    check_coeffs(cos_coeffs, "cos_coefficients");
    const std::vector<float> sc = to_f32(sin_coeffs), cc = to_f32(cos_coeffs);
    c10::OptionalDeviceGuard guard(r.device());
    at::Tensor sn = at::empty(r.sizes(), r.options().dtype(at::kFloat));
    at::Tensor c = at::empty_like(sn);
    void* s = current_stream(r);
    check_launch(launch_evaluate_reduced_sincos(sn.data_ptr(), c.data_ptr(), r.data_ptr(),
                                                r.scalar_type() == at::kDouble, r.numel(), sc.data(),
                                                (int)sc.size(), cc.data(), (int)cc.size(), s),
                 s);
    return {sn, c};
}

// ---------------------------------------------------------------------------
// FP16 experiments: hybrid, fused, forward-with-derivative, multiply
// (spline_ops.cpp:1548-1926)
// ---------------------------------------------------------------------------

#define CHECK_HALF(x) \
    TORCH_CHECK(x.scalar_type() == at::kHalf, #x " must be float16 (no BF16 support for this op)")
#define CHECK_INPUT_FP16(x) \
    CHECK_CUDA(x);          \
    CHECK_CONTIGUOUS(x);    \
    CHECK_HALF(x)

using UnaryLauncher = int (*)(void*, const void*, int64_t, void*);
using BinaryLauncher = int (*)(void*, const void*, const void*, int64_t, void*);
using PairLauncher = int (*)(void*, void*, const void*, int64_t, void*);
using FusedLauncher = int (*)(void*, void*, const void*, const void*, int64_t, void*);

// Shapes must agree: the kernels read both inputs over x.numel() elements.
void check_same_numel(const at::Tensor& a, const at::Tensor& b, const char* an, const char* bn) {
    TORCH_CHECK(a.numel() == b.numel(), an, " and ", bn, " must have the same number of elements");
}

at::Tensor fp16_fwd(at::Tensor x, UnaryLauncher fn) {
    CHECK_INPUT_FP16(x);
    c10::OptionalDeviceGuard guard(x.device());
    at::Tensor out = at::empty_like(x);
    void* s = current_stream(x);
    check_launch(fn(out.data_ptr(), x.data_ptr(), x.numel(), s), s);
    return out;
}

at::Tensor fp16_bwd(at::Tensor grad_out, at::Tensor x, BinaryLauncher fn) {
    CHECK_INPUT_FP16(grad_out);
    CHECK_INPUT_FP16(x);
    check_same_numel(grad_out, x, "grad_out", "x");
    c10::OptionalDeviceGuard guard(x.device());
    at::Tensor grad_in = at::empty_like(x);
    void* s = current_stream(x);
    check_launch(fn(grad_in.data_ptr(), grad_out.data_ptr(), x.data_ptr(), x.numel(), s), s);
    return grad_in;
}

std::vector<at::Tensor> fp16_fused(at::Tensor x, at::Tensor grad_out, FusedLauncher fn) {
    CHECK_INPUT_FP16(x);
    CHECK_INPUT_FP16(grad_out);
    check_same_numel(x, grad_out, "x", "grad_out");
    c10::OptionalDeviceGuard guard(x.device());
    at::Tensor y = at::empty_like(x);
    at::Tensor gi = at::empty_like(x);
    void* s = current_stream(x);
    check_launch(fn(y.data_ptr(), gi.data_ptr(), x.data_ptr(), grad_out.data_ptr(), x.numel(), s), s);
    return {y, gi};
}

std::vector<at::Tensor> fp16_fwd_deriv(at::Tensor x, PairLauncher fn) {
    CHECK_INPUT_FP16(x);
    c10::OptionalDeviceGuard guard(x.device());
    at::Tensor y = at::empty_like(x);
    at::Tensor dy = at::empty_like(x);
    void* s = current_stream(x);
    check_launch(fn(y.data_ptr(), dy.data_ptr(), x.data_ptr(), x.numel(), s), s);
    return {y, dy};
}

at::Tensor multiply(at::Tensor a, at::Tensor b) {
    CHECK_INPUT(a);
    CHECK_INPUT(b);
    TORCH_CHECK(a.scalar_type() == b.scalar_type(), "a and b must have the same dtype");
    check_same_numel(a, b, "a", "b");
    c10::OptionalDeviceGuard guard(a.device());
    at::Tensor out = at::empty_like(a);
    void* s = current_stream(a);
    auto fn = a.scalar_type() == at::kHalf ? launch_multiply_kernel : launch_multiply_kernel_bf16;
    check_launch(fn(out.data_ptr(), a.data_ptr(), b.data_ptr(), a.numel(), s), s);
    return out;
}

// ---------------------------------------------------------------------------
// C++ autograd functions (spline_ops.cpp:1933-2206)
// ---------------------------------------------------------------------------

using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

// sigmoid / tanh: D3 forward, algebraic backward from the saved output.
template <int FAM>
struct AlgebraicFwd : public torch::autograd::Function<AlgebraicFwd<FAM>> {
    static at::Tensor forward(AutogradContext* ctx, at::Tensor x) {
        CHECK_INPUT(x);
        at::Tensor y = run_unary(x, kFwd[FAM][x.scalar_type() == at::kBFloat16][3]);
        ctx->save_for_backward({y});
        return y;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        at::Tensor y = ctx->get_saved_variables()[0];
        at::Tensor go = grads[0].contiguous();
        return {bwd_alg(go, y, FAM)};
    }
};

// SiLU: forward of `degree`, backward with the derivative program of the
// same degree (the fixed op uses D3 forward / D4 backward, :1993-2015).
struct SwishVariantFwd : public torch::autograd::Function<SwishVariantFwd> {
    static at::Tensor forward(AutogradContext* ctx, at::Tensor x, int64_t fwd_degree,
                              int64_t bwd_degree, int64_t coeff_source_id) {
        at::Tensor out = fwd_variant(x, fwd_degree, coeff_source_id, SWISH);
        ctx->save_for_backward({x});
        ctx->saved_data["bwd_degree"] = bwd_degree;
        ctx->saved_data["coeff_source_id"] = coeff_source_id;
        return out;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        at::Tensor x = ctx->get_saved_variables()[0];
        at::Tensor go = grads[0].contiguous();
        at::Tensor gi = bwd_variant(go, x, ctx->saved_data["bwd_degree"].toInt(),
                                    ctx->saved_data["coeff_source_id"].toInt(), SWISH);
        return {gi, at::Tensor(), at::Tensor(), at::Tensor()};
    }
};

struct SwishMulVariantFwd : public torch::autograd::Function<SwishMulVariantFwd> {
    static at::Tensor forward(AutogradContext* ctx, at::Tensor gate, at::Tensor up, int64_t degree,
                              int64_t coeff_source_id) {
        at::Tensor out = swish_mul_fwd_variant(gate, up, degree, coeff_source_id);
        ctx->save_for_backward({gate, up});
        ctx->saved_data["degree"] = degree;
        ctx->saved_data["coeff_source_id"] = coeff_source_id;
        return out;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        auto saved = ctx->get_saved_variables();
        at::Tensor go = grads[0].contiguous();
        auto g = swish_mul_bwd_variant(go, saved[0], saved[1], ctx->saved_data["degree"].toInt(),
                                       ctx->saved_data["coeff_source_id"].toInt());
        return {g[0], g[1], at::Tensor(), at::Tensor()};
    }
};

// GeLU: forward and derivative programs of one degree and source
// (SplineGeLUVariantFwd, spline_ops.cpp:2132-2180).
struct GeluVariantFwd : public torch::autograd::Function<GeluVariantFwd> {
    static at::Tensor forward(AutogradContext* ctx, at::Tensor x, int64_t degree,
                              int64_t coeff_source_id) {
        const int source = normalize_coeff_source_id(coeff_source_id);
        at::Tensor out = fwd_variant(x, degree, source, GELU);
        ctx->save_for_backward({x});
        ctx->saved_data["degree"] = degree;
        ctx->saved_data["coeff_source_id"] = static_cast<int64_t>(source);
        return out;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        at::Tensor x = ctx->get_saved_variables()[0];
        at::Tensor go = grads[0].contiguous();
        at::Tensor gi = bwd_variant(go, x, ctx->saved_data["degree"].toInt(),
                                    ctx->saved_data["coeff_source_id"].toInt(), GELU);
        return {gi, at::Tensor(), at::Tensor()};
    }
};

at::Tensor gelu_fwd_variant_autograd(at::Tensor x, int64_t degree, int64_t coeff_source_id) {
    return GeluVariantFwd::apply(x, degree, coeff_source_id);
}
at::Tensor sigmoid_fwd_autograd(at::Tensor x) { return AlgebraicFwd<SIGMOID>::apply(x); }
at::Tensor tanh_fwd_autograd(at::Tensor x) { return AlgebraicFwd<TANH>::apply(x); }
at::Tensor swish_fwd_autograd(at::Tensor x) { return SwishVariantFwd::apply(x, 3, 4, 0); }
at::Tensor swish_fwd_variant_autograd(at::Tensor x, int64_t degree, int64_t coeff_source_id) {
    normalize_coeff_source_id(coeff_source_id);
    return SwishVariantFwd::apply(x, degree, degree, coeff_source_id);
}
at::Tensor swish_mul_fwd_variant_autograd(at::Tensor gate, at::Tensor up, int64_t degree,
                                          int64_t coeff_source_id) {
    return SwishMulVariantFwd::apply(gate, up, degree, coeff_source_id);
}

// ---------------------------------------------------------------------------
// dispatcher-facing wrappers
// ---------------------------------------------------------------------------

at::Tensor sigmoid_bwd_op(at::Tensor go, at::Tensor x) { return bwd_fixed(go, x, SIGMOID, 4); }
at::Tensor tanh_bwd_op(at::Tensor go, at::Tensor x) { return bwd_fixed(go, x, TANH, 4); }
at::Tensor swish_bwd_op(at::Tensor go, at::Tensor x) { return bwd_fixed(go, x, SWISH, 4); }
at::Tensor sigmoid_bwd_alg_op(at::Tensor go, at::Tensor y) { return bwd_alg(go, y, SIGMOID); }
at::Tensor tanh_bwd_alg_op(at::Tensor go, at::Tensor y) { return bwd_alg(go, y, TANH); }
at::Tensor swish_fwd_variant_op(at::Tensor x, int64_t d, int64_t c) { return fwd_variant(x, d, c, SWISH); }
at::Tensor swish_bwd_variant_op(at::Tensor go, at::Tensor x, int64_t d, int64_t c) {
    return bwd_variant(go, x, d, c, SWISH);
}

}  // namespace

// ===========================================================================
// TORCH_LIBRARY: the reference's schemas (spline_ops.cpp:2212-2250)
// ===========================================================================

TORCH_LIBRARY(spline_ops, m) {
    m.def("sigmoid_fwd(Tensor x) -> Tensor");
    m.def("tanh_fwd(Tensor x) -> Tensor");
    m.def("swish_fwd(Tensor x) -> Tensor");
    m.def("sigmoid_bwd(Tensor grad_out, Tensor x) -> Tensor");
    m.def("tanh_bwd(Tensor grad_out, Tensor x) -> Tensor");
    m.def("swish_bwd(Tensor grad_out, Tensor x) -> Tensor");
    m.def("sigmoid_bwd_alg(Tensor grad_out, Tensor y) -> Tensor");
    m.def("tanh_bwd_alg(Tensor grad_out, Tensor y) -> Tensor");
    m.def("swish_variant_fwd(Tensor x, int degree, int coeff_source_id) -> Tensor");
    m.def("swish_variant_bwd(Tensor grad_out, Tensor x, int degree, int coeff_source_id) -> Tensor");
    m.def("swish_mul_variant_fwd(Tensor gate, Tensor up, int degree, int coeff_source_id) -> Tensor");
    m.def(
        "swish_mul_variant_bwd(Tensor grad_out, Tensor gate, Tensor up, int degree, "
        "int coeff_source_id) -> Tensor[]");
    m.def("swish_mul_packed_variant_fwd(Tensor packed, int degree, int coeff_source_id) -> Tensor");
    m.def("swish_mul_packed_native_fwd(Tensor packed, int coeff_source_id) -> Tensor");
    m.def(
        "swish_mul_packed_native_bwd_fwd(Tensor packed, int degree, int coeff_source_id) -> Tensor");
    m.def(
        "swish_mul_packed_variant_bwd(Tensor grad_out, Tensor packed, int degree, "
        "int coeff_source_id) -> Tensor");
}

TORCH_LIBRARY_IMPL(spline_ops, AutogradCUDA, m) {
    m.impl("sigmoid_fwd", &sigmoid_fwd_autograd);
    m.impl("tanh_fwd", &tanh_fwd_autograd);
    m.impl("swish_fwd", &swish_fwd_autograd);
}

TORCH_LIBRARY_IMPL(spline_ops, CUDA, m) {
    m.impl("sigmoid_bwd", &sigmoid_bwd_op);
    m.impl("tanh_bwd", &tanh_bwd_op);
    m.impl("swish_bwd", &swish_bwd_op);
    m.impl("sigmoid_bwd_alg", &sigmoid_bwd_alg_op);
    m.impl("tanh_bwd_alg", &tanh_bwd_alg_op);
    m.impl("swish_variant_fwd", &swish_fwd_variant_op);
    m.impl("swish_variant_bwd", &swish_bwd_variant_op);
    m.impl("swish_mul_variant_fwd", &swish_mul_fwd_variant);
    m.impl("swish_mul_variant_bwd", &swish_mul_bwd_variant);
    m.impl("swish_mul_packed_variant_fwd", &swish_mul_packed_fwd_variant);
    m.impl("swish_mul_packed_native_fwd", [](at::Tensor packed, int64_t coeff_source_id) {
        return swish_mul_packed_fwd_variant(packed, 0, coeff_source_id);
    });
    m.impl("swish_mul_packed_native_bwd_fwd", &swish_mul_packed_fwd_variant);
    m.impl("swish_mul_packed_variant_bwd", &swish_mul_packed_bwd_variant);
}

// ===========================================================================
// pybind11 module (the reference's function names, spline_ops.cpp:2285-2452)
// ===========================================================================

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "MI355X (gfx950) packed polynomial transcendental kernels";

#define PT_DEF_FWD(fam, FAM, deg, name) \
    m.def(name, [](at::Tensor x) { return fwd_fixed(x, FAM, deg); }, "Polynomial " #fam " forward")
#define PT_DEF_BWD(fam, FAM, deg, name)                                                \
    m.def(name, [](at::Tensor go, at::Tensor x) { return bwd_fixed(go, x, FAM, deg); }, \
          "Polynomial " #fam " backward")

    PT_DEF_FWD(sigmoid, SIGMOID, 3, "sigmoid_fwd");
    PT_DEF_FWD(sigmoid, SIGMOID, 3, "sigmoid_fwd_d3");
    PT_DEF_FWD(sigmoid, SIGMOID, 4, "sigmoid_fwd_d4");
    PT_DEF_FWD(sigmoid, SIGMOID, 5, "sigmoid_fwd_d5");
    PT_DEF_FWD(sigmoid, SIGMOID, 6, "sigmoid_fwd_d6");
    PT_DEF_BWD(sigmoid, SIGMOID, 4, "sigmoid_bwd");
    PT_DEF_BWD(sigmoid, SIGMOID, 3, "sigmoid_bwd_d3");
    PT_DEF_BWD(sigmoid, SIGMOID, 4, "sigmoid_bwd_d4");
    PT_DEF_BWD(sigmoid, SIGMOID, 5, "sigmoid_bwd_d5");
    PT_DEF_BWD(sigmoid, SIGMOID, 6, "sigmoid_bwd_d6");
    PT_DEF_FWD(tanh, TANH, 3, "tanh_fwd");
    PT_DEF_FWD(tanh, TANH, 3, "tanh_fwd_d3");
    PT_DEF_FWD(tanh, TANH, 4, "tanh_fwd_d4");
    PT_DEF_FWD(tanh, TANH, 5, "tanh_fwd_d5");
    PT_DEF_FWD(tanh, TANH, 6, "tanh_fwd_d6");
    PT_DEF_BWD(tanh, TANH, 4, "tanh_bwd");
    PT_DEF_BWD(tanh, TANH, 3, "tanh_bwd_d3");
    PT_DEF_BWD(tanh, TANH, 4, "tanh_bwd_d4");
    PT_DEF_BWD(tanh, TANH, 5, "tanh_bwd_d5");
    PT_DEF_BWD(tanh, TANH, 6, "tanh_bwd_d6");
    PT_DEF_FWD(swish, SWISH, 3, "swish_fwd");
    PT_DEF_FWD(swish, SWISH, 3, "swish_fwd_d3");
    PT_DEF_FWD(swish, SWISH, 4, "swish_fwd_d4");
    PT_DEF_FWD(swish, SWISH, 5, "swish_fwd_d5");
    PT_DEF_FWD(swish, SWISH, 6, "swish_fwd_d6");
    PT_DEF_BWD(swish, SWISH, 4, "swish_bwd");
    PT_DEF_BWD(swish, SWISH, 3, "swish_bwd_d3");
    PT_DEF_BWD(swish, SWISH, 4, "swish_bwd_d4");
    PT_DEF_BWD(swish, SWISH, 5, "swish_bwd_d5");
    PT_DEF_BWD(swish, SWISH, 6, "swish_bwd_d6");
    PT_DEF_FWD(GeLU, GELU, 5, "gelu_fwd");
    PT_DEF_FWD(GeLU, GELU, 3, "gelu_fwd_d3");
    PT_DEF_FWD(GeLU, GELU, 4, "gelu_fwd_d4");
    PT_DEF_FWD(GeLU, GELU, 5, "gelu_fwd_d5");
    PT_DEF_FWD(GeLU, GELU, 6, "gelu_fwd_d6");
    PT_DEF_BWD(GeLU, GELU, 5, "gelu_bwd");
    PT_DEF_BWD(GeLU, GELU, 3, "gelu_bwd_d3");
    PT_DEF_BWD(GeLU, GELU, 4, "gelu_bwd_d4");
    PT_DEF_BWD(GeLU, GELU, 5, "gelu_bwd_d5");
    PT_DEF_BWD(GeLU, GELU, 6, "gelu_bwd_d6");
#undef PT_DEF_FWD
#undef PT_DEF_BWD
    m.def("gelu_fwd_variant",
          [](at::Tensor x, int64_t d, int64_t c) { return fwd_variant(x, d, c, GELU); },
          "GeLU FWD variant by degree/source");
    m.def("gelu_bwd_variant",
          [](at::Tensor go, at::Tensor x, int64_t d, int64_t c) { return bwd_variant(go, x, d, c, GELU); },
          "GeLU BWD variant by degree/source");
    m.def("gelu_ag_variant", &gelu_fwd_variant_autograd,
          "GeLU variant with C++ autograd by degree/source");

    m.def("sigmoid_fwd_variant",
          [](at::Tensor x, int64_t d, int64_t c) { return fwd_variant(x, d, c, SIGMOID); },
          "Sigmoid FWD variant by degree/source");
    m.def("sigmoid_bwd_variant",
          [](at::Tensor go, at::Tensor x, int64_t d, int64_t c) { return bwd_variant(go, x, d, c, SIGMOID); },
          "Sigmoid BWD variant by degree/source");
    m.def("tanh_fwd_variant",
          [](at::Tensor x, int64_t d, int64_t c) { return fwd_variant(x, d, c, TANH); },
          "Tanh FWD variant by degree/source");
    m.def("tanh_bwd_variant",
          [](at::Tensor go, at::Tensor x, int64_t d, int64_t c) { return bwd_variant(go, x, d, c, TANH); },
          "Tanh BWD variant by degree/source");
    m.def("sigmoid_bwd_alg", &sigmoid_bwd_alg_op, "Sigmoid BWD algebraic (from y)");
    m.def("tanh_bwd_alg", &tanh_bwd_alg_op, "Tanh BWD algebraic (from y)");
    m.def("swish_fwd_variant", &swish_fwd_variant_op, "Swish FWD variant by degree/source");
    m.def("swish_bwd_variant", &swish_bwd_variant_op, "Swish BWD variant by degree/source");
    m.def("swish_mul_fwd_variant", &swish_mul_fwd_variant,
          "Swish(gate) * up FWD variant by degree/source");
    m.def("swish_mul_bwd_variant", &swish_mul_bwd_variant,
          "Swish(gate) * up BWD variant by degree/source");
    m.def("swish_mul_packed_fwd_variant", &swish_mul_packed_fwd_variant,
          "Swish(packed gate) * packed up FWD variant by degree/source");
    m.def("swish_mul_packed_bwd_variant", &swish_mul_packed_bwd_variant,
          "Swish(packed gate) * packed up BWD variant by degree/source");
    m.def("swish_ag_variant", &swish_fwd_variant_autograd,
          "Swish variant with C++ autograd by degree/source");
    m.def("swish_mul_ag_variant", &swish_mul_fwd_variant_autograd,
          "Swish(gate) * up variant with C++ autograd by degree/source");
    m.def("sigmoid_ag", &sigmoid_fwd_autograd, "Sigmoid with C++ autograd");
    m.def("tanh_ag", &tanh_fwd_autograd, "Tanh with C++ autograd");
    m.def("swish_ag", &swish_fwd_autograd, "Swish with C++ autograd");

    m.def("softcap_tanh_fwd_bf16", &softcap_tanh_fwd_bf16, py::arg("scores"), py::arg("cap") = 30.0,
          "B2 tanh softcap cap*tanh(s/cap) with the D4 BF16 tanh program");
    m.def("softcap_tanh_native_bf16", &softcap_tanh_native_bf16, py::arg("scores"),
          py::arg("cap") = 30.0, "Native softcap baseline cap*tanh(s/cap) in FP32");
    m.def("softcap_tanh_bwd_bf16", &softcap_tanh_bwd_bf16, py::arg("grad_out"), py::arg("scores"),
          py::arg("cap") = 30.0, "B2 softcap gradient from the differentiated D4 program");
    m.def("softcap_tanh_native_bwd_bf16", &softcap_tanh_native_bwd_bf16, py::arg("grad_out"),
          py::arg("scores"), py::arg("cap") = 30.0,
          "Native softcap gradient baseline grad_out * (1 - tanh^2(s/cap)) in FP32");
    m.def("exp2_d2_f32_to_bf16", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_d2_f32_bf16, at::kBFloat16); },
          "B5 exp2: FP32 range reduction + D2 safe fraction, BF16 out");
    m.def("exp2_d3_f32_to_bf16", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_d3_f32_bf16, at::kBFloat16); },
          "exp2: FP32 range reduction + FA4 D3 fraction, BF16 out");
    m.def("exp2_native_f32_to_bf16", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_native_f32_bf16, at::kBFloat16); },
          "exp2 with v_exp_f32, BF16 out");
    m.def("exp2_d2_f32", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_d2_f32, at::kFloat); },
          "B5 exp2 D2 safe fraction, FP32 out");
    m.def("exp2_d3_f32", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_d3_f32, at::kFloat); },
          "exp2 FA4 D3 fraction, FP32 out");
    m.def("exp2_native_f32", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_native_f32, at::kFloat); },
          "exp2 with v_exp_f32, FP32 out");
    m.def("exp2_pwl2_safe_f32_to_bf16",
          [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_pwl2_safe_f32_bf16, at::kBFloat16); },
          "B5 exp2: FP32 range reduction + PWL2 safe hinge (FP32), BF16 out");
    m.def("exp2_pwl2_safe_f32", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_pwl2_safe_f32, at::kFloat); },
          "B5 exp2 PWL2 safe hinge (FP32), FP32 out");
    m.def("exp2_pwl2_safe_f16_f32_to_bf16",
          [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_pwl2_safe_f16_f32_bf16, at::kBFloat16); },
          "B5 exp2: FP32 range reduction + PWL2 safe hinge on the FP16 fraction (packed FP16), BF16 out");
    m.def("exp2_pwl2_safe_f16_f32",
          [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_pwl2_safe_f16_f32, at::kFloat); },
          "B5 exp2 PWL2 safe hinge on the FP16 fraction (packed FP16), FP32 out");
    m.def("exp2_pwl2_f32_to_bf16", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_pwl2_f32_bf16, at::kBFloat16); },
          "exp2: FP32 range reduction (clamped at -126) + the two-piece PWL2 hinge (FP32), BF16 out");
    m.def("exp2_pwl2_f32", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_pwl2_f32, at::kFloat); },
          "exp2: FP32 range reduction (clamped at -126) + the two-piece PWL2 hinge (FP32), FP32 out");
    m.def("exp2_pwl1_safe_f32_to_bf16",
          [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_pwl1_safe_f32_bf16, at::kBFloat16); },
          "exp2: FP32 range reduction + D1 safe line 1 + f (FP32), BF16 out");
    m.def("exp2_pwl1_safe_f32", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_pwl1_safe_f32, at::kFloat); },
          "exp2: FP32 range reduction + D1 safe line 1 + f (FP32), FP32 out");
    m.def("exp2_pwl1_safe_f16_f32_to_bf16",
          [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_pwl1_safe_f16_f32_bf16, at::kBFloat16); },
          "exp2: FP32 range reduction + D1 safe line on the FP16 fraction, BF16 out");
    m.def("exp2_pwl1_safe_f16_f32", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_pwl1_safe_f16_f32, at::kFloat); },
          "exp2: FP32 range reduction + D1 safe line on the FP16 fraction, FP32 out");
    m.def("exp2_pwl2_safe_bf16_f32_to_bf16",
          [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_pwl2_safe_bf16_f32_bf16, at::kBFloat16); },
          "exp2: FP32 range reduction + PWL2 safe hinge in BF16, BF16 out");
    m.def("exp2_pwl2_safe_bf16_f32", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_pwl2_safe_bf16_f32, at::kFloat); },
          "exp2: FP32 range reduction + PWL2 safe hinge in BF16, FP32 out");
    m.def("exp2_d2_safe_noclamp_f32_to_bf16",
          [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_d2_safe_noclamp_f32_bf16, at::kBFloat16); },
          "exp2: FP32 range reduction + D2 safe fraction, no -127 clamp, BF16 out");
    m.def("exp2_d2_safe_noclamp_f32", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_d2_safe_noclamp_f32, at::kFloat); },
          "exp2: FP32 range reduction + D2 safe fraction, no -127 clamp, FP32 out");
    m.def("exp2_d2_safe_f16_f32_to_bf16",
          [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_d2_safe_f16_f32_bf16, at::kBFloat16); },
          "exp2: FP32 range reduction + D2 safe fraction in packed FP16, BF16 out");
    m.def("exp2_d2_safe_f16_f32", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_d2_safe_f16_f32, at::kFloat); },
          "exp2: FP32 range reduction + D2 safe fraction in packed FP16, FP32 out");
    m.def("exp2_d2_safe_bf16_f32_to_bf16",
          [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_d2_safe_bf16_f32_bf16, at::kBFloat16); },
          "exp2: FP32 range reduction + D2 safe fraction in BF16, BF16 out");
    m.def("exp2_d2_safe_bf16_f32", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_d2_safe_bf16_f32, at::kFloat); },
          "exp2: FP32 range reduction + D2 safe fraction in BF16, FP32 out");
    m.def("exp2_pwl2_f16_f32_to_bf16",
          [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_pwl2_f16_f32_bf16, at::kBFloat16); },
          "exp2: FP32 range reduction + the reference's FP16 hinge (FractionalPwl2Hinge), BF16 out");
    m.def("exp2_pwl2_f16_f32", [](at::Tensor x) { return exp2_f32_to(x, launch_exp2_pwl2_f16_f32, at::kFloat); },
          "exp2: FP32 range reduction + the reference's FP16 hinge (FractionalPwl2Hinge), FP32 out");

#define PT_DEF_SINCOS(name, T, doc) \
    m.def(#name, [](at::Tensor a) { return sincos_table(a, launch_##name, T); }, doc)
#define PT_DEF_SINCOS_COMPUTE(name, T, doc)                                             \
    m.def(#name, [](at::Tensor a, int64_t it) { return sincos_compute(a, it, launch_##name, T); }, \
          doc)
    // Paired FP32 sin/cos kernels used by the RoPE microbenchmarks.
    PT_DEF_SINCOS(sincos_native_f32, at::kFloat, "Paired native FP32 sin/cos");
    PT_DEF_SINCOS(sincos_d3_d4_f32, at::kFloat, "Paired polynomial FP32 sin D3/cos D4");
    PT_DEF_SINCOS(sincos_d3_d4_cycle_f32, at::kFloat,
                  "Paired polynomial FP32 sin D3/cos D4 with cycle-domain symmetry reduction");
    PT_DEF_SINCOS(sincos_d3_d4_magic_bias_f32, at::kFloat,
                  "Paired polynomial FP32 sin D3/cos D4 with conversion-free magic-bias reduction");
    PT_DEF_SINCOS(sincos_d5_d4_half_turn_ls_f32, at::kFloat,
                  "Paired half-turn polynomial FP32 sin D5/cos D4 with least-squares coefficients");
    PT_DEF_SINCOS(sincos_d5_d4_half_turn_sollya_f32, at::kFloat,
                  "Paired half-turn polynomial FP32 sin D5/cos D4 with Sollya coefficients");
    PT_DEF_SINCOS(sincos_d5_d4_half_turn_sollya_fast_f32, at::kFloat,
                  "Paired half-turn polynomial FP32 sin D5/cos D4 with Sollya coefficients and "
                  "one-term pi reduction");
    PT_DEF_SINCOS(sincos_d5_d4_f32, at::kFloat, "Paired polynomial FP32 sin D5/cos D4");
    PT_DEF_SINCOS(sincos_d7_d6_f32, at::kFloat, "Paired polynomial FP32 sin D7/cos D6");
    PT_DEF_SINCOS_COMPUTE(sincos_native_compute_f32, at::kFloat,
                          "Compute-saturated paired native FP32 sin/cos");
    PT_DEF_SINCOS_COMPUTE(sincos_d3_d4_compute_f32, at::kFloat,
                          "Compute-saturated polynomial FP32 sin D3/cos D4");
    PT_DEF_SINCOS_COMPUTE(sincos_d3_d4_cycle_compute_f32, at::kFloat,
                          "Compute-saturated polynomial FP32 sin D3/cos D4 with cycle-domain "
                          "symmetry reduction");
    PT_DEF_SINCOS_COMPUTE(sincos_d3_d4_magic_bias_compute_f32, at::kFloat,
                          "Compute-saturated polynomial FP32 sin D3/cos D4 with conversion-free "
                          "magic-bias reduction");
    PT_DEF_SINCOS_COMPUTE(sincos_d5_d4_half_turn_ls_compute_f32, at::kFloat,
                          "Compute-saturated half-turn polynomial FP32 sin D5/cos D4 with "
                          "least-squares coefficients");
    PT_DEF_SINCOS_COMPUTE(sincos_d5_d4_half_turn_sollya_compute_f32, at::kFloat,
                          "Compute-saturated half-turn polynomial FP32 sin D5/cos D4 with Sollya "
                          "coefficients");
    PT_DEF_SINCOS_COMPUTE(sincos_d5_d4_half_turn_sollya_fast_compute_f32, at::kFloat,
                          "Compute-saturated half-turn polynomial FP32 sin D5/cos D4 with Sollya "
                          "coefficients and one-term pi reduction");
    PT_DEF_SINCOS_COMPUTE(sincos_d5_d4_compute_f32, at::kFloat,
                          "Compute-saturated polynomial FP32 sin D5/cos D4");
    PT_DEF_SINCOS_COMPUTE(sincos_d7_d6_compute_f32, at::kFloat,
                          "Compute-saturated polynomial FP32 sin D7/cos D6");
    PT_DEF_SINCOS(sincos_native_bf16, at::kBFloat16, "Paired native sin/cos with BF16 output");
    PT_DEF_SINCOS(sincos_d3_d4_bf16, at::kBFloat16, "Paired packed-BF16 polynomial sin D3/cos D4");
    PT_DEF_SINCOS(sincos_d3_d4_quarter_turn_bf16, at::kBFloat16,
                  "Paired quarter-turn polynomial sin D3/cos D4 with packed BF16 evaluation and output");
    PT_DEF_SINCOS(sincos_d3_d4_half_turn_bf16, at::kBFloat16,
                  "Paired half-turn polynomial sin D3/cos D4 with packed BF16 evaluation and output");
    PT_DEF_SINCOS(sincos_d5_d6_half_turn_bf16, at::kBFloat16,
                  "Paired half-turn polynomial sin D5/cos D6 with packed BF16 evaluation and output");
    PT_DEF_SINCOS(sincos_d5_d4_half_turn_fp16_bf16, at::kBFloat16,
                  "Paired half-turn polynomial sin D5/cos D4 with packed FP16 evaluation and BF16 output");
    PT_DEF_SINCOS(sincos_native_fp16, at::kHalf, "Paired native sin/cos with FP16 output");
    PT_DEF_SINCOS(sincos_d3_d4_quarter_turn_fp16, at::kHalf,
                  "Paired quarter-turn polynomial sin D3/cos D4 with packed FP16 evaluation and output");
    PT_DEF_SINCOS(sincos_d3_d4_half_turn_fp16, at::kHalf,
                  "Paired half-turn polynomial sin D3/cos D4 with packed FP16 evaluation and output");
    PT_DEF_SINCOS(sincos_d5_d4_half_turn_fp16, at::kHalf,
                  "Paired half-turn polynomial sin D5/cos D4 with packed FP16 evaluation and output");
    PT_DEF_SINCOS(sincos_d5_d6_half_turn_fp16, at::kHalf,
                  "Paired half-turn polynomial sin D5/cos D6 with packed FP16 evaluation and output");
    PT_DEF_SINCOS(sincos_d7_d6_half_turn_fp16, at::kHalf,
                  "Paired half-turn polynomial sin D7/cos D6 with packed FP16 evaluation and output");
    PT_DEF_SINCOS_COMPUTE(sincos_native_bf16_compute, at::kBFloat16,
                          "Compute-saturated native sin/cos with BF16 output");
    PT_DEF_SINCOS_COMPUTE(sincos_d3_d4_bf16_compute, at::kBFloat16,
                          "Compute-saturated packed-BF16 polynomial sin D3/cos D4");
    PT_DEF_SINCOS_COMPUTE(sincos_d3_d4_quarter_turn_bf16_compute, at::kBFloat16,
                          "Compute-saturated quarter-turn polynomial sin D3/cos D4 with packed BF16 "
                          "evaluation and output");
    PT_DEF_SINCOS_COMPUTE(sincos_d3_d4_half_turn_bf16_compute, at::kBFloat16,
                          "Compute-saturated half-turn polynomial sin D3/cos D4 with packed BF16 "
                          "evaluation and output");
    PT_DEF_SINCOS_COMPUTE(sincos_d5_d6_half_turn_bf16_compute, at::kBFloat16,
                          "Compute-saturated half-turn polynomial sin D5/cos D6 with packed BF16 "
                          "evaluation and output");
    PT_DEF_SINCOS_COMPUTE(sincos_d5_d4_half_turn_fp16_bf16_compute, at::kBFloat16,
                          "Compute-saturated half-turn polynomial sin D5/cos D4 with packed FP16 "
                          "evaluation and BF16 output");
    PT_DEF_SINCOS_COMPUTE(sincos_native_fp16_compute, at::kHalf,
                          "Compute-saturated native sin/cos with FP16 output");
    PT_DEF_SINCOS_COMPUTE(sincos_d3_d4_quarter_turn_fp16_compute, at::kHalf,
                          "Compute-saturated quarter-turn polynomial sin D3/cos D4 with packed FP16 "
                          "evaluation and output");
    PT_DEF_SINCOS_COMPUTE(sincos_d3_d4_half_turn_fp16_compute, at::kHalf,
                          "Compute-saturated half-turn polynomial sin D3/cos D4 with packed FP16 "
                          "evaluation and output");
    PT_DEF_SINCOS_COMPUTE(sincos_d5_d4_half_turn_fp16_compute, at::kHalf,
                          "Compute-saturated half-turn polynomial sin D5/cos D4 with packed FP16 "
                          "evaluation and output");
    PT_DEF_SINCOS_COMPUTE(sincos_d5_d6_half_turn_fp16_compute, at::kHalf,
                          "Compute-saturated half-turn polynomial sin D5/cos D6 with packed FP16 "
                          "evaluation and output");
    PT_DEF_SINCOS_COMPUTE(sincos_d7_d6_half_turn_fp16_compute, at::kHalf,
                          "Compute-saturated half-turn polynomial sin D7/cos D6 with packed FP16 "
                          "evaluation and output");
#undef PT_DEF_SINCOS
#undef PT_DEF_SINCOS_COMPUTE
    m.def("rope_sincos_native_fp16",
          [](at::Tensor f, int64_t sl) {
              return rope_table(f, sl, at::kFloat, "frequencies", 2, launch_rope_sincos_native_fp16);
          },
          "RoPE-specific native sin/cos table generation with FP16 output");
    m.def("rope_sincos_fixed_d3_d4_fp16",
          [](at::Tensor inc, int64_t sl) {
              return rope_table(inc, sl, at::kInt, "phase_increments", 2,
                                launch_rope_sincos_fixed_d3_d4_fp16);
          },
          "RoPE-specific fixed-point phase reduction with packed FP16 sin D3/cos D4");
    m.def("rope_sincos_fixed_half_turn_d5_d6_fp16",
          [](at::Tensor inc, int64_t sl) {
              return rope_table(inc, sl, at::kInt, "phase_increments", 4,
                                launch_rope_sincos_fixed_half_turn_d5_d6_fp16);
          },
          "RoPE-specific fixed-point half-turn reduction with FP16 sin D5/cos D6");
    m.def("rope_sincos_fixed_lut_fp16",
          [](at::Tensor inc, at::Tensor table, int64_t sl) {
              return rope_sincos_fixed_lut_fp16(inc, table, sl, -1);
          },
          "RoPE-specific fixed-point phase lookup with packed FP16 linear correction");
    m.def("rope_sincos_native_fp16_compute",
          [](at::Tensor f, int64_t sl, int64_t it) {
              return rope_table_compute(f, sl, it, at::kFloat, "frequencies", 2,
                                        launch_rope_sincos_native_fp16_compute);
          },
          "Compute-saturated RoPE-specific native sin/cos with FP16 output");
    m.def("rope_sincos_fixed_d3_d4_fp16_compute",
          [](at::Tensor inc, int64_t sl, int64_t it) {
              return rope_table_compute(inc, sl, it, at::kInt, "phase_increments", 2,
                                        launch_rope_sincos_fixed_d3_d4_fp16_compute);
          },
          "Compute-saturated RoPE-specific fixed-point reduction with packed FP16 sin D3/cos D4");
    m.def("rope_sincos_fixed_half_turn_d5_d6_fp16_compute",
          [](at::Tensor inc, int64_t sl, int64_t it) {
              return rope_table_compute(inc, sl, it, at::kInt, "phase_increments", 4,
                                        launch_rope_sincos_fixed_half_turn_d5_d6_fp16_compute);
          },
          "Compute-saturated RoPE-specific fixed-point half-turn reduction with FP16 sin D5/cos D6");
    m.def("rope_sincos_fixed_lut_fp16_compute",
          [](at::Tensor inc, at::Tensor table, int64_t sl, int64_t it) {
              TORCH_CHECK(it > 0, "iterations must be positive");
              return rope_sincos_fixed_lut_fp16(inc, table, sl, it);
          },
          "Compute-saturated RoPE-specific fixed-point phase lookup with packed FP16 linear "
          "correction");
    m.def("rope_apply_cached_fp16",
          [](at::Tensor q, at::Tensor k, at::Tensor table) {
              return rope_apply(q, k, table, at::kHalf, at::kHalf, "rope_table",
                                launch_rope_apply_cached_fp16);
          },
          "Fused cached-table FP16 Q/K rotary embedding and transpose");
    m.def("rope_apply_fixed_half_turn_d5_d6_fp16",
          [](at::Tensor q, at::Tensor k, at::Tensor inc) {
              return rope_apply(q, k, inc, at::kHalf, at::kInt, "phase_increments",
                                launch_rope_apply_fixed_half_turn_d5_d6_fp16);
          },
          "Fused polynomial FP16 Q/K rotary embedding and transpose");
    m.def("rope_apply_native_fp16",
          [](at::Tensor q, at::Tensor k, at::Tensor freq) {
              return rope_apply(q, k, freq, at::kHalf, at::kFloat, "frequencies",
                                launch_rope_apply_native_fp16);
          },
          "Fused native-SFU FP16 Q/K rotary embedding and transpose");
    m.def("rope_apply_fixed_half_turn_d5_d6_bf16",
          [](at::Tensor q, at::Tensor k, at::Tensor inc) {
              return rope_apply(q, k, inc, at::kBFloat16, at::kInt, "phase_increments",
                                launch_rope_apply_fixed_half_turn_d5_d6_bf16);
          },
          "Fused polynomial BF16 Q/K rotary embedding and transpose");
    m.def("rope_apply_native_bf16",
          [](at::Tensor q, at::Tensor k, at::Tensor freq) {
              return rope_apply(q, k, freq, at::kBFloat16, at::kFloat, "frequencies",
                                launch_rope_apply_native_bf16);
          },
          "Fused native BF16 Q/K rotary embedding and transpose");

    // fused attention
    m.def("flash_attn_fwd_bf16", &flash_attn_fwd_bf16, py::arg("q"), py::arg("k"), py::arg("v"),
          py::arg("mode"), py::arg("exp2_route") = 4, py::arg("causal") = true,
          py::arg("softmax_scale"), py::arg("softcap") = 0.0, py::arg("sigmoid_bias") = 0.0,
          py::arg("valid_keys") = -1,
          "Fused attention forward with the score programs in the tile loop; "
          "q [B,S,Hq,D], k/v [B,S,Hkv,D] BF16 (D 64 or 128, any S) -> [out [B,S,Hq,D], lse [B,Hq,S] FP32]; "
          "valid_keys >= 1 masks keys from that index on (operands padded at the end)");
    m.def("flash_attn_bwd_bf16", &flash_attn_bwd_bf16, py::arg("q"), py::arg("k"), py::arg("v"),
          py::arg("out"), py::arg("dout"), py::arg("lse"), py::arg("mode"), py::arg("grad") = 0,
          py::arg("exp2_route") = 0, py::arg("causal") = true, py::arg("softmax_scale"),
          py::arg("softcap") = 0.0, py::arg("sigmoid_bias") = 0.0,
          "Fused attention backward -> [dq [B,S,Hq,D], dk, dv [B,S,Hkv,D]] BF16");

    // RoPE reference evaluator (sfu_repro.rope.polynomial_sincos on the device)
    m.def("polynomial_sincos_f32", &polynomial_sincos_f32, py::arg("angles"),
          py::arg("sin_coefficients"), py::arg("cos_coefficients"), py::arg("accurate") = true,
          "Quarter-turn reduction (FP64 or FP32 Cody-Waite) and paired parity polynomials "
          "in FP32; returns [cos, sin]");
    m.def("reduce_to_quarter_turn_f32", &reduce_to_quarter_turn_f32, py::arg("angles"),
          py::arg("accurate") = true, "Quarter-turn reduction; returns [reduced (FP32), quadrant (int64)]");
    m.def("evaluate_reduced_sincos_f32", &evaluate_reduced_sincos_f32, py::arg("reduced"),
          py::arg("sin_coefficients"), py::arg("cos_coefficients"),
          "Paired parity polynomials on reduced FP32 arguments; returns [sin, cos]");

    // FP16 experiments
#define PT_DEF_FP16_FWD(name, doc) \
    m.def(#name, [](at::Tensor x) { return fp16_fwd(x, launch_##name##_kernel); }, doc)
#define PT_DEF_FP16_BWD(name, doc)                                                       \
    m.def(#name, [](at::Tensor go, at::Tensor x) { return fp16_bwd(go, x, launch_##name##_kernel); }, \
          doc)
#define PT_DEF_FUSED(name, doc)                                                          \
    m.def(#name, [](at::Tensor x, at::Tensor go) { return fp16_fused(x, go, launch_##name##_kernel); }, \
          doc)
#define PT_DEF_FWD_DERIV(name, doc) \
    m.def(#name, [](at::Tensor x) { return fp16_fwd_deriv(x, launch_##name##_kernel); }, doc)
    PT_DEF_FP16_FWD(sigmoid_fwd_hybrid, "Sigmoid FWD hybrid 1SFU+3Poly");
    PT_DEF_FP16_FWD(tanh_fwd_hybrid, "Tanh FWD hybrid 1SFU+3Poly");
    PT_DEF_FP16_FWD(swish_fwd_hybrid, "Swish FWD hybrid 1SFU+3Poly");
    PT_DEF_FP16_BWD(sigmoid_bwd_hybrid, "Sigmoid BWD hybrid 1SFU+3Poly");
    PT_DEF_FP16_BWD(tanh_bwd_hybrid, "Tanh BWD hybrid 1SFU+3Poly");
    PT_DEF_FP16_BWD(swish_bwd_hybrid, "Swish BWD hybrid 1SFU+3Poly");
    PT_DEF_FUSED(sigmoid_fused, "Sigmoid fused FWD+BWD");
    PT_DEF_FUSED(tanh_fused, "Tanh fused FWD+BWD");
    PT_DEF_FUSED(swish_fused, "Swish fused FWD+BWD");
    PT_DEF_FWD_DERIV(sigmoid_fwd_deriv_alg, "Sigmoid FWD+deriv (poly+algebraic)");
    PT_DEF_FWD_DERIV(sigmoid_fwd_deriv_poly, "Sigmoid FWD+deriv (poly+poly)");
    PT_DEF_FWD_DERIV(tanh_fwd_deriv_alg, "Tanh FWD+deriv (poly+algebraic)");
    PT_DEF_FWD_DERIV(tanh_fwd_deriv_poly, "Tanh FWD+deriv (poly+poly)");
    PT_DEF_FWD_DERIV(swish_fwd_deriv, "Swish FWD+deriv (shared sigmoid)");
    PT_DEF_FWD_DERIV(swish_fwd_deriv_poly, "Swish FWD+deriv (poly+poly)");
#undef PT_DEF_FP16_FWD
#undef PT_DEF_FP16_BWD
#undef PT_DEF_FUSED
#undef PT_DEF_FWD_DERIV
    m.def("multiply", &multiply, "Element-wise multiply (for backward)");

    m.def("flash_sigmoid_direct_d3_d4_bf16", &flash_sigmoid_direct_d3_d4,
          "B3 deployed direct-D3 probability and factored-D4 derivative (BF16 out)");
    m.def("flash_sigmoid_exp2_d2_bf16", &flash_sigmoid_exp2_d2,
          "B3-D2 sigmoid via range-reduced degree-2 exp2 (probability, derivative), BF16");
    m.def("flash_sigmoid_direct_d3_bf16", &flash_sigmoid_direct_d3,
          "B3 deployed direct-D3 probability (BF16)");
    m.def("flash_sigmoid_native_bf16", &flash_sigmoid_native,
          "B3 hardware control: sigmoid(s - ln 4096) and p (1 - p) via v_exp_f32 / v_rcp_f32");
}
