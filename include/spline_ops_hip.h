/*
 * spline_ops_hip.h -- C ABI of the MI355X (gfx950) polynomial transcendental
 * kernels.  Plain pointers, 64-bit element counts and an opaque HIP stream;
 * no torch types.  Link against libspline_hip.so.
 *
 * Every entry point
 *   - launches asynchronously on `stream` (a hipStream_t; NULL = the null
 *     stream) and never synchronises or allocates;
 *   - returns 0 (hipSuccess) or the hipError_t of the failed launch, or
 *     hipErrorInvalidValue (1) for a negative size or a NULL pointer with a
 *     non-zero size;
 *   - accepts any element count (a 16-byte vector path runs when all pointers
 *     are 16-byte aligned; an element path covers the rest with identical
 *     results) and returns 0 without launching when the count is 0.
 * 16-bit tensors are passed as raw storage: `_bf16` entry points read and
 * write bfloat16, the others float16 (the reference's naming).
 *
 * Names and argument order follow the reference's internal launcher ABI,
 * declared in autonumerics_zero/spline_ops/spline_ops.cpp:14-288 and defined
 * in spline_kernels.cu:1174-1482 (FP16), spline_kernels_bf16.cu:926-1283
 * (BF16) and sincos_kernels.cu:2123-2978.  Differences: `int64_t` counts
 * instead of `int` (the reference silently truncates above 2^31 elements),
 * a returned status instead of `void`, and `void*` for the stream.
 */
#ifndef SPLINE_OPS_HIP_H
#define SPLINE_OPS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- unary activations: out = F(in) ------------------------------------
 * Replaces launch_{sigmoid,tanh,swish}_fwd_d{3..6}_kernel{,_bf16}
 * (spline_ops.cpp:16-60, 141-168; spline_kernels.cu:1176-1230,
 * spline_kernels_bf16.cu:928-1010) and the native SiLU launcher
 * launch_swish_fwd_native_kernel{,_bf16} (spline_kernels.cu:1239,
 * spline_kernels_bf16.cu:1013).  launch_{sigmoid,tanh}_fwd_native_kernel*
 * are the hardware-transcendental baselines of the isolated sweep
 * (the reference times torch.sigmoid/torch.tanh there,
 * autonumerics_zero/experiments/benchmark_report_function_speed.py:107-163). */
#define SPLINE_HIP_UNARY_LAUNCHERS(X)                                          \
    X(launch_sigmoid_fwd_d3_kernel) X(launch_sigmoid_fwd_d4_kernel)            \
    X(launch_sigmoid_fwd_d5_kernel) X(launch_sigmoid_fwd_d6_kernel)            \
    X(launch_sigmoid_fwd_d3_kernel_bf16) X(launch_sigmoid_fwd_d4_kernel_bf16)  \
    X(launch_sigmoid_fwd_d5_kernel_bf16) X(launch_sigmoid_fwd_d6_kernel_bf16)  \
    X(launch_tanh_fwd_d3_kernel) X(launch_tanh_fwd_d4_kernel)                  \
    X(launch_tanh_fwd_d5_kernel) X(launch_tanh_fwd_d6_kernel)                  \
    X(launch_tanh_fwd_d3_kernel_bf16) X(launch_tanh_fwd_d4_kernel_bf16)        \
    X(launch_tanh_fwd_d5_kernel_bf16) X(launch_tanh_fwd_d6_kernel_bf16)        \
    X(launch_swish_fwd_d3_kernel) X(launch_swish_fwd_d4_kernel)                \
    X(launch_swish_fwd_d5_kernel) X(launch_swish_fwd_d6_kernel)                \
    X(launch_swish_fwd_d3_kernel_bf16) X(launch_swish_fwd_d4_kernel_bf16)      \
    X(launch_swish_fwd_d5_kernel_bf16) X(launch_swish_fwd_d6_kernel_bf16)      \
    X(launch_swish_fwd_native_kernel) X(launch_swish_fwd_native_kernel_bf16)   \
    X(launch_sigmoid_fwd_native_kernel) X(launch_sigmoid_fwd_native_kernel_bf16) \
    X(launch_tanh_fwd_native_kernel) X(launch_tanh_fwd_native_kernel_bf16)

/* ---- derivative programs: grad_in = grad_out * F'(in) ------------------
 * Replaces launch_{sigmoid,tanh,swish}_bwd_d{3..6}_kernel{,_bf16}
 * (spline_ops.cpp:62-108; spline_kernels.cu:1196-1262,
 * spline_kernels_bf16.cu:952-1045), launch_swish_bwd_native_kernel{,_bf16},
 * and the algebraic launch_{sigmoid,tanh}_bwd_alg_kernel{,_bf16}
 * (spline_kernels.cu:1387-1392), whose `in` is the cached forward output y. */
#define SPLINE_HIP_BINARY_LAUNCHERS(X)                                         \
    X(launch_sigmoid_bwd_d3_kernel) X(launch_sigmoid_bwd_d4_kernel)            \
    X(launch_sigmoid_bwd_d5_kernel) X(launch_sigmoid_bwd_d6_kernel)            \
    X(launch_sigmoid_bwd_d3_kernel_bf16) X(launch_sigmoid_bwd_d4_kernel_bf16)  \
    X(launch_sigmoid_bwd_d5_kernel_bf16) X(launch_sigmoid_bwd_d6_kernel_bf16)  \
    X(launch_tanh_bwd_d3_kernel) X(launch_tanh_bwd_d4_kernel)                  \
    X(launch_tanh_bwd_d5_kernel) X(launch_tanh_bwd_d6_kernel)                  \
    X(launch_tanh_bwd_d3_kernel_bf16) X(launch_tanh_bwd_d4_kernel_bf16)        \
    X(launch_tanh_bwd_d5_kernel_bf16) X(launch_tanh_bwd_d6_kernel_bf16)        \
    X(launch_swish_bwd_d3_kernel) X(launch_swish_bwd_d4_kernel)                \
    X(launch_swish_bwd_d5_kernel) X(launch_swish_bwd_d6_kernel)                \
    X(launch_swish_bwd_d3_kernel_bf16) X(launch_swish_bwd_d4_kernel_bf16)      \
    X(launch_swish_bwd_d5_kernel_bf16) X(launch_swish_bwd_d6_kernel_bf16)      \
    X(launch_swish_bwd_native_kernel) X(launch_swish_bwd_native_kernel_bf16)   \
    X(launch_sigmoid_bwd_alg_kernel) X(launch_sigmoid_bwd_alg_kernel_bf16)     \
    X(launch_tanh_bwd_alg_kernel) X(launch_tanh_bwd_alg_kernel_bf16)

/* ---- SwiGLU: out = F(gate) * up ----------------------------------------
 * Replaces launch_swish_mul_fwd_{native,d3..d6}_kernel{,_bf16}
 * (spline_kernels.cu:1255-1268, spline_kernels_bf16.cu:1030-1044). */
#define SPLINE_HIP_SWISH_MUL_LAUNCHERS(X)                                      \
    X(launch_swish_mul_fwd_native_kernel) X(launch_swish_mul_fwd_d3_kernel)    \
    X(launch_swish_mul_fwd_d4_kernel) X(launch_swish_mul_fwd_d5_kernel)        \
    X(launch_swish_mul_fwd_d6_kernel)                                          \
    X(launch_swish_mul_fwd_native_kernel_bf16) X(launch_swish_mul_fwd_d3_kernel_bf16) \
    X(launch_swish_mul_fwd_d4_kernel_bf16) X(launch_swish_mul_fwd_d5_kernel_bf16) \
    X(launch_swish_mul_fwd_d6_kernel_bf16)

/* ---- SwiGLU backward: grad_gate = go*up*F'(gate), grad_up = go*F(gate) ---
 * Replaces launch_swish_mul_bwd_{native,d3..d6}_kernel{,_bf16}
 * (spline_kernels.cu:1270-1283, spline_kernels_bf16.cu:1047-1062; the BF16
 * degree-3 entry uses the algebraic derivative, :255-265,375-382). */
#define SPLINE_HIP_SWISH_MUL_BWD_LAUNCHERS(X)                                  \
    X(launch_swish_mul_bwd_native_kernel) X(launch_swish_mul_bwd_d3_kernel)    \
    X(launch_swish_mul_bwd_d4_kernel) X(launch_swish_mul_bwd_d5_kernel)        \
    X(launch_swish_mul_bwd_d6_kernel)                                          \
    X(launch_swish_mul_bwd_native_kernel_bf16) X(launch_swish_mul_bwd_d3_kernel_bf16) \
    X(launch_swish_mul_bwd_d4_kernel_bf16) X(launch_swish_mul_bwd_d5_kernel_bf16) \
    X(launch_swish_mul_bwd_d6_kernel_bf16)

/* ---- packed SwiGLU on [rows, 2H] = [gate | up] -> [rows, H] -------------
 * Replaces launch_swish_mul_packed_fwd_{native,d3..d6}_kernel{,_bf16}
 * (spline_kernels.cu:1285-1302, spline_kernels_bf16.cu:1065-1083). */
#define SPLINE_HIP_PACKED_FWD_LAUNCHERS(X)                                     \
    X(launch_swish_mul_packed_fwd_native_kernel) X(launch_swish_mul_packed_fwd_d3_kernel) \
    X(launch_swish_mul_packed_fwd_d4_kernel) X(launch_swish_mul_packed_fwd_d5_kernel) \
    X(launch_swish_mul_packed_fwd_d6_kernel)                                   \
    X(launch_swish_mul_packed_fwd_native_kernel_bf16) X(launch_swish_mul_packed_fwd_d3_kernel_bf16) \
    X(launch_swish_mul_packed_fwd_d4_kernel_bf16) X(launch_swish_mul_packed_fwd_d5_kernel_bf16) \
    X(launch_swish_mul_packed_fwd_d6_kernel_bf16)

/* ---- packed SwiGLU backward: grad_packed [rows, 2H] from grad_out [rows, H]
 * Replaces launch_swish_mul_packed_bwd_{native,d3..d6}_kernel{,_bf16}
 * (spline_kernels.cu:1304-1320, spline_kernels_bf16.cu:1086-1101). */
#define SPLINE_HIP_PACKED_BWD_LAUNCHERS(X)                                     \
    X(launch_swish_mul_packed_bwd_native_kernel) X(launch_swish_mul_packed_bwd_d3_kernel) \
    X(launch_swish_mul_packed_bwd_d4_kernel) X(launch_swish_mul_packed_bwd_d5_kernel) \
    X(launch_swish_mul_packed_bwd_d6_kernel)                                   \
    X(launch_swish_mul_packed_bwd_native_kernel_bf16) X(launch_swish_mul_packed_bwd_d3_kernel_bf16) \
    X(launch_swish_mul_packed_bwd_d4_kernel_bf16) X(launch_swish_mul_packed_bwd_d5_kernel_bf16) \
    X(launch_swish_mul_packed_bwd_d6_kernel_bf16)

#define SPLINE_HIP_DECLARE_UNARY(name) \
    int name(void* out, const void* in, int64_t size, void* stream);
#define SPLINE_HIP_DECLARE_BINARY(name) \
    int name(void* grad_in, const void* grad_out, const void* in, int64_t size, void* stream);
#define SPLINE_HIP_DECLARE_SWISH_MUL(name) \
    int name(void* out, const void* gate, const void* up, int64_t size, void* stream);
#define SPLINE_HIP_DECLARE_SWISH_MUL_BWD(name)                                \
    int name(void* grad_gate, void* grad_up, const void* grad_out,            \
             const void* gate, const void* up, int64_t size, void* stream);
#define SPLINE_HIP_DECLARE_PACKED_FWD(name) \
    int name(void* out, const void* packed, int64_t rows, int64_t hidden_size, void* stream);
#define SPLINE_HIP_DECLARE_PACKED_BWD(name)                                   \
    int name(void* grad_packed, const void* grad_out, const void* packed,     \
             int64_t rows, int64_t hidden_size, void* stream);

SPLINE_HIP_UNARY_LAUNCHERS(SPLINE_HIP_DECLARE_UNARY)
SPLINE_HIP_BINARY_LAUNCHERS(SPLINE_HIP_DECLARE_BINARY)
SPLINE_HIP_SWISH_MUL_LAUNCHERS(SPLINE_HIP_DECLARE_SWISH_MUL)
SPLINE_HIP_SWISH_MUL_BWD_LAUNCHERS(SPLINE_HIP_DECLARE_SWISH_MUL_BWD)
SPLINE_HIP_PACKED_FWD_LAUNCHERS(SPLINE_HIP_DECLARE_PACKED_FWD)
SPLINE_HIP_PACKED_BWD_LAUNCHERS(SPLINE_HIP_DECLARE_PACKED_BWD)

/* ---- B3: deployed direct-D3 sigmoid with factored-D4 derivative ---------
 * No C launcher exists in the reference: the program is FA4 inline PTX
 * (extras/paper/manuscript/main.tex:1041-1117), emulated on the CPU by
 * scripts/audit_b3_deployed_fit.py:341-366.  y = sigmoid-attention
 * probability for sequence length 4096, dy = its derivative.  The `_f32`
 * form takes FP32 scores and rounds them to BF16 first (cvt.rn.bf16x2.f32). */
int launch_flash_sigmoid_direct_d3_d4_bf16(void* y, void* dy, const void* scores,
                                           int64_t size, void* stream);
int launch_flash_sigmoid_direct_d3_d4_f32_bf16(void* y, void* dy, const void* scores,
                                               int64_t size, void* stream);
/* Forward only (the first listing, main.tex:1041-1070). */
int launch_flash_sigmoid_direct_d3_bf16(void* y, const void* scores, int64_t size,
                                        void* stream);

/* ---- device/launch introspection --------------------------------------- */
/* Number of compute units of the current device and the grid the
 * elementwise launchers use for `size` 16-bit elements and `streams` tensors
 * (inputs + outputs).  For tests and benchmarks. */
int spline_hip_grid_for(int64_t size, int streams, int64_t* grid_out, int* cus_out);

#ifdef __cplusplus
}
#endif
#endif /* SPLINE_OPS_HIP_H */
