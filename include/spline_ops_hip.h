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
    X(launch_tanh_fwd_native_kernel) X(launch_tanh_fwd_native_kernel_bf16)    \
    X(launch_gelu_fwd_d3_kernel) X(launch_gelu_fwd_d4_kernel)                  \
    X(launch_gelu_fwd_d5_kernel) X(launch_gelu_fwd_d6_kernel)                  \
    X(launch_gelu_fwd_d3_kernel_bf16) X(launch_gelu_fwd_d4_kernel_bf16)        \
    X(launch_gelu_fwd_d5_kernel_bf16) X(launch_gelu_fwd_d6_kernel_bf16)        \
    SPLINE_HIP_UNARY_SOLLYA_LAUNCHERS(X)

/* GELU (x * Phi(x) with Phi = 0.5 + sign * t*H(t)): replaces
 * launch_gelu_fwd_d{3..6}_kernel{,_bf16} (spline_ops.cpp:129-132,266-269;
 * spline_kernels.cu:1338-1350, spline_kernels_bf16.cu:1119-1131).
 * BF16 Sollya coefficient set (coeff_source_id 1): replaces
 * launch_{sigmoid,swish,gelu}_fwd_d{3..6}_kernel_bf16_sollya
 * (spline_ops.cpp:180-183,256-259,276-279; spline_kernels_bf16.cu:1146-1239). */
#define SPLINE_HIP_UNARY_SOLLYA_LAUNCHERS(X)                                   \
    X(launch_sigmoid_fwd_d3_kernel_bf16_sollya) X(launch_sigmoid_fwd_d4_kernel_bf16_sollya) \
    X(launch_sigmoid_fwd_d5_kernel_bf16_sollya) X(launch_sigmoid_fwd_d6_kernel_bf16_sollya) \
    X(launch_swish_fwd_d3_kernel_bf16_sollya) X(launch_swish_fwd_d4_kernel_bf16_sollya) \
    X(launch_swish_fwd_d5_kernel_bf16_sollya) X(launch_swish_fwd_d6_kernel_bf16_sollya) \
    X(launch_gelu_fwd_d3_kernel_bf16_sollya) X(launch_gelu_fwd_d4_kernel_bf16_sollya) \
    X(launch_gelu_fwd_d5_kernel_bf16_sollya) X(launch_gelu_fwd_d6_kernel_bf16_sollya)

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
    X(launch_tanh_bwd_alg_kernel) X(launch_tanh_bwd_alg_kernel_bf16)         \
    X(launch_gelu_bwd_d3_kernel) X(launch_gelu_bwd_d4_kernel)                  \
    X(launch_gelu_bwd_d5_kernel) X(launch_gelu_bwd_d6_kernel)                  \
    X(launch_gelu_bwd_d3_kernel_bf16) X(launch_gelu_bwd_d4_kernel_bf16)        \
    X(launch_gelu_bwd_d5_kernel_bf16) X(launch_gelu_bwd_d6_kernel_bf16)        \
    SPLINE_HIP_BINARY_SOLLYA_LAUNCHERS(X)

/* GELU derivative: replaces launch_gelu_bwd_d{3..6}_kernel{,_bf16}
 * (spline_ops.cpp:135-138,272-275; spline_kernels.cu:1352-1364,
 * spline_kernels_bf16.cu:1133-1145).  Sollya set: replaces
 * launch_{sigmoid,swish,gelu}_bwd_d{3..6}_kernel_bf16_sollya
 * (spline_ops.cpp:190-193,260-263,280-283). */
#define SPLINE_HIP_BINARY_SOLLYA_LAUNCHERS(X)                                  \
    X(launch_sigmoid_bwd_d3_kernel_bf16_sollya) X(launch_sigmoid_bwd_d4_kernel_bf16_sollya) \
    X(launch_sigmoid_bwd_d5_kernel_bf16_sollya) X(launch_sigmoid_bwd_d6_kernel_bf16_sollya) \
    X(launch_swish_bwd_d3_kernel_bf16_sollya) X(launch_swish_bwd_d4_kernel_bf16_sollya) \
    X(launch_swish_bwd_d5_kernel_bf16_sollya) X(launch_swish_bwd_d6_kernel_bf16_sollya) \
    X(launch_gelu_bwd_d3_kernel_bf16_sollya) X(launch_gelu_bwd_d4_kernel_bf16_sollya) \
    X(launch_gelu_bwd_d5_kernel_bf16_sollya) X(launch_gelu_bwd_d6_kernel_bf16_sollya)

/* ---- SwiGLU: out = F(gate) * up ----------------------------------------
 * Replaces launch_swish_mul_fwd_{native,d3..d6}_kernel{,_bf16}
 * (spline_kernels.cu:1255-1268, spline_kernels_bf16.cu:1030-1044) and the
 * Sollya set's launch_swish_mul_fwd_d{3..6}_kernel_bf16_sollya
 * (spline_ops.cpp:218-221; spline_kernels_bf16.cu:1174-1186). */
#define SPLINE_HIP_SWISH_MUL_LAUNCHERS(X)                                      \
    X(launch_swish_mul_fwd_native_kernel) X(launch_swish_mul_fwd_d3_kernel)    \
    X(launch_swish_mul_fwd_d4_kernel) X(launch_swish_mul_fwd_d5_kernel)        \
    X(launch_swish_mul_fwd_d6_kernel)                                          \
    X(launch_swish_mul_fwd_native_kernel_bf16) X(launch_swish_mul_fwd_d3_kernel_bf16) \
    X(launch_swish_mul_fwd_d4_kernel_bf16) X(launch_swish_mul_fwd_d5_kernel_bf16) \
    X(launch_swish_mul_fwd_d6_kernel_bf16)                                     \
    X(launch_swish_mul_fwd_d3_kernel_bf16_sollya) X(launch_swish_mul_fwd_d4_kernel_bf16_sollya) \
    X(launch_swish_mul_fwd_d5_kernel_bf16_sollya) X(launch_swish_mul_fwd_d6_kernel_bf16_sollya)

/* ---- SwiGLU backward: grad_gate = go*up*F'(gate), grad_up = go*F(gate) ---
 * Replaces launch_swish_mul_bwd_{native,d3..d6}_kernel{,_bf16}
 * (spline_kernels.cu:1270-1283, spline_kernels_bf16.cu:1047-1062; the BF16
 * degree-3 entry uses the algebraic derivative, :255-265,375-382) and
 * launch_swish_mul_bwd_d{3..6}_kernel_bf16_sollya (spline_ops.cpp:227-230;
 * spline_kernels_bf16.cu:1187-1198: the program pair at every degree). */
#define SPLINE_HIP_SWISH_MUL_BWD_LAUNCHERS(X)                                  \
    X(launch_swish_mul_bwd_native_kernel) X(launch_swish_mul_bwd_d3_kernel)    \
    X(launch_swish_mul_bwd_d4_kernel) X(launch_swish_mul_bwd_d5_kernel)        \
    X(launch_swish_mul_bwd_d6_kernel)                                          \
    X(launch_swish_mul_bwd_native_kernel_bf16) X(launch_swish_mul_bwd_d3_kernel_bf16) \
    X(launch_swish_mul_bwd_d4_kernel_bf16) X(launch_swish_mul_bwd_d5_kernel_bf16) \
    X(launch_swish_mul_bwd_d6_kernel_bf16)                                     \
    X(launch_swish_mul_bwd_d3_kernel_bf16_sollya) X(launch_swish_mul_bwd_d4_kernel_bf16_sollya) \
    X(launch_swish_mul_bwd_d5_kernel_bf16_sollya) X(launch_swish_mul_bwd_d6_kernel_bf16_sollya)

/* ---- packed SwiGLU on [rows, 2H] = [gate | up] -> [rows, H] -------------
 * Replaces launch_swish_mul_packed_fwd_{native,d3..d6}_kernel{,_bf16}
 * (spline_kernels.cu:1285-1302, spline_kernels_bf16.cu:1065-1083) and
 * launch_swish_mul_packed_fwd_d{3..6}_kernel_bf16_sollya (spline_ops.cpp:235-238). */
#define SPLINE_HIP_PACKED_FWD_LAUNCHERS(X)                                     \
    X(launch_swish_mul_packed_fwd_native_kernel) X(launch_swish_mul_packed_fwd_d3_kernel) \
    X(launch_swish_mul_packed_fwd_d4_kernel) X(launch_swish_mul_packed_fwd_d5_kernel) \
    X(launch_swish_mul_packed_fwd_d6_kernel)                                   \
    X(launch_swish_mul_packed_fwd_native_kernel_bf16) X(launch_swish_mul_packed_fwd_d3_kernel_bf16) \
    X(launch_swish_mul_packed_fwd_d4_kernel_bf16) X(launch_swish_mul_packed_fwd_d5_kernel_bf16) \
    X(launch_swish_mul_packed_fwd_d6_kernel_bf16)                              \
    X(launch_swish_mul_packed_fwd_d3_kernel_bf16_sollya) X(launch_swish_mul_packed_fwd_d4_kernel_bf16_sollya) \
    X(launch_swish_mul_packed_fwd_d5_kernel_bf16_sollya) X(launch_swish_mul_packed_fwd_d6_kernel_bf16_sollya)

/* ---- packed SwiGLU backward: grad_packed [rows, 2H] from grad_out [rows, H]
 * Replaces launch_swish_mul_packed_bwd_{native,d3..d6}_kernel{,_bf16}
 * (spline_kernels.cu:1304-1320, spline_kernels_bf16.cu:1086-1101) and
 * launch_swish_mul_packed_bwd_d{3..6}_kernel_bf16_sollya (spline_ops.cpp:244-247). */
#define SPLINE_HIP_PACKED_BWD_LAUNCHERS(X)                                     \
    X(launch_swish_mul_packed_bwd_native_kernel) X(launch_swish_mul_packed_bwd_d3_kernel) \
    X(launch_swish_mul_packed_bwd_d4_kernel) X(launch_swish_mul_packed_bwd_d5_kernel) \
    X(launch_swish_mul_packed_bwd_d6_kernel)                                   \
    X(launch_swish_mul_packed_bwd_native_kernel_bf16) X(launch_swish_mul_packed_bwd_d3_kernel_bf16) \
    X(launch_swish_mul_packed_bwd_d4_kernel_bf16) X(launch_swish_mul_packed_bwd_d5_kernel_bf16) \
    X(launch_swish_mul_packed_bwd_d6_kernel_bf16)                              \
    X(launch_swish_mul_packed_bwd_d3_kernel_bf16_sollya) X(launch_swish_mul_packed_bwd_d4_kernel_bf16_sollya) \
    X(launch_swish_mul_packed_bwd_d5_kernel_bf16_sollya) X(launch_swish_mul_packed_bwd_d6_kernel_bf16_sollya)

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

/* ---- FP16 experiment kernels (spline_ops.cpp:1573-1926 binding;
 * spline_kernels.cu:776-1168, 1394-1480) --------------------------------------
 * Hybrid (replace launch_{sigmoid,tanh,swish}_{fwd,bwd}_hybrid_kernel,
 * :1394-1414): in tensors of at least 8192 elements, a multiple of 8, the
 * first pair of every 8 elements goes through the hardware transcendental
 * program (v_exp_f32 / v_rcp_f32, rounded to FP16) and the other three
 * pairs through the polynomial (forward: sigmoid/tanh/SiLU D3; backward:
 * grad_out * sigmoid/tanh D4 even or SiLU D4 odd); smaller or ragged tensors
 * are all polynomial, as in the reference. */
#define SPLINE_HIP_HYBRID_FWD_LAUNCHERS(X)                                      \
    X(launch_sigmoid_fwd_hybrid_kernel) X(launch_tanh_fwd_hybrid_kernel)        \
    X(launch_swish_fwd_hybrid_kernel)
#define SPLINE_HIP_HYBRID_BWD_LAUNCHERS(X)                                      \
    X(launch_sigmoid_bwd_hybrid_kernel) X(launch_tanh_bwd_hybrid_kernel)        \
    X(launch_swish_bwd_hybrid_kernel)
SPLINE_HIP_HYBRID_FWD_LAUNCHERS(SPLINE_HIP_DECLARE_UNARY)
SPLINE_HIP_HYBRID_BWD_LAUNCHERS(SPLINE_HIP_DECLARE_BINARY)
/* Fused forward + backward (replace launch_{sigmoid,tanh,swish}_fused_kernel,
 * :1416-1443): y = D3(x) and grad_in = grad_out * alg(y) (sigmoid y(1-y),
 * tanh 1-y^2); SiLU: y = SILU_D3(x), grad_in = grad_out * SILU'_D4(x). */
#define SPLINE_HIP_FUSED_LAUNCHERS(X)                                           \
    X(launch_sigmoid_fused_kernel) X(launch_tanh_fused_kernel) X(launch_swish_fused_kernel)
#define SPLINE_HIP_DECLARE_FUSED(name)                                          \
    int name(void* y, void* grad_in, const void* x, const void* grad_out, int64_t size, void* stream);
SPLINE_HIP_FUSED_LAUNCHERS(SPLINE_HIP_DECLARE_FUSED)
/* Forward with derivative, (y, f'(x)) (replace launch_*_fwd_deriv*_kernel,
 * :1448-1474): _alg derives from y; _poly evaluates the D4 derivative
 * program of x; swish_fwd_deriv shares one sigmoid D3: y = x*s,
 * dy = s * fma(x, 1 - s, 1).  Every size gets the vector-path result (the
 * reference's small-size fallback of _alg returns y * alg(y) and that of
 * swish_fwd_deriv switches to the SiLU D3/D4 programs). */
#define SPLINE_HIP_FWD_DERIV_LAUNCHERS(X)                                       \
    X(launch_sigmoid_fwd_deriv_alg_kernel) X(launch_sigmoid_fwd_deriv_poly_kernel) \
    X(launch_tanh_fwd_deriv_alg_kernel) X(launch_tanh_fwd_deriv_poly_kernel)    \
    X(launch_swish_fwd_deriv_kernel) X(launch_swish_fwd_deriv_poly_kernel)
#define SPLINE_HIP_DECLARE_FWD_DERIV(name) \
    int name(void* y, void* dy, const void* x, int64_t size, void* stream);
SPLINE_HIP_FWD_DERIV_LAUNCHERS(SPLINE_HIP_DECLARE_FWD_DERIV)
/* out = a * b (replaces launch_multiply_kernel, :1477-1480, whose scalar
 * fallback drops the tail); the _bf16 form is new (the reference binding
 * accepts BF16 but multiplies it as FP16). */
int launch_multiply_kernel(void* out, const void* a, const void* b, int64_t size, void* stream);
int launch_multiply_kernel_bf16(void* out, const void* a, const void* b, int64_t size, void* stream);

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
/* Hardware control of B3: FA4's SFU sigmoid (sigmoid_variant="sfu", the
 * "native" entry of b3_component_configs, src/sfu_repro/fa4.py:687-693),
 * y = bf16(sigmoid(s - ln 4096)) via v_exp_f32 / v_rcp_f32 in FP32 and
 * dy = bf16(p (1 - p)) from the FP32 probability. */
int launch_flash_sigmoid_native_bf16(void* y, void* dy, const void* scores, int64_t size,
                                     void* stream);
/* B3-D2 sigmoid via a range-reduced degree-2 exp2 (FA4 sigmoid_degree == 2,
 * src/sfu_repro/fa4.py:469-476; model and coefficients from
 * autonumerics_zero/evolution/fit_flash_sigmoid_exp2_d2.py:55-143):
 * y = bf16(2^(n-12) (c0 + f (c1 + f c2))) with clamp(s*log2(e), -200, 200)
 * = n + f (NaN and -inf scores give 0),
 * dy = bf16(y (1 - y)) from the FP32 probability. */
int launch_flash_sigmoid_exp2_d2_bf16(void* y, void* dy, const void* scores, int64_t size,
                                      void* stream);

/* ---- B2: tanh softcap cap * tanh(s / cap) on BF16 scores -----------------
 * No C launcher exists in the reference: FA4 selects the D4 BF16 tanh
 * program for softcap (src/sfu_repro/fa4.py:650-668) and the composition
 * lives in the absent FA4 kernel.  Forward: u = bf16(s * (1/cap)),
 * out = bf16(cap * TANH_FWD_D4_ODD_BF16(u)).  Backward: grad_scores =
 * bf16(grad_out * T'(u)) with the differentiated D4 polynomial (the scale
 * cancels, extras/paper/manuscript/main.tex:443-449, 754-758).  cap must be
 * positive and finite (hipErrorInvalidValue otherwise), here and in the
 * attention softcap modes. */
int launch_softcap_tanh_d4_bf16(void* out, const void* scores, int64_t size, float cap,
                                void* stream);
int launch_softcap_tanh_d4_bwd_bf16(void* grad_scores, const void* grad_out, const void* scores,
                                    int64_t size, float cap, void* stream);
/* Native baseline: cap * tanh(s / cap) in FP32 with v_exp_f32 / v_rcp_f32. */
int launch_softcap_tanh_native_bf16(void* out, const void* scores, int64_t size, float cap,
                                    void* stream);
/* Native backward baseline, FA4's softcap_backward_mode 'native'
 * (src/sfu_repro/fa4.py:306-311): grad_scores = bf16(grad_out *
 * (1 - tanh^2(s / cap))), tanh in FP32 with v_exp_f32 / v_rcp_f32. */
int launch_softcap_tanh_native_bwd_bf16(void* grad_scores, const void* grad_out, const void* scores,
                                        int64_t size, float cap, void* stream);

/* ---- B5: exp2 with FP32 range reduction ---------------------------------
 * FA4's e2e_asm2 reduction (autonumerics_zero/cuda_benchmarks/
 * utils_exp2_cuda.cuh:13-74) with the D2 "safe" fraction
 * (extras/paper/manuscript/appendix_exp2.tex:29-32) or FA4's D3 fraction;
 * `native` is v_exp_f32 (the reference's exp2f baseline,
 * benchmark_exp2_pwl2.cu:101-105).  FP32 input, BF16 or FP32 output. */
int launch_exp2_d2_f32_bf16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_d3_f32_bf16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_native_f32_bf16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_d2_f32(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_d3_f32(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_native_f32(void* y, const void* x, int64_t size, void* stream);
/* B5 PWL2 "safe" hinge p(f) = 1 + a f + c max(f - 1/2, 0), c = 2 (1 - a),
 * p(0) = 1, p(1) = 2 (extras/paper/manuscript/appendix_exp2.tex:22-27), on
 * the same FP32 range reduction, -127 clamp and exponent add; the exp2
 * backends `pwl2_safe` and `pwl2_safe_f16` of src/sfu_repro/fa4.py:33-46
 * (`pwl2_safe_f16` is the public B5 candidate, fa4.py:739-743,
 * configs/torchtitan/b5_pwl2_safe_f16.toml).  pwl2_safe: FP32 arithmetic,
 * a = 0.7980513010, c = 0.4038973979 (sampled minimax, evidence/report-data/
 * b5_exp2_softmax_constrained_fits.json).  pwl2_safe_f16: the fraction
 * rounded to FP16 (RNE) and the hinge in packed FP16 (v_pk_add_f16,
 * v_pk_max_f16, two v_pk_fma_f16: b = fma(f, a, 1), p = fma(h, c, b)) with
 * a = 0.7978515625, c = 0.40380859375 (appendix_exp2.tex:72-76).  FA4's
 * 16-bit instruction order is not in the reference tree; this one is the FP32
 * hinge's. */
int launch_exp2_pwl2_safe_f32_bf16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_pwl2_safe_f32(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_pwl2_safe_f16_f32_bf16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_pwl2_safe_f16_f32(void* y, const void* x, int64_t size, void* stream);
/* The remaining exp2 backends of FA4 (src/sfu_repro/fa4.py:33-46), on the
 * same reduction and exponent add.  The forms are the appendix's
 * (extras/paper/manuscript/appendix_exp2.tex:17-32); their 16-bit programs
 * are not in the reference tree, so the precisions below are this build's:
 *   pwl2             the reference's two-piece FP32 hinge (benchmark_exp2_pwl2.cu:
 *                    126-170: offset 0x3F7D4D54, slope 0x3F522364, change
 *                    0x3EAF5701 at f = 1/2), clamped at -126 instead of the
 *                    reference's -127: its fraction starts below one
 *                    (p(0) = 0.98946), so below -126.987 the reference's
 *                    exponent add produces NaN bits; identical from -126 up;
 *   pwl1_safe        p = 1 + f (FP32), the only endpoint-safe line;
 *   pwl1_safe_f16    p = fp16(fp16(f) + 1);
 *   pwl2_safe_bf16   the PWL2 safe hinge on bf16(f) with bf16(a) = 0.796875,
 *                    bf16(c) = 0.404296875, each FMA rounded to BF16;
 *   d2_safe_noclamp  the D2 safe fraction without the -127 clamp (exponents
 *                    below -127 wrap the exponent field, as in FA4's variant);
 *   d2_safe_f16      p = fp16(fma(fp16(fma(f, c2, c1)), f, 1)) on fp16(f),
 *                    c1 = 0.66015625, c2 = 0.33984375 (the FP16 roundings of
 *                    the D2 fit, summing to one: p(1) = 2);
 *   d2_safe_bf16     the same with BF16 f and BF16 rounding per FMA (the same
 *                    two coefficients are BF16 values);
 *   pwl2_f16         the reference's FP16 hinge (FractionalPwl2Hinge,
 *                    autonumerics_zero/cuda_benchmarks/benchmark_exp2_pwl2.cu:84-99:
 *                    offset 0x3BEA, slope 0x3A91, change 0x357B) on fp16(f),
 *                    clamped at -126 like pwl2 (its fraction starts below one).
 * Every program keeps p(0) = 1 and p(1) = 2 after its rounding except
 * pwl2_f16 (p(0) = 0.98926). */
int launch_exp2_pwl2_f32_bf16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_pwl2_f32(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_pwl1_safe_f32_bf16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_pwl1_safe_f32(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_pwl1_safe_f16_f32_bf16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_pwl1_safe_f16_f32(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_pwl2_safe_bf16_f32_bf16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_pwl2_safe_bf16_f32(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_d2_safe_noclamp_f32_bf16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_d2_safe_noclamp_f32(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_d2_safe_f16_f32_bf16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_d2_safe_f16_f32(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_d2_safe_bf16_f32_bf16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_d2_safe_bf16_f32(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_pwl2_f16_f32_bf16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_pwl2_f16_f32(void* y, const void* x, int64_t size, void* stream);

/* ---- isolated exp2 measurements ------------------------------------------
 * The programs and protocol of the reference's exp2 harness
 * (autonumerics_zero/cuda_benchmarks/benchmark_exp2_pwl2.cu:24-36, 55-266;
 * published as evidence/report-data/exp2_pwl2_isolated_gb200.json), which
 * has no launcher in the reference's extension.
 * Fractional FP16 programs, f in [0, 1] -> 2^f, FP16 in and out (size in
 * elements): `native` v_exp_f16 per lane (the reference's h2exp2);
 * `pwl2_historical` the two-segment fit of FractionalPwl2Historical (:60-82:
 * f clamped to [0, 0x3BFE], segment from the top mantissa bit of fp16(f + 1),
 * p = fma(f, slope, offset), (0x3A91, 0x3BEA) / (0x3CA7, 0x3A8C));
 * `pwl2_hinge` the hinge of FractionalPwl2Hinge (:84-99), the fraction of
 * launch_exp2_pwl2_f16_*. */
int launch_exp2_fraction_native_f16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_fraction_pwl2_historical_f16(void* y, const void* x, int64_t size, void* stream);
int launch_exp2_fraction_pwl2_hinge_f16(void* y, const void* x, int64_t size, void* stream);
/* Compute probes (compute_h2_kernel / compute_f32_kernel, :203-250):
 * `threads` threads (the reference's 65,536; a positive multiple of 256, at
 * most 2^24) in blocks of 256, each reading 8 pairs, in[t + threads c] for
 * chain c, and running `iterations` rounds of x <- feedback(program(x)),
 * then storing chain t % 8 to out[t].  in holds 8 threads pairs, out
 * threads.  f16x2 (FP16 pairs, fractional programs; variant 0 native, 1
 * pwl2_historical, 2 pwl2_hinge): feedback fma(v, 1/2, -1/2) on chains 0-3,
 * fma(v, -1/2, 3/2) on 4-7, one FP16 rounding each.  f32x2 (float2 pairs,
 * full programs on the FP32 range reduction; variant 0 v_exp_f32, 1 FA4 D3,
 * 2 the PWL2 hinge of launch_exp2_pwl2_*): feedback fma(v, 8, -16) on chains
 * 0-3, -8 v on 4-7. */
int launch_exp2_compute_f16x2(int variant, void* out, const void* in, int64_t threads, int iterations,
                              void* stream);
int launch_exp2_compute_f32x2(int variant, void* out, const void* in, int64_t threads, int iterations,
                              void* stream);

/* ---- paired sin/cos tables: FP32 angles [size] -> out [2, size] ----------
 * Plane 0 holds cos, plane 1 sin.  Replaces launch_sincos_*_{bf16,fp16,f32}
 * (declared spline_ops.cpp:16-57, defined sincos_kernels.cu:2125-2668;
 * binding spline_ops.cpp:326-580, 980-1100).  Programs (sincos_kernels.cu):
 *   half_turn   1.5*2^23 shifter, one-term FP32 pi, sign = parity(k), packed
 *               16-bit polynomial (:644-920);
 *   quarter_turn shifter, one-term FP32 pi/2, quadrant swap + signs (:544-642);
 *   d3_d4_bf16  Cody-Waite pi/2 with a converted quadrant, BF16 program
 *               (:940-978);
 *   _f32        FP32 programs (:120-406): d3_d4 / d5_d4 / d7_d6 Cody-Waite
 *               quarter turn, d3_d4_magic_bias shifter quarter turn,
 *               d5_d4_half_turn_{ls,sollya} two-term pi half turn,
 *               d5_d4_half_turn_sollya_fast one-term pi, d3_d4_cycle in
 *               turns folded to [0, 1/8];
 *   native      v_sin_f32 / v_cos_f32 (__sinf / __cosf), rounded to the
 *               output format (the reference calls sincosf). */
#define SPLINE_HIP_SINCOS_LAUNCHERS(X)                                          \
    X(launch_sincos_native_bf16) X(launch_sincos_d3_d4_bf16)                    \
    X(launch_sincos_d3_d4_quarter_turn_bf16) X(launch_sincos_d3_d4_half_turn_bf16) \
    X(launch_sincos_d5_d6_half_turn_bf16) X(launch_sincos_d5_d4_half_turn_fp16_bf16) \
    X(launch_sincos_native_fp16) X(launch_sincos_d3_d4_quarter_turn_fp16)       \
    X(launch_sincos_d3_d4_half_turn_fp16) X(launch_sincos_d5_d4_half_turn_fp16) \
    X(launch_sincos_d5_d6_half_turn_fp16) X(launch_sincos_d7_d6_half_turn_fp16) \
    X(launch_sincos_native_f32) X(launch_sincos_d3_d4_f32)                      \
    X(launch_sincos_d3_d4_cycle_f32) X(launch_sincos_d3_d4_magic_bias_f32)      \
    X(launch_sincos_d5_d4_half_turn_ls_f32) X(launch_sincos_d5_d4_half_turn_sollya_f32) \
    X(launch_sincos_d5_d4_half_turn_sollya_fast_f32) X(launch_sincos_d5_d4_f32) \
    X(launch_sincos_d7_d6_f32)
#define SPLINE_HIP_DECLARE_SINCOS(name) \
    int name(void* out, const void* angles, int64_t size, void* stream);
SPLINE_HIP_SINCOS_LAUNCHERS(SPLINE_HIP_DECLARE_SINCOS)

/* Repeated-evaluation probes of the same programs (replace
 * launch_sincos_*_compute*, sincos_kernels.cu:2233-2668): element i
 * evaluates its program `iterations` (> 0) times on a probe angle that
 * starts at angles[i] and steps p <- fma(p, 0.99999994, 2^-13), and stores
 * the running sums of cos and sin (FP32 adds, or packed 16-bit adds for the
 * 16-bit programs).  They time instruction issue, not memory. */
#define SPLINE_HIP_SINCOS_COMPUTE_LAUNCHERS(X)                                  \
    X(launch_sincos_native_bf16_compute) X(launch_sincos_d3_d4_bf16_compute)    \
    X(launch_sincos_d3_d4_quarter_turn_bf16_compute) X(launch_sincos_d3_d4_half_turn_bf16_compute) \
    X(launch_sincos_d5_d6_half_turn_bf16_compute) X(launch_sincos_d5_d4_half_turn_fp16_bf16_compute) \
    X(launch_sincos_native_fp16_compute) X(launch_sincos_d3_d4_quarter_turn_fp16_compute) \
    X(launch_sincos_d3_d4_half_turn_fp16_compute) X(launch_sincos_d5_d4_half_turn_fp16_compute) \
    X(launch_sincos_d5_d6_half_turn_fp16_compute) X(launch_sincos_d7_d6_half_turn_fp16_compute) \
    X(launch_sincos_native_compute_f32) X(launch_sincos_d3_d4_compute_f32)      \
    X(launch_sincos_d3_d4_cycle_compute_f32) X(launch_sincos_d3_d4_magic_bias_compute_f32) \
    X(launch_sincos_d5_d4_half_turn_ls_compute_f32) X(launch_sincos_d5_d4_half_turn_sollya_compute_f32) \
    X(launch_sincos_d5_d4_half_turn_sollya_fast_compute_f32) X(launch_sincos_d5_d4_compute_f32) \
    X(launch_sincos_d7_d6_compute_f32)
#define SPLINE_HIP_DECLARE_SINCOS_COMPUTE(name) \
    int name(void* out, const void* angles, int64_t size, int64_t iterations, void* stream);
SPLINE_HIP_SINCOS_COMPUTE_LAUNCHERS(SPLINE_HIP_DECLARE_SINCOS_COMPUTE)

/* ---- RoPE ------------------------------------------------------------------
 * Phase increments are int32 Q0.32 turns per position, round(omega_i *
 * 2^32 / (2 pi)) (src/sfu_repro/rope/benchmark_cuda_fused_rope.py:238-241),
 * one per frequency (head_dim / 2 of them).
 *
 * Tables [2, S, F] FP16 for positions 0..S-1 (F even; replace
 * launch_rope_sincos_*_fp16, declared spline_ops.cpp:58-61, defined
 * sincos_kernels.cu:2671-2768):
 *   fixed_half_turn_d5_d6  Q15 half-turn residual, D5/D6 (:1289-1348);
 *   fixed_d3_d4            Q15 quarter-turn residual + quadrant, D3/D4
 *                          (:1242-1287);
 *   fixed_lut              128-entry table of FP16 (sin, cos) pairs per turn
 *                          (phase_table [128, 2], sin first) plus a
 *                          first-order correction (:1350-1385);
 *   native                 FP32 frequencies omega_i, angle = position *
 *                          omega_i, v_sin_f32 / v_cos_f32.
 * The _compute forms (replace the launchers of :2871-2978) store, for entry
 * (pos, f), the packed FP16 sum over positions pos .. pos + iterations - 1.
 *
 * launch_rope_apply_*: Q [B, S, Hq, D], K [B, S, Hk, D] (even/odd pairs
 * interleaved) -> rotated Q [B, Hq, S, D], K [B, Hk, S, D]; replaces
 * launch_rope_apply_{cached,native,fixed_half_turn_d5_d6}_fp16
 * (spline_ops.cpp:66-68; sincos_kernels.cu:2769-2870); the _bf16 entry points
 * are new (the reference's fused RoPE is FP16 only, spline_ops.cpp:838-839).
 * `angle_params` is the increments (fixed), the FP32 frequencies omega_i
 * (native) or a [2, S, D/2] FP16 cos/sin table (cached).  head_dim must be a
 * multiple of 8 and every pointer 16-byte aligned. */
#define SPLINE_HIP_ROPE_TABLE_LAUNCHERS(X)                                      \
    X(launch_rope_sincos_fixed_half_turn_d5_d6_fp16) X(launch_rope_sincos_fixed_d3_d4_fp16) \
    X(launch_rope_sincos_native_fp16)
#define SPLINE_HIP_DECLARE_ROPE_TABLE(name)                                     \
    int name(void* out, const void* params, int64_t sequence_length,            \
             int64_t frequency_count, void* stream);
SPLINE_HIP_ROPE_TABLE_LAUNCHERS(SPLINE_HIP_DECLARE_ROPE_TABLE)
#define SPLINE_HIP_ROPE_TABLE_COMPUTE_LAUNCHERS(X)                              \
    X(launch_rope_sincos_fixed_half_turn_d5_d6_fp16_compute)                    \
    X(launch_rope_sincos_fixed_d3_d4_fp16_compute) X(launch_rope_sincos_native_fp16_compute)
#define SPLINE_HIP_DECLARE_ROPE_TABLE_COMPUTE(name)                             \
    int name(void* out, const void* params, int64_t sequence_length,            \
             int64_t frequency_count, int64_t iterations, void* stream);
SPLINE_HIP_ROPE_TABLE_COMPUTE_LAUNCHERS(SPLINE_HIP_DECLARE_ROPE_TABLE_COMPUTE)
int launch_rope_sincos_fixed_lut_fp16(void* out, const void* phase_increments,
                                      const void* phase_table, int64_t sequence_length,
                                      int64_t frequency_count, void* stream);
int launch_rope_sincos_fixed_lut_fp16_compute(void* out, const void* phase_increments,
                                              const void* phase_table, int64_t sequence_length,
                                              int64_t frequency_count, int64_t iterations,
                                              void* stream);
#define SPLINE_HIP_ROPE_APPLY_LAUNCHERS(X)                                      \
    X(launch_rope_apply_fixed_half_turn_d5_d6_fp16) X(launch_rope_apply_fixed_half_turn_d5_d6_bf16) \
    X(launch_rope_apply_native_fp16) X(launch_rope_apply_native_bf16)          \
    X(launch_rope_apply_cached_fp16)
#define SPLINE_HIP_DECLARE_ROPE_APPLY(name)                                     \
    int name(void* q_out, void* k_out, const void* q, const void* k,            \
             const void* angle_params, int64_t batch, int64_t sequence_length,  \
             int64_t q_heads, int64_t k_heads, int64_t head_dim, void* stream);
SPLINE_HIP_ROPE_APPLY_LAUNCHERS(SPLINE_HIP_DECLARE_ROPE_APPLY)

/* ---- RoPE reference evaluator (src/sfu_repro/rope/polynomial_sincos.py:85-165)
 * FP32 or FP64 angles (angles_f64 = 1) -> FP32 cos and sin planes.  accurate = 1
 * reduces to a quarter turn in FP64 (q = rint(a * 2/pi), r = a - q * pi/2), 0 in
 * FP32 with the two-term Cody-Waite pi/2; then sin = r * S(r^2), cos = C(r^2),
 * each Horner step `v * x + c` rounded after the product and after the sum,
 * then the quadrant swap and signs.  Coefficients are host arrays, lowest power
 * first, 1..8 of each.  No counterpart launcher exists in the reference (its
 * evaluator is tensor arithmetic); these replace that arithmetic on the device. */
int launch_polynomial_sincos_f32(void* cos_out, void* sin_out, const void* angles, int angles_f64,
                                 int64_t size, int accurate, const float* sin_coeffs, int n_sin,
                                 const float* cos_coeffs, int n_cos, void* stream);
/* reduced (FP32) and quadrant (int64, 0..3) of the same reduction. */
int launch_reduce_to_quarter_turn(void* reduced_out, void* quadrant_out, const void* angles,
                                  int angles_f64, int64_t size, int accurate, void* stream);
/* (sin, cos) of reduced FP32 (or FP64, rounded to FP32 first) arguments. */
int launch_evaluate_reduced_sincos(void* sin_out, void* cos_out, const void* reduced,
                                   int reduced_f64, int64_t size, const float* sin_coeffs,
                                   int n_sin, const float* cos_coeffs, int n_cos, void* stream);

/* ---- fused attention forward with the score programs in the tile loop -----
 * No counterpart launcher exists in the reference: its attention programs (B2
 * softcap, B3 sigmoid attention, B5 exp2) run inside a FlashAttention-4 fork
 * that is not part of the reference tree (src/sfu_repro/fa4.py:454-752 selects
 * them; extras/paper/manuscript/main.tex:483-509 describes the fusion).
 * q [B, Hq, S, D], k and v [B, Hkv, S, D] -> out [B, Hq, S, D], BF16;
 * Hq a multiple of Hkv (grouped-query), any S >= 0, head_dim D 64 or 128,
 * every pointer 16-byte aligned; s = q.k * scale.  mode:
 *   0 softmax, hardware exp2 (v_exp_f32)      1 softmax, B5 D2 "safe" exp2
 *   2 softmax, FA4 D3 exp2                     3 softcap cap*tanh(s/cap), FP32
 *     hardware tanh, then softmax              4 softcap with the D4 BF16
 *     program on bf16(s) (B2), then softmax    5 sigmoid attention,
 *     p = sigmoid(s - ln S) (hardware exp/rcp), O = P V unnormalised
 *   6 sigmoid attention with the B3 direct D3 program on bf16(s)
 *     (fitted for S = 4096; other lengths are rejected).
 * causal != 0 masks keys after the query. */
int launch_flash_attention_fwd_bf16(void* out, const void* q, const void* k, const void* v,
                                    int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq,
                                    int64_t head_dim, int mode, int causal, float scale, float cap,
                                    void* stream);
/* General form, the runtime behind the FA4 interface (the flash_attn_fwd that
 * src/sfu_repro/fa4.py:356-428 calls).  strides: 12 element strides, (batch,
 * head, sequence) of q, k, v and out in that order, each a multiple of 8; the
 * head dimension D (64 or 128) is contiguous, so [B, S, H, D] (FA4's layout)
 * and [B, H, S, D] both work.  lse: null, or float [B, Hq, S] receiving
 * ln sum_k exp(s'_k) (s' the scaled, capped score) for the softmax modes;
 * sigmoid modes leave it untouched.  Extra modes:
 *   7 sigmoid attention with the B3-D2 exp2 program (fitted for S = 4096)
 *   8..11 sigmoid attention with the BF16 sigmoid D3..D6 program on
 *     bf16(s + sigmoid_bias)          12 softmax, PWL2 hinge exp2
 *   13 softmax, PWL2 "safe" hinge exp2 (FP32; FA4 backend pwl2_safe)
 *   14 softmax, PWL2 "safe" hinge exp2 with the packed FP16 fraction (FA4
 *     backend pwl2_safe_f16; the programs of launch_exp2_pwl2_safe*).
 *   15..21 softmax with FA4's remaining exp2 backends, the programs of the
 *     launch_exp2_<backend>* entry points: 15 pwl1_safe, 16 pwl1_safe_f16,
 *     17 pwl2_safe_bf16, 18 d2_safe_noclamp (no clamp: exponents below -127
 *     wrap, so the backward needs a finite lse), 19 d2_safe_f16,
 *     20 d2_safe_bf16, 21 pwl2_f16 (clamped at -126, as mode 12).
 * sigmoid_bias: the bias of the hardware and D3..D6 sigmoid modes.
 * exp2_route (modes 1, 2 and 12..21): any even value >= 4 (FA4's
 * exp2_emu_freq, src/sfu_repro/fa4.py:223-233).  Key j of a query row takes
 * the polynomial, else v_exp_f32, when slot(j) % exp2_route < 4 for routes
 * up to 32, with slot(j) = 16 bit5(j) + 4 bits3..4(j) + bits0..1(j) (the
 * slot of j's exponent among the 32 a lane holds per 64-key tile), and when
 * (32 (j / 64) + slot(j)) % exp2_route < 4 above 32, so four of every
 * exp2_route exponents are routed (4: all).  Routes 4, 6, 8, 10, 12, 16, 20,
 * 24 and 32 run kernels specialised for them; the others read the pattern
 * from the kernel arguments. */
int launch_flash_attention_fwd_strided_bf16(void* out, float* lse, const void* q, const void* k,
                                            const void* v, int64_t batch, int64_t q_heads,
                                            int64_t kv_heads, int64_t seq, int64_t head_dim,
                                            const int64_t* strides, int mode, int exp2_route,
                                            int causal, float scale, float cap, float sigmoid_bias,
                                            void* stream);
/* The same forward with keys valid_keys .. seq - 1 masked as padding
 * (1 <= valid_keys <= seq), for callers that keep operands padded at the end
 * (the padded queries' rows are computed and left to the caller to drop).
 * The padded K and V rows are zeroed on chip before use, so they may hold
 * anything (NaN and Inf included).  The padded queries attend to the valid
 * keys: their out rows and lse are finite for finite Q rows.
 * The backward takes no valid_keys.  It serves padded operands when the
 * padded K rows are zero, the padded V, Q and out rows finite and the padded
 * dout rows zero: a zero K row gives the padded keys no share of dQ, and a
 * zero dout row makes a padded query's dP and D zero, so it adds nothing to
 * dK / dV.  Any seq works without padding: the kernels read no row past seq.
 * launch_flash_attention_fwd_strided_bf16 is this with valid_keys = seq. */
int launch_flash_attention_fwd_strided_keys_bf16(void* out, float* lse, const void* q, const void* k,
                                                 const void* v, int64_t batch, int64_t q_heads,
                                                 int64_t kv_heads, int64_t seq, int64_t valid_keys,
                                                 int64_t head_dim, const int64_t* strides, int mode,
                                                 int exp2_route, int causal, float scale, float cap,
                                                 float sigmoid_bias, void* stream);
/* Backward of the same attention (the runtime behind FA4's flash_attn_bwd,
 * src/sfu_repro/fa4.py:430-461): dq [B, S, Hq, D], dk and dv [B, S, Hkv, D]
 * BF16 from q, k, v, out, dout (BF16) and the forward's lse (softmax modes).
 * strides: 24 element strides, (batch, head, sequence) of q, k, v, out, dout,
 * dq, dk, dv.  delta: caller-provided float [B, Hq, S] workspace receiving
 * rowsum(dout * out) (softmax modes; unused for sigmoid modes, where out, lse
 * and delta may be null).  dkv_workspace: with grouped-query heads (Hq > Hkv)
 * a caller-provided, 16-byte aligned float workspace of 2 * B * Hq * S * D
 * elements (per-query-head dK / dV partials, summed deterministically into
 * dk / dv); null otherwise.  grad, the derivative of the score program:
 *   0 the mode's own (softmax, softcap 1 - tanh^2, sigmoid p (1 - p))
 *   1 / 2 / 3  mode 4 only: the D4 derivative polynomial (FA4 "analytical") /
 *              straight-through (ste) / 1 - T(u)^2 (exact_1mt2)
 *   4 / 5      mode 6 only: y (1 - y) (algebraic) / the B3 factored D4
 *              derivative (direct).
 * exp2_route (modes 1, 2 and 12..21): 0 hardware exp2, 4 the polynomial everywhere,
 * any other even value the polynomial for the keys the forward routes with
 * that value (FA4's exp2_emu_freq_bwd). */
int launch_flash_attention_bwd_strided_bf16(void* dq, void* dk, void* dv, float* delta,
                                            float* dkv_workspace, const void* q, const void* k, const void* v,
                                            const void* out, const void* dout, const float* lse,
                                            int64_t batch, int64_t q_heads, int64_t kv_heads,
                                            int64_t seq, int64_t head_dim, const int64_t* strides,
                                            int mode, int grad, int exp2_route, int causal,
                                            float scale, float cap, float sigmoid_bias, void* stream);
/* Backward that keeps dS: no counterpart in the reference (FA4's backward is
 * not part of its tree).  Same arguments and results as
 * launch_flash_attention_bwd_strided_bf16, bit for bit, plus `ds_workspace`:
 * spline_hip_attn_bwd_ds_bytes(batch, q_heads, seq, head_dim, mode) bytes of
 * device memory, 16-byte aligned, whose contents need no initialisation.
 * The dK/dV kernel stores dS there (only the chunks the causal mask keeps)
 * and the dQ kernel multiplies it by K instead of recomputing S, P, dP and
 * the score program.  Where the size helper returns 0 (S not a multiple of
 * 128, plain softmax at head_dim 64, where recomputing is cheaper) or
 * ds_workspace is null, the call is the recomputing backward. */
int64_t spline_hip_attn_bwd_ds_bytes(int64_t batch, int64_t q_heads, int64_t seq, int64_t head_dim, int mode);
int launch_flash_attention_bwd_strided_ds_bf16(void* dq, void* dk, void* dv, float* delta,
                                               float* dkv_workspace, void* ds_workspace, const void* q,
                                               const void* k, const void* v, const void* out,
                                               const void* dout, const float* lse, int64_t batch,
                                               int64_t q_heads, int64_t kv_heads, int64_t seq,
                                               int64_t head_dim, const int64_t* strides, int mode, int grad,
                                               int exp2_route, int causal, float scale, float cap,
                                               float sigmoid_bias, void* stream);
/* Allocation-free form of launch_flash_attention_bwd_strided_bf16: no
 * counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments and results without `delta` and
 * `dkv_workspace`: both live in a device array inside the library
 * (SPLINE_HIP_BWD_SCRATCH_BYTES per GPU, held until the process ends), laid
 * out as delta [B, Hq, S] FP32 (padded to 256 bytes), then with grouped heads
 * (Hq > Hkv) the 2 * B * Hq * S * D FP32 dK / dV partials.  Returns
 * hipErrorOutOfMemory (2) when those exceed SPLINE_HIP_BWD_SCRATCH_BYTES:
 * the limit is B * Hq * S <= 16,777,216 query rows without grouped heads,
 * and <= 65,280 (D = 128) or <= 130,055 (D = 64) with them.  Calls no
 * allocator.  Calls that overlap on one GPU share the array and race: order
 * them on one stream.  The first call on each device looks up the array's
 * device address (hipGetSymbolAddress, once per device): make that first
 * call eagerly, outside HIP graph capture; later calls may be captured. */
#define SPLINE_HIP_BWD_SCRATCH_BYTES (64ll << 20)
int launch_flash_attention_bwd_strided_bf16_noalloc(void* dq, void* dk, void* dv, const void* q,
                                                    const void* k, const void* v, const void* out,
                                                    const void* dout, const float* lse, int64_t batch,
                                                    int64_t q_heads, int64_t kv_heads, int64_t seq,
                                                    int64_t head_dim, const int64_t* strides, int mode,
                                                    int grad, int exp2_route, int causal, float scale,
                                                    float cap, float sigmoid_bias, void* stream);

/* ---- device/launch introspection --------------------------------------- */
/* Number of compute units of the current device and the grid the
 * elementwise launchers use for `size` 16-bit elements and `streams` tensors
 * (inputs + outputs).  For tests and benchmarks. */
int spline_hip_grid_for(int64_t size, int streams, int64_t* grid_out, int* cus_out);

/* Measurement helper, no counterpart in the reference: copies `size` 16-bit
 * elements through the same one-pass driver, launch shape and cache policy
 * as the unary launchers above.  Its time is the achievable ceiling a
 * 1-read/1-write stream of that size reaches on this device. */
int spline_hip_copy16(void* out, const void* in, int64_t size, void* stream);
/* Measurement helpers, no counterpart in the reference: the read-only and
 * write-only ceilings of the same launch shape (non-temporal, one 16-byte
 * vector per thread) over the first size/8*8 16-bit elements.  read16 reads
 * `in` (16-byte aligned) and writes at most 4 bytes to `sink`; fill16
 * writes `word` to every 32-bit word of `out` (16-byte aligned). */
int spline_hip_read16(void* sink, const void* in, int64_t size, void* stream);
int spline_hip_fill16(void* out, int64_t size, uint32_t word, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SPLINE_OPS_HIP_H */
