/*
 * spline_oracle.h -- CPU restatement of the reference's packed FP16/BF16
 * polynomial programs.  TEST INFRASTRUCTURE ONLY: tests/, the smoke check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py may load this
 * library, and only as the checker.  Nothing in the product path links it.
 *
 * All 16-bit values cross this interface as raw bit patterns (uint16_t).
 * Every function returns 0 on success and a negative code on bad arguments.
 */
#ifndef SPLINE_ORACLE_H
#define SPLINE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Storage formats.  ORC_BF16_SOLLYA is BF16 storage with the Sollya
 * coefficient set (coeff_source_id 1, spline_structs_sollya_bf16.cuh); it is
 * accepted by the activation programs only. */
enum { ORC_F16 = 0, ORC_BF16 = 1, ORC_BF16_SOLLYA = 2 };

/* Activation families and directions. */
enum { ORC_SIGMOID = 0, ORC_TANH = 1, ORC_SWISH = 2, ORC_GELU = 3 };
enum { ORC_FWD = 0, ORC_BWD = 1 };

/* BF16 FMA semantics for the activation programs.
 * ORC_RND_SINGLE: one rounding of the exact a*b+c (the reference's
 *                 fma.rn.bf16x2 / __hfma2 semantics).
 * ORC_RND_F32:    round to binary32 first, then to BF16 (what an FP32 FMA
 *                 followed by an RNE pack computes).
 * FP16 always uses single rounding. */
enum { ORC_RND_SINGLE = 0, ORC_RND_F32 = 1 };

/* ---- rounding primitives ---------------------------------------------- */
uint16_t orc_f32_to_bf16_audit(float v);   /* audit round_bf16 bit trick   */
uint16_t orc_f64_to_bf16(double v);        /* RNE                          */
uint16_t orc_f64_to_f16(double v);         /* RNE                          */
double orc_bf16_to_f64(uint16_t b);
double orc_f16_to_f64(uint16_t b);
/* Single-rounding fused multiply-add on 16-bit operands (bit patterns). */
uint16_t orc_fma16(int fmt, uint16_t a, uint16_t b, uint16_t c);
/* Audit emulation of one fma.rn.bf16x2 lane: round_bf16(a*b + c). */
uint16_t orc_bf16_fma_audit(uint16_t a, uint16_t b, uint16_t c);

/* ---- activation programs (spline_structs_odd*.cuh) --------------------- */
/* y[i] = P(x[i]) for the forward program, or the derivative program for
 * dir == ORC_BWD.  degree 3..6. */
int orc_activation(int family, int dir, int degree, int fmt, int rnd,
                   const uint16_t* x, uint16_t* y, int64_t n);
/* The program table entry (shape code, clamp, degree, c[0..6]) for tests
 * that compare the oracle's tables with an independent transcription. */
int orc_program(int family, int dir, int degree, int fmt, int* shape, float* lc,
                int* deg, float* c7);
/* gi = go * G(x)  (binary_vec_kernel). */
int orc_activation_bwd(int family, int degree, int fmt, int rnd,
                       const uint16_t* go, const uint16_t* x, uint16_t* gi,
                       int64_t n);
/* gi = go * alg(y): sigmoid y(1-y), tanh 1-y^2. */
int orc_activation_bwd_alg(int family, int fmt, const uint16_t* go,
                           const uint16_t* y, uint16_t* gi, int64_t n);
/* out = F(gate) * up. */
int orc_swish_mul_fwd(int degree, int fmt, int rnd, const uint16_t* gate,
                      const uint16_t* up, uint16_t* out, int64_t n);
/* grad_gate = (go*up)*F'(gate), grad_up = go*F(gate); BF16 degree 3 uses the
 * algebraic derivative fma(swish, 1-sigma, sigma). */
int orc_swish_mul_bwd(int degree, int fmt, int rnd, const uint16_t* go,
                      const uint16_t* gate, const uint16_t* up,
                      uint16_t* grad_gate, uint16_t* grad_up, int64_t n);

/* ---- B3 deployed direct D3 / factored D4 (audit_b3_deployed_fit.py) ---- */
/* x: BF16 scores.  y = probability, dy = derivative, both BF16.
 * row (optional, may be NULL): selected coefficient row. */
int orc_b3_direct_bf16(const uint16_t* x, uint16_t* y, uint16_t* dy,
                       uint8_t* row, int64_t n);
/* Same program on FP32 scores (rounded to BF16 first, as the audit does). */
int orc_b3_direct_f32(const float* s, uint16_t* y, uint16_t* dy, int64_t n);
/* Deployed constants as BF16 bit patterns: fwd[2][4] (c0..c3 after 1/4096
 * scaling), grad[2][2] (intercept, slope), split, clamp. */
int orc_b3_constants(uint16_t* fwd8, uint16_t* grad4, uint16_t* split_clamp2);

/* B3-D2: sigmoid(s - ln 4096) via a range-reduced degree-2 exp2 with the
 * given FP32 coefficients (c0, c1, c2). */
int orc_b3_exp2_d2_bf16(const uint16_t* x, uint16_t* y, uint16_t* dy, int64_t n,
                        const float* coeffs3);

/* ---- B2 softcap (BF16) ---------------------------------------------------
 * Parity unpinned against the reference: its softcap composition lives in
 * FlashAttention-4, which is not part of the reference tree.  The steps are
 * this build's (u = bf16(s * (1/cap)), the reference's TANH_FWD_D4_ODD_BF16,
 * y = bf16(T * cap)); tests pin them step by step to that D4 program and
 * bound the result against cap * tanh(s / cap). */
int orc_softcap_fwd_bf16(const uint16_t* s, uint16_t* y, int64_t n, float cap);
int orc_softcap_bwd_bf16(const uint16_t* go, const uint16_t* s, uint16_t* g, int64_t n, float cap);

/* ---- B5 exp2: kind 0 = D2 safe, 1 = FA4 D3, 2 = PWL2 hinge, 3 = PWL2 safe
 * (FP32), 4 = PWL2 safe (packed FP16), 5 = PWL1 safe, 6 = PWL1 safe FP16,
 * 7 = PWL2 safe BF16, 8 = D2 safe without the -127 clamp, 9 = D2 safe FP16,
 * 10 = D2 safe BF16, 11 = the reference's FP16 hinge (clamped at -126) ------
 * The FP32 programs are pinned (p(0) = 1, p(1) = 2, the published fit and
 * error metrics); the deployed 16-bit output rounding is parity unpinned
 * (it lives in the absent FlashAttention-4): here one RNE of the FP32
 * result.  Kind 4's FP16 core (f rounded to FP16, h = max(f - 1/2, 0),
 * p = fma(h, c, fma(f, a, 1)), one FP16 rounding per step) is pinned by its
 * published coefficients, its endpoints after FP16 rounding and its
 * published maximum relative error (appendix_exp2.tex:72-76); FA4's own
 * instruction order is not in the reference tree.  Kind 11 is the
 * reference's own FP16 program (benchmark_exp2_pwl2.cu:84-99), pinned by its
 * published fractional error metrics; kinds 5-10 are pinned by their
 * endpoints and fit errors only (parity unpinned: FA4 absent). */
int orc_exp2(int kind, int out_bf16, const float* x, uint16_t* y16, float* y32, int64_t n);
/* The fraction program alone on f in [0, 1] (no range reduction), kinds 5-7
 * and 9-11, and 12: the reference's historical two-segment FP16 fit
 * (benchmark_exp2_pwl2.cu:60-82), pinned by its published fractional error
 * metrics (exp2_pwl2_isolated_gb200.json, fractional_h2 / pwl2_historical). */
int orc_exp2_fraction(int kind, const float* f, float* p, int64_t n);

/* ---- paired sin/cos: prog 0 BF16 D3/D4, 1 BF16 D5/D6, 2 FP16 D3/D4,
 * 3 FP16 D5/D4, 4 FP16 D5/D6, 5 FP16 D7/D6 (half turn) ------------------- */
int orc_sincos(int prog, int out_fmt, int rnd, const float* angles, uint16_t* cos_out,
               uint16_t* sin_out, int64_t n);
/* RoPE: [2, seq, nfreq] FP16 table and fused apply (fmt ORC_F16 / ORC_BF16). */
int orc_rope_sincos_table(const int32_t* inc, uint16_t* out, int64_t seq, int64_t nfreq);
int orc_rope_apply(int fmt, const uint16_t* q, const uint16_t* k, const int32_t* inc,
                   uint16_t* q_out, uint16_t* k_out, int64_t batch, int64_t seq, int64_t hq,
                   int64_t hk, int64_t dim);

/* ---- FP32 sin/cos programs: prog 0 D3/D4, 1 D3/D4 magic bias, 2 D5/D4,
 * 3 D7/D6 (Cody-Waite quarter turn), 4 half-turn D5/D4 LS, 5 half-turn
 * D5/D4 Sollya, 6 its one-term-pi fast form, 7 D3/D4 cycle.  iterations 0:
 * table; > 0: compute probe sums (FP32 adds). */
int orc_sincos_f32(int prog, const float* angles, float* cos_out, float* sin_out, int64_t n,
                   int iterations);
/* ---- every 16-bit sin/cos program: prog 0..5 as orc_sincos, 6 FP16 quarter
 * turn D3/D4, 7 BF16 quarter turn D3/D4, 8 BF16 Cody-Waite D3/D4; outputs in
 * out_fmt; iterations > 0: compute probe sums in out_fmt. */
/* Coefficient tables of the paired sin/cos programs (0 half turn 16-bit,
 * 1 FP32, 2 quarter turn 16-bit, 3 RoPE Q15 quarter turn). */
int orc_sincos_coeffs(int table, int idx, int* ns, float* s, int* nc, float* c);
int orc_sincos16(int prog, int out_fmt, int rnd, const float* angles, uint16_t* cos_out,
                 uint16_t* sin_out, int64_t n, int iterations);
/* RoPE tables [2, seq, nfreq] FP16: kind 0 half-turn D5/D6, 1 quarter-turn
 * D3/D4, 2 LUT (lut = [128, 2] FP16 bits, sin first); iterations > 0: sums
 * over positions p .. p + iterations - 1. */
int orc_rope_table(int kind, const int32_t* inc, const uint16_t* lut, uint16_t* out, int64_t seq,
                   int64_t nfreq, int iterations);
/* Fused FP16 RoPE with a [2, seq, dim/2] FP16 cos/sin table. */
int orc_rope_apply_cached(const uint16_t* q, const uint16_t* k, const uint16_t* table,
                          uint16_t* q_out, uint16_t* k_out, int64_t batch, int64_t seq, int64_t hq,
                          int64_t hk, int64_t dim);

/* ---- FP16 experiments: SiLU value and derivative from one shared sigmoid
 * D3 (y = x*s, dy = s*fma(x, 1-s, 1)); elementwise product (FP16 / BF16). */
int orc_swish_fwd_deriv_shared(const uint16_t* x, uint16_t* y, uint16_t* dy, int64_t n);
int orc_multiply(int fmt, const uint16_t* a, const uint16_t* b, uint16_t* out, int64_t n);

/* Thread count used by the bulk loops (OpenMP when built with it). */
int orc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
