"""The oracle's activation, softcap, exp2, sin/cos and RoPE programs against
the reference's known answers and against the mathematics they approximate.

A dropped Horner term, a wrong sign, a swapped coefficient or a wrong clamp
moves the maximum error far past the bounds below; the per-program bounds
come from the `Err=` figures the reference states next to each program
(spline_structs_odd*.cuh) and the fit tables of the paper."""

import math

import numpy as np
import pytest

ALL = None


def _all(oracle):
    return oracle.all_bits()


def _exact(fam, direction, v):
    s = 1.0 / (1.0 + np.exp(-v))
    if fam == "sigmoid":
        return s if direction == 0 else s * (1 - s)
    if fam == "tanh":
        return np.tanh(v) if direction == 0 else 1 - np.tanh(v) ** 2
    return v * s if direction == 0 else s * (1 + v * (1 - s))


# (fmt, family, direction) -> [(Li, stated Err)] for degrees 3..6, from the
# comments of spline_structs_odd.cuh and spline_structs_odd_bf16.cuh.
STATED = {
    ("f16", "sigmoid", 0): [(6.5, 0.005562), (4.75, 0.004261), (6.0, 0.002594), (7.25, 0.003168)],
    ("f16", "tanh", 0): [(3.25, 0.011089), (2.75, 0.009193), (3.0, 0.005188), (4.5, 0.006221)],
    ("f16", "sigmoid", 1): [(4.5, 0.011002), (5.25, 0.004201), (5.75, 0.002840), (6.25, 0.002963)],
    ("f16", "tanh", 1): [(2.25, 0.044007), (2.5, 0.019043), (3.25, 0.015758), (4.75, 0.017399)],
    ("f16", "swish", 1): [(5.25, 0.017511), (8.0, 0.014858), (6.25, 0.010503), (7.25, 0.010162)],
    ("bf16", "sigmoid", 0): [(6.0, 0.007420), (5.0, 0.005891), (6.25, 0.005891), (8.0, 0.008847)],
    ("bf16", "tanh", 0): [(2.5, 0.014538), (2.5, 0.013285), (4.25, 0.016504), (4.25, 0.014477)],
    ("bf16", "sigmoid", 1): [(4.5, 0.011549), (4.75, 0.007216), (7.5, 0.008373), (7.5, 0.009759)],
    ("bf16", "tanh", 1): [(2.25, 0.046194), (2.25, 0.032650), (4.25, 0.038063), (5.75, 0.036270)],
    ("bf16", "swish", 1): [(4.75, 0.021872), (7.25, 0.018683), (6.25, 0.019464), (10.0, 0.019176)],
}


@pytest.mark.parametrize("key", sorted(STATED))
def test_activation_error_matches_stated_fit(oracle, key):
    fmt, fam, direction = key
    x = _all(oracle)
    with np.errstate(invalid="ignore", over="ignore"):
        v = oracle.bits_to_f32(x, fmt).astype(np.float64)
    for degree, (li, err) in zip((3, 4, 5, 6), STATED[key]):
        y = oracle.bits_to_f32(oracle.activation(fam, direction, degree, fmt, x), fmt)
        m = np.isfinite(v) & (np.abs(v) <= li)
        got = np.abs(y[m] - _exact(fam, direction, v[m])).max()
        # The stated figure was measured on a sampled grid; the exhaustive
        # 16-bit sweep lands within [0.5, 2.5] x of it for every program.
        assert 0.5 * err <= got <= 2.5 * err, (key, degree, got, err)


@pytest.mark.parametrize("degree", [3, 4, 5, 6])
def test_bf16_swish_tails_are_exact(oracle, degree):
    # autonumerics_zero/spline_ops/test_spline_ops.py:159-166
    gate = oracle.f32_to_bf16_bits(np.array([-100, -20, 20, 100], dtype=np.float32))
    up = oracle.f32_to_bf16_bits(np.ones(4, dtype=np.float32))
    out = oracle.bf16_bits_to_f32(oracle.swish_mul_fwd(degree, "bf16", gate, up))
    assert out.tolist() == [0.0, 0.0, 20.0, 100.0]


def test_fp16_sigmoid_d3_error_kat(oracle):
    # test_spline_ops.py:249-259: FP16 sigmoid D3 max error < 0.02 on randn*3
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(1 << 20) * 3).astype(np.float16)
    y = oracle.f16_bits_to_f32(oracle.activation("sigmoid", 0, 3, "f16", x.view(np.uint16)))
    assert np.abs(y - 1 / (1 + np.exp(-x.astype(np.float64)))).max() < 0.02


def test_swiglu_d3_bf16_matches_native_within_reference_tolerance(oracle):
    # test_spline_ops.py:12-50: SwiGLU D3 vs FP32 silu*up, atol 0.07
    gate = np.linspace(-12, 12, 4097, dtype=np.float32)
    up = np.linspace(-1, 1, 4097, dtype=np.float32)
    go = np.linspace(1, -1, 4097, dtype=np.float32)
    gb, ub, gob = (oracle.f32_to_bf16_bits(a) for a in (gate, up, go))
    gq, uq = oracle.bf16_bits_to_f32(gb), oracle.bf16_bits_to_f32(ub)
    goq = oracle.bf16_bits_to_f32(gob)
    out = oracle.bf16_bits_to_f32(oracle.swish_mul_fwd(3, "bf16", gb, ub))
    s = 1 / (1 + np.exp(-gq.astype(np.float64)))
    assert np.abs(out - gq * s * uq).max() < 0.07
    gg, gu = oracle.swish_mul_bwd(3, "bf16", gob, gb, ub)
    assert np.abs(oracle.bf16_bits_to_f32(gg) - goq * uq * s * (1 + gq * (1 - s))).max() < 0.07
    assert np.abs(oracle.bf16_bits_to_f32(gu) - goq * gq * s).max() < 0.07


@pytest.mark.parametrize("fam", ["sigmoid", "tanh", "swish"])
@pytest.mark.parametrize("direction", [0, 1])
@pytest.mark.parametrize("degree", [3, 4, 5, 6])
def test_bf16_fp32_fma_then_rne_equals_single_rounding(oracle, fam, direction, degree):
    """The gfx950 BF16 path (FP32 FMA, then RNE to BF16) gives the same bits
    as a single-rounding BF16 FMA for every input of every program."""
    x = _all(oracle)
    a = oracle.activation(fam, direction, degree, "bf16", x, oracle.RND_SINGLE)
    b = oracle.activation(fam, direction, degree, "bf16", x, oracle.RND_F32)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("prog", [0, 1])
def test_bf16_sincos_fp32_fma_then_rne_equals_single_rounding(oracle, prog):
    # every BF16 reduced argument in [-pi/2, pi/2] (the reduction is exact there)
    x = _all(oracle)
    v = oracle.bf16_bits_to_f32(x)
    with np.errstate(invalid="ignore"):
        a = v[np.isfinite(v) & (np.abs(v) <= 1.5)]
    c1, s1 = oracle.sincos(prog, a, rnd=oracle.RND_SINGLE)
    c2, s2 = oracle.sincos(prog, a, rnd=oracle.RND_F32)
    assert np.array_equal(c1, c2) and np.array_equal(s1, s2)


# ---- B2 softcap -------------------------------------------------------------

def test_softcap_forward_error_bound(oracle):
    x = _all(oracle)
    with np.errstate(invalid="ignore", over="ignore"):
        s = oracle.bf16_bits_to_f32(x).astype(np.float64)
    m = np.isfinite(s)
    y = oracle.bf16_bits_to_f32(oracle.softcap_fwd_bf16(x, 30.0))[m]
    ref = 30.0 * np.tanh(s[m] / 30.0)
    # D4 tanh (max error 0.0133 on its fit range) scaled by cap, plus the BF16
    # rounding of the input scale and of the output (|y| <= 30: half-ulp 0.0625);
    # the exhaustive maximum is 0.4029
    assert np.abs(y - ref).max() < 0.41
    assert np.all(np.abs(y) <= 30.0)
    # odd symmetry is exact (the program restores the sign by XOR)
    pos = x[(x < 0x7F80) & (x > 0)]
    yp = oracle.softcap_fwd_bf16(pos, 30.0)
    yn = oracle.softcap_fwd_bf16(pos | np.uint16(0x8000), 30.0)
    assert np.array_equal(yn, yp ^ np.uint16(0x8000)) or np.array_equal(
        oracle.bf16_bits_to_f32(yn), -oracle.bf16_bits_to_f32(yp))


@pytest.mark.parametrize("cap", [30.0, 7.5, 1.0, 0.3])
def test_softcap_forward_is_the_pinned_tanh_program_between_two_roundings(oracle, cap):
    """The softcap composition, step by step from independently pinned
    parts: u = RNE_bf16(float32(s) * float32(1/cap)) with numpy's float32
    product, T = the reference's TANH_FWD_D4_ODD_BF16 program (pinned by its
    own tests), y = RNE_bf16(float32(T) * float32(cap)).  A dropped or moved
    rounding in the oracle's softcap changes outputs: cap * T taken before T
    is rounded differs on 9,734 of the 65,536 patterns at cap 30."""
    x = _all(oracle)
    s = oracle.bf16_bits_to_f32(x)
    with np.errstate(invalid="ignore", over="ignore"):
        u = oracle.f32_to_bf16_bits((s * np.float32(1.0 / np.float32(cap))).astype(np.float32))
        t = oracle.activation("tanh", oracle.FWD, 4, "bf16", u)
        y = oracle.f32_to_bf16_bits((oracle.bf16_bits_to_f32(t) * np.float32(cap)).astype(np.float32))
    got = oracle.softcap_fwd_bf16(x, cap)
    nan = ((got & 0x7F80) == 0x7F80) & ((got & 0x7F) != 0) & ((y & 0x7F80) == 0x7F80) & ((y & 0x7F) != 0)
    assert np.array_equal(got[~nan], y[~nan])


def test_softcap_backward_is_derivative_of_d4_program(oracle):
    x = _all(oracle)
    with np.errstate(invalid="ignore", over="ignore"):
        s = oracle.bf16_bits_to_f32(x).astype(np.float64)
    m = np.isfinite(s)
    ones = np.full(x.size, 0x3F80, dtype=np.uint16)
    g = oracle.bf16_bits_to_f32(oracle.softcap_bwd_bf16(ones, x, 30.0))[m]
    u = s[m] / 30.0
    # derivative of the D4 odd polynomial with the BF16-rounded coefficients
    c = [1.0859375, -0.322265625, -0.0230712891, 0.0164794922]
    t = np.abs(u)
    d = c[0] + 2 * c[1] * t + 3 * c[2] * t ** 2 + 4 * c[3] * t ** 3
    d = np.where(t < 2.609375, d, 0.0)
    assert np.abs(g - d).max() < 0.02          # BF16 Horner rounding only
    assert np.abs(g - (1 - np.tanh(u) ** 2)).max() < 0.16  # vs the exact tanh'


# ---- B5 exp2 ------------------------------------------------------------------

def test_exp2_d2_invariants_and_fit(oracle):
    n = np.arange(-126, 1, dtype=np.float32)
    # p(0) = 1: integers are exact powers of two
    assert np.array_equal(oracle.exp2(0, n, False), np.exp2(n.astype(np.float64)).astype(np.float32))
    # p(1) = 2 continuity: just below an integer the result meets 2^x with
    # no jump between exponent intervals
    # (from -125 up: below -126 the reconstruction lands in FA4's exponent-0
    # band, whose bit pattern keeps only p's mantissa)
    below = np.nextafter(n[1:], np.float32(-np.inf)).astype(np.float32)
    r = oracle.exp2(0, below, False) / np.exp2(below.astype(np.float64))
    assert np.abs(r - 1).max() < 5e-7
    x = np.linspace(-20, 0, 1_000_001, dtype=np.float32)
    rel = np.abs(oracle.exp2(0, x, False) / np.exp2(x.astype(np.float64)) - 1)
    assert 2.0e-3 < rel.max() < 2.8e-3        # appendix_exp2.tex: 2.679e-3
    rel3 = np.abs(oracle.exp2(1, x, False) / np.exp2(x.astype(np.float64)) - 1)
    assert rel3.max() < 1.0e-4                 # FA4 D3: 8.763e-5
    # masking value and clamp; a NaN exponent takes the clamp (max(NaN, -127)
    # is -127), so it gives +0 like a masked score
    low = np.array([-np.inf, -127.0, -1000.0, np.nan, -np.nan], dtype=np.float32)
    for kind in (0, 1):
        got = oracle.exp2(kind, low, False)
        assert got.view(np.uint32).tolist() == [0, 0, 0, 0, 0], (kind, got)
    # the reference's PWL2 hinge starts below one (p(0) = 0.98946), so at its
    # -127 clamp the exponent field wraps into NaN bits (the fused attention
    # kernels clamp PWL2 at -126 for this reason); from -126 up it is positive
    # and at most 2^-126
    assert np.isnan(oracle.exp2(2, low, False)).all()
    edge = np.array([-126.99, -126.98, -126.5, -126.0], dtype=np.float32)
    assert np.isnan(oracle.exp2(2, edge[:1], False)).all()
    tail = oracle.exp2(2, edge[1:], False)
    assert (tail > 0).all() and (tail <= 2.0 ** -126).all()


def _full_f32_error_input():
    """make_full_f32(1 << 20) of autonumerics_zero/cuda_benchmarks/
    benchmark_exp2_pwl2.cu:335-343: pairs (-16 u, -16 v), u = (2i mod
    1048573) / 1048573, v = (2i + 1 mod 1048573) / 1048573, FP32 arithmetic."""
    i = np.arange(1 << 20, dtype=np.int64)
    u = ((2 * i) % 1048573).astype(np.float32) / np.float32(1048573.0)
    v = ((2 * i + 1) % 1048573).astype(np.float32) / np.float32(1048573.0)
    return np.stack([np.float32(-16.0) * u, np.float32(-16.0) * v], axis=1).reshape(-1)


@pytest.mark.parametrize("kind,golden", [
    # evidence/report-data/exp2_pwl2_isolated_gb200.json "errors", domain full_f32
    (1, (8.51484986e-05, 8.76867888e-05, 1.26746955e-05)),   # variant degree3
    (2, (0.0105388165, 0.0105388165, 0.000954319254)),       # variant pwl2_hinge
])
def test_exp2_full_range_errors_match_published_metrics(oracle, kind, golden):
    """max_abs, max_rel and rmse against exp2 in double over the reference
    benchmark's input set (ErrorMetrics, benchmark_exp2_pwl2.cu:306-323),
    reproduced to the printed precision: a dropped term, a wrong coefficient
    or reduction would move them."""
    x = _full_f32_error_input()
    y = oracle.exp2(kind, x, False).astype(np.float64)
    ref = np.exp2(x.astype(np.float64))
    a = np.abs(y - ref)
    got = (a.max(), (a / np.abs(ref)).max(), np.sqrt((a * a).mean()))
    for g, want in zip(got, golden):
        assert abs(g - want) <= 2e-8 * max(1.0, want / 1e-4) + 1e-6 * want, (got, golden)


def _fractional_h2_error_input():
    """make_fractional_h2(1 << 20) of autonumerics_zero/cuda_benchmarks/
    benchmark_exp2_pwl2.cu:325-333: pairs ((2i mod 65521) / 65521,
    (2i + 1 mod 65521) / 65521) in FP32, rounded to FP16."""
    i = np.arange(1 << 20, dtype=np.int64)
    x = (((2 * i) % 65521).astype(np.float32) / np.float32(65521.0)).astype(np.float16)
    y = (((2 * i + 1) % 65521).astype(np.float32) / np.float32(65521.0)).astype(np.float16)
    return np.stack([x, y], axis=1).reshape(-1).astype(np.float32)


def test_exp2_pwl2_f16_reproduces_the_published_fractional_errors(oracle):
    """The reference's FP16 hinge (FractionalPwl2Hinge,
    benchmark_exp2_pwl2.cu:84-99) on its own fractional input set: max_abs,
    max_rel and rmse against exp2 in double (error_fractional_h2, :346-371)
    equal evidence/report-data/exp2_pwl2_isolated_gb200.json "fractional_h2" /
    "pwl2_hinge" to every printed digit.  This pins the FP16 arithmetic the
    packed programs share: RNE to FP16, the hinge's subtract and maximum, and
    two single-rounding FMAs in that order."""
    f = _fractional_h2_error_input()
    p = oracle.exp2_fraction(oracle.EXP2_PWL2_F16, f).astype(np.float64)
    ref = np.exp2(f.astype(np.float64))
    a = np.abs(p - ref)
    got = (a.max(), (a / ref).max(), np.sqrt((a * a).mean()))
    for g, want in zip(got, (0.018854463, 0.010940964, 0.00662452431)):
        assert abs(g - want) <= 5e-10 + 1e-9 * want, (got, want)


def test_exp2_two_segment_historical_reproduces_the_published_fractional_errors(oracle):
    """The reference's historical two-segment FP16 fraction
    (FractionalPwl2Historical, benchmark_exp2_pwl2.cu:60-82) on its fractional
    input set: max_abs, max_rel and rmse against exp2 in double equal
    exp2_pwl2_isolated_gb200.json "fractional_h2" / "pwl2_historical" to every
    printed digit.  Choosing the segment by f >= 1/2 instead of by the rounded
    sum's mantissa bit, or swapping a segment's slope and offset, moves them."""
    f = _fractional_h2_error_input()
    p = oracle.exp2_fraction(oracle.EXP2_FRAC_PWL2_HISTORICAL, f).astype(np.float64)
    ref = np.exp2(f.astype(np.float64))
    a = np.abs(p - ref)
    got = (a.max(), (a / ref).max(), np.sqrt((a * a).mean()))
    for g, want in zip(got, (0.01953125, 0.010940964, 0.00662853655)):
        assert abs(g - want) <= 5e-10 + 1e-9 * want, (got, want)
    # the segment boundary: fp16(f + 1) rounds 0x37FF (just below 1/2) up to 1.5
    below = np.array([np.float16(0.49951171875)], dtype=np.float32)
    assert oracle.exp2_fraction(oracle.EXP2_FRAC_PWL2_HISTORICAL, below)[0] == np.float32(
        np.float16(0.49951171875 * 1.1630859375 + 0.818359375))


@pytest.mark.parametrize("kind,max_rel,lo,hi", [
    # appendix_exp2.tex table: D1 endpoint constrained 6.148e-2
    ("EXP2_PWL1_SAFE", 6.148e-2, 6.1475e-2, 6.1485e-2),
    # the fit errors (PWL1 6.148e-2, PWL2 1.074e-2, D2 2.679e-3) plus the
    # 16-bit rounding of the fraction and of each step
    ("EXP2_PWL1_SAFE_F16", None, 6.148e-2, 6.30e-2),
    ("EXP2_PWL2_SAFE_BF16", None, 1.074e-2, 1.60e-2),
    ("EXP2_D2_SAFE_F16", None, 2.679e-3, 3.4e-3),
    ("EXP2_D2_SAFE_BF16", None, 2.679e-3, 7.0e-3),
])
def test_exp2_remaining_backends_endpoints_and_fit(oracle, kind, max_rel, lo, hi):
    """The remaining FA4 exp2 backends (this build's 16-bit definitions of the
    appendix's forms): p(0) = 1 and p(1) = 2 after their rounding, so every
    integer gives an exact power of two and the value just below an integer
    meets the next power; maximum relative error on the fit's grid within the
    form's published fit error and that error plus the 16-bit rounding."""
    k = getattr(oracle, kind)
    g = np.linspace(0.0, 1.0, 1_000_001)
    p = oracle.exp2_fraction(k, g.astype(np.float32)).astype(np.float64)
    assert p[0] == 1.0 and p[-1] == 2.0
    rel = np.abs(p / np.exp2(g.astype(np.float32).astype(np.float64)) - 1).max()
    assert lo <= rel < hi, rel
    n = np.arange(-126, 9, dtype=np.float32)
    assert np.array_equal(oracle.exp2(k, n, False), np.exp2(n.astype(np.float64)).astype(np.float32))
    low = np.array([-np.inf, -127.0, -1000.0, np.nan], dtype=np.float32)
    assert oracle.exp2(k, low, False).view(np.uint32).tolist() == [0, 0, 0, 0]


def test_exp2_d2_noclamp_is_d2_above_the_clamp(oracle):
    """d2_safe_noclamp is the D2 safe program without the -127 clamp: equal bit
    for bit from -127 up; below it the exponent field wraps (FA4's unsafe
    variant), so a score far below the row maximum is not 0."""
    x = np.concatenate([np.linspace(-127.0, 8.0, 100_001, dtype=np.float32),
                        np.array([0.0, -0.0, -1e-30, -126.5], dtype=np.float32)])
    assert np.array_equal(oracle.exp2(oracle.EXP2_D2_NOCLAMP, x, False).view(np.uint32),
                          oracle.exp2(oracle.EXP2_D2, x, False).view(np.uint32))
    below = oracle.exp2(oracle.EXP2_D2_NOCLAMP, np.array([-130.0, -200.0], dtype=np.float32), False)
    assert (below != 0).all()


def test_exp2_pwl2_safe_coefficients_endpoints_and_published_errors(oracle):
    """B5 PWL2 "safe" hinge p(f) = 1 + a f + c max(f - 1/2, 0)
    (extras/paper/manuscript/appendix_exp2.tex:22-27).

    * The packed FP16 coefficients a = 0.7978515625, c = 0.40380859375
      (appendix_exp2.tex:72-76) are the FP16 roundings of the FP32 sampled-
      minimax fit (evidence/report-data/b5_exp2_softmax_constrained_fits.json,
      two_piece_linear.sampled_minimax: a = 0.7980513010, c = 0.4038973979).
    * Endpoints: p(0) = 1, so integers give exact powers of two; p(1) = 2
      after FP16 rounding, so just below an integer n the FP16 program gives
      exactly 2^n (the fraction rounds to 1.0 in FP16).
    * Published maximum relative errors: the FP16 program 1.132e-2 ("after
      rounding", appendix_exp2.tex:72-76: the fraction rounded to FP16 on the
      fit's 1,000,001-point grid, against exact 2^f), the FP32 program the
      sampled-minimax 1.0739475e-2 of the evidence file.  A dropped hinge, a
      wrong coefficient or FP32 arithmetic in place of FP16 (1.081e-2) moves
      them out of the stated digits.
    """
    f16 = lambda v: float(np.float16(v))
    assert f16(0.7980513010317143) == 0.7978515625 and f16(0.4038973979365714) == 0.40380859375
    n = np.arange(-126, 9, dtype=np.float32)
    for kind in (oracle.EXP2_PWL2_SAFE, oracle.EXP2_PWL2_SAFE_F16):
        assert np.array_equal(oracle.exp2(kind, n, False), np.exp2(n.astype(np.float64)).astype(np.float32))
    below = np.nextafter(n[1:], np.float32(-np.inf)).astype(np.float32)
    assert np.array_equal(oracle.exp2(oracle.EXP2_PWL2_SAFE_F16, below, False),
                          np.exp2(n[1:].astype(np.float64)).astype(np.float32))
    g = np.linspace(0.0, 1.0, 1_000_001)
    x = g.astype(np.float32)
    rel16 = np.abs(oracle.exp2(oracle.EXP2_PWL2_SAFE_F16, x, False) / np.exp2(g) - 1).max()
    assert 1.1315e-2 <= rel16 < 1.1325e-2, rel16
    rel32 = np.abs(oracle.exp2(oracle.EXP2_PWL2_SAFE, x, False) / np.exp2(x.astype(np.float64)) - 1).max()
    assert abs(rel32 - 1.0739475e-2) < 2e-7, rel32
    # the fraction is rounded to FP16 to nearest, ties to even: f = 1/2 +
    # 1.5 ulp16 is a tie and rounds up to 1/2 + 2 ulp16 (RTZ would give + 1)
    ulp = 2.0 ** -11
    tie = oracle.exp2(oracle.EXP2_PWL2_SAFE_F16, np.array([0.5 + 1.5 * ulp, 0.5 + 2 * ulp], np.float32), False)
    assert tie[0] == tie[1]
    # p >= 1 keeps the exponent field from wrapping at the -127 clamp: masked
    # (-inf), NaN and clamped exponents give +0, and [-127, -126] stays in
    # [0, 2^-126]
    low = np.array([-np.inf, -127.0, -1000.0, np.nan], dtype=np.float32)
    edge = np.linspace(-127.0, -126.0, 4097, dtype=np.float32)
    for kind in (oracle.EXP2_PWL2_SAFE, oracle.EXP2_PWL2_SAFE_F16):
        assert oracle.exp2(kind, low, False).view(np.uint32).tolist() == [0, 0, 0, 0]
        e = oracle.exp2(kind, edge, False)
        assert np.isfinite(e).all() and (e >= 0).all() and (e <= 2.0 ** -126).all()


# ---- sin/cos and RoPE -------------------------------------------------------------

@pytest.mark.parametrize("prog,bound", [(0, 1.3e-2), (1, 9e-3), (2, 1e-2), (3, 1.5e-3), (4, 1.2e-3), (5, 1.2e-3)])
def test_half_turn_sincos_error(oracle, prog, bound):
    a = np.linspace(-64.0, 64.0, 400_003, dtype=np.float32)
    c, s = oracle.sincos(prog, a)
    fmt = "bf16" if prog < 2 else "f16"
    cf, sf = oracle.bits_to_f32(c, fmt), oracle.bits_to_f32(s, fmt)
    a64 = a.astype(np.float64)
    err = max(np.abs(cf - np.cos(a64)).max(), np.abs(sf - np.sin(a64)).max())
    assert err < bound, err
    # Pythagorean identity within the evaluation error
    assert np.abs(cf.astype(np.float64) ** 2 + sf.astype(np.float64) ** 2 - 1).max() < 4 * bound


def test_rope_phase_increments_match_reference_convention(oracle):
    inc = oracle.rope_phase_increments(128, 500000.0)
    assert inc.dtype == np.int32 and inc.size == 64
    assert inc[0] == round(2 ** 32 / (2 * math.pi))
    assert (np.diff(inc.astype(np.int64)) < 0).all()


def test_rope_phase_table_accuracy(oracle):
    inc = oracle.rope_phase_increments(128, 500000.0)
    seq = 4096
    t = oracle.rope_sincos_table(inc, seq)
    phase = (np.arange(seq, dtype=np.uint64)[:, None] * inc.astype(np.uint64)[None]) % (1 << 32)
    ang = phase.astype(np.float64) * (2 * math.pi / 2 ** 32)
    err = max(np.abs(oracle.f16_bits_to_f32(t[0]) - np.cos(ang)).max(),
              np.abs(oracle.f16_bits_to_f32(t[1]) - np.sin(ang)).max())
    assert err < 2e-3, err


@pytest.mark.parametrize("fmt", ["f16", "bf16"])
def test_rope_apply_matches_float64_rotation(oracle, fmt):
    rng = np.random.default_rng(4)
    b, s, hq, hk, d = 1, 512, 2, 1, 64
    q = rng.standard_normal((b, s, hq, d)).astype(np.float32)
    k = rng.standard_normal((b, s, hk, d)).astype(np.float32)
    if fmt == "bf16":
        qb, kb = oracle.f32_to_bf16_bits(q), oracle.f32_to_bf16_bits(k)
    else:
        qb, kb = q.astype(np.float16).view(np.uint16), k.astype(np.float16).view(np.uint16)
    inc = oracle.rope_phase_increments(d, 500000.0)
    qo, ko = oracle.rope_apply(fmt, qb, kb, inc)
    dims = np.arange(0, d, 2, dtype=np.float64)
    ang = np.arange(s)[:, None] * (500000.0 ** (-dims / d))[None]
    for src, out in ((qb, qo), (kb, ko)):
        v = oracle.bits_to_f32(src, fmt).astype(np.float64)
        e, o = v[..., 0::2], v[..., 1::2]
        c, sn = np.cos(ang)[None, :, None], np.sin(ang)[None, :, None]
        ref = np.stack((e * c - o * sn, e * sn + o * c), -1).reshape(v.shape).transpose(0, 2, 1, 3)
        got = oracle.bits_to_f32(out, fmt)
        ulp = 2 ** -8 if fmt == "bf16" else 2 ** -11
        assert np.abs(got - ref).max() < np.abs(v).max() * (3e-3 + 2 * ulp)


# ---- FP16 experiments: shared-sigmoid SiLU derivative, multiply ------------------

def test_swish_fwd_deriv_shared_matches_half_precision_arithmetic(oracle):
    """y = x*s, dy = s*fma(x, 1-s, 1) with s = sigmoid D3 (fwd_deriv_swish_kernel,
    spline_kernels.cu:976-1010), restated with numpy float16 (each op correctly
    rounded; the FMA computed exactly in float64, then rounded once)."""
    x = _all(oracle)
    xf = oracle.f16_bits_to_f32(x).astype(np.float16)
    s = oracle.f16_bits_to_f32(oracle.activation("sigmoid", oracle.FWD, 3, "f16", x)).astype(np.float16)
    with np.errstate(over="ignore", invalid="ignore"):
        y = xf * s
        one_minus = np.float16(1.0) - s
        fma = (xf.astype(np.float64) * one_minus.astype(np.float64) + 1.0).astype(np.float16)
        dy = s * fma
    gy, gdy = oracle.swish_fwd_deriv_shared(x)
    fin = np.isfinite(xf)
    assert np.array_equal(gy[fin], y.view(np.uint16)[fin])
    assert np.array_equal(gdy[fin], dy.view(np.uint16)[fin])
    # and it is the SiLU derivative within the sigmoid D3 error (0.02 in s,
    # amplified by |1 + x(1 - s)| <= 1.3 on the fit range)
    xm = xf.astype(np.float64)[fin & (np.abs(xf) < 8)]
    sg = 1 / (1 + np.exp(-xm))
    ref = sg * (1 + xm * (1 - sg))
    got = oracle.f16_bits_to_f32(gdy[fin & (np.abs(xf) < 8)])
    assert np.abs(got - ref).max() < 0.05


@pytest.mark.parametrize("fmt", ["f16", "bf16"])
def test_multiply_is_one_rounding_of_the_product(oracle, fmt):
    rng = np.random.default_rng(11)
    a = rng.integers(0, 65536, 200_000, dtype=np.uint32).astype(np.uint16)
    b = rng.integers(0, 65536, 200_000, dtype=np.uint32).astype(np.uint16)
    got = oracle.multiply(fmt, a, b)
    with np.errstate(over="ignore", invalid="ignore"):
        if fmt == "f16":
            want = (a.view(np.float16) * b.view(np.float16)).view(np.uint16)
        else:
            want = oracle.f32_to_bf16_bits(oracle.bf16_bits_to_f32(a) * oracle.bf16_bits_to_f32(b))
    gv = oracle.bits_to_f32(got, fmt)
    wv = oracle.bits_to_f32(want, fmt)
    both_nan = np.isnan(gv) & np.isnan(wv)
    assert np.array_equal(got[~both_nan], want[~both_nan])
