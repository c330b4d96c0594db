"""CPU pins of the oracle's FP32 and quarter-turn sin/cos programs, their
compute probes and the RoPE quarter-turn / LUT / cached-table paths
(autonumerics_zero/spline_ops/sincos_kernels.cu:24-406, 544-642, 940-978,
1014-1240, 1242-1652).

What pins each program here, beyond the table it shares with the device code:
* accuracy against float64 sin/cos within the error budgets the reference
  states for the same polynomials (tests/test_rope_polynomial_sincos.py:
  D3/D4 phase 1.6e-4 / norm 2.1e-4, D5/D4 1.5e-5 / 4.5e-5, D7/D6 1.2e-7,
  half-turn least squares 1.4e-3 / 9e-4, half-turn Sollya 6.1e-4, one-term
  pi "inside the approximately 1e-3 phase budget" at 8K positions,
  sincos_kernels.cu:96-97): a wrong coefficient, sign or power fails them;
* exact odd/even symmetry, which a wrong quadrant swap or sign fails;
* exact quadrant KATs where the reduced argument is exactly 0;
* the probe sums against the table program at the stepped probe angles;
* the cached-table RoPE against the phase-increment RoPE with the same table.
"""

import math

import numpy as np
import pytest


def _phase_and_norm(c, s, a64):
    c = c.astype(np.float64)
    s = s.astype(np.float64)
    rc, rs = np.cos(a64), np.sin(a64)
    phase = np.arctan2(s * rc - c * rs, c * rc + s * rs)
    return np.abs(phase).max(), np.abs(c * c + s * s - 1).max()


WIDE = np.linspace(-131_072.0, 131_072.0, 262_145, dtype=np.float32)
QUARTER = np.linspace(-math.pi / 4, math.pi / 4, 100_001, dtype=np.float32)
HALF = np.linspace(-math.pi / 2, math.pi / 2, 65_537, dtype=np.float32)

# Fit interval: the reference budgets for these polynomials, unchanged
# (prog, angles, max |phase| rad, max |c^2+s^2-1|).
F32_FIT_BUDGETS = [
    ("SC32_D3D4", QUARTER, 1.6e-4, 2.1e-4),
    ("SC32_D3D4_SHIFT", QUARTER, 1.6e-4, 2.1e-4),
    ("SC32_CYCLE", QUARTER, 1.6e-4, 2.1e-4),
    ("SC32_D5D4", QUARTER, 1.5e-5, 4.5e-5),
    ("SC32_D7D6", QUARTER, 1.2e-7, 2.4e-7),
    ("SC32_HALF_D5D4_LS", HALF, 1.4e-3, 9.0e-4),
    ("SC32_HALF_D5D4_SOLLYA", HALF, 6.1e-4, 1.2e-3),
    ("SC32_HALF_D5D4_SOLLYA_FAST", HALF, 6.1e-4, 1.2e-3),
]

# Wide range: the FP32 reduction (rounding a*2/pi can move the quotient by
# one near half-integers, leaving |r| slightly beyond the fit interval) adds
# a little; the one-term-pi and cycle-domain reductions lose accuracy with
# |angle| (the reference keeps them for RoPE-sized angles).
F32_WIDE_BUDGETS = [
    ("SC32_D3D4", WIDE, 1.6e-4, 2.4e-4),
    ("SC32_D3D4_SHIFT", WIDE, 1.6e-4, 2.4e-4),
    ("SC32_D5D4", WIDE, 1.8e-5, 4.5e-5),
    ("SC32_D7D6", WIDE, 1.2e-7, 2.4e-7),
    ("SC32_HALF_D5D4_LS", WIDE, 1.4e-3, 9.0e-4),
    ("SC32_HALF_D5D4_SOLLYA", WIDE, 7.0e-4, 1.2e-3),
    ("SC32_HALF_D5D4_SOLLYA_FAST", np.linspace(-8192.0, 8192.0, 262_145, dtype=np.float32),
     1.0e-3, 1.2e-3),
    ("SC32_CYCLE", np.linspace(-4096.0, 4096.0, 262_145, dtype=np.float32), 5.5e-4, 2.1e-4),
]


@pytest.mark.parametrize("name,angles,phase_b,norm_b", F32_FIT_BUDGETS + F32_WIDE_BUDGETS,
                         ids=[b[0] + "-fit" for b in F32_FIT_BUDGETS] +
                             [b[0] + "-wide" for b in F32_WIDE_BUDGETS])
def test_f32_programs_meet_the_reference_budgets(oracle, name, angles, phase_b, norm_b):
    prog = getattr(oracle, name)
    c, s = oracle.sincos_f32(prog, angles)
    a64 = angles.astype(np.float64)
    phase, norm = _phase_and_norm(c, s, a64)
    assert phase <= phase_b, phase
    assert norm <= norm_b, norm
    err = max(np.abs(c - np.cos(a64)).max(), np.abs(s - np.sin(a64)).max())
    assert err <= phase_b + norm_b, err


@pytest.mark.parametrize("prog", range(8))
def test_f32_programs_are_exactly_odd_and_even(oracle, prog):
    a = np.random.default_rng(prog).uniform(-3000, 3000, 200_000).astype(np.float32)
    c1, s1 = oracle.sincos_f32(prog, a)
    c2, s2 = oracle.sincos_f32(prog, -a)
    assert np.array_equal(c1, c2)
    assert np.array_equal(s1, -s2)


def test_f32_constant_terms_and_quadrants(oracle):
    zero = np.array([0.0, -0.0], dtype=np.float32)
    # cos(0) is the constant term of each cosine polynomial, sin(+-0) = 0
    # (+-0 through the radian reductions; the cycle program's wrap
    # 0 - rint(0) gives +0 either way)
    for prog, c0 in ((oracle.SC32_D3D4, 0.999990046024322509765625),
                     (oracle.SC32_D5D4, 0.999993085861206),
                     (oracle.SC32_D7D6, 1.0),
                     (oracle.SC32_HALF_D5D4_LS, 0.999579489231109619140625),
                     (oracle.SC32_HALF_D5D4_SOLLYA, 0.9994032382965087890625),
                     (oracle.SC32_CYCLE, 0.999990046024322509765625)):
        c, s = oracle.sincos_f32(prog, zero)
        assert c.tolist() == [np.float32(c0)] * 2
        assert not s.any()
        if prog != oracle.SC32_CYCLE:
            assert np.signbit(s).tolist() == [False, True]
    # one quarter turn per step: the swap and both signs walk through all
    # four quadrants (reference test_reducer_covers_quadrants_and_primary_interval)
    q = np.array([0, 1, 2, 3, 4, -1, -2, -3], dtype=np.float64)
    a = (q * math.pi / 2).astype(np.float32)
    c, s = oracle.sincos_f32(oracle.SC32_D7D6, a)
    assert np.allclose(c, np.cos(q * math.pi / 2), atol=3e-7)
    assert np.allclose(s, np.sin(q * math.pi / 2), atol=3e-7)


def test_f32_shifter_reduction_agrees_with_cody_waite(oracle):
    """Same D3/D4 program, two reductions: they differ only where rounding
    a*2/pi first moves a half-integer quotient (never by more than the
    program's error)."""
    a = np.random.default_rng(5).uniform(-1e4, 1e4, 500_000).astype(np.float32)
    c1, s1 = oracle.sincos_f32(oracle.SC32_D3D4, a)
    c2, s2 = oracle.sincos_f32(oracle.SC32_D3D4_SHIFT, a)
    same = (c1 == c2) & (s1 == s2)
    assert same.mean() > 0.999
    assert max(np.abs(c1 - c2).max(), np.abs(s1 - s2).max()) < 4.2e-4


# ---- 16-bit quarter-turn programs ---------------------------------------------

@pytest.mark.parametrize("prog,fmt,bound", [(6, "f16", 1.0e-3), (7, "bf16", 6e-3), (8, "bf16", 6e-3)])
def test_quarter_turn_16bit_error_and_symmetry(oracle, prog, fmt, bound):
    a = np.linspace(-64.0, 64.0, 400_003, dtype=np.float32)
    c, s = oracle.sincos16(prog, a)
    cf, sf = oracle.bits_to_f32(c, fmt), oracle.bits_to_f32(s, fmt)
    a64 = a.astype(np.float64)
    err = max(np.abs(cf - np.cos(a64)).max(), np.abs(sf - np.sin(a64)).max())
    assert err < bound, err
    c2, s2 = oracle.sincos16(prog, -a)
    assert np.array_equal(c, c2)
    assert np.array_equal(s ^ np.uint16(0x8000), s2)


@pytest.mark.parametrize("prog", [7, 8])
def test_bf16_quarter_fp32_fma_then_rne_equals_single_rounding(oracle, prog):
    """Every BF16 reduced argument in [-pi/4, pi/4] (where the reduction
    returns the angle itself): the FP32 FMA + RNE path of gfx950 gives the
    bits of the single-rounding BF16 FMA."""
    v = oracle.bf16_bits_to_f32(oracle.all_bits())
    with np.errstate(invalid="ignore"):
        a = v[np.isfinite(v) & (np.abs(v) <= 0.78)]
    c1, s1 = oracle.sincos16(prog, a, rnd=oracle.RND_SINGLE)
    c2, s2 = oracle.sincos16(prog, a, rnd=oracle.RND_F32)
    assert np.array_equal(c1, c2) and np.array_equal(s1, s2)


def test_half_turn_ids_match_orc_sincos(oracle):
    a = np.random.default_rng(1).uniform(-50, 50, 10_000).astype(np.float32)
    for prog in range(6):
        assert all(np.array_equal(x, y) for x, y in zip(oracle.sincos16(prog, a), oracle.sincos(prog, a)))


# ---- compute probes ------------------------------------------------------------

def _probe_angles(p0, iterations):
    """p <- fma(p, 0.99999994, 2^-13) in float32 (exact in float64 for the
    magnitudes used here, so one float32 rounding is the FMA)."""
    out = [p0.astype(np.float32)]
    p = p0.astype(np.float32)
    for _ in range(iterations - 1):
        p = (p.astype(np.float64) * 0.999999940395355224609375 + 0.0001220703125).astype(np.float32)
        out.append(p)
    return out


@pytest.mark.parametrize("prog", range(8))
def test_f32_probe_sums_the_table_at_stepped_angles(oracle, prog):
    a = np.random.default_rng(prog).uniform(0.01, 100.0, 4096).astype(np.float32)
    c1, s1 = oracle.sincos_f32(prog, a, iterations=1)
    c0, s0 = oracle.sincos_f32(prog, a)
    assert np.array_equal(c1, c0) and np.array_equal(s1, s0)
    cs, ss = np.zeros_like(a), np.zeros_like(a)
    for p in _probe_angles(a, 5):
        c, s = oracle.sincos_f32(prog, p)
        cs, ss = cs + c, ss + s
    c5, s5 = oracle.sincos_f32(prog, a, iterations=5)
    assert np.array_equal(c5, cs) and np.array_equal(s5, ss)


@pytest.mark.parametrize("prog,fmt", [(0, "bf16"), (1, "bf16"), (2, "f16"), (3, "f16"), (4, "f16"),
                                      (5, "f16"), (6, "f16"), (7, "bf16"), (8, "bf16"), (3, "bf16")])
def test_16bit_probe_sums_the_table_at_stepped_angles(oracle, prog, fmt):
    a = np.random.default_rng(prog).uniform(0.01, 100.0, 4096).astype(np.float32)
    cs = np.zeros(a.size, dtype=np.float32)
    ss = np.zeros(a.size, dtype=np.float32)
    for p in _probe_angles(a, 4):
        c, s = oracle.sincos16(prog, p, out_fmt=fmt)
        cf, sf = oracle.bits_to_f32(c, fmt), oracle.bits_to_f32(s, fmt)
        if fmt == "f16":
            cs = (cs.astype(np.float16) + cf.astype(np.float16)).astype(np.float32)
            ss = (ss.astype(np.float16) + sf.astype(np.float16)).astype(np.float32)
        else:
            cs = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(cs + cf))
            ss = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(ss + sf))
    c4, s4 = oracle.sincos16(prog, a, out_fmt=fmt, iterations=4)
    assert np.array_equal(oracle.bits_to_f32(c4, fmt), cs)
    assert np.array_equal(oracle.bits_to_f32(s4, fmt), ss)


# ---- RoPE quarter turn, LUT, cached table -----------------------------------------

def lut_table():
    """[128, 2] FP16 (sin, cos) of i/128 turn: the table the LUT program
    indexes (sin in the low half of each 32-bit entry)."""
    t = 2 * math.pi * np.arange(128) / 128
    return np.stack((np.sin(t), np.cos(t)), -1).astype(np.float16).view(np.uint16)


def _exact_angles(inc, seq):
    phase = (np.arange(seq, dtype=np.uint64)[:, None] * inc.astype(np.uint32).astype(np.uint64)[None]) % (1 << 32)
    return phase.astype(np.float64) * (2 * math.pi / 2 ** 32)


@pytest.mark.parametrize("kind,bound", [(1, 1.5e-3), (2, 1.3e-3)])
def test_rope_table_programs_accuracy(oracle, kind, bound):
    inc = oracle.rope_phase_increments(128, 500000.0)
    seq = 4096
    t = oracle.rope_table(kind, inc, seq, lut=lut_table() if kind == 2 else None)
    ang = _exact_angles(inc, seq)
    err = max(np.abs(oracle.f16_bits_to_f32(t[0]) - np.cos(ang)).max(),
              np.abs(oracle.f16_bits_to_f32(t[1]) - np.sin(ang)).max())
    assert err < bound, err


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_rope_table_quadrant_kats(oracle, kind):
    # a quarter turn per position: phases 0, 1/4, 1/2, 3/4 turn are exact
    inc = np.array([1 << 30, -(1 << 30)], dtype=np.int32)
    t = oracle.rope_table(kind, inc, 8, lut=lut_table())
    c = oracle.f16_bits_to_f32(t[0])
    s = oracle.f16_bits_to_f32(t[1])
    walk_c = np.array([1, 0, -1, 0] * 2, dtype=np.float32)
    walk_s = np.array([0, 1, 0, -1] * 2, dtype=np.float32)
    tol = 0.0 if kind != 0 else 2e-3
    assert np.abs(c[:, 0] - walk_c).max() <= tol and np.abs(s[:, 0] - walk_s).max() <= tol
    assert np.abs(c[:, 1] - walk_c).max() <= tol and np.abs(s[:, 1] + walk_s).max() <= tol


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_rope_probe_sums_the_table_over_positions(oracle, kind):
    inc = oracle.rope_phase_increments(64, 10000.0)
    seq, it = 64, 5
    lut = lut_table()
    full = oracle.rope_table(kind, inc, seq + it, lut=lut)
    acc = np.zeros((2, seq, inc.size), dtype=np.float16)
    for j in range(it):
        acc = acc + oracle.f16_bits_to_f32(full[:, j:j + seq]).astype(np.float16)
    got = oracle.rope_table(kind, inc, seq, lut=lut, iterations=it)
    assert np.array_equal(got, acc.view(np.uint16))


def test_rope_cached_table_equals_phase_increment_rope(oracle):
    rng = np.random.default_rng(8)
    b, s, hq, hk, d = 2, 96, 3, 2, 64
    q = rng.standard_normal((b, s, hq, d)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((b, s, hk, d)).astype(np.float16).view(np.uint16)
    inc = oracle.rope_phase_increments(d, 500000.0)
    table = oracle.rope_sincos_table(inc, s)
    want = oracle.rope_apply("f16", q, k, inc)
    got = oracle.rope_apply_cached(q, k, table)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
