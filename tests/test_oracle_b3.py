"""The B3 oracle against the reference's known answers and the mathematics.

Known answers: tests/test_audit_b3_deployed_fit.py:16-74 of the reference
(RNE ties, manifest constants, x = 0, x = split, clamp saturation) and the
hand-written PTX immediates of extras/paper/manuscript/main.tex:1046-1111.
"""

import math

import numpy as np


def bf(oracle, values):
    return oracle.f32_to_bf16_bits(np.asarray(values, dtype=np.float32))


def test_bf16_rounds_halfway_values_to_even(oracle):
    # test_audit_b3_deployed_fit.py:16-19
    for value, want in ((1.00390625, 1.0), (1.01171875, 1.015625), (-1.00390625, -1.0)):
        got = oracle.bf16_bits_to_f32(np.array([oracle.lib().orc_f32_to_bf16_audit(value)],
                                               dtype=np.uint16))[0]
        assert got == want


def test_deployed_constants_match_ptx_immediates(oracle):
    # lop3 selects: row1 ? A : B, immediates main.tex:1094-1107
    fwd, grad, sc = oracle.b3_constants()
    assert [hex(v) for v in fwd[0]] == ["0x3980", "0x3987", "0x3909", "0x37e8"]
    assert [hex(v) for v in fwd[1]] == ["0xbb09", "0x3b8c", "0xbb11", "0x3a09"]
    assert [hex(v) for v in grad[0]] == ["0x3f80", "0xbc10"]
    assert [hex(v) for v in grad[1]] == ["0x3f81", "0xbb38"]
    assert [hex(v) for v in sc] == ["0x3fa0", "0x40c0"]


def test_zero_split_and_clamp_known_answers(oracle):
    x = bf(oracle, [0.0, 1.25, -20.0, -6.0, 20.0, 6.0])
    y, dy, row = oracle.b3_direct_bf16(x, with_row=True)
    yf, df = oracle.bf16_bits_to_f32(y), oracle.bf16_bits_to_f32(dy)
    # x = 0: row 0, y = bf16(1/4096), factor 1 so dy == y  (:51-55)
    assert row[0] == 0 and yf[0] == np.float32(1.0 / 4096) and df[0] == yf[0]
    # x = split: row 1  (:57-62)
    assert row[1] == 1
    # saturation beyond the clamp  (:64-74)
    assert y[2] == y[3] and dy[2] == dy[3]
    assert y[4] == y[5] and dy[4] == dy[5]


def test_split_is_inclusive_and_row_boundary(oracle):
    below = np.array([0x3F9F], dtype=np.uint16)  # largest BF16 below 1.25
    _, _, r = oracle.b3_direct_bf16(below, with_row=True)
    assert r[0] == 0


def test_nan_follows_python_semantics(oracle):
    y, dy = oracle.b3_direct_bf16(np.array([0x7FC0, 0xFFC0], dtype=np.uint16))
    assert (y == 0).all()
    assert np.isnan(oracle.bf16_bits_to_f32(dy)).all()


def test_factored_derivative_is_y_times_affine_factor(oracle):
    """dy == bf16(y * bf16(fma(x, slope, intercept))) recomputed from the
    single-rounding FMA primitive (independent of the audit FMA path)."""
    x = oracle.all_bits()
    y, dy, row = oracle.b3_direct_bf16(x, with_row=True)
    _, grad, sc = oracle.b3_constants()
    xf = oracle.bf16_bits_to_f32(x)
    finite = np.isfinite(xf)
    lib = oracle.lib()
    for i in np.flatnonzero(finite)[::97]:
        xc = np.clip(xf[i], -6.0, 6.0)
        xcb = int(bf(oracle, [xc])[0])
        fac = lib.orc_fma16(oracle.BF16, xcb, int(grad[row[i]][1]), int(grad[row[i]][0]))
        want = oracle.f32_to_bf16_bits(np.array([oracle.bf16_bits_to_f32(np.array([y[i]]))[0]
                                                  * oracle.bf16_bits_to_f32(np.array([fac]))[0]],
                                                 dtype=np.float32))[0]
        assert dy[i] == want


def test_fit_error_against_exact_sigmoid_target(oracle):
    """|y - sigmoid(s - ln 4096)| and |dy - p(1-p)| (exact_targets, audit
    :369-377).  The deployed fit is tight for scores up to 4 and loosens
    toward the clamp at 6, where the cubic of row 1 reaches 0.0568 against
    the exact 0.0896; both figures are properties of the deployed constants."""
    x = oracle.all_bits()
    with np.errstate(invalid='ignore'):
        xf = oracle.bf16_bits_to_f32(x).astype(np.float64)
    fin = np.isfinite(xf)
    for hi, bound in ((4.0, 2.5e-4), (6.0, 3.5e-2)):
        m = fin & (xf >= -6.0) & (xf <= hi)
        y, dy = oracle.b3_direct_bf16(x[m])
        p = 1.0 / (1.0 + np.exp(-(xf[m] - math.log(4096.0))))
        err_y = np.abs(oracle.bf16_bits_to_f32(y) - p).max()
        err_d = np.abs(oracle.bf16_bits_to_f32(dy) - p * (1 - p)).max()
        assert err_y < bound, (hi, err_y)
        assert err_d < bound, (hi, err_d)
    # the value at the clamp is the row-1 cubic evaluated at 6
    y6, _ = oracle.b3_direct_bf16(bf(oracle, [6.0]))
    cubic = (-8.5625 + 17.5 * 6 - 9.0625 * 36 + 2.140625 * 216) / 4096
    assert abs(float(oracle.bf16_bits_to_f32(y6)[0]) - cubic) < 2e-4
