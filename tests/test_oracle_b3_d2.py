"""The B3-D2 (sigmoid via range-reduced degree-2 exp2) oracle against the
reference fitter's own output.

tests/golden/b3_d2_coefficients.json holds the coefficients and metrics that
autonumerics_zero/evolution/fit_flash_sigmoid_exp2_d2.py produced when run
with its defaults (written by tests/golden/make_b3_d2_fixture.py).  The
fitter's metrics are recomputed here from the oracle's probabilities on the
fitter's grid: a different exponent offset, a swapped coefficient or a wrong
reduction would change them."""

import json
import math
import os

import numpy as np
import pytest

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "b3_d2_coefficients.json")


@pytest.fixture(scope="module")
def fit():
    with open(FIXTURE) as f:
        return json.load(f)


def test_fixture_coefficients_are_float32(fit):
    c = np.array(fit["coefficients_float32"], dtype=np.float32)
    assert ["0x%08X" % v for v in c.view(np.uint32)] == fit["coefficients_hex"]
    # the fitter's p(0) = c0 and endpoint jump |c0 + c1 + c2 - 2 c0|
    assert abs(float(c[0]) + float(c[1]) + float(c[2]) - 2 * float(c[0])) == pytest.approx(
        fit["metrics"]["endpoint_jump"], abs=1e-7)


def test_oracle_reproduces_fitter_metrics(oracle, fit):
    """forward / gradient relative L1 (weights N(0,1), grid [-7, 7] x 28001)
    and the central max relative error, from the oracle's FP32 probability
    before BF16 output rounding (recovered by evaluating on FP32 grid points
    that are exact BF16 values is not possible, so the check uses the
    oracle's BF16 outputs with a tolerance of the output rounding)."""
    c = fit["coefficients_float32"]
    n = fit["sequence_length"]
    scores = np.linspace(-7.0, 7.0, 28_001)
    xb = oracle.f32_to_bf16_bits(scores.astype(np.float32))
    s = oracle.bf16_bits_to_f32(xb).astype(np.float64)   # the BF16 scores actually evaluated
    y, dy = oracle.b3_exp2_d2_bf16(xb, c)
    p = oracle.bf16_bits_to_f32(y).astype(np.float64)
    g = oracle.bf16_bits_to_f32(dy).astype(np.float64)
    w = np.exp(-0.5 * s ** 2)
    exp_p = 1.0 / (1.0 + np.exp(-(s - math.log(n))))
    exp_g = exp_p * (1 - exp_p)
    fwd_l1 = np.sum(w * np.abs(p - exp_p)) / np.sum(w * exp_p)
    grad_l1 = np.sum(w * np.abs(g - exp_g)) / np.sum(w * exp_g)
    central = np.abs(s) <= 5.0
    cmax = np.max(np.abs(p[central] - exp_p[central]) / exp_p[central])
    m = fit["metrics"]
    # BF16 output rounding adds at most 2^-9 relative per value
    assert fwd_l1 == pytest.approx(m["forward_relative_l1"], abs=2 ** -9)
    assert grad_l1 == pytest.approx(m["gradient_relative_l1"], abs=2 ** -9)
    assert cmax == pytest.approx(m["central_max_relative"], abs=2 ** -8)
    assert cmax > 0.02  # the fit is loose at the edges of the central band


def test_exact_powers_and_scaling(oracle, fit):
    """At scores where s*log2(e) is an integer k the mantissa is c0, so
    y = bf16(c0 * 2^(k-12)) exactly."""
    c = fit["coefficients_float32"]
    x = oracle.f32_to_bf16_bits(np.array([0.0], dtype=np.float32))
    y, _ = oracle.b3_exp2_d2_bf16(x, c)
    assert oracle.bf16_bits_to_f32(y)[0] == oracle.bf16_bits_to_f32(
        oracle.f32_to_bf16_bits(np.array([c[0] / 4096], dtype=np.float32)))[0]
