"""Float32 paired sin/cos evaluator for RoPE tables, on the HIP device.

Same names, coefficient sets, arguments and results as the reference's
``src/sfu_repro/rope/polynomial_sincos.py:13-165``.  The arithmetic runs in
one HIP kernel (``spline_ops.polynomial_sincos_f32``) that keeps the
reference's operation sequence: the "accurate" reduction in FP64
(``q = round(a * 2/pi)``, ``r = a - q * pi/2``, then FP32), the fast one in
FP32 with a two-term Cody-Waite pi/2, and Horner steps ``v * x + c`` that
round after the product and after the sum.  Inputs must live on the HIP
device; there is no host evaluation.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ..activations import load_spline_ops


@dataclass(frozen=True)
class SincosPolynomial:
    """Parity-preserving polynomial pair on [-pi/4, pi/4]: sin(r) = r * P(r^2),
    cos(r) = Q(r^2), coefficients lowest power first."""

    sin_coefficients: tuple[float, ...]
    cos_coefficients: tuple[float, ...]
    fit_name: str

    @property
    def sin_degree(self) -> int:
        return 2 * len(self.sin_coefficients) - 1

    @property
    def cos_degree(self) -> int:
        return 2 * (len(self.cos_coefficients) - 1)


# The reference's fitted coefficient sets (polynomial_sincos.py:35-81): a
# Sollya fpminimax D3/D4 pair (float32 coefficients, BF16 rotation budget)
# and uniform least-squares D5/D4 and D7/D6 controls.
SOLLYA_D3_D4 = SincosPolynomial(
    sin_coefficients=(0.9990314245223999, -0.16034401953220367),
    cos_coefficients=(0.9999900460243225, -0.4997082054615021, 0.04039861634373665),
    fit_name="sollya_fpminimax_d3_d4_f32",
)

UNIFORM_D5_D4 = SincosPolynomial(
    sin_coefficients=(0.9999962449073792, -0.16661198437213898, 0.008137642405927181),
    cos_coefficients=(0.999993085861206, -0.499763548374176, 0.04051213711500168),
    fit_name="uniform_d5_d4_f32",
)

UNIFORM_D7_D6 = SincosPolynomial(
    sin_coefficients=(1.0, -0.1666664183139801, 0.00833179522305727, -0.00019484198128338903),
    cos_coefficients=(1.0, -0.49999886751174927, 0.041656624525785446, -0.0013605882413685322),
    fit_name="uniform_d7_d6_f32",
)


def _device_tensor(t: torch.Tensor, name: str) -> torch.Tensor:
    if not torch.is_floating_point(t):
        raise TypeError(f"{name} must be a floating-point tensor")
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{name} must be on the HIP device: this evaluator runs as a HIP kernel "
            f"(move it with {name}.cuda())")
    return t


def reduce_to_quarter_turn(
    angles: torch.Tensor,
    *,
    accurate: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Reduce angles to about [-pi/4, pi/4]; returns (float32 residual,
    int64 quadrant in 0..3).  ``accurate`` reduces in FP64 (for cached
    tables); the fast path stays in FP32 and its residual error grows with
    |angle| (polynomial_sincos.py:85-122)."""
    angles = _device_tensor(angles, "angles")
    reduced, quadrant = load_spline_ops().reduce_to_quarter_turn_f32(angles, accurate)
    return reduced, quadrant


def evaluate_reduced_sincos(
    reduced: torch.Tensor,
    polynomial: SincosPolynomial = UNIFORM_D7_D6,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(sin, cos) of the paired parity polynomials on reduced arguments, in
    float32 (polynomial_sincos.py:125-135)."""
    reduced = _device_tensor(reduced, "reduced")
    sin_r, cos_r = load_spline_ops().evaluate_reduced_sincos_f32(
        reduced, list(polynomial.sin_coefficients), list(polynomial.cos_coefficients))
    return sin_r, cos_r


def polynomial_sincos(
    angles: torch.Tensor,
    *,
    polynomial: SincosPolynomial = UNIFORM_D7_D6,
    accurate_reduction: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Sine and cosine together from one range reduction; returns (cos, sin)
    to match the packed Real-RoPE table convention.  Evaluation is float32
    whatever the angle dtype (polynomial_sincos.py:138-165)."""
    angles = _device_tensor(angles, "angles")
    cos, sin = load_spline_ops().polynomial_sincos_f32(
        angles, list(polynomial.sin_coefficients), list(polynomial.cos_coefficients),
        accurate_reduction)
    return cos, sin
