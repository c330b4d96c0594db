"""GPU parity of the RoPE reference evaluator (sfu_repro.rope.polynomial_sincos
on the HIP device) against its numpy oracle, bit for bit, for FP32, FP64 and
FP16 angles, both reductions and the three coefficient sets; and the
reference's own accuracy checks on the device results."""

import math

import numpy as np
import pytest
import torch

from sfu_repro.rope.polynomial_sincos import (
    SOLLYA_D3_D4,
    UNIFORM_D5_D4,
    UNIFORM_D7_D6,
    SincosPolynomial,
    evaluate_reduced_sincos,
    polynomial_sincos,
    reduce_to_quarter_turn,
)

pytestmark = pytest.mark.gpu

POLYS = [SOLLYA_D3_D4, UNIFORM_D5_D4, UNIFORM_D7_D6,
         SincosPolynomial((1.0,), (1.0, -0.5), "tiny"),
         SincosPolynomial(tuple(1.0 / math.factorial(2 * k + 1) * (-1) ** k for k in range(8)),
                          tuple(1.0 / math.factorial(2 * k) * (-1) ** k for k in range(8)), "taylor8")]


def _angles():
    rng = np.random.default_rng(12)
    return np.concatenate([
        np.linspace(-131_072.0, 131_072.0, 65_537),
        rng.uniform(-8192, 8192, 65_536),
        np.arange(-20, 21) * (math.pi / 4),
        [0.0, -0.0, 1e-40, 3e7, -1e12, np.inf, -np.inf, np.nan],
    ])


def _same(got: torch.Tensor, want: np.ndarray, what: str):
    g = got.cpu().numpy()
    assert g.dtype == want.dtype, (what, g.dtype, want.dtype)
    nan = np.isnan(g) & np.isnan(want) if g.dtype.kind == "f" else np.zeros(g.shape, bool)
    bad = (g.view(np.uint8).reshape(g.size, -1) != want.view(np.uint8).reshape(want.size, -1)).any(1)
    bad &= ~nan.reshape(-1)
    assert not bad.any(), f"{what}: {bad.sum()} differ, first {np.flatnonzero(bad)[:5].tolist()}"


@pytest.mark.parametrize("accurate", [True, False])
@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.float16])
@pytest.mark.parametrize("poly", POLYS, ids=[p.fit_name for p in POLYS])
def test_polynomial_sincos_parity(oracle, cuda, poly, dtype, accurate):
    with np.errstate(over="ignore", invalid="ignore"):
        a = _angles().astype(dtype)
    ad = torch.from_numpy(a).to(cuda)
    cos, sin = polynomial_sincos(ad, polynomial=poly, accurate_reduction=accurate)
    src = a.astype(np.float32) if dtype == np.float16 else a
    wc, ws = oracle.ref_polynomial_sincos(src, poly.sin_coefficients, poly.cos_coefficients, accurate)
    _same(cos, wc, f"cos {poly.fit_name}")
    _same(sin, ws, f"sin {poly.fit_name}")


@pytest.mark.parametrize("accurate", [True, False])
def test_reduce_and_evaluate_parity(oracle, cuda, accurate):
    a = _angles()
    r, q = reduce_to_quarter_turn(torch.from_numpy(a).to(cuda), accurate=accurate)
    wr, wq = oracle.ref_reduce_to_quarter_turn(a, accurate)
    _same(r, wr, "reduced")
    assert q.dtype == torch.int64 and np.array_equal(q.cpu().numpy(), wq)
    s, c = evaluate_reduced_sincos(r, UNIFORM_D5_D4)
    ws, wc = oracle.ref_evaluate_reduced_sincos(wr, UNIFORM_D5_D4.sin_coefficients,
                                                UNIFORM_D5_D4.cos_coefficients)
    _same(s, ws, "sin reduced")
    _same(c, wc, "cos reduced")


def test_reference_accuracy_checks_on_device(cuda):
    angles = torch.linspace(-131_072.0, 131_072.0, 262_145, device=cuda)
    cos, sin = polynomial_sincos(angles)
    torch.testing.assert_close(cos, torch.cos(angles.double()).float(), rtol=0.0, atol=1.2e-7)
    torch.testing.assert_close(sin, torch.sin(angles.double()).float(), rtol=0.0, atol=1.2e-7)
    reduced, quadrant = reduce_to_quarter_turn(
        torch.tensor([-2 * math.pi, -math.pi, -math.pi / 2, 0.0, math.pi / 2, math.pi], device=cuda))
    assert reduced.abs().max().item() <= math.pi / 4
    assert quadrant.tolist() == [0, 2, 3, 0, 1, 2]
    with pytest.raises(RuntimeError, match="1 to 8 coefficients"):
        polynomial_sincos(angles[:4], polynomial=SincosPolynomial(tuple([1.0] * 9), (1.0,), "x"))


def test_device_evaluator_equals_the_reference_module(cuda):
    """The device evaluator against the reference module's own CPU outputs
    (tests/golden/rope_evaluator.json, written from
    src/sfu_repro/rope/polynomial_sincos.py by
    tests/golden/make_rope_evaluator_fixture.py): every cos / sin bit over
    131,122 FP32 and FP64 angles, three coefficient sets, both reductions."""
    import hashlib
    import json
    import os

    from golden.make_rope_evaluator_fixture import angle_set

    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "rope_evaluator.json")) as f:
        doc = json.load(f)
    polys = {"SOLLYA_D3_D4": SOLLYA_D3_D4, "UNIFORM_D5_D4": UNIFORM_D5_D4, "UNIFORM_D7_D6": UNIFORM_D7_D6}
    angles = angle_set()

    def canon(t):
        a = t.cpu().numpy()
        b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).copy()
        b[np.isnan(a)] = 0x7FC00000
        return b

    for case in doc["cases"]:
        a = torch.from_numpy(angles.astype(case["dtype"])).to(cuda)
        cos, sin = polynomial_sincos(a, polynomial=polys[case["polynomial"]], accurate_reduction=case["accurate"])
        cb, sb = canon(cos), canon(sin)
        what = (case["dtype"], case["polynomial"], case["accurate"])
        assert cb[::doc["sample_step"]].tolist() == case["cos_sample"], what
        assert sb[::doc["sample_step"]].tolist() == case["sin_sample"], what
        assert hashlib.sha256(cb.tobytes()).hexdigest() == case["cos_sha256"], what
        assert hashlib.sha256(sb.tobytes()).hexdigest() == case["sin_sha256"], what
