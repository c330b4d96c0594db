"""The RoPE reference evaluator's oracle (a numpy restatement of
src/sfu_repro/rope/polynomial_sincos.py:85-165) pinned by the reference's own
tests of that evaluator (tests/test_rope_polynomial_sincos.py:77-250), and
the Python module's constants and host-side behaviour."""

import math

import numpy as np
import pytest

from sfu_repro.rope.polynomial_sincos import (
    SOLLYA_D3_D4,
    UNIFORM_D5_D4,
    UNIFORM_D7_D6,
    polynomial_sincos,
)

WIDE = np.linspace(-131_072.0, 131_072.0, 262_145, dtype=np.float32)


def _ref(oracle, angles, poly, accurate=True):
    return oracle.ref_polynomial_sincos(angles, poly.sin_coefficients, poly.cos_coefficients, accurate)


def _phase_norm(cos, sin, angles):
    # the reference compares against torch.cos / torch.sin of the float32 angles
    rc = np.cos(angles.astype(np.float64)).astype(np.float32).astype(np.float64)
    rs = np.sin(angles.astype(np.float64)).astype(np.float32).astype(np.float64)
    c, s = cos.astype(np.float64), sin.astype(np.float64)
    phase = np.arctan2(s * rc - c * rs, c * rc + s * rs)
    return np.abs(phase).max(), np.abs(c * c + s * s - 1).max()


def test_polynomial_degrees_and_coefficient_budget():
    assert (SOLLYA_D3_D4.sin_degree, SOLLYA_D3_D4.cos_degree) == (3, 4)
    assert (UNIFORM_D5_D4.sin_degree, UNIFORM_D5_D4.cos_degree) == (5, 4)
    assert (UNIFORM_D7_D6.sin_degree, UNIFORM_D7_D6.cos_degree) == (7, 6)
    assert [len(p.sin_coefficients) + len(p.cos_coefficients)
            for p in (SOLLYA_D3_D4, UNIFORM_D5_D4, UNIFORM_D7_D6)] == [5, 6, 8]


def test_d3_d4_candidate_is_within_bfloat16_rotation_budget(oracle):
    cos, sin = _ref(oracle, WIDE, SOLLYA_D3_D4)
    phase, norm = _phase_norm(cos, sin, WIDE)
    assert phase <= 1.6e-4 and norm <= 2.1e-4


def test_accurate_polynomial_matches_float32_sincos_over_wide_range(oracle):
    cos, sin = _ref(oracle, WIDE, UNIFORM_D7_D6)
    a64 = WIDE.astype(np.float64)
    assert np.abs(cos - np.cos(a64).astype(np.float32)).max() <= 1.2e-7
    assert np.abs(sin - np.sin(a64).astype(np.float32)).max() <= 1.2e-7
    assert np.abs(cos.astype(np.float64) ** 2 + sin.astype(np.float64) ** 2 - 1).max() <= 2.4e-7


def test_d5_d4_candidate_is_within_bfloat16_rotation_budget(oracle):
    cos, sin = _ref(oracle, WIDE, UNIFORM_D5_D4)
    phase, norm = _phase_norm(cos, sin, WIDE)
    assert phase <= 1.5e-5 and norm <= 4.5e-5


def test_reducer_covers_quadrants_and_primary_interval(oracle):
    angles = np.array([-2 * math.pi, -math.pi, -math.pi / 2, 0.0, math.pi / 2, math.pi], dtype=np.float32)
    reduced, quadrant = oracle.ref_reduce_to_quarter_turn(angles)
    assert np.abs(reduced).max() <= math.pi / 4
    assert quadrant.tolist() == [0, 2, 3, 0, 1, 2]


def test_fast_reducer_has_explicit_long_context_error_bound(oracle):
    angles = np.linspace(0.0, 8192.0, 262_145, dtype=np.float32)
    ac, as_ = _ref(oracle, angles, UNIFORM_D7_D6)
    fc, fs = _ref(oracle, angles, UNIFORM_D7_D6, accurate=False)
    err = max(np.abs(fc - ac).max(), np.abs(fs - as_).max())
    assert 1.0e-5 < err < 3.0e-4


def test_polynomial_table_and_rotation_match_complex_reference(oracle):
    head_dim = 128
    dims = np.arange(0, head_dim, 2, dtype=np.float64)
    freq = 500_000.0 ** (-dims / head_dim)
    angles = np.outer(np.arange(8192, dtype=np.float64), freq)
    cos, sin = _ref(oracle, angles, UNIFORM_D7_D6)
    assert max(np.abs(cos - np.cos(angles).astype(np.float32)).max(),
               np.abs(sin - np.sin(angles).astype(np.float32)).max()) <= 1.2e-7
    rng = np.random.default_rng(1234)
    v = rng.standard_normal((1, 512, 4, head_dim)).astype(np.float32)
    e, o = v[..., 0::2].astype(np.float64), v[..., 1::2].astype(np.float64)
    c32, s32 = cos[None, :512, None], sin[None, :512, None]
    cand = np.stack((e * c32 - o * s32, e * s32 + o * c32), -1).reshape(v.shape)
    cc, ss = np.cos(angles[:512])[None, :, None], np.sin(angles[:512])[None, :, None]
    ref = np.stack((e * cc - o * ss, e * ss + o * cc), -1).reshape(v.shape)
    assert np.abs(cand - ref).max() <= 6e-7 + 1e-6 * np.abs(ref).max()


def test_evaluator_refuses_host_tensors():
    torch = pytest.importorskip("torch")
    with pytest.raises(RuntimeError, match="must be on the HIP device"):
        polynomial_sincos(torch.zeros(4))
    with pytest.raises(TypeError, match="floating-point"):
        polynomial_sincos(torch.zeros(4, dtype=torch.int32))


def _fixture():
    import json
    import os

    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "rope_evaluator.json")) as f:
        return json.load(f)


def _canonical(a):
    b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).copy()
    b[np.isnan(a)] = 0x7FC00000
    return b


def test_oracle_equals_the_reference_module_bit_for_bit(oracle):
    """tests/golden/rope_evaluator.json holds the reference module's own
    outputs (src/sfu_repro/rope/polynomial_sincos.py run on CPU torch by
    tests/golden/make_rope_evaluator_fixture.py) for FP32 and FP64 angles, the
    three coefficient sets and both reductions; the oracle reproduces every
    cos and sin bit pattern (SHA-256 over 131,122 angles, plus sampled
    values for a readable diff)."""
    import hashlib

    from golden.make_rope_evaluator_fixture import angle_set

    doc = _fixture()
    angles = angle_set()
    assert angles.size == doc["count"] and len(doc["cases"]) == 12
    polys = {"SOLLYA_D3_D4": SOLLYA_D3_D4, "UNIFORM_D5_D4": UNIFORM_D5_D4, "UNIFORM_D7_D6": UNIFORM_D7_D6}
    step = doc["sample_step"]
    with np.errstate(over="ignore", invalid="ignore"):
        for case in doc["cases"]:
            poly = polys[case["polynomial"]]
            cos, sin = _ref(oracle, angles.astype(case["dtype"]), poly, case["accurate"])
            cb, sb = _canonical(cos), _canonical(sin)
            what = (case["dtype"], case["polynomial"], case["accurate"])
            assert cb[::step].tolist() == case["cos_sample"], what
            assert sb[::step].tolist() == case["sin_sample"], what
            assert hashlib.sha256(cb.tobytes()).hexdigest() == case["cos_sha256"], what
            assert hashlib.sha256(sb.tobytes()).hexdigest() == case["sin_sha256"], what
