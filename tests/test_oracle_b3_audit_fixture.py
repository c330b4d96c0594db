"""The B3 oracle against the reference's own CPU emulation, bit for bit.

``tests/golden/b3_audit_table.npz`` holds the output of
``evaluate_deployed`` (scripts/audit_b3_deployed_fit.py:341-366) on every BF16
input, written by ``tests/golden/make_b3_audit_fixture.py``.  The oracle's
restatement must reproduce y, dy and the row index on all 65,536 patterns
(NaN dy compared as NaN).  A planted variant of the oracle that keeps only the
last of the four Horner roundings must fail the same comparison: that shows
the fixture pins the rounding sequence, which the known-answer tests of
test_oracle_b3.py do not.
"""

import hashlib
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _fixture():
    with open(os.path.join(GOLDEN, "b3_audit_table.json")) as f:
        doc = json.load(f)
    t = np.load(os.path.join(GOLDEN, "b3_audit_table.npz"))
    for k in ("y", "dy", "row"):
        assert hashlib.sha256(t[k].tobytes()).hexdigest() == doc["sha256"][k], k
    return t["y"], t["dy"], t["row"], doc


def _is_nan_bf16(b):
    return ((b & 0x7F80) == 0x7F80) & ((b & 0x007F) != 0)


def test_fixture_constants_are_the_ptx_immediates(oracle):
    _, _, _, doc = _fixture()
    fwd, grad, _ = oracle.b3_constants()
    got_fwd = [[float(v) for v in oracle.bf16_bits_to_f32(np.array(r, dtype=np.uint16))] for r in fwd]
    got_grad = [[float(v) for v in oracle.bf16_bits_to_f32(np.array(r, dtype=np.uint16))] for r in grad]
    assert got_fwd == doc["deployed_forward_rows"]
    assert got_grad == doc["deployed_gradient_factors"]


def test_oracle_equals_reference_emulation_on_every_input(oracle):
    fy, fdy, frow, _ = _fixture()
    x = oracle.all_bits()
    y, dy, row = oracle.b3_direct_bf16(x, with_row=True)
    assert np.array_equal(row, frow)
    assert np.array_equal(y, fy), np.flatnonzero(y != fy)[:8]
    nan_f = _is_nan_bf16(fdy)
    assert np.array_equal(_is_nan_bf16(dy), nan_f)
    assert np.array_equal(dy[~nan_f], fdy[~nan_f]), np.flatnonzero((dy != fdy) & ~nan_f)[:8]
    # the NaN rows are exactly the NaN scores: y = max(0, NaN) = 0, dy = NaN
    x_nan = _is_nan_bf16(x)
    assert np.array_equal(nan_f, x_nan)
    assert (fy[x_nan] == 0).all()


def _dropped_rounding_variant(oracle, x):
    """B3 with the intermediate Horner roundings removed (only the last kept):
    a planted mistake in a CPU restatement, not a program of this build."""
    fwd, grad, sc = oracle.b3_constants()
    xf = oracle.bf16_bits_to_f32(x).astype(np.float64)
    split = float(oracle.bf16_bits_to_f32(np.array([sc[0]], dtype=np.uint16))[0])
    clamp = float(oracle.bf16_bits_to_f32(np.array([sc[1]], dtype=np.uint16))[0])
    row = (xf >= split).astype(np.int64)
    xc = np.clip(xf, -clamp, clamp)
    c = np.stack([oracle.bf16_bits_to_f32(np.array(r, dtype=np.uint16)).astype(np.float64) for r in fwd])
    v = c[row, 3]
    for k in (2, 1, 0):
        v = xc * v + c[row, k]
    y = oracle.f32_to_bf16_bits(np.maximum(v, 0.0).astype(np.float32))
    return y


def test_fixture_rejects_a_dropped_rounding_variant(oracle):
    fy, _, _, _ = _fixture()
    x = oracle.all_bits()
    finite = ~_is_nan_bf16(x)
    y_bad = _dropped_rounding_variant(oracle, x[finite])
    assert int((y_bad != fy[finite]).sum()) > 100
