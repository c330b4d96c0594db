"""The oracle's program tables equal the reference's coefficient headers
literal for literal: for every activation struct of
spline_structs_odd.cuh (FP16), spline_structs_odd_bf16.cuh (BF16) and
spline_structs_sollya_bf16.cuh (BF16 Sollya set), the clamp Lc and each
coefficient c0..cN, as float32 values of the decimal literals that the
headers convert with __float2half2_rn / __float2bfloat162_rn, and the
composed structs (SiLU = x * sigmoid) call the sigmoid program of the same
degree; and the paired sin/cos programs' tables equal the float literals of
the corresponding sincos_kernels.cu programs, in order.  The literals come
from tests/golden/struct_coefficients.json (written by
make_struct_coefficients_fixture.py beside it).

The GPU parity tests compare the HIP programs with the oracle bit for bit
on every input, so this pins the kernels' tables too.  ERF structs (no
launcher or binding in the reference) and the algebraic derivatives (no
coefficients) are not programs of this build's tables."""

import json
import os
import re

import numpy as np
import pytest

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "struct_coefficients.json")
NAME = re.compile(r"^(SIGMOID|TANH|SWISH|GELU)_(FWD|BWD)_D(\d)_(ODD|EVEN)(_SOLLYA)?(_BF16)?$")


def _structs():
    with open(FIXTURE) as f:
        d = json.load(f)
    out = []
    for fn, structs in sorted(d["structs"].items()):
        for name, entry in sorted(structs.items()):
            if NAME.match(name):
                out.append((fn, name, entry))
    return out


STRUCTS = _structs()


def test_fixture_covers_every_program():
    # 4 families x 2 directions x 4 degrees per header
    by_file = {}
    for fn, name, _ in STRUCTS:
        by_file.setdefault(fn, set()).add(name)
    assert {fn: len(v) for fn, v in by_file.items()} == {
        "spline_structs_odd.cuh": 32, "spline_structs_odd_bf16.cuh": 32, "spline_structs_sollya_bf16.cuh": 32}


@pytest.mark.parametrize("fn,name,entry", STRUCTS, ids=[f"{n}" for _, n, _ in STRUCTS])
def test_oracle_table_equals_header_literals(oracle, fn, name, entry):
    fam, direction, degree, _, sollya, bf16 = NAME.match(name).groups()
    fmt = "bf16_sollya" if sollya else ("bf16" if bf16 else "f16")
    shape, lc, deg, coeffs = oracle.program(fam.lower(), 0 if direction == "FWD" else 1, int(degree), fmt)
    if "c" not in entry:
        # composed: x * SIGMOID_FWD_D<degree>
        assert shape == "x_times", (name, shape)
        assert entry.get("calls") == [f"SIGMOID_FWD_D{degree}_ODD{sollya or ''}{bf16 or ''}"], entry
        return
    assert deg == int(degree), (name, deg)
    assert np.float32(lc) == np.float32(float(entry["lc"])), (name, lc, entry["lc"])
    for k in range(deg + 1):
        lit = entry["c"].get(f"c{k}")
        want = np.float32(float(lit)) if lit is not None else np.float32(0.0)
        assert np.float32(coeffs[k]) == want, (name, k, coeffs[k], lit)


# ---- paired sin/cos programs (sincos_kernels.cu) ---------------------------
# (oracle table, index) -> (reference program, literal order in its body):
# "hi" = sin then cos coefficients, highest power of r^2 first; "lo" = sin
# then cos, lowest power first (the evaluate_half_turn_d5_d4 call sites);
# q15 programs open with their 2^-15 scale.
SINCOS_MAP = {
    (0, 0): ("PolynomialD3D4HalfTurnBF16", "hi"), (0, 1): ("PolynomialD5D6HalfTurnBF16", "hi"),
    (0, 2): ("PolynomialD3D4HalfTurnFP16", "hi"), (0, 3): ("evaluate_half_turn_d5_d4_fp16", "hi"),
    (0, 4): ("PolynomialD5D6HalfTurnFP16", "hi"), (0, 5): ("PolynomialD7D6HalfTurnFP16", "hi"),
    (0, 6): ("evaluate_half_turn_q15_d5_d6_fp16", "hi"),
    (1, 0): ("PolynomialD3D4", "hi"), (1, 1): ("PolynomialD3D4MagicBias", "hi"), (1, 2): ("PolynomialD5D4", "hi"),
    (1, 3): ("PolynomialD7D6", "hi"), (1, 4): ("PolynomialD5D4HalfTurnLS", "lo"),
    (1, 5): ("PolynomialD5D4HalfTurnSollya", "lo"), (1, 6): ("PolynomialD5D4HalfTurnSollyaFast", "hi"),
    (2, 0): ("evaluate_quarter_turn_d3_d4_fp16", "hi"), (2, 1): ("PolynomialD3D4QuarterTurnBF16", "hi"),
    (2, 2): ("PolynomialD3D4BF16", "hi"), (3, 0): ("evaluate_quarter_turn_q15_d3_d4_fp16", "hi"),
}


def _literal(text: str) -> np.float32:
    t = text.rstrip("f")
    return np.float32(float.fromhex(t) if "0x" in t.lower() else float(t))


@pytest.mark.parametrize("key", sorted(SINCOS_MAP), ids=[SINCOS_MAP[k][0] for k in sorted(SINCOS_MAP)])
def test_sincos_tables_equal_reference_literals(oracle, key):
    with open(FIXTURE) as f:
        lits = json.load(f)["sincos_literals"]
    name, order = SINCOS_MAP[key]
    values = [_literal(t) for t in lits[name]]
    if "q15" in name:
        assert values[0] == np.float32(2.0 ** -15), (name, values[0])
        values = values[1:]
    s, c = oracle.sincos_coefficients(*key)
    want = [np.float32(v) for v in s] + [np.float32(v) for v in c]
    if order == "lo":
        want = want[:len(s)][::-1] + want[len(s):][::-1]
    assert values == want, (name, values, want)
