"""The oracle's program tables equal the reference's coefficient headers
literal for literal: for every activation struct of
spline_structs_odd.cuh (FP16), spline_structs_odd_bf16.cuh (BF16) and
spline_structs_sollya_bf16.cuh (BF16 Sollya set), the clamp Lc and each
coefficient c0..cN, as float32 values of the decimal literals that the
headers convert with __float2half2_rn / __float2bfloat162_rn, and the
composed structs (SiLU = x * sigmoid) call the sigmoid program of the same
degree.  The literals come from tests/golden/struct_coefficients.json
(written by make_struct_coefficients_fixture.py beside it).

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
