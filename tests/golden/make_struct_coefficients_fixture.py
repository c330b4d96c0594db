"""Write tests/golden/struct_coefficients.json: the clamp Lc and the
coefficient literals c0..c6 of every activation struct in the reference's
three coefficient headers (autonumerics_zero/spline_ops/
spline_structs_odd.cuh, spline_structs_odd_bf16.cuh,
spline_structs_sollya_bf16.cuh), exactly as the source writes them (decimal
strings), plus, for the composed structs that hold no coefficients, the
struct they call; and, for the paired sin/cos programs of sincos_kernels.cu,
the float literals of each program's body in source order.  The fixture is
data: numbers and names, no source text.

Run in the build container (where /root/reference exists):

    python tests/golden/make_struct_coefficients_fixture.py
"""

import json
import os
import re
import sys

REF = "/root/reference/autonumerics_zero/spline_ops"
FILES = ["spline_structs_odd.cuh", "spline_structs_odd_bf16.cuh", "spline_structs_sollya_bf16.cuh"]
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "struct_coefficients.json")

STRUCT = re.compile(r"^struct (\w+) \{(.*?)^\};", re.S | re.M)
CONV = r"__float2(?:half2|bfloat162)_rn\(\s*([-+0-9.eE]+)f?\s*\)"
CLAMP = re.compile(r"__hmin2\(\s*\w+\s*,\s*" + CONV + r"\s*\)")
COEFF = re.compile(r"\b(c\d)\s*=\s*" + CONV)
CALLS = re.compile(r"\b([A-Z][A-Z0-9_]+)::evaluate\b")


def extract(text: str) -> dict:
    out = {}
    for name, body in STRUCT.findall(text):
        entry = {}
        m = CLAMP.search(body)
        if m:
            entry["lc"] = m.group(1)
        coeffs = dict(COEFF.findall(body))
        if coeffs:
            entry["c"] = coeffs
        calls = sorted(set(CALLS.findall(body)) - {name})
        if calls:
            entry["calls"] = calls
        out[name] = entry
    return out


# sin/cos programs (structs and helper functions) whose bodies hold their
# coefficients
SINCOS_FILE = "sincos_kernels.cu"
SINCOS_PROGRAMS = [
    "PolynomialD3D4HalfTurnBF16", "PolynomialD5D6HalfTurnBF16", "PolynomialD3D4HalfTurnFP16",
    "evaluate_half_turn_d5_d4_fp16", "PolynomialD5D6HalfTurnFP16", "PolynomialD7D6HalfTurnFP16",
    "evaluate_half_turn_q15_d5_d6_fp16", "PolynomialD3D4", "PolynomialD3D4MagicBias", "PolynomialD5D4",
    "PolynomialD7D6", "PolynomialD5D4HalfTurnLS", "PolynomialD5D4HalfTurnSollya",
    "PolynomialD5D4HalfTurnSollyaFast", "evaluate_quarter_turn_d3_d4_fp16", "PolynomialD3D4QuarterTurnBF16",
    "PolynomialD3D4BF16", "evaluate_quarter_turn_q15_d3_d4_fp16",
]
FLOAT_LIT = re.compile(r"(?<![\w.])-?\d+\.\d*(?:[eE][-+]?\d+)?f\b|(?<![\w.])-?0x[0-9a-fA-F.]+p[-+]?\d+f?")


def sincos_literals(text: str) -> dict:
    out = {}
    for name in SINCOS_PROGRAMS:
        m = re.search(r"(?:struct|void)\s+" + name + r"\b[^{;]*\{", text)
        if not m:
            raise SystemExit(f"{name} not found in {SINCOS_FILE}")
        i = j = m.end()
        depth = 1
        while depth:
            depth += {"{": 1, "}": -1}.get(text[j], 0)
            j += 1
        out[name] = FLOAT_LIT.findall(text[i:j])
    return out


def main() -> int:
    fixture = {"source": "autonumerics_zero/spline_ops/" + "{" + ",".join(FILES + [SINCOS_FILE]) + "}",
               "structs": {}}
    for fn in FILES:
        with open(os.path.join(REF, fn)) as f:
            fixture["structs"][fn] = extract(f.read())
    with open(os.path.join(REF, SINCOS_FILE)) as f:
        fixture["sincos_literals"] = sincos_literals(f.read())
    with open(OUT, "w") as f:
        json.dump(fixture, f, indent=1, sort_keys=True)
        f.write("\n")
    n = sum(len(v) for v in fixture["structs"].values())
    print(f"wrote {OUT}: {n} structs")
    return 0


if __name__ == "__main__":
    sys.exit(main())
