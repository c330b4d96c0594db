#!/usr/bin/env python3
"""Write the B3-D2 (sigmoid via exp2, degree 2) coefficient fixture.

The reference stores no coefficients for this program: they exist only as
the output of its fitter,
autonumerics_zero/evolution/fit_flash_sigmoid_exp2_d2.py (differential
evolution, seed 1234, maxiter 300, then Nelder-Mead; FP32-rounded).  This
script imports that fitter from a local checkout of the reference, runs it
with its defaults and writes the coefficients, their FP32 bit patterns and
the fitter's own metrics to b3_d2_coefficients.json beside this file.  It
runs in the build container only; the JSON is the committed fixture.

    python tests/golden/make_b3_d2_fixture.py /root/reference
"""

import json
import os
import struct
import sys


def main(reference_root: str) -> None:
    sys.path.insert(0, os.path.join(reference_root, "autonumerics_zero", "evolution"))
    import fit_flash_sigmoid_exp2_d2 as fitter  # reference code, this container only

    args = fitter.parse_args([])
    coefficients, metrics = fitter.fit(args)
    doc = {
        "source": "autonumerics_zero/evolution/fit_flash_sigmoid_exp2_d2.py (run with defaults)",
        "sequence_length": args.sequence_length,
        "score_sigma": args.score_sigma,
        "seed": args.seed,
        "maxiter": args.maxiter,
        "coefficients_float32": [float(c) for c in coefficients],
        "coefficients_hex": ["0x%08X" % struct.unpack("<I", struct.pack("<f", c))[0]
                             for c in coefficients],
        "metrics": {k: float(v) for k, v in vars(metrics).items()},
    }
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "b3_d2_coefficients.json")
    with open(out, "w") as f:
        json.dump(doc, f, indent=2)
        f.write("\n")
    print(json.dumps(doc, indent=2))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
