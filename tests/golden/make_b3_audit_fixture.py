#!/usr/bin/env python3
"""Write the B3 fixture: the reference's own CPU emulation over every BF16 input.

The reference's bit-exactness target for B3 is its audit emulation of the
deployed packed-BF16 program, ``evaluate_deployed`` in
scripts/audit_b3_deployed_fit.py:341-366 (with ``round_bf16`` / ``bf16_fma`` /
``bf16_multiply`` at :319-338).  This script imports that module from a local
checkout of the reference (stdlib only; nothing else of the reference is
loaded), builds the ``DirectB3Spec`` from the constants the reference's test
pins (tests/test_audit_b3_deployed_fit.py:30-37: sequence length 4096, the two
D3 rows and the two factored-D4 rows) plus the split 1.25 and clamp 6.0 of the
hand-written PTX (extras/paper/manuscript/main.tex:1094-1111: immediates
0x3fa0, 0x40c0), and evaluates all 65,536 BF16 bit patterns.

Output, beside this file:

* ``b3_audit_table.npz``: ``y``, ``dy`` (BF16 bits: the upper half of the
  float32 the audit returns), ``row`` (the audit's row index), each indexed by
  the input bit pattern;
* ``b3_audit_table.json``: provenance and a SHA-256 of each table.

Where the audit's dy is a NaN (NaN scores: ``max(round_bf16(0.0), nan)`` makes
y = 0 and dy = 0 * NaN), the table holds the canonical quiet NaN 0x7FC0 and the
checks compare NaN-ness only.  Runs in the build container only:

    python tests/golden/make_b3_audit_fixture.py /root/reference
"""

import hashlib
import importlib.util
import json
import math
import os
import struct
import sys

import numpy as np

SPEC_ROWS = {
    "sequence_length": 4096,
    "clamp": 6.0,
    "split": 1.25,
    "forward_rows": ((1.0, 1.0546875, 0.53515625, 0.11328125),
                     (-8.5625, 17.5, -9.0625, 2.140625)),
    "gradient_factors": ((1.0, -0.0087890625), (1.0078125, -0.0028076171875)),
}


def _upper_bf16(value: float) -> int:
    bits = struct.unpack("<I", struct.pack("<f", value))[0]
    if math.isnan(value):
        return 0x7FC0
    assert bits & 0xFFFF == 0, "audit output is not a BF16 value"
    return bits >> 16


def main(reference_root: str) -> None:
    path = os.path.join(reference_root, "scripts", "audit_b3_deployed_fit.py")
    spec_mod = importlib.util.spec_from_file_location("audit_b3_deployed_fit", path)
    audit = importlib.util.module_from_spec(spec_mod)
    sys.modules[spec_mod.name] = audit  # dataclasses resolve annotations through sys.modules
    spec_mod.loader.exec_module(audit)  # reference code, this container only

    spec = audit.DirectB3Spec(
        sequence_length=SPEC_ROWS["sequence_length"],
        clamp=SPEC_ROWS["clamp"],
        split=SPEC_ROWS["split"],
        midpoints=(0.0, 0.0),  # not read by evaluate_deployed
        forward_rows=SPEC_ROWS["forward_rows"],
        gradient_factors=SPEC_ROWS["gradient_factors"],
    )
    y = np.zeros(1 << 16, dtype=np.uint16)
    dy = np.zeros(1 << 16, dtype=np.uint16)
    row = np.zeros(1 << 16, dtype=np.uint8)
    for b in range(1 << 16):
        score = struct.unpack("<f", struct.pack("<I", b << 16))[0]
        v = audit.evaluate_deployed(score, spec)
        y[b] = _upper_bf16(v.forward)
        dy[b] = _upper_bf16(v.derivative)
        row[b] = v.row_index

    here = os.path.dirname(os.path.abspath(__file__))
    np.savez_compressed(os.path.join(here, "b3_audit_table.npz"), y=y, dy=dy, row=row)
    doc = {
        "source": "scripts/audit_b3_deployed_fit.py:341-366 evaluate_deployed, all 65,536 BF16 inputs",
        "spec": {k: v for k, v in SPEC_ROWS.items()},
        "deployed_forward_rows": [list(r) for r in spec.deployed_forward_rows],
        "deployed_gradient_factors": [list(r) for r in spec.deployed_gradient_factors],
        "nan_dy_encoding": "0x7FC0 where the audit's dy is NaN",
        "sha256": {
            "y": hashlib.sha256(y.tobytes()).hexdigest(),
            "dy": hashlib.sha256(dy.tobytes()).hexdigest(),
            "row": hashlib.sha256(row.tobytes()).hexdigest(),
        },
    }
    with open(os.path.join(here, "b3_audit_table.json"), "w") as f:
        json.dump(doc, f, indent=2)
        f.write("\n")
    print(json.dumps(doc["sha256"], indent=2))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
