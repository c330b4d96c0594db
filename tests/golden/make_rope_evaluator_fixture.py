#!/usr/bin/env python3
"""Write the RoPE evaluator fixture: the reference's float32 polynomial sin/cos.

``sfu_repro.rope.polynomial_sincos`` of the reference
(src/sfu_repro/rope/polynomial_sincos.py:85-165: reduce_to_quarter_turn,
evaluate_reduced_sincos, polynomial_sincos) is imported from a local checkout
(it needs only CPU torch) and evaluated on CPU on a fixed angle set: a
linspace over +-131072 rad, 65,536 uniform angles in +-8192 (numpy seed 12),
the multiples of pi/4 from -5 pi to 5 pi and the specials 0, -0, 1e-40,
3e7, -1e12, +-inf, NaN.  Cases: FP32 and FP64 angles x the three coefficient
sets (SOLLYA_D3_D4, UNIFORM_D5_D4, UNIFORM_D7_D6) x both reductions
(accurate FP64, fast FP32 Cody-Waite).

Output ``rope_evaluator.json`` beside this file: per case the SHA-256 of the
float32 cos and sin bytes (NaN canonicalised to 0x7FC00000) over the whole
set, and the bit patterns of every 512th angle's outputs for diagnostics.
Runs in the build container only:

    python tests/golden/make_rope_evaluator_fixture.py /root/reference
"""

import hashlib
import importlib.util
import json
import math
import os
import sys

import numpy as np

SAMPLE_STEP = 512


def angle_set() -> np.ndarray:
    rng = np.random.default_rng(12)
    return np.concatenate([
        np.linspace(-131_072.0, 131_072.0, 65_537),
        rng.uniform(-8192, 8192, 65_536),
        np.arange(-20, 21) * (math.pi / 4),
        [0.0, -0.0, 1e-40, 3e7, -1e12, np.inf, -np.inf, np.nan],
    ])


def canonical_bits(t) -> np.ndarray:
    a = np.ascontiguousarray(t.numpy(), dtype=np.float32).view(np.uint32).copy()
    a[np.isnan(t.numpy())] = 0x7FC00000
    return a


def cases(module):
    for dtype in ("float32", "float64"):
        for name in ("SOLLYA_D3_D4", "UNIFORM_D5_D4", "UNIFORM_D7_D6"):
            for accurate in (True, False):
                yield dtype, name, getattr(module, name), accurate


def main(reference_root: str) -> None:
    import torch

    path = os.path.join(reference_root, "src", "sfu_repro", "rope", "polynomial_sincos.py")
    spec = importlib.util.spec_from_file_location("reference_polynomial_sincos", path)
    ref = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = ref  # dataclasses resolve annotations through sys.modules
    spec.loader.exec_module(ref)  # reference code, this container only

    angles = angle_set()
    doc = {"source": "src/sfu_repro/rope/polynomial_sincos.py:85-165 polynomial_sincos on CPU torch "
                     f"{torch.__version__}",
           "angles": "make_rope_evaluator_fixture.angle_set()", "count": int(angles.size),
           "sample_step": SAMPLE_STEP, "nan_encoding": "0x7FC00000", "cases": []}
    with np.errstate(over="ignore", invalid="ignore"):
        for dtype, name, poly, accurate in cases(ref):
            a = torch.from_numpy(angles.astype(dtype))
            cos, sin = ref.polynomial_sincos(a, polynomial=poly, accurate_reduction=accurate)
            cb, sb = canonical_bits(cos), canonical_bits(sin)
            doc["cases"].append({
                "dtype": dtype, "polynomial": name, "accurate": accurate,
                "cos_sha256": hashlib.sha256(cb.tobytes()).hexdigest(),
                "sin_sha256": hashlib.sha256(sb.tobytes()).hexdigest(),
                "cos_sample": [int(v) for v in cb[::SAMPLE_STEP]],
                "sin_sample": [int(v) for v in sb[::SAMPLE_STEP]],
            })
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rope_evaluator.json")
    with open(out, "w") as f:
        json.dump(doc, f)
        f.write("\n")
    print(f"{len(doc['cases'])} cases over {angles.size} angles -> {out}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
