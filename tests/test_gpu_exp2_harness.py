"""GPU parity of the isolated exp2 programs of the reference's harness
(autonumerics_zero/cuda_benchmarks/benchmark_exp2_pwl2.cu), through the C ABI:

* the fractional FP16 programs (f in [0, 1] -> 2^f): the historical
  two-segment fit and the PWL2 hinge bit for bit against the oracle (whose
  programs reproduce the published fractional error metrics), v_exp_f16
  within one FP16 ULP of exp2;
* the compute probes: 65,536 threads x 8 chains of program + feedback FMA,
  bit for bit against a CPU emulation of the chains through the oracle for
  the polynomial programs (the emulation's FP16 / FP32 feedback rounds once
  from an exact double); the hardware variants stay finite and in domain
  (their chains amplify one-ULP differences, so they have no exact
  reference)."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

THREADS, CHAINS = 1 << 16, 8


def fractional_pairs(n):
    """The harness's make_fractional_h2(n): pairs ((2i mod 65521) / 65521,
    (2i + 1 mod 65521) / 65521) in FP32, rounded to FP16."""
    i = np.arange(n, dtype=np.int64)
    x = (((2 * i) % 65521).astype(np.float32) / np.float32(65521.0)).astype(np.float16)
    y = (((2 * i + 1) % 65521).astype(np.float32) / np.float32(65521.0)).astype(np.float16)
    return np.stack([x, y], axis=1).reshape(-1)


def full_pairs(n):
    """The harness's make_full_f32(n): pairs (-16 u, -16 v), u = (2i mod
    1048573) / 1048573, v = (2i + 1 mod 1048573) / 1048573."""
    i = np.arange(n, dtype=np.int64)
    u = ((2 * i) % 1048573).astype(np.float32) / np.float32(1048573.0)
    v = ((2 * i + 1) % 1048573).astype(np.float32) / np.float32(1048573.0)
    return np.stack([np.float32(-16.0) * u, np.float32(-16.0) * v], axis=1).reshape(-1)


def _f16_device(a, cuda):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(cuda)


EDGES = np.array([0.0, -0.0, 2.0 ** -24, 0.49951171875, 0.5, 0.50048828125, 0.9990234375, 0.99951171875, 1.0,
                  -0.25, 1.5, 65504.0, -np.inf, np.inf], dtype=np.float16)


@pytest.mark.parametrize("name,kind", [("pwl2_historical", 12), ("pwl2_hinge", 11), ("native", None)])
def test_fraction_programs(capi, oracle, cuda, name, kind):
    # the harness's 2^21 values plus edges, an odd count so the tail path runs too
    f = np.concatenate([fractional_pairs(1 << 20), EDGES[: 13 if kind == 11 else None]])
    if kind == 11:  # the hinge has no clamp: keep it on its domain [0, 1]
        f = f[(f >= 0) & (f <= 1)]
    f = np.concatenate([f, f[:3]])
    assert f.size % 8 != 0
    x = _f16_device(f, cuda)
    y = torch.empty_like(x)
    print(f"exp2 fraction {name} {f.size}", flush=True)
    capi.call(f"launch_exp2_fraction_{name}_f16", y, x, f.size)
    torch.cuda.synchronize()
    got = y.cpu().numpy().view(np.float16)
    if kind is not None:
        want = oracle.exp2_fraction(kind, f.astype(np.float32)).astype(np.float16)
        bad = np.flatnonzero(got.view(np.uint16) != want.view(np.uint16))
        assert bad.size == 0, (bad[:8], f[bad[:8]], got[bad[:8]], want[bad[:8]])
    else:
        dom = (f >= 0) & (f <= 1)
        ref = np.exp2(f[dom].astype(np.float64))
        ulp = np.abs(got[dom].astype(np.float64) - ref) / 2.0 ** -10  # FP16 ULP on [1, 2]
        assert ulp.max() <= 1.0, ulp.max()


def _emulate_f16(oracle, kind, x, iterations):
    """x: [CHAINS, THREADS, 2] FP16 -> the chains after `iterations` rounds."""
    x = x.copy()
    for _ in range(iterations):
        v = oracle.exp2_fraction(kind, x.astype(np.float32).reshape(-1)).reshape(x.shape).astype(np.float64)
        x[:4] = (v[:4] * 0.5 - 0.5).astype(np.float16)
        x[4:] = (v[4:] * -0.5 + 1.5).astype(np.float16)
    return x


def _emulate_f32(oracle, kind, x, iterations):
    x = x.copy()
    for _ in range(iterations):
        v = oracle.exp2(kind, x.reshape(-1), False).reshape(x.shape).astype(np.float64)
        x[:4] = (v[:4] * 8.0 - 16.0).astype(np.float32)
        x[4:] = (v[4:] * -8.0).astype(np.float32)
    return x


def _stored(x):
    """out[t] = chain t % 8 of thread t."""
    t = np.arange(THREADS)
    return x[t % CHAINS, t]


@pytest.mark.parametrize("variant,kind", [(0, None), (1, 12), (2, 11)])
def test_compute_probe_f16x2(capi, oracle, cuda, variant, kind):
    iterations = 24
    inp = fractional_pairs(THREADS * CHAINS)
    x = _f16_device(inp, cuda)
    out = torch.empty(THREADS * 2, dtype=torch.int16, device=cuda)
    print(f"exp2 compute f16x2 variant {variant}", flush=True)
    capi.call("launch_exp2_compute_f16x2", ctypes_int(variant), out, x, THREADS, ctypes_int(iterations))
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.float16).reshape(THREADS, 2)
    if kind is None:
        assert np.isfinite(got).all() and (got >= 0).all() and (got <= 1).all()
        return
    want = _stored(_emulate_f16(oracle, kind, inp.reshape(CHAINS, THREADS, 2), iterations))
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("variant,kind", [(0, None), (1, 1), (2, 2)])
def test_compute_probe_f32x2(capi, oracle, cuda, variant, kind):
    iterations = 24
    inp = full_pairs(THREADS * CHAINS)
    x = torch.from_numpy(inp).to(cuda)
    out = torch.empty(THREADS * 2, dtype=torch.float32, device=cuda)
    print(f"exp2 compute f32x2 variant {variant}", flush=True)
    capi.call("launch_exp2_compute_f32x2", ctypes_int(variant), out, x, THREADS, ctypes_int(iterations))
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(THREADS, 2)
    if kind is None:
        assert np.isfinite(got).all() and (got >= -16).all() and (got <= 0).all()
        return
    want = _stored(_emulate_f32(oracle, kind, inp.reshape(CHAINS, THREADS, 2), iterations))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def ctypes_int(v):
    import ctypes

    return ctypes.c_int(v)


def test_probe_arguments_rejected(capi, cuda):
    """An unknown variant, a negative iteration count or a thread count that
    is not a positive multiple of 256 (at most 2^24) is refused before any
    launch."""
    buf = torch.empty(THREADS * CHAINS * 2, dtype=torch.float32, device=cuda)
    for name in ("launch_exp2_compute_f16x2", "launch_exp2_compute_f32x2"):
        for variant, threads, iterations in ((3, THREADS, 1), (-1, THREADS, 1), (0, THREADS, -1), (0, 0, 1),
                                             (0, 300, 1), (0, (1 << 24) + 256, 1)):
            with pytest.raises(RuntimeError):
                capi.call(name, ctypes_int(variant), buf, buf, threads, ctypes_int(iterations))
    torch.cuda.synchronize()
