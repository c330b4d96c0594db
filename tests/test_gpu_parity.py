"""GPU parity: every HIP program against the CPU oracle, bit for bit.

The unary programs are lane-independent functions of one 16-bit value, so
they are checked on all 65536 input patterns.  Binary programs (derivative
times grad_out, SwiGLU products) are checked on seeded random operands that
include the exhaustive input sweep for the program argument.  All calls go
through the C ABI (include/spline_ops_hip.h) via ctypes.
"""

import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

FAMILIES = ("sigmoid", "tanh", "swish")
DTYPES = {"f16": torch.float16, "bf16": torch.bfloat16}


def _name(fam, direction, degree, fmt):
    suffix = "_bf16" if fmt == "bf16" else ""
    return f"launch_{fam}_{direction}_d{degree}_kernel{suffix}"


def _dev(bits: np.ndarray, fmt: str, device) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.uint16).view(np.int16)).to(device).view(DTYPES[fmt])


def _host(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def assert_bits_equal(got: np.ndarray, want: np.ndarray, fmt: str, what: str):
    """Bit equality, with any NaN matching any NaN."""
    expmask, mantmask = (0x7C00, 0x03FF) if fmt == "f16" else (0x7F80, 0x007F)
    g_nan = ((got & expmask) == expmask) & ((got & mantmask) != 0)
    w_nan = ((want & expmask) == expmask) & ((want & mantmask) != 0)
    bad = (got != want) & ~(g_nan & w_nan)
    if bad.any():
        idx = np.flatnonzero(bad)[:8]
        raise AssertionError(
            f"{what}: {bad.sum()} of {got.size} differ; first at {idx.tolist()}: "
            f"got {[hex(v) for v in got[idx]]} want {[hex(v) for v in want[idx]]}")


@pytest.mark.parametrize("fmt", ["f16", "bf16"])
@pytest.mark.parametrize("degree", [3, 4, 5, 6])
@pytest.mark.parametrize("fam", FAMILIES)
def test_forward_exhaustive(capi, oracle, cuda, fam, degree, fmt):
    x = oracle.all_bits()
    xd = _dev(x, fmt, cuda)
    yd = torch.empty_like(xd)
    capi.call(_name(fam, "fwd", degree, fmt), yd, xd, x.size)
    torch.cuda.synchronize()
    want = oracle.activation(fam, oracle.FWD, degree, fmt, x)
    assert_bits_equal(_host(yd), want, fmt, f"{fam} fwd d{degree} {fmt}")


@pytest.mark.parametrize("fmt", ["f16", "bf16"])
@pytest.mark.parametrize("degree", [3, 4, 5, 6])
@pytest.mark.parametrize("fam", FAMILIES)
def test_backward_program_times_grad(capi, oracle, cuda, fam, degree, fmt):
    rng = np.random.default_rng(1000 + degree)
    x = np.tile(oracle.all_bits(), 2)
    go = oracle.f32_to_bf16_bits(rng.standard_normal(x.size).astype(np.float32)) if fmt == "bf16" \
        else rng.standard_normal(x.size).astype(np.float16).view(np.uint16)
    go[:65536] = 0x3C00 if fmt == "f16" else 0x3F80  # grad_out = 1 exposes F'(x) itself
    xd, god = _dev(x, fmt, cuda), _dev(go, fmt, cuda)
    gi = torch.empty_like(xd)
    capi.call(_name(fam, "bwd", degree, fmt), gi, god, xd, x.size)
    torch.cuda.synchronize()
    want = oracle.activation_bwd(fam, degree, fmt, go, x)
    assert_bits_equal(_host(gi), want, fmt, f"{fam} bwd d{degree} {fmt}")


@pytest.mark.parametrize("fmt", ["f16", "bf16"])
@pytest.mark.parametrize("fam", ["sigmoid", "tanh"])
def test_algebraic_backward(capi, oracle, cuda, fam, fmt):
    rng = np.random.default_rng(7)
    y = oracle.all_bits()
    go = rng.integers(0, 65536, y.size, dtype=np.uint32).astype(np.uint16)
    yd, god = _dev(y, fmt, cuda), _dev(go, fmt, cuda)
    gi = torch.empty_like(yd)
    suffix = "_bf16" if fmt == "bf16" else ""
    capi.call(f"launch_{fam}_bwd_alg_kernel{suffix}", gi, god, yd, y.size)
    torch.cuda.synchronize()
    want = oracle.activation_bwd_alg(fam, fmt, go, y)
    assert_bits_equal(_host(gi), want, fmt, f"{fam} bwd_alg {fmt}")


def _operands(oracle, fmt, n, seed):
    rng = np.random.default_rng(seed)
    vals = rng.standard_normal((3, n)).astype(np.float32) * np.float32(3.0)
    if fmt == "bf16":
        ops = [oracle.f32_to_bf16_bits(v) for v in vals]
    else:
        ops = [v.astype(np.float16).view(np.uint16) for v in vals]
    ops[1][:65536] = oracle.all_bits()  # the gate sweeps every pattern
    return ops


@pytest.mark.parametrize("fmt", ["f16", "bf16"])
@pytest.mark.parametrize("degree", [3, 4, 5, 6])
def test_swish_mul_forward_and_backward(capi, oracle, cuda, degree, fmt):
    n = 65536 * 2 + 13  # ragged tail
    go, gate, up = _operands(oracle, fmt, n, 40 + degree)
    god, gd, ud = (_dev(a, fmt, cuda) for a in (go, gate, up))
    out = torch.empty_like(gd)
    suffix = "_bf16" if fmt == "bf16" else ""
    capi.call(f"launch_swish_mul_fwd_d{degree}_kernel{suffix}", out, gd, ud, n)
    gg, gu = torch.empty_like(gd), torch.empty_like(gd)
    capi.call(f"launch_swish_mul_bwd_d{degree}_kernel{suffix}", gg, gu, god, gd, ud, n)
    torch.cuda.synchronize()
    assert_bits_equal(_host(out), oracle.swish_mul_fwd(degree, fmt, gate, up), fmt,
                      f"swish_mul fwd d{degree} {fmt}")
    want_gg, want_gu = oracle.swish_mul_bwd(degree, fmt, go, gate, up)
    assert_bits_equal(_host(gg), want_gg, fmt, f"swish_mul bwd grad_gate d{degree} {fmt}")
    assert_bits_equal(_host(gu), want_gu, fmt, f"swish_mul bwd grad_up d{degree} {fmt}")


@pytest.mark.parametrize("fmt", ["f16", "bf16"])
@pytest.mark.parametrize("degree", [3, 4, 5, 6, 0])
@pytest.mark.parametrize("hidden", [2048, 520, 6, 10, 1030])
def test_packed_matches_separate(capi, cuda, degree, fmt, hidden):
    """Packed [rows, 2H] kernels equal the separate-tensor kernels bit for bit
    (reference test_spline_ops.py:190-204)."""
    rows = 37
    torch.manual_seed(degree + hidden)
    packed = (torch.randn(rows, 2 * hidden, device=cuda) * 3).to(DTYPES[fmt])
    go = torch.randn(rows, hidden, device=cuda).to(DTYPES[fmt])
    gate, up = (p.contiguous() for p in packed.chunk(2, dim=-1))
    suffix = "_bf16" if fmt == "bf16" else ""
    dname = "native" if degree == 0 else f"d{degree}"
    out_p = torch.empty(rows, hidden, device=cuda, dtype=DTYPES[fmt])
    capi.call(f"launch_swish_mul_packed_fwd_{dname}_kernel{suffix}", out_p, packed, rows, hidden)
    out_s = torch.empty_like(gate)
    capi.call(f"launch_swish_mul_fwd_{dname}_kernel{suffix}", out_s, gate, up, gate.numel())
    grad_p = torch.empty_like(packed)
    capi.call(f"launch_swish_mul_packed_bwd_{dname}_kernel{suffix}", grad_p, go, packed, rows, hidden)
    gg, gu = torch.empty_like(gate), torch.empty_like(gate)
    capi.call(f"launch_swish_mul_bwd_{dname}_kernel{suffix}", gg, gu, go, gate, up, gate.numel())
    torch.cuda.synchronize()
    assert torch.equal(out_p.view(torch.int16), out_s.view(torch.int16))
    if degree != 0:
        # The packed native backward rounds go*up first (a different program).
        assert torch.equal(grad_p.view(torch.int16), torch.cat((gg, gu), -1).view(torch.int16))


def test_b3_exhaustive(capi, oracle, cuda):
    x = oracle.all_bits()
    xd = _dev(x, "bf16", cuda)
    y, dy = torch.empty_like(xd), torch.empty_like(xd)
    capi.call("launch_flash_sigmoid_direct_d3_d4_bf16", y, dy, xd, x.size)
    y_only = torch.empty_like(xd)
    capi.call("launch_flash_sigmoid_direct_d3_bf16", y_only, xd, x.size)
    torch.cuda.synchronize()
    want_y, want_dy = oracle.b3_direct_bf16(x)
    assert_bits_equal(_host(y), want_y, "bf16", "B3 y")
    assert_bits_equal(_host(dy), want_dy, "bf16", "B3 dy")
    assert_bits_equal(_host(y_only), want_y, "bf16", "B3 forward-only y")


def test_b3_against_reference_emulation_fixture(capi, oracle, cuda):
    """HIP B3 == the reference's own evaluate_deployed table
    (scripts/audit_b3_deployed_fit.py:341-366, tests/golden/b3_audit_table.npz),
    with no oracle in between; C1's 2^20 seed-0 scores looked up in the same table."""
    t = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "b3_audit_table.npz"))
    fy, fdy = t["y"], t["dy"]
    nan_f = ((fdy & 0x7F80) == 0x7F80) & ((fdy & 0x7F) != 0)
    g = torch.Generator().manual_seed(0)
    c1 = (torch.rand(2 ** 20, generator=g) * 32 - 16).to(torch.bfloat16)
    for x in (oracle.all_bits(), c1.view(torch.int16).numpy().view(np.uint16)):
        xd = _dev(x, "bf16", cuda)
        y, dy = torch.empty_like(xd), torch.empty_like(xd)
        capi.call("launch_flash_sigmoid_direct_d3_d4_bf16", y, dy, xd, x.size)
        torch.cuda.synchronize()
        gy, gdy = _host(y), _host(dy)
        assert np.array_equal(gy, fy[x]), np.flatnonzero(gy != fy[x])[:8]
        nan = nan_f[x]
        assert np.array_equal(((gdy & 0x7F80) == 0x7F80) & ((gdy & 0x7F) != 0), nan)
        assert np.array_equal(gdy[~nan], fdy[x][~nan])


def test_b3_config1_uniform_scores(capi, oracle, cuda):
    """2^20 BF16 scores drawn U[-16, 16] from seed 0."""
    g = torch.Generator().manual_seed(0)
    s = (torch.rand(2 ** 20, generator=g) * 32 - 16).to(torch.bfloat16)
    bits = s.view(torch.int16).numpy().view(np.uint16)
    xd = s.to(cuda)
    y, dy = torch.empty_like(xd), torch.empty_like(xd)
    capi.call("launch_flash_sigmoid_direct_d3_d4_bf16", y, dy, xd, s.numel())
    torch.cuda.synchronize()
    want_y, want_dy = oracle.b3_direct_bf16(bits)
    assert_bits_equal(_host(y), want_y, "bf16", "B3 C1 y")
    assert_bits_equal(_host(dy), want_dy, "bf16", "B3 C1 dy")


def test_b3_fp32_scores(capi, oracle, cuda):
    rng = np.random.default_rng(3)
    s = (rng.standard_normal(4099) * 8).astype(np.float32)
    s[:6] = [np.inf, -np.inf, np.nan, 1.25, 1.2499999, 3.0e38]
    sd = torch.from_numpy(s).to(cuda)
    y = torch.empty(s.size, dtype=torch.bfloat16, device=cuda)
    dy = torch.empty_like(y)
    capi.call("launch_flash_sigmoid_direct_d3_d4_f32_bf16", y, dy, sd, s.size)
    torch.cuda.synchronize()
    want_y, want_dy = oracle.b3_direct_f32(s)
    assert_bits_equal(_host(y), want_y, "bf16", "B3 f32 y")
    assert_bits_equal(_host(dy), want_dy, "bf16", "B3 f32 dy")


@pytest.mark.parametrize("n", [1, 7, 8, 9, 4095, 4097])
@pytest.mark.parametrize("offset", [0, 1, 3])
def test_ragged_and_unaligned(capi, oracle, cuda, n, offset):
    """Tails and misaligned views give the same values as the vector path."""
    rng = np.random.default_rng(n + 31 * offset)
    x = rng.integers(0, 65536, n + offset, dtype=np.uint32).astype(np.uint16)
    xd = _dev(x, "bf16", cuda)[offset:]
    y = torch.empty(n + offset, dtype=torch.bfloat16, device=cuda)[offset:]
    capi.call("launch_swish_fwd_d3_kernel_bf16", y, xd, n)
    torch.cuda.synchronize()
    want = oracle.activation("swish", oracle.FWD, 3, "bf16", x[offset:])
    assert_bits_equal(_host(y), want, "bf16", f"swish bf16 n={n} offset={offset}")


def test_zero_size_and_bad_args(capi, cuda):
    x = torch.empty(0, dtype=torch.float16, device=cuda)
    assert capi.call("launch_swish_fwd_d3_kernel", x, x, 0) == 0
    import ctypes
    rc = capi.launch_swish_fwd_d3_kernel(ctypes.c_void_p(0), ctypes.c_void_p(0), ctypes.c_int64(-1),
                                         capi.stream())
    assert rc != 0
    # softcap: cap must be positive and finite; nothing is launched otherwise
    s = torch.zeros(64, dtype=torch.bfloat16, device=cuda)
    for cap in (0.0, -30.0, float("inf"), float("nan")):
        for name in ("launch_softcap_tanh_d4_bf16", "launch_softcap_tanh_native_bf16"):
            rc = getattr(capi, name)(capi.ptr(s), capi.ptr(s), ctypes.c_int64(64), ctypes.c_float(cap),
                                     capi.stream())
            assert rc != 0, (name, cap)
        for name in ("launch_softcap_tanh_d4_bwd_bf16", "launch_softcap_tanh_native_bwd_bf16"):
            rc = getattr(capi, name)(capi.ptr(s), capi.ptr(s), capi.ptr(s), ctypes.c_int64(64),
                                     ctypes.c_float(cap), capi.stream())
            assert rc != 0, (name, cap)
    # the attention softcap modes check cap before an empty batch returns
    strides = (ctypes.c_int64 * 12)(*([128 * 128, 128 * 128, 128] * 4))
    null = ctypes.c_void_p(0)
    for mode in (3, 4):
        for cap, ok in ((30.0, True), (float("inf"), False), (0.0, False)):
            rc = capi.launch_flash_attention_fwd_strided_bf16(
                null, null, null, null, null, ctypes.c_int64(0), ctypes.c_int64(1), ctypes.c_int64(1),
                ctypes.c_int64(128), ctypes.c_int64(128), strides, ctypes.c_int(mode), ctypes.c_int(4),
                ctypes.c_int(0), ctypes.c_float(1.0), ctypes.c_float(cap), ctypes.c_float(0.0), capi.stream())
            assert (rc == 0) == ok, (mode, cap, rc)


@pytest.mark.parametrize("reps", [1024, 2047, 2048, 2056])
@pytest.mark.parametrize("fmt", ["f16", "bf16"])
def test_large_streaming_paths(capi, oracle, cuda, reps, fmt):
    """Outputs >= 64 MiB take the non-temporal store path, inputs >= 256 MiB
    (2048 tiles) also non-temporal loads.  Tiling all 65536 patterns makes the expected
    output the tiled oracle table (a size-independent check)."""
    x = torch.from_numpy(oracle.all_bits().view(np.int16)).to(cuda).repeat(reps)
    x = x.view(DTYPES[fmt])
    want = torch.from_numpy(oracle.activation("swish", oracle.FWD, 3, fmt,
                                              oracle.all_bits()).view(np.int16)).to(cuda)
    y = torch.empty_like(x)
    capi.call(_name("swish", "fwd", 3, fmt), y, x, x.numel())
    torch.cuda.synchronize()
    got = y.view(torch.int16).view(reps, 65536)
    nan_ok = torch.isnan(y.view(reps, 65536).float()) & torch.isnan(want.view(DTYPES[fmt]).float())[None]
    assert bool(((got == want[None]) | nan_ok).all())


@pytest.mark.parametrize("n", [1, 7, 8, 4099, 1 << 20])
def test_copy_helper(capi, cuda, n):
    """spline_hip_copy16 (the bench's copy ceiling) moves every element."""
    x = torch.arange(n, device=cuda, dtype=torch.int32).to(torch.int16)
    y = torch.full_like(x, -1)
    capi.call("spline_hip_copy16", y, x, n)
    torch.cuda.synchronize()
    assert torch.equal(x, y)
    xu = torch.arange(n + 1, device=cuda, dtype=torch.int32).to(torch.int16)[1:]
    yu = torch.full((n + 1,), -1, device=cuda, dtype=torch.int16)[1:]
    capi.call("spline_hip_copy16", yu, xu, n)
    torch.cuda.synchronize()
    assert torch.equal(xu, yu)
