"""GPU parity of the attention-side programs (B2 softcap, B5 exp2) against
the CPU oracle, through the C ABI, plus error bounds of the native baselines
against FP32 torch."""

import ctypes

import numpy as np
import pytest
import torch

from test_gpu_parity import _dev, _host, assert_bits_equal

pytestmark = pytest.mark.gpu


def _f32_inputs(seed, n=1 << 18):
    rng = np.random.default_rng(seed)
    x = np.concatenate([
        -rng.random(n, dtype=np.float32) * 140.0,             # softmax exponents
        np.linspace(-3.0, 1.0, 4099, dtype=np.float32),
        np.array([0.0, -0.0, -1e-30, -1e-40, -126.5, -127.0, -127.25, -128.0,
                  -np.inf, np.nan, -np.nan, 0.999999, 1.5, 60.25], dtype=np.float32),
    ])
    return x.astype(np.float32)


# caps below 1 and far above the scores cover the saturated and the
# near-linear ends; the magnitude form must match the signed program for all.
@pytest.mark.parametrize("cap", [30.0, 50.0, 1.0, 0.3, 7.5, 1000.0])
def test_softcap_forward_exhaustive(capi, oracle, cuda, cap):
    s = oracle.all_bits()
    sd = _dev(s, "bf16", cuda)
    y = torch.empty_like(sd)
    rc = capi.launch_softcap_tanh_d4_bf16(capi.ptr(y), capi.ptr(sd), ctypes.c_int64(s.size),
                                          ctypes.c_float(cap), capi.stream())
    assert rc == 0
    torch.cuda.synchronize()
    assert_bits_equal(_host(y), oracle.softcap_fwd_bf16(s, cap), "bf16", f"softcap cap={cap}")


@pytest.mark.parametrize("cap", [30.0, 0.3, 1000.0])
def test_softcap_backward(capi, oracle, cuda, cap):
    rng = np.random.default_rng(5)
    s = np.tile(oracle.all_bits(), 2)
    go = oracle.f32_to_bf16_bits(rng.standard_normal(s.size).astype(np.float32))
    go[:65536] = 0x3F80
    sd, god = _dev(s, "bf16", cuda), _dev(go, "bf16", cuda)
    g = torch.empty_like(sd)
    rc = capi.launch_softcap_tanh_d4_bwd_bf16(capi.ptr(g), capi.ptr(god), capi.ptr(sd),
                                              ctypes.c_int64(s.size), ctypes.c_float(cap),
                                              capi.stream())
    assert rc == 0
    torch.cuda.synchronize()
    assert_bits_equal(_host(g), oracle.softcap_bwd_bf16(go, s, cap), "bf16", f"softcap bwd cap={cap}")


def test_softcap_config3_distribution(spline_ops, cuda):
    """BASELINE config 3 recipe (reduced size): N(0, 15^2) scores with 1 %
    outliers at +-200; error against FP32 30*tanh(s/30)."""
    g = torch.Generator().manual_seed(0)
    s = torch.randn(1 << 20, generator=g) * 15
    mask = torch.rand(s.shape, generator=g) < 0.01
    sign = torch.where(torch.rand(s.shape, generator=g) < 0.5, -1.0, 1.0)
    s = torch.where(mask, 200.0 * sign, s).to(torch.bfloat16)
    y = spline_ops.softcap_tanh_fwd_bf16(s.to(cuda), 30.0).float().cpu()
    ref = 30.0 * torch.tanh(s.float() / 30.0)
    # D4 tanh error 0.0133 (x cap) plus BF16 rounding of the output
    assert float((y - ref).abs().max()) < 0.6


@pytest.mark.parametrize("kind,name", [(0, "d2"), (1, "d3"), (3, "pwl2_safe"), (4, "pwl2_safe_f16"), (5, "pwl1_safe"),
                                       (6, "pwl1_safe_f16"), (7, "pwl2_safe_bf16"), (8, "d2_safe_noclamp"),
                                       (9, "d2_safe_f16"), (10, "d2_safe_bf16"), (11, "pwl2_f16")])
@pytest.mark.parametrize("out_bf16", [True, False])
def test_exp2_programs(capi, oracle, cuda, kind, name, out_bf16):
    x = _f32_inputs(11 + kind)
    xd = torch.from_numpy(x).to(cuda)
    if out_bf16:
        y = torch.empty(x.size, dtype=torch.bfloat16, device=cuda)
        capi.call(f"launch_exp2_{name}_f32_bf16", y, xd, x.size)
        torch.cuda.synchronize()
        assert_bits_equal(_host(y), oracle.exp2(kind, x, True), "bf16", f"exp2 {name} bf16")
    else:
        y = torch.empty(x.size, dtype=torch.float32, device=cuda)
        capi.call(f"launch_exp2_{name}_f32", y, xd, x.size)
        torch.cuda.synchronize()
        want = oracle.exp2(kind, x, False)
        assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("out_bf16", [True, False])
def test_exp2_pwl2_program(capi, oracle, cuda, out_bf16):
    """The reference's two-piece FP32 hinge (FA4 backend pwl2), clamped at
    -126: bit for bit the oracle's program (the reference's, clamped at -127)
    on fmax(x, -126), NaN taking the clamp as in v_max_f32.  Below -126.987
    the reference's clamp would give NaN bits; here every output is finite."""
    x = _f32_inputs(13)
    xd = torch.from_numpy(x).to(cuda)
    xc = np.fmax(x, np.float32(-126.0))
    if out_bf16:
        y = torch.empty(x.size, dtype=torch.bfloat16, device=cuda)
        capi.call("launch_exp2_pwl2_f32_bf16", y, xd, x.size)
        torch.cuda.synchronize()
        assert_bits_equal(_host(y), oracle.exp2(2, xc, True), "bf16", "exp2 pwl2 bf16")
    else:
        y = torch.empty(x.size, dtype=torch.float32, device=cuda)
        capi.call("launch_exp2_pwl2_f32", y, xd, x.size)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), oracle.exp2(2, xc, False).view(np.uint32))
        assert np.isfinite(got[x < 100]).all()


def test_exp2_config5_and_native(spline_ops, cuda):
    """BASELINE config 5 recipe (one head block): logits N(0, 4^2) minus the
    row max; D2 relative error vs FP32 torch.exp2 and the native baseline."""
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(64, 4096, 128, generator=g) * 4
    x = (logits - logits.amax(-1, keepdim=True)).to(cuda)
    ref = torch.exp2(x)
    d2 = spline_ops.exp2_d2_f32_to_bf16(x).float()
    nat = spline_ops.exp2_native_f32_to_bf16(x).float()
    d2_32 = spline_ops.exp2_d2_f32(x)
    big = ref > 1e-30
    rel = ((d2_32 - ref).abs() / ref)[big]
    assert float(rel.max()) < 2.8e-3          # sampled-minimax D2 bound 2.679e-3
    assert float(((d2 - ref).abs() / ref)[big].max()) < 2.8e-3 + 2 ** -8
    assert float(((nat - ref).abs() / ref)[big].max()) < 2 ** -8 + 1e-5


def test_b3_exp2_d2_exhaustive(capi, oracle, cuda):
    import json
    import os

    with open(os.path.join(os.path.dirname(__file__), "golden", "b3_d2_coefficients.json")) as f:
        coeffs = json.load(f)["coefficients_float32"]
    s = oracle.all_bits()
    sd = _dev(s, "bf16", cuda)
    y, dy = torch.empty_like(sd), torch.empty_like(sd)
    capi.call("launch_flash_sigmoid_exp2_d2_bf16", y, dy, sd, s.size)
    torch.cuda.synchronize()
    want_y, want_dy = oracle.b3_exp2_d2_bf16(s, coeffs)
    assert_bits_equal(_host(y), want_y, "bf16", "B3-D2 y")
    assert_bits_equal(_host(dy), want_dy, "bf16", "B3-D2 dy")


def _ulps_bf16(got: np.ndarray, want: np.ndarray) -> np.ndarray:
    """ULP distance of BF16 bit patterns (sign-magnitude -> ordered integers)."""
    def key(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(key(got) - key(want))


def test_b3_native_control(capi, oracle, cuda):
    """The B3 hardware control (v_exp_f32 / v_rcp_f32 in FP32, one RNE per
    output) on every BF16 score: within one BF16 ULP of sigmoid(s - ln 4096)
    and of p (1 - p), both correctly rounded from float64."""
    s = oracle.all_bits()
    x = oracle.bf16_bits_to_f32(s).astype(np.float64)
    fin = np.isfinite(x)
    sd = _dev(s, "bf16", cuda)
    y, dy = torch.empty_like(sd), torch.empty_like(sd)
    capi.call("launch_flash_sigmoid_native_bf16", y, dy, sd, s.size)
    torch.cuda.synchronize()
    with np.errstate(over="ignore"):
        p = 1.0 / (1.0 + np.exp(-(x - np.log(4096.0))))
    want_y = oracle.f32_to_bf16_bits(p.astype(np.float32))
    gy, gdy = _host(y), _host(dy)
    # FP32 denormal results flush: ULPs are counted where p is a normal number
    norm = fin & (p >= 2.0 ** -120)
    assert _ulps_bf16(gy[norm], want_y[norm]).max() <= 1
    assert (np.abs(oracle.bf16_bits_to_f32(gy[fin & ~norm])) <= 2.0 ** -120).all()
    # p (1 - p) cancels near p = 1, where the FP32 p (v_exp_f32, v_rcp_f32:
    # a few FP32 ULPs) carries up to ~2^-22 absolute error; elsewhere the
    # BF16 rounding of dy dominates
    err = np.abs(oracle.bf16_bits_to_f32(gdy[fin]).astype(np.float64) - (p * (1 - p))[fin])
    tol = 2.0 ** -8 * np.abs(p * (1 - p))[fin] + 2.0 ** -21
    assert (err <= tol).all()
    nan = np.isnan(x)
    assert np.isnan(oracle.bf16_bits_to_f32(gy[nan])).all()
