"""GPU parity of the FP16 experiment kernels (hybrid, fused, forward with
derivative, multiply; autonumerics_zero/spline_ops/spline_kernels.cu:776-1168)
through the C ABI: polynomial lanes bit for bit against the oracle, the
hybrid's transcendental lanes bit for bit against the native kernel of the
same program, and the pybind surface."""

import numpy as np
import pytest
import torch

from test_gpu_parity import _dev, _host, assert_bits_equal

pytestmark = pytest.mark.gpu

FAMS = ("sigmoid", "tanh", "swish")


def _operands(n, seed):
    rng = np.random.default_rng(seed)
    x = np.concatenate([np.arange(65536, dtype=np.uint32).astype(np.uint16),
                        rng.integers(0, 65536, max(0, n - 65536), dtype=np.uint32).astype(np.uint16)])[:n]
    go = (rng.standard_normal(n) * 2).astype(np.float16).view(np.uint16)
    return np.ascontiguousarray(x), go


def _sfu_lanes(n):
    """Element mask of the transcendental lanes: the first pair of every
    8 elements when the hybrid split applies (n >= 8192, n % 8 == 0)."""
    m = np.zeros(n, dtype=bool)
    if n >= 8192 and n % 8 == 0:
        m[(np.arange(n) % 8) < 2] = True
    return m


@pytest.mark.parametrize("n", [65536, 65536 + 8, 4096, 65536 + 3])
@pytest.mark.parametrize("fam", FAMS)
def test_hybrid_forward(capi, oracle, cuda, fam, n):
    x, _ = _operands(n, 1)
    xd = _dev(x, "f16", cuda)
    y = torch.empty_like(xd)
    nat = torch.empty_like(xd)
    capi.call(f"launch_{fam}_fwd_hybrid_kernel", y, xd, n)
    capi.call(f"launch_{fam}_fwd_native_kernel", nat, xd, n)
    torch.cuda.synchronize()
    got = _host(y)
    want = oracle.activation(fam, oracle.FWD, 3, "f16", x)
    sfu = _sfu_lanes(n)
    want = np.where(sfu, _host(nat), want).astype(np.uint16)
    assert_bits_equal(got, want, "f16", f"{fam} fwd hybrid n={n}")


def _native_bwd(fam, x64):
    s = 1 / (1 + np.exp(-x64))
    if fam == "sigmoid":
        return s * (1 - s)
    if fam == "tanh":
        return 1 - np.tanh(x64) ** 2
    return s * (1 + x64 * (1 - s))


@pytest.mark.parametrize("n", [65536, 4096 + 5])
@pytest.mark.parametrize("fam", FAMS)
def test_hybrid_backward(capi, oracle, cuda, fam, n):
    x, go = _operands(n, 2)
    xd, god = _dev(x, "f16", cuda), _dev(go, "f16", cuda)
    gi = torch.empty_like(xd)
    capi.call(f"launch_{fam}_bwd_hybrid_kernel", gi, god, xd, n)
    torch.cuda.synchronize()
    got = _host(gi)
    want = oracle.activation_bwd(fam, 4, "f16", go, x)
    sfu = _sfu_lanes(n)
    assert_bits_equal(got[~sfu], want[~sfu], "f16", f"{fam} bwd hybrid poly lanes")
    if sfu.any():
        with np.errstate(invalid="ignore"):
            xv = oracle.f16_bits_to_f32(x[sfu]).astype(np.float64)
        gv = oracle.f16_bits_to_f32(go[sfu]).astype(np.float64)
        ok = np.isfinite(xv) & (np.abs(xv) < 60)
        ref = gv[ok] * _native_bwd(fam, xv[ok])
        g = oracle.f16_bits_to_f32(got[sfu][ok]).astype(np.float64)
        # FP32 transcendental derivative rounded to FP16, then one FP16 product
        tol = 2 ** -9 * np.abs(ref) + 2e-6 * np.abs(gv[ok]) + 2 ** -24
        assert (np.abs(g - ref) <= tol).all()


@pytest.mark.parametrize("n", [65536, 4097])
@pytest.mark.parametrize("fam", FAMS)
def test_fused_forward_backward(capi, oracle, cuda, fam, n):
    x, go = _operands(n, 3)
    xd, god = _dev(x, "f16", cuda), _dev(go, "f16", cuda)
    y, gi = torch.empty_like(xd), torch.empty_like(xd)
    capi.call(f"launch_{fam}_fused_kernel", y, gi, xd, god, n)
    torch.cuda.synchronize()
    want_y = oracle.activation(fam, oracle.FWD, 3, "f16", x)
    if fam == "swish":
        want_gi = oracle.activation_bwd(fam, 4, "f16", go, x)
    else:
        want_gi = oracle.activation_bwd_alg(fam, "f16", go, want_y)
    assert_bits_equal(_host(y), want_y, "f16", f"{fam} fused y")
    assert_bits_equal(_host(gi), want_gi, "f16", f"{fam} fused gi")


@pytest.mark.parametrize("n", [65536, 1001])
@pytest.mark.parametrize("name", ["sigmoid_fwd_deriv_alg", "sigmoid_fwd_deriv_poly", "tanh_fwd_deriv_alg",
                                  "tanh_fwd_deriv_poly", "swish_fwd_deriv", "swish_fwd_deriv_poly"])
def test_forward_with_derivative(capi, oracle, cuda, name, n):
    x, _ = _operands(n, 4)
    xd = _dev(x, "f16", cuda)
    y, dy = torch.empty_like(xd), torch.empty_like(xd)
    capi.call(f"launch_{name}_kernel", y, dy, xd, n)
    torch.cuda.synchronize()
    fam = name.split("_")[0]
    if name == "swish_fwd_deriv":
        want_y, want_dy = oracle.swish_fwd_deriv_shared(x)
    else:
        want_y = oracle.activation(fam, oracle.FWD, 3, "f16", x)
        if name.endswith("alg"):
            ones = np.full(n, 0x3C00, dtype=np.uint16)
            want_dy = oracle.activation_bwd_alg(fam, "f16", ones, want_y)
        else:
            want_dy = oracle.activation(fam, oracle.BWD, 4, "f16", x)
    assert_bits_equal(_host(y), want_y, "f16", name + " y")
    assert_bits_equal(_host(dy), want_dy, "f16", name + " dy")


@pytest.mark.parametrize("n", [1 << 18, 1003])
@pytest.mark.parametrize("fmt", ["f16", "bf16"])
def test_multiply(capi, oracle, cuda, fmt, n):
    rng = np.random.default_rng(5)
    a = rng.integers(0, 65536, n, dtype=np.uint32).astype(np.uint16)
    b = rng.integers(0, 65536, n, dtype=np.uint32).astype(np.uint16)
    ad, bd = _dev(a, fmt, cuda), _dev(b, fmt, cuda)
    out = torch.empty_like(ad)
    capi.call("launch_multiply_kernel" + ("_bf16" if fmt == "bf16" else ""), out, ad, bd, n)
    torch.cuda.synchronize()
    assert_bits_equal(_host(out), oracle.multiply(fmt, a, b), fmt, f"multiply {fmt}")


def test_binding_surface(spline_ops, oracle, cuda):
    x = torch.randn(64, 256, device=cuda).half() * 3
    go = torch.randn(64, 256, device=cuda).half()
    y, gi = spline_ops.sigmoid_fused(x, go)
    bits = lambda t: t.reshape(-1).view(torch.int16).cpu().numpy().view(np.uint16)
    wy = oracle.activation("sigmoid", oracle.FWD, 3, "f16", bits(x))
    assert np.array_equal(bits(y), wy)
    assert np.array_equal(bits(gi), oracle.activation_bwd_alg("sigmoid", "f16", bits(go), wy))
    ys, dys = spline_ops.swish_fwd_deriv(x)
    wy, wdy = oracle.swish_fwd_deriv_shared(bits(x))
    assert np.array_equal(bits(ys), wy) and np.array_equal(bits(dys), wdy)
    assert torch.equal(spline_ops.multiply(go, dys), go * dys)
    xb = x.bfloat16()
    assert torch.equal(spline_ops.multiply(xb, xb), (xb.float() * xb.float()).bfloat16())
    h = spline_ops.tanh_fwd_hybrid(x)
    assert h.shape == x.shape and h.dtype == torch.float16
    with pytest.raises(RuntimeError, match=r"x must be float16 \(no BF16 support for this op\)"):
        spline_ops.sigmoid_fwd_hybrid(xb)
    with pytest.raises(RuntimeError, match="same number of elements"):
        spline_ops.tanh_fused(x, go[:10])
