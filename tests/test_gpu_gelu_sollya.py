"""GPU parity of the GeLU programs (FP16, BF16) and of the BF16 Sollya
coefficient set (sigmoid, SiLU, SwiGLU, GeLU) against the CPU oracle, bit for
bit, through the C ABI; then the binding surface that selects them
(autonumerics_zero/spline_ops/spline_ops.cpp:1187-1502, 2401-2420)."""

import numpy as np
import pytest
import torch

from test_gpu_parity import DTYPES, _dev, _host, _operands, assert_bits_equal

pytestmark = pytest.mark.gpu

# (family, oracle format, launcher suffix)
UNARY = [("gelu", "f16", ""), ("gelu", "bf16", "_bf16")] + [
    (fam, "bf16_sollya", "_bf16_sollya") for fam in ("sigmoid", "swish", "gelu")]


def _store(fmt):
    return "f16" if fmt == "f16" else "bf16"


@pytest.mark.parametrize("degree", [3, 4, 5, 6])
@pytest.mark.parametrize("fam,fmt,sfx", UNARY)
def test_forward_exhaustive(capi, oracle, cuda, fam, fmt, sfx, degree):
    x = oracle.all_bits()
    xd = _dev(x, _store(fmt), cuda)
    y = torch.empty_like(xd)
    capi.call(f"launch_{fam}_fwd_d{degree}_kernel{sfx}", y, xd, x.size)
    torch.cuda.synchronize()
    want = oracle.activation(fam, oracle.FWD, degree, fmt, x)
    assert_bits_equal(_host(y), want, _store(fmt), f"{fam} fwd d{degree} {fmt}")


@pytest.mark.parametrize("degree", [3, 4, 5, 6])
@pytest.mark.parametrize("fam,fmt,sfx", UNARY)
def test_backward_program_times_grad(capi, oracle, cuda, fam, fmt, sfx, degree):
    store = _store(fmt)
    rng = np.random.default_rng(2000 + degree)
    x = np.tile(oracle.all_bits(), 2)
    g = rng.standard_normal(x.size).astype(np.float32)
    go = oracle.f32_to_bf16_bits(g) if store == "bf16" else g.astype(np.float16).view(np.uint16)
    go[:65536] = 0x3C00 if store == "f16" else 0x3F80
    xd, god = _dev(x, store, cuda), _dev(go, store, cuda)
    gi = torch.empty_like(xd)
    capi.call(f"launch_{fam}_bwd_d{degree}_kernel{sfx}", gi, god, xd, x.size)
    torch.cuda.synchronize()
    want = oracle.activation_bwd(fam, degree, fmt, go, x)
    assert_bits_equal(_host(gi), want, store, f"{fam} bwd d{degree} {fmt}")


@pytest.mark.parametrize("degree", [3, 4, 5, 6])
def test_sollya_swish_mul(capi, oracle, cuda, degree):
    n = 65536 * 2 + 13
    go, gate, up = _operands(oracle, "bf16", n, 70 + degree)
    god, gd, ud = (_dev(a, "bf16", cuda) for a in (go, gate, up))
    out = torch.empty_like(gd)
    capi.call(f"launch_swish_mul_fwd_d{degree}_kernel_bf16_sollya", out, gd, ud, n)
    gg, gu = torch.empty_like(gd), torch.empty_like(gd)
    capi.call(f"launch_swish_mul_bwd_d{degree}_kernel_bf16_sollya", gg, gu, god, gd, ud, n)
    torch.cuda.synchronize()
    assert_bits_equal(_host(out), oracle.swish_mul_fwd(degree, "bf16_sollya", gate, up), "bf16",
                      f"sollya swish_mul fwd d{degree}")
    want_gg, want_gu = oracle.swish_mul_bwd(degree, "bf16_sollya", go, gate, up)
    assert_bits_equal(_host(gg), want_gg, "bf16", f"sollya swish_mul grad_gate d{degree}")
    assert_bits_equal(_host(gu), want_gu, "bf16", f"sollya swish_mul grad_up d{degree}")


@pytest.mark.parametrize("degree", [3, 4, 5, 6])
@pytest.mark.parametrize("hidden", [2048, 6])
def test_sollya_packed_matches_separate(capi, cuda, degree, hidden):
    rows = 37
    torch.manual_seed(degree * 7 + hidden)
    packed = (torch.randn(rows, 2 * hidden, device=cuda) * 3).bfloat16()
    go = torch.randn(rows, hidden, device=cuda).bfloat16()
    gate, up = (p.contiguous() for p in packed.chunk(2, dim=-1))
    sfx = f"d{degree}_kernel_bf16_sollya"
    out_p = torch.empty(rows, hidden, device=cuda, dtype=torch.bfloat16)
    capi.call(f"launch_swish_mul_packed_fwd_{sfx}", out_p, packed, rows, hidden)
    out_s = torch.empty_like(gate)
    capi.call(f"launch_swish_mul_fwd_{sfx}", out_s, gate, up, gate.numel())
    grad_p = torch.empty_like(packed)
    capi.call(f"launch_swish_mul_packed_bwd_{sfx}", grad_p, go, packed, rows, hidden)
    gg, gu = torch.empty_like(gate), torch.empty_like(gate)
    capi.call(f"launch_swish_mul_bwd_{sfx}", gg, gu, go, gate, up, gate.numel())
    torch.cuda.synchronize()
    assert torch.equal(out_p.view(torch.int16), out_s.view(torch.int16))
    assert torch.equal(grad_p.view(torch.int16), torch.cat((gg, gu), -1).view(torch.int16))


# ---- binding ------------------------------------------------------------------


def _eq(a, b):
    torch.testing.assert_close(a, b, rtol=0.0, atol=0.0)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_gelu_binding_functions(spline_ops, cuda, dt):
    x = torch.linspace(-8, 8, 10007, device=cuda).to(dt)
    go = torch.linspace(1, -1, 10007, device=cuda).to(dt)
    _eq(spline_ops.gelu_fwd(x), spline_ops.gelu_fwd_d5(x))
    _eq(spline_ops.gelu_bwd(go, x), spline_ops.gelu_bwd_d5(go, x))
    for d in (3, 4, 5, 6):
        _eq(getattr(spline_ops, f"gelu_fwd_d{d}")(x), spline_ops.gelu_fwd_variant(x, d, 0))
        _eq(getattr(spline_ops, f"gelu_bwd_d{d}")(go, x), spline_ops.gelu_bwd_variant(go, x, d, 0))
    ref = torch.nn.functional.gelu(x.float())
    # D5 GeLU: fit error of Phi plus the 16-bit rounding of Phi and of x * Phi,
    # both growing with |x| (measured on the oracle: FP16 0.0013 (|x| + 1),
    # BF16 0.0225 (|x| + 1) at most on [-8, 8])
    rel = 0.002 if dt == torch.float16 else 0.03
    err = (spline_ops.gelu_fwd(x).float() - ref).abs() / (x.float().abs() + 1)
    assert float(err.max()) < rel


def test_gelu_autograd_variant(spline_ops, cuda):
    for c in (0, 1):
        x = torch.linspace(-6, 6, 4099, device=cuda, dtype=torch.bfloat16).requires_grad_(True)
        y = spline_ops.gelu_ag_variant(x, 4, c)
        g = torch.linspace(1, -1, 4099, device=cuda, dtype=torch.bfloat16)
        y.backward(g)
        _eq(y, spline_ops.gelu_fwd_variant(x.detach(), 4, c))
        _eq(x.grad, spline_ops.gelu_bwd_variant(g, x.detach(), 4, c))


def test_sollya_through_the_binding(spline_ops, capi, cuda):
    x = torch.linspace(-9, 9, 8195, device=cuda, dtype=torch.bfloat16)
    go = torch.linspace(-1, 1, 8195, device=cuda, dtype=torch.bfloat16)
    for fam in ("sigmoid", "swish", "gelu"):
        for d in (3, 4, 5, 6):
            y = torch.empty_like(x)
            capi.call(f"launch_{fam}_fwd_d{d}_kernel_bf16_sollya", y, x, x.numel())
            gi = torch.empty_like(x)
            capi.call(f"launch_{fam}_bwd_d{d}_kernel_bf16_sollya", gi, go, x, x.numel())
            torch.cuda.synchronize()
            _eq(getattr(spline_ops, f"{fam}_fwd_variant")(x, d, 1), y)
            _eq(getattr(spline_ops, f"{fam}_bwd_variant")(go, x, d, 1), gi)
    xe = x[:8194].contiguous()  # packed hidden size must be even
    packed = torch.cat((xe, xe)).reshape(1, -1)
    _eq(spline_ops.swish_mul_packed_fwd_variant(packed, 3, 1),
        spline_ops.swish_mul_fwd_variant(xe, xe, 3, 1).reshape(1, -1))
    # Sollya D3 uses the program pair, not the algebraic D3 backward
    a = spline_ops.swish_mul_bwd_variant(go, x, x, 3, 1)
    b = spline_ops.swish_mul_bwd_variant(go, x, x, 3, 0)
    assert not torch.equal(a[0], b[0])


def test_sollya_errors(spline_ops, cuda):
    h = torch.zeros(8, device=cuda, dtype=torch.float16)
    b = torch.zeros(8, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="FP16 spline kernels only support coeff_source=current"):
        spline_ops.gelu_fwd_variant(h, 3, 1)
    with pytest.raises(RuntimeError, match="Unsupported GeLU forward degree: 7"):
        spline_ops.gelu_fwd_variant(b, 7, 0)
    with pytest.raises(RuntimeError, match="Unsupported swish forward degree: 0"):
        spline_ops.swish_fwd_variant(b, 0, 1)  # no native entry in the Sollya set
    with pytest.raises(RuntimeError, match="coeff_source=sollya has no tanh forward programs"):
        spline_ops.tanh_fwd_variant(b, 3, 1)


def test_compiled_gelu(cuda):
    from spline_compile import make_spline_gelu, spline_gelu

    import spline_ops

    x0 = torch.linspace(-5, 5, 4097, device=cuda, dtype=torch.bfloat16)
    g = torch.linspace(1, -1, 4097, device=cuda, dtype=torch.bfloat16)
    for act, d, c in ((spline_gelu, 5, 0), (make_spline_gelu(4, "sollya"), 4, 1)):
        x = x0.clone().requires_grad_(True)
        y = torch.compile(act, fullgraph=True)(x)
        y.backward(g)
        _eq(y, spline_ops.gelu_fwd_variant(x0, d, c))
        _eq(x.grad, spline_ops.gelu_bwd_variant(g, x0, d, c))


def test_gelu_resolver(cuda, monkeypatch):
    from sfu_repro import activations

    import spline_ops

    x = torch.linspace(-4, 4, 4100, device=cuda, dtype=torch.float16)
    name, act = activations.resolve_mlp_activation_impl("spline_gelu")
    assert name == "spline_gelu[d5,current]"
    _eq(act(x), spline_ops.gelu_fwd_variant(x, 5, 0))
    name, act = activations.resolve_mlp_activation_impl("spline_gelu_compile", degree=3)
    _eq(act(x), spline_ops.gelu_fwd_variant(x, 3, 0))
    monkeypatch.setenv("SFU_REPRO_ALLOW_SOLLYA_SWEEP", "1")
    xb = x.bfloat16()
    _, act = activations.resolve_mlp_activation_impl("spline_gelu", degree=6, coeff_source="sollya")
    _eq(act(xb), spline_ops.gelu_fwd_variant(xb, 6, 1))
    _, mul = activations.resolve_mlp_activation_mul_impl("spline_silu", degree=4,
                                                         coeff_source="sollya")
    _eq(mul(xb, xb), spline_ops.swish_mul_fwd_variant(xb, xb, 4, 1))
    assert DTYPES["bf16"] == torch.bfloat16
