"""Routed exp2 (B5: four of every `route` keys take the polynomial) must
route exactly the keys the reference routes.  The ordinary parity
tolerances cannot see a misrouted key (the routed-vs-hardware difference is
a fraction of a BF16 ULP per element), so these tests compare against three
references at once -- the correct routing, hardware exp2 everywhere, and
the routing shifted by four slots -- and require the kernel to be much
closer to the first:

* forward: the log-sum-exp is an FP32 output, so it resolves the routed
  polynomial's error exactly; the inputs put every row's maximum in the
  first key tile, so the kernel's online maximum never moves and its
  exponents are the reference's;
* backward: P is recomputed from the saved log-sum-exp, the reference does
  the same, and the PWL2 program's error is large enough to stand out of
  the BF16 rounding of dQ, dK, dV in an L2 norm over all elements.

Also covers the S = 384 backward cases that reach the 4-wave dQ blocks at
head_dim 128 (the 8-wave blocks need an even number of 128-row query blocks,
ceil(S / 128) even; S = 384 has three)."""

import math

import pytest
import torch

import attention_reference as AR
from attention_reference import default_bias, reference_bwd, reference_fwd
from test_gpu_flash_attention_bwd import _close, _inputs, bwd, fwd

pytestmark = pytest.mark.gpu


def _shifted_routing():
    """Context: the reference with every key's routing slot moved by four."""
    class Shift:
        def __enter__(self):
            self.orig = AR.route_slot
            AR.route_slot = lambda keys: self.orig(keys) + 4

        def __exit__(self, *exc):
            AR.route_slot = self.orig
    return Shift()


def _max_in_first_tile(seed, s=256, d=128):
    """Inputs whose every row maximum lies in keys 0..63: later keys are
    scaled down, and the first seed (from `seed` on) for which that holds
    for every row is taken."""
    for sd in range(seed, seed + 64):
        q, k, v, do = _inputs(1, 4, 2, s, sd, d=d)
        kf = k.float()
        kf[:, 64:] *= 0.25  # later keys score lower
        k = kf.bfloat16()
        qf, kh, _ = AR._heads(q, k, v)
        a = qf @ kh.transpose(-1, -2)
        if bool((a[..., :64].amax(-1) > a[..., 64:].amax(-1)).all()):
            return q, k, v, do
    raise AssertionError("no seed puts every row maximum in the first key tile")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("mode,route", [("softmax_pwl2", 10), ("softmax_pwl2", 6), ("softmax_d2", 6),
                                        ("softmax_d2", 12), ("softmax_pwl2_safe_f16", 12),
                                        ("softmax_pwl2_safe", 10), ("softmax_d2_safe_bf16", 12)])
def test_forward_routing_is_exact(capi, oracle, cuda, mode, route, causal):
    q, k, v, _ = _max_in_first_tile(700 + route + 3 * causal)
    scale = 1 / math.sqrt(128)
    out, lse = fwd(capi, cuda, q, k, v, mode, causal, scale, route=route)
    out, lse = out.cpu().float(), lse.cpu()
    o_r, l_r = reference_fwd(oracle, q, k, v, mode, causal, scale, route=route)
    o_h, l_h = reference_fwd(oracle, q, k, v, "softmax_native", causal, scale)
    with _shifted_routing():
        o_w, l_w = reference_fwd(oracle, q, k, v, mode, causal, scale, route=route)
    err = (lse - l_r).abs().mean().item()
    gap = min((l_r - l_h).abs().mean().item(), (l_r - l_w).abs().mean().item())
    print(f"{mode} route {route} causal {causal}: lse err {err:.3g}, gap {gap:.3g}", flush=True)
    assert gap > 1e-5
    assert err < 0.1 * gap, (err, gap)
    if mode not in ("softmax_pwl2", "softmax_pwl2_safe_f16"):
        # D2 is continuous across integer exponents (p(0) = 1, p(1) = 2), so
        # every row agrees; PWL2 jumps there (p(1-) = 1.98154 against
        # 2 p(0) = 1.97892), and an exponent that the kernel's FP32 fma and
        # the reference's two roundings put on opposite sides of an integer
        # moves that row by up to 1.3e-3 of one probability; the FP16 PWL2
        # rounds the fraction to FP16, a step of up to 4e-4 of a probability
        # wherever those two exponents round to neighbouring FP16 fractions
        assert (lse - l_r).abs().max().item() < 0.25 * gap
    # the BF16 output: within the usual tolerance of the routed reference
    ok, info = _close(out, o_r, rel=1.5e-2)
    assert ok, info


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("mode,route", [("softmax_pwl2", 6), ("softmax_pwl2", 10), ("softmax_pwl2_safe_f16", 12),
                                        ("softmax_pwl2_safe_f16", 16)])
def test_backward_routing_is_exact(capi, oracle, cuda, mode, route, causal):
    """The gradients' BF16 rounding sets a noise floor (an L2 error of about
    0.15 here) that the routed program's effect must clear: at route 32 (one
    key in eight routed) it does not, so routing is checked at 6-16; route 32
    runs the same slot function and is checked against the reference at the
    usual tolerance (test_gpu_flash_attention_bwd.py)."""
    q, k, v, do = _inputs(1, 4, 2, 256, 800 + route + causal)
    scale = 1 / math.sqrt(128)
    out, lse = fwd(capi, cuda, q, k, v, mode, causal, scale, route=route)
    got = bwd(capi, cuda, q, k, v, out, do, lse, mode, 0, causal, scale, route=route)[:3]
    args = (oracle, q, k, v, out, do, lse, mode, 0, causal, scale, 30.0)
    ref_r = reference_bwd(*args, route, 0.0)
    ref_h = reference_bwd(*args, 0, 0.0)
    with _shifted_routing():
        ref_w = reference_bwd(*args, route, 0.0)
    flat = lambda ts: torch.cat([t.reshape(-1).double() for t in ts])
    g, r, h, w = flat(got), flat(ref_r), flat(ref_h), flat(ref_w)
    err = (g - r).norm().item()
    gap_h, gap_w = (r - h).norm().item(), (r - w).norm().item()
    print(f"route {route} causal {causal}: err {err:.4g}, gap hw {gap_h:.4g}, gap shifted {gap_w:.4g}", flush=True)
    # a kernel routing like the alternative would sit about sqrt(err^2 + gap^2) away
    assert err < 0.8 * gap_h, (err, gap_h)
    assert err < 0.8 * gap_w, (err, gap_w)
    assert (g - h).norm().item() > 1.2 * err
    assert (g - w).norm().item() > 1.2 * err


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("mode,route", [("softmax_native", 0), ("softmax_d2", 12), ("sigmoid_native", 0)])
def test_backward_seq_384_four_wave_dq(capi, oracle, cuda, mode, route, causal):
    """S = 384 at head_dim 128: the dQ kernel falls back to 4-wave blocks for
    the modes that otherwise run 8-wave blocks."""
    q, k, v, do = _inputs(1, 4, 2, 384, 850 + AR.M[mode] + route + causal)
    scale = 1 / math.sqrt(128)
    out, lse = fwd(capi, cuda, q, k, v, mode, causal, scale, route=route if route else 4)
    dq, dk, dv, _ = bwd(capi, cuda, q, k, v, out, do, lse, mode, 0, causal, scale, route=route)
    rq, rk, rv = reference_bwd(oracle, q, k, v, out, do, lse, mode, 0, causal, scale, 30.0, route,
                               default_bias(mode, 384))
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert torch.isfinite(got).all(), name
        ok, info = _close(got, ref)
        assert ok, (mode, route, causal, name, info)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("mode,route", [("softmax_pwl1_safe", 14), ("softmax_pwl1_safe_f16", 22),
                                        ("softmax_pwl2_safe", 40), ("softmax_d2_safe_bf16", 64)])
def test_runtime_routes(capi, oracle, cuda, mode, route, causal):
    """Routes without a template instantiation (FA4 accepts any even
    frequency >= 4) read their pattern from the kernel arguments.  Forward:
    the lse is much closer to the reference routed this way than to hardware
    exp2, to the shifted routing and, above 32, to the pattern restarted at
    every 64-key tile (route 32's).  Backward: discriminated the same way at
    14 and 22, with the PWL1 programs, whose 6.6 % error stands well above
    the gradients' BF16 noise (PWL2's 1 % barely clears it at route 14); at
    40 and 64 (one key in 10 or 16 routed) against the reference at the
    usual tolerance.  All four programs are continuous at integer exponents,
    so no exponent rounded to the other side of an integer moves a row."""
    q, k, v, do = _inputs(1, 4, 2, 256, 1900 + route + causal)
    scale = 1 / math.sqrt(128)
    print(f"runtime route {mode} {route} causal {causal}", flush=True)
    out, lse = fwd(capi, cuda, q, k, v, mode, causal, scale, route=route)
    lse_c = lse.cpu()
    l_r = reference_fwd(oracle, q, k, v, mode, causal, scale, route=route)[1]
    alternatives = [reference_fwd(oracle, q, k, v, "softmax_native", causal, scale)[1]]
    with _shifted_routing():
        alternatives.append(reference_fwd(oracle, q, k, v, mode, causal, scale, route=route)[1])
    if route > 32:
        alternatives.append(reference_fwd(oracle, q, k, v, mode, causal, scale, route=32)[1])
    err = (lse_c - l_r).abs().mean().item()
    gap = min((l_r - a).abs().mean().item() for a in alternatives)
    print(f"  lse err {err:.3g}, gap {gap:.3g}", flush=True)
    assert gap > 1e-5
    assert err < 0.1 * gap, (err, gap)
    got = bwd(capi, cuda, q, k, v, out, do, lse, mode, 0, causal, scale, route=route)[:3]
    args = (oracle, q, k, v, out, do, lse, mode, 0, causal, scale, 30.0)
    ref_r = reference_bwd(*args, route, 0.0)
    for name, g_, r_ in zip(("dq", "dk", "dv"), got, ref_r):
        assert torch.isfinite(g_).all(), name
        ok, info = _close(g_, r_)
        assert ok, (name, info)
    if route <= 32:
        flat = lambda ts: torch.cat([t.reshape(-1).double() for t in ts])
        ref_h = reference_bwd(*args, 0, 0.0)
        with _shifted_routing():
            ref_w = reference_bwd(*args, route, 0.0)
        g, r, h, w = flat(got), flat(ref_r), flat(ref_h), flat(ref_w)
        e = (g - r).norm().item()
        print(f"  bwd err {e:.4g}, gap hw {(r - h).norm().item():.4g}, shifted {(r - w).norm().item():.4g}",
              flush=True)
        assert e < 0.8 * (r - h).norm().item() and e < 0.8 * (r - w).norm().item()
