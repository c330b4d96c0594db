"""The FA4 interface on the GPU: sfu_repro.fa4 configurations resolved
against this build's runtime (the fused HIP attention), called through
FA4AttentionWrapper with autograd, for the B2, B3 and B5 component configs.
Forward outputs and q/k/v gradients are compared with the CPU references of
attention_reference (oracle programs, same routing)."""

import dataclasses
import math

import pytest
import torch

from attention_reference import reference_bwd, reference_fwd
from sfu_repro.fa4 import (
    FA4AttentionWrapper,
    FA4Config,
    b2_component_configs,
    b3_component_configs,
    b5_component_configs,
    build_fa4_module,
    patch_attention_modules,
    resolve_fa4_config,
)

pytestmark = pytest.mark.gpu


def _qkv(b, h, hkv, s, seed, qmul=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(b, h, s, 128, generator=g) * qmul).bfloat16()
    k = torch.randn(b, hkv, s, 128, generator=g).bfloat16()
    v = torch.randn(b, hkv, s, 128, generator=g).bfloat16()
    do = torch.randn(b, h, s, 128, generator=g).bfloat16()
    return q, k, v, do


def _run(module, cuda, q, k, v, do):
    qd, kd, vd = (t.to(cuda).requires_grad_() for t in (q, k, v))
    out = module(qd, kd, vd)
    out.backward(do.to(cuda))
    torch.cuda.synchronize()
    return out.detach(), qd.grad.cpu().float(), kd.grad.cpu().float(), vd.grad.cpu().float()


def _close(got, ref, rel):
    err = (got - ref).abs().max().item()
    tol = rel * ref.abs().max().item() + 2e-3
    return err <= tol, (err, tol)


def _fa4_layout(t):
    return t.transpose(1, 2).contiguous()


CASES = [
    ("b2", "native", "softcap_native", 0, 0, 6.0),
    ("b2", "polynomial", "softcap_d4", 1, 0, 6.0),
    ("b5", "native", "softmax_native", 0, 0, 1.0),
    ("b5", "d2_safe", "softmax_d2", 0, 32, 1.0),
    ("b5", "pwl2_safe_f16", "softmax_pwl2_safe_f16", 0, 32, 1.0),
]


@pytest.mark.parametrize("group,name,mode,grad,route_bwd,qmul", CASES)
def test_component_configs_through_the_wrapper(oracle, cuda, group, name, mode, grad, route_bwd, qmul):
    configs = {"b2": b2_component_configs, "b5": b5_component_configs}[group]()
    module = build_fa4_module(configs[name], head_dim=128)
    q, k, v, do = _qkv(1, 4, 2, 256, 40 + len(name), qmul)
    out, dq, dk, dv = _run(module, cuda, q, k, v, do)
    scale = 1 / math.sqrt(128)
    route_fwd = configs[name].exp2_emu_freq or 4
    qa, ka, va, doa = (_fa4_layout(t) for t in (q, k, v, do))
    ref_out, _ = reference_fwd(oracle, qa, ka, va, mode, True, scale, 30.0, route_fwd)
    ok, info = _close(out.cpu().float().transpose(1, 2), ref_out, 1.5e-2)
    assert ok, ("out", info)
    # gradients given the kernel's own out / lse (recomputed through the runtime)
    from sfu_repro import fa4_runtime as rt

    resolved = module.config
    o4, lse = rt.flash_attn_fwd(qa.to(cuda), ka.to(cuda), va.to(cuda), softmax_scale=None, causal=True,
                                softcap=resolved.softcap, score_mod=resolved.score_mod,
                                exp2_emu_backend=resolved.exp2_emu_backend, exp2_emu_freq=resolved.exp2_emu_freq)
    rq, rk, rv = reference_bwd(oracle, qa, ka, va, o4, doa, lse, mode, grad, True, scale, 30.0, route_bwd, 0.0)
    for label, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        ok, info = _close(got, ref.transpose(1, 2), 2.5e-2)
        assert ok, (label, info)


@pytest.mark.parametrize("name,mode,grad", [("native", "sigmoid_native", 0), ("polynomial", "sigmoid_b3", 5)])
def test_b3_configs_through_the_wrapper(oracle, cuda, name, mode, grad):
    config = dataclasses.replace(b3_component_configs()[name], sigmoid_qk_norm=False)
    module = build_fa4_module(config, head_dim=128, sequence_length=4096)
    q, k, v, do = _qkv(1, 2, 1, 4096, 60 + grad)
    out, dq, dk, dv = _run(module, cuda, q, k, v, do)
    scale = 1 / math.sqrt(128)
    qa, ka, va, doa = (_fa4_layout(t) for t in (q, k, v, do))
    ref_out, _ = reference_fwd(oracle, qa, ka, va, mode, True, scale)
    ok, info = _close(out.cpu().float().transpose(1, 2), ref_out, 1.5e-2)
    assert ok, ("out", info)
    o4 = _fa4_layout(out.cpu()).to(cuda)
    lse = torch.zeros(1, 2, 4096, device=cuda)
    bias = -math.log(4096) if mode == "sigmoid_native" else 0.0
    rq, rk, rv = reference_bwd(oracle, qa, ka, va, o4, doa, lse, mode, grad, True, scale, 30.0, 0, bias)
    for label, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        ok, info = _close(got, ref.transpose(1, 2), 2.5e-2)
        assert ok, (label, info)


def test_qk_norm_and_module_patching(cuda):
    """sigmoid_qk_norm adds RMSNorm on q and k; patch_attention_modules
    swaps every inner_attention slot once."""
    config = b3_component_configs()["native"]
    resolved = resolve_fa4_config(config, sequence_length=4096)

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.head_dim = 128
            self.inner_attention = torch.nn.Identity()
            self.proj = torch.nn.Linear(4, 4)

    model = torch.nn.Sequential(Block(), Block()).to(cuda).bfloat16()
    assert patch_attention_modules(model, resolved) == 2
    assert patch_attention_modules(model, resolved) == 0
    wrapper = model[0].inner_attention
    assert isinstance(wrapper, FA4AttentionWrapper) and wrapper.q_norm is not None
    q, k, v, _ = _qkv(1, 2, 2, 4096, 70)
    out = wrapper(q.to(cuda), k.to(cuda), v.to(cuda))
    qn = torch.nn.functional.rms_norm(q.to(cuda).float(), (128,)).bfloat16()
    kn = torch.nn.functional.rms_norm(k.to(cuda).float(), (128,)).bfloat16()
    plain = FA4AttentionWrapper(dataclasses.replace(resolved, sigmoid_qk_norm=False), 128)
    ref = plain(qn, kn, v.to(cuda))
    assert (out.float() - ref.float()).abs().max().item() <= 2e-2 * ref.float().abs().max().item() + 2e-3


def test_unbuilt_programs_fail_loudly(cuda):
    cfg = FA4Config(mode="softcap", softcap=30.0, softcap_backend="cute", softcap_backward_mode="analytical")
    q, k, v, _ = _qkv(1, 1, 1, 128, 80)
    with pytest.raises(NotImplementedError, match="cute"):  # at build time, before any launch
        build_fa4_module(cfg, head_dim=128)(q.to(cuda), k.to(cuda), v.to(cuda))
    with pytest.raises(TypeError, match="bfloat16"):
        build_fa4_module(FA4Config(), head_dim=128)(q.half().to(cuda), k.half().to(cuda), v.half().to(cuda))


@pytest.mark.parametrize("group,name,mode,grad,route_bwd,qmul", [
    ("b5", "native", "softmax_native", 0, 0, 1.0),
    ("b5", "d2_safe", "softmax_d2", 0, 32, 1.0),
    ("b5", "pwl2_safe_f16", "softmax_pwl2_safe_f16", 0, 32, 1.0),
    ("b2", "polynomial", "softcap_d4", 1, 0, 6.0),
])
def test_causal_lengths_off_the_block_grid(oracle, cuda, group, name, mode, grad, route_bwd, qmul):
    """S = 200: forward and backward run at S = 200 with no padding (their
    last query and key blocks partial; rows past S are neither read nor
    stored); results match the references evaluated at S = 200."""
    configs = {"b2": b2_component_configs, "b5": b5_component_configs}[group]()
    module = build_fa4_module(configs[name], head_dim=128)
    q, k, v, do = _qkv(1, 4, 2, 200, 50 + len(name), qmul)
    out, dq, dk, dv = _run(module, cuda, q, k, v, do)
    assert out.shape == (1, 4, 200, 128) and dk.shape == (1, 2, 200, 128)
    scale = 1 / math.sqrt(128)
    route_fwd = configs[name].exp2_emu_freq or 4
    qa, ka, va, doa = (_fa4_layout(t) for t in (q, k, v, do))
    ref_out, ref_lse = reference_fwd(oracle, qa, ka, va, mode, True, scale, 30.0, route_fwd)
    ok, info = _close(out.cpu().float().transpose(1, 2), ref_out, 1.5e-2)
    assert ok, ("out", info)
    from sfu_repro import fa4_runtime as rt

    resolved = module.config
    o4, lse = rt.flash_attn_fwd(qa.to(cuda), ka.to(cuda), va.to(cuda), softmax_scale=None, causal=True,
                                softcap=resolved.softcap, score_mod=resolved.score_mod,
                                exp2_emu_backend=resolved.exp2_emu_backend, exp2_emu_freq=resolved.exp2_emu_freq)
    assert lse.shape == (1, 4, 200) and (lse.cpu() - ref_lse).abs().max().item() < 2e-2
    rq, rk, rv = reference_bwd(oracle, qa, ka, va, o4, doa, lse, mode, grad, True, scale, 30.0, route_bwd, 0.0)
    for label, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert torch.isfinite(got).all(), label
        ok, info = _close(got, ref.transpose(1, 2), 2.5e-2)
        assert ok, (label, info)


@pytest.mark.parametrize("mode,mode_name", [(0, "softmax_native"), (4, "softcap_d4"), (5, "sigmoid_native")])
def test_non_causal_lengths_off_the_block_grid(oracle, cuda, mode, mode_name):
    """Non-causal attention at S = 200 through the runtime (the kernel reads no
    row past S) against the references at S = 200."""
    from sfu_repro import fa4_runtime as rt

    q, k, v, do = (_fa4_layout(t) for t in _qkv(1, 4, 2, 200, 90 + mode, 6.0 if mode == 4 else 1.0))
    scale = 1 / math.sqrt(128)
    kwargs = {}
    if mode == 4:
        kwargs["score_mod"] = rt.create_softcap_scoremod_backend(30.0, degree=4, backend="device")
        kwargs["softcap"] = 30.0
    if mode == 5:
        kwargs.update(sigmoid_attention=True, sigmoid_sfu_freq=16, sigmoid_sfu_res=16)
    qd, kd, vd, dod = (t.to(cuda) for t in (q, k, v, do))
    out, lse = rt.flash_attn_fwd(qd, kd, vd, softmax_scale=scale, causal=False, **kwargs)
    assert out.shape == (1, 200, 4, 128)
    bias = -math.log(200) if mode == 5 else 0.0
    ref_out, ref_lse = reference_fwd(oracle, q, k, v, mode_name, False, scale, 30.0, 4, bias)
    ok, info = _close(out.cpu().float(), ref_out, 1.5e-2)
    assert ok, ("out", info)
    if ref_lse is not None:
        assert (lse.cpu() - ref_lse).abs().max().item() < 2e-2
    grad = 1 if mode == 4 else 0
    bwd_kwargs = dict(kwargs)
    if mode == 4:
        bwd_kwargs["score_mod_bwd"] = None
    dq, dk, dv = rt.flash_attn_bwd(qd, kd, vd, out, dod, lse, softmax_scale=scale, causal=False, **bwd_kwargs)
    rq, rk, rv = reference_bwd(oracle, q, k, v, out.cpu(), do, lse.cpu(), mode_name, grad, False, scale, 30.0, 0,
                               bias)
    for label, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        got = got.cpu().float()
        assert torch.isfinite(got).all(), label
        ok, info = _close(got, ref, 2.5e-2)
        assert ok, (label, info)
