"""Resolver errors of the sfu_repro activation layer (no GPU needed;
src/sfu_repro/activations.py:35-45, 246-249, 307-308)."""

import pytest


def test_unknown_activation_and_sources(monkeypatch):
    from sfu_repro import activations

    with pytest.raises(ValueError, match="unknown activation 'relu'"):
        activations.resolve_mlp_activation_impl("relu")
    with pytest.raises(ValueError, match="unknown coeff_source"):
        activations.resolve_mlp_activation_impl("spline_silu_compile", coeff_source="x")
    monkeypatch.delenv("SFU_REPRO_ALLOW_SOLLYA_SWEEP", raising=False)
    with pytest.raises(ValueError, match="Sollya coefficients are benchmark-only"):
        activations.resolve_mlp_activation_impl("spline_silu_compile", coeff_source="sollya")
    with pytest.raises(ValueError, match="backward_impl must be"):
        activations.resolve_mlp_activation_packed_impl("spline_silu_compile", backward_impl="x")
    assert activations.resolve_mlp_activation_impl("native_silu")[0] == "native_silu"
    name, act = activations.resolve_mlp_activation_impl("spline_gelu")
    assert name == "spline_gelu[d5,current]" and act.__name__ == "spline_gelu_d5_current_direct"
    name, _ = activations.resolve_mlp_activation_impl("spline_gelu_compile", degree=4)
    assert name == "spline_gelu_compile[d4,current]"
    with pytest.raises(ValueError, match="Sollya coefficients are benchmark-only"):
        activations.resolve_mlp_activation_impl("spline_gelu", coeff_source="sollya")
    monkeypatch.setenv("SFU_REPRO_ALLOW_SOLLYA_SWEEP", "1")
    assert activations.resolve_mlp_activation_impl(
        "spline_gelu", degree=6, coeff_source="sollya")[0] == "spline_gelu[d6,sollya]"


def test_spline_compile_factories_validate_arguments():
    import spline_compile

    with pytest.raises(ValueError, match="Unknown coeff_source"):
        spline_compile.make_spline_silu(3, "nope")
    with pytest.raises(ValueError, match="Unknown packed SwiGLU backward_impl"):
        spline_compile.make_spline_silu_packed(3, "current", backward_impl="bad")
    act = spline_compile.make_spline_silu_packed(3, "current")
    assert act.__spline_op__ == "spline_ops::swish_mul_packed_variant_fwd"
    assert spline_compile.make_spline_gelu() is spline_compile.spline_gelu
    assert spline_compile.make_spline_gelu(4, "sollya").__name__ == "spline_gelu_d4_sollya"


def test_extension_rejects_host_tensors():
    import torch

    import spline_ops

    for name in ("gelu_fwd", "gelu_fwd_d3", "gelu_fwd_d6", "gelu_bwd", "gelu_fwd_variant",
                 "gelu_bwd_variant", "gelu_ag_variant"):
        assert hasattr(spline_ops, name), name

    with pytest.raises(RuntimeError, match="x must be a CUDA tensor"):
        spline_ops.swish_fwd(torch.zeros(4, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="scores must be a CUDA tensor"):
        spline_ops.flash_sigmoid_direct_d3_d4_bf16(torch.zeros(4, dtype=torch.bfloat16))
