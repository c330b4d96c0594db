"""Activation resolvers over the MI355X polynomial kernels.

Same names, return values and errors as the reference's
``src/sfu_repro/activations.py``: each ``resolve_*`` returns
``(implementation_name, callable)``; ``native_*`` names map to PyTorch's own
functions, ``spline_silu`` calls the pybind functions directly (with C++
autograd when gradients are needed) and ``spline_silu_compile`` goes through
the ``spline_compile`` dispatcher ops; ``spline_gelu`` /
``spline_gelu_compile`` do the same for the GeLU programs.
"""

from __future__ import annotations

import os
from functools import lru_cache

import torch
import torch.nn.functional as F

PUBLIC_MLP_ACTIVATIONS = (
    "native_silu",
    "spline_silu",
    "spline_silu_compile",
    "native_gelu",
    "spline_gelu",
    "spline_gelu_compile",
)

_COEFF_SOURCE_TO_ID = {"current": 0, "sollya": 1}


def _env_flag(name: str) -> bool:
    value = os.environ.get(name)
    return value is not None and value.lower() in ("1", "true", "yes", "on")


def _ensure_coeff_source_allowed(coeff_source: str) -> None:
    """src/sfu_repro/activations.py:35-45"""
    if coeff_source not in _COEFF_SOURCE_TO_ID:
        raise ValueError(
            f"unknown coeff_source {coeff_source!r}; expected one of {tuple(_COEFF_SOURCE_TO_ID)}")
    if coeff_source == "sollya" and not _env_flag("SFU_REPRO_ALLOW_SOLLYA_SWEEP"):
        raise ValueError(
            "Sollya coefficients are benchmark-only. Set "
            "SFU_REPRO_ALLOW_SOLLYA_SWEEP=1 for an explicit sweep.")


def _coeff_source_id(coeff_source: str) -> int:
    _ensure_coeff_source_allowed(coeff_source)
    return _COEFF_SOURCE_TO_ID[coeff_source]


@lru_cache(maxsize=1)
def load_spline_ops():
    """Import the compiled HIP extension; fail loudly when it is absent."""
    try:
        import spline_ops
    except (ImportError, OSError) as error:
        raise RuntimeError(
            "The compiled spline_ops extension is unavailable. Build it with "
            "fast-polynomial-transcendentals_amd/build.py first.") from error
    return spline_ops


@lru_cache(maxsize=1)
def _spline_compile():
    try:
        import spline_compile
    except (ImportError, OSError) as error:
        raise RuntimeError(
            "spline_compile is unavailable. Build the spline_ops extension first.") from error
    return spline_compile


def _contiguous(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def _require_fused_current_swiglu(name, coeff_source, function, role, expected_op) -> None:
    """The production path must resolve to the fused dispatcher op."""
    if name != "spline_silu_compile" or coeff_source != "current":
        return
    resolved = getattr(function, "__spline_op__", None)
    if resolved != expected_op:
        raise RuntimeError(
            f"{role} requested the production fused path but resolved to "
            f"{getattr(function, '__name__', function)!r} ({resolved=!r}) instead of "
            f"{expected_op!r}. Check SPLINE_COMPILE_DISABLE_FUSED_SWIGLU and rebuild spline_ops.")


def _make_direct_spline_silu(degree: int, coeff_source: str):
    ops = load_spline_ops()
    cid = _coeff_source_id(coeff_source)

    def activation(t: torch.Tensor) -> torch.Tensor:
        t = _contiguous(t)
        if torch.is_grad_enabled() and t.requires_grad:
            return ops.swish_ag_variant(t, degree, cid)
        return ops.swish_fwd_variant(t, degree, cid)

    activation.__name__ = f"spline_silu_d{degree}_{coeff_source}_direct"
    return activation


def _make_direct_spline_silu_mul(degree: int, coeff_source: str):
    ops = load_spline_ops()
    cid = _coeff_source_id(coeff_source)
    if cid != 0:
        return None

    def activation_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
        gate, up = _contiguous(gate), _contiguous(up)
        if torch.is_grad_enabled() and (gate.requires_grad or up.requires_grad):
            return ops.swish_mul_ag_variant(gate, up, degree, cid)
        return ops.swish_mul_fwd_variant(gate, up, degree, cid)

    activation_mul.__name__ = f"spline_silu_mul_d{degree}_{coeff_source}_direct"
    return activation_mul


def _make_direct_spline_gelu(degree: int, coeff_source: str):
    """src/sfu_repro/activations.py:170-181"""
    ops = load_spline_ops()
    cid = _coeff_source_id(coeff_source)

    def activation(x: torch.Tensor) -> torch.Tensor:
        x = _contiguous(x)
        if torch.is_grad_enabled() and x.requires_grad:
            return ops.gelu_ag_variant(x, degree, cid)
        return ops.gelu_fwd_variant(x, degree, cid)

    activation.__name__ = f"spline_gelu_d{degree}_{coeff_source}_direct"
    return activation


def resolve_mlp_activation_impl(name: str, *, degree: int | None = None,
                                coeff_source: str = "current"):
    """Resolve a native or polynomial elementwise activation (reference :184-249)."""
    if name == "native_silu":
        return "native_silu", F.silu
    if name == "native_gelu":
        return "native_gelu", F.gelu
    if name == "spline_silu":
        d = 3 if degree is None else int(degree)
        return f"spline_silu[d{d},{coeff_source}]", _make_direct_spline_silu(d, coeff_source)
    if name == "spline_silu_compile":
        _ensure_coeff_source_allowed(coeff_source)
        sc = _spline_compile()
        d = 3 if degree is None else int(degree)
        activation = (sc.spline_silu if degree is None and coeff_source == "current"
                      else sc.make_spline_silu(degree=d, coeff_source=coeff_source))
        return f"spline_silu_compile[d{d},{coeff_source}]", activation
    if name == "spline_gelu":
        d = 5 if degree is None else int(degree)
        return f"spline_gelu[d{d},{coeff_source}]", _make_direct_spline_gelu(d, coeff_source)
    if name == "spline_gelu_compile":
        _ensure_coeff_source_allowed(coeff_source)
        sc = _spline_compile()
        d = 5 if degree is None else int(degree)
        activation = (sc.spline_gelu if degree is None and coeff_source == "current"
                      else sc.make_spline_gelu(degree=d, coeff_source=coeff_source))
        return f"spline_gelu_compile[d{d},{coeff_source}]", activation
    raise ValueError(f"unknown activation {name!r}; expected one of "
                     + ", ".join(PUBLIC_MLP_ACTIVATIONS))


def resolve_mlp_activation_mul_impl(name: str, *, degree: int | None = None,
                                    coeff_source: str = "current"):
    """Resolve ``activation(gate) * up``, preferring the fused kernel (reference :252-296)."""
    if name == "native_silu":
        return "native_silu_mul", lambda gate, up: F.silu(gate) * up
    if name == "spline_silu":
        d = 3 if degree is None else int(degree)
        activation_mul = _make_direct_spline_silu_mul(d, coeff_source)
        if activation_mul is not None:
            return f"spline_silu_mul[d{d},{coeff_source}]", activation_mul
    if name == "spline_silu_compile":
        _ensure_coeff_source_allowed(coeff_source)
        d = 3 if degree is None else int(degree)
        activation_mul = _spline_compile().make_spline_silu_mul(degree=d, coeff_source=coeff_source)
        _require_fused_current_swiglu(name, coeff_source, activation_mul,
                                      "SwiGLU activation-multiply",
                                      "spline_ops::swish_mul_variant_fwd")
        impl = ("spline_ops::swish_mul_variant_fwd" if coeff_source == "current"
                else "spline_silu_compile_mul_unfused")
        return f"{impl}[d{d},{coeff_source}]", activation_mul
    activation_name, activation = resolve_mlp_activation_impl(name, degree=degree,
                                                              coeff_source=coeff_source)
    return f"{activation_name}_mul", lambda gate, up: activation(gate) * up


def resolve_mlp_activation_packed_impl(name: str, *, degree: int | None = None,
                                       coeff_source: str = "current",
                                       backward_impl: str = "matched"):
    """Resolve a packed ``[..., 2 * hidden]`` SwiGLU (reference :299-346)."""
    if backward_impl not in ("matched", "native"):
        raise ValueError("backward_impl must be 'matched' or 'native'")
    if name == "native_silu":
        return "native_silu_packed", _spline_compile().make_native_silu_packed()
    if name == "spline_silu_compile":
        _ensure_coeff_source_allowed(coeff_source)
        d = 3 if degree is None else int(degree)
        activation = _spline_compile().make_spline_silu_packed(
            degree=d, coeff_source=coeff_source, backward_impl=backward_impl)
        expected = ("spline_ops::swish_mul_packed_variant_fwd" if backward_impl == "matched"
                    else "spline_ops::swish_mul_packed_native_bwd_fwd")
        _require_fused_current_swiglu(name, coeff_source, activation, "packed SwiGLU", expected)
        return f"{expected}[d{d},{coeff_source},{backward_impl}_bwd]", activation
    activation_name, activation_mul = resolve_mlp_activation_mul_impl(
        name, degree=degree, coeff_source=coeff_source)

    def activation_packed(packed: torch.Tensor) -> torch.Tensor:
        gate, up = packed.chunk(2, dim=-1)
        return activation_mul(gate, up)

    return f"{activation_name}_packed", activation_packed


__all__ = [
    "PUBLIC_MLP_ACTIVATIONS",
    "load_spline_ops",
    "resolve_mlp_activation_impl",
    "resolve_mlp_activation_mul_impl",
    "resolve_mlp_activation_packed_impl",
]
