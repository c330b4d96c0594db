"""torch.compile layer over the MI355X ``spline_ops`` extension.

Same public surface as the reference module
(``autonumerics_zero/spline_ops/spline_compile.py``):

* ``register_fake`` / ``register_autograd`` for the dispatcher ops that the
  extension registers in C++ (``torch.ops.spline_ops.*``, reference :34-238);
* opaque ``torch.library.custom_op`` wrappers ``spline_compile::*`` for the
  fixed-degree activations (reference :260-540);
* the drop-in callables ``spline_silu``, ``spline_sigmoid``, ``spline_tanh``,
  ``spline_gelu`` and the factories ``make_spline_silu``,
  ``make_spline_silu_mul``, ``make_spline_silu_packed``,
  ``make_native_silu_packed``, ``make_spline_gelu`` (reference :583-720).
"""

from __future__ import annotations

import os
from functools import lru_cache

import torch

import spline_ops as _spline_ops  # the HIP extension; import fails loudly if absent

_COEFF_SOURCE_TO_ID = {"current": 0, "sollya": 1}

_ops = torch.ops.spline_ops
_swish_variant_fwd_cpp = _ops.swish_variant_fwd.default
_swish_variant_bwd_cpp = _ops.swish_variant_bwd.default
_swish_mul_variant_fwd_cpp = _ops.swish_mul_variant_fwd.default
_swish_mul_variant_bwd_cpp = _ops.swish_mul_variant_bwd.default
_swish_mul_packed_variant_fwd_cpp = _ops.swish_mul_packed_variant_fwd.default
_swish_mul_packed_native_fwd_cpp = _ops.swish_mul_packed_native_fwd.default
_swish_mul_packed_native_bwd_fwd_cpp = _ops.swish_mul_packed_native_bwd_fwd.default
_swish_mul_packed_variant_bwd_cpp = _ops.swish_mul_packed_variant_bwd.default


# ---------------------------------------------------------------------------
# fake (meta) kernels of the C++ ops
# ---------------------------------------------------------------------------

def _half_last(packed: torch.Tensor) -> torch.Tensor:
    return packed.new_empty((*packed.shape[:-1], packed.shape[-1] // 2))


_FAKES = {
    "swish_variant_fwd": lambda x, degree, coeff_source_id: torch.empty_like(x),
    "swish_variant_bwd": lambda grad_out, x, degree, coeff_source_id: torch.empty_like(x),
    "swish_mul_variant_fwd": lambda gate, up, degree, coeff_source_id: torch.empty_like(up),
    "swish_mul_variant_bwd": lambda grad_out, gate, up, degree, coeff_source_id: [
        torch.empty_like(gate), torch.empty_like(up)],
    "swish_mul_packed_variant_fwd": lambda packed, degree, coeff_source_id: _half_last(packed),
    "swish_mul_packed_variant_bwd":
        lambda grad_out, packed, degree, coeff_source_id: torch.empty_like(packed),
    "swish_mul_packed_native_fwd": lambda packed, coeff_source_id: _half_last(packed),
    "swish_mul_packed_native_bwd_fwd": lambda packed, degree, coeff_source_id: _half_last(packed),
}
for _name, _fake in _FAKES.items():
    torch.library.register_fake(f"spline_ops::{_name}")(_fake)


# ---------------------------------------------------------------------------
# autograd of the C++ ops
# ---------------------------------------------------------------------------

def _save_x_and_args(ctx, inputs, output):
    del output
    x, degree, coeff_source_id = inputs
    ctx.save_for_backward(x)
    ctx.degree = degree
    ctx.coeff_source_id = coeff_source_id


def _swish_variant_backward(ctx, grad_out):
    (x,) = ctx.saved_tensors
    return _swish_variant_bwd_cpp(grad_out.contiguous(), x, ctx.degree, ctx.coeff_source_id), None, None


def _swish_mul_setup(ctx, inputs, output):
    del output
    gate, up, degree, coeff_source_id = inputs
    ctx.save_for_backward(gate, up)
    ctx.degree = degree
    ctx.coeff_source_id = coeff_source_id


def _swish_mul_backward(ctx, grad_out):
    gate, up = ctx.saved_tensors
    grad_gate, grad_up = _swish_mul_variant_bwd_cpp(
        grad_out.contiguous(), gate, up, ctx.degree, ctx.coeff_source_id)
    return grad_gate, grad_up, None, None


def _packed_backward(ctx, grad_out):
    (packed,) = ctx.saved_tensors
    grad = _swish_mul_packed_variant_bwd_cpp(
        grad_out.contiguous(), packed, ctx.degree, ctx.coeff_source_id)
    return (grad,) + (None,) * ctx.n_args


def _packed_setup(ctx, inputs, output):
    del output
    packed, degree, coeff_source_id = inputs
    ctx.save_for_backward(packed)
    ctx.degree, ctx.coeff_source_id, ctx.n_args = degree, coeff_source_id, 2


def _packed_native_bwd_setup(ctx, inputs, output):
    # Polynomial forward, native backward: the derivative is degree 0.
    del output
    packed, _degree, coeff_source_id = inputs
    ctx.save_for_backward(packed)
    ctx.degree, ctx.coeff_source_id, ctx.n_args = 0, coeff_source_id, 2


def _packed_native_setup(ctx, inputs, output):
    del output
    packed, coeff_source_id = inputs
    ctx.save_for_backward(packed)
    ctx.degree, ctx.coeff_source_id, ctx.n_args = 0, coeff_source_id, 1


torch.library.register_autograd("spline_ops::swish_variant_fwd", _swish_variant_backward,
                                setup_context=_save_x_and_args)
torch.library.register_autograd("spline_ops::swish_mul_variant_fwd", _swish_mul_backward,
                                setup_context=_swish_mul_setup)
torch.library.register_autograd("spline_ops::swish_mul_packed_variant_fwd", _packed_backward,
                                setup_context=_packed_setup)
torch.library.register_autograd("spline_ops::swish_mul_packed_native_fwd", _packed_backward,
                                setup_context=_packed_native_setup)
torch.library.register_autograd("spline_ops::swish_mul_packed_native_bwd_fwd", _packed_backward,
                                setup_context=_packed_native_bwd_setup)


# ---------------------------------------------------------------------------
# opaque custom ops for the fixed-degree activations
# ---------------------------------------------------------------------------

@torch.library.custom_op("spline_compile::swish_fwd", mutates_args=())
def _swish_fwd(x: torch.Tensor) -> torch.Tensor:
    return _spline_ops.swish_fwd(x)


@torch.library.custom_op("spline_compile::swish_bwd", mutates_args=())
def _swish_bwd(grad_out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    return _spline_ops.swish_bwd(grad_out, x)


@torch.library.custom_op("spline_compile::sigmoid_fwd", mutates_args=())
def _sigmoid_fwd(x: torch.Tensor) -> torch.Tensor:
    return _spline_ops.sigmoid_fwd(x)


@torch.library.custom_op("spline_compile::sigmoid_bwd_alg", mutates_args=())
def _sigmoid_bwd_alg(grad_out: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    return _spline_ops.sigmoid_bwd_alg(grad_out, y)


@torch.library.custom_op("spline_compile::tanh_fwd", mutates_args=())
def _tanh_fwd(x: torch.Tensor) -> torch.Tensor:
    return _spline_ops.tanh_fwd(x)


@torch.library.custom_op("spline_compile::tanh_bwd_alg", mutates_args=())
def _tanh_bwd_alg(grad_out: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    return _spline_ops.tanh_bwd_alg(grad_out, y)


@torch.library.custom_op("spline_compile::swish_variant_fwd", mutates_args=())
def _swish_variant_fwd(x: torch.Tensor, degree: int, coeff_source_id: int) -> torch.Tensor:
    return _spline_ops.swish_fwd_variant(x, degree, coeff_source_id)


@torch.library.custom_op("spline_compile::swish_variant_bwd", mutates_args=())
def _swish_variant_bwd(grad_out: torch.Tensor, x: torch.Tensor, degree: int,
                       coeff_source_id: int) -> torch.Tensor:
    return _spline_ops.swish_bwd_variant(grad_out, x, degree, coeff_source_id)


@torch.library.custom_op("spline_compile::swish_mul_variant_fwd", mutates_args=())
def _swish_mul_variant_fwd(gate: torch.Tensor, up: torch.Tensor, degree: int,
                           coeff_source_id: int) -> torch.Tensor:
    return _spline_ops.swish_mul_fwd_variant(gate, up, degree, coeff_source_id)


@torch.library.custom_op("spline_compile::swish_mul_variant_bwd", mutates_args=())
def _swish_mul_variant_bwd(grad_out: torch.Tensor, gate: torch.Tensor, up: torch.Tensor,
                           degree: int, coeff_source_id: int) -> tuple[torch.Tensor, torch.Tensor]:
    grad_gate, grad_up = _spline_ops.swish_mul_bwd_variant(grad_out, gate, up, degree,
                                                           coeff_source_id)
    return grad_gate, grad_up


@torch.library.custom_op("spline_compile::gelu_fwd", mutates_args=())
def _gelu_fwd(x: torch.Tensor) -> torch.Tensor:
    return _spline_ops.gelu_fwd(x)


@torch.library.custom_op("spline_compile::gelu_bwd", mutates_args=())
def _gelu_bwd(grad_out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    return _spline_ops.gelu_bwd(grad_out, x)


@torch.library.custom_op("spline_compile::gelu_variant_fwd", mutates_args=())
def _gelu_variant_fwd(x: torch.Tensor, degree: int, coeff_source_id: int) -> torch.Tensor:
    return _spline_ops.gelu_fwd_variant(x, degree, coeff_source_id)


@torch.library.custom_op("spline_compile::gelu_variant_bwd", mutates_args=())
def _gelu_variant_bwd(grad_out: torch.Tensor, x: torch.Tensor, degree: int,
                      coeff_source_id: int) -> torch.Tensor:
    return _spline_ops.gelu_bwd_variant(grad_out, x, degree, coeff_source_id)


for _op in (_swish_fwd, _sigmoid_fwd, _tanh_fwd, _gelu_fwd):
    _op.register_fake(lambda x: torch.empty_like(x))
for _op in (_swish_bwd, _sigmoid_bwd_alg, _tanh_bwd_alg, _gelu_bwd):
    _op.register_fake(lambda grad_out, x: torch.empty_like(x))
_gelu_variant_fwd.register_fake(lambda x, degree, coeff_source_id: torch.empty_like(x))
_gelu_variant_bwd.register_fake(
    lambda grad_out, x, degree, coeff_source_id: torch.empty_like(x))
_swish_variant_fwd.register_fake(lambda x, degree, coeff_source_id: torch.empty_like(x))
_swish_variant_bwd.register_fake(
    lambda grad_out, x, degree, coeff_source_id: torch.empty_like(x))
_swish_mul_variant_fwd.register_fake(
    lambda gate, up, degree, coeff_source_id: torch.empty_like(up))
_swish_mul_variant_bwd.register_fake(
    lambda grad_out, gate, up, degree, coeff_source_id: (torch.empty_like(gate),
                                                         torch.empty_like(up)))


def _setup_save_input(ctx, inputs, output):
    ctx.save_for_backward(inputs[0])


def _setup_save_output(ctx, inputs, output):
    ctx.save_for_backward(output)  # algebraic backward needs y, not x


_swish_fwd.register_autograd(
    lambda ctx, g: _swish_bwd(g.contiguous(), ctx.saved_tensors[0]),
    setup_context=_setup_save_input)
_sigmoid_fwd.register_autograd(
    lambda ctx, g: _sigmoid_bwd_alg(g.contiguous(), ctx.saved_tensors[0]),
    setup_context=_setup_save_output)
_tanh_fwd.register_autograd(
    lambda ctx, g: _tanh_bwd_alg(g.contiguous(), ctx.saved_tensors[0]),
    setup_context=_setup_save_output)
_swish_variant_fwd.register_autograd(
    lambda ctx, g: (_swish_variant_bwd(g.contiguous(), ctx.saved_tensors[0], ctx.degree,
                                       ctx.coeff_source_id), None, None),
    setup_context=_save_x_and_args)
_gelu_fwd.register_autograd(
    lambda ctx, g: _gelu_bwd(g.contiguous(), ctx.saved_tensors[0]),
    setup_context=_setup_save_input)
_gelu_variant_fwd.register_autograd(
    lambda ctx, g: (_gelu_variant_bwd(g.contiguous(), ctx.saved_tensors[0], ctx.degree,
                                      ctx.coeff_source_id), None, None),
    setup_context=_save_x_and_args)


def _swish_mul_custom_backward(ctx, grad_out):
    gate, up = ctx.saved_tensors
    grad_gate, grad_up = _swish_mul_variant_bwd(grad_out.contiguous(), gate, up, ctx.degree,
                                                ctx.coeff_source_id)
    return grad_gate, grad_up, None, None


_swish_mul_variant_fwd.register_autograd(_swish_mul_custom_backward, setup_context=_swish_mul_setup)


# ---------------------------------------------------------------------------
# public API
# ---------------------------------------------------------------------------

def _coeff_source_id(coeff_source: str) -> int:
    try:
        return _COEFF_SOURCE_TO_ID[coeff_source]
    except KeyError as exc:
        raise ValueError(
            f"Unknown coeff_source '{coeff_source}'. Expected one of: {tuple(_COEFF_SOURCE_TO_ID)}"
        ) from exc


def _env_flag(name: str, default: bool = False) -> bool:
    value = os.environ.get(name)
    if value is None:
        return default
    return value.lower() in ("1", "true", "yes", "on")


def spline_silu(x):
    """Polynomial SiLU (D3 forward, D4 derivative), torch.compile-compatible."""
    return _swish_fwd(x)


def spline_sigmoid(x):
    """Polynomial sigmoid (D3 forward, algebraic derivative), torch.compile-compatible."""
    return _sigmoid_fwd(x)


def spline_tanh(x):
    """Polynomial tanh (D3 forward, algebraic derivative), torch.compile-compatible."""
    return _tanh_fwd(x)


def spline_gelu(x):
    """Polynomial GeLU (D5 forward and derivative), torch.compile-compatible."""
    return _gelu_fwd(x)


@lru_cache(maxsize=None)
def make_spline_gelu(degree: int | None = None, coeff_source: str = "current"):
    resolved_degree = 5 if degree is None else int(degree)
    coeff_source_id = _coeff_source_id(coeff_source)
    if resolved_degree == 5 and coeff_source_id == 0:
        return spline_gelu

    def activation(x):
        return _gelu_variant_fwd(x, resolved_degree, coeff_source_id)

    activation.__name__ = f"spline_gelu_d{resolved_degree}_{coeff_source}"
    return activation


@lru_cache(maxsize=None)
def make_spline_silu(degree: int | None = None, coeff_source: str = "current"):
    resolved_degree = 3 if degree is None else int(degree)
    coeff_source_id = _coeff_source_id(coeff_source)

    def activation(x):
        return _swish_variant_fwd_cpp(x, resolved_degree, coeff_source_id)

    suffix = "_cpp" if (resolved_degree == 3 and coeff_source_id == 0) else ""
    activation.__name__ = f"spline_silu_d{resolved_degree}_{coeff_source}{suffix}"
    return activation


@lru_cache(maxsize=None)
def make_spline_silu_mul(degree: int | None = None, coeff_source: str = "current"):
    resolved_degree = 3 if degree is None else int(degree)
    coeff_source_id = _coeff_source_id(coeff_source)
    if coeff_source_id != 0 or _env_flag("SPLINE_COMPILE_DISABLE_FUSED_SWIGLU"):
        activation = make_spline_silu(resolved_degree, coeff_source)

        def activation_mul(gate, up):
            return activation(gate.contiguous()) * up.contiguous()

        activation_mul.__name__ = f"spline_silu_mul_d{resolved_degree}_{coeff_source}"
        return activation_mul

    def activation_mul(gate, up):
        return _swish_mul_variant_fwd_cpp(gate.contiguous(), up.contiguous(), resolved_degree,
                                          coeff_source_id)

    activation_mul.__name__ = f"spline_silu_mul_d{resolved_degree}_{coeff_source}_fused"
    activation_mul.__spline_op__ = "spline_ops::swish_mul_variant_fwd"
    return activation_mul


@lru_cache(maxsize=None)
def make_spline_silu_packed(degree: int | None = None, coeff_source: str = "current",
                            backward_impl: str = "matched"):
    resolved_degree = 3 if degree is None else int(degree)
    coeff_source_id = _coeff_source_id(coeff_source)
    if backward_impl not in ("matched", "native"):
        raise ValueError(
            f"Unknown packed SwiGLU backward_impl '{backward_impl}'. "
            "Expected one of: matched, native")
    if coeff_source_id != 0 or _env_flag("SPLINE_COMPILE_DISABLE_FUSED_SWIGLU"):
        activation_mul = make_spline_silu_mul(resolved_degree, coeff_source)

        def activation_packed(packed):
            gate, up = packed.chunk(2, dim=-1)
            poly_out = activation_mul(gate, up)
            if backward_impl == "matched":
                return poly_out
            native_out = torch.nn.functional.silu(gate) * up
            return poly_out.detach() + (native_out - native_out.detach())

        activation_packed.__name__ = f"spline_silu_packed_d{resolved_degree}_{coeff_source}"
        return activation_packed

    matched = backward_impl == "matched"
    packed_op = _swish_mul_packed_variant_fwd_cpp if matched else _swish_mul_packed_native_bwd_fwd_cpp

    def activation_packed(packed):
        return packed_op(packed.contiguous(), resolved_degree, coeff_source_id)

    activation_packed.__name__ = (
        f"spline_silu_packed_d{resolved_degree}_{coeff_source}_{backward_impl}_bwd_fused")
    activation_packed.__spline_op__ = (
        "spline_ops::swish_mul_packed_variant_fwd" if matched
        else "spline_ops::swish_mul_packed_native_bwd_fwd")
    return activation_packed


@lru_cache(maxsize=None)
def make_native_silu_packed():
    def activation_packed(packed):
        return _swish_mul_packed_native_fwd_cpp(packed.contiguous(), 0)

    activation_packed.__name__ = "native_silu_packed_fused"
    activation_packed.__spline_op__ = "spline_ops::swish_mul_packed_native_fwd"
    return activation_packed
