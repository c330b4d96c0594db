"""Model-level patching of Hugging Face models with the MI355X polynomial
kernels, and the prefill / decode timing of a patched model.

The library counterpart of the reference's ``scripts/benchmark_open_weights.py``
patch families (``:101-345`` variant grammar, ``:487-1436`` loaders,
collectors and patches, ``:1438-1648`` Gemma2 attention, ``:1712-1825``
timing): a variant string such as ``spline_silu_d3_current+fused_swiglu_d3_current``
selects which slots of a loaded model are replaced by ``spline_ops`` kernels:

* ``spline_silu_d{3..6}_{current,sollya}`` / ``spline_gelu_d…``: the ``act_fn``
  / ``activation`` / ``act`` attribute of every SiLU / GeLU module;
* ``fused_swiglu_d{3..6}_{current,sollya}``: dense MLPs (``gate_proj`` /
  ``up_proj`` / ``down_proj`` or ``w1`` / ``w2`` / ``w3``) run
  ``swish_mul_fwd_variant``; packed MoE experts (``_apply_gate`` of the
  Transformers experts classes) run ``swish_mul_packed_fwd_variant``;
* ``spline_router_sigmoid_d{3..6}_{current,sollya}``: the sigmoid of GLM /
  Kimi MoE routers;
* ``gemma_tanh_current``: Gemma2's eager attention softcap through the tanh
  kernel; ``gemma_fa4_tanh_native`` / ``gemma_fa4_tanh_d4_current``: Gemma2
  attention through this build's fused attention with the hardware or D4
  softcap (head_dim 128, unpadded batches, sequence within the sliding window).

GPT-OSS gates use the fused SwiGLU on ``alpha * gate`` (the reference's
``apply_gptoss_gate_patch``); the MXFP4 Triton path of GPT-OSS is not built
(no Triton here) and raises when a model carries it.

Models come from ``transformers`` configs with random weights (no checkpoint
download is needed or possible); the timing functions are the reference's
protocol (CUDA events around ``model(...)`` calls).
"""

from __future__ import annotations

import argparse
import json
import re
from dataclasses import asdict, dataclass, field
from types import MethodType
from typing import Any, Callable, NamedTuple

import torch

SILU_RE = re.compile(r"^spline_silu_d(?P<degree>[0-9]+)_(?P<source>current|sollya)$")
GELU_RE = re.compile(r"^spline_gelu_d(?P<degree>[0-9]+)_(?P<source>current|sollya)$")
FUSED_SWIGLU_RE = re.compile(r"^fused_swiglu_d(?P<degree>[0-9]+)_(?P<source>current|sollya)$")
GEMMA_TANH_RE = re.compile(r"^gemma_tanh_(?P<source>current)$")
GEMMA_FA4_TANH_RE = re.compile(
    r"^gemma_fa4_tanh_(?:(?P<native>native)|d(?P<degree>[0-9]+)_(?P<source>current|sollya))$")
ROUTER_SIGMOID_RE = re.compile(r"^spline_router_sigmoid_d(?P<degree>[0-9]+)_(?P<source>current|sollya)$")
SOURCE_IDS = {"current": 0, "sollya": 1}


@dataclass(frozen=True)
class VariantSpec:
    """One patch configuration (scripts/benchmark_open_weights.py:101-115)."""

    name: str
    silu_degree: int | None = None
    silu_source: str = "current"
    gelu_degree: int | None = None
    gelu_source: str = "current"
    dense_swiglu_degree: int | None = None
    dense_swiglu_source: str = "current"
    gemma_tanh_source: str | None = None
    gemma_fa4_tanh_backend: str | None = None
    gemma_fa4_tanh_degree: int | None = None
    gemma_fa4_tanh_source: str = "current"
    router_sigmoid_degree: int | None = None
    router_sigmoid_source: str = "current"


@dataclass
class Result:
    model: str
    variant: str
    dtype: str
    device: str
    batch_size: int
    seq_len: int
    patched_silu_modules: int = 0
    patched_router_sigmoid_modules: int = 0
    patched_gemma_softcap: bool = False
    prefill_ms: float | None = None
    prefill_tokens_per_s: float | None = None
    prefill_repetition_ms: list[float] = field(default_factory=list)
    decode_ms_per_token: float | None = None
    decode_tokens_per_s: float | None = None
    decode_repetition_ms: list[float] = field(default_factory=list)
    error: str | None = None
    notes: list[str] = field(default_factory=list)


def parse_variant(raw: str) -> VariantSpec:
    """Parse ``native`` or ``part+part+...`` (same grammar and errors as
    scripts/benchmark_open_weights.py:220-299)."""
    fields: dict[str, Any] = {}
    parts = tuple(part.strip() for part in raw.split("+"))
    if not parts or any(not part for part in parts):
        raise argparse.ArgumentTypeError(f"Invalid empty variant component in {raw!r}")
    if "native" in parts and len(parts) != 1:
        raise argparse.ArgumentTypeError("native cannot be combined with another variant")
    for part in parts:
        if part == "native":
            continue
        if m := SILU_RE.match(part):
            fields.update(silu_degree=int(m["degree"]), silu_source=m["source"])
        elif m := GELU_RE.match(part):
            fields.update(gelu_degree=int(m["degree"]), gelu_source=m["source"])
        elif m := FUSED_SWIGLU_RE.match(part):
            fields.update(dense_swiglu_degree=int(m["degree"]), dense_swiglu_source=m["source"])
        elif m := GEMMA_TANH_RE.match(part):
            fields.update(gemma_tanh_source=m["source"])
        elif m := GEMMA_FA4_TANH_RE.match(part):
            if m["native"]:
                fields.update(gemma_fa4_tanh_backend="native")
            else:
                fields.update(gemma_fa4_tanh_backend="device", gemma_fa4_tanh_degree=int(m["degree"]),
                              gemma_fa4_tanh_source=m["source"])
        elif m := ROUTER_SIGMOID_RE.match(part):
            fields.update(router_sigmoid_degree=int(m["degree"]), router_sigmoid_source=m["source"])
        else:
            raise argparse.ArgumentTypeError(
                f"Unknown variant part {part!r}. Expected native, "
                "spline_silu_d{3,4,5,6}_{current,sollya}, "
                "spline_gelu_d{3,4,5,6}_{current,sollya}, "
                "fused_swiglu_d{3,4,5}_{current,sollya}, "
                "spline_router_sigmoid_d{3,4,5,6}_{current,sollya}, "
                "gemma_tanh_current, gemma_fa4_tanh_native, or "
                "gemma_fa4_tanh_d{3,4,5,6}_{current,sollya}.")
    return VariantSpec(name=raw, **fields)


def required_interventions(spec: VariantSpec) -> frozenset[str]:
    """Patch families a variant asks for (scripts/benchmark_open_weights.py:302-319)."""
    required: set[str] = set()
    if any(d is not None for d in (spec.silu_degree, spec.gelu_degree, spec.dense_swiglu_degree)):
        required.add("activation")
    if spec.router_sigmoid_degree is not None:
        required.add("router")
    if spec.gemma_tanh_source is not None or spec.gemma_fa4_tanh_backend is not None:
        required.add("softcap")
    return frozenset(required)


def require_applied_interventions(spec: VariantSpec, result: Result) -> None:
    """Reject a variant that patched none of its intended slots
    (scripts/benchmark_open_weights.py:322-343)."""
    if spec.name == "native":
        return
    required = required_interventions(spec)
    if not required:
        raise RuntimeError(f"Variant {spec.name!r} does not request an intervention")
    missing = []
    if "activation" in required and result.patched_silu_modules <= 0:
        missing.append("activation/MLP")
    if "router" in required and result.patched_router_sigmoid_modules <= 0:
        missing.append("router sigmoid")
    if "softcap" in required and not result.patched_gemma_softcap:
        missing.append("attention softcap")
    if missing:
        raise RuntimeError(f"Variant {spec.name!r} patched zero intended " + ", ".join(missing) + " modules")


# ---------------------------------------------------------------------------
# kernels
# ---------------------------------------------------------------------------


def _ops():
    try:
        import spline_ops
    except (ImportError, OSError) as exc:
        raise RuntimeError(
            "Could not import spline_ops. Build it with `python fast-polynomial-transcendentals_amd/build.py` "
            "and put fast-polynomial-transcendentals_amd/python on PYTHONPATH.") from exc
    return spline_ops


def _check_degree(degree: int, what: str) -> None:
    if degree not in {3, 4, 5, 6}:
        raise ValueError(f"{what} only supports D3/D4/D5/D6, got D{degree}")


def load_spline_silu(degree: int, coeff_source: str) -> Callable[[torch.Tensor], torch.Tensor]:
    ops, source = _ops(), SOURCE_IDS[coeff_source]

    def activation(x: torch.Tensor) -> torch.Tensor:
        return ops.swish_fwd_variant(x, degree, source)

    activation.__name__ = f"spline_silu_d{degree}_{coeff_source}_direct"
    return activation


def load_spline_gelu(degree: int, coeff_source: str) -> Callable[[torch.Tensor], torch.Tensor]:
    ops, source = _ops(), SOURCE_IDS[coeff_source]

    def activation(x: torch.Tensor) -> torch.Tensor:
        return ops.gelu_fwd_variant(x, degree, source)

    activation.__name__ = f"spline_gelu_d{degree}_{coeff_source}_direct"
    return activation


def load_spline_tanh() -> Callable[[torch.Tensor], torch.Tensor]:
    ops = _ops()

    def activation(x: torch.Tensor) -> torch.Tensor:
        return ops.tanh_fwd(x.contiguous())

    activation.__name__ = "spline_tanh_direct"
    return activation


def load_spline_sigmoid(degree: int, coeff_source: str) -> Callable[[torch.Tensor], torch.Tensor]:
    """Router sigmoid: FP32 logits go through the BF16 program and come back
    in the input dtype (scripts/benchmark_open_weights.py:597-626)."""
    _check_degree(degree, "Router sigmoid polynomial")
    ops, source = _ops(), SOURCE_IDS[coeff_source]

    def activation(x: torch.Tensor) -> torch.Tensor:
        kernel_input = x if x.dtype in (torch.float16, torch.bfloat16) else x.to(torch.bfloat16)
        out = ops.sigmoid_fwd_variant(kernel_input.contiguous(), degree, source)
        return out if out.dtype == x.dtype else out.to(x.dtype)

    activation.__name__ = f"spline_router_sigmoid_d{degree}_{coeff_source}"
    return activation


def dense_swiglu_poly(gate: torch.Tensor, up: torch.Tensor, *, degree: int, coeff_source: str) -> torch.Tensor:
    _check_degree(degree, "Dense fused polynomial SwiGLU")
    if gate.numel() == 0:
        return torch.empty_like(up)
    if gate.dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError("Dense fused polynomial SwiGLU only supports fp16/bf16 odd/even kernels.")
    return _ops().swish_mul_fwd_variant(gate.contiguous(), up.contiguous(), degree, SOURCE_IDS[coeff_source])


def packed_swiglu_poly(packed_gate_up: torch.Tensor, *, degree: int, coeff_source: str) -> torch.Tensor:
    _check_degree(degree, "Packed fused polynomial SwiGLU")
    if packed_gate_up.numel() == 0:
        return packed_gate_up[..., : packed_gate_up.shape[-1] // 2].contiguous()
    if packed_gate_up.dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError("Packed fused polynomial SwiGLU only supports fp16/bf16 odd/even kernels.")
    return _ops().swish_mul_packed_fwd_variant(packed_gate_up.contiguous(), degree, SOURCE_IDS[coeff_source])


class FunctionActivation(torch.nn.Module):
    """A function as a module slot (keeps ``nn.Module`` attributes modules)."""

    def __init__(self, fn: Callable[[torch.Tensor], torch.Tensor]) -> None:
        super().__init__()
        self.fn = fn

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return x if x.numel() == 0 else self.fn(x.contiguous())


def make_contiguous_activation(fn: Callable[[torch.Tensor], torch.Tensor]) -> Callable[[torch.Tensor], torch.Tensor]:
    def activation(x: torch.Tensor) -> torch.Tensor:
        return x if x.numel() == 0 else fn(x.contiguous())

    activation.__name__ = getattr(fn, "__name__", "contiguous_activation")
    return activation


# ---------------------------------------------------------------------------
# slots
# ---------------------------------------------------------------------------


class ActivationSlot(NamedTuple):
    name: str
    module: torch.nn.Module
    attr: str
    fn: Callable[..., Any]


class MethodSlot(NamedTuple):
    """A module whose bound method ``attr`` (``forward``, ``_apply_gate``,
    ``route_tokens_to_experts``) is replaced."""

    name: str
    module: torch.nn.Module
    attr: str
    fn: Callable[..., Any]


def _names(module, fn, attrs, fn_words):
    config = getattr(module, "config", None)
    for attr in attrs:
        name = getattr(config, attr, None)
        if isinstance(name, str) and fn_words(name.lower()):
            return True
    for name in (fn.__class__.__name__, getattr(fn, "__name__", "")):
        if isinstance(name, str) and fn_words(name.lower()):
            return True
    return False


def looks_like_silu_module(module: torch.nn.Module, fn: Any) -> bool:
    """scripts/benchmark_open_weights.py:649-664 (config hidden_act, the
    function's class or name)."""
    if isinstance(fn, torch.nn.SiLU):
        return True
    return _names(module, fn, ("hidden_act", "hidden_activation"), lambda n: n in {"silu", "swish", "siluactivation"})


def looks_like_gelu_module(module: torch.nn.Module, fn: Any) -> bool:
    if isinstance(fn, torch.nn.GELU):
        return True
    return _names(module, fn, ("hidden_act", "hidden_activation", "activation_function"), lambda n: "gelu" in n)


def _act_slots(model, looks_like):
    slots = []
    for name, module in model.named_modules():
        for attr in ("act_fn", "activation", "act"):
            fn = getattr(module, attr, None)
            if fn is not None and looks_like(module, fn):
                slots.append(ActivationSlot(name, module, attr, fn))
    return slots


def collect_silu_act_fns(model: torch.nn.Module) -> list[ActivationSlot]:
    return _act_slots(model, looks_like_silu_module)


def collect_gelu_act_fns(model: torch.nn.Module) -> list[ActivationSlot]:
    return _act_slots(model, looks_like_gelu_module)


def collect_dense_swiglu_fns(model: torch.nn.Module) -> list[MethodSlot]:
    """Dense MLPs with Llama (gate/up/down_proj) or Phi (w1/w2/w3) names and
    a SiLU act_fn (scripts/benchmark_open_weights.py:714-726)."""
    slots = []
    for name, module in model.named_modules():
        llama = all(hasattr(module, a) for a in ("gate_proj", "up_proj", "down_proj"))
        phi = all(hasattr(module, a) for a in ("w1", "w2", "w3"))
        fn = getattr(module, "act_fn", None)
        if (llama or phi) and fn is not None and looks_like_silu_module(module, fn):
            slots.append(MethodSlot(name, module, "forward", module.forward))
    return slots


def collect_packed_experts_gate_fns(model: torch.nn.Module) -> list[MethodSlot]:
    """Transformers experts classes with a concatenated [gate; up] projection
    and an ``_apply_gate`` hook (scripts/benchmark_open_weights.py:772-796);
    the hook runs under the ``batched_mm`` / ``grouped_mm`` experts
    implementations."""
    slots = []
    for name, module in model.named_modules():
        if not all(hasattr(module, a) for a in ("_apply_gate", "act_fn", "gate_up_proj", "down_proj")):
            continue
        if not getattr(module, "has_gate", False) or not getattr(module, "is_concatenated", False):
            continue
        if looks_like_silu_module(module, module.act_fn):
            slots.append(MethodSlot(name, module, "_apply_gate", module._apply_gate))
    return slots


def collect_gptoss_gate_fns(model: torch.nn.Module) -> list[MethodSlot]:
    """GPT-OSS experts (interleaved gate/up with alpha and limit)."""
    slots = []
    for name, module in model.named_modules():
        fn = getattr(module, "_apply_gate", None)
        if fn is None or not all(hasattr(module, a) for a in ("alpha", "limit")):
            continue
        if "gptoss" in module.__class__.__name__.lower():
            slots.append(MethodSlot(name, module, "_apply_gate", fn))
    return slots


def collect_mxfp4_swiglu_fns(model: torch.nn.Module) -> list[MethodSlot]:
    return [MethodSlot(name, module, "forward", module.forward) for name, module in model.named_modules()
            if module.__class__.__name__ == "Mxfp4GptOssExperts"]


def collect_sigmoid_router_fns(model: torch.nn.Module) -> list[MethodSlot]:
    """Sigmoid MoE routers: GLM-4 MoE-lite (``route_tokens_to_experts`` of the
    MoE block in older Transformers, the router's ``forward`` in current
    ones) and Kimi's remote-code gate (scripts/benchmark_open_weights.py:899-920)."""
    slots = []
    for name, module in model.named_modules():
        cls = module.__class__.__name__
        if cls == "Glm4MoeLiteMoE" and hasattr(module, "route_tokens_to_experts"):
            slots.append(MethodSlot(name, module, "route_tokens_to_experts", module.route_tokens_to_experts))
        elif cls in ("Glm4MoeLiteTopkRouter", "KimiMoEGate"):
            slots.append(MethodSlot(name, module, "forward", module.forward))
    return slots


# ---------------------------------------------------------------------------
# patches (each returns how many slots it patched; a spec without the family
# restores the originals)
# ---------------------------------------------------------------------------


def _restore(slots) -> None:
    for slot in slots:
        setattr(slot.module, slot.attr, slot.fn)


def _apply_activation(slots: list[ActivationSlot], degree, source, loader) -> int:
    if degree is None:
        _restore(slots)
        return 0
    activation = make_contiguous_activation(loader(degree, source))
    for slot in slots:
        replacement = FunctionActivation(activation) if isinstance(slot.fn, torch.nn.Module) else activation
        setattr(slot.module, slot.attr, replacement)
    return len(slots)


def apply_silu_patch(slots: list[ActivationSlot], spec: VariantSpec) -> int:
    return _apply_activation(slots, spec.silu_degree, spec.silu_source, load_spline_silu)


def apply_gelu_patch(slots: list[ActivationSlot], spec: VariantSpec) -> int:
    return _apply_activation(slots, spec.gelu_degree, spec.gelu_source, load_spline_gelu)


def apply_dense_swiglu_patch(slots: list[MethodSlot], spec: VariantSpec) -> int:
    """MLP forward = down(SwiGLU(gate(x), up(x))) with the fused kernel
    (scripts/benchmark_open_weights.py:1118-1157)."""
    if spec.dense_swiglu_degree is None:
        _restore(slots)
        return 0
    degree, source = spec.dense_swiglu_degree, spec.dense_swiglu_source
    for slot in slots:
        def forward(self, x, *, degree=degree, source=source):
            if hasattr(self, "gate_proj"):
                return self.down_proj(dense_swiglu_poly(self.gate_proj(x), self.up_proj(x), degree=degree,
                                                        coeff_source=source))
            return self.w2(dense_swiglu_poly(self.w1(x), self.w3(x), degree=degree, coeff_source=source))

        slot.module.forward = MethodType(forward, slot.module)
    return len(slots)


def apply_packed_experts_gate_patch(slots: list[MethodSlot], spec: VariantSpec) -> int:
    """``_apply_gate(gate_up)`` = packed SwiGLU kernel on [gate; up]
    (scripts/benchmark_open_weights.py:1293-1322)."""
    if spec.dense_swiglu_degree is None:
        _restore(slots)
        return 0
    degree, source = spec.dense_swiglu_degree, spec.dense_swiglu_source
    for slot in slots:
        def apply_gate(self, packed_gate_up, *, degree=degree, source=source):
            return packed_swiglu_poly(packed_gate_up, degree=degree, coeff_source=source)

        slot.module._apply_gate = MethodType(apply_gate, slot.module)
    return len(slots)


def apply_gptoss_gate_patch(slots: list[MethodSlot], spec: VariantSpec) -> int:
    """GPT-OSS: glu = gate * sigmoid(alpha * gate), out = (up + 1) * glu, via
    swish(alpha * gate) * (up + 1) / alpha (scripts/benchmark_open_weights.py:1325-1351)."""
    if spec.silu_degree is None:
        _restore(slots)
        return 0
    for slot in slots:
        module = slot.module

        def apply_gate(gate_up, *, module=module, degree=spec.silu_degree, source=spec.silu_source):
            gate, up = gate_up[..., ::2], gate_up[..., 1::2]
            gate = gate.clamp(min=None, max=module.limit)
            up = up.clamp(min=-module.limit, max=module.limit)
            return dense_swiglu_poly(gate * module.alpha, up + 1, degree=degree, coeff_source=source) / module.alpha

        module._apply_gate = apply_gate
    return len(slots)


def apply_mxfp4_swiglu_patch(slots: list[MethodSlot], spec: VariantSpec) -> int:
    if spec.silu_degree is None or not slots:
        _restore(slots)
        return 0
    raise NotImplementedError("GPT-OSS MXFP4 experts run a Triton matmul_ogs kernel; the fused polynomial "
                              "activation for it is not built here")


def _grouped_topk(scores, bias, n_group, topk_group, top_k, fill):
    """Group-limited top-k of DeepSeek-V3-style routers."""
    tokens, experts = scores.shape
    choice = scores + bias
    group_scores = choice.view(tokens, n_group, experts // n_group).topk(2, dim=-1)[0].sum(dim=-1)
    group_idx = torch.topk(group_scores, k=topk_group, dim=-1, sorted=False)[1]
    group_mask = torch.zeros_like(group_scores).scatter_(1, group_idx, 1)
    score_mask = group_mask.unsqueeze(-1).expand(tokens, n_group, experts // n_group).reshape(tokens, experts)
    choice = choice.masked_fill(~score_mask.bool(), fill)
    return torch.topk(choice, k=top_k, dim=-1, sorted=False)[1]


def apply_sigmoid_router_patch(slots: list[MethodSlot], spec: VariantSpec) -> int:
    """Router scores = spline sigmoid of the FP32 logits, the routing math
    unchanged (scripts/benchmark_open_weights.py:923-1069)."""
    if spec.router_sigmoid_degree is None:
        _restore(slots)
        return 0
    sigmoid_fn = load_spline_sigmoid(spec.router_sigmoid_degree, spec.router_sigmoid_source)
    for slot in slots:
        module, cls = slot.module, slot.module.__class__.__name__
        if cls == "Glm4MoeLiteTopkRouter":
            def forward(self, hidden_states, *, sigmoid_fn=sigmoid_fn):
                hidden_states = hidden_states.view(-1, self.hidden_dim)
                logits = torch.nn.functional.linear(hidden_states.float(), self.weight.float())
                scores = sigmoid_fn(logits)
                idx = _grouped_topk(scores, self.e_score_correction_bias, self.num_group, self.topk_group,
                                    self.top_k, float("-inf"))
                weights = scores.gather(1, idx)
                if self.norm_topk_prob:
                    weights = weights / (weights.sum(dim=-1, keepdim=True) + 1e-20)
                return logits, weights * self.routed_scaling_factor, idx

            setattr(module, "forward", MethodType(forward, module))
        elif cls == "Glm4MoeLiteMoE":
            def route(self, router_logits, *, sigmoid_fn=sigmoid_fn):
                scores = sigmoid_fn(router_logits)
                idx = _grouped_topk(scores, self.gate.e_score_correction_bias, self.n_group, self.topk_group,
                                    self.top_k, float("-inf"))
                weights = scores.gather(1, idx)
                if self.norm_topk_prob:
                    weights = weights / (weights.sum(dim=-1, keepdim=True) + 1e-20)
                return idx, weights * self.routed_scaling_factor

            setattr(module, "route_tokens_to_experts", MethodType(route, module))
        elif cls == "KimiMoEGate":
            def forward(self, hidden_states, *, sigmoid_fn=sigmoid_fn):
                b, s, h = hidden_states.shape
                logits = torch.nn.functional.linear(hidden_states.view(-1, h).float(), self.weight.float())
                scores = sigmoid_fn(logits)
                # the checkpoint's remote code updates scores in place with the bias
                scores += self.e_score_correction_bias.unsqueeze(0)
                idx = _grouped_topk(scores, torch.zeros_like(self.e_score_correction_bias), self.num_expert_group,
                                    self.topk_group, self.top_k, 0.0)
                weights = scores.gather(1, idx)
                if self.top_k > 1 and self.moe_renormalize:
                    weights = weights / (weights.sum(dim=-1, keepdim=True) + 1e-20)
                return idx, weights * self.routed_scaling_factor

            setattr(module, "forward", MethodType(forward, module))
        else:
            raise RuntimeError(f"Unsupported sigmoid router class: {cls}")
    return len(slots)


# ---- Gemma2 attention ----------------------------------------------------------

_ORIGINAL_GEMMA_EAGER_ATTENTION: Callable[..., Any] | None = None


def restore_gemma_attention() -> None:
    global _ORIGINAL_GEMMA_EAGER_ATTENTION
    if _ORIGINAL_GEMMA_EAGER_ATTENTION is None:
        return
    from transformers.models.gemma2 import modeling_gemma2

    modeling_gemma2.eager_attention_forward = _ORIGINAL_GEMMA_EAGER_ATTENTION


def build_gemma_fused_attention_forward(spec: VariantSpec) -> Callable[..., tuple[torch.Tensor, None]]:
    """Gemma2 eager-attention replacement running this build's fused
    attention with the softcap in the tile loop (the reference routes it to
    FA4, scripts/benchmark_open_weights.py:1505-1587)."""
    from . import fa4_runtime

    backend = spec.gemma_fa4_tanh_backend
    if backend not in {"native", "device"}:
        raise ValueError(f"Unsupported Gemma FA4 tanh backend: {backend!r}")
    if backend == "device":
        fa4_runtime.create_softcap_scoremod_backend(30.0, degree=spec.gemma_fa4_tanh_degree, backend="device",
                                                    coeff_source=spec.gemma_fa4_tanh_source)

    def attention_forward(module, query, key, value, attention_mask, dropout=0.0, scaling=None, softcap=None,
                          **kwargs):
        if module.training or dropout:
            raise RuntimeError("Gemma fused-attention patch only supports inference")
        if kwargs.get("output_attentions", False):
            raise RuntimeError("Gemma fused-attention patch does not materialize attention weights")
        if softcap is None or softcap <= 0:
            raise RuntimeError(f"Gemma fused attention requires a positive softcap, got {softcap!r}")
        b, _, sq, d = query.shape
        sk = key.shape[-2]
        if sq != sk:
            raise NotImplementedError("the fused attention covers prefill (query length = key length)")
        if attention_mask is not None:
            allowed = attention_mask[:, 0, -1] == 0
            if not bool(allowed.all()):
                raise NotImplementedError("the fused attention takes unpadded batches")
        window = kwargs.get("sliding_window", getattr(module, "sliding_window", None))
        if window is not None and int(window) < sk:
            raise NotImplementedError(f"sequence {sk} exceeds the sliding window {window}")
        score_mod = None
        native_cap = float(softcap)
        if backend == "device":
            score_mod = fa4_runtime.create_softcap_scoremod_backend(
                float(softcap), degree=spec.gemma_fa4_tanh_degree, backend="device",
                coeff_source=spec.gemma_fa4_tanh_source)
            native_cap = 0.0
        out, _ = fa4_runtime.flash_attn_fwd(
            query.transpose(1, 2).contiguous(), key.transpose(1, 2).contiguous(),
            value.transpose(1, 2).contiguous(), softmax_scale=scaling if scaling is not None else d ** -0.5,
            causal=True, softcap=native_cap, score_mod=score_mod)
        return out, None

    return attention_forward


def apply_gemma_attention_patch(spec: VariantSpec) -> bool:
    """Gemma2 attention softcap: the eager path with the tanh kernel, or the
    fused attention (scripts/benchmark_open_weights.py:1590-1648)."""
    restore_gemma_attention()
    if spec.gemma_tanh_source is None and spec.gemma_fa4_tanh_backend is None:
        return False
    from transformers.models.gemma2 import modeling_gemma2

    global _ORIGINAL_GEMMA_EAGER_ATTENTION
    if _ORIGINAL_GEMMA_EAGER_ATTENTION is None:
        _ORIGINAL_GEMMA_EAGER_ATTENTION = modeling_gemma2.eager_attention_forward
    if spec.gemma_fa4_tanh_backend is not None:
        modeling_gemma2.eager_attention_forward = build_gemma_fused_attention_forward(spec)
        return True
    tanh_fn = load_spline_tanh()

    def poly_eager_attention_forward(module, query, key, value, attention_mask, dropout=0.0, scaling=None,
                                     softcap=None, **kwargs):
        if scaling is None:
            scaling = module.head_dim ** -0.5
        key_states = modeling_gemma2.repeat_kv(key, module.num_key_value_groups)
        value_states = modeling_gemma2.repeat_kv(value, module.num_key_value_groups)
        weights = torch.matmul(query, key_states.transpose(2, 3)) * scaling
        if softcap is not None:
            weights = tanh_fn(weights / softcap) * softcap
        if attention_mask is not None:
            weights = weights + attention_mask[:, :, :, : key_states.shape[-2]]
        weights = torch.nn.functional.softmax(weights, dim=-1, dtype=torch.float32).to(query.dtype)
        weights = torch.nn.functional.dropout(weights, p=dropout, training=module.training)
        out = torch.matmul(weights, value_states).transpose(1, 2).contiguous()
        return out, weights

    modeling_gemma2.eager_attention_forward = poly_eager_attention_forward
    return True


# ---------------------------------------------------------------------------
# whole-model wiring and timing
# ---------------------------------------------------------------------------


@dataclass
class ModelSlots:
    silu: list = field(default_factory=list)
    gelu: list = field(default_factory=list)
    dense_swiglu: list = field(default_factory=list)
    packed_experts_gate: list = field(default_factory=list)
    gptoss_gate: list = field(default_factory=list)
    mxfp4_swiglu: list = field(default_factory=list)
    sigmoid_router: list = field(default_factory=list)


def collect_slots(model: torch.nn.Module) -> ModelSlots:
    return ModelSlots(silu=collect_silu_act_fns(model), gelu=collect_gelu_act_fns(model),
                      dense_swiglu=collect_dense_swiglu_fns(model),
                      packed_experts_gate=collect_packed_experts_gate_fns(model),
                      gptoss_gate=collect_gptoss_gate_fns(model), mxfp4_swiglu=collect_mxfp4_swiglu_fns(model),
                      sigmoid_router=collect_sigmoid_router_fns(model))


def apply_variant(slots: ModelSlots, spec: VariantSpec, result: Result) -> Result:
    """Every patch family of ``spec`` in the reference's order
    (scripts/benchmark_open_weights.py:2106-2191), then the coverage check."""
    result.patched_silu_modules = apply_silu_patch(slots.silu, spec) + apply_gelu_patch(slots.gelu, spec)
    for count, note in (
        (apply_dense_swiglu_patch(slots.dense_swiglu, spec), "dense MLP forward -> swish_mul_fwd_variant"),
        (apply_packed_experts_gate_patch(slots.packed_experts_gate, spec),
         "MoE expert gates -> swish_mul_packed_fwd_variant"),
        (apply_gptoss_gate_patch(slots.gptoss_gate, spec), "GPT-OSS gated SwiGLU -> swish_mul_fwd_variant"),
        (apply_mxfp4_swiglu_patch(slots.mxfp4_swiglu, spec), "GPT-OSS MXFP4 experts"),
    ):
        result.patched_silu_modules += count
        if count:
            result.notes.append(f"patched {count}: {note}")
    result.patched_router_sigmoid_modules = apply_sigmoid_router_patch(slots.sigmoid_router, spec)
    result.patched_gemma_softcap = apply_gemma_attention_patch(spec)
    require_applied_interventions(spec, result)
    return result


def cuda_elapsed_ms(start: torch.cuda.Event, stop: torch.cuda.Event) -> float:
    stop.synchronize()
    return float(start.elapsed_time(stop))


def make_tokens(*, batch_size: int, seq_len: int, vocab_size: int, device, seed: int) -> torch.Tensor:
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randint(1, vocab_size, (batch_size, seq_len), device=device, generator=g)


@torch.inference_mode()
def benchmark_prefill(model, tokens, *, warmup: int, steps: int) -> tuple[float, float, list[float]]:
    """Mean ms and tokens/s of full forward passes (scripts/benchmark_open_weights.py:1712-1736)."""
    for _ in range(warmup):
        model(input_ids=tokens, use_cache=False)
    torch.cuda.synchronize()
    pairs = []
    for _ in range(steps):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        model(input_ids=tokens, use_cache=False)
        stop.record()
        pairs.append((start, stop))
    torch.cuda.synchronize()
    reps = [float(a.elapsed_time(b)) for a, b in pairs]
    mean = sum(reps) / len(reps)
    return mean, tokens.numel() * 1000.0 / mean, reps


@torch.inference_mode()
def benchmark_decode(model, tokens, *, warmup: int, repeats: int, decode_steps: int,
                     seed: int) -> tuple[float, float, list[float]]:
    """ms per decoded token after a prefill of ``tokens`` with the KV cache
    (scripts/benchmark_open_weights.py:1739-1825; the dynamic cache)."""
    batch = tokens.shape[0]
    vocab = int(model.get_input_embeddings().num_embeddings)
    g = torch.Generator(device=tokens.device).manual_seed(seed + 17)

    def loop(timed: bool) -> float:
        out = model(input_ids=tokens, use_cache=True)
        past = out.past_key_values
        nxt = torch.randint(1, vocab, (batch, 1), device=tokens.device, generator=g)
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(decode_steps):
            out = model(input_ids=nxt, past_key_values=past, use_cache=True)
            past = out.past_key_values
        stop.record()
        return cuda_elapsed_ms(start, stop) if timed else 0.0

    for _ in range(warmup):
        loop(False)
    reps = [loop(True) for _ in range(repeats)]
    ms = sum(reps) / (len(reps) * decode_steps)
    return ms, batch * 1000.0 / ms, reps


# Architectures the timing entry point builds from configs (random weights):
# the dims of the reference's open-weight models with fewer layers.
PRESETS: dict[str, dict[str, Any]] = {
    "llama3-8b-2l": dict(model_type="llama", hidden_size=4096, intermediate_size=14336, num_hidden_layers=2,
                         num_attention_heads=32, num_key_value_heads=8, vocab_size=128256, hidden_act="silu"),
    "gemma2-d128-2l": dict(model_type="gemma2", hidden_size=2304, intermediate_size=9216, num_hidden_layers=2,
                           num_attention_heads=8, num_key_value_heads=4, head_dim=128, vocab_size=256000,
                           hidden_activation="gelu_pytorch_tanh", attn_logit_softcapping=50.0,
                           final_logit_softcapping=30.0, sliding_window=4096),
    "glm4-moe-lite-2l": dict(model_type="glm4_moe_lite", hidden_size=2048, intermediate_size=10240,
                             moe_intermediate_size=1536, num_hidden_layers=2, num_attention_heads=16,
                             num_key_value_heads=16, n_routed_experts=64, num_experts_per_tok=4, n_group=1,
                             topk_group=1, first_k_dense_replace=1, vocab_size=151552),
}


def build_model(preset: str, *, dtype: torch.dtype, device, attn_implementation: str = "eager",
                experts_implementation: str | None = None, overrides: dict | None = None):
    """A randomly initialised model of a preset architecture."""
    import transformers

    kwargs = dict(PRESETS[preset])
    kwargs.update(overrides or {})
    model_type = kwargs.pop("model_type")
    config = transformers.AutoConfig.for_model(model_type, **kwargs)
    config._attn_implementation = attn_implementation
    if experts_implementation is not None:
        config._experts_implementation = experts_implementation
    with torch.device(device):
        model = transformers.AutoModelForCausalLM.from_config(config, dtype=dtype)
    return model.eval()


def run_variant(model, slots: ModelSlots, spec: VariantSpec, tokens, *, model_id: str, mode: str, warmup: int,
                steps: int, decode_steps: int, seed: int) -> Result:
    result = Result(model=model_id, variant=spec.name, dtype=str(next(model.parameters()).dtype),
                    device=str(tokens.device), batch_size=tokens.shape[0], seq_len=tokens.shape[1])
    apply_variant(slots, spec, result)
    if mode in ("prefill", "both"):
        result.prefill_ms, result.prefill_tokens_per_s, result.prefill_repetition_ms = benchmark_prefill(
            model, tokens, warmup=warmup, steps=steps)
    if mode in ("decode", "both"):
        result.decode_ms_per_token, result.decode_tokens_per_s, result.decode_repetition_ms = benchmark_decode(
            model, tokens, warmup=1, repeats=max(1, steps // 2), decode_steps=decode_steps, seed=seed)
    return result


def main(argv: list[str] | None = None) -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--preset", default="llama3-8b-2l", choices=sorted(PRESETS))
    p.add_argument("--variants", default="native,spline_silu_d3_current,fused_swiglu_d3_current")
    p.add_argument("--batch-size", type=int, default=1)
    p.add_argument("--seq-len", type=int, default=2048)
    p.add_argument("--mode", default="prefill", choices=("prefill", "decode", "both"))
    p.add_argument("--warmup", type=int, default=2)
    p.add_argument("--steps", type=int, default=5)
    p.add_argument("--decode-steps", type=int, default=32)
    p.add_argument("--seed", type=int, default=0)
    args = p.parse_args(argv)
    device = torch.device("cuda:0")
    model = build_model(args.preset, dtype=torch.bfloat16, device=device)
    slots = collect_slots(model)
    tokens = make_tokens(batch_size=args.batch_size, seq_len=args.seq_len,
                         vocab_size=int(model.get_input_embeddings().num_embeddings), device=device, seed=args.seed)
    for raw in args.variants.split(","):
        spec = parse_variant(raw.strip())
        try:
            res = run_variant(model, slots, spec, tokens, model_id=args.preset, mode=args.mode,
                              warmup=args.warmup, steps=args.steps, decode_steps=args.decode_steps, seed=args.seed)
        except (RuntimeError, NotImplementedError) as exc:
            res = Result(model=args.preset, variant=spec.name, dtype="bf16", device=str(device),
                         batch_size=args.batch_size, seq_len=args.seq_len, error=str(exc))
        print(json.dumps({k: v for k, v in asdict(res).items() if not k.endswith("repetition_ms")}), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
