"""The B1--B5 model converter for TorchTitan models on MI355X.

Same contract as the reference's ``src/sfu_repro/torchtitan/plugin.py:196-483``:
``SFUReproConverter(job_config, parallel_dims).convert(model)`` changes only the
operation the ``[sfu]`` case names --

* B1: every Llama ``FeedForward`` (w1, w2, w3) becomes a fused gate/up
  projection ``w_in = [w1; w3]`` followed by the packed SwiGLU (D3 polynomial,
  or native SiLU for the control) and ``w_out = w2``;
* B2 / B3 / B5: attention modules' ``inner_attention`` become
  :class:`sfu_repro.fa4.FA4AttentionWrapper` over this build's fused attention
  (softcap D4, B3 sigmoid attention at sequence length 4096, routed exp2);
* B4: routed ``GroupedExperts`` run gate / up / down per expert group with the
  fused SwiGLU between them.

TorchTitan's classes are matched when TorchTitan is importable; otherwise
modules are recognised by TorchTitan's class names and attributes, so a model
built the same way converts identically (the tests build such models).
"""

from __future__ import annotations

from typing import Any

import torch
from torch import nn

from sfu_repro.activations import resolve_mlp_activation_mul_impl, resolve_mlp_activation_packed_impl
from sfu_repro.fa4 import (
    FA4Config,
    b2_component_configs,
    b3_component_configs,
    b5_component_configs,
    patch_attention_modules,
    resolve_fa4_config,
)

try:  # the public TorchTitan checkout, when present
    from torchtitan.models.llama3.model.model import Attention as _TTAttention
    from torchtitan.models.llama3.model.model import FeedForward as _TTFeedForward
    from torchtitan.models.moe.moe import GroupedExperts as _TTGroupedExperts
except ImportError:  # pragma: no cover - TorchTitan is an optional dependency
    _TTAttention = _TTFeedForward = _TTGroupedExperts = None


def _is(module: nn.Module, tt_class, name: str, attrs: tuple[str, ...]) -> bool:
    if tt_class is not None:
        return isinstance(module, tt_class)
    return type(module).__name__ == name and all(hasattr(module, a) for a in attrs)


def is_llama_feed_forward(module: nn.Module) -> bool:
    return _is(module, _TTFeedForward, "FeedForward", ("w1", "w2", "w3"))


def is_llama_attention(module: nn.Module) -> bool:
    return _is(module, _TTAttention, "Attention", ("inner_attention",))


def is_grouped_experts(module: nn.Module) -> bool:
    return _is(module, _TTGroupedExperts, "GroupedExperts", ("w1", "w2", "w3"))


# ---- B1: fused gate/up projection + packed SwiGLU ----------------------------

_FUSED_CLASSES: dict[type, type] = {}


class ConfiguredFusedLlamaFeedForward(nn.Module):
    """Llama MLP with the fused gate/up projection and packed SwiGLU
    (src/sfu_repro/torchtitan/plugin.py:196-246)."""

    sfu_activation_packed: Any

    @classmethod
    @torch.no_grad()
    def from_unfused(cls, module: nn.Module, activation_packed: Any) -> nn.Module:
        dim, hidden = module.w2.weight.shape
        device, dtype = module.w1.weight.device, module.w1.weight.dtype
        w_in = nn.Linear(dim, 2 * hidden, bias=False, device=device, dtype=dtype)
        w_out = nn.Linear(hidden, dim, bias=False, device=device, dtype=dtype)
        if device.type != "meta":
            w_in.weight.copy_(torch.cat((module.w1.weight, module.w3.weight), dim=0))
            w_out.weight.copy_(module.w2.weight)
        del module.w1, module.w2, module.w3
        module.w_in, module.w_out = w_in, w_out
        module.sfu_activation_packed = activation_packed
        # a subclass of the module's own class, so isinstance checks and the
        # rest of its interface keep working
        if not isinstance(module, cls):
            base = type(module)
            if base not in _FUSED_CLASSES:
                _FUSED_CLASSES[base] = type(cls.__name__, (cls, base), {})
            module.__class__ = _FUSED_CLASSES[base]
        return module

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.w_out(self.sfu_activation_packed(self.w_in(x)))

    def init_weights(self, init_std: float) -> None:
        hidden = self.w_out.weight.shape[-1]
        nn.init.trunc_normal_(self.w_in.weight, mean=0.0, std=0.02)
        with torch.no_grad():
            self.w_in.weight[hidden:].mul_(init_std / 0.02)
        nn.init.trunc_normal_(self.w_out.weight, mean=0.0, std=init_std)


def _patch_llama_mlp(model: nn.Module, variant: str) -> int:
    impl = "native_silu" if variant == "native" else "spline_silu_compile"
    _, activation_packed = resolve_mlp_activation_packed_impl(impl, degree=3, coeff_source="current",
                                                              backward_impl="matched")
    patched = 0
    for module in list(model.modules()):
        if is_llama_feed_forward(module):
            ConfiguredFusedLlamaFeedForward.from_unfused(module, activation_packed)
            patched += 1
    return patched


# ---- B3 initialisation of the wrapper's q/k norms -------------------------------


def _install_fa4_initializers(model: nn.Module) -> int:
    """Attention modules whose ``init_weights`` also resets the RMSNorms the
    B3 wrapper adds (src/sfu_repro/torchtitan/plugin.py:272-292)."""
    patched = 0
    for module in model.modules():
        if not is_llama_attention(module) or not hasattr(module.inner_attention, "config"):
            continue
        base_init = getattr(module, "init_weights", None)

        def init_weights(init_std: float, *, module=module, base_init=base_init) -> None:
            if base_init is not None:
                base_init(init_std)
            for norm in (getattr(module.inner_attention, "q_norm", None),
                         getattr(module.inner_attention, "k_norm", None)):
                if norm is not None:
                    norm.reset_parameters()

        if not getattr(module, "_sfu_init_installed", False):
            module.init_weights = init_weights
            module._sfu_init_installed = True
        patched += 1
    return patched


# ---- B4: grouped experts ---------------------------------------------------------


def run_grouped_experts_polynomial(w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor, x: torch.Tensor,
                                   num_tokens_per_expert: torch.Tensor, activation_mul: Any) -> torch.Tensor:
    """Tokens sorted by expert: per expert group, gate = x w1^T, up = x w3^T,
    out = act_mul(gate, up) w2^T in BF16 (src/sfu_repro/torchtitan/plugin.py:295-312)."""
    counts = [int(c) for c in num_tokens_per_expert.tolist()]
    outs, start = [], 0
    xb = x.bfloat16()
    for e, n in enumerate(counts):
        if n == 0:
            continue
        xe = xb[start:start + n]
        gate = xe @ w1[e].bfloat16().transpose(-2, -1)
        up = xe @ w3[e].bfloat16().transpose(-2, -1)
        outs.append(activation_mul(gate, up) @ w2[e].bfloat16().transpose(-2, -1))
        start += n
    out = torch.cat(outs, dim=0) if outs else xb.new_zeros((0, w2.shape[1]))
    if start < x.shape[0]:  # padding rows past the counted tokens
        out = torch.cat((out, out.new_zeros((x.shape[0] - start, out.shape[1]))), dim=0)
    return out.type_as(x)


def _patch_grouped_experts(model: nn.Module, variant: str) -> int:
    impl = "native_silu" if variant == "native" else "spline_silu_compile"
    _, activation_mul = resolve_mlp_activation_mul_impl(impl, degree=3, coeff_source="current")
    patched = 0
    for module in model.modules():
        if not is_grouped_experts(module):
            continue

        def forward(x: torch.Tensor, num_tokens_per_expert: torch.Tensor, *, module=module) -> torch.Tensor:
            w1, w2, w3 = module.w1, module.w2, module.w3
            if hasattr(w1, "to_local"):  # DTensor shards: this rank's experts
                w1, w2, w3 = w1.to_local(), w2.to_local(), w3.to_local()
            return run_grouped_experts_polynomial(w1, w2, w3, x, num_tokens_per_expert, module.sfu_activation_mul)

        module.sfu_activation_mul = activation_mul
        module.forward = forward
        patched += 1
    return patched


def _attention_config(case: str, variant: str) -> FA4Config | None:
    if case == "b1":
        return FA4Config(mode="softmax")
    if case == "b2":
        return b2_component_configs()[variant]
    if case == "b3":
        return b3_component_configs(sequence_length=4096)[variant]
    if case == "b5":
        return b5_component_configs()[variant]
    return None


class SFUReproConverter:
    """Apply one B1--B5 intervention (src/sfu_repro/torchtitan/plugin.py:375-483);
    the checks on the job config and the patch counts are the reference's."""

    def __init__(self, job_config: Any, parallel_dims: Any):
        self.job_config = job_config
        self.parallel_dims = parallel_dims
        self.case = str(job_config.sfu.case).lower()
        self.variant = str(job_config.sfu.variant).lower()
        self.strict = bool(job_config.sfu.strict)
        if self.case not in {"b1", "b2", "b3", "b4", "b5"}:
            raise ValueError(f"unknown SFU case {self.case!r}")
        allowed = set(b5_component_configs()) if self.case == "b5" else {"native", "polynomial"}
        if self.variant not in allowed:
            raise ValueError(f"unknown SFU variant {self.variant!r}")
        expected_model = "sfu_deepseek_v3" if self.case == "b4" else "sfu_llama3"
        if self.strict and job_config.model.name != expected_model:
            raise ValueError(f"{self.case.upper()} requires model.name={expected_model!r}, "
                             f"got {job_config.model.name!r}")
        seq_len = int(job_config.training.seq_len)
        if self.case == "b3" and seq_len != 4096:
            raise ValueError("B3's direct D3/D4 fit requires training.seq_len=4096")
        if self.case == "b5" and seq_len != 4096:
            raise ValueError("B5's routed-exp2 probe requires training.seq_len=4096")
        if self.case == "b5" and bool(job_config.compile.enable):
            raise ValueError("B5's public model probe requires compile.enable=false")
        if self.case == "b5" and self.strict:
            shape = (int(job_config.training.local_batch_size), int(job_config.training.global_batch_size),
                     int(job_config.training.steps))
            if shape != (1, 1, 80):
                raise ValueError(f"B5's public model probe requires local/global batch 1 and 80 steps, got {shape}")
        if self.case == "b1" and getattr(parallel_dims, "tp", 1) != 1:
            raise ValueError("B1's fused gate/up projection requires tensor_parallel_degree=1")

    def convert(self, model: nn.Module) -> dict:
        patched_attention = patched_activation = 0
        config = _attention_config(self.case, self.variant)
        if config is not None:
            incompatible = sorted({str(getattr(m, "attn_type", "unknown")) for m in model.modules()
                                   if is_llama_attention(m) and getattr(m, "attn_type", None) != "sdpa"})
            if incompatible:
                raise ValueError(f"{self.case.upper()} requires TorchTitan SDPA attention before the FA4 "
                                 f"adapter; observed {incompatible}")
            resolved = resolve_fa4_config(config, sequence_length=int(self.job_config.training.seq_len))
            patched_attention = patch_attention_modules(model, resolved)
            initialized = _install_fa4_initializers(model)
            if initialized != patched_attention:
                raise RuntimeError("FA4 patch count and initialization-hook count disagree: "
                                   f"{patched_attention} != {initialized}")
        if self.case == "b1":
            patched_activation = _patch_llama_mlp(model, self.variant)
        elif self.case == "b4":
            patched_activation = _patch_grouped_experts(model, self.variant)
        expected = 29 if self.case == "b4" else int(getattr(model, "n_layers", 0))
        observed = patched_activation if self.case in {"b1", "b4"} else patched_attention
        if self.strict and observed != expected:
            raise RuntimeError(f"{self.case.upper()} {self.variant} expected {expected} patched modules, "
                               f"observed {observed}")
        return {"attention": patched_attention, "activation": patched_activation}

    def post_optimizer_hook(self, model) -> None:
        del model


def register() -> bool:
    """Register the converter with TorchTitan when it is installed."""
    try:
        from torchtitan.protocols.model_converter import register_model_converter
    except ImportError:
        return False
    register_model_converter(SFUReproConverter, "sfu_repro")
    return True


register()

__all__ = ["ConfiguredFusedLlamaFeedForward", "SFUReproConverter", "register", "run_grouped_experts_polynomial"]
