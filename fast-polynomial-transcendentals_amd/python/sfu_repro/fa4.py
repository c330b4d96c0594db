"""FA4 configuration layer and attention wrapper over the MI355X fused
attention kernels.

Same public surface as the reference's ``src/sfu_repro/fa4.py``: the
declarative :class:`FA4Config`, its validation (same rules and messages),
``resolve_fa4_config`` binding a config to a runtime mapping, the B2 / B3 /
B5 component configurations, the exp2 routing parser, the autograd function,
:class:`FA4AttentionWrapper` and ``patch_attention_modules``.  The runtime is
this build's own (:mod:`sfu_repro.fa4_runtime`, the HIP kernels of
``flash_attn.hip``): the reference's is a FlashAttention-4 checkout outside
its tree.  Configuration parsing and validation need no GPU; kernel calls
fail loudly when the HIP extension is missing.

Inputs to :class:`FA4AttentionWrapper` use ``(batch, heads, sequence, dim)``;
the runtime takes ``(batch, sequence, heads, dim)``.
"""

from __future__ import annotations

import logging
import os
from collections.abc import Callable, Mapping
from dataclasses import dataclass
from typing import Any

import torch
from torch import nn

LOGGER = logging.getLogger(__name__)

FLASH_SIGMOID_DIRECT_SEQUENCE_LENGTH = 4096

# Backend names FA4 accepts (src/sfu_repro/fa4.py:33-45).  Validation takes
# all of them, as the reference does; the runtime builds d3, d2_safe and
# pwl2 and names the others when asked for them.
SUPPORTED_EXP2_BACKENDS = (
    "d3",
    "pwl2",
    "pwl1_safe",
    "pwl1_safe_f16",
    "pwl2_safe",
    "pwl2_safe_f16",
    "pwl2_safe_bf16",
    "d2_safe",
    "d2_safe_noclamp",
    "d2_safe_f16",
    "d2_safe_bf16",
    "pwl2_f16",
)

_SOFTCAP_BACKENDS = ("native", "cute", "device")
_SOFTCAP_BACKWARD_MODES = ("analytical", "ste", "exact_1mt2", "native")
_COEFF_SOURCES = ("current", "sollya")
_SIGMOID_DEGREES = (2, 3, 4, 5, 6)


@dataclass(frozen=True)
class FA4Config:
    """Declarative attention configuration (fields and defaults of
    src/sfu_repro/fa4.py:51-76)."""

    mode: str = "softmax"
    exp2_emu_backend: str = "d3"
    exp2_emu_freq: int | None = None
    exp2_emu_freq_bwd: int = 0
    softcap: float = 30.0
    softcap_backend: str = "native"
    softcap_degree: int = 4
    softcap_coeff_source: str = "current"
    softcap_backward_mode: str = "analytical"
    sigmoid_variant: str = "poly"
    sigmoid_poly_backend: str = "cute"
    sigmoid_degree: int = 3
    sigmoid_degree_bwd: int | None = None
    sigmoid_coeff_source: str = "current"
    sigmoid_backward_mode: str = "algebraic"
    sigmoid_sfu_freq: int = 16
    sigmoid_sfu_res: int = 0
    sigmoid_sfu_freq_bwd: int | None = None
    sigmoid_sfu_res_bwd: int | None = None
    sigmoid_bias: float | None = None
    sigmoid_qk_norm: bool = True
    audit_coefficients: bool = True


@dataclass(frozen=True)
class ResolvedFA4Config:
    """A validated config bound to a runtime (src/sfu_repro/fa4.py:79-104)."""

    mode: str
    flash_attn_fwd: Callable[..., Any]
    flash_attn_bwd: Callable[..., Any]
    exp2_emu_backend: str = "d3"
    exp2_emu_freq: int | None = None
    exp2_emu_freq_bwd: int = 0
    softcap: float = 0.0
    score_mod: Callable[..., Any] | None = None
    score_mod_bwd: Callable[..., Any] | None = None
    sigmoid_attention: bool = False
    sigmoid_sfu_freq: int = 16
    sigmoid_sfu_res: int = 0
    sigmoid_sfu_freq_bwd: int | None = None
    sigmoid_sfu_res_bwd: int | None = None
    sigmoid_use_direct_bwd_poly: bool = False
    sigmoid_bias: float | None = None
    sigmoid_poly_backend: str = "cute"
    sigmoid_degree: int = 3
    sigmoid_degree_bwd: int | None = None
    sigmoid_coeff_source: str = "current"
    sigmoid_qk_norm: bool = True
    implementation_summary: str = ""


@dataclass(frozen=True)
class Exp2Variant:
    """One exp2 route of the softmax benchmark: four of every
    ``frequency`` exponents take ``backend`` (0 = none, None = automatic)."""

    name: str
    backend: str
    forward_frequency: int | None
    backward_frequency: int

    @staticmethod
    def _fraction(frequency: int) -> float:
        return 0.0 if frequency == 0 else min(1.0, 4.0 / frequency)

    @property
    def nominal_forward_polynomial_fraction(self) -> float | None:
        if self.forward_frequency is None:
            return None
        return self._fraction(self.forward_frequency)

    @property
    def nominal_backward_polynomial_fraction(self) -> float:
        return self._fraction(self.backward_frequency)

    @property
    def nominal_forward_pwl_fraction(self) -> float | None:
        """Older name of :attr:`nominal_forward_polynomial_fraction`."""
        return self.nominal_forward_polynomial_fraction

    @property
    def nominal_backward_pwl_fraction(self) -> float:
        """Older name of :attr:`nominal_backward_polynomial_fraction`."""
        return self.nominal_backward_polynomial_fraction


# name=backend:forward:backward (src/sfu_repro/fa4.py:140-154)
DEFAULT_EXP2_VARIANTS = ",".join(
    ["sfu=d3:0:0", "d3_auto=d3:auto:0"]
    + [f"d2_safe_{label}=d2_safe:{freq}:0"
       for label, freq in (("12p5", 32), ("16p7", 24), ("20", 20), ("25", 16), ("33p3", 12),
                           ("40", 10), ("50", 8), ("66p7", 6), ("100", 4))]
)


def _validate_exp2_route(frequency: int | None, label: str) -> int | None:
    if frequency is None:
        return None
    frequency = int(frequency)
    if frequency < 0 or (frequency != 0 and (frequency < 4 or frequency % 2)):
        raise ValueError(f"{label} frequency must be 0 or an even integer >= 4, got {frequency}")
    return frequency


def parse_exp2_frequency(value: str, *, allow_auto: bool) -> int | None:
    """One routing frequency: 'auto' (forward only), 0, or an even integer >= 4."""
    if allow_auto and value == "auto":
        return None
    try:
        frequency = int(value)
    except ValueError as error:
        allowed = "'auto', 0, or an even integer >= 4" if allow_auto else "0 or an even integer >= 4"
        raise ValueError(f"frequency must be {allowed}, got {value!r}") from error
    return _validate_exp2_route(frequency, "exp2")


def parse_exp2_variants(value: str) -> tuple[Exp2Variant, ...]:
    """Comma-separated ``name=backend:forward_frequency:backward_frequency``."""
    variants: list[Exp2Variant] = []
    for spec in (part.strip() for part in value.split(",")):
        if not spec:
            continue
        try:
            name, route = spec.split("=", maxsplit=1)
            backend, forward, backward = route.split(":")
        except ValueError as error:
            raise ValueError(
                f"variant must have name=backend:forward_frequency:backward_frequency syntax, got {spec!r}"
            ) from error
        name, backend = name.strip(), backend.strip()
        if not name:
            raise ValueError("variant name must not be empty")
        if backend not in SUPPORTED_EXP2_BACKENDS:
            raise ValueError(f"unsupported exp2 backend {backend!r}")
        variants.append(Exp2Variant(
            name=name, backend=backend,
            forward_frequency=parse_exp2_frequency(forward.strip(), allow_auto=True),
            backward_frequency=int(parse_exp2_frequency(backward.strip(), allow_auto=False))))
    if not variants:
        raise ValueError("at least one variant is required")
    if len({v.name for v in variants}) != len(variants):
        raise ValueError("variant names must be unique")
    return tuple(variants)


def _env_flag(name: str) -> bool:
    value = os.environ.get(name)
    return value is not None and value.lower() in ("1", "true", "yes", "on")


def _validate_sigmoid_sfu_route(frequency: int, residue_count: int, label: str) -> tuple[int, int]:
    frequency, residue_count = int(frequency), int(residue_count)
    if frequency <= 0:
        raise ValueError(f"{label} sigmoid_sfu_freq must be positive, got {frequency}")
    if residue_count < 0 or residue_count > frequency:
        raise ValueError(
            f"{label} sigmoid_sfu_res must lie in [0, sigmoid_sfu_freq], got {residue_count} for {frequency}")
    return frequency, residue_count


def _uses_sollya(config: FA4Config) -> bool:
    softcap = config.mode == "softcap" and config.softcap_coeff_source == "sollya"
    sigmoid = (config.mode == "sigmoid_attention" and config.sigmoid_variant == "poly"
               and config.sigmoid_coeff_source == "sollya")
    return softcap or sigmoid


def _is_device_current_poly(config: FA4Config, degree: int) -> bool:
    return (config.mode == "sigmoid_attention" and config.sigmoid_variant == "poly"
            and config.sigmoid_poly_backend == "device" and config.sigmoid_coeff_source == "current"
            and int(config.sigmoid_degree) == degree and config.sigmoid_bias is None)


def _uses_direct_flash_sigmoid(config: FA4Config) -> bool:
    """The B3 direct D3 program (src/sfu_repro/fa4.py:254-262)."""
    return _is_device_current_poly(config, 3)


def _uses_bias_aware_d2(config: FA4Config) -> bool:
    """The bias-aware FlashSigmoid D2 exp2 program (src/sfu_repro/fa4.py:391-398)."""
    return _is_device_current_poly(config, 2)


def _validate_softcap(config: FA4Config) -> None:
    if config.softcap_backend not in _SOFTCAP_BACKENDS:
        raise ValueError(f"unsupported softcap backend {config.softcap_backend!r}")
    if config.softcap_backward_mode not in _SOFTCAP_BACKWARD_MODES:
        raise ValueError(f"unsupported softcap backward mode {config.softcap_backward_mode!r}")
    if config.softcap_coeff_source not in _COEFF_SOURCES:
        raise ValueError(f"unsupported softcap coefficient source {config.softcap_coeff_source!r}")
    if config.softcap <= 0:
        raise ValueError("softcap must be positive")
    native = config.softcap_backend == "native"
    if native and config.softcap_backward_mode != "native":
        raise ValueError("native softcap requires softcap_backward_mode='native'")
    if not native and config.softcap_backward_mode == "native":
        raise ValueError("polynomial softcap cannot use softcap_backward_mode='native'")
    if config.softcap_coeff_source == "sollya" and config.softcap_backend != "device":
        raise ValueError("Sollya softcap fits require softcap_backend='device'")


def _validate_sigmoid(config: FA4Config, sequence_length: int | None) -> None:
    if config.sigmoid_variant not in ("poly", "sfu"):
        raise ValueError(f"unsupported sigmoid variant {config.sigmoid_variant!r}")
    if config.sigmoid_poly_backend not in ("cute", "device"):
        raise ValueError(f"unsupported sigmoid polynomial backend {config.sigmoid_poly_backend!r}")
    if config.sigmoid_backward_mode not in ("algebraic", "direct"):
        raise ValueError(f"unsupported sigmoid backward mode {config.sigmoid_backward_mode!r}")
    if config.sigmoid_coeff_source not in _COEFF_SOURCES:
        raise ValueError(f"unsupported sigmoid coefficient source {config.sigmoid_coeff_source!r}")
    if int(config.sigmoid_degree) not in _SIGMOID_DEGREES:
        raise ValueError("sigmoid_degree must be one of 2, 3, 4, 5, or 6")
    if config.sigmoid_degree_bwd is not None and int(config.sigmoid_degree_bwd) not in _SIGMOID_DEGREES:
        raise ValueError("sigmoid_degree_bwd must be one of 2, 3, 4, 5, or 6")
    poly = config.sigmoid_variant == "poly"
    if poly and config.sigmoid_poly_backend == "cute":
        raise ValueError("causal polynomial sigmoid attention requires sigmoid_poly_backend='device'")
    if poly and config.sigmoid_coeff_source == "sollya" and config.sigmoid_poly_backend != "device":
        raise ValueError("Sollya sigmoid fits require sigmoid_poly_backend='device'")

    fwd_freq, fwd_res = _validate_sigmoid_sfu_route(config.sigmoid_sfu_freq, config.sigmoid_sfu_res, "forward")
    bwd_freq = fwd_freq if config.sigmoid_sfu_freq_bwd is None else config.sigmoid_sfu_freq_bwd
    bwd_res = fwd_res if config.sigmoid_sfu_res_bwd is None else config.sigmoid_sfu_res_bwd
    bwd_freq, bwd_res = _validate_sigmoid_sfu_route(bwd_freq, bwd_res, "backward")
    if poly and (fwd_res != 0 or bwd_res != 0):
        raise ValueError("sigmoid_variant='poly' must route every forward/backward lane through the polynomial")
    if not poly and (fwd_res != fwd_freq or bwd_res != bwd_freq):
        raise ValueError("sigmoid_variant='sfu' must route every forward/backward lane through the SFU")
    if _uses_bias_aware_d2(config) and config.sigmoid_backward_mode != "algebraic":
        raise ValueError("bias-aware FlashSigmoid D2 requires sigmoid_backward_mode='algebraic'")
    if _uses_direct_flash_sigmoid(config):
        if sequence_length is None:
            raise ValueError("direct FlashSigmoid D3 requires an explicit sequence_length")
        if int(sequence_length) != FLASH_SIGMOID_DIRECT_SEQUENCE_LENGTH:
            raise ValueError(
                "direct FlashSigmoid D3/D4 is fitted for sequence length "
                f"{FLASH_SIGMOID_DIRECT_SEQUENCE_LENGTH}, got {sequence_length}")


def validate_fa4_config(config: FA4Config, *, sequence_length: int | None = None) -> FA4Config:
    """Validate a declarative config without touching the GPU
    (src/sfu_repro/fa4.py:265-416); returns the config."""
    if config.mode not in ("softmax", "softcap", "sigmoid_attention"):
        raise ValueError(f"unsupported FA4 mode {config.mode!r}")
    if config.exp2_emu_backend not in SUPPORTED_EXP2_BACKENDS:
        raise ValueError(f"unsupported exp2 backend {config.exp2_emu_backend!r}")
    _validate_exp2_route(config.exp2_emu_freq, "forward exp2")
    _validate_exp2_route(config.exp2_emu_freq_bwd, "backward exp2")
    if _uses_sollya(config) and not _env_flag("SFU_REPRO_ALLOW_SOLLYA_SWEEP"):
        raise ValueError(
            "Sollya coefficient sources are benchmark-only. Set "
            "SFU_REPRO_ALLOW_SOLLYA_SWEEP=1 for an explicit sweep.")
    if config.mode == "softcap":
        _validate_softcap(config)
    elif config.mode == "sigmoid_attention":
        _validate_sigmoid(config, sequence_length)
    return config


def _load_fa4_runtime() -> Mapping[str, Any]:
    """The kernels this configuration layer drives (the HIP fused attention)."""
    from . import fa4_runtime

    return fa4_runtime.runtime()


def _audit(config: FA4Config, runtime: Mapping[str, Any], degree_bwd: int) -> None:
    audited = list(runtime["run_polynomial_coefficient_audit"]())
    selections: list[tuple[str, int, str]] = []
    if config.mode == "softcap" and config.softcap_backend != "native":
        selections.append(("tanh_fwd", int(config.softcap_degree), config.softcap_coeff_source))
    if config.mode == "sigmoid_attention" and config.sigmoid_variant == "poly":
        d2 = _uses_bias_aware_d2(config)
        source = config.sigmoid_coeff_source
        selections.append(("flash_sigmoid_exp2" if d2 else "sigmoid_fwd", int(config.sigmoid_degree), source))
        if config.sigmoid_backward_mode == "direct":
            selections.append(("sigmoid_bwd", degree_bwd, source))
        elif degree_bwd != int(config.sigmoid_degree):
            family = "flash_sigmoid_exp2" if d2 and degree_bwd == 2 else "sigmoid_fwd"
            selections.append((family, degree_bwd, source))
    if selections:
        audited.extend(runtime["audit_polynomial_selection"](tuple(selections)))
    LOGGER.info("FA4 polynomial audit passed: %s", ", ".join(audited))


def resolve_fa4_config(config: FA4Config, *, sequence_length: int | None = None,
                       runtime: Mapping[str, Any] | None = None) -> ResolvedFA4Config:
    """Validate ``config`` and bind it to ``runtime`` (by default this
    build's HIP kernels), as src/sfu_repro/fa4.py:454-647."""
    validate_fa4_config(config, sequence_length=sequence_length)
    runtime = _load_fa4_runtime() if runtime is None else runtime
    degree_bwd = int(config.sigmoid_degree if config.sigmoid_degree_bwd is None else config.sigmoid_degree_bwd)
    if config.audit_coefficients:
        _audit(config, runtime, degree_bwd)
    kernels = {"flash_attn_fwd": runtime["flash_attn_fwd"], "flash_attn_bwd": runtime["flash_attn_bwd"]}

    if config.mode == "softmax":
        route = "automatic" if config.exp2_emu_freq is None else config.exp2_emu_freq
        return ResolvedFA4Config(
            mode="softmax", **kernels, exp2_emu_backend=config.exp2_emu_backend,
            exp2_emu_freq=config.exp2_emu_freq, exp2_emu_freq_bwd=config.exp2_emu_freq_bwd,
            sigmoid_qk_norm=False,
            implementation_summary=(f"FA4 softmax exp2 backend={config.exp2_emu_backend}, "
                                    f"forward_freq={route}, backward_freq={config.exp2_emu_freq_bwd}"))

    if config.mode == "softcap":
        if config.softcap_backend == "native":
            return ResolvedFA4Config(mode="softcap", **kernels, softcap=float(config.softcap),
                                     sigmoid_qk_norm=False, implementation_summary="FA4 native SFU tanh softcap")
        degree, source = int(config.softcap_degree), config.softcap_coeff_source
        if config.softcap_backend == "device":
            paths = [runtime["audit_attention_handwritten_fast_path"]("tanh_fwd", degree, source)]
            if config.softcap_backward_mode == "analytical":
                paths.append(runtime["audit_attention_handwritten_fast_path"]("tanh_grad_analytical", degree, source))
        else:
            paths = [f"CuTe tanh D{degree} {source}"]
        score_mod = runtime["create_softcap_scoremod_backend"](
            config.softcap, degree=config.softcap_degree, backend=config.softcap_backend, coeff_source=source)
        score_mod_bwd = runtime["create_softcap_scoremod_bwd_backend"](
            config.softcap, degree=config.softcap_degree, backend=config.softcap_backend,
            backward_mode=config.softcap_backward_mode, coeff_source=source)
        return ResolvedFA4Config(mode="softcap", **kernels, score_mod=score_mod, score_mod_bwd=score_mod_bwd,
                                 sigmoid_qk_norm=False, implementation_summary="; ".join(paths))

    fwd_freq, fwd_res = _validate_sigmoid_sfu_route(config.sigmoid_sfu_freq, config.sigmoid_sfu_res, "forward")
    paths: list[str] = []
    direct = _uses_direct_flash_sigmoid(config)
    if config.sigmoid_variant == "sfu":
        paths.append("FA4 native SFU sigmoid + algebraic sigmoid gradient")
    elif _uses_bias_aware_d2(config):
        paths.append("FA4 bias-aware D2 exp2 polynomial")
    elif config.sigmoid_poly_backend == "device":
        source = config.sigmoid_coeff_source
        audit_path = runtime["audit_attention_handwritten_fast_path"]
        paths.append(audit_path("flash_sigmoid_direct" if direct else "sigmoid_fwd", int(config.sigmoid_degree), source))
        if config.sigmoid_backward_mode == "direct":
            family = "flash_sigmoid_direct_with_grad" if direct and degree_bwd == 4 else "sigmoid_grad"
            paths.append(audit_path(family, degree_bwd, source))
    return ResolvedFA4Config(
        mode="sigmoid_attention", **kernels, sigmoid_attention=True, sigmoid_sfu_freq=fwd_freq,
        sigmoid_sfu_res=fwd_res, sigmoid_sfu_freq_bwd=config.sigmoid_sfu_freq_bwd,
        sigmoid_sfu_res_bwd=config.sigmoid_sfu_res_bwd,
        sigmoid_use_direct_bwd_poly=config.sigmoid_backward_mode == "direct",
        sigmoid_bias=config.sigmoid_bias, sigmoid_poly_backend=config.sigmoid_poly_backend,
        sigmoid_degree=int(config.sigmoid_degree),
        sigmoid_degree_bwd=degree_bwd if config.sigmoid_degree_bwd is not None else None,
        sigmoid_coeff_source=config.sigmoid_coeff_source, sigmoid_qk_norm=config.sigmoid_qk_norm,
        implementation_summary="; ".join(paths))


def b2_component_configs() -> dict[str, FA4Config]:
    """B2: native vs device D4 softcap 30 (src/sfu_repro/fa4.py:650-668)."""
    return {
        "native": FA4Config(mode="softcap", softcap=30.0, softcap_backend="native",
                            softcap_backward_mode="native"),
        "polynomial": FA4Config(mode="softcap", softcap=30.0, softcap_backend="device", softcap_degree=4,
                                softcap_coeff_source="current", softcap_backward_mode="analytical"),
    }


def b3_component_configs(*, sequence_length: int = FLASH_SIGMOID_DIRECT_SEQUENCE_LENGTH) -> dict[str, FA4Config]:
    """B3: SFU sigmoid attention vs the direct D3 / D4 programs, fitted for
    sequence length 4096 only (src/sfu_repro/fa4.py:671-709)."""
    if int(sequence_length) != FLASH_SIGMOID_DIRECT_SEQUENCE_LENGTH:
        raise ValueError(
            f"B3 direct D3/D4 requires sequence length {FLASH_SIGMOID_DIRECT_SEQUENCE_LENGTH}, got {sequence_length}")
    configs = {
        "native": FA4Config(mode="sigmoid_attention", sigmoid_variant="sfu", sigmoid_sfu_freq=16,
                            sigmoid_sfu_res=16, sigmoid_qk_norm=True),
        "polynomial": FA4Config(mode="sigmoid_attention", sigmoid_variant="poly", sigmoid_poly_backend="device",
                                sigmoid_degree=3, sigmoid_degree_bwd=4, sigmoid_coeff_source="current",
                                sigmoid_backward_mode="direct", sigmoid_sfu_freq=16, sigmoid_sfu_res=0,
                                sigmoid_qk_norm=True),
    }
    for config in configs.values():
        validate_fa4_config(config, sequence_length=sequence_length)
    return configs


def softmax_exp2_config(variant: Exp2Variant) -> FA4Config:
    """A validated softmax config for one exp2 benchmark variant."""
    return validate_fa4_config(FA4Config(mode="softmax", exp2_emu_backend=variant.backend,
                                         exp2_emu_freq=variant.forward_frequency,
                                         exp2_emu_freq_bwd=variant.backward_frequency))


def b5_component_configs() -> dict[str, FA4Config]:
    """B5: the retained routed-exp2 schedules (src/sfu_repro/fa4.py:722-752):
    all-SFU, and four of every 12 (forward) / 32 (backward) exponents
    through the named program."""
    variants = (Exp2Variant("native", "d3", 0, 0), Exp2Variant("pwl2_safe_f16", "pwl2_safe_f16", 12, 32),
                Exp2Variant("d2_safe", "d2_safe", 12, 32))
    return {v.name: softmax_exp2_config(v) for v in variants}


class _FA4Function(torch.autograd.Function):
    """Forward / backward through the runtime (argument order of
    src/sfu_repro/fa4.py:755-861)."""

    @staticmethod
    def forward(ctx, q, k, v, softmax_scale, causal, softcap, sigmoid_attention, sigmoid_sfu_freq,
                sigmoid_sfu_res, sigmoid_sfu_freq_bwd, sigmoid_sfu_res_bwd, sigmoid_use_direct_bwd_poly,
                sigmoid_bias, sigmoid_poly_backend, sigmoid_degree, sigmoid_degree_bwd, sigmoid_coeff_source,
                exp2_emu_backend, exp2_emu_freq, exp2_emu_freq_bwd, score_mod, score_mod_bwd, flash_attn_fwd,
                flash_attn_bwd):
        fused_softcap = softcap if score_mod is None else 0.0
        out, lse = flash_attn_fwd(
            q, k, v, softmax_scale=softmax_scale, causal=causal, softcap=fused_softcap, score_mod=score_mod,
            sigmoid_attention=sigmoid_attention, sigmoid_sfu_freq=sigmoid_sfu_freq,
            sigmoid_sfu_res=sigmoid_sfu_res, sigmoid_bias=sigmoid_bias, sigmoid_poly_backend=sigmoid_poly_backend,
            sigmoid_degree=sigmoid_degree, sigmoid_coeff_source=sigmoid_coeff_source,
            exp2_emu_backend=exp2_emu_backend, exp2_emu_freq=exp2_emu_freq)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.kw = dict(
            softmax_scale=softmax_scale, causal=causal, softcap=fused_softcap, score_mod=score_mod,
            score_mod_bwd=score_mod_bwd, sigmoid_attention=sigmoid_attention, sigmoid_bias=sigmoid_bias,
            sigmoid_sfu_freq=sigmoid_sfu_freq if sigmoid_sfu_freq_bwd is None else sigmoid_sfu_freq_bwd,
            sigmoid_sfu_res=sigmoid_sfu_res if sigmoid_sfu_res_bwd is None else sigmoid_sfu_res_bwd,
            sigmoid_use_direct_bwd_poly=sigmoid_use_direct_bwd_poly, sigmoid_poly_backend=sigmoid_poly_backend,
            sigmoid_degree=(sigmoid_degree if sigmoid_use_direct_bwd_poly or sigmoid_degree_bwd is None
                            else sigmoid_degree_bwd),
            sigmoid_gradient_degree=sigmoid_degree if sigmoid_degree_bwd is None else sigmoid_degree_bwd,
            sigmoid_coeff_source=sigmoid_coeff_source, exp2_emu_backend=exp2_emu_backend,
            exp2_emu_freq=exp2_emu_freq_bwd)
        ctx.flash_attn_bwd = flash_attn_bwd
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        kw = dict(ctx.kw)
        softmax_scale, causal, softcap = kw.pop("softmax_scale"), kw.pop("causal"), kw.pop("softcap")
        dq, dk, dv = ctx.flash_attn_bwd(q, k, v, out, dout.contiguous(), lse, softmax_scale, causal, softcap, **kw)
        return (dq, dk, dv) + (None,) * 21


def _fa4(q, k, v, *, softmax_scale: float | None, causal: bool, config: ResolvedFA4Config) -> torch.Tensor:
    return _FA4Function.apply(
        q, k, v, softmax_scale, causal, config.softcap, config.sigmoid_attention, config.sigmoid_sfu_freq,
        config.sigmoid_sfu_res, config.sigmoid_sfu_freq_bwd, config.sigmoid_sfu_res_bwd,
        config.sigmoid_use_direct_bwd_poly, config.sigmoid_bias, config.sigmoid_poly_backend,
        config.sigmoid_degree, config.sigmoid_degree_bwd, config.sigmoid_coeff_source, config.exp2_emu_backend,
        config.exp2_emu_freq, config.exp2_emu_freq_bwd, config.score_mod, config.score_mod_bwd,
        config.flash_attn_fwd, config.flash_attn_bwd)


class FA4AttentionWrapper(nn.Module):
    """Causal attention module over the resolved kernels
    (src/sfu_repro/fa4.py:500-549): q, k, v ``(batch, heads, sequence,
    dim)``; sigmoid attention with ``sigmoid_qk_norm`` RMS-normalises q and
    k first."""

    def __init__(self, config: ResolvedFA4Config, head_dim: int):
        super().__init__()
        self.config = config
        self.head_dim = int(head_dim)
        norm = config.sigmoid_attention and config.sigmoid_qk_norm
        self.q_norm: nn.Module | None = nn.RMSNorm(self.head_dim) if norm else None
        self.k_norm: nn.Module | None = nn.RMSNorm(self.head_dim) if norm else None

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                score_mod: Callable[..., Any] | None = None, scale: float | None = None,
                **kwargs: Any) -> torch.Tensor:
        if score_mod is not None:
            raise NotImplementedError("external score_mod is unsupported; select it in FA4Config")
        kwargs.pop("enable_gqa", None)
        if kwargs:
            raise TypeError("unsupported FA4 attention kwargs: " + ", ".join(sorted(kwargs)))
        if self.q_norm is not None:
            q, k = self.q_norm(q), self.k_norm(k)
        dtype = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else q.dtype
        out = _fa4(q.transpose(1, 2).contiguous().to(dtype), k.transpose(1, 2).contiguous().to(dtype),
                   v.transpose(1, 2).contiguous().to(dtype), softmax_scale=scale, causal=True, config=self.config)
        return out.transpose(1, 2).contiguous()


def build_fa4_module(config: FA4Config, *, head_dim: int, sequence_length: int | None = None) -> FA4AttentionWrapper:
    """Resolve ``config`` and construct its attention module."""
    return FA4AttentionWrapper(resolve_fa4_config(config, sequence_length=sequence_length), head_dim=head_dim)


def patch_attention_modules(model: nn.Module, config: ResolvedFA4Config) -> int:
    """Replace every ``inner_attention`` slot of modules that also carry
    ``head_dim`` (src/sfu_repro/fa4.py:566-588); returns how many."""
    patched = 0
    for module in model.modules():
        if not hasattr(module, "inner_attention") or not hasattr(module, "head_dim"):
            continue
        if isinstance(module.inner_attention, FA4AttentionWrapper):
            continue
        wrapper = FA4AttentionWrapper(config=config, head_dim=module.head_dim)
        parameter = next(module.parameters(), None)
        if parameter is not None and parameter.device.type != "meta":
            wrapper = wrapper.to(device=parameter.device, dtype=parameter.dtype)
        elif parameter is not None:
            wrapper = wrapper.to(dtype=parameter.dtype)
        module.inner_attention = wrapper
        if hasattr(module, "use_flex_attn"):
            module.use_flex_attn = False
        if hasattr(module, "attn_score_modifier"):
            module.attn_score_modifier = None
        patched += 1
    return patched


__all__ = [
    "DEFAULT_EXP2_VARIANTS",
    "Exp2Variant",
    "FA4AttentionWrapper",
    "FA4Config",
    "FLASH_SIGMOID_DIRECT_SEQUENCE_LENGTH",
    "ResolvedFA4Config",
    "SUPPORTED_EXP2_BACKENDS",
    "b2_component_configs",
    "b3_component_configs",
    "b5_component_configs",
    "build_fa4_module",
    "parse_exp2_frequency",
    "parse_exp2_variants",
    "patch_attention_modules",
    "resolve_fa4_config",
    "softmax_exp2_config",
    "validate_fa4_config",
]
