"""The FA4 configuration layer (sfu_repro.fa4) on the CPU: the cases of the
reference's tests/test_fa4_config.py:54-205 (B2 / B3 / B5 program selection,
the fitted-length guard, the exp2 routing parser), with a stand-in runtime
as the reference uses, plus the mapping of FA4's keyword arguments onto this
build's kernel modes (sfu_repro.fa4_runtime.select_forward / select_backward)."""

from typing import Any, Callable

import pytest

from sfu_repro import fa4_runtime as rt
from sfu_repro.fa4 import (
    DEFAULT_EXP2_VARIANTS,
    FA4Config,
    FLASH_SIGMOID_DIRECT_SEQUENCE_LENGTH,
    b2_component_configs,
    b3_component_configs,
    b5_component_configs,
    parse_exp2_frequency,
    parse_exp2_variants,
    resolve_fa4_config,
    softmax_exp2_config,
    validate_fa4_config,
)


def _stand_in_runtime() -> dict[str, Callable[..., Any]]:
    """Runtime mapping with the reference's keys and no kernels."""
    return {
        "flash_attn_fwd": lambda *a, **k: (None, None),
        "flash_attn_bwd": lambda *a, **k: (None, None, None),
        "run_polynomial_coefficient_audit": lambda: ("manifest",),
        "audit_polynomial_selection": lambda sel: (f"selected:{sel!r}",),
        "audit_attention_handwritten_fast_path": lambda fam, deg, src: f"device {fam} D{deg} {src}",
        "create_softcap_scoremod_backend": lambda *a, **k: (lambda x: x),
        "create_softcap_scoremod_bwd_backend": lambda *a, **k: (lambda x: x),
    }


def test_b2_native_and_device_d4_routes():
    configs = b2_component_configs()
    native, poly = configs["native"], configs["polynomial"]
    assert (native.mode, native.softcap, native.softcap_backend, native.softcap_backward_mode) == (
        "softcap", 30.0, "native", "native")
    assert (poly.softcap_backend, poly.softcap_degree, poly.softcap_coeff_source,
            poly.softcap_backward_mode) == ("device", 4, "current", "analytical")
    rt_ = _stand_in_runtime()
    r_native = resolve_fa4_config(native, runtime=rt_)
    r_poly = resolve_fa4_config(poly, runtime=rt_)
    assert r_native.softcap == 30.0 and r_native.score_mod is None
    assert r_poly.softcap == 0.0 and r_poly.score_mod is not None
    assert "tanh_fwd D4 current" in r_poly.implementation_summary
    assert "tanh_grad_analytical D4 current" in r_poly.implementation_summary


def test_b3_native_sfu_and_direct_device_d3_d4():
    configs = b3_component_configs(sequence_length=4096)
    native, poly = configs["native"], configs["polynomial"]
    assert (native.sigmoid_variant, native.sigmoid_sfu_freq, native.sigmoid_sfu_res,
            native.sigmoid_qk_norm) == ("sfu", 16, 16, True)
    assert (poly.sigmoid_variant, poly.sigmoid_poly_backend, poly.sigmoid_degree, poly.sigmoid_degree_bwd,
            poly.sigmoid_backward_mode, poly.sigmoid_sfu_res, poly.sigmoid_qk_norm) == (
        "poly", "device", 3, 4, "direct", 0, True)
    r = resolve_fa4_config(poly, sequence_length=4096, runtime=_stand_in_runtime())
    assert r.sigmoid_attention and r.sigmoid_use_direct_bwd_poly
    assert (r.sigmoid_degree, r.sigmoid_degree_bwd) == (3, 4)
    assert "flash_sigmoid_direct D3 current" in r.implementation_summary
    assert "flash_sigmoid_direct_with_grad D4 current" in r.implementation_summary


@pytest.mark.parametrize("n", (1, 2048, 4095, 4097, 8192))
def test_b3_rejects_other_sequence_lengths(n):
    with pytest.raises(ValueError, match="requires sequence length 4096"):
        b3_component_configs(sequence_length=n)


def test_direct_b3_needs_an_explicit_length():
    poly = b3_component_configs()["polynomial"]
    with pytest.raises(ValueError, match="explicit sequence_length"):
        validate_fa4_config(poly)
    assert validate_fa4_config(poly, sequence_length=FLASH_SIGMOID_DIRECT_SEQUENCE_LENGTH) is poly


def test_exp2_variants_keep_auto_and_fractions():
    v = parse_exp2_variants("sfu=d3:0:0,mixed=d2_safe:8:12,auto=d3:auto:0")
    assert [x.name for x in v] == ["sfu", "mixed", "auto"]
    assert v[0].nominal_forward_polynomial_fraction == 0.0
    assert v[1].nominal_forward_polynomial_fraction == 0.5
    assert v[1].nominal_backward_polynomial_fraction == pytest.approx(1 / 3)
    assert v[2].forward_frequency is None and v[2].nominal_forward_pwl_fraction is None
    assert softmax_exp2_config(v[1]) == FA4Config(mode="softmax", exp2_emu_backend="d2_safe",
                                                  exp2_emu_freq=8, exp2_emu_freq_bwd=12)
    assert len(parse_exp2_variants(DEFAULT_EXP2_VARIANTS)) == 11


def test_b5_routed_schedules():
    configs = b5_component_configs()
    assert tuple(configs) == ("native", "pwl2_safe_f16", "d2_safe")
    want = {"native": ("d3", 0, 0), "pwl2_safe_f16": ("pwl2_safe_f16", 12, 32), "d2_safe": ("d2_safe", 12, 32)}
    for name, (backend, f, b) in want.items():
        c = configs[name]
        assert (c.mode, c.exp2_emu_backend, c.exp2_emu_freq, c.exp2_emu_freq_bwd) == ("softmax", backend, f, b)
        assert validate_fa4_config(c) is c


@pytest.mark.parametrize("spec,match", (
    ("bad=d3:5:0", "even integer"),
    ("bad=d3:4:auto", "frequency"),
    ("bad=unknown:4:0", "unsupported exp2 backend"),
    ("same=d3:0:0,same=d2_safe:4:0", "names must be unique"),
    ("missing", "variant must have"),
    ("", "at least one variant"),
))
def test_exp2_parser_rejects_ambiguous_routes(spec, match):
    with pytest.raises(ValueError, match=match):
        parse_exp2_variants(spec)


def test_exp2_frequency_parser():
    assert parse_exp2_frequency("auto", allow_auto=True) is None
    with pytest.raises(ValueError, match="frequency"):
        parse_exp2_frequency("auto", allow_auto=False)
    with pytest.raises(ValueError, match="even integer"):
        parse_exp2_frequency("7", allow_auto=True)


@pytest.mark.parametrize("config,match", (
    (FA4Config(mode="bogus"), "unsupported FA4 mode"),
    (FA4Config(mode="softcap", softcap_backend="native", softcap_backward_mode="analytical"),
     "requires softcap_backward_mode='native'"),
    (FA4Config(mode="softcap", softcap_backend="device", softcap_backward_mode="native"),
     "cannot use softcap_backward_mode='native'"),
    (FA4Config(mode="softcap", softcap=0.0, softcap_backend="native", softcap_backward_mode="native"),
     "softcap must be positive"),
    (FA4Config(mode="sigmoid_attention", sigmoid_poly_backend="cute"), "requires sigmoid_poly_backend='device'"),
    (FA4Config(mode="sigmoid_attention", sigmoid_variant="sfu", sigmoid_sfu_res=0),
     "must route every forward/backward lane through the SFU"),
    (FA4Config(mode="sigmoid_attention", sigmoid_poly_backend="device", sigmoid_degree=2,
               sigmoid_backward_mode="direct"), "bias-aware FlashSigmoid D2"),
    (FA4Config(mode="sigmoid_attention", sigmoid_poly_backend="device", sigmoid_degree=7),
     "sigmoid_degree must be one of"),
))
def test_validation_rules(config, match):
    with pytest.raises(ValueError, match=match):
        validate_fa4_config(config, sequence_length=4096)


def test_sollya_sources_need_the_sweep_flag(monkeypatch):
    c = FA4Config(mode="softcap", softcap_backend="device", softcap_coeff_source="sollya")
    monkeypatch.delenv("SFU_REPRO_ALLOW_SOLLYA_SWEEP", raising=False)
    with pytest.raises(ValueError, match="benchmark-only"):
        validate_fa4_config(c)
    monkeypatch.setenv("SFU_REPRO_ALLOW_SOLLYA_SWEEP", "1")
    assert validate_fa4_config(c) is c


# ---- this build's runtime: FA4 keyword arguments -> kernel programs ----------------

def test_forward_program_selection():
    sel = rt.select_forward
    assert sel(seqlen=256) == (rt.MODE_SOFTMAX_NATIVE, 4, 1.0, 0.0)
    assert sel(seqlen=256, exp2_emu_freq=0) == (rt.MODE_SOFTMAX_NATIVE, 4, 1.0, 0.0)
    assert sel(seqlen=256, exp2_emu_backend="d2_safe", exp2_emu_freq=12)[:2] == (rt.MODE_SOFTMAX_D2, 12)
    assert sel(seqlen=256, exp2_emu_backend="d3", exp2_emu_freq=4)[:2] == (rt.MODE_SOFTMAX_D3, 4)
    assert sel(seqlen=256, exp2_emu_backend="pwl2", exp2_emu_freq=8)[:2] == (rt.MODE_SOFTMAX_PWL2, 8)
    assert sel(seqlen=256, exp2_emu_backend="pwl2_safe", exp2_emu_freq=12)[:2] == (rt.MODE_SOFTMAX_PWL2_SAFE, 12)
    assert sel(seqlen=256, exp2_emu_backend="pwl2_safe_f16", exp2_emu_freq=12)[:2] == \
        (rt.MODE_SOFTMAX_PWL2_SAFE_F16, 12)
    # every exp2 backend FA4 accepts resolves to a kernel program
    from sfu_repro.fa4 import SUPPORTED_EXP2_BACKENDS

    # the reference's list, in its order (src/sfu_repro/fa4.py:33-46)
    assert SUPPORTED_EXP2_BACKENDS == ("d3", "pwl2", "pwl1_safe", "pwl1_safe_f16", "pwl2_safe", "pwl2_safe_f16",
                                       "pwl2_safe_bf16", "d2_safe", "d2_safe_noclamp", "d2_safe_f16",
                                       "d2_safe_bf16", "pwl2_f16")
    modes = {sel(seqlen=256, exp2_emu_backend=name, exp2_emu_freq=12)[0] for name in SUPPORTED_EXP2_BACKENDS}
    assert len(modes) == len(SUPPORTED_EXP2_BACKENDS) == 12
    assert sel(seqlen=256, exp2_emu_backend="pwl2_f16", exp2_emu_freq=32)[:2] == (rt.MODE_SOFTMAX_PWL1_SAFE + 6, 32)
    with pytest.raises(NotImplementedError, match="d2_safe_bf16_fast"):
        sel(seqlen=256, exp2_emu_backend="d2_safe_bf16_fast", exp2_emu_freq=12)
    # any even frequency >= 4 (the reference's validation, fa4.py:226-233)
    assert sel(seqlen=256, exp2_emu_backend="d3", exp2_emu_freq=14)[:2] == (rt.MODE_SOFTMAX_D3, 14)
    assert sel(seqlen=256, exp2_emu_backend="d2_safe", exp2_emu_freq=128)[:2] == (rt.MODE_SOFTMAX_D2, 128)
    with pytest.raises(ValueError, match="even integer"):
        sel(seqlen=256, exp2_emu_backend="d3", exp2_emu_freq=5)
    assert sel(seqlen=256, softcap=30.0) == (rt.MODE_SOFTCAP_NATIVE, 4, 30.0, 0.0)
    mod = rt.create_softcap_scoremod_backend(30.0, degree=4, backend="device")
    assert sel(seqlen=256, score_mod=mod) == (rt.MODE_SOFTCAP_D4, 4, 30.0, 0.0)
    # sigmoid attention: SFU, B3 direct, B3-D2, biased D3..D6
    m, _, _, bias = sel(seqlen=4096, sigmoid_attention=True, sigmoid_sfu_res=16)
    assert m == rt.MODE_SIGMOID_NATIVE and bias == pytest.approx(-8.317766166719343)
    assert sel(seqlen=4096, sigmoid_attention=True, sigmoid_poly_backend="device")[0] == rt.MODE_SIGMOID_B3
    assert sel(seqlen=4096, sigmoid_attention=True, sigmoid_poly_backend="device",
               sigmoid_degree=2)[0] == rt.MODE_SIGMOID_B3_D2
    with pytest.raises(ValueError, match="fitted for sequence length 4096"):
        sel(seqlen=2048, sigmoid_attention=True, sigmoid_poly_backend="device")
    m, _, _, bias = sel(seqlen=2048, sigmoid_attention=True, sigmoid_poly_backend="device", sigmoid_degree=5,
                        sigmoid_bias=-3.0)
    assert (m, bias) == (rt.MODE_SIGMOID_D3 + 2, -3.0)
    with pytest.raises(NotImplementedError, match="mixed"):
        sel(seqlen=4096, sigmoid_attention=True, sigmoid_sfu_res=4)
    # FA4's CuTe FP32 sigmoid polynomial (the runtime's default backend) is not built
    with pytest.raises(NotImplementedError, match="CuTe FP32 sigmoid"):
        sel(seqlen=4096, sigmoid_attention=True)
    with pytest.raises(NotImplementedError, match="CuTe FP32 sigmoid"):
        sel(seqlen=2048, sigmoid_attention=True, sigmoid_degree=5, sigmoid_bias=-3.0)
    # the SFU route takes no polynomial, whatever the backend
    assert sel(seqlen=4096, sigmoid_attention=True, sigmoid_sfu_res=16)[0] == rt.MODE_SIGMOID_NATIVE


def test_backward_program_selection():
    sel = rt.select_backward
    assert sel(seqlen=256) == (rt.MODE_SOFTMAX_NATIVE, rt.GRAD_NATURAL, 0, 1.0, 0.0)
    assert sel(seqlen=256, exp2_emu_backend="d2_safe", exp2_emu_freq=32)[:3] == (rt.MODE_SOFTMAX_D2, 0, 32)
    assert sel(seqlen=256, exp2_emu_backend="pwl2_safe_f16", exp2_emu_freq=32)[:3] == \
        (rt.MODE_SOFTMAX_PWL2_SAFE_F16, 0, 32)
    for mode_name, grad in (("analytical", rt.GRAD_ANALYTICAL), ("ste", rt.GRAD_STE),
                            ("exact_1mt2", rt.GRAD_EXACT_1MT2)):
        fwd = rt.create_softcap_scoremod_backend(30.0)
        bwd = rt.create_softcap_scoremod_bwd_backend(30.0, backward_mode=mode_name)
        assert sel(seqlen=256, score_mod=fwd, score_mod_bwd=bwd)[:2] == (rt.MODE_SOFTCAP_D4, grad)
    assert sel(seqlen=256, softcap=30.0)[:2] == (rt.MODE_SOFTCAP_NATIVE, rt.GRAD_NATURAL)
    b3 = dict(seqlen=4096, sigmoid_attention=True, sigmoid_poly_backend="device", sigmoid_degree=3)
    assert sel(**b3, sigmoid_use_direct_bwd_poly=True, sigmoid_gradient_degree=4)[:2] == (
        rt.MODE_SIGMOID_B3, rt.GRAD_DIRECT)
    assert sel(**b3)[:2] == (rt.MODE_SIGMOID_B3, rt.GRAD_ALGEBRAIC)
    with pytest.raises(NotImplementedError):
        sel(seqlen=256, sigmoid_attention=True, sigmoid_poly_backend="device", sigmoid_degree=4,
            sigmoid_bias=-1.0, sigmoid_use_direct_bwd_poly=True)


def test_softcap_factories_reject_unbuilt_programs():
    with pytest.raises(NotImplementedError, match="D4"):
        rt.create_softcap_scoremod_backend(30.0, degree=3)
    with pytest.raises(NotImplementedError, match="Sollya"):
        rt.create_softcap_scoremod_backend(30.0, coeff_source="sollya")
    with pytest.raises(NotImplementedError, match="CuTe FP32"):
        rt.create_softcap_scoremod_backend(30.0, backend="cute")
    with pytest.raises(NotImplementedError, match="CuTe FP32"):
        rt.create_softcap_scoremod_bwd_backend(30.0, backend="cute")
    with pytest.raises(ValueError, match="unsupported softcap backend"):
        rt.create_softcap_scoremod_backend(30.0, backend="ptx")
    with pytest.raises(ValueError, match="backward mode"):
        rt.create_softcap_scoremod_bwd_backend(30.0, backward_mode="native")


def test_audits_name_built_programs():
    assert rt.audit_polynomial_selection((("tanh_fwd", 4, "current"),)) == ("tanh_fwd D4 current",)
    with pytest.raises(NotImplementedError):
        rt.audit_polynomial_selection((("tanh_fwd", 5, "current"),))
    assert rt.audit_attention_handwritten_fast_path("flash_sigmoid_direct", 3, "current").startswith(
        "device flash_sigmoid_direct D3 current")
