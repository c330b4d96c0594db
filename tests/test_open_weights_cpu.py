"""Model-level patching (sfu_repro.open_weights) on the CPU: the variant
grammar and coverage rules of the reference's
scripts/benchmark_open_weights.py:220-343, the slot collectors on small
randomly initialised Transformers models, and the patch wiring with a
stand-in ops object that computes each kernel's function with torch, so a
patched model must reproduce the unpatched one exactly."""

import argparse

import pytest
import torch
import torch.nn.functional as F

from sfu_repro import open_weights as ow

TINY = {
    "llama3-8b-2l": dict(hidden_size=64, intermediate_size=128, num_attention_heads=4, num_key_value_heads=2,
                         vocab_size=128),
    "gemma2-d128-2l": dict(hidden_size=64, intermediate_size=128, num_attention_heads=2, num_key_value_heads=1,
                           head_dim=32, vocab_size=128),
    "glm4-moe-lite-2l": dict(hidden_size=64, intermediate_size=128, moe_intermediate_size=32, num_attention_heads=4,
                             num_key_value_heads=4, n_routed_experts=8, num_experts_per_tok=2, vocab_size=128),
}


class TorchOps:
    """The functions of the spline_ops kernels the patches call, in torch."""

    calls: list

    def __init__(self):
        self.calls = []

    def swish_fwd_variant(self, x, d, s):
        self.calls.append(("silu", d, s))
        return F.silu(x)

    def gelu_fwd_variant(self, x, d, s):
        self.calls.append(("gelu", d, s))
        return F.gelu(x, approximate="tanh")

    def sigmoid_fwd_variant(self, x, d, s):
        self.calls.append(("sigmoid", d, s))
        return torch.sigmoid(x)

    def tanh_fwd(self, x):
        self.calls.append(("tanh",))
        return torch.tanh(x)

    def swish_mul_fwd_variant(self, g, u, d, s):
        self.calls.append(("swiglu", d, s))
        return F.silu(g) * u

    def swish_mul_packed_fwd_variant(self, p, d, s):
        self.calls.append(("packed", d, s))
        g, u = p.chunk(2, dim=-1)
        return F.silu(g) * u


@pytest.fixture
def ops(monkeypatch):
    o = TorchOps()
    monkeypatch.setattr(ow, "_ops", lambda: o)
    return o


def _model(preset, dtype=torch.bfloat16, **kw):
    torch.manual_seed(0)
    return ow.build_model(preset, dtype=dtype, device="cpu", overrides=TINY[preset], **kw)


def _logits(model, tokens):
    with torch.no_grad():
        return model(input_ids=tokens, use_cache=False).logits.float()


def test_variant_grammar():
    spec = ow.parse_variant("spline_silu_d3_current+fused_swiglu_d4_sollya+spline_router_sigmoid_d5_current")
    assert (spec.silu_degree, spec.silu_source, spec.dense_swiglu_degree, spec.dense_swiglu_source,
            spec.router_sigmoid_degree) == (3, "current", 4, "sollya", 5)
    fa = ow.parse_variant("gemma_fa4_tanh_d4_current")
    assert (fa.gemma_fa4_tanh_backend, fa.gemma_fa4_tanh_degree) == ("device", 4)
    assert ow.parse_variant("gemma_fa4_tanh_native").gemma_fa4_tanh_backend == "native"
    assert ow.parse_variant("native") == ow.VariantSpec(name="native")
    for bad, match in (("native+spline_silu_d3_current", "cannot be combined"), ("spline_silu_d3", "Unknown"),
                       ("spline_silu_d3_current+", "empty")):
        with pytest.raises(argparse.ArgumentTypeError, match=match):
            ow.parse_variant(bad)


def test_coverage_rules():
    spec = ow.parse_variant("spline_silu_d3_current+gemma_tanh_current")
    assert ow.required_interventions(spec) == {"activation", "softcap"}
    res = ow.Result("m", spec.name, "bf16", "cpu", 1, 8, patched_silu_modules=2)
    with pytest.raises(RuntimeError, match="attention softcap"):
        ow.require_applied_interventions(spec, res)
    res.patched_gemma_softcap = True
    ow.require_applied_interventions(spec, res)


@pytest.mark.parametrize("preset,expect", [
    ("llama3-8b-2l", dict(silu=2, gelu=0, dense_swiglu=2, packed_experts_gate=0, sigmoid_router=0)),
    ("gemma2-d128-2l", dict(silu=0, gelu=2, dense_swiglu=0, packed_experts_gate=0, sigmoid_router=0)),
    ("glm4-moe-lite-2l", dict(silu=3, gelu=0, dense_swiglu=2, packed_experts_gate=1, sigmoid_router=1)),
])
def test_collectors(preset, expect):
    slots = ow.collect_slots(_model(preset, torch.float32))
    assert {k: len(getattr(slots, k)) for k in expect} == expect


@pytest.mark.parametrize("variant,calls", [
    ("spline_silu_d3_current", {("silu", 3, 0)}),
    ("fused_swiglu_d4_sollya", {("swiglu", 4, 1)}),
    ("spline_silu_d5_current+fused_swiglu_d3_current", {("swiglu", 3, 0)}),
])
def test_llama_patches_reproduce_the_model(ops, variant, calls):
    model = _model("llama3-8b-2l")
    tokens = torch.randint(1, 128, (2, 16), generator=torch.Generator().manual_seed(1))
    ref = _logits(model, tokens)
    slots = ow.collect_slots(model)
    res = ow.apply_variant(slots, ow.parse_variant(variant), ow.Result("m", variant, "bf16", "cpu", 2, 16))
    assert res.patched_silu_modules >= 2
    assert torch.equal(_logits(model, tokens), ref)
    assert set(ops.calls) == calls
    # native restores every original
    ops.calls.clear()
    ow.apply_variant(slots, ow.parse_variant("native"), ow.Result("m", "native", "bf16", "cpu", 2, 16))
    assert torch.equal(_logits(model, tokens), ref) and not ops.calls


def test_moe_expert_gates_and_router(ops):
    model = _model("glm4-moe-lite-2l", experts_implementation="batched_mm")
    tokens = torch.randint(1, 128, (1, 12), generator=torch.Generator().manual_seed(2))
    ref = _logits(model, tokens)
    slots = ow.collect_slots(model)
    spec = ow.parse_variant("fused_swiglu_d3_current")
    res = ow.apply_variant(slots, spec, ow.Result("m", spec.name, "bf16", "cpu", 1, 12))
    assert res.patched_silu_modules == 3  # two dense MLPs + one experts block
    assert torch.equal(_logits(model, tokens), ref)
    assert ("packed", 3, 0) in ops.calls and ("swiglu", 3, 0) in ops.calls
    # router: same experts and weights up to the BF16 sigmoid of the kernel path
    router = slots.sigmoid_router[0].module
    h = torch.randn(12, 64, dtype=torch.bfloat16, generator=torch.Generator().manual_seed(3))
    logits0, w0, i0 = router(h)
    ow.apply_variant(slots, ow.parse_variant("spline_router_sigmoid_d3_current"),
                     ow.Result("m", "r", "bf16", "cpu", 1, 12))
    logits1, w1, i1 = router(h)
    assert torch.equal(logits0, logits1)
    # the kernel path rounds the logits to BF16 first: expert sets agree
    # wherever the original choice has a clear margin, weights within BF16
    choice = torch.sigmoid(logits0) + router.e_score_correction_bias
    top = choice.topk(3, dim=-1).values
    clear = (top[:, 1] - top[:, 2]) > 1e-2
    same = (i0.sort(-1).values == i1.sort(-1).values).all(-1)
    assert clear.any() and same[clear].all()
    assert (w0.sort(-1).values - w1.sort(-1).values)[same].abs().max() < 2e-2


def test_gemma_eager_softcap_patch(ops):
    model = _model("gemma2-d128-2l")
    tokens = torch.randint(1, 128, (1, 16), generator=torch.Generator().manual_seed(4))
    ref = _logits(model, tokens)
    spec = ow.parse_variant("gemma_tanh_current")
    res = ow.apply_variant(ow.collect_slots(model), spec, ow.Result("m", spec.name, "bf16", "cpu", 1, 16))
    try:
        got = _logits(model, tokens)
        assert res.patched_gemma_softcap and ("tanh",) in ops.calls
        assert (got - ref).abs().max() < 2e-2 * ref.abs().max()
    finally:
        ow.restore_gemma_attention()


def test_unbuilt_paths_raise():
    with pytest.raises(ValueError, match="D3/D4/D5/D6"):
        ow.load_spline_sigmoid(7, "current")
    slot = ow.MethodSlot("x", torch.nn.Identity(), "forward", lambda x: x)
    with pytest.raises(NotImplementedError, match="MXFP4"):
        ow.apply_mxfp4_swiglu_patch([slot], ow.parse_variant("spline_silu_d3_current"))
