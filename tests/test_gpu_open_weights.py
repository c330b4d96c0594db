"""Model-level patching on the GPU with the real kernels: small randomly
initialised Transformers models (BF16) patched with each family of
sfu_repro.open_weights.  Each patched slot must compute exactly what the
spline_ops kernel computes on the same operands, and the patched model must
stay within the polynomial programs' error of the unpatched one."""

import pytest
import torch

from sfu_repro import open_weights as ow

pytestmark = pytest.mark.gpu

SMALL = {
    "llama3-8b-2l": dict(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=2,
                         vocab_size=512),
    "gemma2-d128-2l": dict(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=2,
                           head_dim=128, vocab_size=512),
    "glm4-moe-lite-2l": dict(hidden_size=256, intermediate_size=512, moe_intermediate_size=128,
                             num_attention_heads=4, num_key_value_heads=4, n_routed_experts=8, num_experts_per_tok=2,
                             vocab_size=512),
}


def _model(cuda, preset, **kw):
    torch.manual_seed(0)
    return ow.build_model(preset, dtype=torch.bfloat16, device=cuda, overrides=SMALL[preset], **kw)


def _logits(model, tokens):
    with torch.no_grad():
        return model(input_ids=tokens, use_cache=False).logits.float()


def _apply(model, variant, slots=None):
    """Patch `model`; slots are collected once, before any patch (as the
    reference does), and reused for later variants."""
    slots = ow.collect_slots(model) if slots is None else slots
    return slots, ow.apply_variant(slots, ow.parse_variant(variant), ow.Result("m", variant, "bf16", "cuda", 1, 1))


def _rel(a, b):
    return ((a - b).abs().max() / b.abs().max()).item()


def test_llama_silu_and_fused_swiglu(cuda, spline_ops):
    model = _model(cuda, "llama3-8b-2l")
    tokens = torch.randint(1, 512, (2, 128), device=cuda, generator=torch.Generator(device=cuda).manual_seed(1))
    ref = _logits(model, tokens)
    mlp = model.model.layers[0].mlp
    x = torch.randn(2, 128, 256, device=cuda, dtype=torch.bfloat16)
    slots = ow.collect_slots(model)
    for variant in ("spline_silu_d3_current", "fused_swiglu_d3_current", "fused_swiglu_d5_sollya"):
        _, res = _apply(model, variant, slots)
        assert res.patched_silu_modules == 2
        with torch.no_grad():
            got = mlp(x)
            g, u = mlp.gate_proj(x), mlp.up_proj(x)
            spec = ow.parse_variant(variant)
            if spec.dense_swiglu_degree:
                want = mlp.down_proj(spline_ops.swish_mul_fwd_variant(g, u, spec.dense_swiglu_degree,
                                                                      ow.SOURCE_IDS[spec.dense_swiglu_source]))
            else:
                want = mlp.down_proj(spline_ops.swish_fwd_variant(g, 3, 0) * u)
        assert torch.equal(got, want), variant
        assert _rel(_logits(model, tokens), ref) < 0.05, variant
    ow.apply_variant(slots, ow.parse_variant("native"), ow.Result("m", "native", "bf16", "cuda", 1, 1))
    assert torch.equal(_logits(model, tokens), ref)


def test_glm_moe_expert_gates_and_router(cuda, spline_ops):
    model = _model(cuda, "glm4-moe-lite-2l", experts_implementation="batched_mm")
    tokens = torch.randint(1, 512, (1, 128), device=cuda, generator=torch.Generator(device=cuda).manual_seed(2))
    ref = _logits(model, tokens)
    slots, res = _apply(model, "fused_swiglu_d3_current+spline_router_sigmoid_d4_current")
    assert res.patched_silu_modules == 3 and res.patched_router_sigmoid_modules == 1
    experts = slots.packed_experts_gate[0].module
    gu = torch.randn(64, 256, device=cuda, dtype=torch.bfloat16)
    assert torch.equal(experts._apply_gate(gu), spline_ops.swish_mul_packed_fwd_variant(gu, 3, 0))
    router = slots.sigmoid_router[0].module
    logits = torch.randn(16, 8, device=cuda)
    want = spline_ops.sigmoid_fwd_variant(logits.bfloat16(), 4, 0).float()
    with torch.no_grad():
        _, w, idx = router(torch.randn(16, 256, device=cuda, dtype=torch.bfloat16))
    assert idx.shape == (16, 2) and torch.isfinite(w).all()
    assert want.shape == logits.shape
    assert _rel(_logits(model, tokens), ref) < 0.1


def test_gptoss_gate(cuda, spline_ops):
    import transformers

    torch.manual_seed(0)
    cfg = transformers.AutoConfig.for_model(
        "gpt_oss", hidden_size=256, intermediate_size=256, num_hidden_layers=1, num_attention_heads=4,
        num_key_value_heads=2, head_dim=64, num_local_experts=4, num_experts_per_tok=2, vocab_size=512)
    cfg._attn_implementation = "eager"
    with torch.device(cuda):
        model = transformers.AutoModelForCausalLM.from_config(cfg, dtype=torch.bfloat16).eval()
    tokens = torch.randint(1, 512, (1, 64), device=cuda, generator=torch.Generator(device=cuda).manual_seed(3))
    ref = _logits(model, tokens)
    slots, res = _apply(model, "spline_silu_d3_current")
    assert len(slots.gptoss_gate) == 1 and res.patched_silu_modules >= 1
    m = slots.gptoss_gate[0].module
    gu = torch.randn(32, 512, device=cuda, dtype=torch.bfloat16)
    gate = gu[..., ::2].clamp(max=m.limit)
    up = gu[..., 1::2].clamp(-m.limit, m.limit)
    want = spline_ops.swish_mul_fwd_variant((gate * m.alpha).contiguous(), (up + 1).contiguous(), 3, 0) / m.alpha
    assert torch.equal(m._apply_gate(gu), want)
    assert _rel(_logits(model, tokens), ref) < 0.1


@pytest.mark.parametrize("variant,seq", [("gemma_tanh_current", 256), ("gemma_fa4_tanh_native", 256),
                                         ("gemma_fa4_tanh_d4_current", 256), ("gemma_fa4_tanh_d4_current", 200)])
def test_gemma_softcap_patches(cuda, variant, seq):
    # 200 tokens: the fused attention pads the causal prefill to whole blocks
    model = _model(cuda, "gemma2-d128-2l")
    tokens = torch.randint(1, 512, (2, seq), device=cuda, generator=torch.Generator(device=cuda).manual_seed(4))
    ref = _logits(model, tokens)
    try:
        _, res = _apply(model, variant)
        assert res.patched_gemma_softcap
        got = _logits(model, tokens)
        assert torch.isfinite(got).all()
        assert _rel(got, ref) < 0.05, variant
    finally:
        ow.restore_gemma_attention()
    assert torch.equal(_logits(model, tokens), ref)


def test_gemma_fused_attention_rejects_padding(cuda):
    model = _model(cuda, "gemma2-d128-2l")
    tokens = torch.randint(1, 512, (2, 128), device=cuda)
    mask = torch.ones(2, 128, dtype=torch.long, device=cuda)
    mask[1, :5] = 0
    try:
        _apply(model, "gemma_fa4_tanh_native")
        with pytest.raises(NotImplementedError, match="unpadded"):
            with torch.no_grad():
                model(input_ids=tokens, attention_mask=mask, use_cache=False)
    finally:
        ow.restore_gemma_attention()
