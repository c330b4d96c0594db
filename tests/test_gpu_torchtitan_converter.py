"""The TorchTitan converter on the GPU: TorchTitan-shaped models (tests/
torchtitan_like.py) converted for B1..B5 run forward and backward through the
HIP kernels (fused attention, packed / fused SwiGLU) and stay close to the
unconverted model (native variants) or to the native control (polynomial
variants)."""

import copy
from types import SimpleNamespace

import pytest
import torch

from sfu_repro.torchtitan import SFUConfig
from sfu_repro.torchtitan.plugin import SFUReproConverter
from torchtitan_like import GroupedExperts, Transformer

pytestmark = pytest.mark.gpu


def _job(case, variant, seq_len=256, model="sfu_llama3"):
    return SimpleNamespace(sfu=SFUConfig(case=case, variant=variant, strict=True), model=SimpleNamespace(name=model),
                           training=SimpleNamespace(seq_len=seq_len, local_batch_size=1, global_batch_size=1,
                                                    steps=80),
                           compile=SimpleNamespace(enable=False))


def _model(cuda, seed=0):
    torch.manual_seed(seed)
    return Transformer(dim=512, hidden=1024, n_layers=2, n_heads=4, n_kv_heads=2).to(cuda, torch.bfloat16)


def _rel(a, b):
    return ((a.float() - b.float()).abs().max() / b.float().abs().max()).item()


def _convert(model, case, variant, seq_len=256):
    return SFUReproConverter(_job(case, variant, seq_len), SimpleNamespace(tp=1)).convert(model)


@pytest.mark.parametrize("variant,tol", [("native", 0.03), ("polynomial", 0.05)])
def test_b1_fused_mlp_and_fa4_softmax(cuda, variant, tol):
    base = _model(cuda)
    model = copy.deepcopy(base)
    counts = _convert(model, "b1", variant)
    assert counts == {"attention": 2, "activation": 2}
    assert type(model.layers[0].feed_forward).__name__ == "ConfiguredFusedLlamaFeedForward"
    x = torch.randn(2, 256, 512, device=cuda, dtype=torch.bfloat16, requires_grad=True)
    with torch.no_grad():
        ref = base(x)
    out = model(x)
    assert _rel(out, ref) < tol
    out.float().square().mean().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()
    assert all(torch.isfinite(p.grad).all() for p in model.parameters() if p.grad is not None)


def test_b1_at_head_dim_64(cuda):
    """The reference's training model has head_dim 64 (Llama 1B: dim 2048,
    32 heads); a model with that head size converts and trains."""
    torch.manual_seed(0)
    base = Transformer(dim=512, hidden=1024, n_layers=2, n_heads=8, n_kv_heads=2).to(cuda, torch.bfloat16)
    model = copy.deepcopy(base)
    assert _convert(model, "b1", "polynomial") == {"attention": 2, "activation": 2}
    x = torch.randn(1, 256, 512, device=cuda, dtype=torch.bfloat16, requires_grad=True)
    with torch.no_grad():
        ref = base(x)
    out = model(x)
    assert _rel(out, ref) < 0.05
    out.float().square().mean().backward()
    assert torch.isfinite(x.grad).all()


def test_b2_softcap_variants_agree(cuda):
    outs = {}
    x = torch.randn(1, 256, 512, device=cuda, dtype=torch.bfloat16) * 4
    for variant in ("native", "polynomial"):
        model = _model(cuda)
        assert _convert(model, "b2", variant)["attention"] == 2
        with torch.no_grad():
            outs[variant] = model(x)
    assert _rel(outs["polynomial"], outs["native"]) < 0.05


def test_b3_sigmoid_attention_at_4096(cuda):
    outs = {}
    x = torch.randn(1, 4096, 512, device=cuda, dtype=torch.bfloat16)
    for variant in ("native", "polynomial"):
        model = _model(cuda)
        assert _convert(model, "b3", variant, seq_len=4096)["attention"] == 2
        wrapper = model.layers[0].attention.inner_attention
        assert wrapper.q_norm is not None  # B3 adds QK RMSNorm
        model.layers[0].attention.init_weights(0.02)  # resets the added norms too
        model = model.to(cuda, torch.bfloat16)
        with torch.no_grad():
            outs[variant] = model(x)
    a, b = outs["polynomial"].float().flatten(), outs["native"].float().flatten()
    assert torch.nn.functional.cosine_similarity(a, b, dim=0).item() > 0.95


def test_b4_grouped_experts(cuda):
    torch.manual_seed(1)
    experts = GroupedExperts(256, 512, 8).to(cuda, torch.bfloat16)
    counts = torch.tensor([40, 0, 17, 64, 3, 33, 8, 27], device=cuda)
    x = torch.randn(int(counts.sum()), 256, device=cuda, dtype=torch.bfloat16)
    with torch.no_grad():
        ref = experts(x, counts)
    holder = torch.nn.ModuleDict({"experts": experts})
    for variant, tol in (("native", 0.02), ("polynomial", 0.05)):
        conv = SFUReproConverter(_job("b4", variant, model="sfu_deepseek_v3"), SimpleNamespace(tp=1))
        conv.strict = False
        assert conv.convert(holder)["activation"] == 1
        with torch.no_grad():
            got = experts(x, counts)
        assert got.shape == ref.shape and _rel(got, ref) < tol, variant
