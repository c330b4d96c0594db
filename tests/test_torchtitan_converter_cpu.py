"""The converter's job-config checks (src/sfu_repro/torchtitan/plugin.py:375-424),
which need no GPU, and module recognition on TorchTitan-shaped models."""

from types import SimpleNamespace

import pytest

from sfu_repro.torchtitan import JobConfig, SFUConfig
from sfu_repro.torchtitan.plugin import (
    SFUReproConverter,
    is_grouped_experts,
    is_llama_attention,
    is_llama_feed_forward,
)
from torchtitan_like import GroupedExperts, Transformer


def _job(case="b1", variant="native", model="sfu_llama3", seq_len=4096, compile_=False, batch=(1, 1, 80),
         strict=True):
    return SimpleNamespace(
        sfu=SFUConfig(case=case, variant=variant, strict=strict), model=SimpleNamespace(name=model),
        training=SimpleNamespace(seq_len=seq_len, local_batch_size=batch[0], global_batch_size=batch[1],
                                 steps=batch[2]),
        compile=SimpleNamespace(enable=compile_))


@pytest.mark.parametrize("kwargs,match", [
    (dict(case="b6"), "unknown SFU case"),
    (dict(variant="d2_safe"), "unknown SFU variant"),
    (dict(case="b5", variant="polynomial"), "unknown SFU variant"),
    (dict(case="b4"), "requires model.name='sfu_deepseek_v3'"),
    (dict(case="b3", seq_len=2048), "requires training.seq_len=4096"),
    (dict(case="b5", variant="d2_safe", seq_len=2048), "requires training.seq_len=4096"),
    (dict(case="b5", variant="d2_safe", compile_=True), "compile.enable=false"),
    (dict(case="b5", variant="d2_safe", batch=(2, 2, 80)), "local/global batch 1 and 80 steps"),
])
def test_job_config_checks(kwargs, match):
    with pytest.raises(ValueError, match=match):
        SFUReproConverter(_job(**kwargs), SimpleNamespace(tp=1))


def test_tensor_parallel_rejected_for_b1():
    with pytest.raises(ValueError, match="tensor_parallel_degree=1"):
        SFUReproConverter(_job(), SimpleNamespace(tp=2))


def test_accepts_valid_configs():
    for kwargs in (dict(), dict(case="b2", variant="polynomial"), dict(case="b4", model="sfu_deepseek_v3"),
                   dict(case="b5", variant="d2_safe")):
        SFUReproConverter(_job(**kwargs), SimpleNamespace(tp=1))
    assert JobConfig().sfu == SFUConfig()


def test_module_recognition():
    m = Transformer(dim=64, hidden=128)
    assert sum(is_llama_feed_forward(x) for x in m.modules()) == 2
    assert sum(is_llama_attention(x) for x in m.modules()) == 2
    assert is_grouped_experts(GroupedExperts(16, 32, 4))
