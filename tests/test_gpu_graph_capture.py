"""HIP-graph capture of the drop-in ops, forward and backward.

The reference's launchers are graph-capture-safe: they launch on the current
stream, allocate nothing themselves and never synchronise
(autonumerics_zero/spline_ops/spline_ops.cpp:314-323 syncs only under
SPLINE_OPS_SYNC_DEBUG).  This build's launchers keep that contract, so a
torch.cuda.CUDAGraph can hold the forward and derivative launches of every
hot-path family.  The graph is replayed several times with new inputs
copied in eagerly between the replays (and eager launches of the same ops in
between), and every replay must equal the eager result on the same inputs
bit for bit."""

import pytest
import torch

pytestmark = pytest.mark.gpu

S_ATTN = 256  # attention sequence length (a multiple of 128)
S_RAGGED = 200  # and one that is not


def _shifted(logits: torch.Tensor) -> torch.Tensor:
    """Logits minus their row maximum (the B5 softmax exponent), on the host:
    the graph holds only this build's launches and torch's own copies."""
    return logits - logits.amax(-1, keepdim=True)


def _inputs(seed: int) -> dict:
    g = torch.Generator().manual_seed(seed)
    n = (1 << 16) + 5  # ragged: exercises the tail path inside the graph
    dims = torch.arange(0, 128, 2, dtype=torch.float64)
    omega = 500000.0 ** (-dims / 128)
    inc = torch.round(omega * 2.0 ** 32 / (2 * torch.pi)).to(torch.int64).to(torch.int32)
    return {
        "x16": (torch.randn(n, generator=g) * 4).to(torch.float16),
        "xb": (torch.randn(n, generator=g) * 4).to(torch.bfloat16),
        "scores": (torch.randn(n, generator=g) * 15).to(torch.bfloat16),
        "b3": (torch.rand(n, generator=g) * 32 - 16).to(torch.bfloat16),
        "logits": _shifted(torch.randn(8, 512, generator=g) * 4),
        "packed": torch.randn(24, 2 * 520, generator=g).to(torch.bfloat16),
        "rq": torch.randn(1, 64, 4, 128, generator=g).to(torch.bfloat16),
        "rk": torch.randn(1, 64, 2, 128, generator=g).to(torch.bfloat16),
        "inc": inc,
        "q": torch.randn(1, S_ATTN, 4, 128, generator=g).to(torch.bfloat16),
        "k": torch.randn(1, S_ATTN, 2, 128, generator=g).to(torch.bfloat16),
        "v": torch.randn(1, S_ATTN, 2, 128, generator=g).to(torch.bfloat16),
        "dout": torch.randn(1, S_ATTN, 4, 128, generator=g).to(torch.bfloat16),
        # a length that is not a multiple of 128 (the ragged kernels)
        "q2": torch.randn(1, S_RAGGED, 4, 128, generator=g).to(torch.bfloat16),
        "k2": torch.randn(1, S_RAGGED, 2, 128, generator=g).to(torch.bfloat16),
        "v2": torch.randn(1, S_RAGGED, 2, 128, generator=g).to(torch.bfloat16),
        "dout2": torch.randn(1, S_RAGGED, 4, 128, generator=g).to(torch.bfloat16),
        "gx": torch.randn(n, generator=g).to(torch.bfloat16),
        "gpacked": torch.randn(24, 520, generator=g).to(torch.bfloat16),
    }


def _run(spline_ops, t: dict) -> list:
    """One launch of each family; returns every output tensor."""
    outs = [
        spline_ops.sigmoid_fwd_variant(t["x16"], 3, 0),
        spline_ops.tanh_fwd_variant(t["xb"], 4, 0),
        spline_ops.swish_fwd_variant(t["xb"], 3, 1),
        spline_ops.softcap_tanh_fwd_bf16(t["scores"], 30.0),
        spline_ops.exp2_d2_f32_to_bf16(t["logits"]),
        spline_ops.swish_mul_packed_fwd_variant(t["packed"], 3, 0),
    ]
    outs += list(spline_ops.flash_sigmoid_direct_d3_d4_bf16(t["b3"]))
    outs += list(spline_ops.rope_apply_fixed_half_turn_d5_d6_bf16(t["rq"], t["rk"], t["inc"]))
    # softmax with the routed D2 exp2 (B5 forward schedule) and the B2 softcap
    outs += list(spline_ops.flash_attn_fwd_bf16(t["q"], t["k"], t["v"], 1, 12, True, 128 ** -0.5))
    outs += list(spline_ops.flash_attn_fwd_bf16(t["q"], t["k"], t["v"], 4, 4, False, 128 ** -0.5, 30.0))
    outs += list(spline_ops.flash_attn_fwd_bf16(t["q2"], t["k2"], t["v2"], 1, 12, True, 128 ** -0.5))
    return outs


def _run_backward(spline_ops, t: dict) -> list:
    """The derivative launches: activation and SwiGLU programs, the softcap
    gradient, and the attention backward (delta, dK/dV with the grouped-head
    partials, their reduction, dQ) behind its own forward."""
    outs = [
        spline_ops.sigmoid_bwd_variant(t["gx"], t["xb"], 4, 0),
        spline_ops.softcap_tanh_bwd_bf16(t["gx"], t["scores"], 30.0),
        spline_ops.swish_mul_packed_bwd_variant(t["gpacked"], t["packed"], 3, 0),
    ]
    scale = 128 ** -0.5
    out, lse = spline_ops.flash_attn_fwd_bf16(t["q"], t["k"], t["v"], 0, 4, True, scale)
    outs += list(spline_ops.flash_attn_bwd_bf16(t["q"], t["k"], t["v"], out, t["dout"], lse, 0, 0, 0, True,
                                                scale, 0.0, 0.0))
    out2, lse2 = spline_ops.flash_attn_fwd_bf16(t["q2"], t["k2"], t["v2"], 0, 4, False, scale)
    outs += list(spline_ops.flash_attn_bwd_bf16(t["q2"], t["k2"], t["v2"], out2, t["dout2"], lse2, 0, 0, 0, False,
                                                scale, 0.0, 0.0))
    return outs


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


def _check_replays(run):
    import spline_ops

    static = {k: v.to("cuda:0") for k, v in _inputs(0).items()}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run(spline_ops, static)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = run(spline_ops, static)

    for seed in (1, 2, 3):
        fresh = _inputs(seed)
        for name, tensor in static.items():
            tensor.copy_(fresh[name])
        graph.replay()
        torch.cuda.synchronize()
        eager = run(spline_ops, static)
        torch.cuda.synchronize()
        assert len(captured) == len(eager)
        for i, (a, b) in enumerate(zip(captured, eager)):
            assert a.shape == b.shape and a.dtype == b.dtype, (seed, i)
            assert torch.equal(_bits(a), _bits(b)), f"replay {seed}: output {i} differs from eager"


@pytest.mark.parametrize("sync_debug", [False, True])
def test_graph_replays_match_eager(cuda, monkeypatch, sync_debug):
    # SPLINE_OPS_SYNC_DEBUG synchronises after every launch except while the
    # stream is being captured, so capture works with it on too
    if sync_debug:
        monkeypatch.setenv("SPLINE_OPS_SYNC_DEBUG", "1")
    _check_replays(_run)


def test_backward_graph_replays_match_eager(cuda):
    _check_replays(_run_backward)
