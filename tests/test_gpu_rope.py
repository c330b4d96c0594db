"""GPU parity of the sin/cos programs and fused RoPE against the CPU oracle
(through the C ABI), and accuracy against a float64 RoPE reference."""

import math

import numpy as np
import pytest
import torch

from test_gpu_parity import _host, assert_bits_equal

pytestmark = pytest.mark.gpu

TABLES = [
    ("launch_sincos_d3_d4_half_turn_bf16", 0, "bf16"),
    ("launch_sincos_d5_d6_half_turn_bf16", 1, "bf16"),
    ("launch_sincos_d3_d4_half_turn_fp16", 2, "f16"),
    ("launch_sincos_d5_d4_half_turn_fp16", 3, "f16"),
    ("launch_sincos_d5_d6_half_turn_fp16", 4, "f16"),
    ("launch_sincos_d7_d6_half_turn_fp16", 5, "f16"),
    ("launch_sincos_d5_d4_half_turn_fp16_bf16", 3, "bf16"),
]


def _angles(ragged, n_random=1 << 18):
    rng = np.random.default_rng(2)
    # special angles first: the length is cut to whole vectors at the end
    a = np.concatenate([
        np.array([0.0, -0.0, 1e-30, math.pi / 2, math.pi, 4095.0, np.inf, -np.inf, np.nan, 3e7,
                  -1e10], dtype=np.float32),
        rng.uniform(-100.0, 100.0, n_random).astype(np.float32),
        np.linspace(-4 * math.pi, 4 * math.pi, 8197, dtype=np.float32),
        np.arange(4096, dtype=np.float32) * np.float32(0.0157),
    ])
    n = (a.size // 8) * 8
    return np.ascontiguousarray(a[: n - 3] if ragged else a[:n])


@pytest.mark.parametrize("ragged", [False, True])
@pytest.mark.parametrize("name,prog,out_fmt", TABLES)
def test_sincos_tables(capi, oracle, cuda, name, prog, out_fmt, ragged):
    a = _angles(ragged)
    ad = torch.from_numpy(a).to(cuda)
    dt = torch.bfloat16 if out_fmt == "bf16" else torch.float16
    out = torch.empty(2, a.size, dtype=dt, device=cuda)
    capi.call(name, out, ad, a.size)
    torch.cuda.synchronize()
    want_c, want_s = oracle.sincos(prog, a, out_fmt)
    got = _host(out.reshape(-1)).reshape(2, -1)
    assert_bits_equal(got[0], want_c, out_fmt, name + " cos")
    assert_bits_equal(got[1], want_s, out_fmt, name + " sin")


@pytest.mark.parametrize("name,fmt", [("launch_sincos_native_bf16", torch.bfloat16),
                                      ("launch_sincos_native_fp16", torch.float16)])
def test_sincos_native_baselines(capi, cuda, name, fmt):
    a = torch.linspace(-50, 50, 1 << 16, device=cuda)
    out = torch.empty(2, a.numel(), dtype=fmt, device=cuda)
    capi.call(name, out, a, a.numel())
    torch.cuda.synchronize()
    tol = 2 ** -8 if fmt == torch.bfloat16 else 2 ** -10
    assert float((out[0].float() - torch.cos(a)).abs().max()) < tol + 1e-4
    assert float((out[1].float() - torch.sin(a)).abs().max()) < tol + 1e-4


def test_rope_phase_table(capi, oracle, cuda):
    inc = oracle.rope_phase_increments(128, 500000.0)
    seq = 4096
    incd = torch.from_numpy(inc).to(cuda)
    out = torch.empty(2, seq, inc.size, dtype=torch.float16, device=cuda)
    capi.call("launch_rope_sincos_fixed_half_turn_d5_d6_fp16", out, incd, seq, inc.size)
    torch.cuda.synchronize()
    want = oracle.rope_sincos_table(inc, seq)
    assert_bits_equal(_host(out.reshape(-1)), want.reshape(-1), "f16", "rope table")


def _rope_inputs(fmt, b, s, hq, hk, d, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, s, hq, d, generator=g).to(fmt)
    k = torch.randn(b, s, hk, d, generator=g).to(fmt)
    return q, k


def _rope_reference(values, theta):
    """float64 angles, float32 rotation, transposed output
    (src/sfu_repro/rope/benchmark_cuda_fused_rope.py:71-97)."""
    b, s, h, d = values.shape
    dims = torch.arange(0, d, 2, dtype=torch.float64)
    freq = theta ** (-dims / d)
    ang = torch.arange(s, dtype=torch.float64)[:, None] * freq[None]
    cos = torch.cos(ang).float()[None, :, None, :]
    sin = torch.sin(ang).float()[None, :, None, :]
    pairs = values.float().reshape(b, s, h, d // 2, 2)
    e, o = pairs[..., 0], pairs[..., 1]
    rot = torch.stack((e * cos - o * sin, e * sin + o * cos), -1).flatten(-2)
    return rot.transpose(1, 2).contiguous()


@pytest.mark.parametrize("fmt,name", [(torch.float16, "fp16"), (torch.bfloat16, "bf16")])
@pytest.mark.parametrize("shape", [(2, 64, 4, 2, 128), (1, 37, 9, 3, 64), (1, 4096, 1, 1, 128),
                                   (3, 17, 2, 1, 8), (1, 33, 5, 5, 24), (1, 8, 16, 16, 256)])
def test_rope_apply_parity(capi, oracle, cuda, fmt, name, shape):
    b, s, hq, hk, d = shape
    q, k = _rope_inputs(fmt, b, s, hq, hk, d, seed=sum(shape))
    inc = oracle.rope_phase_increments(d, 500000.0)
    qd, kd, incd = q.to(cuda), k.to(cuda), torch.from_numpy(inc).to(cuda)
    qo = torch.empty(b, hq, s, d, dtype=fmt, device=cuda)
    ko = torch.empty(b, hk, s, d, dtype=fmt, device=cuda)
    capi.call(f"launch_rope_apply_fixed_half_turn_d5_d6_{name}", qo, ko, qd, kd, incd, b, s, hq, hk, d)
    torch.cuda.synchronize()
    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)
    want_q, want_k = oracle.rope_apply("f16" if name == "fp16" else "bf16", bits(q), bits(k), inc)
    ofmt = "f16" if name == "fp16" else "bf16"
    assert_bits_equal(_host(qo).reshape(-1), want_q.reshape(-1), ofmt, f"rope q {name} {shape}")
    assert_bits_equal(_host(ko).reshape(-1), want_k.reshape(-1), ofmt, f"rope k {name} {shape}")


@pytest.mark.parametrize("fmt", [torch.float16, torch.bfloat16])
def test_rope_accuracy_and_native(spline_ops, cuda, fmt):
    """BASELINE config 5 RoPE recipe at reduced batch: theta 500000,
    positions 0..4095, head_dim 128."""
    b, s, h, d = 1, 4096, 4, 128
    q, k = _rope_inputs(fmt, b, s, h, h, d, seed=9)
    dims = torch.arange(0, d, 2, dtype=torch.float64)
    freq = 500000.0 ** (-dims / d)
    inc = torch.round(freq * (2.0 ** 32) / (2 * math.pi)).to(torch.int64).to(torch.int32)
    tag = "fp16" if fmt == torch.float16 else "bf16"
    poly = getattr(spline_ops, f"rope_apply_fixed_half_turn_d5_d6_{tag}")
    nat = getattr(spline_ops, f"rope_apply_native_{tag}")
    qo, ko = poly(q.to(cuda), k.to(cuda), inc.to(cuda))
    qn, kn = nat(q.to(cuda), k.to(cuda), freq.float().to(cuda))
    ref_q, ref_k = _rope_reference(q, 500000.0), _rope_reference(k, 500000.0)
    scale = float(q.float().abs().max())
    out_ulp = 2 ** -8 if fmt == torch.bfloat16 else 2 ** -11
    for got, ref in ((qo, ref_q), (ko, ref_k), (qn, ref_q), (kn, ref_k)):
        err = float((got.float().cpu() - ref).abs().max())
        assert err < scale * (3e-3 + 2 * out_ulp), err
