"""GPU parity of the FP32 and quarter-turn sin/cos programs, every compute
probe, the RoPE quarter-turn / LUT / native tables (and their probes) and
the cached-table RoPE apply, against the CPU oracle bit for bit through the
C ABI; native (hardware sin/cos) entry points against float64 within a
stated bound; and the drop-in pybind surface for the same programs."""

import math

import numpy as np
import pytest
import torch

from test_gpu_parity import _host, assert_bits_equal

pytestmark = pytest.mark.gpu

F32_TABLES = [
    ("d3_d4", "SC32_D3D4"), ("d3_d4_magic_bias", "SC32_D3D4_SHIFT"), ("d5_d4", "SC32_D5D4"),
    ("d7_d6", "SC32_D7D6"), ("d5_d4_half_turn_ls", "SC32_HALF_D5D4_LS"),
    ("d5_d4_half_turn_sollya", "SC32_HALF_D5D4_SOLLYA"),
    ("d5_d4_half_turn_sollya_fast", "SC32_HALF_D5D4_SOLLYA_FAST"), ("d3_d4_cycle", "SC32_CYCLE"),
]

# (entry stem, oracle 16-bit program id, output format)
TABLES16 = [
    ("sincos_d3_d4_bf16", 8, "bf16"),
    ("sincos_d3_d4_quarter_turn_bf16", 7, "bf16"),
    ("sincos_d3_d4_half_turn_bf16", 0, "bf16"),
    ("sincos_d5_d6_half_turn_bf16", 1, "bf16"),
    ("sincos_d5_d4_half_turn_fp16_bf16", 3, "bf16"),
    ("sincos_d3_d4_quarter_turn_fp16", 6, "f16"),
    ("sincos_d3_d4_half_turn_fp16", 2, "f16"),
    ("sincos_d5_d4_half_turn_fp16", 3, "f16"),
    ("sincos_d5_d6_half_turn_fp16", 4, "f16"),
    ("sincos_d7_d6_half_turn_fp16", 5, "f16"),
]


def _angles(ragged, n_random=1 << 18):
    rng = np.random.default_rng(3)
    # special angles first: the length is cut to whole vectors at the end
    a = np.concatenate([
        np.array([0.0, -0.0, 1e-30, -1e-30, 1e-40, 4095.0, 3e7, -1e10,
                  np.inf, -np.inf, np.nan, -np.nan, 3.4e38, -3.4e38], dtype=np.float32),
        (np.arange(-16, 17) * (math.pi / 4)).astype(np.float32),
        rng.uniform(-200.0, 200.0, n_random).astype(np.float32),
        rng.uniform(-2e5, 2e5, 4096).astype(np.float32),
        np.linspace(-4 * math.pi, 4 * math.pi, 8197, dtype=np.float32),
    ])
    n = (a.size // 8) * 8
    return np.ascontiguousarray(a[: n - 3] if ragged else a[:n])


def _f32_bits_equal(got: np.ndarray, want: np.ndarray, what: str):
    g = got.view(np.uint32)
    w = want.view(np.uint32)
    nan = np.isnan(got) & np.isnan(want)
    bad = (g != w) & ~nan
    if bad.any():
        idx = np.flatnonzero(bad)[:8]
        raise AssertionError(f"{what}: {bad.sum()} of {g.size} differ; first at {idx.tolist()}: "
                             f"got {got[idx].tolist()} want {want[idx].tolist()}")


@pytest.mark.parametrize("ragged", [False, True])
@pytest.mark.parametrize("stem,prog", F32_TABLES)
def test_f32_tables(capi, oracle, cuda, stem, prog, ragged):
    a = _angles(ragged)
    ad = torch.from_numpy(a).to(cuda)
    out = torch.empty(2, a.size, dtype=torch.float32, device=cuda)
    capi.call(f"launch_sincos_{stem}_f32", out, ad, a.size)
    torch.cuda.synchronize()
    want_c, want_s = oracle.sincos_f32(getattr(oracle, prog), a)
    got = out.cpu().numpy()
    _f32_bits_equal(got[0], want_c, stem + " cos")
    _f32_bits_equal(got[1], want_s, stem + " sin")


@pytest.mark.parametrize("stem,prog", F32_TABLES)
def test_f32_compute_probes(capi, oracle, cuda, stem, prog):
    a = np.random.default_rng(7).uniform(-100.0, 100.0, 8192 * 4 + 5).astype(np.float32)
    ad = torch.from_numpy(a).to(cuda)
    out = torch.empty(2, a.size, dtype=torch.float32, device=cuda)
    capi.call(f"launch_sincos_{stem}_compute_f32", out, ad, a.size, 7)
    torch.cuda.synchronize()
    want_c, want_s = oracle.sincos_f32(getattr(oracle, prog), a, iterations=7)
    got = out.cpu().numpy()
    _f32_bits_equal(got[0], want_c, stem + " compute cos")
    _f32_bits_equal(got[1], want_s, stem + " compute sin")


@pytest.mark.parametrize("ragged", [False, True])
@pytest.mark.parametrize("stem,prog,fmt", TABLES16)
def test_16bit_tables(capi, oracle, cuda, stem, prog, fmt, ragged):
    a = _angles(ragged)
    ad = torch.from_numpy(a).to(cuda)
    dt = torch.bfloat16 if fmt == "bf16" else torch.float16
    out = torch.empty(2, a.size, dtype=dt, device=cuda)
    capi.call(f"launch_{stem}", out, ad, a.size)
    torch.cuda.synchronize()
    want_c, want_s = oracle.sincos16(prog, a, out_fmt=fmt)
    got = _host(out.reshape(-1)).reshape(2, -1)
    assert_bits_equal(got[0], want_c, fmt, stem + " cos")
    assert_bits_equal(got[1], want_s, fmt, stem + " sin")


@pytest.mark.parametrize("n", [8192 * 4, 8192 * 4 + 6])
@pytest.mark.parametrize("stem,prog,fmt", TABLES16)
def test_16bit_compute_probes(capi, oracle, cuda, stem, prog, fmt, n):
    a = np.random.default_rng(prog).uniform(-100.0, 100.0, n).astype(np.float32)
    ad = torch.from_numpy(a).to(cuda)
    dt = torch.bfloat16 if fmt == "bf16" else torch.float16
    out = torch.empty(2, a.size, dtype=dt, device=cuda)
    capi.call(f"launch_{stem}_compute", out, ad, a.size, 6)
    torch.cuda.synchronize()
    want_c, want_s = oracle.sincos16(prog, a, out_fmt=fmt, iterations=6)
    got = _host(out.reshape(-1)).reshape(2, -1)
    assert_bits_equal(got[0], want_c, fmt, stem + " compute cos")
    assert_bits_equal(got[1], want_s, fmt, stem + " compute sin")


@pytest.mark.parametrize("name,dt,tol", [("launch_sincos_native_f32", torch.float32, 2e-5),
                                         ("launch_sincos_native_bf16", torch.bfloat16, 2 ** -8 + 2e-5),
                                         ("launch_sincos_native_fp16", torch.float16, 2 ** -11 + 2e-5)])
def test_native_tables_and_probes(capi, cuda, name, dt, tol):
    a = torch.linspace(-50, 50, (1 << 16) + 4, device=cuda)
    a64 = a.double().cpu()
    out = torch.empty(2, a.numel(), dtype=dt, device=cuda)
    capi.call(name, out, a, a.numel())
    torch.cuda.synchronize()
    assert float((out[0].double().cpu() - torch.cos(a64)).abs().max()) < tol
    assert float((out[1].double().cpu() - torch.sin(a64)).abs().max()) < tol
    probe = name.replace("_f32", "") + ("_compute_f32" if dt == torch.float32 else "_compute")
    capi.call(probe, out, a, a.numel(), 3)
    torch.cuda.synchronize()
    p = a.float().cpu()
    ref_c = torch.zeros_like(a64)
    ref_s = torch.zeros_like(a64)
    for _ in range(3):
        ref_c += torch.cos(p.double())
        ref_s += torch.sin(p.double())
        p = (p.double() * 0.999999940395355224609375 + 0.0001220703125).float()
    sum_tol = 3 * tol + (3 * 2 ** -7 if dt == torch.bfloat16 else 3 * 2 ** -10 if dt == torch.float16 else 1e-6)
    assert float((out[0].double().cpu() - ref_c).abs().max()) < sum_tol
    assert float((out[1].double().cpu() - ref_s).abs().max()) < sum_tol


# ---- RoPE ------------------------------------------------------------------------

def _lut():
    t = 2 * math.pi * np.arange(128) / 128
    return np.stack((np.sin(t), np.cos(t)), -1).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("iterations", [0, 5])
@pytest.mark.parametrize("kind,stem", [(0, "fixed_half_turn_d5_d6"), (1, "fixed_d3_d4"), (2, "fixed_lut")])
def test_rope_tables(capi, oracle, cuda, kind, stem, iterations):
    inc = oracle.rope_phase_increments(128, 500000.0)
    seq = 4096 + 3
    incd = torch.from_numpy(inc).to(cuda)
    out = torch.empty(2, seq, inc.size, dtype=torch.float16, device=cuda)
    lut = _lut()
    name = f"launch_rope_sincos_{stem}_fp16" + ("_compute" if iterations else "")
    args = [out, incd]
    if kind == 2:
        args.append(torch.from_numpy(lut.view(np.int16)).to(cuda))
    args += [seq, inc.size]
    if iterations:
        args.append(iterations)
    capi.call(name, *args)
    torch.cuda.synchronize()
    want = oracle.rope_table(kind, inc, seq, lut=lut, iterations=iterations)
    assert_bits_equal(_host(out.reshape(-1)), want.reshape(-1), "f16", name)


def test_rope_native_table_and_probe(capi, oracle, cuda):
    d, seq = 128, 2048
    dims = np.arange(0, d, 2, dtype=np.float64)
    freq = (500000.0 ** (-dims / d)).astype(np.float32)
    fd = torch.from_numpy(freq).to(cuda)
    out = torch.empty(2, seq, freq.size, dtype=torch.float16, device=cuda)
    capi.call("launch_rope_sincos_native_fp16", out, fd, seq, freq.size)
    torch.cuda.synchronize()
    ang = (np.arange(seq, dtype=np.float32)[:, None] * freq[None]).astype(np.float64)
    got = out.cpu().numpy().astype(np.float64)
    # __sinf scales to revolutions in FP32 first: up to 326 revolutions here,
    # so that product alone may be off by 2e-5 revolutions (1.2e-4 rad)
    tol = 2 ** -11 + 5e-4
    assert np.abs(got[0] - np.cos(ang)).max() < tol
    assert np.abs(got[1] - np.sin(ang)).max() < tol
    capi.call("launch_rope_sincos_native_fp16_compute", out, fd, seq, freq.size, 4)
    torch.cuda.synchronize()
    pos = np.arange(seq, dtype=np.float32)[:, None]
    ref = [sum(np.cos((pos + j).astype(np.float32) * freq[None]).astype(np.float64) for j in range(4)),
           sum(np.sin((pos + j).astype(np.float32) * freq[None]).astype(np.float64) for j in range(4))]
    got = out.cpu().numpy().astype(np.float64)
    assert np.abs(got[0] - ref[0]).max() < 4 * tol + 4 * 2 ** -9
    assert np.abs(got[1] - ref[1]).max() < 4 * tol + 4 * 2 ** -9


@pytest.mark.parametrize("shape", [(2, 64, 4, 2, 128), (1, 37, 9, 3, 64)])
def test_rope_apply_cached(capi, oracle, cuda, shape):
    b, s, hq, hk, d = shape
    g = torch.Generator().manual_seed(sum(shape))
    q = torch.randn(b, s, hq, d, generator=g).half()
    k = torch.randn(b, s, hk, d, generator=g).half()
    inc = oracle.rope_phase_increments(d, 500000.0)
    table = oracle.rope_table(1, inc, s)  # any FP16 table: the quarter-turn one
    td = torch.from_numpy(table.view(np.int16)).to(cuda)
    qo = torch.empty(b, hq, s, d, dtype=torch.float16, device=cuda)
    ko = torch.empty(b, hk, s, d, dtype=torch.float16, device=cuda)
    capi.call("launch_rope_apply_cached_fp16", qo, ko, q.to(cuda), k.to(cuda), td, b, s, hq, hk, d)
    torch.cuda.synchronize()
    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)
    want_q, want_k = oracle.rope_apply_cached(bits(q), bits(k), table)
    assert_bits_equal(_host(qo).reshape(-1), want_q.reshape(-1), "f16", f"cached q {shape}")
    assert_bits_equal(_host(ko).reshape(-1), want_k.reshape(-1), "f16", f"cached k {shape}")


# ---- pybind surface ---------------------------------------------------------------

def test_binding_sincos_family(spline_ops, oracle, cuda):
    a = torch.linspace(-30, 30, 4096, device=cuda).reshape(64, 64)
    out = spline_ops.sincos_d7_d6_f32(a)
    assert out.shape == (2, 64, 64) and out.dtype == torch.float32
    want_c, want_s = oracle.sincos_f32(oracle.SC32_D7D6, a.cpu().numpy().reshape(-1))
    _f32_bits_equal(out[0].cpu().numpy().reshape(-1), want_c, "binding d7_d6")
    _f32_bits_equal(out[1].cpu().numpy().reshape(-1), want_s, "binding d7_d6 sin")
    probe = spline_ops.sincos_d3_d4_quarter_turn_bf16_compute(a, 3)
    assert probe.shape == (2, 64, 64) and probe.dtype == torch.bfloat16
    wc, ws = oracle.sincos16(7, a.cpu().numpy().reshape(-1), iterations=3)
    assert_bits_equal(_host(probe[0].reshape(-1)), wc, "bf16", "binding probe cos")
    with pytest.raises(RuntimeError, match="even number of elements"):
        spline_ops.sincos_d3_d4_bf16(torch.zeros(3, device=cuda))
    with pytest.raises(RuntimeError, match="multiple of four elements"):
        spline_ops.sincos_d3_d4_half_turn_fp16_compute(torch.zeros(6, device=cuda), 2)
    with pytest.raises(RuntimeError, match="iterations must be positive"):
        spline_ops.sincos_d3_d4_compute_f32(torch.zeros(4, device=cuda), 0)
    with pytest.raises(RuntimeError, match="angles must be float32"):
        spline_ops.sincos_d5_d4_f32(torch.zeros(4, device=cuda, dtype=torch.float16))


def test_binding_rope_family(spline_ops, oracle, cuda):
    inc = torch.from_numpy(oracle.rope_phase_increments(64, 10000.0)).to(cuda)
    lut = torch.from_numpy(_lut().view(np.int16)).to(cuda).view(torch.float16)
    t = spline_ops.rope_sincos_fixed_lut_fp16(inc, lut, 100)
    assert t.shape == (2, 100, 32) and t.dtype == torch.float16
    want = oracle.rope_table(2, inc.cpu().numpy(), 100, lut=_lut())
    assert_bits_equal(_host(t.reshape(-1)), want.reshape(-1), "f16", "binding lut")
    tc = spline_ops.rope_sincos_fixed_d3_d4_fp16_compute(inc, 100, 3)
    want = oracle.rope_table(1, inc.cpu().numpy(), 100, iterations=3)
    assert_bits_equal(_host(tc.reshape(-1)), want.reshape(-1), "f16", "binding quarter probe")
    with pytest.raises(RuntimeError, match=r"phase_table must have shape \[128, 2\]"):
        spline_ops.rope_sincos_fixed_lut_fp16(inc, lut[:64], 10)
    with pytest.raises(RuntimeError, match="multiple of four elements"):
        spline_ops.rope_sincos_fixed_half_turn_d5_d6_fp16(inc[:6], 10)
    q = torch.randn(1, 16, 2, 64, device=cuda).half()
    k = torch.randn(1, 16, 1, 64, device=cuda).half()
    table = spline_ops.rope_sincos_fixed_half_turn_d5_d6_fp16(inc, 16)
    qc, kc = spline_ops.rope_apply_cached_fp16(q, k, table)
    qf, kf = spline_ops.rope_apply_fixed_half_turn_d5_d6_fp16(q, k, inc)
    assert torch.equal(qc, qf) and torch.equal(kc, kf)
    with pytest.raises(RuntimeError, match=r"rope_table must have shape \[2, sequence_length, head_dim / 2\]"):
        spline_ops.rope_apply_cached_fp16(q, k, table[:, :8].contiguous())
