"""Every BASELINE configuration at its own full shape, bit for bit against
the CPU oracle, through the C ABI; and element counts past 2^31 for the
unary and packed SwiGLU paths (reference
autonumerics_zero/spline_ops/test_spline_ops.py:207-235).

A unary 16-bit program is a function of the input's 16 bits, so at full
size (C2: 117M elements, C3: 2^29) the expected output is the oracle's
65,536-entry table gathered on the device by the input bits; backward
kernels (grad_out times the derivative program, one rounding) compare
against that table times grad_out rounded once, which is the oracle's own
definition of the product (the product of two 16-bit values is exact in
FP32).  C4, C5 exp2 and C5 RoPE are small enough for the oracle to evaluate
directly (a few seconds of CPU)."""

import ctypes

import numpy as np
import pytest
import torch

from test_gpu_parity import _host, assert_bits_equal

pytestmark = pytest.mark.gpu


def _table(oracle, fn, fmt, cuda):
    """The oracle's output for all 65,536 input patterns, on the device."""
    t = fn(oracle.all_bits())
    return torch.from_numpy(t.astype(np.uint16).view(np.int16)).to(cuda)


def _gather(table, x):
    return table[x.reshape(-1).view(torch.int16).long() & 0xFFFF]


def _assert_equal16(got, want, what):
    got = got.reshape(-1).view(torch.int16)
    want = want.reshape(-1).view(torch.int16)
    bad = got != want
    if bool(bad.any()):
        idx = torch.nonzero(bad)[:8].reshape(-1).tolist()
        raise AssertionError(f"{what}: {int(bad.sum())} of {got.numel()} differ; first at {idx}: "
                             f"got {[hex(int(got[i]) & 0xFFFF) for i in idx]} "
                             f"want {[hex(int(want[i]) & 0xFFFF) for i in idx]}")


def test_c2_silu_fp16_full(capi, oracle, cuda):
    """C2: B1 SiLU D3 FP16 on [8192, 14336] N(0, 2^2)
    gate activations, forward and backward (grad_out * SiLU'(x))."""
    print("C2 SiLU FP16 [8192, 14336]", flush=True)
    g = torch.Generator(device=cuda).manual_seed(0)
    x = (torch.randn(8192, 14336, device=cuda, generator=g) * 2).half()
    y = torch.empty_like(x)
    capi.call("launch_swish_fwd_d3_kernel", y, x, x.numel())
    fwd = _table(oracle, lambda b: oracle.activation("swish", oracle.FWD, 3, "f16", b), "f16", cuda)
    torch.cuda.synchronize()
    _assert_equal16(y, _gather(fwd, x), "C2 SiLU D3 fwd")
    go = torch.randn(8192, 14336, device=cuda, generator=g).half()
    gi = torch.empty_like(x)
    capi.call("launch_swish_bwd_d3_kernel", gi, go, x, x.numel())
    der = _table(oracle, lambda b: oracle.activation("swish", oracle.BWD, 3, "f16", b), "f16", cuda)
    torch.cuda.synchronize()
    want = (go.float().reshape(-1) * _gather(der, x).view(torch.float16).float()).half()
    _assert_equal16(gi, want, "C2 SiLU D3 bwd")


def _c3_scores(cuda):
    g = torch.Generator(device=cuda).manual_seed(0)
    shape = (4, 32, 2048, 2048)
    s = torch.randn(shape, device=cuda, generator=g) * 15
    mask = torch.rand(shape, device=cuda, generator=g) < 0.01
    sign = torch.where(torch.rand(shape, device=cuda, generator=g) < 0.5, -200.0, 200.0)
    return torch.where(mask, sign, s).to(torch.bfloat16)


def test_c3_softcap_full(capi, oracle, cuda):
    """C3: B2 softcap cap 30 on BF16 [4, 32, 2048,
    2048], N(0, 15^2) with 1 % outliers at +-200; forward and backward."""
    print("C3 softcap [4, 32, 2048, 2048]", flush=True)
    sc = _c3_scores(cuda)
    n = sc.numel()
    y = torch.empty_like(sc)
    assert capi.launch_softcap_tanh_d4_bf16(capi.ptr(y), capi.ptr(sc), ctypes.c_int64(n), ctypes.c_float(30.0),
                                            capi.stream()) == 0
    fwd = _table(oracle, lambda b: oracle.softcap_fwd_bf16(b, 30.0), "bf16", cuda)
    torch.cuda.synchronize()
    _assert_equal16(y, _gather(fwd, sc), "C3 softcap fwd")
    go = torch.randn(sc.shape, device=cuda, generator=torch.Generator(device=cuda).manual_seed(1)).bfloat16()
    gs = torch.empty_like(sc)
    assert capi.launch_softcap_tanh_d4_bwd_bf16(capi.ptr(gs), capi.ptr(go), capi.ptr(sc), ctypes.c_int64(n),
                                                ctypes.c_float(30.0), capi.stream()) == 0
    ones = np.full(65536, 0x3F80, dtype=np.uint16)
    der = _table(oracle, lambda b: oracle.softcap_bwd_bf16(ones, b, 30.0), "bf16", cuda)
    torch.cuda.synchronize()
    want = (go.float().reshape(-1) * _gather(der, sc).view(torch.bfloat16).float()).bfloat16()
    _assert_equal16(gs, want, "C3 softcap bwd")


def test_c4_routed_swiglu_full(capi, oracle, cuda):
    """C4: 64 experts with Zipf(1.1) token counts
    (numpy default_rng(0), 8192 tokens), H = 2048, N(0, 1) gate / up;
    SwiGLU D3 BF16 forward and backward on the separate and the packed
    [rows, 2H] layouts."""
    p = np.arange(1, 65, dtype=np.float64) ** -1.1
    counts = np.random.default_rng(0).multinomial(64 * 128, p / p.sum())
    rows, h = int(counts.sum()), 2048
    print(f"C4 SwiGLU rows {rows} (max expert {counts.max()}) H {h}", flush=True)
    g = torch.Generator().manual_seed(4)
    gate, up, go = (torch.randn(rows, h, generator=g).bfloat16() for _ in range(3))
    bits = [t.view(torch.int16).numpy().view(np.uint16).reshape(-1) for t in (gate, up, go)]
    gd, ud, god = gate.to(cuda), up.to(cuda), go.to(cuda)
    n = rows * h
    out = torch.empty_like(gd)
    gg, gu = torch.empty_like(gd), torch.empty_like(gd)
    capi.call("launch_swish_mul_fwd_d3_kernel_bf16", out, gd, ud, n)
    capi.call("launch_swish_mul_bwd_d3_kernel_bf16", gg, gu, god, gd, ud, n)
    packed = torch.cat((gd, ud), -1)
    out_p = torch.empty_like(gd)
    grad_p = torch.empty_like(packed)
    capi.call("launch_swish_mul_packed_fwd_d3_kernel_bf16", out_p, packed, rows, h)
    capi.call("launch_swish_mul_packed_bwd_d3_kernel_bf16", grad_p, god, packed, rows, h)
    torch.cuda.synchronize()
    want = oracle.swish_mul_fwd(3, "bf16", bits[0], bits[1])
    want_gg, want_gu = oracle.swish_mul_bwd(3, "bf16", bits[2], bits[0], bits[1])
    assert_bits_equal(_host(out).reshape(-1), want, "bf16", "C4 fwd separate")
    assert_bits_equal(_host(out_p).reshape(-1), want, "bf16", "C4 fwd packed")
    assert_bits_equal(_host(gg).reshape(-1), want_gg, "bf16", "C4 bwd grad_gate separate")
    assert_bits_equal(_host(gu).reshape(-1), want_gu, "bf16", "C4 bwd grad_up separate")
    gp = _host(grad_p).reshape(rows, 2 * h)
    assert_bits_equal(np.ascontiguousarray(gp[:, :h]).reshape(-1), want_gg, "bf16", "C4 bwd grad_gate packed")
    assert_bits_equal(np.ascontiguousarray(gp[:, h:]).reshape(-1), want_gu, "bf16", "C4 bwd grad_up packed")


@pytest.mark.parametrize("kind,name", [(0, "d2"), (1, "d3"), (2, "pwl2"), (3, "pwl2_safe"), (4, "pwl2_safe_f16"),
                                       (5, "pwl1_safe"), (6, "pwl1_safe_f16"), (7, "pwl2_safe_bf16"),
                                       (8, "d2_safe_noclamp"), (9, "d2_safe_f16"), (10, "d2_safe_bf16"),
                                       (11, "pwl2_f16")])
def test_c5_exp2_full(capi, oracle, cuda, kind, name):
    """C5 B5: exp2 of FP32 logits [4, 32, 4096, 128]
    N(0, 4^2) minus the row max, BF16 out, for every FA4 exp2 backend (the
    logits stay far above the -126 clamp of the hinges)."""
    print(f"C5 exp2 {name} [4, 32, 4096, 128]", flush=True)
    g = torch.Generator(device=cuda).manual_seed(5)
    lg = torch.randn(4, 32, 4096, 128, device=cuda, generator=g) * 4
    x = lg - lg.amax(-1, keepdim=True)
    y = torch.empty(x.shape, dtype=torch.bfloat16, device=cuda)
    capi.call(f"launch_exp2_{name}_f32_bf16", y, x, x.numel())
    torch.cuda.synchronize()
    assert_bits_equal(_host(y).reshape(-1), oracle.exp2(kind, x.cpu().numpy().reshape(-1), True), "bf16",
                      f"C5 exp2 {name}")


def test_c5_rope_full(capi, oracle, cuda):
    """C5 RoPE: BF16 Q, K [4, 4096, 32, 128], theta 500000, positions
    0..4095, fused half-turn D5/D6 rotation, outputs [B, H, S, D]."""
    print("C5 RoPE [4, 4096, 32, 128]", flush=True)
    b, s, h, d = 4, 4096, 32, 128
    g = torch.Generator().manual_seed(6)
    q = torch.randn(b, s, h, d, generator=g).bfloat16()
    k = torch.randn(b, s, h, d, generator=g).bfloat16()
    inc = oracle.rope_phase_increments(d, 500000.0)
    qo = torch.empty(b, h, s, d, dtype=torch.bfloat16, device=cuda)
    ko = torch.empty_like(qo)
    capi.call("launch_rope_apply_fixed_half_turn_d5_d6_bf16", qo, ko, q.to(cuda), k.to(cuda),
              torch.from_numpy(inc).to(cuda), b, s, h, h, d)
    torch.cuda.synchronize()
    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)
    want_q, want_k = oracle.rope_apply("bf16", bits(q), bits(k), inc)
    assert_bits_equal(_host(qo).reshape(-1), want_q.reshape(-1), "bf16", "C5 RoPE q")
    assert_bits_equal(_host(ko).reshape(-1), want_k.reshape(-1), "bf16", "C5 RoPE k")


def test_unary_past_2_31_elements(capi, oracle, cuda):
    """2^31 + 40 BF16 elements (4 GiB in, 4 GiB out) cycling through every
    bit pattern: the whole output against the oracle's table, in chunks."""
    n = (1 << 31) + 40
    print(f"unary sigmoid D3 BF16, {n} elements", flush=True)
    x = torch.empty(n, dtype=torch.int16, device=cuda)
    step = 1 << 28
    for start in range(0, n, step):
        stop = min(n, start + step)
        x[start:stop] = torch.arange(start, stop, dtype=torch.int64, device=cuda).to(torch.int16)
    x = x.view(torch.bfloat16)
    y = torch.empty_like(x)
    capi.call("launch_sigmoid_fwd_d3_kernel_bf16", y, x, n)
    table = _table(oracle, lambda b: oracle.activation("sigmoid", oracle.FWD, 3, "bf16", b), "bf16", cuda)
    torch.cuda.synchronize()
    for start in range(0, n, step):
        stop = min(n, start + step)
        _assert_equal16(y[start:stop], _gather(table, x[start:stop]), f"sigmoid D3 past 2^31 [{start}:{stop}]")


@pytest.mark.parametrize("hidden", [512, 768])
def test_packed_swiglu_past_2_31_elements(capi, oracle, cuda, hidden):
    """Packed [rows, 2H] with rows * 2H just past 2^31 elements (the
    reference's row-offset boundary test): forward, and for H = 768 the
    backward, on the rows around the boundary against the oracle."""
    boundary = (1 << 31) // (2 * hidden)
    rows = boundary + 8
    print(f"packed SwiGLU H {hidden}, rows {rows}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(hidden)
    packed = torch.randn(rows, 2 * hidden, device=cuda, generator=g).bfloat16()
    out = torch.empty(rows, hidden, dtype=torch.bfloat16, device=cuda)
    capi.call("launch_swish_mul_packed_fwd_d3_kernel_bf16", out, packed, rows, hidden)
    probe = torch.tensor([0, 1, boundary - 1, boundary, boundary + 1, rows - 1], device=cuda)
    torch.cuda.synchronize()
    pr = _host(packed.index_select(0, probe).contiguous())
    gate, up = np.ascontiguousarray(pr[:, :hidden]), np.ascontiguousarray(pr[:, hidden:])
    assert_bits_equal(_host(out.index_select(0, probe).contiguous()).reshape(-1),
                      oracle.swish_mul_fwd(3, "bf16", gate.reshape(-1), up.reshape(-1)), "bf16",
                      f"packed fwd H={hidden} past 2^31")
    del out
    if hidden == 768:
        go = torch.randn(rows, hidden, device=cuda, generator=g).bfloat16()
        grad = torch.empty_like(packed)
        capi.call("launch_swish_mul_packed_bwd_d3_kernel_bf16", grad, go, packed, rows, hidden)
        torch.cuda.synchronize()
        gr = _host(grad.index_select(0, probe).contiguous())
        want_gg, want_gu = oracle.swish_mul_bwd(3, "bf16", _host(go.index_select(0, probe).contiguous()).reshape(-1),
                                                gate.reshape(-1), up.reshape(-1))
        assert_bits_equal(np.ascontiguousarray(gr[:, :hidden]).reshape(-1), want_gg, "bf16",
                          "packed bwd grad_gate past 2^31")
        assert_bits_equal(np.ascontiguousarray(gr[:, hidden:]).reshape(-1), want_gu, "bf16",
                          "packed bwd grad_up past 2^31")
