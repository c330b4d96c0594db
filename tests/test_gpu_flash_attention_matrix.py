"""Forward parity of every fused-attention score mode at both head sizes,
with batched, grouped-query operands in FA4's layout: out (BF16) and, for
the softmax and softcap modes, the FP32 log-sum-exp, against the float32
CPU reference that evaluates the same score programs through the oracle.

Two sequences, eight query heads over two KV heads (four per group), S =
256: every block of the grid maps its own (batch, query head) to the right
KV head.  The B3 programs, fitted for S = 4096, run at that length.  The
backward of the programs not otherwise tested at head_dim 64 follows."""

import math

import pytest
import torch

from attention_reference import M, reference_fwd
from test_gpu_flash_attention_bwd import _close, _inputs, fwd

pytestmark = pytest.mark.gpu

MODES = [m for m in M if not m.startswith("sigmoid_b3")]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("mode", MODES)
def test_forward_matrix(capi, oracle, cuda, mode, d, causal):
    seed = 900 + 3 * M[mode] + d + int(causal)
    print(f"fwd {mode} d {d} causal {causal} seed {seed}", flush=True)
    q, k, v, _ = _inputs(2, 8, 2, 256, seed, qmul=6.0 if mode.startswith("softcap") else 1.0, d=d)
    scale = 1 / math.sqrt(d)
    out, lse = fwd(capi, cuda, q, k, v, mode, causal, scale, route=4)
    ref_out, ref_lse = reference_fwd(oracle, q, k, v, mode, causal, scale, 30.0, 4)
    got = out.cpu().float()
    assert torch.isfinite(got).all()
    ok, info = _close(got, ref_out, rel=1.5e-2)
    assert ok, ("out", mode, d, causal, info)
    if ref_lse is not None:
        # hardware modes: FP32 exponent sums; exp2 programs: the same programs
        # in the reference, given the same exponents (it follows the kernel's
        # running maximum), so only the dot products' rounding and the
        # summation order differ (measured up to 1.5e-3); the softcap D4
        # program: its BF16-rounded capped scores
        bound = (1e-3 if mode in ("softmax_native", "softcap_native") else 4e-3 if mode.startswith("softmax")
                 else 2e-2)
        err = (lse.cpu() - ref_lse).abs().max().item()
        assert err < bound, ("lse", mode, d, causal, err)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("mode", ["sigmoid_b3", "sigmoid_b3_d2"])
def test_forward_b3_programs_at_4096(capi, oracle, cuda, mode, d):
    print(f"fwd {mode} d {d} S 4096", flush=True)
    q, k, v, _ = _inputs(1, 4, 1, 4096, 950 + d + M[mode], d=d)
    scale = 1 / math.sqrt(d)
    out, _ = fwd(capi, cuda, q, k, v, mode, True, scale)
    ref_out, _ = reference_fwd(oracle, q, k, v, mode, True, scale)
    got = out.cpu().float()
    assert torch.isfinite(got).all()
    ok, info = _close(got, ref_out, rel=1.5e-2)
    assert ok, (mode, d, info)


# backward at head_dim 64 for the programs that test_head_dim_64
# (test_gpu_flash_attention_bwd.py) does not reach: routed D3 / PWL2,
# hardware softcap, the STE and 1 - T^2 softcap derivatives, biased sigmoid
# programs and the B3 programs; batched and grouped like the forward matrix
BWD64 = [("softmax_d3", 0, 12), ("softmax_pwl2", 0, 10), ("softcap_native", 0, 0), ("softcap_d4", 2, 0),
         ("softcap_d4", 3, 0), ("sigmoid_d3", 0, 0), ("sigmoid_d5", 0, 0)]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("mode,grad,route", BWD64)
def test_backward_head_dim_64_grouped(capi, oracle, cuda, mode, grad, route, causal):
    from attention_reference import default_bias, reference_bwd
    from test_gpu_flash_attention_bwd import bwd

    seed = 1000 + 5 * M[mode] + grad + route + int(causal)
    print(f"bwd d64 {mode} grad {grad} route {route} causal {causal} seed {seed}", flush=True)
    q, k, v, do = _inputs(2, 8, 2, 256, seed, qmul=6.0 if mode.startswith("softcap") else 1.0, d=64)
    scale = 1 / math.sqrt(64)
    out, lse = fwd(capi, cuda, q, k, v, mode, causal, scale, route=route if route else 4)
    dq, dk, dv, _ = bwd(capi, cuda, q, k, v, out, do, lse, mode, grad, causal, scale, route=route)
    rq, rk, rv = reference_bwd(oracle, q, k, v, out, do, lse, mode, grad, causal, scale, 30.0, route,
                               default_bias(mode, 256))
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert torch.isfinite(got).all(), name
        ok, info = _close(got, ref)
        assert ok, (mode, grad, route, causal, name, info)


@pytest.mark.parametrize("mode,grad", [("sigmoid_b3", 4), ("sigmoid_b3", 5), ("sigmoid_b3_d2", 0)])
def test_backward_b3_programs_head_dim_64(capi, oracle, cuda, mode, grad):
    from attention_reference import reference_bwd
    from test_gpu_flash_attention_bwd import bwd

    print(f"bwd d64 {mode} grad {grad} S 4096", flush=True)
    q, k, v, do = _inputs(1, 2, 1, 4096, 1100 + grad + M[mode], d=64)
    scale = 1 / math.sqrt(64)
    out, lse = fwd(capi, cuda, q, k, v, mode, True, scale)
    dq, dk, dv, _ = bwd(capi, cuda, q, k, v, out, do, lse, mode, grad, True, scale)
    rq, rk, rv = reference_bwd(oracle, q, k, v, out, do, lse, mode, grad, True, scale, 30.0, 0, 0.0)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert torch.isfinite(got).all(), name
        ok, info = _close(got, ref)
        assert ok, (mode, grad, name, info)


@pytest.mark.parametrize("mode,mode_id,grad,cap", [("softmax_native", 0, 0, 0.0), ("softmax_d2", 1, 0, 0.0),
                                                   ("softcap_d4", 4, 1, 30.0), ("sigmoid_b3", 6, 5, 0.0)])
def test_fused_qkv_views_match_contiguous(spline_ops, cuda, mode, mode_id, grad, cap):
    """Q, K and V as views of one fused [B, S, 3, H, D] projection (head
    stride D, sequence stride 3 H D): the kernels take any element strides
    with a contiguous head dimension, so the result must equal the
    contiguous operands' bit for bit, forward and backward."""
    s = 4096 if mode == "sigmoid_b3" else 384
    g = torch.Generator().manual_seed(77 + mode_id)
    qkv = (torch.randn(1, s, 3, 4, 128, generator=g) * (4.0 if cap else 1.0)).bfloat16().to(cuda)
    do = torch.randn(1, s, 4, 128, generator=g).bfloat16().to(cuda)
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    assert not q.is_contiguous() and q.stride() == (s * 3 * 4 * 128, 3 * 4 * 128, 128, 1)
    scale, bias = 128 ** -0.5, 0.0
    args = (mode_id, 4, True, scale, cap, bias)
    out_v, lse_v = spline_ops.flash_attn_fwd_bf16(q, k, v, *args)
    out_c, lse_c = spline_ops.flash_attn_fwd_bf16(q.contiguous(), k.contiguous(), v.contiguous(), *args)
    assert torch.equal(out_v.view(torch.int16), out_c.view(torch.int16))
    assert torch.equal(lse_v, lse_c)
    grads_v = spline_ops.flash_attn_bwd_bf16(q, k, v, out_v, do, lse_v, mode_id, grad, 0, True, scale, cap,
                                             bias)
    grads_c = spline_ops.flash_attn_bwd_bf16(q.contiguous(), k.contiguous(), v.contiguous(), out_c, do, lse_c,
                                             mode_id, grad, 0, True, scale, cap, bias)
    for name, a, b in zip(("dq", "dk", "dv"), grads_v, grads_c):
        assert torch.isfinite(a.float()).all(), name
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), name


@pytest.mark.parametrize("causal", [True, False])
def test_shortest_sequence(capi, oracle, cuda, causal):
    """S = 128, one query block: the smallest length the kernels take."""
    from attention_reference import reference_bwd
    from test_gpu_flash_attention_bwd import bwd

    q, k, v, do = _inputs(1, 4, 2, 128, 1300 + int(causal))
    scale = 128 ** -0.5
    out, lse = fwd(capi, cuda, q, k, v, "softmax_native", causal, scale)
    ref_out, ref_lse = reference_fwd(oracle, q, k, v, "softmax_native", causal, scale, 30.0, 4)
    ok, info = _close(out.cpu().float(), ref_out, rel=1.5e-2)
    assert ok, info
    assert (lse.cpu() - ref_lse).abs().max().item() < 1e-3
    dq, dk, dv, _ = bwd(capi, cuda, q, k, v, out, do, lse, "softmax_native", 0, causal, scale)
    rq, rk, rv = reference_bwd(oracle, q, k, v, out, do, lse, "softmax_native", 0, causal, scale, 30.0, 0, 0.0)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        ok, info = _close(got, ref)
        assert ok, (name, info)


@pytest.mark.parametrize("mode,causal", [("softmax_native", False), ("softmax_d2", False), ("softcap_d4", False),
                                         ("sigmoid_native", False), ("softmax_native", True)])
def test_valid_keys_mask_padding(capi, oracle, cuda, mode, causal):
    """launch_flash_attention_fwd_strided_keys_bf16 with valid_keys = 200 of
    256: the keys from 200 on are masked whatever they hold (random rows
    here), so the first 200 rows equal the reference at S = 200."""
    import ctypes

    from attention_reference import default_bias
    from test_gpu_flash_attention_bwd import _strides

    q, k, v, _ = _inputs(1, 4, 2, 256, 1400 + M[mode] + int(causal), qmul=6.0 if mode == "softcap_d4" else 1.0)
    scale = 128 ** -0.5
    bias = default_bias(mode, 200)
    qd, kd, vd = q.to(cuda), k.to(cuda), v.to(cuda)
    out = torch.empty_like(qd)
    lse = torch.zeros(1, 4, 256, dtype=torch.float32, device=cuda)
    rc = capi.launch_flash_attention_fwd_strided_keys_bf16(
        capi.ptr(out), capi.ptr(lse), capi.ptr(qd), capi.ptr(kd), capi.ptr(vd), ctypes.c_int64(1),
        ctypes.c_int64(4), ctypes.c_int64(2), ctypes.c_int64(256), ctypes.c_int64(200), ctypes.c_int64(128),
        _strides(qd, kd, vd, out), ctypes.c_int(M[mode]), ctypes.c_int(4), ctypes.c_int(int(causal)),
        ctypes.c_float(scale), ctypes.c_float(30.0), ctypes.c_float(bias), capi.stream())
    assert rc == 0
    torch.cuda.synchronize()
    ref_out, ref_lse = reference_fwd(oracle, q[:, :200], k[:, :200], v[:, :200], mode, causal, scale, 30.0, 4, bias)
    got = out.cpu().float()[:, :200]
    assert torch.isfinite(got).all()
    ok, info = _close(got, ref_out, rel=1.5e-2)
    assert ok, (mode, causal, info)
    if ref_lse is not None:
        assert (lse.cpu()[..., :200] - ref_lse).abs().max().item() < 2e-2
    for bad in (0, 257):
        rc = capi.launch_flash_attention_fwd_strided_keys_bf16(
            capi.ptr(out), capi.ptr(lse), capi.ptr(qd), capi.ptr(kd), capi.ptr(vd), ctypes.c_int64(1),
            ctypes.c_int64(4), ctypes.c_int64(2), ctypes.c_int64(256), ctypes.c_int64(bad), ctypes.c_int64(128),
            _strides(qd, kd, vd, out), ctypes.c_int(M[mode]), ctypes.c_int(4), ctypes.c_int(int(causal)),
            ctypes.c_float(scale), ctypes.c_float(30.0), ctypes.c_float(bias), capi.stream())
        assert rc != 0, bad


@pytest.mark.parametrize("seq,valid", [(256, 200), (256, 129), (333, 70)])
@pytest.mark.parametrize("mode", ["softmax_native", "softcap_d4", "sigmoid_native"])
def test_valid_keys_padding_nan_inf(capi, cuda, mode, seq, valid):
    """Padded K / V rows holding NaN and +-Inf change nothing: the outputs of
    every query row and the lse equal, bit for bit, those with zero padding
    (keys past valid_keys are zeroed on chip before P.V)."""
    import ctypes

    from test_gpu_flash_attention_bwd import _strides

    print(f"valid_keys nan/inf {mode} seq {seq} valid {valid}", flush=True)
    q, k, v, _ = _inputs(1, 4, 2, seq, 1600 + seq + valid + M[mode], qmul=2.0)
    zk, zv = k.clone(), v.clone()
    zk[:, valid:] = 0
    zv[:, valid:] = 0
    bk, bv = k.clone(), v.clone()
    bk[:, valid::3], bk[:, valid + 1::3], bk[:, valid + 2::3] = float("nan"), float("inf"), -float("inf")
    bv[:, valid::3], bv[:, valid + 1::3], bv[:, valid + 2::3] = float("inf"), float("nan"), -float("inf")
    scale = 128 ** -0.5
    results = []
    for kk, vv in ((zk, zv), (bk, bv)):
        qd, kd, vd = q.to(cuda), kk.to(cuda), vv.to(cuda)
        out = torch.empty_like(qd)
        lse = torch.zeros(1, 4, seq, dtype=torch.float32, device=cuda)
        for causal in (0, 1):
            rc = capi.launch_flash_attention_fwd_strided_keys_bf16(
                capi.ptr(out), capi.ptr(lse), capi.ptr(qd), capi.ptr(kd), capi.ptr(vd), ctypes.c_int64(1),
                ctypes.c_int64(4), ctypes.c_int64(2), ctypes.c_int64(seq), ctypes.c_int64(valid),
                ctypes.c_int64(128), _strides(qd, kd, vd, out), ctypes.c_int(M[mode]), ctypes.c_int(4),
                ctypes.c_int(causal), ctypes.c_float(scale), ctypes.c_float(30.0), ctypes.c_float(-5.0),
                capi.stream())
            assert rc == 0
            torch.cuda.synchronize()
            results.append((out.cpu().clone(), lse.cpu().clone()))
    for (zo, zl), (bo, bl) in zip(results[:2], results[2:]):
        assert torch.isfinite(bo.float()).all()
        assert torch.equal(zo.view(torch.int16), bo.view(torch.int16))
        assert torch.equal(zl, bl)


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("s", [1, 77, 200, 333])
def test_any_length_equals_padded(capi, cuda, s, d):
    """A sequence of any length runs without padding: the kernel reads no row
    past S, and its outputs equal, bit for bit, those of the same operands
    zero-padded to a multiple of 128 with the padded keys masked
    (launch_flash_attention_fwd_strided_keys_bf16, valid_keys = S)."""
    import ctypes

    from test_gpu_flash_attention_bwd import _strides

    padded = (s + 127) // 128 * 128
    q, k, v, _ = _inputs(2, 4, 2, s, 1500 + s + d, qmul=2.0, d=d)
    pad = lambda t: torch.cat((t, t.new_zeros(t.shape[0], padded - s, *t.shape[2:])), 1)
    qp, kp, vp = pad(q).to(cuda), pad(k).to(cuda), pad(v).to(cuda)
    scale = d ** -0.5
    for mode, route in (("softmax_native", 4), ("softmax_d2", 12), ("softcap_d4", 4), ("sigmoid_native", 4),
                        ("softmax_pwl2", 4), ("sigmoid_d3", 4)):
        bias = -math.log(padded)
        for causal in (True, False):
            out, lse = fwd(capi, cuda, q, k, v, mode, causal, scale, route=route, bias=bias)
            pout = torch.empty_like(qp)
            plse = torch.zeros(2, 4, padded, dtype=torch.float32, device=cuda)
            rc = capi.launch_flash_attention_fwd_strided_keys_bf16(
                capi.ptr(pout), capi.ptr(plse), capi.ptr(qp), capi.ptr(kp), capi.ptr(vp), ctypes.c_int64(2),
                ctypes.c_int64(4), ctypes.c_int64(2), ctypes.c_int64(padded), ctypes.c_int64(s),
                ctypes.c_int64(d), _strides(qp, kp, vp, pout), ctypes.c_int(M[mode]), ctypes.c_int(route),
                ctypes.c_int(int(causal)), ctypes.c_float(scale), ctypes.c_float(30.0), ctypes.c_float(bias),
                capi.stream())
            assert rc == 0
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int16), pout[:, :s].view(torch.int16)), (mode, causal)
            assert torch.equal(lse, plse[:, :, :s].contiguous()), (mode, causal)


@pytest.mark.parametrize("hq,hkv", [(4, 2), (2, 2)])
@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("s", [1, 77, 200, 333])
def test_backward_any_length_equals_padded(capi, cuda, s, d, hq, hkv):
    """The backward at any S reads no row past the sequence; dq, dk, dv equal,
    bit for bit, those of the operands zero-padded to a multiple of 128 with
    the lse padded with +inf (grouped heads through the partials workspace,
    plain heads directly)."""
    from test_gpu_flash_attention_bwd import bwd

    padded = (s + 127) // 128 * 128
    q, k, v, do = _inputs(2, hq, hkv, s, 1700 + s + d + hq, qmul=2.0, d=d)
    pad = lambda t, val=0.0: torch.cat((t, t.new_full((t.shape[0], padded - t.shape[1], *t.shape[2:]), val)), 1)
    scale = d ** -0.5
    bias = -math.log(padded)
    for mode, grad, route in (("softmax_native", 0, 0), ("softmax_d2", 0, 32), ("softcap_d4", 1, 0),
                              ("sigmoid_native", 0, 0), ("sigmoid_d3", 0, 0), ("softmax_pwl2", 0, 4)):
        for causal in (True, False):
            out, lse = fwd(capi, cuda, q, k, v, mode, causal, scale, route=route or 4, bias=bias)
            got = bwd(capi, cuda, q, k, v, out, do, lse, mode, grad, causal, scale, route=route, bias=bias)[:3]
            lse_p = pad(lse.transpose(1, 2), math.inf).transpose(1, 2).contiguous()
            want = bwd(capi, cuda, pad(q), pad(k), pad(v), pad(out), pad(do), lse_p, mode, grad, causal, scale,
                       route=route, bias=bias)[:3]
            for name, a, b in zip(("dq", "dk", "dv"), got, want):
                assert torch.equal(a.view(torch.int32), b[:, :s].contiguous().view(torch.int32)), (mode, causal, name)


@pytest.mark.parametrize("route", [4, 6])
@pytest.mark.parametrize("mode", ["softmax_pwl2_safe_f16", "softmax_pwl1_safe_f16", "softmax_d2_safe_f16",
                                  "softmax_pwl2_f16"])
def test_packed_f16_programs_odd_query_block_count(capi, oracle, cuda, mode, route):
    """An odd number of 128-query blocks at head_dim 128: the packed FP16
    exp2 programs run 8-wave blocks there too, the last one holding 128
    queries past the sequence.  Non-causal S = 333 (ragged) against the
    reference; causal S = 384 (aligned) bit for bit against the first 384
    queries of the same operands at S = 512, an even block count, where each
    wave sees the same key tiles in the same order."""
    seed = 1700 + M[mode] + route
    print(f"fwd odd blocks {mode} route {route} seed {seed}", flush=True)
    scale = 1 / math.sqrt(128)
    q, k, v, _ = _inputs(1, 4, 2, 333, seed)
    out, lse = fwd(capi, cuda, q, k, v, mode, False, scale, route=route)
    ref_out, ref_lse = reference_fwd(oracle, q, k, v, mode, False, scale, 30.0, route)
    got = out.cpu().float()
    assert torch.isfinite(got).all()
    ok, info = _close(got, ref_out, rel=1.5e-2)
    assert ok, ("out", mode, route, info)
    assert (lse.cpu() - ref_lse).abs().max().item() < 2e-2

    q, k, v, _ = _inputs(1, 4, 2, 512, seed + 1)
    out_l, lse_l = fwd(capi, cuda, q, k, v, mode, True, scale, route=route)
    out_s, lse_s = fwd(capi, cuda, q[:, :384].contiguous(), k[:, :384].contiguous(), v[:, :384].contiguous(),
                       mode, True, scale, route=route)
    assert torch.equal(out_s.view(torch.int16), out_l[:, :384].view(torch.int16))
    assert torch.equal(lse_s, lse_l[..., :384])
