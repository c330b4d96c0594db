"""GPU parity of the dS-keeping attention backward
(launch_flash_attention_bwd_strided_ds_bf16): its dK/dV kernel stores dS in
the workspace and its dQ kernel multiplies the stored dS by K instead of
recomputing S, P, dP and the score program.  Both read the same BF16 dS
values and accumulate in the same order, so dQ, dK and dV must equal the
recomputing backward (launch_flash_attention_bwd_strided_bf16, itself checked
against a float32 reference in test_gpu_flash_attention_bwd.py) bit for bit,
for every score mode and derivative program, causal or not, grouped heads or
not, head_dim 64 and 128.  The workspace is filled with NaN before each call,
so a chunk read but never written would show."""

import ctypes
import math
import os

import pytest
import torch

from attention_reference import M, default_bias as _bias
from test_gpu_flash_attention_bwd import CASES, _inputs, _strides, fwd

pytestmark = pytest.mark.gpu


def ds_bytes(capi, b, hq, s, d, mode):
    fn = capi.lib.spline_hip_attn_bwd_ds_bytes
    fn.restype = ctypes.c_int64
    return fn(ctypes.c_int64(b), ctypes.c_int64(hq), ctypes.c_int64(s), ctypes.c_int64(d), ctypes.c_int(mode))


def bwd_pair(capi, cuda, q, k, v, out, do, lse, mode, grad, causal, scale, route=0, cap=30.0):
    """(recomputing, dS-keeping) backward outputs and the workspace size."""
    b, s, hq, d = q.shape
    hkv = k.shape[2]
    qd, kd, vd, dod = q.to(cuda), k.to(cuda), v.to(cuda), do.to(cuda)
    bias = _bias(mode, s)
    nbytes = ds_bytes(capi, b, hq, s, d, M[mode])
    # 16 bytes of slack keep a non-null workspace where the path does not apply
    ws_ds = torch.full((max(nbytes, 16) // 2,), float("nan"), dtype=torch.bfloat16, device=cuda)
    results = []
    for entry in ("launch_flash_attention_bwd_strided_bf16", "launch_flash_attention_bwd_strided_ds_bf16"):
        dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
        delta = torch.empty(b, hq, s, dtype=torch.float32, device=cuda)
        ws = torch.empty(2, b, hq, s, d, dtype=torch.float32, device=cuda) if hq != hkv else None
        head = [capi.ptr(dq), capi.ptr(dk), capi.ptr(dv), capi.ptr(delta),
                capi.ptr(ws) if ws is not None else ctypes.c_void_p(0)]
        if entry.endswith("_ds_bf16"):
            head.append(capi.ptr(ws_ds))
        rc = getattr(capi, entry)(
            *head, capi.ptr(qd), capi.ptr(kd), capi.ptr(vd), capi.ptr(out), capi.ptr(dod), capi.ptr(lse),
            ctypes.c_int64(b), ctypes.c_int64(hq), ctypes.c_int64(hkv), ctypes.c_int64(s), ctypes.c_int64(d),
            _strides(qd, kd, vd, out, dod, dq, dk, dv), ctypes.c_int(M[mode]), ctypes.c_int(grad),
            ctypes.c_int(route), ctypes.c_int(int(causal)), ctypes.c_float(scale), ctypes.c_float(cap),
            ctypes.c_float(bias), capi.stream())
        assert rc == 0, entry
        torch.cuda.synchronize()
        results.append((dq.cpu(), dk.cpu(), dv.cpu()))
    return results[0], results[1], nbytes


def _assert_identical(rec, kept, label):
    for name, a, b in zip(("dq", "dk", "dv"), rec, kept):
        assert torch.isfinite(a.float()).all(), (label, name)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), (label, name)


def _run(capi, cuda, mode, grad, route, causal, b=1, hq=4, hkv=2, s=256, d=128, seed=0):
    q, k, v, do = _inputs(b, hq, hkv, s, seed, qmul=6.0 if mode.startswith("softcap") else 1.0, d=d)
    scale = 1 / math.sqrt(d)
    out, lse = fwd(capi, cuda, q, k, v, mode, causal, scale, route=route if route else 4)
    rec, kept, nbytes = bwd_pair(capi, cuda, q, k, v, out, do, lse, mode, grad, causal, scale, route=route)
    _assert_identical(rec, kept, (mode, grad, route, causal, b, hq, hkv, s, d))
    return nbytes


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("mode,grad,route", CASES)
def test_ds_backward_equals_recomputing_backward(capi, cuda, mode, grad, route, causal):
    """head_dim 128, four query heads per two KV heads: every mode keeps dS."""
    nbytes = _run(capi, cuda, mode, grad, route, causal, seed=300 + M[mode] * 5 + grad + route)
    assert nbytes == 4 * 256 * 256 * 2


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("mode,grad,route", [("softcap_d4", 1, 0), ("softcap_d4", 3, 0), ("softcap_native", 0, 0),
                                             ("sigmoid_native", 0, 0), ("sigmoid_d3", 0, 0),
                                             ("softmax_native", 0, 0), ("softmax_d2", 0, 32)])
def test_ds_backward_head_dim_64(capi, cuda, mode, grad, route, causal):
    """head_dim 64: the modes with a score program keep dS; plain softmax
    recomputes (the size helper returns 0 and the call is the recomputing
    backward)."""
    nbytes = _run(capi, cuda, mode, grad, route, causal, d=64, seed=400 + M[mode] + grad)
    plain = mode.startswith("softmax")
    assert nbytes == (0 if plain else 4 * 256 * 256 * 2)


@pytest.mark.parametrize("d", [64, 128])
def test_ds_backward_b3_at_its_length(capi, cuda, d):
    """B3 (fitted for S = 4096), direct and algebraic derivatives, causal, one
    query head per KV head (no grouped partials)."""
    for grad in (5, 4):
        _run(capi, cuda, "sigmoid_b3", grad, 0, True, hq=2, hkv=2, s=4096, d=d, seed=500 + grad)


@pytest.mark.parametrize("s", [128, 384, 640])
def test_ds_backward_batches_and_lengths(capi, cuda, s):
    """Two sequences, plain heads and grouped heads, lengths that are odd
    multiples of 128 (the dQ blocks of 128 queries meet the causal diagonal in
    every position)."""
    for hq, hkv in ((2, 2), (8, 2)):
        _run(capi, cuda, "softcap_d4", 1, 0, True, b=2, hq=hq, hkv=hkv, s=s, seed=600 + s + hq)
        _run(capi, cuda, "softmax_d2", 0, 12, False, b=2, hq=hq, hkv=hkv, s=s, seed=700 + s + hq)


@pytest.mark.parametrize("s", [200, 333])
def test_ds_backward_ragged_lengths_recompute(capi, cuda, s):
    """Lengths that are not a multiple of 128 take the recomputing backward
    whatever the workspace (the size helper returns 0)."""
    assert _run(capi, cuda, "softcap_d4", 1, 0, True, s=s, seed=800 + s) == 0


def test_ds_backward_rejects_a_misaligned_workspace(capi, cuda):
    b, hq, hkv, s, d = 1, 2, 2, 128, 128
    q, k, v, do = _inputs(b, hq, hkv, s, 7, d=d)
    scale = 1 / math.sqrt(d)
    out, lse = fwd(capi, cuda, q, k, v, "softcap_native", True, scale, route=4)
    qd, kd, vd, dod = q.to(cuda), k.to(cuda), v.to(cuda), do.to(cuda)
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    delta = torch.empty(b, hq, s, dtype=torch.float32, device=cuda)
    ws_ds = torch.empty(ds_bytes(capi, b, hq, s, d, M["softcap_native"]) // 2 + 8, dtype=torch.bfloat16, device=cuda)
    rc = capi.launch_flash_attention_bwd_strided_ds_bf16(
        capi.ptr(dq), capi.ptr(dk), capi.ptr(dv), capi.ptr(delta), ctypes.c_void_p(0),
        ctypes.c_void_p(ws_ds.data_ptr() + 8), capi.ptr(qd), capi.ptr(kd), capi.ptr(vd), capi.ptr(out),
        capi.ptr(dod), capi.ptr(lse), ctypes.c_int64(b), ctypes.c_int64(hq), ctypes.c_int64(hkv), ctypes.c_int64(s),
        ctypes.c_int64(d), _strides(qd, kd, vd, out, dod, dq, dk, dv), ctypes.c_int(M["softcap_native"]),
        ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(1), ctypes.c_float(scale), ctypes.c_float(30.0),
        ctypes.c_float(0.0), capi.stream())
    assert rc == 1  # hipErrorInvalidValue


def test_binding_keeps_ds_within_its_budget(cuda, spline_ops, monkeypatch):
    """spline_ops.flash_attn_bwd_bf16 allocates the dS workspace up to
    SPLINE_ATTN_DS_MAX_BYTES; with the budget at 0 it recomputes.  Both give
    the same bits."""
    b, s, hq, hkv, d = 1, 256, 4, 2, 128
    q, k, v, do = (t.to(cuda) for t in _inputs(b, hq, hkv, s, 11, qmul=6.0, d=d))
    scale = 1 / math.sqrt(d)
    out, lse = spline_ops.flash_attn_fwd_bf16(q, k, v, M["softcap_d4"], 4, True, scale, 30.0, 0.0, -1)
    grads = []
    for budget in ("0", str(1 << 30)):
        monkeypatch.setenv("SPLINE_ATTN_DS_MAX_BYTES", budget)
        grads.append(spline_ops.flash_attn_bwd_bf16(q, k, v, out, do, lse, M["softcap_d4"], 1, 0, True, scale,
                                                    30.0, 0.0))
    for a, c in zip(*grads):
        assert torch.equal(a.view(torch.int16), c.view(torch.int16))
    monkeypatch.setenv("SPLINE_ATTN_DS_MAX_BYTES", "lots")
    with pytest.raises(RuntimeError, match="SPLINE_ATTN_DS_MAX_BYTES"):
        spline_ops.flash_attn_bwd_bf16(q, k, v, out, do, lse, M["softcap_d4"], 1, 0, True, scale, 30.0, 0.0)
