"""The allocation-free attention backward
(launch_flash_attention_bwd_strided_bf16_noalloc) against the entry point it
wraps (launch_flash_attention_bwd_strided_bf16 with caller workspaces),
through the C ABI: identical dq, dk, dv bits on two calls in a row, the
second with a smaller problem, the size limit reported as an error, and
replays of a captured HIP graph.  Both entry points run the same kernels,
so the results must be equal bit for bit."""

import ctypes
import math

import pytest
import torch

from attention_reference import M, default_bias
from test_gpu_flash_attention_bwd import _inputs, _strides, bwd, fwd

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20  # SPLINE_HIP_BWD_SCRATCH_BYTES


def bwd_noalloc(capi, cuda, q, k, v, out, do, lse, mode, grad, causal, scale, cap=30.0, route=0):
    b, s, hq, d = q.shape
    hkv = k.shape[2]
    qd, kd, vd, dod = q.to(cuda), k.to(cuda), v.to(cuda), do.to(cuda)
    dq = torch.empty_like(qd)
    dk = torch.empty_like(kd)
    dv = torch.empty_like(vd)
    rc = capi.launch_flash_attention_bwd_strided_bf16_noalloc(
        capi.ptr(dq), capi.ptr(dk), capi.ptr(dv), capi.ptr(qd), capi.ptr(kd), capi.ptr(vd), capi.ptr(out),
        capi.ptr(dod), capi.ptr(lse), ctypes.c_int64(b), ctypes.c_int64(hq), ctypes.c_int64(hkv),
        ctypes.c_int64(s), ctypes.c_int64(d), _strides(qd, kd, vd, out, dod, dq, dk, dv),
        ctypes.c_int(M[mode]), ctypes.c_int(grad), ctypes.c_int(route), ctypes.c_int(int(causal)),
        ctypes.c_float(scale), ctypes.c_float(cap), ctypes.c_float(default_bias(mode, s)), capi.stream())
    assert rc == 0, rc
    torch.cuda.synchronize()
    return dq.cpu().float(), dk.cpu().float(), dv.cpu().float()


def _check(capi, cuda, shape, mode, grad, route, causal, seed):
    b, hq, hkv, s, d = shape
    print(f"no-alloc backward: shape {shape} mode {mode} grad {grad} route {route} causal {causal}",
          flush=True)
    q, k, v, do = _inputs(b, hq, hkv, s, seed, d=d)
    scale = 1.0 / math.sqrt(d)
    out, lse = fwd(capi, cuda, q, k, v, mode, causal, scale, route=max(route, 4) if route else 4)
    want = bwd(capi, cuda, q, k, v, out, do, lse, mode, grad, causal, scale, route=route)[:3]
    got = bwd_noalloc(capi, cuda, q, k, v, out, do, lse, mode, grad, causal, scale, route=route)
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        assert torch.equal(g.view(torch.int32), w.view(torch.int32)), f"{name} differs for {shape} {mode}"


# grouped heads first (delta + partials in the array), then a smaller,
# ungrouped problem that reuses the same array
SEQUENCE = [
    ((2, 8, 2, 512, 128), "softmax_native", 0, 0, True),
    ((1, 4, 4, 256, 64), "softmax_d2", 0, 32, False),
]


def test_noalloc_matches_workspace_entry_point(capi, cuda):
    for i, (shape, mode, grad, route, causal) in enumerate(SEQUENCE):
        _check(capi, cuda, shape, mode, grad, route, causal, seed=500 + i)


def test_noalloc_softcap_and_sigmoid(capi, cuda):
    _check(capi, cuda, (1, 4, 2, 384, 128), "softcap_d4", 1, 0, True, seed=510)
    _check(capi, cuda, (1, 4, 1, 256, 64), "sigmoid_native", 0, 0, False, seed=511)


def test_noalloc_rejects_problems_beyond_the_array(capi, cuda):
    # grouped heads at D 128: 2 * 65,536 rows * 128 * 4 B of partials > 64 MiB.
    # The entry point returns before touching any pointer, so null is fine.
    b, hq, hkv, s, d = 1, 16, 8, 4096, 128
    assert 4 * b * hq * s + 8 * b * hq * s * d > SCRATCH_BYTES
    strides = (ctypes.c_int64 * 24)(*([8] * 24))
    rc = capi.launch_flash_attention_bwd_strided_bf16_noalloc(
        *([ctypes.c_void_p(0)] * 9), ctypes.c_int64(b), ctypes.c_int64(hq), ctypes.c_int64(hkv),
        ctypes.c_int64(s), ctypes.c_int64(d), strides, ctypes.c_int(M["softmax_native"]), ctypes.c_int(0),
        ctypes.c_int(0), ctypes.c_int(1), ctypes.c_float(0.1), ctypes.c_float(30.0), ctypes.c_float(0.0),
        capi.stream())
    assert rc == 2  # hipErrorOutOfMemory


def test_noalloc_under_graph_capture(capi, cuda):
    """The reason for the entry point: a captured backward (grouped heads, so
    both the delta rows and the dK / dV partials live in the library's array)
    replays to the eager result every time, with eager work between replays."""
    b, hq, hkv, s, d = 1, 4, 2, 256, 128
    print("no-alloc backward under graph capture", flush=True)
    q, k, v, do = _inputs(b, hq, hkv, s, 520, d=d)
    scale = 1.0 / math.sqrt(d)
    out, lse = fwd(capi, cuda, q, k, v, "softmax_native", True, scale)
    want = bwd(capi, cuda, q, k, v, out, do, lse, "softmax_native", 0, True, scale)[:3]
    qd, kd, vd, dod = q.to(cuda), k.to(cuda), v.to(cuda), do.to(cuda)
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    strides = _strides(qd, kd, vd, out, dod, dq, dk, dv)

    def launch():
        rc = capi.launch_flash_attention_bwd_strided_bf16_noalloc(
            capi.ptr(dq), capi.ptr(dk), capi.ptr(dv), capi.ptr(qd), capi.ptr(kd), capi.ptr(vd), capi.ptr(out),
            capi.ptr(dod), capi.ptr(lse), ctypes.c_int64(b), ctypes.c_int64(hq), ctypes.c_int64(hkv),
            ctypes.c_int64(s), ctypes.c_int64(d), strides, ctypes.c_int(M["softmax_native"]), ctypes.c_int(0),
            ctypes.c_int(0), ctypes.c_int(1), ctypes.c_float(scale), ctypes.c_float(30.0), ctypes.c_float(0.0),
            capi.stream())
        assert rc == 0, rc

    launch()  # first call on this device: the array's address is looked up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch()
    for _ in range(3):
        for t in (dq, dk, dv):
            t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name, got, w in zip(("dq", "dk", "dv"), (dq, dk, dv), want):
            assert torch.equal(got.cpu().float().view(torch.int32), w.view(torch.int32)), name
