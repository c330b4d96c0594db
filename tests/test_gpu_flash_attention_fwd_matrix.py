"""Forward parity of every fused-attention score mode at both head sizes,
with batched, grouped-query operands in FA4's layout: out (BF16) and, for
the softmax and softcap modes, the FP32 log-sum-exp, against the float32
CPU reference that evaluates the same score programs through the oracle.

Two sequences, eight query heads over two KV heads (four per group), S =
256: every block of the grid maps its own (batch, query head) to the right
KV head.  The B3 programs, fitted for S = 4096, run at that length."""

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
        # hardware modes: FP32 exponent sums; programs: the same programs in
        # the reference, so only the BF16 products and summation order differ
        bound = 1e-3 if mode in ("softmax_native", "softcap_native") else 2e-2
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
