"""Workspace size of the dS-keeping attention backward
(spline_hip_attn_bwd_ds_bytes, a host function: runs without a GPU): B * Hq
* S^2 BF16 for lengths that are a multiple of 128, every mode at head_dim 128
and the modes with a score program at head_dim 64; 0 where the backward
recomputes (plain softmax at head_dim 64, other lengths, invalid shapes)."""

import ctypes

import pytest

import capi_helpers
from attention_reference import M


@pytest.fixture(scope="module")
def size_fn():
    import torch  # noqa: F401  (torch's HIP runtime is the one the library binds to)

    fn = ctypes.CDLL(capi_helpers.LIB).spline_hip_attn_bwd_ds_bytes
    fn.restype = ctypes.c_int64
    fn.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int]
    return fn


@pytest.mark.parametrize("mode", sorted(M))
def test_every_mode_keeps_ds_at_head_dim_128(size_fn, mode):
    assert size_fn(2, 32, 4096, 128, M[mode]) == 2 * 32 * 4096 * 4096 * 2


@pytest.mark.parametrize("mode", sorted(M))
def test_head_dim_64_keeps_ds_for_score_programs_only(size_fn, mode):
    plain = mode.startswith("softmax")
    assert size_fn(1, 32, 4096, 64, M[mode]) == (0 if plain else 32 * 4096 * 4096 * 2)


@pytest.mark.parametrize("args", [(1, 4, 200, 128, 0), (1, 4, 4000, 128, 4), (0, 4, 256, 128, 0),
                                  (1, 0, 256, 128, 0), (1, 4, 0, 128, 0), (1, 4, 256, 96, 0),
                                  (1, 4, 256, 128, -1), (1, 4, 256, 128, 22),
                                  (1 << 20, 1 << 20, 1 << 20, 128, 0)])
def test_no_workspace_where_the_backward_recomputes(size_fn, args):
    assert size_fn(*args) == 0
