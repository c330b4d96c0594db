"""The C-ABI library loads and exports every symbol include/spline_ops_hip.h
declares (no compute: runs without a GPU)."""

import ctypes
import os

import capi_helpers


def test_header_declares_the_hot_path():
    names = capi_helpers.declared_symbols()
    assert len(names) >= 100
    for must in ("launch_swish_fwd_d3_kernel", "launch_swish_mul_packed_fwd_d3_kernel_bf16",
                 "launch_flash_sigmoid_direct_d3_d4_bf16", "launch_tanh_fwd_d4_kernel_bf16"):
        assert must in names


def test_library_exports_every_declared_symbol():
    import torch  # noqa: F401  (torch's HIP runtime is the one the library binds to)

    assert os.path.exists(capi_helpers.LIB), "build the library first (__graft_entry__.build())"
    lib = ctypes.CDLL(capi_helpers.LIB)
    missing = [n for n in capi_helpers.declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing
