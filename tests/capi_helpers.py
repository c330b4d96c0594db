"""ctypes access to the C ABI of libspline_hip.so for the GPU parity tests.

Device memory comes from torch tensors; the stream is torch's current HIP
stream, so results are ordered with torch's own work.
"""

import ctypes
import os
import re
import subprocess

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "fast-polynomial-transcendentals_amd", "python", "libspline_hip.so")
HEADER = os.path.join(ROOT, "include", "spline_ops_hip.h")


def declared_symbols():
    """Function names declared by include/spline_ops_hip.h (after macro expansion)."""
    out = subprocess.run(["gcc", "-E", "-P", "-x", "c", HEADER], check=True,
                         stdout=subprocess.PIPE, text=True).stdout
    names = re.findall(r"\b(?:int|int64_t)\s+(\w+)\s*\(", out)
    return sorted(set(names))


class CApi:
    def __init__(self):
        # torch first: its HIP runtime must be the one the library binds to.
        import torch  # noqa: F401

        self.lib = ctypes.CDLL(LIB)

    def __getattr__(self, name):
        fn = getattr(self.lib, name)
        fn.restype = ctypes.c_int
        return fn

    @staticmethod
    def ptr(t: torch.Tensor):
        return ctypes.c_void_p(t.data_ptr())

    @staticmethod
    def stream():
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def call(self, name, *args):
        conv = []
        for a in args:
            if isinstance(a, torch.Tensor):
                conv.append(self.ptr(a))
            elif isinstance(a, int):
                conv.append(ctypes.c_int64(a))
            else:
                conv.append(a)
        rc = getattr(self, name)(*conv, self.stream())
        if rc != 0:
            raise RuntimeError(f"{name} returned {rc}")
        return rc
