"""Build recipe for the MI355X spline_ops library (in-tree, gfx950 only).

Produces, next to the Python modules in ``python/``:

* ``libspline_hip.so`` -- the hand-written HIP kernels and their C ABI
  (``include/spline_ops_hip.h``), compiled with hipcc for gfx950;
* ``spline_ops.so`` -- the PyTorch-ROCm extension (pybind11 module plus the
  ``torch.ops.spline_ops`` schemas) that calls the C ABI.

Run ``python fast-polynomial-transcendentals_amd/build.py`` (or
``__graft_entry__.build()``).  Object files go to ``_build/`` beside this
file; every call recompiles what changed (make-like timestamps) unless
``force=True``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
PYDIR = os.path.join(PKG, "python")
BUILD = os.path.join(PKG, "_build")
INCLUDE = os.path.join(ROOT, "include")

ARCH = os.environ.get("PT_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_SOURCES = ["launch.hip", "activations.hip", "swiglu.hip", "attention.hip", "exp2_probes.hip", "experiments.hip", "sincos.hip", "rope.hip", "flash_attn.hip", "flash_attn_bwd.hip"]
HIP_HEADERS = ["elementwise.hpp", "ops.hpp", "programs.hpp", "trig.hpp", "score_programs.hpp", "flash_attn.hpp"]

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # Every rounding step of the programs is explicit; never let the compiler
    # fuse a multiply into a following add.
    "-ffp-contract=off",
    # Packed FP32 instructions stay off: only scalar FP32 and packed FP16.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

LIB_HIP = os.path.join(PYDIR, "libspline_hip.so")
EXT_NAME = "spline_ops"
EXT = os.path.join(PYDIR, EXT_NAME + ".so")


def _newer(target: str, deps: list[str]) -> bool:
    if not os.path.exists(target):
        return True
    t = os.path.getmtime(target)
    return any(os.path.getmtime(d) > t for d in deps if os.path.exists(d))


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + proc.stdout)
        raise RuntimeError(f"build step failed: {os.path.basename(cmd[-1])}")
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops" not in line and "not a recognized feature" not in line
    ).strip()
    if out:
        sys.stderr.write(out + "\n")


def build_hip(force: bool = False, jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    headers = [os.path.join(CSRC, h) for h in HIP_HEADERS] + [os.path.join(INCLUDE, "spline_ops_hip.h")]
    objs, todo = [], []
    for src in HIP_SOURCES:
        s = os.path.join(CSRC, src)
        o = os.path.join(BUILD, src.replace(".hip", ".o"))
        objs.append(o)
        if force or _newer(o, [s, __file__] + headers):
            todo.append([HIPCC, *HIP_FLAGS, "-I", INCLUDE, "-I", CSRC, "-c", "-o", o, s])
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(todo) or 1))) as ex:
        list(ex.map(_run, todo))
    if force or todo or _newer(LIB_HIP, objs):
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", LIB_HIP, *objs])
    return LIB_HIP


def build_ext(force: bool = False) -> str:
    import torch  # noqa: F401  (headers and libraries come from the install)
    from torch.utils import cpp_extension as ce

    src = os.path.join(CSRC, "binding", "spline_ops.cpp")
    if not (force or _newer(EXT, [src, LIB_HIP, __file__, os.path.join(INCLUDE, "spline_ops_hip.h")])):
        return EXT
    import torch as _t

    abi = int(_t._C._GLIBCXX_USE_CXX11_ABI)
    incs = []
    for p in ce.include_paths():
        incs += ["-I", p]
    incs += ["-I", sysconfig.get_paths()["include"], "-I", INCLUDE, "-I", "/opt/rocm/include"]
    libdir = ce.library_paths()[0]
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-Wno-deprecated-declarations",
        *incs, src, "-o", EXT,
        "-L", libdir, "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip",
        "-ltorch_hip", "-lamdhip64",
        "-L", PYDIR, "-lspline_hip",
        f"-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}",
    ]
    _run(cmd)
    return EXT


def build(force: bool = False) -> None:
    build_hip(force=force)
    build_ext(force=force)


if __name__ == "__main__":
    build(force="--force" in sys.argv)
    print(LIB_HIP)
    print(EXT)
