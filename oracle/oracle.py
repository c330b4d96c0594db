"""ctypes front end of the CPU oracle (``libspline_oracle.so``).

TEST INFRASTRUCTURE ONLY.  ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker or as the timed CPU baseline.  The product path never imports it.

Every array argument is a NumPy array of raw 16-bit bit patterns
(``numpy.uint16``); helpers convert to and from torch tensors by viewing the
bits, never by value.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libspline_oracle.so")

F16, BF16, BF16_SOLLYA = 0, 1, 2
SIGMOID, TANH, SWISH, GELU = 0, 1, 2, 3
FWD, BWD = 0, 1
RND_SINGLE, RND_F32 = 0, 1

_FAMILY = {"sigmoid": SIGMOID, "tanh": TANH, "swish": SWISH, "gelu": GELU}
# "bf16_sollya": BF16 storage with the Sollya coefficient set (activation
# programs only).
_FMT = {"f16": F16, "fp16": F16, "float16": F16, "bf16": BF16, "bfloat16": BF16,
        "bf16_sollya": BF16_SOLLYA}

_lib = None


def build() -> str:
    """Compile the oracle in place (gcc via the Makefile beside this file)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(l: ctypes.CDLL) -> None:
    u16p = ctypes.POINTER(ctypes.c_uint16)
    u8p = ctypes.POINTER(ctypes.c_uint8)
    f32p = ctypes.POINTER(ctypes.c_float)
    i64 = ctypes.c_int64
    ci = ctypes.c_int
    l.orc_f32_to_bf16_audit.argtypes = [ctypes.c_float]
    l.orc_f32_to_bf16_audit.restype = ctypes.c_uint16
    l.orc_f64_to_bf16.argtypes = [ctypes.c_double]
    l.orc_f64_to_bf16.restype = ctypes.c_uint16
    l.orc_f64_to_f16.argtypes = [ctypes.c_double]
    l.orc_f64_to_f16.restype = ctypes.c_uint16
    l.orc_bf16_to_f64.argtypes = [ctypes.c_uint16]
    l.orc_bf16_to_f64.restype = ctypes.c_double
    l.orc_f16_to_f64.argtypes = [ctypes.c_uint16]
    l.orc_f16_to_f64.restype = ctypes.c_double
    l.orc_fma16.argtypes = [ci, ctypes.c_uint16, ctypes.c_uint16, ctypes.c_uint16]
    l.orc_fma16.restype = ctypes.c_uint16
    l.orc_bf16_fma_audit.argtypes = [ctypes.c_uint16] * 3
    l.orc_bf16_fma_audit.restype = ctypes.c_uint16
    l.orc_activation.argtypes = [ci, ci, ci, ci, ci, u16p, u16p, i64]
    l.orc_activation_bwd.argtypes = [ci, ci, ci, ci, u16p, u16p, u16p, i64]
    ip = ctypes.POINTER(ctypes.c_int)
    l.orc_program.argtypes = [ci, ci, ci, ci, ip, f32p, ip, f32p]
    l.orc_program.restype = ctypes.c_int
    l.orc_sincos_coeffs.argtypes = [ci, ci, ip, f32p, ip, f32p]
    l.orc_sincos_coeffs.restype = ctypes.c_int
    l.orc_activation_bwd_alg.argtypes = [ci, ci, u16p, u16p, u16p, i64]
    l.orc_swish_mul_fwd.argtypes = [ci, ci, ci, u16p, u16p, u16p, i64]
    l.orc_swish_mul_bwd.argtypes = [ci, ci, ci, u16p, u16p, u16p, u16p, u16p, i64]
    l.orc_b3_direct_bf16.argtypes = [u16p, u16p, u16p, u8p, i64]
    l.orc_b3_direct_f32.argtypes = [f32p, u16p, u16p, i64]
    l.orc_b3_constants.argtypes = [u16p, u16p, u16p]
    l.orc_num_threads.argtypes = []
    i32p = ctypes.POINTER(ctypes.c_int32)
    l.orc_b3_exp2_d2_bf16.argtypes = [u16p, u16p, u16p, i64, f32p]
    l.orc_b3_exp2_d2_bf16.restype = ctypes.c_int
    l.orc_softcap_fwd_bf16.argtypes = [u16p, u16p, i64, ctypes.c_float]
    l.orc_softcap_bwd_bf16.argtypes = [u16p, u16p, u16p, i64, ctypes.c_float]
    l.orc_exp2.argtypes = [ci, ci, f32p, u16p, f32p, i64]
    l.orc_exp2_fraction.argtypes = [ci, f32p, f32p, i64]
    l.orc_exp2_fraction.restype = ctypes.c_int
    l.orc_sincos.argtypes = [ci, ci, ci, f32p, u16p, u16p, i64]
    l.orc_rope_sincos_table.argtypes = [i32p, u16p, i64, i64]
    l.orc_rope_apply.argtypes = [ci, u16p, u16p, i32p, u16p, u16p, i64, i64, i64, i64, i64]
    l.orc_sincos_f32.argtypes = [ci, f32p, f32p, f32p, i64, ci]
    l.orc_sincos16.argtypes = [ci, ci, ci, f32p, u16p, u16p, i64, ci]
    l.orc_rope_table.argtypes = [ci, i32p, u16p, u16p, i64, i64, ci]
    l.orc_rope_apply_cached.argtypes = [u16p, u16p, u16p, u16p, u16p, i64, i64, i64, i64, i64]
    l.orc_swish_fwd_deriv_shared.argtypes = [u16p, u16p, u16p, i64]
    l.orc_multiply.argtypes = [ci, u16p, u16p, u16p, i64]
    for name in (
        "orc_activation", "orc_activation_bwd", "orc_activation_bwd_alg",
        "orc_swish_mul_fwd", "orc_swish_mul_bwd", "orc_b3_direct_bf16",
        "orc_b3_direct_f32", "orc_b3_constants", "orc_num_threads", "orc_softcap_fwd_bf16",
        "orc_softcap_bwd_bf16", "orc_exp2", "orc_sincos", "orc_rope_sincos_table",
        "orc_rope_apply", "orc_sincos_f32", "orc_sincos16", "orc_rope_table",
        "orc_rope_apply_cached", "orc_swish_fwd_deriv_shared", "orc_multiply",
    ):
        getattr(l, name).restype = ctypes.c_int


def _u16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype != np.uint16:
        raise TypeError(f"expected uint16 bit patterns, got {a.dtype}")
    return a


def _p(a: np.ndarray, ctype=ctypes.c_uint16):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _check(rc: int) -> None:
    if rc != 0:
        raise ValueError(f"oracle rejected the arguments (code {rc})")


def fmt_id(fmt) -> int:
    if isinstance(fmt, int):
        return fmt
    return _FMT[str(fmt).replace("torch.", "")]


def family_id(family) -> int:
    return family if isinstance(family, int) else _FAMILY[family]


def activation(family, direction: int, degree: int, fmt, x: np.ndarray,
               rnd: int = RND_SINGLE) -> np.ndarray:
    x = _u16(x)
    y = np.empty_like(x)
    _check(lib().orc_activation(family_id(family), direction, degree, fmt_id(fmt), rnd,
                                _p(x), _p(y), x.size))
    return y


SHAPES = {0: "half_odd", 1: "odd", 2: "odd_min1", 3: "swish", 4: "even", 5: "x_times",
          6: "x_half_odd"}


def program(family, direction: int, degree: int, fmt):
    """The oracle's table entry: (shape name, clamp, degree, coefficients
    c[0..degree] as float32 literals)."""
    shape, deg = ctypes.c_int(), ctypes.c_int()
    lc = ctypes.c_float()
    c = (ctypes.c_float * 7)()
    _check(lib().orc_program(family_id(family), direction, degree, fmt_id(fmt),
                             ctypes.byref(shape), ctypes.byref(lc), ctypes.byref(deg), c))
    return SHAPES[shape.value], lc.value, deg.value, [c[i] for i in range(deg.value + 1)]


def sincos_coefficients(table: int, idx: int):
    """(sin coefficients, cos coefficients) of a paired sin/cos program, as
    float32 values, highest power of r^2 first: table 0 the 16-bit half-turn
    programs, 1 the FP32 programs, 2 the 16-bit quarter-turn programs, 3 the
    RoPE Q15 quarter-turn program."""
    ns, nc = ctypes.c_int(), ctypes.c_int()
    s, c = (ctypes.c_float * 4)(), (ctypes.c_float * 4)()
    _check(lib().orc_sincos_coeffs(table, idx, ctypes.byref(ns), s, ctypes.byref(nc), c))
    return [s[i] for i in range(ns.value)], [c[i] for i in range(nc.value)]


def activation_bwd(family, degree: int, fmt, go: np.ndarray, x: np.ndarray,
                   rnd: int = RND_SINGLE) -> np.ndarray:
    go, x = _u16(go), _u16(x)
    gi = np.empty_like(x)
    _check(lib().orc_activation_bwd(family_id(family), degree, fmt_id(fmt), rnd,
                                    _p(go), _p(x), _p(gi), x.size))
    return gi


def activation_bwd_alg(family, fmt, go: np.ndarray, y: np.ndarray) -> np.ndarray:
    go, y = _u16(go), _u16(y)
    gi = np.empty_like(y)
    _check(lib().orc_activation_bwd_alg(family_id(family), fmt_id(fmt), _p(go), _p(y),
                                        _p(gi), y.size))
    return gi


def swish_mul_fwd(degree: int, fmt, gate: np.ndarray, up: np.ndarray,
                  rnd: int = RND_SINGLE) -> np.ndarray:
    gate, up = _u16(gate), _u16(up)
    out = np.empty_like(gate)
    _check(lib().orc_swish_mul_fwd(degree, fmt_id(fmt), rnd, _p(gate), _p(up), _p(out),
                                   gate.size))
    return out


def swish_mul_bwd(degree: int, fmt, go: np.ndarray, gate: np.ndarray, up: np.ndarray,
                  rnd: int = RND_SINGLE):
    go, gate, up = _u16(go), _u16(gate), _u16(up)
    gg = np.empty_like(gate)
    gu = np.empty_like(gate)
    _check(lib().orc_swish_mul_bwd(degree, fmt_id(fmt), rnd, _p(go), _p(gate), _p(up),
                                   _p(gg), _p(gu), gate.size))
    return gg, gu


def b3_direct_bf16(x: np.ndarray, with_row: bool = False):
    x = _u16(x)
    y = np.empty_like(x)
    dy = np.empty_like(x)
    row = np.empty(x.shape, dtype=np.uint8)
    _check(lib().orc_b3_direct_bf16(_p(x), _p(y), _p(dy), _p(row, ctypes.c_uint8), x.size))
    return (y, dy, row) if with_row else (y, dy)


def b3_direct_f32(s: np.ndarray):
    s = np.ascontiguousarray(s, dtype=np.float32)
    y = np.empty(s.shape, dtype=np.uint16)
    dy = np.empty(s.shape, dtype=np.uint16)
    _check(lib().orc_b3_direct_f32(_p(s, ctypes.c_float), _p(y), _p(dy), s.size))
    return y, dy


def b3_exp2_d2_bf16(x: np.ndarray, coeffs) -> tuple:
    x = _u16(x)
    c = np.ascontiguousarray(coeffs, dtype=np.float32)
    y = np.empty_like(x)
    dy = np.empty_like(x)
    _check(lib().orc_b3_exp2_d2_bf16(_p(x), _p(y), _p(dy), x.size, _p(c, ctypes.c_float)))
    return y, dy


def b3_constants():
    fwd = np.empty(8, dtype=np.uint16)
    grad = np.empty(4, dtype=np.uint16)
    sc = np.empty(2, dtype=np.uint16)
    _check(lib().orc_b3_constants(_p(fwd), _p(grad), _p(sc)))
    return fwd.reshape(2, 4), grad.reshape(2, 2), sc


def softcap_fwd_bf16(s: np.ndarray, cap: float) -> np.ndarray:
    s = _u16(s)
    y = np.empty_like(s)
    _check(lib().orc_softcap_fwd_bf16(_p(s), _p(y), s.size, cap))
    return y


def softcap_bwd_bf16(go: np.ndarray, s: np.ndarray, cap: float) -> np.ndarray:
    go, s = _u16(go), _u16(s)
    g = np.empty_like(s)
    _check(lib().orc_softcap_bwd_bf16(_p(go), _p(s), _p(g), s.size, cap))
    return g


EXP2_D2, EXP2_D3, EXP2_PWL2, EXP2_PWL2_SAFE, EXP2_PWL2_SAFE_F16 = 0, 1, 2, 3, 4
(EXP2_PWL1_SAFE, EXP2_PWL1_SAFE_F16, EXP2_PWL2_SAFE_BF16, EXP2_D2_NOCLAMP, EXP2_D2_SAFE_F16,
 EXP2_D2_SAFE_BF16, EXP2_PWL2_F16) = range(5, 12)
# fraction-only program (exp2_fraction): the reference's historical two-segment FP16 fit
EXP2_FRAC_PWL2_HISTORICAL = 12
# FA4 backend name -> oracle kind
EXP2_BACKEND_KIND = {"d2_safe": 0, "d3": 1, "pwl2": 2, "pwl2_safe": 3, "pwl2_safe_f16": 4, "pwl1_safe": 5,
                     "pwl1_safe_f16": 6, "pwl2_safe_bf16": 7, "d2_safe_noclamp": 8, "d2_safe_f16": 9,
                     "d2_safe_bf16": 10, "pwl2_f16": 11}


def exp2(kind: int, x: np.ndarray, out_bf16: bool = True) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y16 = np.empty(x.shape, dtype=np.uint16)
    y32 = np.empty(x.shape, dtype=np.float32)
    _check(lib().orc_exp2(kind, int(out_bf16), _p(x, ctypes.c_float), _p(y16),
                          _p(y32, ctypes.c_float), x.size))
    return y16 if out_bf16 else y32


def exp2_fraction(kind: int, f: np.ndarray) -> np.ndarray:
    """p(f) of an exp2 program's fraction alone (no range reduction)."""
    f = np.ascontiguousarray(f, dtype=np.float32)
    p = np.empty(f.shape, dtype=np.float32)
    _check(lib().orc_exp2_fraction(kind, _p(f, ctypes.c_float), _p(p, ctypes.c_float), f.size))
    return p


# half-turn sin/cos programs (same ids as the device SinCosId enum)
SC_BF16_D3D4, SC_BF16_D5D6, SC_F16_D3D4, SC_F16_D5D4, SC_F16_D5D6, SC_F16_D7D6 = range(6)


def sincos(prog: int, angles: np.ndarray, out_fmt=None, rnd: int = RND_SINGLE):
    """(cos bits, sin bits) of the half-turn program `prog`."""
    a = np.ascontiguousarray(angles, dtype=np.float32)
    if out_fmt is None:
        out_fmt = BF16 if prog in (SC_BF16_D3D4, SC_BF16_D5D6) else F16
    c = np.empty(a.shape, dtype=np.uint16)
    s = np.empty(a.shape, dtype=np.uint16)
    _check(lib().orc_sincos(prog, fmt_id(out_fmt), rnd, _p(a, ctypes.c_float), _p(c), _p(s),
                            a.size))
    return c, s


# every 16-bit program (orc_sincos16): the half-turn ids above plus
SC_F16_QUARTER_D3D4, SC_BF16_QUARTER_D3D4, SC_BF16_CW_D3D4 = 6, 7, 8
# FP32 programs (orc_sincos_f32)
SC32_D3D4, SC32_D3D4_SHIFT, SC32_D5D4, SC32_D7D6 = 0, 1, 2, 3
SC32_HALF_D5D4_LS, SC32_HALF_D5D4_SOLLYA, SC32_HALF_D5D4_SOLLYA_FAST, SC32_CYCLE = 4, 5, 6, 7


def sincos16(prog: int, angles: np.ndarray, out_fmt=None, iterations: int = 0,
             rnd: int = RND_SINGLE):
    """(cos bits, sin bits) of any 16-bit program; iterations > 0 gives the
    compute probe's sums."""
    a = np.ascontiguousarray(angles, dtype=np.float32)
    if out_fmt is None:
        out_fmt = BF16 if prog in (SC_BF16_D3D4, SC_BF16_D5D6, SC_BF16_QUARTER_D3D4,
                                   SC_BF16_CW_D3D4) else F16
    c = np.empty(a.shape, dtype=np.uint16)
    s = np.empty(a.shape, dtype=np.uint16)
    _check(lib().orc_sincos16(prog, fmt_id(out_fmt), rnd, _p(a, ctypes.c_float), _p(c), _p(s),
                              a.size, iterations))
    return c, s


def sincos_f32(prog: int, angles: np.ndarray, iterations: int = 0):
    """(cos, sin) float32 of an FP32 program; iterations > 0: probe sums."""
    a = np.ascontiguousarray(angles, dtype=np.float32)
    c = np.empty(a.shape, dtype=np.float32)
    s = np.empty(a.shape, dtype=np.float32)
    _check(lib().orc_sincos_f32(prog, _p(a, ctypes.c_float), _p(c, ctypes.c_float),
                                _p(s, ctypes.c_float), a.size, iterations))
    return c, s


ROPE_HALF_D5D6, ROPE_QUARTER_D3D4, ROPE_LUT = 0, 1, 2


def rope_table(kind: int, inc: np.ndarray, seq: int, lut: np.ndarray = None,
               iterations: int = 0) -> np.ndarray:
    """[2, seq, F] FP16 bits of a RoPE table program (or its probe sums)."""
    inc = np.ascontiguousarray(inc, dtype=np.int32)
    out = np.empty((2, seq, inc.size), dtype=np.uint16)
    lp = None
    if lut is not None:
        lut = _u16(lut)
        lp = _p(lut)
    _check(lib().orc_rope_table(kind, _p(inc, ctypes.c_int32), lp, _p(out), seq, inc.size,
                                iterations))
    return out


def rope_apply_cached(q: np.ndarray, k: np.ndarray, table: np.ndarray):
    """FP16 q [B,S,Hq,D], k [B,S,Hk,D] rotated by a [2,S,D/2] FP16 table."""
    q, k, table = _u16(q), _u16(k), _u16(table)
    b, s, hq, d = q.shape
    hk = k.shape[2]
    qo = np.empty((b, hq, s, d), dtype=np.uint16)
    ko = np.empty((b, hk, s, d), dtype=np.uint16)
    _check(lib().orc_rope_apply_cached(_p(q), _p(k), _p(table), _p(qo), _p(ko), b, s, hq, hk, d))
    return qo, ko


def rope_sincos_table(inc: np.ndarray, seq: int) -> np.ndarray:
    inc = np.ascontiguousarray(inc, dtype=np.int32)
    out = np.empty((2, seq, inc.size), dtype=np.uint16)
    _check(lib().orc_rope_sincos_table(_p(inc, ctypes.c_int32), _p(out), seq, inc.size))
    return out


def rope_apply(fmt, q: np.ndarray, k: np.ndarray, inc: np.ndarray):
    """q [B,S,Hq,D], k [B,S,Hk,D] bit patterns -> ([B,Hq,S,D], [B,Hk,S,D])."""
    q, k = _u16(q), _u16(k)
    inc = np.ascontiguousarray(inc, dtype=np.int32)
    b, s, hq, d = q.shape
    hk = k.shape[2]
    qo = np.empty((b, hq, s, d), dtype=np.uint16)
    ko = np.empty((b, hk, s, d), dtype=np.uint16)
    _check(lib().orc_rope_apply(fmt_id(fmt), _p(q), _p(k), _p(inc, ctypes.c_int32), _p(qo), _p(ko),
                                b, s, hq, hk, d))
    return qo, ko


def swish_fwd_deriv_shared(x: np.ndarray):
    """FP16 (y, dy) of the shared-sigmoid SiLU forward-with-derivative."""
    x = _u16(x)
    y = np.empty_like(x)
    dy = np.empty_like(x)
    _check(lib().orc_swish_fwd_deriv_shared(_p(x), _p(y), _p(dy), x.size))
    return y, dy


def multiply(fmt, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a, b = _u16(a), _u16(b)
    out = np.empty_like(a)
    _check(lib().orc_multiply(fmt_id(fmt), _p(a), _p(b), _p(out), a.size))
    return out


# ---- RoPE reference evaluator (src/sfu_repro/rope/polynomial_sincos.py:85-165)
# A numpy restatement with the same operation sequence: every numpy float32 /
# float64 operation is one IEEE round-to-nearest-even step, as the
# reference's tensor arithmetic is.

def ref_reduce_to_quarter_turn(angles: np.ndarray, accurate: bool = True):
    """(float32 residual, int64 quadrant 0..3)  (polynomial_sincos.py:85-122)."""
    with np.errstate(invalid="ignore", over="ignore"):
        if accurate:
            work = np.asarray(angles).astype(np.float64)
            q = np.rint(work * (2.0 / np.pi))
            reduced = work - q * (np.pi / 2.0)
        else:
            work = np.asarray(angles).astype(np.float32)
            q = np.rint(work * np.float32(2.0 / np.pi))
            reduced = (work - q * np.float32(1.570796251296997)) - q * np.float32(7.549789415861596e-08)
        qi = np.where(np.abs(q) < 2.0 ** 63, q, 0).astype(np.int64)
        qi = np.where(np.abs(q) < 2.0 ** 63, qi, np.iinfo(np.int64).min)
    return reduced.astype(np.float32), qi & 3


def _ref_horner(x: np.ndarray, coefficients) -> np.ndarray:
    value = np.full_like(x, np.float32(coefficients[-1]))
    for c in reversed(coefficients[:-1]):
        value = value * x + np.float32(c)
    return value


def ref_evaluate_reduced_sincos(reduced: np.ndarray, sin_coefficients, cos_coefficients):
    """(sin, cos) float32 of reduced arguments (polynomial_sincos.py:125-135)."""
    r = np.asarray(reduced).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        sq = r * r
        return r * _ref_horner(sq, sin_coefficients), _ref_horner(sq, cos_coefficients)


def ref_polynomial_sincos(angles: np.ndarray, sin_coefficients, cos_coefficients,
                          accurate: bool = True):
    """(cos, sin) float32 (polynomial_sincos.py:138-165)."""
    reduced, q = ref_reduce_to_quarter_turn(angles, accurate)
    s, c = ref_evaluate_reduced_sincos(reduced, sin_coefficients, cos_coefficients)
    swap = (q & 1).astype(bool)
    sm = np.where(swap, c, s)
    cm = np.where(swap, s, c)
    sin = np.where((q & 2).astype(bool), -sm, sm)
    cos = np.where(((q + 1) & 2).astype(bool), -cm, cm)
    return cos.astype(np.float32), sin.astype(np.float32)


def rope_phase_increments(head_dim: int, theta: float) -> np.ndarray:
    """round(omega_i * 2^32 / (2 pi)) as int32, omega_i = theta^(-2i/head_dim)
    (src/sfu_repro/rope/benchmark_cuda_fused_rope.py:238-241)."""
    dims = np.arange(0, head_dim, 2, dtype=np.float64)
    omega = theta ** (-dims / head_dim)
    return np.round(omega * (2.0 ** 32) / (2.0 * np.pi)).astype(np.int64).astype(np.int32)


def num_threads() -> int:
    return int(lib().orc_num_threads())


# ---- bit-pattern helpers ---------------------------------------------------

def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """RNE float32 -> BF16 bit patterns (NaN kept quiet)."""
    u = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7F800000) == 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    keep = (u >> 16).astype(np.uint16) | np.where((u & 0x7FFFFF) != 0, 0x40, 0).astype(np.uint16)
    return np.where(nan, keep, r).astype(np.uint16)


def f16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return np.asarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def bits_to_f32(b: np.ndarray, fmt) -> np.ndarray:
    return f16_bits_to_f32(b) if fmt_id(fmt) == F16 else bf16_bits_to_f32(b)


def all_bits() -> np.ndarray:
    """Every 16-bit pattern, 0..65535."""
    return np.arange(65536, dtype=np.uint32).astype(np.uint16)
