"""Python face of the CPU oracle.  TEST INFRASTRUCTURE ONLY.

Only tests/, the smoke check and bench.py's CPU-baseline leg import this module.  It wraps
two checker libraries built by oracle/Makefile:

* ``libkq_oracle.so`` -- the repo's C restatement (kq_oracle.c) of the Kindi CPU path
  (q4kernels.h:12-83, kcpu4.c:337-341) and of GGML's Q8_K quantizer and integer dots.
* ``_ref/libkcpu4.so`` -- the reference's own kcpu4.c compiled from its sources, used to pin
  the restatement (``kc_matvec``/``kc_dequant``, kcpu4.c:337-341, with the ``Mat`` struct of
  kcpu4.c:26 / cpu4.py:28-29).  Absent when it was never built; callers then skip.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
QK = 256
BLOCK = {12: 144, 14: 210}
Q8K_BYTES = 292

_PU8 = C.POINTER(C.c_uint8)
_PF = C.POINTER(C.c_float)
_PD = C.POINTER(C.c_double)
_PI32 = C.POINTER(C.c_int32)


def _p(a, t):
    return a.ctypes.data_as(t)


def build():
    """Compile the oracle (and the reference library when its sources are present)."""
    subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(HERE, "libkq_oracle.so")
        if not os.path.exists(path):
            raise RuntimeError("oracle library not built: run `make -C oracle`")
        L = C.CDLL(path)
        L.kqo_decode_block.argtypes = [_PU8, C.c_int, _PF]
        L.kqo_dequant_row.argtypes = [_PU8, C.c_int, C.c_int, C.c_int, C.c_int, _PF]
        L.kqo_dot_f32.argtypes = [_PU8, C.c_int, C.c_int, C.c_int, _PF]
        L.kqo_dot_f32.restype = C.c_float
        L.kqo_matvec_f32.argtypes = [_PU8, C.c_int, C.c_int, C.c_int, _PF, _PF]
        L.kqo_quantize_q8k.argtypes = [_PF, C.c_int64, _PU8]
        L.kqo_subblock_sums.argtypes = [_PU8, C.c_int, C.c_int, C.c_int, _PU8, C.c_int, _PI32]
        L.kqo_gemv_q8k.argtypes = [_PU8, C.c_int, C.c_int, C.c_int, _PU8, C.c_int, _PD, C.c_int64]
        L.kqo_gemv_q8k_ggml.argtypes = [_PU8, C.c_int, C.c_int, C.c_int, _PU8, C.c_int, _PF, C.c_int64]
        L.kqo_expf.argtypes = [C.c_float]
        L.kqo_expf.restype = C.c_float
        L.kqo_rms_norm.argtypes = [_PF, _PF, C.c_int, _PF, C.c_int, _PF, C.c_int]
        L.kqo_swiglu.argtypes = [_PF, _PF, C.c_int64, _PF]
        L.kqo_expf_n.argtypes = [_PF, C.c_int64, _PF]
        L.kqo_argmax.argtypes = [_PF, C.c_int64]
        L.kqo_argmax.restype = C.c_int
        _lib = L
    return _lib


def _u8(a):
    a = np.ascontiguousarray(a)
    assert a.dtype == np.uint8
    return a


def decode_block(b, ty):
    out = np.empty(QK, np.float32)
    lib().kqo_decode_block(_p(_u8(b), _PU8), ty, _p(out, _PF))
    return out


def dequant_row(W, R, C_, ty, row):
    out = np.empty(C_, np.float32)
    lib().kqo_dequant_row(_p(_u8(W), _PU8), R, C_, ty, row, _p(out, _PF))
    return out


def dequant(W, R, C_, ty):
    return np.stack([dequant_row(W, R, C_, ty, r) for r in range(R)])


def matvec_f32(W, R, C_, ty, x):
    """Kindi fp32-activation GEMV in q4_dot's lane order (q4kernels.h:37-71)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(R, np.float32)
    lib().kqo_matvec_f32(_p(_u8(W), _PU8), R, C_, ty, _p(x, _PF), _p(y, _PF))
    return y


def quantize_q8k(x):
    """GGML quantize_row_q8_K_ref per row of x [N][C] -> uint8 [N][C/256*292]."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    N, C_ = x.shape
    out = np.empty((N, C_ // QK * Q8K_BYTES), np.uint8)
    lib().kqo_quantize_q8k(_p(x, _PF), N * C_, _p(out, _PU8))
    return out


def q8k_fields(xq):
    """Split Q8_K bytes [..., G*292] into (d float32 [...,G], qs int8 [...,G,256], bsums int16 [...,G,16])."""
    xq = np.ascontiguousarray(xq)
    b = xq.reshape(xq.shape[:-1] + (-1, Q8K_BYTES))
    d = b[..., 0:4].copy().view(np.float32)[..., 0]
    qs = b[..., 4:260].copy().view(np.int8)
    bs = b[..., 260:292].copy().view(np.int16)
    return d, qs, bs


def subblock_sums(W, R, C_, ty, xq, N):
    nsub = 8 if ty == 12 else 16
    S = np.empty((N, R, C_ // QK, nsub), np.int32)
    lib().kqo_subblock_sums(_p(_u8(W), _PU8), R, C_, ty, _p(_u8(xq), _PU8), N, _p(S, _PI32))
    return S


def gemv_q8k(W, R, C_, ty, xq, N):
    """Y[N][R] in double from the exact integer sub-block sums."""
    y = np.empty((N, R), np.float64)
    lib().kqo_gemv_q8k(_p(_u8(W), _PU8), R, C_, ty, _p(_u8(xq), _PU8), N, _p(y, _PD), R)
    return y


def gemv_q8k_ggml(W, R, C_, ty, xq, N):
    """Y[N][R] with GGML's generic fp32 accumulation order."""
    y = np.empty((N, R), np.float32)
    lib().kqo_gemv_q8k_ggml(_p(_u8(W), _PU8), R, C_, ty, _p(_u8(xq), _PU8), N, _p(y, _PF), R)
    return y


# ------------------------------------------------------------------ the reference's own CPU path
class Mat(C.Structure):
    """kcpu4.c:26 / cpu4.py:28-29."""
    _fields_ = [("W", _PU8), ("S", _PF), ("R", C.c_int), ("C", C.c_int), ("type", C.c_int),
                ("offset", C.c_uint64), ("bytes", C.c_uint64)]


_ref = None


def ref_path():
    return os.path.join(HERE, "_ref", "libkcpu4.so")


def ref_available():
    return os.path.exists(ref_path())


def ref():
    global _ref
    if _ref is None:
        L = C.CDLL(ref_path())
        L.kc_matvec.argtypes = [C.POINTER(Mat), _PF, _PF]
        L.kc_dequant.argtypes = [C.POINTER(Mat), C.c_int, _PF]
        _ref = L
    return _ref


def ref_mat(W, R, C_, ty):
    W = _u8(W)
    return Mat(_p(W, _PU8), None, R, C_, ty, 0, W.nbytes), W


def ref_matvec(W, R, C_, ty, x):
    m, keep = ref_mat(W, R, C_, ty)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(R, np.float32)
    ref().kc_matvec(C.byref(m), _p(x, _PF), _p(y, _PF))
    return y


def ref_dequant_row(W, R, C_, ty, row):
    m, keep = ref_mat(W, R, C_, ty)
    y = np.empty(C_, np.float32)
    ref().kc_dequant(C.byref(m), row, _p(y, _PF))
    return y


# ---------------------------------------------------------------- producers of the GEMV inputs
def expf(x):
    """The library's binary32 exp, elementwise (kqo_expf)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().kqo_expf_n(_p(x, _PF), x.size, _p(y, _PF))
    return y


def rms_norm(h, w, residual=None, order=0):
    """q4_rms per row of h [N][D] (order 0: that kernel's double-sum order; 1: the CPU engine's
    sequential sum).  Returns (h after the residual add, xn)."""
    h = np.array(np.atleast_2d(h), np.float32, order="C")
    w = np.ascontiguousarray(w, np.float32)
    N, D = h.shape
    res = None if residual is None else np.ascontiguousarray(np.atleast_2d(residual), np.float32)
    xn = np.empty_like(h)
    for n in range(N):
        hr = h[n].copy()
        rr = res[n] if res is not None else hr
        lib().kqo_rms_norm(_p(hr, _PF), _p(np.ascontiguousarray(rr), _PF), 1 if res is not None else 0,
                           _p(w, _PF), D, _p(xn[n], _PF), order)
        h[n] = hr
    return h, xn


def swiglu(g, u):
    """silu(g) * u elementwise (kqo_swiglu)."""
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    y = np.empty_like(g)
    lib().kqo_swiglu(_p(g, _PF), _p(u, _PF), g.size, _p(y, _PF))
    return y


def argmax(y):
    """k_argmax's pick over y (kqo_argmax)."""
    y = np.ascontiguousarray(y, np.float32).reshape(-1)
    return int(lib().kqo_argmax(_p(y, _PF), y.size))
