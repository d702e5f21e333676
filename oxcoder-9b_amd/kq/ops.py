"""Tensor-level calls into libkq on torch-ROCm device tensors.

torch supplies device memory and the current stream; every computation runs in libkq's HIP
kernels through the C ABI of include/kq.h.  Shapes are checked here (ValueError) before any
launch, and a nonzero status from the library raises (ValueError for bad arguments, KQError for
HIP failures).
"""
import ctypes as C

import torch

from . import _lib
from .formats import BLOCK, Q8K_BYTES, QK, check_shape


def _stream(device):
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _dev(t, name, dtype=None):
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError("%s must be a device tensor" % name)
    if dtype is not None and t.dtype != dtype:
        raise ValueError("%s must be %s, got %s" % (name, dtype, t.dtype))
    if t.dim() > 0 and t.shape[-1] > 1 and t.stride(-1) != 1:
        # kernels read consecutive elements of a row; rows may be strided (ld arguments)
        raise ValueError("%s must have unit stride along its last dimension" % name)
    return C.c_void_p(t.data_ptr())


def _weights(w, R, C_, ty):
    check_shape(R, C_, ty)
    if w.dtype != torch.uint8 or not w.is_contiguous():
        raise ValueError("weights must be a contiguous uint8 tensor")
    if w.numel() < R * (C_ // QK) * BLOCK[ty]:
        raise ValueError("weight buffer holds %d bytes, %dx%d type %d needs %d"
                         % (w.numel(), R, C_, ty, R * (C_ // QK) * BLOCK[ty]))
    return _dev(w, "w")


def gemv(w, R, C_, ty, x, y):
    """y[R] = W x with fp32 x[C] (Kindi numerics, kq_gemv)."""
    pw = _weights(w, R, C_, ty)
    if x.numel() < C_ or y.numel() < R:
        raise ValueError("x or y too small")
    _lib.check(_lib.kq().kq_gemv(pw, R, C_, ty, _dev(x, "x", torch.float32), _dev(y, "y", torch.float32),
                                 _stream(w.device)))
    return y


def gemv_multi(mats, x, ys):
    """Up to 3 matrices [(w, R, C, type)] sharing fp32 x [C], one launch per type, or one for both
    types at C <= 4096 when one type has a single matrix (kq_gemv_multi; the multi-matrix gemv of
    the CPU engine, kcpu4.c:100-118)."""
    n = len(mats)
    if not 1 <= n <= 3 or len(ys) != n:
        raise ValueError("1..3 matrices with one output each")
    C_ = mats[0][2]
    if any(m[2] != C_ for m in mats) or x.numel() < C_:
        raise ValueError("matrices sharing an input must have the same column count")
    W = (C.c_void_p * n)(*[_weights(w, R, C_, ty).value for (w, R, _, ty) in mats])
    Rs = (C.c_int * n)(*[m[1] for m in mats])
    Ts = (C.c_int * n)(*[m[3] for m in mats])
    for (w, R, _, ty), y in zip(mats, ys):
        if y.numel() < R:
            raise ValueError("output too small")
    Y = (C.c_void_p * n)(*[_dev(y, "y", torch.float32).value for y in ys])
    _lib.check(_lib.kq().kq_gemv_multi(n, W, Rs, C_, Ts, _dev(x, "x", torch.float32), Y, _stream(mats[0][0].device)))
    return ys


def q8k_quantize(x, out=None):
    """x [N][C] fp32 (row stride x.stride(0)) -> Q8_K bytes uint8 [N][C/256*292]."""
    if x.dim() == 1:
        x = x.unsqueeze(0)
    N, C_ = x.shape
    if x.stride(1) != 1:
        raise ValueError("x rows must be contiguous")
    if out is None:
        out = torch.empty((N, C_ // QK * Q8K_BYTES), dtype=torch.uint8, device=x.device)
    elif out.numel() < N * (C_ // QK) * Q8K_BYTES:
        raise ValueError("out too small for %d Q8_K rows of %d" % (N, C_))
    _lib.check(_lib.kq().kq_q8k_quantize(_dev(x, "x", torch.float32), x.stride(0), C_, N,
                                         _dev(out, "out", torch.uint8), _stream(x.device)))
    return out


def _rows(x, name):
    """[N][n] fp32 device rows (1-D: one row) with contiguous rows; returns (2-D view, N, n, ld)."""
    if x.dim() == 1:
        x = x.unsqueeze(0)
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("%s must be [N][n] with contiguous rows" % name)
    _dev(x, name, torch.float32)
    return x, x.shape[0], x.shape[1], x.stride(0)


def _q8k_out(xq, N, n, device):
    if xq is None:
        return torch.empty((N, n // QK * Q8K_BYTES), dtype=torch.uint8, device=device)
    if xq.numel() < N * (n // QK) * Q8K_BYTES:
        raise ValueError("xq too small for %d Q8_K rows of %d" % (N, n))
    return xq


def rms_q8k(h, w, residual=None, xn=None, xq=None):
    """RMSNorm of the rows of h (in place residual add when ``residual`` is given), writing the
    Q8_K blocks of xn = (h * s) * w and, if ``xn`` is given, xn itself (kq_rms_q8k; q4_rms,
    q4.cu:39-46).  Returns (xn, xq)."""
    h2, N, D, ld = _rows(h, "h")
    if w.numel() < D:
        raise ValueError("w must hold D=%d floats" % D)
    for t, name in ((residual, "residual"), (xn, "xn")):
        if t is not None:
            t2, n2, d2, ld2 = _rows(t, name)
            if (n2, d2, ld2) != (N, D, ld):
                raise ValueError("%s must have the shape and row stride of h" % name)
    xq = _q8k_out(xq, N, D, h.device)
    _lib.check(_lib.kq().kq_rms_q8k(C.c_void_p(h2.data_ptr()),
                                    C.c_void_p(residual.data_ptr()) if residual is not None else None,
                                    1 if residual is not None else 0, _dev(w, "w", torch.float32), D, N, ld,
                                    C.c_void_p(xn.data_ptr()) if xn is not None else None,
                                    _dev(xq, "xq", torch.uint8), _stream(h.device)))
    return xn, xq


def swiglu_q8k(gate, up, y=None, xq=None):
    """Q8_K blocks of y = silu(gate) * up and, if ``y`` is given, y itself (kq_swiglu_q8k;
    q4_silu, q4.cu:36-38).  Returns (y, xq)."""
    g2, N, n, ld = _rows(gate, "gate")
    for t, name in ((up, "up"), (y, "y")):
        if t is not None:
            t2, n2, d2, ld2 = _rows(t, name)
            if (n2, d2, ld2) != (N, n, ld):
                raise ValueError("%s must have the shape and row stride of gate" % name)
    xq = _q8k_out(xq, N, n, gate.device)
    _lib.check(_lib.kq().kq_swiglu_q8k(C.c_void_p(g2.data_ptr()), _dev(up, "up", torch.float32), n, N, ld,
                                       C.c_void_p(y.data_ptr()) if y is not None else None,
                                       _dev(xq, "xq", torch.uint8), _stream(gate.device)))
    return y, xq


def argmax_workspace(device):
    """Zero-filled workspace for argmax / gemv_q8k_argmax (kq_argmax_workspace() bytes, 256-aligned)."""
    n = int(_lib.kq().kq_argmax_workspace())
    buf = torch.zeros(n + 256, dtype=torch.uint8, device=device)
    off = (-buf.data_ptr()) % 256
    return buf[off:off + n]


def argmax(y, ws, out=None):
    """Index of the largest y (k_argmax's rule) into out (device int32[1]); returns out."""
    y = y.reshape(-1)
    if y.stride(0) != 1:
        raise ValueError("y must be contiguous")
    out = torch.empty(1, dtype=torch.int32, device=y.device) if out is None else out
    _lib.check(_lib.kq().kq_argmax(_dev(y, "y", torch.float32), y.numel(), _dev(ws, "ws", torch.uint8),
                                   _dev(out, "out", torch.int32), _stream(y.device)))
    return out


def gemv_q8k_argmax(w, R, C_, ty, xq, y, ws, out=None):
    """y = W xq (one Q8_K token) and out = argmax(y), fused (kq_gemv_q8k_argmax); returns out."""
    pw = _weights(w, R, C_, ty)
    if xq.numel() < (C_ // QK) * Q8K_BYTES or y.numel() < R:
        raise ValueError("xq or y too small")
    out = torch.empty(1, dtype=torch.int32, device=w.device) if out is None else out
    _lib.check(_lib.kq().kq_gemv_q8k_argmax(pw, R, C_, ty, _dev(xq, "xq", torch.uint8), _dev(y, "y", torch.float32),
                                            _dev(ws, "ws", torch.uint8), _dev(out, "out", torch.int32),
                                            _stream(w.device)))
    return out


def gemv_q8k(w, R, C_, ty, xq, N, y, ldy=None):
    """Y[n][r] for N Q8_K activation rows (kq_gemv_q8k, N <= 16)."""
    pw = _weights(w, R, C_, ty)
    ldy = R if ldy is None else ldy
    if xq.numel() < N * (C_ // QK) * Q8K_BYTES or y.numel() < (N - 1) * ldy + R:
        raise ValueError("xq or y too small")
    _lib.check(_lib.kq().kq_gemv_q8k(pw, R, C_, ty, _dev(xq, "xq", torch.uint8), N,
                                     _dev(y, "y", torch.float32), ldy, _stream(w.device)))
    return y


def gemv_q8k_x(mats, x, ys, xq=None):
    """Up to 3 matrices [(w, R, C, type)] sharing one fp32 activation x[C] (16-byte aligned), one token,
    x quantized to Q8_K inside the GEMV launch (kq_gemv_q8k_x).  ``xq`` (uint8, C/256*292 bytes)
    receives the Q8_K bytes when given; it is required for C > 4096."""
    n = len(mats)
    if not 1 <= n <= 3 or len(ys) != n:
        raise ValueError("1..3 matrices with one output each")
    C_ = mats[0][2]
    if any(m[2] != C_ for m in mats):
        raise ValueError("matrices sharing an input must have the same column count")
    if x.numel() < C_:
        raise ValueError("x too small")
    W = (C.c_void_p * n)(*[_weights(w, R, C_, ty).value for (w, R, _, ty) in mats])
    Rs = (C.c_int * n)(*[m[1] for m in mats])
    Ts = (C.c_int * n)(*[m[3] for m in mats])
    for (w, R, _, ty), y in zip(mats, ys):
        if y.numel() < R:
            raise ValueError("output too small")
    Y = (C.c_void_p * n)(*[_dev(y, "y", torch.float32).value for y in ys])
    pq = None
    if xq is not None:
        if xq.numel() < (C_ // QK) * Q8K_BYTES:
            raise ValueError("xq too small")
        pq = _dev(xq, "xq", torch.uint8)
    _lib.check(_lib.kq().kq_gemv_q8k_x(n, W, Rs, C_, Ts, _dev(x, "x", torch.float32), Y, pq,
                                       _stream(mats[0][0].device)))
    return ys


def gemv_q8k_multi(mats, xq, N, ys):
    """Up to 3 matrices [(w, R, C, type)] sharing one Q8_K input, one launch per type, or one for
    both types at one token and C <= 4096 when one type has a single matrix (kq_gemv_q8k_multi).
    ys[i] is [N][ld_i] or [R_i]."""
    n = len(mats)
    if not 1 <= n <= 3 or len(ys) != n:
        raise ValueError("1..3 matrices with one output each")
    C_ = mats[0][2]
    if any(m[2] != C_ for m in mats):
        raise ValueError("matrices sharing an input must have the same column count")
    W = (C.c_void_p * n)(*[_weights(w, R, C_, ty).value for (w, R, _, ty) in mats])
    Rs = (C.c_int * n)(*[m[1] for m in mats])
    Ts = (C.c_int * n)(*[m[3] for m in mats])
    lds = []
    for (w, R, _, ty), y in zip(mats, ys):
        ld = y.stride(0) if y.dim() == 2 else R
        if y.numel() < (N - 1) * ld + R:
            raise ValueError("output too small")
        lds.append(ld)
    Y = (C.c_void_p * n)(*[_dev(y, "y", torch.float32).value for y in ys])
    L = (C.c_int64 * n)(*lds)
    if xq.numel() < N * (C_ // QK) * Q8K_BYTES:
        raise ValueError("xq too small")
    _lib.check(_lib.kq().kq_gemv_q8k_multi(n, W, Rs, C_, Ts, _dev(xq, "xq", torch.uint8), N, Y, L,
                                           _stream(mats[0][0].device)))
    return ys


def gemm_workspace_bytes(R, C_, M):
    """Device bytes of workspace a prefill GEMM of R weight rows x C_ columns over M activation rows
    needs (activation fragments, and the K split's partial sums when it splits)."""
    return int(_lib.kq().kq_gemm_q8k_workspace(R, C_, M))


def gemm_workspace(R, C_, M, device):
    """A workspace tensor for gemm_q8k (kq_gemm_q8k_workspace bytes, 256-byte aligned)."""
    return torch.empty(gemm_workspace_bytes(R, C_, M) + 256, dtype=torch.uint8, device=device)


def _aligned(ws, n):
    off = (-ws.data_ptr()) % 256
    if ws.numel() - off < n:
        raise ValueError("workspace holds %d usable bytes, %d needed" % (ws.numel() - off, n))
    return C.c_void_p(ws.data_ptr() + off), ws.numel() - off


def gemm_q8k(w, R, C_, ty, xq, M, y, ldy=None, ws=None):
    """Y[m][r] for M Q8_K activation rows (prefill).  With ``ws`` (a device uint8 tensor of at least
    gemm_workspace_bytes + 256 bytes) this is the faster kq_gemm_q8k_ws; without it, kq_gemm_q8k
    (operands read straight from the Q8_K rows).  Neither allocates."""
    pw = _weights(w, R, C_, ty)
    ldy = R if ldy is None else ldy
    if xq.numel() < M * (C_ // QK) * Q8K_BYTES or y.numel() < (M - 1) * ldy + R:
        raise ValueError("xq or y too small")
    px, py, st = _dev(xq, "xq", torch.uint8), _dev(y, "y", torch.float32), _stream(w.device)
    if ws is None:
        _lib.check(_lib.kq().kq_gemm_q8k(pw, R, C_, ty, px, M, py, ldy, st))
    else:
        _dev(ws, "ws", torch.uint8)
        pws, nws = _aligned(ws, gemm_workspace_bytes(R, C_, M))
        _lib.check(_lib.kq().kq_gemm_q8k_ws(pw, R, C_, ty, px, M, py, ldy, pws, nws, st))
    return y


def gemm_multi_workspace_bytes(Rs, C_, M):
    """Device bytes of workspace gemm_q8k_multi needs for matrices of Rs rows sharing M activation
    rows of C_ columns (kq_gemm_q8k_multi_workspace)."""
    n = len(Rs)
    return int(_lib.kq().kq_gemm_q8k_multi_workspace(n, (C.c_int * n)(*Rs), C_, M))


def gemm_q8k_multi(mats, xq, M, ys, ws):
    """Prefill GEMM of up to 3 matrices [(w, R, C, type)] sharing M Q8_K activation rows, one
    fragment copy and one GEMM launch per type (kq_gemm_q8k_multi_ws); ys[i] is [M][ld_i] or flat
    (rows of R_i); ws a device uint8 tensor of at least gemm_multi_workspace_bytes + 256 bytes.
    Each ys[i] equals gemm_q8k(..., ws=...) of that matrix alone, bit for bit."""
    n = len(mats)
    if not 1 <= n <= 3 or len(ys) != n:
        raise ValueError("1..3 matrices with one output each")
    C_ = mats[0][2]
    if any(m[2] != C_ for m in mats):
        raise ValueError("matrices sharing an input must have the same column count")
    if xq.numel() < M * (C_ // QK) * Q8K_BYTES:
        raise ValueError("xq too small")
    W = (C.c_void_p * n)(*[_weights(w, R, C_, ty).value for (w, R, _, ty) in mats])
    Rs = (C.c_int * n)(*[m[1] for m in mats])
    Ts = (C.c_int * n)(*[m[3] for m in mats])
    lds = []
    for (w, R, _, ty), y in zip(mats, ys):
        ld = y.stride(0) if y.dim() == 2 else R
        if y.numel() < (M - 1) * ld + R:
            raise ValueError("output too small")
        lds.append(ld)
    Y = (C.c_void_p * n)(*[_dev(y, "y", torch.float32).value for y in ys])
    L = (C.c_int64 * n)(*lds)
    _dev(ws, "ws", torch.uint8)
    pws, nws = _aligned(ws, gemm_multi_workspace_bytes([m[1] for m in mats], C_, M))
    _lib.check(_lib.kq().kq_gemm_q8k_multi_ws(n, W, Rs, C_, Ts, _dev(xq, "xq", torch.uint8), M, Y, L, pws, nws,
                                              _stream(mats[0][0].device)))
    return ys


def gemm_f32_multi_workspace_bytes(Rs, C_, M):
    """Device bytes of workspace gemm_f32_multi needs (kq_gemm_f32_multi_workspace)."""
    n = len(Rs)
    return int(_lib.kq().kq_gemm_f32_multi_workspace(n, (C.c_int * n)(*Rs), C_, M))


def gemm_f32_multi(mats, X, ys, ws):
    """Prefill GEMM of up to 3 matrices [(w, R, C, type)] on fp32 activations X [M][C] (unit stride
    along C): one launch quantizes X into the workspace (Q8_K rows and the fragment copy), then one
    GEMM launch per type (kq_gemm_f32_multi).  ys[i] is [M][ld_i] or flat (rows of R_i); ws a device
    uint8 tensor of at least gemm_f32_multi_workspace_bytes + 256 bytes."""
    n = len(mats)
    if not 1 <= n <= 3 or len(ys) != n:
        raise ValueError("1..3 matrices with one output each")
    M, C_ = X.shape
    if any(m[2] != C_ for m in mats):
        raise ValueError("matrices sharing an input must have its column count")
    if X.stride(1) != 1:
        raise ValueError("X needs unit stride along its rows")
    W = (C.c_void_p * n)(*[_weights(w, R, C_, ty).value for (w, R, _, ty) in mats])
    Rs = (C.c_int * n)(*[m[1] for m in mats])
    Ts = (C.c_int * n)(*[m[3] for m in mats])
    lds = []
    for (w, R, _, ty), y in zip(mats, ys):
        ld = y.stride(0) if y.dim() == 2 else R
        if y.numel() < (M - 1) * ld + R:
            raise ValueError("output too small")
        lds.append(ld)
    Y = (C.c_void_p * n)(*[_dev(y, "y", torch.float32).value for y in ys])
    L = (C.c_int64 * n)(*lds)
    _dev(ws, "ws", torch.uint8)
    pws, nws = _aligned(ws, gemm_f32_multi_workspace_bytes([m[1] for m in mats], C_, M))
    _lib.check(_lib.kq().kq_gemm_f32_multi(n, W, Rs, C_, Ts, _dev(X, "X", torch.float32), X.stride(0), M, Y, L,
                                           pws, nws, _stream(mats[0][0].device)))
    return ys


def subblock_sums(w, R, C_, ty, xq, N):
    """Exact int32 sub-block sums [N][R][G][8 or 16] (kq_subblock_sums)."""
    pw = _weights(w, R, C_, ty)
    nsub = 8 if ty == 12 else 16
    S = torch.empty((N, R, C_ // QK, nsub), dtype=torch.int32, device=w.device)
    _lib.check(_lib.kq().kq_subblock_sums(pw, R, C_, ty, _dev(xq, "xq", torch.uint8), N,
                                          _dev(S, "S", torch.int32), _stream(w.device)))
    return S


def dequant_rows(w, R, C_, ty, row0, nrows, y=None):
    """Rows row0..row0+nrows-1 decoded to fp32 [nrows][C] (kq_dequant_rows)."""
    pw = _weights(w, R, C_, ty)
    if y is None:
        y = torch.empty((nrows, C_), dtype=torch.float32, device=w.device)
    ld = y.stride(0) if y.dim() == 2 else C_
    if y.numel() < (nrows - 1) * ld + C_:
        raise ValueError("y holds %d floats, %d rows of %d need %d" % (y.numel(), nrows, C_, (nrows - 1) * ld + C_))
    _lib.check(_lib.kq().kq_dequant_rows(pw, R, C_, ty, row0, nrows, _dev(y, "y", torch.float32), ld,
                                         _stream(w.device)))
    return y
