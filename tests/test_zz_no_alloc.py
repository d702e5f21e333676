"""kq_gemm_q8k_static (the entry point that allocates nothing) against kq_gemm_q8k_ws, through the
C ABI: bit-identical outputs on two calls in a row, the second with a smaller input (the static
array keeps the first call's contents, which must not leak into the second), including K-split
GEMMs whose partial sums live in the array; sizes beyond the array rejected before any launch."""
import ctypes as ct

import numpy as np
import pytest
import torch

from kq import _lib, ops, quantize as kqq

pytestmark = pytest.mark.gpu


def p(t):
    return ct.c_void_p(t.data_ptr())


def run_pair(dev, orc, lib, ty, R, C, M, seed):
    print("no-alloc gemm", ty, R, C, M, flush=True)
    W = torch.from_numpy(kqq.synthetic_matrix(R, C, ty, seed=seed)).to(dev)
    xq = torch.from_numpy(orc.quantize_q8k(kqq.synthetic_activations(M, C, seed=seed + 1))).to(dev)
    need = ops.gemm_workspace_bytes(R, C, M)
    assert need <= _lib.KQ_GEMM_STATIC_SCRATCH_BYTES
    ws = ops.gemm_workspace(R, C, M, dev)
    wsp, wsn = ops._aligned(ws, need)
    s = ct.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    y_ws = torch.full((M, R + 4), -1.0, device=dev)
    y_st = torch.full((M, R + 4), -2.0, device=dev)
    _lib.check(lib.kq_gemm_q8k_ws(p(W), R, C, ty, p(xq), M, p(y_ws), R + 4, wsp, wsn, s))
    _lib.check(lib.kq_gemm_q8k_static(p(W), R, C, ty, p(xq), M, p(y_st), R + 4, s))
    torch.cuda.synchronize()
    a, b = y_ws.cpu().numpy(), y_st.cpu().numpy()
    np.testing.assert_array_equal(b[:, :R], a[:, :R])
    assert np.all(b[:, R:] == -2.0)
    return need


def test_static_gemm_matches_workspace_form(dev, orc):
    lib = _lib.kq()
    # first call: a 256-token chunk of the Q6_K down projection (K split 4 ways: fragments and
    # partial sums fill 19 MB of the array); second: a smaller GEMM, also split
    n1 = run_pair(dev, orc, lib, 14, 4096, 12288, 256, 3)
    n2 = run_pair(dev, orc, lib, 12, 1024, 4096, 100, 4)
    assert n2 < n1
    # and an unsplit one after both
    run_pair(dev, orc, lib, 12, 520, 512, 37, 5)


def test_static_gemm_rejects_oversized(dev):
    lib = _lib.kq()
    R, C, M = 4096, 12288, 4096                  # needs 48 MB of fragments
    assert ops.gemm_workspace_bytes(R, C, M) > _lib.KQ_GEMM_STATIC_SCRATCH_BYTES
    w = torch.zeros(16, dtype=torch.uint8, device=dev)
    rc = lib.kq_gemm_q8k_static(p(w), R, C, 14, p(w), M, p(w), R, None)
    assert rc == _lib.KQ_ERR_ARG
    assert b"static scratch" in lib.kq_last_error()
