"""Parity of the fused producers (kq_rms_q8k, kq_swiglu_q8k) with the CPU oracle: h, the fp32
outputs and the Q8_K bytes bit-exact; the fused Q8_K bytes equal the stand-alone quantizer's on
the fp32 output."""
import numpy as np
import pytest
import torch

from kq import ops

pytestmark = pytest.mark.gpu
F32 = np.float32


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rms_inputs(N, D, seed):
    rng = np.random.default_rng(seed)
    h = (rng.standard_normal((N, D)) * rng.choice([1e-3, 1.0, 40.0], (N, 1))).astype(F32)
    r = rng.standard_normal((N, D)).astype(F32)
    w = (1 + 0.2 * rng.standard_normal(D)).astype(F32)
    if N > 1:
        h[1] = 0.0                                   # all-zero row: s = 1/sqrt(1e-6), xn = 0
        r[1] = 0.0
    return h, r, w


# D covers every row-length instantiation of the kernel: 768 (4 values per thread), 2560 (16), 4096
# (16), 8192 (32, the last with 16 waves), 12288 (48, 8 waves), 16384 (64, the largest D)
@pytest.mark.parametrize("N,D", [(1, 256), (1, 4096), (3, 4096), (2, 12288), (5, 768), (1, 2560), (2, 8192),
                                 (1, 16384)])
@pytest.mark.parametrize("add", [False, True])
def test_rms_q8k_bit_exact(dev, orc, N, D, add):
    h, r, w = rms_inputs(N, D, seed=D + N)
    hd, rd, wd = dev_t(h, dev), dev_t(r, dev), dev_t(w, dev)
    xn = torch.empty_like(hd)
    _, xq = ops.rms_q8k(hd, wd, residual=rd if add else None, xn=xn)
    h_want, xn_want = orc.rms_norm(h, w, r if add else None)
    np.testing.assert_array_equal(host(hd), h_want)
    np.testing.assert_array_equal(host(xn), xn_want)
    np.testing.assert_array_equal(host(xq), orc.quantize_q8k(xn_want))
    # the fused bytes are the stand-alone quantizer's bytes of the same values
    np.testing.assert_array_equal(host(xq), host(ops.q8k_quantize(xn)))


def test_rms_q8k_strided_in_place_and_without_xn(dev, orc):
    N, D, ld = 3, 1024, 1024 + 36
    h, r, w = rms_inputs(N, ld, seed=7)
    w = w[:D].copy()
    hd = dev_t(h, dev)[:, :D]
    rd = dev_t(r, dev)[:, :D]
    assert hd.stride(0) == ld
    h_want, xn_want = orc.rms_norm(h[:, :D], w, r[:, :D])
    _, xq = ops.rms_q8k(hd, dev_t(w, dev), residual=rd)                 # no fp32 output
    np.testing.assert_array_equal(host(hd), h_want)
    np.testing.assert_array_equal(host(xq), orc.quantize_q8k(xn_want))
    # in place: xn = h (second call without residual normalises the updated h)
    _, xn2 = orc.rms_norm(h_want, w)
    _, xq2 = ops.rms_q8k(hd, dev_t(w, dev), xn=hd)
    np.testing.assert_array_equal(host(hd), xn2)
    np.testing.assert_array_equal(host(xq2), orc.quantize_q8k(xn2))


def swiglu_inputs(N, n, seed):
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal((N, n)) * 3).astype(F32)
    u = rng.standard_normal((N, n)).astype(F32)
    g[0, :8] = [0.0, -0.0, 100.0, -100.0, 88.0, -88.0, 90.0, -104.0]
    if N > 1:
        u[1, 256:512] = 0.0                          # zero block: d = 0
    return g, u


@pytest.mark.parametrize("N,n", [(1, 256), (1, 12288), (4, 12288), (3, 1280)])
def test_swiglu_q8k_bit_exact(dev, orc, N, n):
    g, u = swiglu_inputs(N, n, seed=n + N)
    gd, ud = dev_t(g, dev), dev_t(u, dev)
    y = torch.empty_like(gd)
    _, xq = ops.swiglu_q8k(gd, ud, y=y)
    y_want = orc.swiglu(g, u)
    np.testing.assert_array_equal(host(y), y_want)
    np.testing.assert_array_equal(host(xq), orc.quantize_q8k(y_want))
    _, xq_only = ops.swiglu_q8k(gd, ud)                                  # no fp32 output
    np.testing.assert_array_equal(host(xq_only), host(xq))


def test_swiglu_q8k_strided(dev, orc):
    N, n, ld = 3, 512, 512 + 20
    g, u = swiglu_inputs(N, ld, seed=3)
    gd, ud = dev_t(g, dev)[:, :n], dev_t(u, dev)[:, :n]
    y = torch.zeros((N, ld), device=dev)[:, :n]
    _, xq = ops.swiglu_q8k(gd, ud, y=y)
    y_want = orc.swiglu(np.ascontiguousarray(g[:, :n]), np.ascontiguousarray(u[:, :n]))
    np.testing.assert_array_equal(host(y), y_want)
    np.testing.assert_array_equal(host(xq), orc.quantize_q8k(y_want))
