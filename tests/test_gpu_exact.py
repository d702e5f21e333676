"""Integer exactness of every product path, shown bit for bit.

The fp32 bar (1e-5 * max|y|) cannot see a one-unit error in an integer partial at K = 12288.  Here
the inputs make every result an exact integer that fp32 holds: weight blocks with d = dmin = 1
(fp16), activation blocks whose largest magnitude is a single -127 (so the Q8_K block has d = 1 and
q = x exactly) and small integer activations elsewhere.  Every weight is then an integer
(sc*q - m for Q4_K, sc*(q - 32) for Q6_K), every per-super-block value is exact, and as long as
sum_k |w_k| |x_k| < 2^24 for every output (asserted on the inputs) every fp32 step of every
kernel's epilogue and reduction is exact.  Each kernel's output must then equal the oracle's
(an exact integer evaluated in double) bit for bit: the two weight planes of the GEMM and of the
MFMA batch, its fp16 min term, the K split's partial sums, the v_dot4 GEMV and the fp32-activation
GEMV.
"""
import numpy as np
import pytest
import torch

from kq import ops, quantize as kqq

pytestmark = pytest.mark.gpu
ONE_F16 = np.array([1.0], np.float16).view(np.uint8)


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def exact_weights(R, C, ty, seed, q6_scale=20):
    """Random block bytes with every fp16 block scale 1.0 (Q6_K sub-block scales in
    [-q6_scale, q6_scale]), in the Kindi layout."""
    rng = np.random.default_rng(seed)
    G = C // 256
    if ty == 12:
        raw = rng.integers(0, 256, (R, G, 144), dtype=np.uint8)
        raw[:, :, 0:2] = ONE_F16
        raw[:, :, 2:4] = ONE_F16
    else:
        raw = rng.integers(0, 256, (R, G, 210), dtype=np.uint8)
        raw[:, :, 192:208] = rng.integers(-q6_scale, q6_scale + 1, (R, G, 16)).astype(np.int8).view(np.uint8)
        raw[:, :, 208:210] = ONE_F16
    return kqq.tile(raw.reshape(-1), R, C, ty)


def exact_activations(M, C, seed, amp):
    """Integers in [-amp, amp] with one -127 per 256-block (the block's first largest |x|)."""
    assert amp < 127
    rng = np.random.default_rng(seed)
    x = rng.integers(-amp, amp + 1, (M, C)).astype(np.float32)
    G = C // 256
    pos = rng.integers(0, 256, (M, G))
    x.reshape(M, G, 256)[np.arange(M)[:, None], np.arange(G)[None, :], pos] = -127.0
    return x


def prepare(orc, R, C, ty, M, seed, amp):
    W = exact_weights(R, C, ty, seed)
    X = exact_activations(M, C, seed + 1, amp)
    xq = orc.quantize_q8k(X)
    d, qs, _ = orc.q8k_fields(xq)
    assert np.all(d == 1.0) and np.array_equal(qs.reshape(M, C).astype(np.float32), X)
    # every partial sum of every kernel is bounded by sum_k |w_k||x_k|: keep it below 2^24
    dense = orc.dequant(W, R, C, ty).astype(np.float64)
    assert np.array_equal(dense, np.round(dense)), "weights must be integers"
    bound = np.abs(X).astype(np.float64) @ np.abs(dense).T
    assert bound.max() < 2 ** 24, bound.max()
    # with integer operands below 2^24 the double product is exact in any order, so the dense
    # product is the oracle's integer result; shown on a sample of tokens
    ref = X.astype(np.float64) @ dense.T
    toks = sorted({0, M // 2, M - 1})
    assert np.array_equal(orc.gemv_q8k(W, R, C, ty, xq[toks], len(toks)), ref[toks])
    return W, X, xq, ref


def assert_exact(got, ref, tag):
    bad = np.flatnonzero(got.astype(np.float64).reshape(-1) != ref.reshape(-1))
    assert bad.size == 0, "%s: %d outputs differ, first at %d: %r vs %r" % (
        tag, bad.size, bad[0], got.reshape(-1)[bad[0]], ref.reshape(-1)[bad[0]])


@pytest.mark.parametrize("ty,R,C,M,amp", [
    (12, 1024, 4096, 300, 3),      # K split 4 ways (48 tiles)
    (12, 12288, 4096, 512, 3),     # unsplit, the config-4 shape
    (12, 256, 12288, 130, 1),      # K = 12288, split
    (14, 4096, 12288, 512, 1),     # the config-4 shape: K split 2 ways
    (14, 512, 4096, 257, 3),       # split, three token tiles
    (14, 136, 256, 37, 3),         # R % 64 = 8, one super-block, ragged M
])
def test_gemm_exact(dev, orc, ty, R, C, M, amp):
    print("gemm exact", ty, R, C, M, flush=True)
    W, X, xq, ref = prepare(orc, R, C, ty, M, seed=R + C + M, amp=amp)
    wd, xqd = dev_t(W, dev), dev_t(xq, dev)
    y = torch.empty((M, R), device=dev)
    ops.gemm_q8k(wd, R, C, ty, xqd, M, y, ws=ops.gemm_workspace(R, C, M, dev))
    assert_exact(host(y), ref, "kq_gemm_q8k_ws")
    y2 = torch.empty((M, R), device=dev)
    ops.gemm_q8k(wd, R, C, ty, xqd, M, y2)
    assert_exact(host(y2), ref, "kq_gemm_q8k")


@pytest.mark.parametrize("ty,R,C,amp", [(12, 4096, 4096, 3), (14, 4096, 4096, 3), (12, 4096, 12288, 1),
                                        (12, 1024, 12288, 1), (14, 1024, 12288, 1), (12, 64, 16640, 1),
                                        (14, 40, 16640, 1)])
def test_gemv_batches_exact(dev, orc, ty, R, C, amp):
    """Every kernel choice of kq_gemv_q8k: the v_dot4 GEMVs (N = 1, 2 and few rows), the phase form
    of the MFMA kernel (Q4_K: N = 2..4, and N = 1 with 4096 < C <= 12288 and at least 4096 rows;
    Q6_K: N = 3..8 from 4096 rows), the plane form (N = 16; Q4_K N = 8) and, beyond 16384 columns,
    the v_dot4 kernel again: every row exact."""
    print("gemv exact", ty, R, C, flush=True)
    W, X, xq, ref = prepare(orc, R, C, ty, 16, seed=R + C + 7, amp=amp)
    wd, xqd = dev_t(W, dev), dev_t(xq, dev)
    for N in (1, 2, 3, 4, 8, 16):
        y = torch.empty((N, R), device=dev)
        ops.gemv_q8k(wd, R, C, ty, xqd, N, y)
        assert_exact(host(y), ref[:N], "gemv N=%d" % N)


@pytest.mark.parametrize("ty", [12, 14])
def test_gemv_f32_exact(dev, orc, ty):
    """The fp32-activation GEMV on integer weights and activations: exact as well."""
    R, C = 2048, 4096
    W, X, xq, ref = prepare(orc, R, C, ty, 2, seed=99 + ty, amp=3)
    wd = dev_t(W, dev)
    for n in range(2):
        y = torch.empty(R, device=dev)
        ops.gemv(wd, R, C, ty, dev_t(X[n], dev), y)
        assert_exact(host(y), ref[n], "f32 gemv")


@pytest.mark.parametrize("ty", [12, 14])
def test_small_batch_extreme_blocks(dev, orc, ty):
    """The integers at their largest: every code at its maximum (Q4_K 15, Q6_K 63) or minimum, scales and
    mins at their extremes (Q4_K 63, Q6_K -128 / 127), fp16 block scales 1, and activation blocks of
    +-127 (Q8_K d = 1): per-piece sums near 2^17, products with the scales near 2^24, super-block
    integers near 2^28.  Rows of every batch size through every kernel choice (v_dot4, the phase and the
    plane MFMA forms) must equal the one-token rows bit for bit, and the oracle within the bar."""
    R, C = 4096, 4096
    G = C // 256
    rng = np.random.default_rng(5 + ty)
    if ty == 12:
        raw = np.zeros((R, G, 144), np.uint8)
        raw[:, :, 0:2] = ONE_F16
        raw[:, :, 2:4] = ONE_F16
        raw[:, :, 4:16] = 0xFF                                      # every 6-bit scale and min 63
        raw[:, :, 16:] = np.where(rng.random((R, G, 128)) < 0.5, 0xFF, 0x00).astype(np.uint8)
    else:
        raw = np.zeros((R, G, 210), np.uint8)
        raw[:, :, 0:192] = np.where(rng.random((R, G, 192)) < 0.5, 0xFF, 0x00).astype(np.uint8)   # codes 63 or 0
        raw[:, :, 192:208] = np.where(rng.random((R, G, 16)) < 0.5, 0x80, 0x7F).astype(np.uint8)   # -128 / 127
        raw[:, :, 208:210] = ONE_F16
    W = kqq.tile(raw.reshape(-1), R, C, ty)
    X = np.where(rng.random((16, C)) < 0.5, 127.0, -127.0).astype(np.float32)
    xq = orc.quantize_q8k(X)
    wd, xqd = dev_t(W, dev), dev_t(xq, dev)
    single = torch.empty((16, R), device=dev)
    for n in range(16):
        ops.gemv_q8k(wd, R, C, ty, xqd[n:n + 1], 1, single[n])
    s = host(single)
    ref = orc.gemv_q8k(W, R, C, ty, xq, 16)
    err = np.abs(s.astype(np.float64) - ref).max()
    assert err <= 1e-5 * np.abs(ref).max(), err
    for N in (2, 3, 4, 5, 8, 16):
        y = torch.empty((N, R), device=dev)
        ops.gemv_q8k(wd, R, C, ty, xqd, N, y)
        np.testing.assert_array_equal(host(y), s[:N], err_msg="N=%d" % N)


@pytest.mark.parametrize("ty,C", [(12, 4096), (14, 12288)])
def test_gemm_extreme_blocks(dev, orc, ty, C):
    """The prefill GEMM (both entry points, K split or not) on the same extreme blocks: codes, scales and
    mins at their extremes, activations +-127, so every plane and the shifted sweep sums reach their
    largest magnitudes (Q6_K: 256 * (x.H) near 2^27); within the bar of the oracle."""
    R, M = 512, 300
    G = C // 256
    rng = np.random.default_rng(50 + ty)
    if ty == 12:
        raw = np.zeros((R, G, 144), np.uint8)
        raw[:, :, 0:2] = ONE_F16
        raw[:, :, 2:4] = ONE_F16
        raw[:, :, 4:16] = 0xFF
        raw[:, :, 16:] = np.where(rng.random((R, G, 128)) < 0.5, 0xFF, 0x00).astype(np.uint8)
    else:
        raw = np.zeros((R, G, 210), np.uint8)
        raw[:, :, 0:192] = np.where(rng.random((R, G, 192)) < 0.5, 0xFF, 0x00).astype(np.uint8)
        raw[:, :, 192:208] = np.where(rng.random((R, G, 16)) < 0.5, 0x80, 0x7F).astype(np.uint8)
        raw[:, :, 208:210] = ONE_F16
    W = kqq.tile(raw.reshape(-1), R, C, ty)
    X = np.where(rng.random((M, C)) < 0.5, 127.0, -127.0).astype(np.float32)
    xq = orc.quantize_q8k(X)
    ref = orc.gemv_q8k(W, R, C, ty, xq, M)
    wd, xqd = dev_t(W, dev), dev_t(xq, dev)
    for ws in (None, ops.gemm_workspace(R, C, M, dev)):
        y = torch.empty((M, R), device=dev)
        ops.gemm_q8k(wd, R, C, ty, xqd, M, y, ws=ws)
        got = host(y).astype(np.float64)
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
