"""Parity of the HIP kernels (through libkq's C ABI) with the CPU oracle.

Bars: decode, Q8_K bytes and integer sub-block sums bit-exact; fp32 outputs within
1e-5 * max|y_ref| (y_ref = oracle evaluated in double from the exact integer sums); batched rows
bit-identical to the single-token result.
"""
import ctypes as ct

import numpy as np
import pytest
import torch

from helpers import reference_unit_inputs
from kq import _lib, ops, quantize as kqq
from kq.formats import Q4_K, Q6_K

pytestmark = pytest.mark.gpu
TOL = 1e-5


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def assert_close_inf(got, want, tol=TOL):
    scale = np.abs(want).max()
    err = np.abs(got.astype(np.float64) - want).max()
    assert err <= tol * scale, "max err %.3g vs %.3g * %.3g" % (err, tol, scale)


def synth(R, C, ty, seed):
    return kqq.synthetic_matrix(R, C, ty, seed)


# --------------------------------------------------------------------------------------- decode
@pytest.mark.parametrize("tag,ty", [("tq", 12), ("tq", 14), ("syn", 12), ("syn", 14)])
def test_dequant_golden_bit_exact(dev, golden, orc, tag, ty):
    k = "%s_%d_" % (tag, ty)
    R, C, _ = (int(v) for v in golden[k + "shape"])
    W = golden[k + "w"]
    y = host(ops.dequant_rows(dev_t(W, dev), R, C, ty, 0, R))
    for i, r in enumerate(golden[k + "rows"]):
        np.testing.assert_array_equal(y[r], golden[k + "deq"][i])
    np.testing.assert_array_equal(y, orc.dequant(W, R, C, ty))


def test_dequant_single_row_offset(dev, orc):
    R, C = 64, 2048
    W = synth(R, C, Q6_K, 9)
    out = torch.full((3, C + 16), -1.0, device=dev)
    ops.dequant_rows(dev_t(W, dev), R, C, Q6_K, 37, 3, out)
    y = host(out)
    for i in range(3):
        np.testing.assert_array_equal(y[i, :C], orc.dequant_row(W, R, C, Q6_K, 37 + i))
    assert np.all(y[:, C:] == -1.0)


# ----------------------------------------------------------------------------------------- Q8_K
def q8k_cases():
    rng = np.random.default_rng(21)
    x = rng.standard_normal((6, 4096)).astype(np.float32)
    x[1] *= 1e-3
    x[2] *= 250.0
    x[3, 512:768] = 0.0                               # zero block
    x[4, :256] = 0.0
    x[4, 0] = -127.0                                  # iscale = 1: round-half-even cases
    x[4, 1:9] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.4999999, 126.5]
    x[5, 256:512] = 0.0
    x[5, 256 + 3], x[5, 256 + 10] = -5.0, 5.0         # |x| tie: first wins
    x[5, 1024:1280] = 7.0                             # constant block
    return x


def test_q8k_quantize_bit_exact(dev, orc):
    x = q8k_cases()
    got = host(ops.q8k_quantize(dev_t(x, dev)))
    np.testing.assert_array_equal(got, orc.quantize_q8k(x))


def test_q8k_quantize_strided_rows(dev, orc):
    rng = np.random.default_rng(4)
    big = rng.standard_normal((5, 1536 + 40)).astype(np.float32)
    xd = dev_t(big, dev)[:, :1536]
    assert xd.stride(0) == 1576
    got = host(ops.q8k_quantize(xd))
    np.testing.assert_array_equal(got, orc.quantize_q8k(big[:, :1536]))


def test_q8k_quantize_large(dev, orc):
    """Full prefill activation size (M = 2048, K = 12288)."""
    x = kqq.synthetic_activations(2048, 12288, seed=3)
    got = host(ops.q8k_quantize(dev_t(x, dev)))
    np.testing.assert_array_equal(got, orc.quantize_q8k(x))


# --------------------------------------------------------------------------- integer sub-blocks
@pytest.mark.parametrize("ty", [12, 14])
def test_subblock_sums_reference_inputs(dev, orc, ty):
    W, x, R, C = reference_unit_inputs()[ty]
    xs = np.stack([x, -x, 3 * x]).astype(np.float32)
    xq = orc.quantize_q8k(xs)
    got = host(ops.subblock_sums(dev_t(W, dev), R, C, ty, dev_t(xq, dev), 3))
    np.testing.assert_array_equal(got, orc.subblock_sums(W, R, C, ty, xq, 3))


@pytest.mark.parametrize("ty,R,C", [(12, 64, 4096), (14, 64, 4096), (12, 16, 4352), (14, 24, 12288),
                                    (12, 16, 61440)])
def test_subblock_sums_synthetic(dev, orc, ty, R, C):
    W = synth(R, C, ty, 5)
    xq = orc.quantize_q8k(kqq.synthetic_activations(2, C, seed=5))
    got = host(ops.subblock_sums(dev_t(W, dev), R, C, ty, dev_t(xq, dev), 2))
    np.testing.assert_array_equal(got, orc.subblock_sums(W, R, C, ty, xq, 2))


def test_subblock_sums_random_bytes_extremes(dev, orc):
    """All-0xFF and random bytes: the largest integer magnitudes a block can produce."""
    rng = np.random.default_rng(8)
    for ty, bs in ((12, 144), (14, 210)):
        R, C = 16, 1024
        W = rng.integers(0, 256, R * 4 * bs, dtype=np.uint8)
        W[: 8 * bs] = 0xFF
        x = np.full((1, C), -1.0, np.float32)   # every q8 = +127 after the sign convention
        xq = orc.quantize_q8k(x)
        got = host(ops.subblock_sums(dev_t(W, dev), R, C, ty, dev_t(xq, dev), 1))
        np.testing.assert_array_equal(got, orc.subblock_sums(W, R, C, ty, xq, 1))


# ------------------------------------------------------------------------------------ Q8_K GEMV
GEMV_SHAPES = [
    (12, 8, 256), (14, 8, 256),            # one super-block column
    (12, 40, 4352), (14, 40, 4352),        # G = 17: two column passes, ragged
    (12, 4096, 4096),                      # single Q4_K GEMV, W 4096 x 4096
    (12, 1024, 4096), (12, 12288, 4096),   # k/v and gate/up shapes
    (14, 4096, 12288),                     # Q6_K down
    (14, 1024, 4096),                      # Q6_K attn_v
    (12, 64, 12288),                       # Q4_K, three passes on the pass-split kernel
    (14, 48, 8192), (14, 16, 8448),        # Q6_K: two passes (split kernel); three, the last one column
    (12, 16, 61440), (14, 8, 61440),       # the largest C: 15 passes, sequential kernel, full pass tree
]


@pytest.mark.parametrize("ty,R,C", GEMV_SHAPES)
def test_gemv_q8k_vs_oracle(dev, orc, ty, R, C):
    W = synth(R, C, ty, R + C + ty)
    x = kqq.synthetic_activations(1, C, seed=R)
    xq = orc.quantize_q8k(x)
    y = torch.empty(R, device=dev)
    ops.gemv_q8k(dev_t(W, dev), R, C, ty, dev_t(xq, dev), 1, y)
    assert_close_inf(host(y), orc.gemv_q8k(W, R, C, ty, xq, 1)[0])


@pytest.mark.parametrize("ty", [12, 14])
def test_gemv_q8k_reference_inputs(dev, orc, ty):
    W, x, R, C = reference_unit_inputs()[ty]
    xq = orc.quantize_q8k(x[None])
    y = torch.empty(R, device=dev)
    ops.gemv_q8k(dev_t(W, dev), R, C, ty, dev_t(xq, dev), 1, y)
    assert_close_inf(host(y), orc.gemv_q8k(W, R, C, ty, xq, 1)[0])


@pytest.mark.parametrize("ty,R,C", [
    (12, 12288, 4096), (14, 4096, 12288), (12, 64, 4352),   # decode shapes; G = 17 (a padded pass)
    (14, 8, 256), (12, 24, 16384), (14, 40, 16640),         # half row tile, one column; G = 64; G = 65
    (14, 4088, 4096), (12, 4096, 12288),                    # either side of the 4096-row MFMA threshold
    (12, 1000, 4096),                                       # Q4_K below it: v_dot4 to 3 tokens, then MFMA
    (12, 4096, 8448), (14, 4096, 12032),                    # G = 33 / 47: a last chunk of 1 / 3 super-blocks
    (14, 4096, 16384), (12, 4104, 14336),                   # G = 64 / 56 on many rows: the plane form's 16 / 14 waves
    (12, 136, 7936), (14, 4104, 3840),                      # two-group plane form: G = 31 / 15 (a half-empty last piece)
])
def test_batched_rows_bit_identical_to_single(dev, orc, ty, R, C):
    """Speculative-verify invariant: every row of a batch equals its N = 1 result bit for bit."""
    W = dev_t(synth(R, C, ty, 77), dev)
    X = kqq.synthetic_activations(16, C, seed=C)
    xq = orc.quantize_q8k(X)
    xqd = dev_t(xq, dev)
    single = torch.empty((16, R), device=dev)
    for n in range(16):
        ops.gemv_q8k(W, R, C, ty, xqd[n:n + 1], 1, single[n])
    s = host(single)
    for N in (2, 3, 4, 5, 7, 8, 9, 13, 16):
        yb = torch.empty((N, R + 8), device=dev)
        ops.gemv_q8k(W, R, C, ty, xqd[:N], N, yb, R + 8)
        np.testing.assert_array_equal(host(yb)[:, :R], s[:N])
    assert_close_inf(s, orc.gemv_q8k(host(W), R, C, ty, xq, 16))


def test_small_batch_forms_sweep(dev, orc):
    """Every small-batch kernel choice over seeded shapes: super-blocks per row G = 1, 2, 3, 5, 16, 17,
    33, 47, 48 (whole and partial chunks of 4), rows below, at and above 4096 and not a multiple of 16,
    N = 2..8 (the phase form of the MFMA kernel, the v_dot4 kernels for few rows, the plane form
    beyond): each row bit-identical to its one-token result and the batch within the bar of the
    oracle.  The oracle runs on every fourth case (it is the slow part)."""
    cases = [(12, 4104, 256), (14, 4104, 256), (12, 4096, 512), (14, 4112, 768), (12, 4088, 1280),
             (14, 4096, 1280), (12, 4096, 4352), (14, 4096, 4352), (12, 4104, 8448), (14, 4096, 8448),
             (12, 4096, 12032), (14, 4104, 12032), (12, 24, 12288), (14, 40, 4096), (12, 8200, 4096),
             (14, 8200, 4352)]
    for i, (ty, R, C) in enumerate(cases):
        print("forms sweep", ty, R, C, flush=True)
        W = synth(R, C, ty, 500 + i)
        Wd = dev_t(W, dev)
        X = kqq.synthetic_activations(8, C, seed=600 + i)
        xq = orc.quantize_q8k(X)
        xqd = dev_t(xq, dev)
        single = torch.empty((8, R), device=dev)
        for n in range(8):
            ops.gemv_q8k(Wd, R, C, ty, xqd[n:n + 1], 1, single[n])
        s = host(single)
        for N in (2, 3, 4, 5, 6, 7, 8):
            yb = torch.empty((N, R), device=dev)
            ops.gemv_q8k(Wd, R, C, ty, xqd, N, yb)
            np.testing.assert_array_equal(host(yb), s[:N], err_msg="%d %d %d N=%d" % (ty, R, C, N))
        if i % 4 == 0:
            assert_close_inf(s, orc.gemv_q8k(W, R, C, ty, xq, 8))


@pytest.mark.parametrize("ty", [12, 14])
def test_batched_reference_inputs_bit_identical(dev, orc, ty):
    """The reference unit test's random block bytes (any scale/min bit pattern) through the
    batched path: rows equal the N = 1 results bit for bit and the oracle within the bar."""
    W, x, R, C = reference_unit_inputs()[ty]
    X = np.stack([x * (i + 1) * (-1) ** i for i in range(7)]).astype(np.float32)
    xq = orc.quantize_q8k(X)
    Wd, xqd = dev_t(W, dev), dev_t(xq, dev)
    yb = torch.empty((7, R), device=dev)
    ops.gemv_q8k(Wd, R, C, ty, xqd, 7, yb)
    for n in range(7):
        y1 = torch.empty(R, device=dev)
        ops.gemv_q8k(Wd, R, C, ty, xqd[n:n + 1], 1, y1)
        np.testing.assert_array_equal(host(yb)[n], host(y1))
    assert_close_inf(host(yb), orc.gemv_q8k(W, R, C, ty, xq, 7))


@pytest.mark.parametrize("C,N", [(4096, 1), (4096, 3), (4096, 6), (4096, 16), (12288, 2), (12288, 4)])
def test_gemv_q8k_multi_matches_single(dev, orc, C, N):
    """q/k/v-style group (two Q4_K, one Q6_K) in one call equals three single calls bit for bit; at
    C = 12288 and two tokens the Q4_K matrices take the MFMA kernel and the Q6_K one the v_dot4 GEMV
    within the same call."""
    print("multi", C, N, flush=True)
    mats_h = [(synth(R, C, ty, 50 + i), R, C, ty) for i, (R, ty) in enumerate([(4096, 12), (1024, 12), (1024, 14)])]
    mats = [(dev_t(W, dev), R, C_, ty) for (W, R, C_, ty) in mats_h]
    xq = orc.quantize_q8k(kqq.synthetic_activations(N, C, seed=N))
    xqd = dev_t(xq, dev)
    ys = [torch.full((N, R + 4), -7.0, device=dev) for (_, R, _, _) in mats]
    ops.gemv_q8k_multi(mats, xqd, N, ys)
    for (w, R, C_, ty), y, (W, _, _, _) in zip(mats, ys, mats_h):
        ref = torch.empty((N, R), device=dev)
        ops.gemv_q8k(w, R, C_, ty, xqd, N, ref)
        got = host(y)
        np.testing.assert_array_equal(got[:, :R], host(ref))
        assert np.all(got[:, R:] == -7.0)
        assert_close_inf(got[:, :R], orc.gemv_q8k(W, R, C_, ty, xq, N))


@pytest.mark.parametrize("shapes,C", [
    (((4096, 12), (1024, 12), (1024, 14)), 4096),    # a Q4_K_M layer's q, k and Q6_K v
    (((4096, 12), (1024, 14)), 4096),                # one of each
    (((1024, 14), (2048, 14), (4096, 12)), 4096),    # two Q6_K and one Q4_K
    (((40, 12), (8, 14), (96, 12)), 256),            # a few tiles, one super-block
    (((16, 14), (4104, 12)), 2048),                  # G = 8, R % 16 = 8
    (((12288, 12), (8, 14)), 3840),                  # G = 15, a one-tile second type
])
def test_gemv_q8k_multi_mixed_types_one_token(dev, orc, shapes, C):
    """One token over matrices of both types sharing an input (C <= 4096): one launch holds both
    types' waves, and every output equals the one-matrix call bit for bit, columns past R untouched."""
    print("multi mixed", shapes, C, flush=True)
    mats_h = [(synth(R, C, ty, 70 + i), R, C, ty) for i, (R, ty) in enumerate(shapes)]
    mats = [(dev_t(W, dev), R, C_, ty) for (W, R, C_, ty) in mats_h]
    xq = orc.quantize_q8k(kqq.synthetic_activations(1, C, seed=C + 3))
    xqd = dev_t(xq, dev)
    ys = [torch.full((R + 4,), -7.0, device=dev) for (_, R, _, _) in mats]
    ops.gemv_q8k_multi(mats, xqd, 1, ys)
    for (w, R, C_, ty), y, (W, _, _, _) in zip(mats, ys, mats_h):
        ref = torch.empty(R, device=dev)
        ops.gemv_q8k(w, R, C_, ty, xqd, 1, ref)
        got = host(y)
        np.testing.assert_array_equal(got[:R], host(ref))
        assert np.all(got[R:] == -7.0)
        if R <= 4104:
            assert_close_inf(got[:R], orc.gemv_q8k(W, R, C_, ty, xq, 1)[0])


@pytest.mark.parametrize("shapes,C", [
    (((4096, 12), (1024, 12), (1024, 12)), 4096),    # q, k, v
    (((12288, 12), (12288, 12)), 4096),              # gate, up
    (((4096, 12), (1024, 12), (1024, 14)), 4096),    # both types in one launch
    (((40, 14), (8, 14)), 256),                      # one super-block
    (((136, 12),), 3840),                            # G = 15
    (((4096, 14),), 1024),
    (((4096, 12), (4096, 14)), 12288),               # C > 4096: quantizer launch, then the GEMV
    (((1024, 14), (2048, 14)), 8448),                # G = 33
])
def test_gemv_q8k_x_matches_quantize_then_gemv(dev, orc, shapes, C):
    """kq_gemv_q8k_x (fp32 x quantized to Q8_K inside the GEMV launch, every workgroup into its LDS)
    equals kq_q8k_quantize followed by kq_gemv_q8k_multi bit for bit, the optional xq output equals
    the quantizer's bytes, and nothing is written past R; with a zero block, a tied maximum and a
    block of one repeated value in x."""
    print("gemv_q8k_x", shapes, C, flush=True)
    mats_h = [(synth(R, C, ty, 60 + i), R, C, ty) for i, (R, ty) in enumerate(shapes)]
    mats = [(dev_t(W, dev), R, C_, ty) for (W, R, C_, ty) in mats_h]
    x = kqq.synthetic_activations(1, C, seed=C + 5)[0].copy()
    x[:256] = 0.0
    if C >= 768:
        x[256 + 5], x[256 + 9] = -7.0, 7.0
        x[512:768] = 0.3
    xd = dev_t(x, dev)
    xq_ref = ops.q8k_quantize(xd)
    ys = [torch.full((R + 4,), -7.0, device=dev) for (_, R, _, _) in mats]
    xq_out = torch.full(((C // 256) * 292,), 0x55, dtype=torch.uint8, device=dev)
    ops.gemv_q8k_x(mats, xd, ys, xq_out)
    np.testing.assert_array_equal(host(xq_out), host(xq_ref).reshape(-1))
    refs = [torch.empty(R, device=dev) for (_, R, _, _) in mats]
    ops.gemv_q8k_multi(mats, xq_ref, 1, refs)
    for (w, R, C_, ty), y, ref in zip(mats, ys, refs):
        got = host(y)
        np.testing.assert_array_equal(got[:R], host(ref))
        assert np.all(got[R:] == -7.0)
    if C <= 4096:   # without the xq output too
        ys2 = [torch.empty(R, device=dev) for (_, R, _, _) in mats]
        ops.gemv_q8k_x(mats, xd, ys2)
        for y2, ref in zip(ys2, refs):
            np.testing.assert_array_equal(host(y2), host(ref))
    W, R, C_, ty = mats_h[0]
    assert_close_inf(host(ys[0])[:R], orc.gemv_q8k(W, R, C_, ty, orc.quantize_q8k(x[None]), 1)[0])


def test_gemv_q8k_x_special_values_bytes(dev):
    """The in-launch quantization (four blocks per wave side by side, a zero block by a select) writes
    the stand-alone quantizer's bytes for blocks holding NaN, +-inf, subnormals, signed zeros, a
    NaN among zeros and values at the rounding edges."""
    C = 4096
    x = kqq.synthetic_activations(1, C, seed=17)[0].copy()
    x[0:256] = 0.0
    x[3] = np.nan                                     # a NaN among zeros
    x[256:512] = np.float32(1e-40) * np.arange(256)   # subnormals
    x[512 + 7] = np.inf
    x[768 + 1] = -np.inf
    x[1024:1280] = -0.0
    x[1280 + 9] = np.nan
    x[1536:1792] = (np.arange(256) - 128) * np.float32(0.5)  # exact halves: round-half-even after scaling
    x[1792:2048] = 127.0 * np.sign(np.arange(256) - 100.5).astype(np.float32)
    xd = dev_t(x, dev)
    ref = host(ops.q8k_quantize(xd)).reshape(-1)
    W = dev_t(synth(1024, C, 12, 3), dev)
    out = torch.full(((C // 256) * 292,), 0x55, dtype=torch.uint8, device=dev)
    ops.gemv_q8k_x([(W, 1024, C, 12)], xd, [torch.empty(1024, device=dev)], out)
    np.testing.assert_array_equal(host(out), ref)


@pytest.mark.parametrize("ty,R,C,M", [
    (12, 512, 4096, 64), (14, 256, 12288, 40),       # one M tile, partial
    (12, 136, 256, 300), (14, 136, 256, 300),        # R % 128 = 8, one super-block, ragged M
    (12, 1024, 4096, 512), (14, 512, 4352, 257),     # several tiles both ways; G = 17
])
def test_gemm_q8k_vs_oracle(dev, orc, ty, R, C, M):
    W = synth(R, C, ty, 31)
    X = kqq.synthetic_activations(M, C, seed=M)
    xq = orc.quantize_q8k(X)
    y = torch.full((M, R + 8), -3.0, device=dev)
    ops.gemm_q8k(dev_t(W, dev), R, C, ty, dev_t(xq, dev), M, y, R + 8)
    got = host(y)
    assert np.all(got[:, R:] == -3.0)
    assert_close_inf(got[:, :R], orc.gemv_q8k(W, R, C, ty, xq, M))
    # the fragment-order path (caller workspace) gives the same bits unless it splits K
    y2 = torch.full((M, R + 8), -4.0, device=dev)
    ops.gemm_q8k(dev_t(W, dev), R, C, ty, dev_t(xq, dev), M, y2, R + 8, ws=ops.gemm_workspace(R, C, M, dev))
    got2 = host(y2)
    if gemm_splits_k(R, C, M):
        assert_close_inf(got2[:, :R], orc.gemv_q8k(W, R, C, ty, xq, M))
    else:
        np.testing.assert_array_equal(got2[:, :R], got[:, :R])
    assert np.all(got2[:, R:] == -4.0)


def gemm_splits_k(R, C, M):
    """Whether kq_gemm_q8k_ws splits K for this shape: its workspace then holds partial sums beyond
    the activation fragments (M rounded up to 256 rows of C bytes)."""
    return ops.gemm_workspace_bytes(R, C, M) > -(-M // 256) * 256 * C


@pytest.mark.parametrize("ty,R,C,M,S", [
    (14, 1024, 12288, 64, 8),     # 16 tiles: 8 splits of 6 super-blocks
    (12, 1024, 4096, 100, 4),     # 4 splits of 4
    (12, 2048, 4352, 130, 4),     # G = 17: splits of 5, 5, 5, 2
    (14, 512, 2048, 257, 2),      # G = 8: 2 splits of 4, three token tiles
    (14, 64, 61440, 40, 8),       # the largest C: 8 splits of 30 super-blocks
])
def test_gemm_q8k_split_k(dev, orc, ty, R, C, M, S):
    """Grids too small to fill the GPU split K over S workgroups per tile and add the partial sums
    in a fixed order: within the bar of the oracle, the same bits call after call, columns past R
    untouched."""
    need = ops.gemm_workspace_bytes(R, C, M)
    frag = -(-M // 256) * 256 * C
    assert need == -(-frag // 256) * 256 + S * M * R * 4
    W = synth(R, C, ty, 77)
    xq = orc.quantize_q8k(kqq.synthetic_activations(M, C, seed=M + 5))
    wd, xqd = dev_t(W, dev), dev_t(xq, dev)
    ws = ops.gemm_workspace(R, C, M, dev)
    y = torch.full((M, R + 16), -5.0, device=dev)
    ops.gemm_q8k(wd, R, C, ty, xqd, M, y, R + 16, ws=ws)
    got = host(y)
    assert np.all(got[:, R:] == -5.0)
    assert_close_inf(got[:, :R], orc.gemv_q8k(W, R, C, ty, xq, M))
    ws.fill_(0x7f)                                  # stale partials from elsewhere must not matter
    y2 = torch.full((M, R + 16), -6.0, device=dev)
    ops.gemm_q8k(wd, R, C, ty, xqd, M, y2, R + 16, ws=ws)
    np.testing.assert_array_equal(host(y2)[:, :R], got[:, :R])


@pytest.mark.parametrize("C,M", [(4096, 256), (4096, 300), (12288, 130), (2048, 2048), (16640, 64)])
def test_gemm_q8k_multi_matches_single(dev, orc, C, M):
    """A q/k/v-style group (two Q4_K matrices, one Q6_K) in one kq_gemm_q8k_multi_ws call: one
    fragment copy, one launch per type, each matrix keeping the K split of its own call, so every
    output equals kq_gemm_q8k_ws on that matrix alone bit for bit (splitting and unsplit shapes
    alike), columns past R untouched; the small matrices also against the oracle."""
    print("gemm multi", C, M, flush=True)
    shapes = [(4096, 12), (1024, 12), (1024, 14)]
    mats_h = [(synth(R, C, ty, 90 + i), R, C, ty) for i, (R, ty) in enumerate(shapes)]
    mats = [(dev_t(W, dev), R, C_, ty) for (W, R, C_, ty) in mats_h]
    xq = orc.quantize_q8k(kqq.synthetic_activations(M, C, seed=M + 11))
    xqd = dev_t(xq, dev)
    need = ops.gemm_multi_workspace_bytes([R for R, _ in shapes], C, M)
    frag = -(-M // 256) * 256 * C                   # fragment copy (a multiple of 256 bytes)
    assert need == frag + sum(ops.gemm_workspace_bytes(R, C, M) - frag for R, _ in shapes)
    ws = torch.full((need + 256,), 0x55, dtype=torch.uint8, device=dev)
    ys = [torch.full((M, R + 4), -7.0, device=dev) for (_, R, _, _) in mats]
    ops.gemm_q8k_multi(mats, xqd, M, ys, ws)
    for (w, R, C_, ty), y, (W, _, _, _) in zip(mats, ys, mats_h):
        ref = torch.empty((M, R), device=dev)
        ops.gemm_q8k(w, R, C_, ty, xqd, M, ref, ws=ops.gemm_workspace(R, C_, M, dev))
        got = host(y)
        np.testing.assert_array_equal(got[:, :R], host(ref))
        assert np.all(got[:, R:] == -7.0)
        if R <= 1024:
            assert_close_inf(got[:, :R], orc.gemv_q8k(W, R, C_, ty, xq, M))


@pytest.mark.parametrize("C,M,ldx", [(4096, 256, 4096), (4096, 300, 4352), (12288, 130, 12288), (2048, 257, 2048),
                                    (16640, 40, 16640), (256, 1, 256)])
def test_gemm_f32_multi_matches_quantize_then_gemm(dev, orc, C, M, ldx):
    """kq_gemm_f32_multi (one launch quantizing the fp32 rows into the workspace and writing the GEMM's
    fragment copy, then the grouped GEMM) equals kq_q8k_quantize followed by kq_gemm_q8k_ws on each
    matrix bit for bit, with strided input rows and a ragged last token tile (its pad rows zero)."""
    print("gemm f32 multi", C, M, ldx, flush=True)
    shapes = [(4096, 12), (1024, 14), (1024, 12)]
    mats_h = [(synth(R, C, ty, 70 + i), R, C, ty) for i, (R, ty) in enumerate(shapes)]
    mats = [(dev_t(W, dev), R, C_, ty) for (W, R, C_, ty) in mats_h]
    Xw = np.zeros((M, ldx), np.float32)
    Xw[:, :C] = kqq.synthetic_activations(M, C, seed=M + 23)
    X = dev_t(Xw, dev)[:, :C]
    need = ops.gemm_f32_multi_workspace_bytes([R for R, _ in shapes], C, M)
    ws = torch.full((need + 256,), 0x33, dtype=torch.uint8, device=dev)
    ys = [torch.full((M, R + 4), -7.0, device=dev) for (_, R, _, _) in mats]
    ops.gemm_f32_multi(mats, X, ys, ws)
    # the workspace: the Q8_K rows (256-byte aligned), then the fragment copy of M rounded up to 256 rows
    G = C // 256
    want = orc.quantize_q8k(Xw[:, :C]).reshape(M, G, 292)
    wsh = host(ws)[(-ws.data_ptr()) % 256:]
    nq = -(-M * G * 292 // 256) * 256
    np.testing.assert_array_equal(wsh[:M * G * 292].reshape(M, G, 292), want)
    Mp = -(-M // 256) * 256
    qs = np.zeros((Mp, G, 256), np.uint8)
    qs[:M] = want[:, :, 4:260]
    # frag[m/32][g][ks][lane][16] = qs[32 (m/32) + lane % 32][g][32 ks + 16 (lane / 32) .. +16]
    frag = qs.reshape(Mp // 32, 32, G, 8, 2, 16).transpose(0, 2, 3, 4, 1, 5).reshape(-1)
    np.testing.assert_array_equal(wsh[nq:nq + Mp * C], frag)
    xq = ops.q8k_quantize(X)
    for (w, R, C_, ty), y in zip(mats, ys):
        ref = torch.empty((M, R), device=dev)
        ops.gemm_q8k(w, R, C_, ty, xq, M, ref, ws=ops.gemm_workspace(R, C_, M, dev))
        got = host(y)
        np.testing.assert_array_equal(got[:, :R], host(ref))
        assert np.all(got[:, R:] == -7.0)


def test_gemm_q8k_multi_one_type_and_single(dev, orc):
    """Grouped calls of one matrix, and of three Q6_K matrices (one launch), equal single calls."""
    C, M = 4352, 200
    xq = orc.quantize_q8k(kqq.synthetic_activations(M, C, seed=5))
    xqd = dev_t(xq, dev)
    for shapes in ([(1024, 12)], [(512, 14), (136, 14), (2048, 14)]):
        mats = [(dev_t(synth(R, C, ty, 30 + i), dev), R, C, ty) for i, (R, ty) in enumerate(shapes)]
        ws = torch.empty(ops.gemm_multi_workspace_bytes([R for R, _ in shapes], C, M) + 256, dtype=torch.uint8,
                         device=dev)
        ys = [torch.empty((M, R), device=dev) for R, _ in shapes]
        ops.gemm_q8k_multi(mats, xqd, M, ys, ws)
        for (w, R, C_, ty), y in zip(mats, ys):
            ref = torch.empty((M, R), device=dev)
            ops.gemm_q8k(w, R, C_, ty, xqd, M, ref, ws=ops.gemm_workspace(R, C_, M, dev))
            np.testing.assert_array_equal(host(y), host(ref))


@pytest.mark.parametrize("ty", [12, 14])
def test_gemm_q8k_reference_inputs(dev, orc, ty):
    """The reference unit test's random block bytes (any scale/min bit pattern) through the GEMM."""
    W, x, R, C = reference_unit_inputs()[ty]
    X = np.stack([x * (i + 1) * (-1) ** i for i in range(37)]).astype(np.float32)
    xq = orc.quantize_q8k(X)
    y = torch.empty((37, R), device=dev)
    ops.gemm_q8k(dev_t(W, dev), R, C, ty, dev_t(xq, dev), 37, y)
    assert_close_inf(host(y), orc.gemv_q8k(W, R, C, ty, xq, 37))


@pytest.mark.parametrize("ty", [12, 14])
def test_gemm_q8k_ws_matches_direct(dev, orc, ty):
    """kq_gemm_q8k_ws (caller workspace, shared by two calls of different M) equals kq_gemm_q8k
    (operands straight from the Q8_K rows) bit for bit, and both equal the oracle within the bar."""
    R, C = 264, 1024
    W = synth(R, C, ty, 41)
    wd = dev_t(W, dev)
    ws = ops.gemm_workspace(R, C, 300, dev)
    assert not gemm_splits_k(R, C, 300) and not gemm_splits_k(R, C, 77)
    for M in (300, 77):
        xq = orc.quantize_q8k(kqq.synthetic_activations(M, C, seed=900 + M))
        xqd = dev_t(xq, dev)
        y_ws = torch.full((M, R), -1.0, device=dev)
        y_lib = torch.full((M, R), -2.0, device=dev)
        ops.gemm_q8k(wd, R, C, ty, xqd, M, y_ws, ws=ws)
        ops.gemm_q8k(wd, R, C, ty, xqd, M, y_lib)
        np.testing.assert_array_equal(host(y_ws), host(y_lib))
        assert_close_inf(host(y_ws), orc.gemv_q8k(W, R, C, ty, xq, M))


def test_gemm_q8k_ws_rejects_small_or_misaligned_workspace(dev):
    R, C, M = 64, 512, 130
    w = dev_t(synth(R, C, 12, 5), dev)
    xq = torch.zeros(M * (C // 256) * 292, dtype=torch.uint8, device=dev)
    y = torch.empty((M, R), device=dev)
    need = ops.gemm_workspace_bytes(R, C, M)
    assert need == 256 * C          # M rounded up to 128 rows, one byte per quant
    small = torch.empty(need, dtype=torch.uint8, device=dev)
    lib = _lib.kq()
    args = lambda ws, n: (ct.c_void_p(w.data_ptr()), R, C, 12, ct.c_void_p(xq.data_ptr()), M,
                          ct.c_void_p(y.data_ptr()), R, ws, n, None)
    base = small.data_ptr() + (-small.data_ptr()) % 256
    assert lib.kq_gemm_q8k_ws(*args(ct.c_void_p(base), need - 256)) == -1
    assert b"workspace" in lib.kq_last_error()
    assert lib.kq_gemm_q8k_ws(*args(ct.c_void_p(base + 16), need)) == -1
    assert b"aligned" in lib.kq_last_error()


# ------------------------------------------------------------------------------- fp32-x GEMV
@pytest.mark.parametrize("ty", [12, 14])
def test_gemv_f32_reference_unit_test(dev, orc, ty):
    """The reference unit test (test_quant.py:30-32) on the GPU drop-in, plus the tier bar
    against the restated q4_dot."""
    W, x, R, C = reference_unit_inputs()[ty]
    y = torch.empty(R, device=dev)
    ops.gemv(dev_t(W, dev), R, C, ty, dev_t(x, dev), y)
    got = host(y)
    dense = orc.dequant(W, R, C, ty).astype(np.float64)
    np.testing.assert_allclose(got, dense @ x.astype(np.float64), atol=0.00015, rtol=0.00001)
    assert_close_inf(got, orc.matvec_f32(W, R, C, ty, x).astype(np.float64))


@pytest.mark.parametrize("ty,R,C", [(12, 4096, 4096), (14, 4096, 12288), (12, 40, 4352), (14, 8, 256),
                                    (12, 16, 61440), (14, 8, 61440)])
def test_gemv_f32_vs_oracle(dev, orc, ty, R, C):
    W = synth(R, C, ty, 3 * R + ty)
    x = kqq.synthetic_activations(1, C, seed=C + 1)[0]
    y = torch.empty(R, device=dev)
    ops.gemv(dev_t(W, dev), R, C, ty, dev_t(x, dev), y)
    assert_close_inf(host(y), orc.matvec_f32(W, R, C, ty, x).astype(np.float64))


@pytest.mark.parametrize("shapes,C", [
    (((4096, 12), (1024, 12), (1024, 14)), 4096),    # mixed types: one launch
    (((1024, 14), (2048, 14), (4096, 12)), 4096),
    (((40, 12), (8, 14)), 256),
    (((4096, 12), (1024, 12), (1024, 14)), 12288),   # three passes: one launch per type
    (((12288, 12), (12288, 12)), 4096),              # one type
])
def test_gemv_f32_multi_matches_single(dev, orc, shapes, C):
    """kq_gemv_multi (fp32 activations, up to 3 matrices sharing x, both types in one launch where it
    can) equals kq_gemv on each matrix alone bit for bit, nothing written past R."""
    print("f32 multi", shapes, C, flush=True)
    mats_h = [(synth(R, C, ty, 30 + i), R, C, ty) for i, (R, ty) in enumerate(shapes)]
    mats = [(dev_t(W, dev), R, C_, ty) for (W, R, C_, ty) in mats_h]
    x = kqq.synthetic_activations(1, C, seed=C + 9)[0]
    xd = dev_t(x, dev)
    ys = [torch.full((R + 4,), -7.0, device=dev) for (_, R, _, _) in mats]
    ops.gemv_multi(mats, xd, ys)
    for (w, R, C_, ty), y, (W, _, _, _) in zip(mats, ys, mats_h):
        ref = torch.empty(R, device=dev)
        ops.gemv(w, R, C_, ty, xd, ref)
        got = host(y)
        np.testing.assert_array_equal(got[:R], host(ref))
        assert np.all(got[R:] == -7.0)
        if R <= 4096:
            assert_close_inf(got[:R], orc.matvec_f32(W, R, C_, ty, x).astype(np.float64))


@pytest.mark.parametrize("ty", [12, 14])
@pytest.mark.parametrize("scale", [1e-20, 1e20])
def test_gemv_f32_activation_scales(dev, orc, ty, scale):
    """The fp32-x GEMV multiplies each code as an f16 subnormal (code * 2^-24 or 2^-20) and keeps
    the accumulator scaled by that power of two; activations many decades from 1 stay within the
    bar of the oracle."""
    R, C = 1024, 4096
    W = synth(R, C, ty, 11 + ty)
    x = (kqq.synthetic_activations(1, C, seed=5)[0] * np.float32(scale)).astype(np.float32)
    y = torch.empty(R, device=dev)
    ops.gemv(dev_t(W, dev), R, C, ty, dev_t(x, dev), y)
    assert_close_inf(host(y), orc.matvec_f32(W, R, C, ty, x).astype(np.float64))


def test_random_shapes_sweep(dev, orc):
    """Seeded sweep over ragged shapes (R = 8..520, C = 256..8192, N = 1..16, M = 1..300, both types):
    GEMV rows within the bar of the oracle and bit-equal to their one-token results; the fp32-activation
    GEMV within the bar of q4_dot's restatement; the GEMM (both entry points, split or not) within the
    bar."""
    rng = np.random.default_rng(2024)
    for case in range(24):
        ty = (12, 14)[case % 2]
        R = 8 * int(rng.integers(1, 66))
        C = 256 * int(rng.integers(1, 33))
        N = int(rng.integers(1, 17))
        M = int(rng.integers(1, 301))
        W = synth(R, C, ty, 1000 + case)
        Wd = dev_t(W, dev)
        X = kqq.synthetic_activations(max(N, M), C, seed=2000 + case)
        xq = orc.quantize_q8k(X)
        xqd = dev_t(xq, dev)
        tag = (case, ty, R, C, N, M)
        yb = torch.empty((N, R), device=dev)
        ops.gemv_q8k(Wd, R, C, ty, xqd, N, yb)
        ref = orc.gemv_q8k(W, R, C, ty, xq[:N], N)
        assert_close_inf(host(yb), ref)
        y1 = torch.empty(R, device=dev)
        n = int(rng.integers(0, N))
        ops.gemv_q8k(Wd, R, C, ty, xqd[n:n + 1], 1, y1)
        assert np.array_equal(host(y1), host(yb)[n]), tag
        if C <= 4096:   # the same row with its quantization inside the GEMV launch
            yx = torch.empty(R, device=dev)
            ops.gemv_q8k_x([(Wd, R, C, ty)], dev_t(np.ascontiguousarray(X[n]), dev), [yx])
            assert np.array_equal(host(yx), host(y1)), tag
        yf = torch.empty(R, device=dev)     # fp32 activations (Kindi numerics)
        ops.gemv(Wd, R, C, ty, dev_t(np.ascontiguousarray(X[n]), dev), yf)
        assert_close_inf(host(yf), orc.matvec_f32(W, R, C, ty, X[n]).astype(np.float64))
        refm = orc.gemv_q8k(W, R, C, ty, xq[:M], M)
        ym = torch.empty((M, R), device=dev)
        ops.gemm_q8k(Wd, R, C, ty, xqd, M, ym)
        assert_close_inf(host(ym), refm)
        ops.gemm_q8k(Wd, R, C, ty, xqd, M, ym, ws=ops.gemm_workspace(R, C, M, dev))
        assert_close_inf(host(ym), refm)
