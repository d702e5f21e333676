"""Parity at the benchmarked sizes.

* Prefill GEMM at M = 512 and 2048 tokens on 12288x4096 Q4_K and 4096x12288 Q6_K, called exactly as
  bench.py times it (kq_gemm_q8k_ws with a preallocated workspace; the Q6_K M = 512 launch splits K
  two ways): every output against the batched GEMV of the same rows, sampled 8-row tiles (the first
  and last, and both sides of a 64-row tile boundary) over every token against the oracle, and every
  row of a few tokens (both ends of the first 128-token tile, the last two tokens) against the oracle.
* The 151936x4096 Q6_K output head of the full decode stream through kq_gemv_q8k and
  kq_gemv_q8k_argmax, and a 248320x4096 Q4_K head (the real model's output size) through the fused
  pick, against the oracle's GEMV and k_argmax.
* The odd layers' Q4_K ffn_down (4096x12288) against the oracle.

Bar: within 1e-5 * max|y_ref| (y_ref from the oracle's exact integer sums, evaluated in double); the
pick equal to the oracle's k_argmax of the logits; the fused logits bit-identical to the GEMV's.
"""
import numpy as np
import pytest
import torch

from kq import ops, quantize as kqq

pytestmark = pytest.mark.gpu
TOL = 1e-5
BS = {12: 144, 14: 210}


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def assert_close_inf(got, want, tag="", tol=TOL):
    scale = np.abs(want).max()
    err = np.abs(got.astype(np.float64) - want).max()
    assert err <= tol * scale, "%s: max err %.3g vs %.3g * %.3g" % (tag, err, tol, scale)


def tile_rows(W, C, ty, tiles):
    """Bytes and row indices of the chosen 8-row tiles: in the Kindi layout [R/8][G][8][bs] the G
    block columns of one tile are contiguous, so a tile slice is itself a valid 8-row matrix."""
    n = (C // 256) * 8 * BS[ty]
    return (np.concatenate([W[t * n:(t + 1) * n] for t in tiles]),
            np.array([8 * t + i for t in tiles for i in range(8)]))


CONFIG4 = [(12, 12288, 4096, 512), (12, 12288, 4096, 2048), (14, 4096, 12288, 512), (14, 4096, 12288, 2048)]


@pytest.mark.parametrize("ty,R,C,M", CONFIG4)
def test_gemm_prefill_full_size(dev, orc, ty, R, C, M):
    print("gemm", ty, R, C, M, flush=True)
    W = kqq.synthetic_matrix(R, C, ty, seed=60 + ty)          # the weights bench.py times
    X = kqq.synthetic_activations(M, C, seed=M)
    wd = dev_t(W, dev)
    xqd = ops.q8k_quantize(dev_t(X, dev))
    xq = host(xqd)
    ws = ops.gemm_workspace(R, C, M, dev)
    y = torch.empty((M, R), device=dev)
    ops.gemm_q8k(wd, R, C, ty, xqd, M, y, ws=ws)
    got = host(y)
    assert np.isfinite(got).all()

    # every output against the batched GEMV (16 tokens per call; its rows are pinned to the oracle
    # and bit-identical to one-token decode)
    yb = torch.empty((M, R), device=dev)
    for n0 in range(0, M, 16):
        ops.gemv_q8k(wd, R, C, ty, xqd[n0:n0 + 16], 16, yb[n0:n0 + 16])
    assert_close_inf(got, host(yb).astype(np.float64), "gemm vs batched gemv")

    # sampled tiles x every token against the oracle
    last = R // 8 - 1
    Ws, rows = tile_rows(W, C, ty, [0, 7, 8, last // 2, last])
    assert_close_inf(got[:, rows], orc.gemv_q8k(Ws, len(rows), C, ty, xq, M), "sampled rows")

    # every row of a few tokens against the oracle
    toks = [0, 127, 128, M - 2, M - 1]
    assert_close_inf(got[toks], orc.gemv_q8k(W, R, C, ty, xq[toks], len(toks)), "sampled tokens")

    # the entry point without a workspace: the same bits when the workspace form does not split K
    if M == 512:
        y2 = torch.empty((M, R), device=dev)
        ops.gemm_q8k(wd, R, C, ty, xqd, M, y2)
        got2 = host(y2)
        splits = ops.gemm_workspace_bytes(R, C, M) > -(-M // 256) * 256 * C
        if splits:
            assert_close_inf(got2, host(yb).astype(np.float64), "direct form")
        else:
            np.testing.assert_array_equal(got2, got)


@pytest.fixture(scope="module")
def head_q6k(dev):
    """The decode stream's Q6_K lm_head (bench.py: seed 999)."""
    R, C = 151936, 4096
    W = kqq.synthetic_matrix(R, C, 14, seed=999)
    return W, dev_t(W, dev), R, C


@pytest.mark.parametrize("seed", [0, 3])
def test_head_151936_q6k(dev, orc, head_q6k, seed):
    W, wd, R, C = head_q6k
    print("head q6k seed", seed, flush=True)
    xq = orc.quantize_q8k(kqq.synthetic_activations(1, C, seed=seed))
    xqd = dev_t(xq, dev)
    y = torch.empty(R, device=dev)
    ops.gemv_q8k(wd, R, C, 14, xqd, 1, y)
    logits = host(y)
    ref = orc.gemv_q8k(W, R, C, 14, xq, 1)[0]
    assert_close_inf(logits, ref, "head gemv")
    ws = ops.argmax_workspace(dev)
    yf = torch.full((R,), -9.0, device=dev)
    out = ops.gemv_q8k_argmax(wd, R, C, 14, xqd, yf, ws)
    np.testing.assert_array_equal(host(yf), logits)
    top = int(host(out)[0])
    assert top == orc.argmax(logits)
    # the pick is also the oracle's own top logit unless two logits lie within the bar of each other
    srt = np.sort(ref)
    if srt[-1] - srt[-2] > 2 * TOL * np.abs(ref).max():
        assert top == int(np.argmax(ref))


@pytest.mark.parametrize("seed", [0, 3])
def test_engine_head_f32_151936_q6k(dev, orc, head_q6k, seed):
    """Engine.head in the reference's numerics (mode "f32"): the fp32-activation GEMV, then the
    argmax over its logits, as Engine.head runs gemv([head]) + k_argmax (engine.py:326-328).  The
    logits within the bar of the oracle's restatement of q4_dot (kc_matvec bit for bit), the pick
    the oracle's k_argmax of the logits."""
    from kq.gpu4 import Engine, Weights
    W, wd, R, C = head_q6k
    print("engine head f32 seed", seed, flush=True)
    w = Weights(dev)
    w.cache["output.weight"] = (wd, R, C, 14)
    eng = Engine(w, mode="f32", chunk=0)
    x = kqq.synthetic_activations(1, C, seed=seed)[0]
    top = eng.head("output.weight", dev_t(x, dev))
    logits = host(eng.logits[:R])
    ref = orc.matvec_f32(W, R, C, 14, x)
    assert_close_inf(logits, ref.astype(np.float64), "head f32")
    assert top == orc.argmax(logits)
    srt = np.sort(ref)
    if srt[-1] - srt[-2] > 2 * TOL * np.abs(ref).max():
        assert top == int(np.argmax(ref))
    y = torch.empty(R, device=dev)                          # a caller's logits buffer
    assert eng.head("output.weight", dev_t(x, dev), y) == top
    np.testing.assert_array_equal(host(y), logits)


def random_q4k_blocks(R, C, seed):
    """Random Q4_K block bytes (any scale/min pattern) with d, dmin drawn from fp16 values of the
    size a N(0, 0.02) row gives, in the Kindi layout."""
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, (R, C // 256, 144), dtype=np.uint8)
    raw[:, :, 0:2] = (rng.uniform(2e-4, 6e-4, (R, C // 256)).astype(np.float16).view(np.uint8)
                      .reshape(R, C // 256, 2))
    raw[:, :, 2:4] = (rng.uniform(5e-4, 2e-3, (R, C // 256)).astype(np.float16).view(np.uint8)
                      .reshape(R, C // 256, 2))
    return kqq.tile(raw.reshape(-1), R, C, 12)


def test_head_248320_q4k_fused_pick(dev, orc):
    """A Q4_K head of the real model's output size (output.weight 248320x4096, q4pack.py:22)."""
    R, C = 248320, 4096
    print("head q4k 248320", flush=True)
    W = random_q4k_blocks(R, C, 5)
    wd = dev_t(W, dev)
    xq = orc.quantize_q8k(kqq.synthetic_activations(1, C, seed=11))
    xqd = dev_t(xq, dev)
    y = torch.empty(R, device=dev)
    ws = ops.argmax_workspace(dev)
    out = ops.gemv_q8k_argmax(wd, R, C, 12, xqd, y, ws)
    logits = host(y)
    assert_close_inf(logits, orc.gemv_q8k(W, R, C, 12, xq, 1)[0], "q4k head")
    assert int(host(out)[0]) == orc.argmax(logits)
    y1 = torch.empty(R, device=dev)
    ops.gemv_q8k(wd, R, C, 12, xqd, 1, y1)
    np.testing.assert_array_equal(host(y1), logits)


@pytest.mark.parametrize("N", [1, 2, 4])
def test_q4k_down_4096x12288(dev, orc, N):
    """The odd layers' ffn_down is Q4_K 4096x12288 in the full decode stream (seed as bench.py)."""
    R, C = 4096, 12288
    W = kqq.synthetic_matrix(R, C, 12, seed=172)
    xq = orc.quantize_q8k(kqq.synthetic_activations(N, C, seed=9))
    y = torch.empty((N, R), device=dev)
    ops.gemv_q8k(dev_t(W, dev), R, C, 12, dev_t(xq, dev), N, y)
    assert_close_inf(host(y), orc.gemv_q8k(W, R, C, 12, xq, N), "down q4k")
