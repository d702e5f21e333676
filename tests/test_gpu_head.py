"""Greedy pick over the logits: kq_argmax and the fused head GEMV + argmax (kq_gemv_q8k_argmax)
against the oracle's k_argmax (kindi.cu:637-661): the index exactly, the fused GEMV's logits bit
for bit equal to kq_gemv_q8k's."""
import numpy as np
import pytest
import torch

from kq import ops, quantize as kqq

pytestmark = pytest.mark.gpu
F32 = np.float32


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def pick(out):
    torch.cuda.synchronize()
    return int(out.cpu()[0])


def argmax_cases():
    rng = np.random.default_rng(12)
    y = rng.standard_normal(151936).astype(F32)
    ties = y.copy()
    ties[[123457, 40000, 150001]] = 7.5                      # equal maxima: 40000 wins
    special = ties.copy()
    special[[3, 99]] = np.nan
    special[200] = np.inf
    return [
        ("random", y), ("ties", ties), ("inf and nan", special),
        ("all -inf", np.full(5000, -np.inf, F32)), ("below -1e30", np.full(777, -3e30, F32)),
        ("one", np.array([-5.0], F32)), ("ragged", rng.standard_normal(1025).astype(F32)),
        ("negative", (-1 - rng.random(300000)).astype(F32)),
    ]


def test_argmax_vs_oracle_and_repeated_calls(dev, orc):
    ws = ops.argmax_workspace(dev)
    out = torch.empty(1, dtype=torch.int32, device=dev)
    for rep in range(2):                                     # the workspace is reused call after call
        for name, y in argmax_cases():
            ops.argmax(dev_t(y, dev), ws, out)
            assert pick(out) == orc.argmax(y), (name, rep)
    torch.cuda.synchronize()
    assert int(ws.to(torch.int32).abs().sum()) == 0           # every call leaves it zero for the next


def head_matrix(R, C, ty, seed, dup=None):
    """Kindi-layout weights; dup = (src, dst rows): rows dst get row src's bytes (equal logits)."""
    w = kqq.synthetic_fp32(R, C, seed)
    if dup is not None:
        src, dst = dup
        w[list(dst)] = w[src]
    return kqq.tile(kqq.quantize(w, ty), R, C, ty)


@pytest.mark.parametrize("ty", [12, 14])
@pytest.mark.parametrize("R,C", [(8, 256), (4096, 4096), (32776, 4096), (1024, 12288)])
def test_gemv_argmax_fused(dev, orc, ty, R, C):
    W = head_matrix(R, C, ty, seed=R + C + ty)
    x = kqq.synthetic_activations(1, C, seed=5)
    wd, xq = dev_t(W, dev), ops.q8k_quantize(dev_t(x, dev))
    ws = ops.argmax_workspace(dev)
    y = torch.empty(R, device=dev)
    out = ops.gemv_q8k_argmax(wd, R, C, ty, xq, y, ws)
    y_ref = torch.empty(R, device=dev)
    ops.gemv_q8k(wd, R, C, ty, xq, 1, y_ref)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    assert pick(out) == orc.argmax(y.cpu().numpy())


@pytest.mark.parametrize("ty", [12, 14])
def test_gemv_argmax_ties_pick_the_first_row(dev, orc, ty):
    """Rows with the same bytes give the same logit bits; the smallest of them must win."""
    R, C = 16384, 4096
    base = kqq.synthetic_fp32(R, C, seed=3)
    x = kqq.synthetic_activations(1, C, seed=6)
    best = int(np.argmax(base @ x[0]))
    W = head_matrix(R, C, ty, seed=3, dup=(best, [best + 8001, 15999]))
    wd, xq = dev_t(W, dev), ops.q8k_quantize(dev_t(x, dev))
    ws = ops.argmax_workspace(dev)
    y = torch.empty(R, device=dev)
    out = ops.gemv_q8k_argmax(wd, R, C, ty, xq, y, ws)
    yh = y.cpu().numpy()
    top = np.flatnonzero(yh == yh.max())
    assert len(top) >= 3 and pick(out) == top[0] == orc.argmax(yh)
