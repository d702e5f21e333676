"""Run-to-run determinism of every path whose result crosses workgroups or waves: the multi-matrix
decode GEMV (one pass), the pass-split GEMV (partials merged in LDS), the sequential three-pass
Q6_K GEMV, the MFMA small-batch GEMV, the prefill GEMM with and without its K split (ordered
reduce), the fused head's argmax (ticket and 64-bit atomic maximum), and the producers.  The
paths run interleaved 30 times on fixed inputs; every output must equal the first call's bit for
bit, and the fused head's index the argmax of its own logits."""
import numpy as np
import pytest
import torch

from kq import ops, quantize as kqq

pytestmark = pytest.mark.gpu
Q4, Q6 = 12, 14
REPEATS = 30


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def mat(R, C, ty, seed, dev):
    return (dev_t(kqq.synthetic_matrix(R, C, ty, seed), dev), R, C, ty)


def test_repeated_calls_are_bit_identical(dev):
    gate, up = mat(12288, 4096, Q4, 1, dev), mat(12288, 4096, Q4, 2, dev)
    down6 = mat(4096, 12288, Q6, 3, dev)            # sequential kernel, three passes in registers
    down4 = mat(4096, 12288, Q4, 4, dev)            # pass-split kernel, three pass waves per unit
    head = mat(32768, 4096, Q6, 5, dev)             # fused greedy pick
    x4 = ops.q8k_quantize(dev_t(kqq.synthetic_activations(8, 4096, seed=6), dev))
    x12 = ops.q8k_quantize(dev_t(kqq.synthetic_activations(1, 12288, seed=7), dev))
    X128 = ops.q8k_quantize(dev_t(kqq.synthetic_activations(128, 12288, seed=8), dev))
    X300 = ops.q8k_quantize(dev_t(kqq.synthetic_activations(300, 4096, seed=9), dev))
    rng = np.random.default_rng(10)
    h0 = dev_t((rng.standard_normal(4096) * 3).astype(np.float32), dev)
    res = dev_t(rng.standard_normal(4096).astype(np.float32), dev)
    wn = dev_t((1 + 0.2 * rng.standard_normal(4096)).astype(np.float32), dev)
    g = dev_t((rng.standard_normal(12288) * 2).astype(np.float32), dev)
    u = dev_t(rng.standard_normal(12288).astype(np.float32), dev)
    ws_gemm = ops.gemm_workspace(4096, 12288, 128, dev)
    ws_gemm2 = ops.gemm_workspace(12288, 4096, 300, dev)
    ws_arg = ops.argmax_workspace(dev)

    def run():
        out = {}
        gy, uy = torch.empty(12288, device=dev), torch.empty(12288, device=dev)
        ops.gemv_q8k_multi([gate, up], x4[:1], 1, [gy, uy])
        out["gate"], out["up"] = gy, uy
        for name, m in (("down6", down6), ("down4", down4)):
            y = torch.empty(4096, device=dev)
            ops.gemv_q8k(m[0], 4096, 12288, m[3], x12, 1, y)
            out[name] = y
        Y8 = torch.empty((8, 12288), device=dev)
        ops.gemv_q8k(gate[0], 12288, 4096, Q4, x4, 8, Y8)
        out["mfma8"] = Y8
        Yk = torch.empty((128, 4096), device=dev)
        ops.gemm_q8k(down6[0], 4096, 12288, Q6, X128, 128, Yk, ws=ws_gemm)      # K split 4 ways
        out["gemm_split"] = Yk
        Yg = torch.empty((300, 12288), device=dev)
        ops.gemm_q8k(gate[0], 12288, 4096, Q4, X300, 300, Yg, ws=ws_gemm2)      # no split
        out["gemm"] = Yg
        logits = torch.empty(32768, device=dev)
        idx = ops.gemv_q8k_argmax(head[0], 32768, 4096, Q6, x4[:1], logits, ws_arg)
        out["logits"], out["pick"] = logits, idx.clone()
        h = h0.clone()
        xn = torch.empty(4096, device=dev)
        _, xq = ops.rms_q8k(h, wn, residual=res, xn=xn)
        out["h"], out["xn"], out["xq_rms"] = h, xn, xq
        y, xq2 = ops.swiglu_q8k(g, u, y=torch.empty(12288, device=dev))
        out["silu"], out["xq_silu"] = y, xq2
        torch.cuda.synchronize()
        return {k: v.cpu().numpy() for k, v in out.items()}

    first = run()
    assert int(first["pick"][0]) == int(np.argmax(first["logits"]))
    for rep in range(1, REPEATS):
        again = run()
        for k, v in first.items():
            assert np.array_equal(v.view(np.uint8), again[k].view(np.uint8)), (rep, k)
