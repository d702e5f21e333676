"""The entry points on a side stream and inside a captured HIP graph: every replay gives the bits of
the eager calls, with eager work between the replays.  (No kernel records a memset node: the argmax
workspace is reset by its own last workgroup, and the GEMM's K-split partial sums are overwritten,
not accumulated.)"""
import pytest
import torch

from kq import ops, quantize as kqq

pytestmark = pytest.mark.gpu


def test_side_stream_and_graph_replays_match_eager(dev):
    g0 = torch.Generator(device="cpu").manual_seed(11)
    C, R1, R2, M = 4096, 4096, 1024, 96
    W1 = torch.from_numpy(kqq.synthetic_matrix(R1, C, 12, 3)).to(dev)
    W2 = torch.from_numpy(kqq.synthetic_matrix(R2, C, 14, 4)).to(dev)
    Wd = torch.from_numpy(kqq.synthetic_matrix(1024, 12288, 14, 5)).to(dev)
    h = torch.randn(1, C, generator=g0).to(dev)
    wn = (torch.rand(C, generator=g0) + 0.5).to(dev)
    gate = torch.randn(1, 12288, generator=g0).to(dev)
    up = torch.randn(1, 12288, generator=g0).to(dev)
    X = torch.randn(M, C, generator=g0).to(dev)
    ws = ops.gemm_workspace(R1, C, M, dev)                    # 64 tiles: K split 4 ways
    aws = ops.argmax_workspace(dev)

    def buffers():
        return {
            "xq1": torch.zeros(1, (C // 256) * 292, dtype=torch.uint8, device=dev),
            "xq2": torch.zeros(1, 48 * 292, dtype=torch.uint8, device=dev),
            "xqm": torch.zeros(M, (C // 256) * 292, dtype=torch.uint8, device=dev),
            "y1": torch.zeros(R1, device=dev), "y2": torch.zeros(R2, device=dev),
            "y3": torch.zeros(1024, device=dev), "y4": torch.zeros(R1, device=dev),
            "ym": torch.zeros(M, R1, device=dev), "idx": torch.zeros(1, dtype=torch.int32, device=dev),
        }

    def run(b):
        ops.rms_q8k(h, wn, xq=b["xq1"])                                            # RMSNorm -> Q8_K
        ops.gemv_q8k_multi([(W1, R1, C, 12), (W2, R2, C, 14)], b["xq1"], 1, [b["y1"], b["y2"]])
        ops.swiglu_q8k(gate, up, xq=b["xq2"])                                      # SwiGLU -> Q8_K
        ops.gemv_q8k(Wd, 1024, 12288, 14, b["xq2"], 1, b["y3"])
        ops.q8k_quantize(X, b["xqm"])
        ops.gemm_q8k(W1, R1, C, 12, b["xqm"], M, b["ym"], ws=ws)                  # split-K prefill
        ops.gemv_q8k_argmax(W1, R1, C, 12, b["xq1"], b["y4"], aws, b["idx"])     # head + greedy pick

    ref = buffers()
    run(ref)
    torch.cuda.synchronize()

    out = buffers()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run(out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for k in ref:
        assert torch.equal(out[k], ref[k]), ("side stream", k)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(out)
    for rep in range(3):
        for t in out.values():                   # eager work between the replays
            t.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k in ref:
            assert torch.equal(out[k], ref[k]), ("replay", rep, k)
