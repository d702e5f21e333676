"""The Engine/Weights operator surface (mirror of scripts/kindi_q4/kindi/gpu4.py:17-110) on the
GPU: results, return value, argument errors, and the full decode-layer shapes."""
import numpy as np
import pytest
import torch

from kq import ops, quantize as kqq
from kq.gpu4 import Engine, Weights

pytestmark = pytest.mark.gpu

LAYER = [  # name, R, C, type: one 9B-class decode layer (q, k, v, o, gate, up: Q4_K; down: Q6_K)
    ("attn_q", 4096, 4096, 12), ("attn_k", 1024, 4096, 12), ("attn_v", 1024, 4096, 12),
    ("attn_output", 4096, 4096, 12), ("ffn_gate", 12288, 4096, 12), ("ffn_up", 12288, 4096, 12),
    ("ffn_down", 4096, 12288, 14),
]


@pytest.fixture(scope="module")
def layer(dev):
    w = Weights(dev)
    host = {}
    for i, (name, R, C, ty) in enumerate(LAYER):
        W = kqq.synthetic_matrix(R, C, ty, seed=i)
        host[name] = (W, R, C, ty)
        w.add(name, W, R, C, ty)
    return w, host


def test_weights_tuple_contract(layer):
    w, host = layer
    buf, R, C, ty = w["ffn_down"]
    assert (R, C, ty) == (4096, 12288, 14) and buf.dtype == torch.uint8 and buf.is_cuda
    assert buf.numel() == 4096 * 48 * 210


@pytest.mark.parametrize("mode", ["q8k", "f32"])
def test_engine_gemv_layer(layer, orc, dev, mode):
    """gemv(names, x, outs) -> 1 for the attention and FFN groups; outputs vs the oracle."""
    w, host = layer
    eng = Engine(w, mode=mode)
    groups = [(["attn_q", "attn_k", "attn_v"], 4096), (["attn_output"], 4096),
              (["ffn_gate", "ffn_up"], 4096), (["ffn_down"], 12288)]
    for g, (names, C) in enumerate(groups):
        x = kqq.synthetic_activations(1, C, seed=100 + g)[0]
        outs = [torch.empty(host[n][1], device=dev) for n in names]
        assert eng.gemv(names, torch.from_numpy(x).to(dev), outs) == 1
        torch.cuda.synchronize()
        for n, y in zip(names, outs):
            W, R, C_, ty = host[n]
            if mode == "q8k":
                want = orc.gemv_q8k(W, R, C_, ty, orc.quantize_q8k(x[None]), 1)[0]
            else:
                want = orc.matvec_f32(W, R, C_, ty, x).astype(np.float64)
            got = y.cpu().numpy()
            assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max(), n


@pytest.mark.parametrize("mode", ["q8k", "f32"])
def test_engine_gemv_q4k_m_attention_group(dev, orc, mode):
    """A Q4_K_M layer's attention group (Q4_K q, k and a Q6_K v, as half the real model's layers have):
    gemv(names, x, outs) sends both types through one launch; every output equals the one-matrix
    call bit for bit and the oracle within the bar."""
    w = Weights(dev)
    host = {}
    for i, (name, R, ty) in enumerate([("attn_q", 4096, 12), ("attn_k", 1024, 12), ("attn_v", 1024, 14)]):
        W = kqq.synthetic_matrix(R, 4096, ty, seed=40 + i)
        host[name] = (W, R, 4096, ty)
        w.add(name, W, R, 4096, ty)
    eng = Engine(w, mode=mode)
    x = kqq.synthetic_activations(1, 4096, seed=41)[0]
    xd = torch.from_numpy(x).to(dev)
    names = ["attn_q", "attn_k", "attn_v"]
    outs = [torch.empty(host[n][1], device=dev) for n in names]
    assert eng.gemv(names, xd, outs) == 1
    for n, y in zip(names, outs):
        one = torch.empty(host[n][1], device=dev)
        assert eng.gemv([n], xd, [one]) == 1
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy(), one.cpu().numpy())
        W, R, C_, ty = host[n]
        if mode == "q8k":
            want = orc.gemv_q8k(W, R, C_, ty, orc.quantize_q8k(x[None]), 1)[0]
        else:
            want = orc.matvec_f32(W, R, C_, ty, x).astype(np.float64)
        got = y.cpu().numpy()
        assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max(), n


def test_engine_batch_and_gemm_agree(layer, dev):
    w, _ = layer
    eng = Engine(w, mode="q8k")
    X = torch.from_numpy(kqq.synthetic_activations(8, 4096, seed=9)).to(dev)
    yb = torch.empty((8, 12288), device=dev)
    ym = torch.empty((8, 12288), device=dev)
    assert eng.gemv_batch(["ffn_gate"], X, [yb]) == 1
    assert eng.gemm(["ffn_gate"], X, [ym]) == 1
    y1 = torch.empty(12288, device=dev)
    eng.gemv(["ffn_gate"], X[5], [y1])
    torch.cuda.synchronize()
    assert torch.equal(yb[5], y1)
    np.testing.assert_allclose(ym.cpu().numpy(), yb.cpu().numpy(), rtol=0, atol=1e-5 * yb.abs().max().item())


def test_engine_rejects_bad_calls(layer, dev):
    w, _ = layer
    eng = Engine(w, mode="q8k")
    x = torch.zeros(4096, device=dev)
    with pytest.raises(ValueError):
        eng.gemv(["attn_q", "ffn_down"], x, [torch.empty(4096, device=dev), torch.empty(4096, device=dev)])
    with pytest.raises(ValueError):
        eng.gemv(["attn_q"], x, [torch.empty(100, device=dev)])
    with pytest.raises(ValueError):
        eng.gemv_batch(["attn_q"], torch.zeros((17, 4096), device=dev), [torch.empty((17, 4096), device=dev)])
    with pytest.raises(KeyError):
        eng.gemv(["missing"], x, [torch.empty(4096, device=dev)])
    with pytest.raises(ValueError, match="unit stride|contiguous"):
        eng.gemv(["attn_q"], torch.zeros(8192, device=dev)[::2], [torch.empty(4096, device=dev)])
    with pytest.raises(ValueError, match="unit stride|contiguous"):
        eng.gemv(["attn_q"], x, [torch.empty(8192, device=dev)[::2]])
    with pytest.raises(ValueError, match="one output per matrix"):
        eng.gemv_batch(["attn_q", "attn_k"], torch.zeros((2, 4096), device=dev), [torch.empty((2, 4096), device=dev)])
    with pytest.raises(ValueError, match="one output per matrix"):
        eng.gemm(["attn_q", "attn_k"], torch.zeros((2, 4096), device=dev), [torch.empty((2, 4096), device=dev)])


def test_engine_batch_of_one_row_into_a_flat_output(layer, dev):
    """gemv_batch and gemm with one row and a 1-D output (row stride R) equal gemv."""
    w, _ = layer
    eng = Engine(w, mode="q8k")
    x = torch.from_numpy(kqq.synthetic_activations(1, 4096, seed=17)).to(dev)
    ref = torch.empty(4096, device=dev)
    eng.gemv(["attn_q"], x[0], [ref])
    for fn in (eng.gemv_batch, eng.gemm):
        y = torch.full((4096,), float("nan"), device=dev)
        fn(["attn_q"], x, [y])
        torch.cuda.synchronize()
        err = (y - ref).abs().max().item()
        assert err <= 1e-5 * ref.abs().max().item(), (fn.__name__, err)


def test_dequant_row_matches_oracle(layer, orc, dev):
    w, host = layer
    eng = Engine(w)
    for name in ("attn_k", "ffn_down"):
        W, R, C, ty = host[name]
        row = eng.dequant(name, R - 3)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(row.cpu().numpy(), orc.dequant_row(W, R, C, ty, R - 3))


def test_engine_producers_feed_gemv(layer, orc, dev):
    """rmsfold_q8k -> gemv_q8 (q/k/v) and swiglu_q8k -> gemv_q8 (down) give the same outputs, bit for
    bit, as gemv on the producers' fp32 outputs (which quantizes them itself)."""
    w, host = layer
    eng = Engine(w, mode="q8k")
    rng = np.random.default_rng(3)
    h = torch.from_numpy(rng.standard_normal(4096).astype(np.float32)).to(dev)
    res = torch.from_numpy(rng.standard_normal(4096).astype(np.float32)).to(dev)
    wn = torch.from_numpy((1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)).to(dev)
    xn = torch.empty(4096, device=dev)
    names = ["attn_q", "attn_k", "attn_v"]
    outs = [torch.empty(R, device=dev) for _, R, _, _ in LAYER[:3]]
    h0 = h.cpu().numpy().copy()
    _, xq = eng.rmsfold_q8k(h, wn, residual=res, xn=xn)
    assert eng.gemv_q8(names, xq, outs) == 1
    ref = [torch.empty_like(o) for o in outs]
    eng.gemv(names, xn, ref)
    for a, b in zip(outs, ref):
        assert torch.equal(a, b)
    h_want, xn_want = orc.rms_norm(h0, wn.cpu().numpy(), res.cpu().numpy())
    np.testing.assert_array_equal(h.cpu().numpy(), h_want[0])
    np.testing.assert_array_equal(xn.cpu().numpy(), xn_want[0])
    g = torch.from_numpy((rng.standard_normal(12288) * 2).astype(np.float32)).to(dev)
    u = torch.from_numpy(rng.standard_normal(12288).astype(np.float32)).to(dev)
    y = torch.empty(12288, device=dev)
    out = torch.empty(4096, device=dev)
    _, xq2 = eng.swiglu_q8k(g, u, y=y)
    eng.gemv_q8(["ffn_down"], xq2, [out])
    ref2 = torch.empty_like(out)
    eng.gemv(["ffn_down"], y, [ref2])
    assert torch.equal(out, ref2)


def test_engine_head_greedy_pick(dev, orc):
    """Engine.head -> int: the argmax of the logits (k_argmax's rule), logits left in y."""
    R, C = 8192, 4096
    w = Weights(dev)
    W = kqq.synthetic_matrix(R, C, 14, seed=31)
    w.add("output.weight", W, R, C, 14)
    eng = Engine(w, mode="q8k")
    x = torch.from_numpy(kqq.synthetic_activations(1, C, seed=2)[0]).to(dev)
    y = torch.empty(R, device=dev)
    tok = eng.head("output.weight", x, y)
    assert tok == orc.argmax(y.cpu().numpy())
    assert eng.head("output.weight", x) == tok            # engine-owned logits, workspace reused


def test_engine_feed_rows_dispatch(layer, dev):
    """feed_rows: up to 16 rows through the batched GEMV (rows equal one-token decode bit for bit),
    more through the GEMM (same values within the GEMM's own bar, bit-equal to Engine.gemm)."""
    w, host = layer
    eng = Engine(w, mode="q8k")
    X = torch.from_numpy(kqq.synthetic_activations(40, 4096, seed=9)).to(dev)
    names = ["ffn_gate"]
    y5 = torch.empty((5, 12288), device=dev)
    eng.feed_rows(names, X[:5], [y5])
    for n in range(5):
        one = torch.empty(12288, device=dev)
        eng.gemv(names, X[n], [one])
        assert torch.equal(y5[n], one)
    y40 = torch.empty((40, 12288), device=dev)
    eng.feed_rows(names, X, [y40])
    ref = torch.empty_like(y40)
    eng.gemm(names, X, [ref])
    assert torch.equal(y40, ref)
    fp = eng.fingerprint()
    assert len(fp["libkq"]) == 16 and fp["mode"] == "q8k"


def test_engine_f32_mode_batched_rows_are_decode_rows(layer, dev):
    """Mode "f32" keeps the reference's numerics on the batched paths too: gemv_batch, feed_rows
    (batched and prefill sizes) and gemm give every row bit-identical to gemv on that row (the
    reference's Q4 engine prefills token by token, gpu4.py:109-110), into 2-D and flat outputs."""
    w, host = layer
    eng = Engine(w, mode="f32")
    names = ["attn_q", "attn_k", "attn_v"]
    X = torch.from_numpy(kqq.synthetic_activations(20, 4096, seed=21)).to(dev)
    single = {n: torch.empty((20, host[n][1]), device=dev) for n in names}
    for r in range(20):
        eng.gemv(names, X[r], [single[n][r] for n in names])
    for call, rows in ((eng.gemv_batch, 6), (eng.feed_rows, 6), (eng.feed_rows, 20), (eng.gemm, 20)):
        outs = [torch.full((rows, host[n][1]), -1.0, device=dev) for n in names]
        assert call(names, X[:rows], outs) == 1
        for n, y in zip(names, outs):
            assert torch.equal(y, single[n][:rows]), (call.__name__, rows, n)
    flat = torch.empty(20 * 1024, device=dev)
    eng.gemm(["attn_k"], X, [flat])
    assert torch.equal(flat.view(20, 1024), single["attn_k"])


def test_engine_prefill_gemm_split_k_layer(layer, dev):
    """A 48-token prefill chunk through Engine.gemm for matrices of different R sharing one
    workspace: q/k/v (grids of 64 and 16 tiles: K split 4 ways) and down (K split 8 ways).  Every
    row is within the bar of its one-token GEMV, and a second call gives the same bits."""
    w, _ = layer
    eng = Engine(w, mode="q8k")
    M = 48
    for names, C in ((["attn_q", "attn_k", "attn_v"], 4096), (["ffn_down"], 12288)):
        X = torch.from_numpy(kqq.synthetic_activations(M, C, seed=C + 3)).to(dev)
        outs = [torch.empty((M, w[n][1]), device=dev) for n in names]
        assert eng.gemm(names, X, outs) == 1
        again = [torch.empty_like(o) for o in outs]
        eng.gemm(names, X, again)
        for n, y, y2 in zip(names, outs, again):
            R = w[n][1]
            ref = torch.empty((16, R), device=dev)
            for r0 in range(0, M, 16):
                eng.gemv_batch([n], X[r0:r0 + 16], [ref])
                want = ref.cpu().numpy()
                got = y[r0:r0 + 16].cpu().numpy()
                assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max(), (n, r0)
            assert torch.equal(y, y2), n


def test_engine_default_prefill_chunks(layer, dev, monkeypatch):
    """A 300-token prompt through a default-constructed Engine (KINDI_CHUNK unset: chunks of 256
    tokens, chunk.py:82,90): the rows of each chunk equal one kq_gemm_q8k_ws call on that chunk bit
    for bit, for matrices that do and do not split K."""
    monkeypatch.delenv("KINDI_CHUNK", raising=False)
    w, _ = layer
    eng = Engine(w)
    assert eng.chunk == 256
    M = 300
    for names, C in ((["attn_q", "attn_k", "attn_v"], 4096), (["ffn_gate", "ffn_up"], 4096), (["ffn_down"], 12288)):
        X = torch.from_numpy(kqq.synthetic_activations(M, C, seed=C + 11)).to(dev)
        outs = [torch.empty((M, w[n][1]), device=dev) for n in names]
        assert eng.gemm(names, X, outs) == 1
        for n, y in zip(names, outs):
            wt, R, C_, ty = w[n]
            for m0, mc in ((0, 256), (256, 44)):
                xq = ops.q8k_quantize(X[m0:m0 + mc])
                ref = torch.empty((mc, R), device=dev)
                ops.gemm_q8k(wt, R, C_, ty, xq, mc, ref, ws=ops.gemm_workspace(R, C_, mc, dev))
                assert torch.equal(y[m0:m0 + mc], ref), (n, m0)


@pytest.mark.parametrize("name,N", [("ffn_gate", 17), ("attn_q", 300)])
def test_engine_feed_rows_long_inputs(layer, dev, orc, name, N):
    """feed_rows on a default Engine with more rows than a batch (17) and more than a chunk (300)
    against the oracle."""
    w, host = layer
    eng = Engine(w)
    W, R, C, ty = host[name]
    X = kqq.synthetic_activations(N, C, seed=N)
    y = torch.empty((N, R), device=dev)
    assert eng.feed_rows([name], torch.from_numpy(X).to(dev), [y]) == 1
    torch.cuda.synchronize()
    want = orc.gemv_q8k(W, R, C, ty, orc.quantize_q8k(X), N)
    got = y.cpu().numpy()
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def test_engine_feed_rows_without_chunked_prefill(layer, dev, monkeypatch):
    """KINDI_CHUNK=0: no GEMM; longer inputs go through the batched GEMV 16 rows at a time, every
    row bit-identical to one-token decode."""
    monkeypatch.setenv("KINDI_CHUNK", "0")
    w, _ = layer
    eng = Engine(w)
    assert eng.chunk == 0 and eng.gemm_ws is None
    X = torch.from_numpy(kqq.synthetic_activations(37, 4096, seed=4)).to(dev)
    y = torch.empty((37, 1024), device=dev)
    eng.feed_rows(["attn_k"], X, [y])
    flat = torch.empty(37 * 1024, device=dev)                # a flat output holds rows of R
    eng.feed_rows(["attn_k"], X, [flat])
    for n in (0, 16, 36):
        one = torch.empty(1024, device=dev)
        eng.gemv(["attn_k"], X[n], [one])
        assert torch.equal(y[n], one), n
        assert torch.equal(flat[n * 1024:(n + 1) * 1024], one), n
    with pytest.raises(ValueError, match="chunked prefill is off"):
        eng.gemm(["attn_k"], X, [y])
    with pytest.raises(ValueError, match="output buffer too small"):
        eng.feed_rows(["attn_k"], X, [torch.empty(36 * 1024, device=dev)])


@pytest.mark.parametrize("mode", ["q8k", "f32"])
def test_engine_gemv_ignores_extra_outputs(layer, dev, mode):
    """More outputs than names: the extra ones are left alone, as the reference's zip does."""
    w, _ = layer
    eng = Engine(w, mode=mode)
    x = torch.from_numpy(kqq.synthetic_activations(1, 4096, seed=8)[0]).to(dev)
    outs = [torch.empty(4096, device=dev), torch.empty(1024, device=dev), torch.full((7,), -1.0, device=dev)]
    assert eng.gemv(["attn_q", "attn_k"], x, outs) == 1
    ref = [torch.empty(4096, device=dev), torch.empty(1024, device=dev)]
    eng.gemv(["attn_q", "attn_k"], x, ref)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], ref[0]) and torch.equal(outs[1], ref[1])
    assert torch.all(outs[2] == -1.0)


def test_engine_first_calls_capture_into_a_graph(layer, dev):
    """Nothing in an Engine call allocates, so a fresh Engine's first calls can be captured into a
    HIP graph: a 300-token prefill of the down projection (two chunks, K split), a decode GEMV of
    q/k/v and the token embedding.  Three replays, with eager calls of the same engine (which
    overwrite its Q8_K workspace) between them, each equal bit for bit to the eager results."""
    w, _ = layer
    eng = Engine(w)
    X = torch.from_numpy(kqq.synthetic_activations(300, 12288, seed=5)).to(dev)
    x = torch.from_numpy(kqq.synthetic_activations(1, 4096, seed=6)[0]).to(dev)
    qkv = ["attn_q", "attn_k", "attn_v"]

    def outputs():
        return [torch.full((300, 4096), float("nan"), device=dev)] + \
               [torch.full((R,), float("nan"), device=dev) for R in (4096, 1024, 1024)] + \
               [torch.full((4096,), float("nan"), device=dev)]      # one decoded row of ffn_gate

    cap = outputs()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):                         # the engine's first calls
        eng.gemm(["ffn_down"], X, [cap[0]])
        eng.gemv(qkv, x, cap[1:4])
        eng.dequant("ffn_gate", 77, cap[4])
    ref = outputs()
    eng.gemm(["ffn_down"], X, [ref[0]])
    eng.gemv(qkv, x, ref[1:4])
    eng.dequant("ffn_gate", 77, ref[4])
    torch.cuda.synchronize()
    other = torch.empty(12288, device=dev)
    for rep in range(3):
        for t in cap:
            t.fill_(float("nan"))
        eng.gemv(["ffn_gate"], X[rep, :4096], [other])   # eager work on the same workspace
        g.replay()
        eng.gemv(["ffn_up"], X[rep + 1, :4096], [other])
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(cap, ref)):
            assert torch.equal(a, b), (rep, i)
