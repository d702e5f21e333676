"""PackWeights (the device tensor cache over a Kindi pack, gpu4.py:17-48) and Engine.embed on the
GPU: bytes as written, the byte budget with the embedding and head spared, an Engine backed by a
pack giving the same outputs as one backed by in-memory weights, and the embedding row decode."""
import numpy as np
import pytest
import torch

from kq import pack, quantize as kqq
from kq.gpu4 import Engine, Weights

pytestmark = pytest.mark.gpu

DIMS = {"layers": 1, "width": 4096}
SPEC = {"token_embd.weight": (2048, 4096, 12), "output.weight": (2048, 4096, 14),
        "blk.0.ffn_gate.weight": (12288, 4096, 12), "blk.0.ffn_up.weight": (12288, 4096, 12),
        "blk.0.ffn_down.weight": (4096, 12288, 14), "blk.0.post_attention_norm.weight": (1, 4096, 0)}


@pytest.fixture(scope="module")
def built(tmp_path_factory):
    tensors = {}
    for i, (name, (R, C, ty)) in enumerate(SPEC.items()):
        data = (1 + 0.1 * np.random.default_rng(i).standard_normal(C)).astype(np.float32) if ty == 0 \
            else kqq.synthetic_matrix(R, C, ty, seed=20 + i)
        tensors[name] = (data, R, C, ty)
    p = tmp_path_factory.mktemp("pk") / "pack"
    pack.write_pack(p, tensors, dims=DIMS)
    return p, tensors


def shapes():
    return {n: (R, C) for n, (R, C, _) in SPEC.items()}


def test_pack_weights_bytes_and_budget(dev, built):
    p, tensors = built
    # an explicit budget below 1.6 GB would not pin by the reference's rule (gpu4.py:24): pin here
    w = pack.open_pack(p, full=True, limit=60_000_000, device=dev, dims=DIMS, shapes=shapes(), pin_boundaries=True)
    for name in ("token_embd.weight", "output.weight", "blk.0.ffn_gate.weight"):
        buf, R, C, ty = w[name]
        assert (R, C, ty) == tensors[name][1:] and buf.is_cuda
        np.testing.assert_array_equal(buf.cpu().numpy(), tensors[name][0])
    assert w.misses == 3 and w.hits == 0
    # 28.3 MB more does not fit the 60 MB budget: the gate goes, embedding and head stay
    w["blk.0.ffn_up.weight"]
    assert "blk.0.ffn_gate.weight" not in w.cache and "token_embd.weight" in w.cache and "output.weight" in w.cache
    w["output.weight"]
    assert w.hits == 1 and w.used <= 60_000_000
    np.testing.assert_array_equal(w.f32("blk.0.post_attention_norm.weight").cpu().numpy(),
                                  tensors["blk.0.post_attention_norm.weight"][0])
    w.close()


def test_engine_on_pack_matches_in_memory_weights(dev, built, orc):
    p, tensors = built
    pw = pack.PackWeights(p, device=dev)
    mem = Weights(dev)
    for name, (data, R, C, ty) in tensors.items():
        if ty:
            mem.add(name, data, R, C, ty)
    x = torch.from_numpy(kqq.synthetic_activations(1, 4096, seed=4)[0]).to(dev)
    outs = []
    for w in (pw, mem):
        eng = Engine(w, mode="q8k")               # workspace sized from the pack index
        ys = [torch.empty(12288, device=dev), torch.empty(12288, device=dev)]
        eng.gemv(["blk.0.ffn_gate.weight", "blk.0.ffn_up.weight"], x, ys)
        emb = eng.embed(1234)
        outs.append((ys, emb.clone()))
        with pytest.raises(ValueError, match="Invalid token"):
            eng.embed(2048)
    for a, b in zip(outs[0][0], outs[1][0]):
        assert torch.equal(a, b)
    np.testing.assert_array_equal(outs[0][1].cpu().numpy(),
                                  orc.dequant_row(tensors["token_embd.weight"][0], 2048, 4096, 12, 1234))
    pw.close()


def test_large_tensor_read_by_several_readers(dev, tmp_path):
    """A tensor from PARALLEL_MIN up is read by READERS host threads in contiguous ranges (the last
    one partial): the device bytes equal the file's, and a second PackWeights on the same pack, read
    while the first's cache holds the tensor, agrees."""
    R, C = 21848, 4096                        # 21848 x 16 x 144 B = 50.3 MB: below the threshold
    R2 = 47000                                 # Q6_K 47000 x 16 x 210 = 157.9 MB (not a multiple of 8 MiB)
    rng = np.random.default_rng(5)
    big = rng.integers(0, 256, R2 * 16 * 210, dtype=np.uint8)
    small = rng.integers(0, 256, R * 16 * 144, dtype=np.uint8)
    tensors = {"output.weight": (big, R2, C, 14), "token_embd.weight": (small, R, C, 12)}
    p = tmp_path / "pack"
    pack.write_pack(p, tensors, dims={"layers": 0, "width": 4096})
    assert big.nbytes >= pack.PARALLEL_MIN and small.nbytes < pack.PARALLEL_MIN
    w = pack.PackWeights(p, device=dev)
    for name, (data, rows, ne0, ty) in tensors.items():
        buf, r, c, t = w[name]
        assert (r, c, t) == (rows, ne0, ty)
        assert np.array_equal(buf.cpu().numpy(), data), name
    assert w.read_bytes == big.nbytes + small.nbytes
    w2 = pack.PackWeights(p, device=dev)
    assert torch.equal(w2["output.weight"][0], w["output.weight"][0])
    w.close()
    w2.close()
