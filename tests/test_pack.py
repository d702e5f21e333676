"""Kindi pack format on the host: writer, verify_pack's checks and messages (q4pack.py:86-108),
and the 9B profile table (q4pack.py:21-35).  No GPU."""
import json
import os

import numpy as np
import pytest

from kq import pack, quantize as kqq

TINY_DIMS = {"layers": 1, "width": 256}
TINY = {"token_embd.weight": (16, 256, 12), "output.weight": (16, 256, 14), "output_norm.weight": (1, 256, 0),
        "blk.0.ffn_down.weight": (8, 512, 14), "blk.0.ssm_alpha.weight": (32, 256, 0)}


def tiny_tensors():
    out = {}
    for i, (name, (R, C, ty)) in enumerate(TINY.items()):
        data = (np.random.default_rng(i).standard_normal((R, C)).astype(np.float32) if ty == 0
                else kqq.synthetic_matrix(R, C, ty, seed=i))
        out[name] = (data, R, C, ty)
    return out


def tiny_shapes():
    return {n: (R, C) for n, (R, C, _) in TINY.items()}


@pytest.fixture
def tiny_pack(tmp_path):
    p = tmp_path / "pack"
    pack.write_pack(p, tiny_tensors(), dims=TINY_DIMS)
    return p


def test_written_pack_verifies_and_is_aligned(tiny_pack):
    man = pack.verify_pack(tiny_pack, full=True, dims=TINY_DIMS, shapes=tiny_shapes())
    assert man["pack_format"] == "kindi-q4-v1" and man["head"] == "output.weight"
    index = json.loads((tiny_pack / "index.json").read_text())["tensors"]
    raw = np.fromfile(tiny_pack / "weights.bin", np.uint8)
    for name, (data, R, C, ty) in tiny_tensors().items():
        rec = index[name]
        if ty == 0:
            f = np.fromfile(tiny_pack / "f32.bin", "<f4", count=R * C, offset=rec["f32_off"])
            np.testing.assert_array_equal(f, data.reshape(-1))
        else:
            assert rec["offset"] % pack.PAGE == 0 and rec["padded_bytes"] % pack.PAGE == 0
            np.testing.assert_array_equal(raw[rec["offset"]:rec["offset"] + rec["bytes"]], data)


def _rewrite_index(p, idx):
    """Replace index.json and refresh its manifest record, so only the index content is wrong."""
    f = p / "index.json"
    f.write_text(json.dumps(idx))
    man = json.loads((p / "kindi_pack.json").read_text())
    man["files"]["index.json"] = {"size": f.stat().st_size, "sha256": pack.digest(f)}
    (p / "kindi_pack.json").write_text(json.dumps(man))


def _edit_index(p, name, **kv):
    idx = json.loads((p / "index.json").read_text())
    idx["tensors"][name].update(kv)
    _rewrite_index(p, idx)


@pytest.mark.parametrize("damage,msg", [
    ("flip", "Pack checksum mismatch: weights.bin"),
    ("truncate", "Pack size mismatch: weights.bin"),
    ("format", "Unsupported pack"),
    ("dims", "Unsupported Q4 profile"),
    ("offset", "Invalid packed tensor span"),
    ("bytes", "Invalid packed tensor dimensions"),
    ("f32", "Invalid float tensor span"),
    ("missing", "Missing/extra tensors"),
    ("storage", "Unexpected tensor storage: blk.0.ssm_alpha.weight"),
])
def test_verify_pack_rejects_damage(tiny_pack, damage, msg):
    p = tiny_pack
    if damage == "flip":
        with open(p / "weights.bin", "r+b") as f:
            f.seek(100)
            b = f.read(1)
            f.seek(100)
            f.write(bytes([b[0] ^ 1]))
        pack.verify_pack(p, full=False, dims=TINY_DIMS, shapes=tiny_shapes())   # sizes still agree
    elif damage == "truncate":
        os.truncate(p / "weights.bin", os.path.getsize(p / "weights.bin") - 1)
    elif damage in ("format", "dims"):
        man = json.loads((p / "kindi_pack.json").read_text())
        if damage == "format":
            man["pack_format"] = "kindi-q4-v0"
        else:
            man["dimensions"] = {"layers": 2, "width": 256}
        (p / "kindi_pack.json").write_text(json.dumps(man))
    elif damage == "offset":
        _edit_index(p, "output.weight", offset=4096)
    elif damage == "bytes":
        _edit_index(p, "output.weight", bytes=100)
    elif damage == "f32":
        _edit_index(p, "output_norm.weight", f32_off=2)
    elif damage == "missing":
        idx = json.loads((p / "index.json").read_text())
        del idx["tensors"]["blk.0.ffn_down.weight"]
        _rewrite_index(p, idx)
    elif damage == "storage":
        _edit_index(p, "blk.0.ssm_alpha.weight", type=12)
    with pytest.raises(ValueError, match=msg):
        pack.verify_pack(p, full=True, dims=TINY_DIMS, shapes=tiny_shapes())


def test_profile_table_of_the_9b_model():
    """427 tensors: 3 shared, 8 attention layers of 11 and 24 gated-delta-net layers of 14; the
    float-stored ones are the norms, ssm_a/dt, conv1d and the alpha/beta gates."""
    s = pack.profile_shapes()
    assert len(s) == 3 + 8 * 11 + 24 * 14
    assert s["blk.3.attn_q.weight"] == (8192, 4096) and "blk.3.attn_qkv.weight" not in s
    assert s["blk.0.attn_qkv.weight"] == (8192, 4096) and s["blk.31.ffn_down.weight"] == (4096, 12288)
    assert s["output.weight"] == (248320, 4096)
    floats = [n for n, (r, _) in s.items() if pack._float_storage(n, r)]
    assert len(floats) == 1 + 8 * 4 + 24 * 8
    quant = {n: rc for n, rc in s.items() if not pack._float_storage(n, rc[0])}
    assert all(r % 8 == 0 and c % 256 == 0 for r, c in quant.values())


def test_rejects_manifest_traversal(tiny_pack):
    """A manifest file name with a directory part is refused before any file is opened
    (q4pack.py:92; tests/kindi_q4/test_pack_validation.py's traversal case)."""
    man = json.loads((tiny_pack / "kindi_pack.json").read_text())
    man["files"] = {"../x": {}}
    (tiny_pack / "kindi_pack.json").write_text(json.dumps(man))
    with pytest.raises(ValueError, match="Invalid manifest path"):
        pack.verify_pack(tiny_pack, full=True, dims=TINY_DIMS, shapes=tiny_shapes())


def test_rejects_the_9b_dimensions_changed(tiny_pack):
    """A pack whose manifest dimensions differ from the 9B profile in one field is refused by the
    default profile check before any tensor is read."""
    man = json.loads((tiny_pack / "kindi_pack.json").read_text())
    man["dimensions"] = dict(pack.PROFILE_DIMS, width=5120)
    (tiny_pack / "kindi_pack.json").write_text(json.dumps(man))
    with pytest.raises(ValueError, match="Unsupported Q4 profile"):
        pack.verify_pack(tiny_pack)


@pytest.mark.parametrize("mode,expected", [(None, True), ("full", True), ("size", False)])
def test_verification_mode_is_explicit(monkeypatch, mode, expected):
    if mode is None:
        monkeypatch.delenv("KINDI_Q4_VERIFY", raising=False)
    else:
        monkeypatch.setenv("KINDI_Q4_VERIFY", mode)
    assert pack.verification_full() is expected


def test_verification_mode_typo_is_an_error(monkeypatch, tiny_pack):
    monkeypatch.setenv("KINDI_Q4_VERIFY", "typo")
    with pytest.raises(ValueError, match="KINDI_Q4_VERIFY must be full or size"):
        pack.verification_full()
    with pytest.raises(ValueError, match="KINDI_Q4_VERIFY must be full or size"):
        pack.open_pack(tiny_pack, device="cpu", dims=TINY_DIMS, shapes=tiny_shapes())


def test_open_pack_takes_the_mode_from_the_environment(monkeypatch, tiny_pack):
    """A flipped byte keeps every size: "size" mode opens the pack, "full" mode finds the checksum
    mismatch.  Opening reads no tensor, so this runs without a device."""
    with open(tiny_pack / "weights.bin", "r+b") as f:
        f.seek(100)
        b = f.read(1)
        f.seek(100)
        f.write(bytes([b[0] ^ 1]))
    monkeypatch.setenv("KINDI_Q4_VERIFY", "size")
    w = pack.open_pack(tiny_pack, device="cpu", dims=TINY_DIMS, shapes=tiny_shapes())
    assert "output.weight" in w
    w.close()
    monkeypatch.setenv("KINDI_Q4_VERIFY", "full")
    with pytest.raises(ValueError, match="Pack checksum mismatch: weights.bin"):
        pack.open_pack(tiny_pack, device="cpu", dims=TINY_DIMS, shapes=tiny_shapes())


def test_engine_over_a_pack_sizes_its_workspace_from_the_index(tiny_pack):
    """A PackWeights reads tensors lazily (its cache starts empty), so the Engine takes the widest
    quantized tensor from the pack index: 512 columns (ffn_down) in the tiny pack.  No device
    work: the engine's workspace is a host tensor here."""
    from kq import ops
    from kq.gpu4 import Engine
    w = pack.PackWeights(tiny_pack, device="cpu")
    try:
        assert len(w.cache) == 0
        eng = Engine(w, mode="q8k")
        assert eng.max_cols == 512
        assert eng.chunk == 256 and eng.xq.numel() == 256 * (512 // 256) * 292
        # the GEMM workspace covers any chunk of 1..256 fp32 rows (quantized into it) through up to
        # three matrices of any quantized tensor shape of the pack
        need = max(ops.gemm_f32_multi_workspace_bytes([R] * 3, C, m) for R, C in [(16, 256), (8, 512)]
                   for m in range(1, 257))
        assert need >= max(ops.gemm_workspace_bytes(R, C, m) for R, C in [(16, 256), (8, 512)] for m in range(1, 257))
        assert eng.gemm_ws.numel() == need + 256
        assert eng.logits.numel() == 16 and eng.row.numel() == 512
    finally:
        w.close()


@pytest.mark.parametrize("value,chunk", [(None, 256), ("128", 128), ("0", 0), ("1", 0), ("", 0)])
def test_engine_chunk_follows_kindi_chunk(tiny_pack, monkeypatch, value, chunk):
    """The prefill chunk is KINDI_CHUNK (chunk.py:82,90: default 256; 0, 1 or empty turn chunked
    prefill off); with it off the engine keeps no GEMM workspace.  Host only."""
    from kq.gpu4 import Engine
    if value is None:
        monkeypatch.delenv("KINDI_CHUNK", raising=False)
    else:
        monkeypatch.setenv("KINDI_CHUNK", value)
    w = pack.PackWeights(tiny_pack, device="cpu")
    try:
        eng = Engine(w, mode="q8k")
        assert eng.chunk == chunk
        assert (eng.gemm_ws is None) == (chunk == 0)
        assert eng.max_rows == max(chunk, 16)
    finally:
        w.close()


def test_side_readers_wait_for_the_callers_stream(tiny_pack, monkeypatch):
    """A large tensor is read by several threads, each copying on its own stream.  Before any reader
    starts, those streams are made to wait for the caller's stream: the new device buffer may reuse
    memory freed there (an evicted tensor) that queued kernels still read.  Host only: the streams
    and the reads are stand-ins that record the order of events."""
    import torch
    events = []

    class Stream:
        def __init__(self, name):
            self.name = name

        def wait_stream(self, other):
            events.append(("wait", self.name, other.name))

    caller = Stream("caller")
    monkeypatch.setattr(torch.cuda, "current_stream", lambda device=None: caller)
    monkeypatch.setattr(pack, "PARALLEL_MIN", 0)
    w = pack.PackWeights(tiny_pack, device="cpu")
    try:
        w._stage, w._events = [], []                 # staging set up (not used by the stand-in reads)
        w._streams = [None] + [Stream("s%d" % t) for t in range(1, pack.READERS)]

        def read(t, buf, base, lo, hi):
            events.append(("read", t))
            return hi - lo

        monkeypatch.setattr(w, "_read_range", read)
        buf = w["token_embd.weight"][0]
        assert buf.numel() == 16 * 144
        waits = [e for e in events if e[0] == "wait"]
        assert sorted(waits) == [("wait", "s%d" % t, "caller") for t in range(1, pack.READERS)]
        first_read = min(i for i, e in enumerate(events) if e[0] == "read")
        assert all(i < first_read for i, e in enumerate(events) if e[0] == "wait")
    finally:
        w.close()


@pytest.mark.parametrize("env,limit,pin", [
    ({}, 1 << 62, True),                                                   # unset: unlimited, pinned
    ({"KINDI_Q4_GPU_CACHE_BYTES": "5800000000"}, 5_800_000_000, True),     # the reference's default
    ({"KINDI_Q4_GPU_CACHE_BYTES": "1600000000"}, 1_600_000_000, True),     # pinning starts at 1.6 GB
    ({"KINDI_Q4_GPU_CACHE_BYTES": "1599999999"}, 1_599_999_999, False),
    ({"KINDI_Q4_GPU_CACHE_BYTES": "900000000"}, 900_000_000, False),       # the lower bound
    ({"KINDI_Q4_GPU_CACHE_BYTES": "288000000000"}, 288_000_000_000, True),  # the MI355X's HBM
    ({"KINDI_Q4_GPU_CACHE_BYTES": "5800000000", "KINDI_Q4_PIN_BOUNDARIES": "0"}, 5_800_000_000, False),
    ({"KINDI_Q4_PIN_BOUNDARIES": "yes"}, 1 << 62, False),                  # only "1" pins, as gpu4.py:24
])
def test_cache_config_follows_the_reference_variables(env, limit, pin):
    """KINDI_Q4_GPU_CACHE_BYTES and KINDI_Q4_PIN_BOUNDARIES read as gpu4.Weights reads them
    (gpu4.py:21-24), with the budget's upper bound widened to 288 GB and no budget when unset."""
    assert pack.cache_config(env=env)[:2] == (limit, pin)
    assert pack.cache_config(env=dict(env, KINDI_Q4_STREAM="1"))[2] is True
    assert pack.cache_config(env=env)[2] is False


@pytest.mark.parametrize("value", ["899999999", "288000000001", "0", "-5"])
def test_cache_budget_out_of_range_is_an_error(value):
    with pytest.raises(ValueError, match="GPU tensor cache must be 0.9..288 GB"):
        pack.cache_config(env={"KINDI_Q4_GPU_CACHE_BYTES": value})


def test_cache_arguments_override_the_environment():
    """Explicit arguments win over the variables (tests use budgets below the range); an explicit
    budget still follows the pinning rule unless pinning is given too."""
    env = {"KINDI_Q4_GPU_CACHE_BYTES": "5", "KINDI_Q4_PIN_BOUNDARIES": "1"}
    assert pack.cache_config(limit=60_000_000, env=env)[:2] == (60_000_000, False)
    assert pack.cache_config(limit=60_000_000, pin_boundaries=True, env=env)[:2] == (60_000_000, True)
    assert pack.cache_config(limit=2_000_000_000, env={})[:2] == (2_000_000_000, True)


@pytest.mark.parametrize("pin,evicted", [(True, "blk.0.ffn_gate.weight"), (False, "token_embd.weight")])
def test_eviction_spares_the_boundaries_only_when_pinned(tiny_pack, monkeypatch, pin, evicted):
    """The LRU budget evicts the oldest tensor that is not the embedding or the head when pinning
    is on (gpu4.py:33-35), the oldest of all when it is off.  Host only: the cache holds stand-ins."""
    monkeypatch.setenv("KINDI_Q4_GPU_CACHE_BYTES", "1000000000")
    monkeypatch.setenv("KINDI_Q4_PIN_BOUNDARIES", "1" if pin else "0")
    import torch
    w = pack.PackWeights(tiny_pack, device="cpu")
    try:
        assert w.limit == 1_000_000_000 and w.pin_boundaries is False     # below 1.6 GB: never pinned
        w.pin_boundaries = pin
        w.limit = 300
        for name in ("token_embd.weight", "blk.0.ffn_gate.weight", "output.weight"):
            w.cache[name] = (torch.empty(100, dtype=torch.uint8), 0, 0, 12)
            w.used += 100
        w._evict_for(100)
        assert evicted not in w.cache and len(w.cache) == 2 and w.used == 200
    finally:
        w.close()


def test_engine_gemm_workspace_by_mode_and_groups(tiny_pack):
    """Mode "f32" keeps no GEMM workspace (it prefills row by row); with ``groups`` the workspace
    is sized for the groups gemm will see, three matrices at a time.  Host only."""
    from kq import ops
    from kq.gpu4 import Engine
    w = pack.PackWeights(tiny_pack, device="cpu")
    try:
        assert Engine(w, mode="f32").gemm_ws is None
        for name in ("token_embd.weight", "output.weight", "blk.0.ffn_down.weight"):
            w.cache[name] = (None,) + tuple(int(w.index[name][k]) for k in ("rows", "ne0", "type"))
        g = [["token_embd.weight", "output.weight"], ["blk.0.ffn_down.weight"]]
        eng = Engine(w, mode="q8k", groups=g)
        need = max(max(ops.gemm_f32_multi_workspace_bytes(Rs, C, m) for m in range(1, 257))
                   for Rs, C in [([16, 16], 256), ([8], 512)])
        assert eng.gemm_ws.numel() == need + 256
        with pytest.raises(ValueError, match="share their column count"):
            Engine(w, mode="q8k", groups=[["output.weight", "blk.0.ffn_down.weight"]])
    finally:
        w.close()


def test_engine_built_before_its_weights_rejects_gemm():
    """An Engine over weights that are added after it was built has no GEMM workspace for them:
    gemm says so instead of failing on a null workspace.  Host only (rejected before any launch)."""
    import torch
    from kq.gpu4 import Engine, Weights
    w = Weights("cpu")
    eng = Engine(w, mode="q8k")
    w.add("m", np.zeros(16 * 144, np.uint8), 16, 256, 12)
    with pytest.raises(ValueError, match="GEMM workspace"):
        eng.gemm(["m"], torch.zeros(20, 256), [torch.empty(20, 16)])
