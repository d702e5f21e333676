"""Kindi Q4 weight packs on the MI355X: verification, a device tensor cache, and a pack writer.

A pack (scripts/kindi_q4/kindi/q4pack.py) is a directory with
  weights.bin         quantized tensors in the 8-row interleave [R/8][G][8][bs], each starting at a
                      16 KiB boundary and padded to one (q4pack.py:19, 151-160);
  f32.bin             float tensors (norm weights, small gates), little-endian fp32;
  index.json          {"tensors": {name: {rows, ne0, type, offset, bytes, padded_bytes} or
                      {rows, ne0, type: 0, f32_off}}} (q4pack.py:145-160);
  kindi_pack.json     manifest: pack_format "kindi-q4-v1", head, hadamard_block, dimensions,
                      files {name: {size, sha256}} (q4pack.py:163-174).

``verify_pack`` applies the reference's checks (q4pack.py:86-108) in the same order with the same
messages; ``open_pack`` takes its full-or-size mode from KINDI_Q4_VERIFY unless told
(q4pack.py:80-84, gpu4.py:55).  ``PackWeights`` is the device side of gpu4.Weights
(gpu4.py:17-48): ``w[name] -> (buf, R, C, type)`` with ``buf`` a device uint8 tensor in the Kindi
layout, read with 8 MiB preads through two pinned staging buffers whose copies overlap the next
read (large tensors by several reader threads over contiguous ranges), a least-recently used byte
budget that spares the embedding and the head, and POSIX_FADV_DONTNEED after each tensor so the
host page cache does not keep a second copy.  The budget and the pinning rule come from
KINDI_Q4_GPU_CACHE_BYTES / KINDI_Q4_PIN_BOUNDARIES as in gpu4.py:21-24 (``cache_config``); on a
288 GB MI355X the default (unset) budget is unlimited, so the whole 9B pack (5.6 GB) stays resident.  ``write_pack`` builds a pack from tensors already in
the Kindi layout (the converter from GGUF, q4pack.convert, is not part of this path).
"""
import concurrent.futures as cf
import hashlib
import json
import os
from collections import OrderedDict
from pathlib import Path

import numpy as np
import torch

from .formats import BLOCK

PAGE = 16384
PACK_FORMAT = "kindi-q4-v1"
# Dimensions of the one validated profile (q4pack.py:79), the dense Qwen3.5 / OxCoder 9B.
PROFILE_DIMS = {"layers": 32, "width": 4096, "ffn": 12288, "heads": 16, "kv_heads": 4, "head_dim": 256,
                "rope_dim": 64, "groups": 16, "state_size": 128, "gdn_inner": 4096, "rope_base": 10000000.0,
                "full_attention_interval": 4}
PINNED = ("token_embd.weight", "output.weight")
STAGE_BYTES = 8 << 20
READERS = 4              # host threads reading one large tensor (each: two pinned buffers, a stream)
PARALLEL_MIN = 64 << 20  # tensors from this size are read by all READERS
# Device cache budget from KINDI_Q4_GPU_CACHE_BYTES (gpu4.py:21-22).  The reference accepts
# 0.9..5.8 GB for an 8 GB card; here the upper bound is the MI355X's 288 GB of HBM, and with the
# variable unset the budget is unlimited (the reference's default, 5.8 GB, is its card's limit).
CACHE_MIN, CACHE_MAX = 900_000_000, 288_000_000_000
PIN_MIN = 1_600_000_000  # the embedding and head are spared only from this budget up (gpu4.py:24)


def cache_config(limit=None, pin_boundaries=None, env=None):
    """(limit, pin_boundaries, disk_bypass) as gpu4.Weights reads them (gpu4.py:21-24).

    * limit: the argument when given; else KINDI_Q4_GPU_CACHE_BYTES when set, which must lie in
      0.9..288 GB; else unlimited.
    * pin_boundaries: the argument when given; else KINDI_Q4_PIN_BOUNDARIES (default "1") equal to
      "1" and a budget of at least 1.6 GB.
    * disk_bypass: KINDI_Q4_STREAM == "1".  On the device path it changes nothing (the budget alone
      forces eviction), as in the reference's CUDA engine.
    """
    env = os.environ if env is None else env
    if limit is None:
        v = env.get("KINDI_Q4_GPU_CACHE_BYTES")
        if v is None:
            limit = 1 << 62
        else:
            limit = int(v)
            if not CACHE_MIN <= limit <= CACHE_MAX:
                raise ValueError("GPU tensor cache must be 0.9..288 GB")
    limit = int(limit)
    if pin_boundaries is None:
        pin_boundaries = env.get("KINDI_Q4_PIN_BOUNDARIES", "1") == "1" and limit >= PIN_MIN
    return limit, bool(pin_boundaries), env.get("KINDI_Q4_STREAM", "0") == "1"


def profile_shapes(layers=32):
    """name -> (rows, ne0) of the 9B profile (q4pack.py:21-35): every fourth layer (i % 4 == 3) is
    full attention, the others gated delta-net; all layers have the FFN and two norms."""
    shapes = {"output.weight": (248320, 4096), "token_embd.weight": (248320, 4096), "output_norm.weight": (1, 4096)}
    for layer in range(layers):
        p = "blk.%d." % layer
        blk = {"attn_norm.weight": (1, 4096), "post_attention_norm.weight": (1, 4096),
               "ffn_gate.weight": (12288, 4096), "ffn_up.weight": (12288, 4096), "ffn_down.weight": (4096, 12288)}
        if layer % 4 == 3:
            blk.update({"attn_q.weight": (8192, 4096), "attn_k.weight": (1024, 4096), "attn_v.weight": (1024, 4096),
                        "attn_output.weight": (4096, 4096), "attn_q_norm.weight": (1, 256),
                        "attn_k_norm.weight": (1, 256)})
        else:
            blk.update({"attn_qkv.weight": (8192, 4096), "attn_gate.weight": (4096, 4096),
                        "ssm_out.weight": (4096, 4096), "ssm_alpha.weight": (32, 4096), "ssm_beta.weight": (32, 4096),
                        "ssm_a": (1, 32), "ssm_dt.bias": (1, 32), "ssm_conv1d.weight": (8192, 4),
                        "ssm_norm.weight": (1, 128)})
        shapes.update({p + k: v for k, v in blk.items()})
    return shapes


def _float_storage(name, rows):
    return rows == 1 or name.endswith(("ssm_alpha.weight", "ssm_beta.weight", "ssm_conv1d.weight"))


def validate_shapes(index, shapes):
    """q4pack.validate_shapes (q4pack.py:37-44) against the given profile."""
    if set(index) != set(shapes):
        raise ValueError("Missing/extra tensors for dense Qwen3.5 9B")
    for name, (rows, cols) in shapes.items():
        rec = index[name]
        if (rec["rows"], rec["ne0"]) != (rows, cols):
            raise ValueError("Unexpected shape: " + name)
        if (rec["type"] == 0) != _float_storage(name, rows):
            raise ValueError("Unexpected tensor storage: " + name)


def digest(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for b in iter(lambda: f.read(4 << 20), b""):
            h.update(b)
    return h.hexdigest()


def verification_full():
    """The verification mode from KINDI_Q4_VERIFY (q4pack.py:80-84): "full" (the default when it is
    unset) checks sizes and sha256, "size" checks sizes only; any other value is an error rather
    than a silent choice."""
    mode = os.environ.get("KINDI_Q4_VERIFY", "full")
    if mode not in ("full", "size"):
        raise ValueError("KINDI_Q4_VERIFY must be full or size")
    return mode == "full"


def verify_pack(pack, full=True, dims=PROFILE_DIMS, shapes=None):
    """Checks of q4pack.verify_pack (q4pack.py:86-108); returns the manifest.  ``dims`` and
    ``shapes`` default to the 9B profile."""
    pack = Path(pack)
    man = json.loads((pack / "kindi_pack.json").read_text())
    if man["pack_format"] != PACK_FORMAT:
        raise ValueError("Unsupported pack")
    if man.get("dimensions") != dims or man.get("head") != "output.weight" or man.get("hadamard_block") != 1:
        raise ValueError("Unsupported Q4 profile")
    for name, rec in man["files"].items():
        if Path(name).name != name:
            raise ValueError("Invalid manifest path")
        path = pack / name
        if path.stat().st_size != rec["size"]:
            raise ValueError("Pack size mismatch: " + name)
        if full and digest(path) != rec["sha256"]:
            raise ValueError("Pack checksum mismatch: " + name)
    index = json.loads((pack / "index.json").read_text())["tensors"]
    validate_shapes(index, profile_shapes() if shapes is None else shapes)
    for rec in index.values():
        if rec["type"] in BLOCK:
            expected = rec["rows"] * (rec["ne0"] // 256) * BLOCK[rec["type"]]
            if rec["rows"] % 8 or rec["ne0"] % 256 or expected != rec["bytes"]:
                raise ValueError("Invalid packed tensor dimensions")
            if (rec["offset"] < 0 or rec["offset"] % PAGE
                    or rec["padded_bytes"] != (expected + PAGE - 1) // PAGE * PAGE
                    or rec["offset"] + rec["padded_bytes"] > man["files"]["weights.bin"]["size"]):
                raise ValueError("Invalid packed tensor span")
        elif rec["type"] == 0:
            if (rec["f32_off"] < 0 or rec["f32_off"] % 4
                    or rec["f32_off"] + rec["rows"] * rec["ne0"] * 4 > man["files"]["f32.bin"]["size"]):
                raise ValueError("Invalid float tensor span")
        else:
            raise ValueError("Invalid tensor type")
    return man


def write_pack(out, tensors, dims=PROFILE_DIMS, model="synthetic"):
    """Write a pack.  tensors: name -> (data, rows, ne0, type); type 12/14: uint8 bytes already in
    the Kindi layout; type 0: float32 values (rows x ne0).  Quantized tensors go to weights.bin at
    16 KiB boundaries in the given order, floats to f32.bin.  Returns the manifest."""
    out = Path(out)
    out.mkdir(parents=True, exist_ok=False)
    index = {}
    with open(out / "weights.bin", "wb") as wb, open(out / "f32.bin", "wb") as fb:
        for name, (data, rows, ne0, ty) in tensors.items():
            rec = {"rows": int(rows), "ne0": int(ne0), "dims": [int(rows), int(ne0)], "type": int(ty), "folded": False}
            if ty == 0:
                a = np.ascontiguousarray(data, dtype="<f4").reshape(-1)
                if a.size != rows * ne0:
                    raise ValueError("float tensor %s has %d values, %dx%d expected" % (name, a.size, rows, ne0))
                rec["f32_off"] = fb.tell()
                fb.write(a.tobytes())
            else:
                a = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
                nbytes = rows * (ne0 // 256) * BLOCK[ty]
                if a.size != nbytes:
                    raise ValueError("tensor %s has %d bytes, %d expected" % (name, a.size, nbytes))
                rec["offset"] = wb.tell()
                rec["bytes"] = nbytes
                rec["padded_bytes"] = (nbytes + PAGE - 1) // PAGE * PAGE
                wb.write(a.tobytes())
                wb.write(bytes(rec["padded_bytes"] - nbytes))
            index[name] = rec
    (out / "index.json").write_text(json.dumps({"tensors": index}, sort_keys=True))
    man = {"pack_format": PACK_FORMAT, "model": model, "head": "output.weight", "hadamard_block": 1,
           "dimensions": dims, "quantization": "mixed Q4_K/Q6_K; original blocks preserved",
           "layout": "8-row-block-interleave",
           "files": {p.name: {"size": p.stat().st_size, "sha256": digest(p)} for p in sorted(out.iterdir())}}
    (out / "kindi_pack.json").write_text(json.dumps(man, indent=2) + "\n")
    return man


class PackWeights:
    """Device tensor cache over a pack: ``w[name] -> (buf, R, C, type)`` (gpu4.py:25-48)."""

    def __init__(self, pack, index=None, limit=None, device="cuda", pin_boundaries=None):
        self.pack = Path(pack)
        self.device = torch.device(device)
        self.index = index if index is not None else json.loads((self.pack / "index.json").read_text())["tensors"]
        self.fd = os.open(str(self.pack / "weights.bin"), os.O_RDONLY)
        self.cache = OrderedDict()
        self.used = self.read_bytes = self.hits = self.misses = 0
        self.limit, self.pin_boundaries, self.disk_bypass = cache_config(limit, pin_boundaries)
        self._stage = None
        self._pool = None
        self._f32 = {}

    def close(self):
        if self._pool is not None:
            self._pool.shutdown(wait=True)
            self._pool = None
        if self.fd is not None:
            os.close(self.fd)
            self.fd = None

    def __del__(self):
        self.close()

    def __contains__(self, name):
        return name in self.index and self.index[name]["type"] in BLOCK

    def _staging(self):
        """Per reader: two pinned staging buffers, their events and a copy stream (reader 0 copies on
        the caller's stream)."""
        if self._stage is None:
            self._stage = [[torch.empty(STAGE_BYTES, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
                           for _ in range(READERS)]
            self._events = [[torch.cuda.Event(), torch.cuda.Event()] for _ in range(READERS)]
            self._streams = [None] + [torch.cuda.Stream(device=self.device) for _ in range(READERS - 1)]
        return self._stage, self._events

    def _read_range(self, t, buf, base, lo, hi):
        """Bytes [lo, hi) of the tensor at file offset ``base`` into buf, by reader t: 8 MiB preads into
        the reader's two pinned buffers, each copy to the device overlapping the next read."""
        stage, events = self._stage[t], self._events[t]
        stream = self._streams[t] or torch.cuda.current_stream(self.device)
        try:
            with torch.cuda.stream(stream):
                for i, off in enumerate(range(lo, hi, STAGE_BYTES)):
                    n = min(STAGE_BYTES, hi - off)
                    s, ev = stage[i % 2], events[i % 2]
                    ev.synchronize()                           # its previous copy has finished
                    view = memoryview(s.numpy())[:n]
                    if os.preadv(self.fd, [view], base + off) != n:
                        raise IOError("Truncated Q4 weight tensor")
                    buf[off:off + n].copy_(s[:n], non_blocking=True)
                    ev.record(stream)
        finally:
            for ev in events:                                  # no copy outlives the call, even on error
                ev.synchronize()
        return hi - lo

    def _evict_for(self, size):
        protected = set(PINNED) if self.pin_boundaries else set()
        while self.cache and self.used + size > self.limit:
            key = next((k for k in self.cache if k not in protected), next(iter(self.cache)))
            self.used -= self.cache[key][0].numel()
            del self.cache[key]

    def __getitem__(self, name):
        if name in self.cache:
            self.hits += 1
            self.cache.move_to_end(name)
            return self.cache[name]
        self.misses += 1
        rec = self.index[name]
        if rec["type"] not in BLOCK:
            raise ValueError("not a quantized tensor: " + name)
        size = rec["bytes"]
        self._evict_for(size)
        buf = torch.empty(size, dtype=torch.uint8, device=self.device)
        self._staging()
        if size < PARALLEL_MIN or READERS < 2:
            self.read_bytes += self._read_range(0, buf, rec["offset"], 0, size)
        else:
            # READERS contiguous ranges (whole staging chunks), read at once: the copies from the
            # page cache (or the device's queue depth) bound a single reader
            if self._pool is None:
                self._pool = cf.ThreadPoolExecutor(READERS - 1)
            # buf may reuse memory freed on the caller's stream (an evicted tensor) that kernels
            # queued there still read: the readers' own copy streams start after them
            cur = torch.cuda.current_stream(self.device)
            for st in self._streams[1:]:
                st.wait_stream(cur)
            chunks = (size + STAGE_BYTES - 1) // STAGE_BYTES
            cut = [min(size, (chunks * t // READERS) * STAGE_BYTES) for t in range(READERS + 1)]
            futs = [self._pool.submit(self._read_range, t, buf, rec["offset"], cut[t], cut[t + 1])
                    for t in range(1, READERS)]
            try:
                done = self._read_range(0, buf, rec["offset"], cut[0], cut[1])
            finally:
                cf.wait(futs)                                  # every reader has stopped writing into buf
            self.read_bytes += done + sum(f.result() for f in futs)
        os.posix_fadvise(self.fd, rec["offset"], rec["padded_bytes"], os.POSIX_FADV_DONTNEED)
        value = (buf, int(rec["rows"]), int(rec["ne0"]), int(rec["type"]))
        self.cache[name] = value
        self.used += size
        return value

    def f32(self, name):
        """A float tensor of the pack (norm weights, gates) as a device fp32 tensor, kept."""
        if name not in self._f32:
            rec = self.index[name]
            if rec["type"] != 0:
                raise ValueError("not a float tensor: " + name)
            n = rec["rows"] * rec["ne0"]
            a = np.fromfile(self.pack / "f32.bin", dtype="<f4", count=n, offset=rec["f32_off"])
            if a.size != n:
                raise IOError("Truncated float tensor")
            self._f32[name] = torch.from_numpy(a.astype(np.float32)).to(self.device)
        return self._f32[name]


def open_pack(pack, full=None, limit=None, device="cuda", dims=PROFILE_DIMS, shapes=None, pin_boundaries=None):
    """verify_pack, then a PackWeights over the pack (the Engine's weights, gpu4.py:55-59).
    ``full=None`` takes the mode from KINDI_Q4_VERIFY, as the Engine does; ``limit`` and
    ``pin_boundaries`` left None come from the environment (cache_config)."""
    verify_pack(pack, full=verification_full() if full is None else full, dims=dims, shapes=shapes)
    return PackWeights(pack, limit=limit, device=device, pin_boundaries=pin_boundaries)
