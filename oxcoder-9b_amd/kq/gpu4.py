"""MI355X counterpart of the Kindi Q4 GPU operator surface (scripts/kindi_q4/kindi/gpu4.py).

``Weights[name] -> (buf, R, C, type)`` mirrors gpu4.Weights.__getitem__ (gpu4.py:25-48): ``buf``
is a device uint8 tensor in the Kindi 8-row layout, R/C/type int32 as in the pack index.  Here
the tensors are registered in memory (device resident); ``kq.pack.PackWeights`` gives the same
contract over a Kindi pack on disk (verified as q4pack.verify_pack does), and either can back an
Engine.

``Engine.gemv(names, x, outs, parts_ok=False) -> 1`` mirrors gpu4.Engine.gemv (gpu4.py:95-99):
for each name, ``outs[i][:R] = W_name @ x`` on the current stream, asynchronously, returning 1
(the number of column parts, as the reference does).  Two numerics modes:

* ``"f32"`` -- fp32 activations, the reference's numerics (kq_gemv).
* ``"q8k"`` -- the input is quantized once to Q8_K (kq_q8k_quantize) into a preallocated
  workspace, then every named matrix runs the int8 GEMV (kq_gemv_q8k).

``gemv_batch`` (speculative verify, N <= 16 rows) and ``gemm`` (prefill chunk, any M) extend the
same contract to several activation rows: X is [N][C] fp32, each out is [N][R] (row stride
``out.stride(0)``), the batched layout of the ternary engine's k_tc_mv (tc.cu:306-310).

The producers of the GEMV inputs write the Q8_K activation directly: ``rmsfold_q8k`` (the
residual add + RMSNorm of Engine.rmsfold, gpu4.py:104-106 / q4_rms, q4.cu:39-46) and
``swiglu_q8k`` (q4_silu, q4.cu:36-38, as the FFN launches it, engine.py:287); ``gemv_q8`` then
runs the named matrices on that Q8_K input with no further quantization.  ``head`` is the output
head with the greedy pick (Engine.head, engine.py:323-331): the GEMV computes the argmax of the
logits as it stores them (kq_gemv_q8k_argmax).
"""
import torch

from . import ops
from .formats import BLOCK, Q8K_BYTES, QK, check_shape


class Weights:
    def __init__(self, device="cuda"):
        self.device = torch.device(device)
        self.cache = {}

    def add(self, name, packed, R, C, ty):
        """Register a Kindi-layout tensor (numpy uint8 or torch uint8), copied to the device once."""
        check_shape(R, C, ty)
        buf = torch.as_tensor(packed, dtype=torch.uint8).reshape(-1).to(self.device)
        if buf.numel() != R * (C // QK) * {12: 144, 14: 210}[ty]:
            raise ValueError("Invalid packed tensor dimensions for " + name)
        self.cache[name] = (buf, int(R), int(C), int(ty))
        return self.cache[name]

    def __getitem__(self, name):
        return self.cache[name]

    def __contains__(self, name):
        return name in self.cache


def _widest(weights):
    """Most columns of any quantized tensor the weights hold: from the pack index when there is
    one (a PackWeights reads tensors lazily, so its cache starts empty), else from the resident
    tensors."""
    index = getattr(weights, "index", None)
    if index is not None:
        return max([r["ne0"] for r in index.values() if r["type"] in BLOCK] or [QK])
    return max([C for (_, _, C, _) in weights.cache.values()] or [QK])


class Engine:
    def __init__(self, weights, mode="q8k", max_cols=None, max_rows=16):
        if mode not in ("q8k", "f32"):
            raise ValueError("mode must be 'q8k' or 'f32'")
        self.w = weights
        self.mode = mode
        self.device = weights.device
        cols = max_cols or _widest(weights)
        self.max_cols = cols
        self.max_rows = max_rows
        # Q8_K workspace, preallocated like the reference's device scratch (gpu4.py:70-79).
        self.xq = torch.empty(max_rows * (cols // QK) * Q8K_BYTES, dtype=torch.uint8, device=self.device)
        self.gemm_ws = None   # prefill GEMM workspace (activation fragments, K-split partial sums), grown on demand

    def _check_out(self, y, R, N=1):
        need = (N - 1) * (y.stride(0) if y.dim() == 2 else R) + R
        if y.dtype != torch.float32 or y.numel() < need:
            raise ValueError("output buffer too small or not float32")

    def _quantize(self, X, C):
        N = X.shape[0]
        if C > self.max_cols or N > self.max_rows:
            raise ValueError("input %dx%d exceeds the engine workspace %dx%d" % (N, C, self.max_rows, self.max_cols))
        return ops.q8k_quantize(X, self.xq[: N * (C // QK) * Q8K_BYTES].view(N, -1))

    def gemv(self, names, x, outs, parts_ok=False):
        mats = [self.w[n] for n in names]
        if len(outs) < len(mats):
            raise ValueError("one output per matrix")
        C = mats[0][2]
        if any(m[2] != C for m in mats) or x.numel() < C:
            raise ValueError("matrices sharing x must have the same column count")
        for (w, R, _, _), y in zip(mats, outs):
            self._check_out(y, R)
        if self.mode == "f32":
            for (w, R, C_, ty), y in zip(mats, outs):
                ops.gemv(w, R, C_, ty, x, y)
            return 1
        xq = self._quantize(x.reshape(1, -1)[:, :C], C)
        # matrices sharing the input go three at a time into one launch (kcpu4.c:100-118)
        for i in range(0, len(mats), 3):
            ops.gemv_q8k_multi(mats[i:i + 3], xq, 1, list(outs[i:i + 3]))
        return 1

    def gemv_q8(self, names, xq, outs, N=1):
        """gemv on an activation already in Q8_K (from rmsfold_q8k / swiglu_q8k); returns 1."""
        mats = [self.w[n] for n in names]
        if len(outs) < len(mats):
            raise ValueError("one output per matrix")
        C = mats[0][2]
        if any(m[2] != C for m in mats):
            raise ValueError("matrices sharing xq must have the same column count")
        if xq.numel() < N * (C // QK) * Q8K_BYTES:
            raise ValueError("xq holds fewer than %d Q8_K rows of %d" % (N, C))
        for (w, R, _, _), y in zip(mats, outs):
            self._check_out(y, R, N)
        for i in range(0, len(mats), 3):
            ops.gemv_q8k_multi(mats[i:i + 3], xq, N, list(outs[i:i + 3]))
        return 1

    def rmsfold_q8k(self, h, w, residual=None, xn=None):
        """h += residual (when given, in place), then RMSNorm(h) * w written as Q8_K into the engine
        workspace (and to xn when given).  Returns (xn, xq) for gemv_q8.  xq is a view of the engine's
        one Q8_K workspace (like the reference's reused xp scratch, gpu4.py:70-79): the next call that
        quantizes (gemv in "q8k" mode, gemv_batch, gemm, head, rmsfold_q8k, swiglu_q8k) overwrites it."""
        N = 1 if h.dim() == 1 else h.shape[0]
        D = h.shape[-1]
        if D > self.max_cols or N > self.max_rows:
            raise ValueError("input %dx%d exceeds the engine workspace %dx%d" % (N, D, self.max_rows, self.max_cols))
        return ops.rms_q8k(h, w, residual=residual, xn=xn, xq=self.xq[: N * (D // QK) * Q8K_BYTES].view(N, -1))

    def swiglu_q8k(self, gate, up, y=None):
        """silu(gate) * up written as Q8_K into the engine workspace (and to y when given).
        Returns (y, xq) for gemv_q8; xq is valid until the next quantizing call, as for rmsfold_q8k."""
        N = 1 if gate.dim() == 1 else gate.shape[0]
        n = gate.shape[-1]
        if n > self.max_cols or N > self.max_rows:
            raise ValueError("input %dx%d exceeds the engine workspace %dx%d" % (N, n, self.max_rows, self.max_cols))
        return ops.swiglu_q8k(gate, up, y=y, xq=self.xq[: N * (n // QK) * Q8K_BYTES].view(N, -1))

    def head(self, name, x, y=None):
        """Greedy next token: y = W_name x (the logits, kept in ``y`` or the engine's buffer) and the
        index of the largest logit, read back to the host as Engine.head does (engine.py:323-331,
        gemv + k_argmax); the GEMV finds the argmax itself (kq_gemv_q8k_argmax)."""
        w, R, C, ty = self.w[name]
        if self.mode != "q8k":
            raise ValueError("head: the fused greedy pick runs on Q8_K activations (mode 'q8k')")
        if y is None:
            if getattr(self, "logits", None) is None or self.logits.numel() < R:
                self.logits = torch.empty(R, dtype=torch.float32, device=self.device)
            y = self.logits[:R]
        self._check_out(y, R)
        if getattr(self, "argmax_ws", None) is None:
            self.argmax_ws = ops.argmax_workspace(self.device)
            self.argmax_out = torch.empty(1, dtype=torch.int32, device=self.device)
        xq = self._quantize(x.reshape(1, -1)[:, :C], C)
        ops.gemv_q8k_argmax(w, R, C, ty, xq, y, self.argmax_ws, self.argmax_out)
        return int(self.argmax_out.cpu()[0])

    def feed_rows(self, names, X, outs, batch_max=16):
        """Several activation rows through the named matrices, as the engine's batched prompt and
        verify paths need (Runner batching, cache.py:587-600; chunk.feed, chunk.py:378): up to
        ``batch_max`` rows go through the batched GEMV, whose rows are bit-identical to one-token
        decode (so a verified draft continues exactly as decode would), more rows through the
        prefill GEMM."""
        N = X.shape[0]
        if N <= batch_max:
            return self.gemv_batch(names, X, outs)
        return self.gemm(names, X, outs)

    def fingerprint(self):
        """Identity of this engine's arithmetic for a state cache (engine_fingerprint,
        cache.py:55-95): the libkq source hash and the numerics mode."""
        from . import _lib
        return {"libkq": _lib.kq().kq_source_hash().decode(), "mode": self.mode,
                "weights": "kindi-q4-v1: Q4_K/Q6_K row tiles"}

    def gemv_batch(self, names, X, outs):
        """Speculative-verify GEMV: X [N][C], N <= 16; out[n][r] bit-identical to gemv on row n."""
        N, C = X.shape
        if not 1 <= N <= 16:
            raise ValueError("batch of %d rows: 1..16 supported" % N)
        if len(outs) < len(names):
            raise ValueError("one output per matrix")
        xq = self._quantize(X, C)
        for name, y in zip(names, outs):
            w, R, C_, ty = self.w[name]
            if C_ != C:
                raise ValueError("column count mismatch for " + name)
            self._check_out(y, R, N)
            ops.gemv_q8k(w, R, C_, ty, xq, N, y, y.stride(0) if y.dim() == 2 else R)
        return 1

    def gemm(self, names, X, outs):
        """Prefill GEMM over M rows of X [M][C] (M <= max_rows of the engine workspace)."""
        M, C = X.shape
        if len(outs) < len(names):
            raise ValueError("one output per matrix")
        xq = self._quantize(X, C)
        need = max(ops.gemm_workspace_bytes(self.w[name][1], C, M) for name in names) + 256
        if self.gemm_ws is None or self.gemm_ws.numel() < need:
            self.gemm_ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        for name, y in zip(names, outs):
            w, R, C_, ty = self.w[name]
            if C_ != C:
                raise ValueError("column count mismatch for " + name)
            self._check_out(y, R, M)
            ops.gemm_q8k(w, R, C_, ty, xq, M, y, y.stride(0) if y.dim() == 2 else R, ws=self.gemm_ws)
        return 1

    def embed(self, tok, out=None, name="token_embd.weight"):
        """Row ``tok`` of the token embedding, decoded to fp32 (Engine.embed with q4_embed,
        gpu4.py:100-103, q4.cu:28-32; kq_dequant_rows)."""
        w, R, C, ty = self.w[name]
        if not 0 <= tok < R:
            raise ValueError("Invalid token")
        return self.dequant(name, tok, out)

    def dequant(self, name, row, out=None):
        """One decoded row (kc_dequant, kcpu4.c:341; q4_embed, q4.cu:28-32)."""
        w, R, C, ty = self.w[name]
        if not 0 <= row < R:
            raise ValueError("Invalid row")
        return ops.dequant_rows(w, R, C, ty, row, 1, out)[0] if out is None else ops.dequant_rows(w, R, C, ty, row, 1, out)
