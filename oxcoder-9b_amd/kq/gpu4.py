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
* ``"q8k"`` -- the input is quantized to Q8_K and every named matrix runs the int8 GEMV: for up to
  4096 columns inside the GEMV launch itself (kq_gemv_q8k_x, one launch per three matrices), beyond
  that once (kq_q8k_quantize) into a preallocated workspace, then kq_gemv_q8k_multi; the same bits
  either way.

``gemv_batch`` (speculative verify, N <= 16 rows) and ``gemm`` (prefill chunk, any M) extend the
same contract to several activation rows: X is [N][C] fp32, each out is [N][R] (row stride
``out.stride(0)``), the batched layout of the ternary engine's k_tc_mv (tc.cu:306-310).  In
``"q8k"`` mode they run the batched Q8_K GEMV and the prefill GEMM; in ``"f32"`` mode every row goes
through the fp32 GEMV as one decode step would (the reference's Q4 engine prefills token by token,
gpu4.py:109-110), so each output row equals ``gemv`` on that row bit for bit.

The producers of the GEMV inputs write the Q8_K activation directly: ``rmsfold_q8k`` (the
residual add + RMSNorm of Engine.rmsfold, gpu4.py:104-106 / q4_rms, q4.cu:39-46) and
``swiglu_q8k`` (q4_silu, q4.cu:36-38, as the FFN launches it, engine.py:287); ``gemv_q8`` then
runs the named matrices on that Q8_K input with no further quantization.  ``head`` is the output
head with the greedy pick (Engine.head, engine.py:323-331): in ``"q8k"`` mode the GEMV computes the
argmax of the logits as it stores them (kq_gemv_q8k_argmax); in ``"f32"`` mode the fp32 GEMV and
then the argmax over the logits (kq_gemv, kq_argmax), the reference's gemv([head]) + k_argmax.
"""
import os

import torch

from . import ops
from ._lib import KQ_MAX_BATCH
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


def _tensor_shapes(weights):
    """(R, C) of every quantized tensor the weights hold: from the pack index when there is one (a
    PackWeights reads tensors lazily, so its cache starts empty), else from the resident tensors."""
    index = getattr(weights, "index", None)
    if index is not None:
        return sorted({(int(r["rows"]), int(r["ne0"])) for r in index.values() if r["type"] in BLOCK})
    return sorted({(R, C) for (_, R, C, _) in weights.cache.values()})


def chunk_from_env():
    """Tokens per prefill GEMM call, KINDI_CHUNK as the reference's chunked prefill reads it
    (chunk.py:82,90: default 256; "0", "" or "1" turn chunked prefill off, and prompts then go
    through the batched GEMV, 16 rows at a time)."""
    v = os.environ.get("KINDI_CHUNK", "256")
    if v in ("0", "", "1"):
        return 0
    n = int(v)
    if n < 2:
        raise ValueError("KINDI_CHUNK must be a positive token count")
    return n


class Engine:
    """Every buffer a call uses is allocated here, as the reference engine preallocates its device
    scratch (gpu4.py:70-79): the Q8_K activations of up to max(chunk, 16) rows, the prefill GEMM
    workspace (mode "q8k") for any chunk of up to ``chunk`` rows of any of the weights' matrices
    (or of the listed ``groups``), the argmax workspace and the logits (as many as the tallest
    matrix has rows).  No call allocates device
    memory, so any call can be captured into a HIP graph, the first one included."""

    def __init__(self, weights, mode="q8k", max_cols=None, chunk=None, batch_max=KQ_MAX_BATCH, groups=None):
        if mode not in ("q8k", "f32"):
            raise ValueError("mode must be 'q8k' or 'f32'")
        if not 1 <= batch_max <= KQ_MAX_BATCH:
            raise ValueError("batch_max must be 1..%d" % KQ_MAX_BATCH)
        self.w = weights
        self.mode = mode
        self.device = weights.device
        shapes = _tensor_shapes(weights)
        cols = max_cols or max([C for _, C in shapes] or [QK])
        self.max_cols = cols
        self.chunk = chunk_from_env() if chunk is None else int(chunk)
        if self.chunk < 0 or self.chunk == 1:
            raise ValueError("chunk must be 0 (no prefill GEMM) or at least 2 tokens")
        self.batch_max = batch_max
        self.max_rows = max(self.chunk, KQ_MAX_BATCH)
        dev = self.device
        # Q8_K workspace (the reference's reused xp scratch, gpu4.py:70-79)
        self.xq = torch.empty(self.max_rows * (cols // QK) * Q8K_BYTES, dtype=torch.uint8, device=dev)
        # prefill GEMM workspace (mode "q8k" only: "f32" prefills row by row): the most any chunk
        # (1..chunk rows) of the matrix groups gemm will see needs.  With ``groups`` (lists of names
        # that share an input, e.g. [q, k, v], [gate, up]) it is sized for those, three at a time as
        # gemm sends them; without, for any three matrices of one shape (which bounds every mix).
        self.gemm_ws = None
        if self.chunk and mode == "q8k":
            if groups is not None:
                sets = []
                for g in groups:
                    Rs = [self.w[n][1] for n in g]
                    Cs = {self.w[n][2] for n in g}
                    if len(Cs) != 1:
                        raise ValueError("matrices of a group must share their column count")
                    sets += [(Rs[i:i + 3], Cs.pop()) for i in range(0, len(Rs), 3)]
            else:
                sets = [([R, R, R], C) for R, C in shapes if C <= cols]
            need = max([self._gemm_need(Rs, C, self.chunk) for Rs, C in sets] or [0])
            if need:
                self.gemm_ws = torch.empty(need + 256, dtype=torch.uint8, device=dev)
        self.argmax_ws = ops.argmax_workspace(dev)
        self.argmax_out = torch.empty(1, dtype=torch.int32, device=dev)
        self.logits = torch.empty(max([R for R, _ in shapes] or [1]), dtype=torch.float32, device=dev)
        self.row = torch.empty(cols, dtype=torch.float32, device=dev)     # embed / dequant output

    @staticmethod
    def _gemm_need(Rs, C, chunk):
        """Workspace bytes of the largest of the chunks 1..chunk rows of one group (the K split, and
        so the partial planes, depend on the chunk's row count)."""
        return max(ops.gemm_f32_multi_workspace_bytes(Rs, C, m) for m in range(1, chunk + 1))

    def _check_out(self, y, R, N=1):
        need = (N - 1) * (y.stride(0) if y.dim() == 2 else R) + R
        if y.dtype != torch.float32 or y.numel() < need:
            raise ValueError("output buffer too small or not float32")

    def _quantize(self, X, C):
        N = X.shape[0]
        if C > self.max_cols or N > self.max_rows:
            raise ValueError("input %dx%d exceeds the engine workspace %dx%d" % (N, C, self.max_rows, self.max_cols))
        return ops.q8k_quantize(X, self.xq[: N * (C // QK) * Q8K_BYTES].view(N, -1))

    def _mats(self, names, outs):
        """The named matrices and one output each (extra outputs are ignored, as zip does in the
        reference's gemv, gpu4.py:96)."""
        mats = [self.w[n] for n in names]
        if len(outs) < len(mats):
            raise ValueError("one output per matrix")
        return mats, list(outs)[:len(mats)]

    def gemv(self, names, x, outs, parts_ok=False):
        mats, outs = self._mats(names, outs)
        C = mats[0][2]
        if any(m[2] != C for m in mats) or x.numel() < C:
            raise ValueError("matrices sharing x must have the same column count")
        for (w, R, _, _), y in zip(mats, outs):
            self._check_out(y, R)
        if self.mode == "f32":
            # matrices sharing the input go three at a time into one launch per type (kcpu4.c:100-118)
            for i in range(0, len(mats), 3):
                ops.gemv_multi(mats[i:i + 3], x, outs[i:i + 3])
            return 1
        if C <= 4096 and x.is_contiguous() and x.data_ptr() % 16 == 0:
            # one column pass: each launch quantizes x itself (kq_gemv_q8k_x, the quantizer's bytes),
            # matrices sharing the input three at a time (kcpu4.c:100-118)
            for i in range(0, len(mats), 3):
                ops.gemv_q8k_x(mats[i:i + 3], x.reshape(-1), outs[i:i + 3])
            return 1
        xq = self._quantize(x.reshape(1, -1)[:, :C], C)
        # matrices sharing the input go three at a time into one launch (kcpu4.c:100-118)
        for i in range(0, len(mats), 3):
            ops.gemv_q8k_multi(mats[i:i + 3], xq, 1, outs[i:i + 3])
        return 1

    def gemv_q8(self, names, xq, outs, N=1):
        """gemv on an activation already in Q8_K (from rmsfold_q8k / swiglu_q8k); returns 1."""
        mats, outs = self._mats(names, outs)
        C = mats[0][2]
        if any(m[2] != C for m in mats):
            raise ValueError("matrices sharing xq must have the same column count")
        if xq.numel() < N * (C // QK) * Q8K_BYTES:
            raise ValueError("xq holds fewer than %d Q8_K rows of %d" % (N, C))
        for (w, R, _, _), y in zip(mats, outs):
            self._check_out(y, R, N)
        for i in range(0, len(mats), 3):
            ops.gemv_q8k_multi(mats[i:i + 3], xq, N, outs[i:i + 3])
        return 1

    def rmsfold_q8k(self, h, w, residual=None, xn=None):
        """h += residual (when given, in place), then RMSNorm(h) * w written as Q8_K into the engine
        workspace (and to xn when given).  Returns (xn, xq) for gemv_q8.  xq is a view of the engine's
        one Q8_K workspace (like the reference's reused xp scratch, gpu4.py:70-79): the next call that
        quantizes (gemv in "q8k" mode, gemv_batch, feed_rows, head, rmsfold_q8k, swiglu_q8k)
        overwrites it."""
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
        """Greedy next token: y = W_name x (the logits, kept in ``y`` or the engine's preallocated
        buffer) and the index of the largest logit, read back to the host as Engine.head does
        (engine.py:323-331).  Mode "f32" runs the reference's own sequence: the fp32-activation GEMV,
        then the argmax over the logits (gemv([head]) + k_argmax, engine.py:326-328; kq_gemv then
        kq_argmax).  Mode "q8k" quantizes x and the GEMV finds the argmax itself as it stores the
        logits (kq_gemv_q8k_argmax)."""
        w, R, C, ty = self.w[name]
        if y is None:
            if self.logits.numel() < R:
                raise ValueError("head: %d logits, the engine holds %d" % (R, self.logits.numel()))
            y = self.logits[:R]
        self._check_out(y, R)
        if x.numel() < C:
            raise ValueError("head: x holds %d values, the matrix has %d columns" % (x.numel(), C))
        if self.mode == "f32":
            ops.gemv(w, R, C, ty, x.reshape(-1), y)
            ops.argmax(y.reshape(-1)[:R], self.argmax_ws, self.argmax_out)
        else:
            xq = self._quantize(x.reshape(1, -1)[:, :C], C)
            ops.gemv_q8k_argmax(w, R, C, ty, xq, y, self.argmax_ws, self.argmax_out)
        return int(self.argmax_out.cpu()[0])

    def feed_rows(self, names, X, outs, batch_max=None):
        """Several activation rows through the named matrices, as the engine's batched prompt and
        verify paths need (Runner batching up to batch_max rows, cache.py:587-600; chunked prefill,
        chunk.py:165-177,378): up to ``batch_max`` rows (16 by default) go through the batched GEMV,
        whose rows are bit-identical to one-token decode (a verified draft continues exactly as
        decode would); more rows through the prefill GEMM in chunks of ``chunk`` tokens, or, with
        chunked prefill off (chunk 0), through the batched GEMV 16 rows at a time."""
        N = X.shape[0]
        bm = self.batch_max if batch_max is None else batch_max
        if N <= bm:
            return self.gemv_batch(names, X, outs)
        if not self.chunk:
            mats, outs = self._mats(names, outs)
            for (_, R, _, _), y in zip(mats, outs):
                self._check_out(y, R, N)
            for n0 in range(0, N, KQ_MAX_BATCH):
                n1 = min(N, n0 + KQ_MAX_BATCH)
                # a 2-D output is sliced by rows; a flat one holds rows of R
                views = [y[n0:n1] if y.dim() == 2 else y[n0 * R:n1 * R] for (_, R, _, _), y in zip(mats, outs)]
                self.gemv_batch(names, X[n0:n1], views)
            return 1
        return self.gemm(names, X, outs)

    def fingerprint(self):
        """Identity of this engine's arithmetic for a state cache (engine_fingerprint,
        cache.py:55-95): the libkq source hash and the numerics mode."""
        from . import _lib
        return {"libkq": _lib.kq().kq_source_hash().decode(), "mode": self.mode,
                "weights": "kindi-q4-v1: Q4_K/Q6_K row tiles"}

    def _rows_f32(self, mats, X, outs):
        """Mode "f32": every row of X through the fp32 GEMV (kq_gemv_multi), three matrices a launch."""
        for n in range(X.shape[0]):
            ys = [y[n] if y.dim() == 2 else y[n * R:(n + 1) * R] for (_, R, _, _), y in zip(mats, outs)]
            for i in range(0, len(mats), 3):
                ops.gemv_multi(mats[i:i + 3], X[n], ys[i:i + 3])
        return 1

    def gemv_batch(self, names, X, outs):
        """Speculative-verify GEMV: X [N][C], N <= 16; out[n][r] bit-identical to gemv on row n."""
        N, C = X.shape
        if not 1 <= N <= KQ_MAX_BATCH:
            raise ValueError("batch of %d rows: 1..%d supported" % (N, KQ_MAX_BATCH))
        mats, outs = self._mats(names, outs)
        for (w, R, C_, ty), y in zip(mats, outs):
            if C_ != C:
                raise ValueError("column count mismatch")
            self._check_out(y, R, N)
        if self.mode == "f32":
            return self._rows_f32(mats, X, outs)
        xq = self._quantize(X, C)
        for (w, R, C_, ty), y in zip(mats, outs):
            ops.gemv_q8k(w, R, C_, ty, xq, N, y, y.stride(0) if y.dim() == 2 else R)
        return 1

    def gemm(self, names, X, outs):
        """Prefill GEMM over any number M of rows of X [M][C], in chunks of ``chunk`` tokens as the
        reference's chunked prefill feeds them (chunk.py:165-177,378): the named matrices go three at
        a time through kq_gemm_f32_multi, which quantizes the chunk once into the engine's GEMM
        workspace (Q8_K rows and the GEMM's fragment copy in one launch) and runs one GEMM launch per
        weight type.  Chunk results equal kq_q8k_quantize then one kq_gemm_q8k_ws call per matrix on
        that chunk, bit for bit.  In "f32" mode every row goes through the fp32 GEMV instead, as in
        gemv_batch.  Allocates nothing."""
        M, C = X.shape
        if not self.chunk:
            raise ValueError("chunked prefill is off (chunk 0): use feed_rows or gemv_batch")
        mats, outs = self._mats(names, outs)
        for (w, R, C_, ty), y in zip(mats, outs):
            if C_ != C:
                raise ValueError("column count mismatch")
            self._check_out(y, R, M)
        if self.mode == "f32":
            return self._rows_f32(mats, X, outs)
        if C > self.max_cols:
            raise ValueError("input of %d columns exceeds the engine workspace (%d)" % (C, self.max_cols))
        have = 0 if self.gemm_ws is None else self.gemm_ws.numel() - 256
        for i in range(0, len(mats), 3):
            need = max(ops.gemm_f32_multi_workspace_bytes([m[1] for m in mats[i:i + 3]], C, mc)
                       for mc in {min(self.chunk, M), M - (M - 1) // self.chunk * self.chunk})
            if need > have:
                raise ValueError("gemm: this call needs %d bytes of GEMM workspace, the engine holds %d (build the "
                                 "Engine after its weights are added, or list this group in groups=)" % (need, have))
        for m0 in range(0, M, self.chunk):
            mc = min(self.chunk, M - m0)
            # a flat output holds rows of R
            views = [y[m0:m0 + mc] if y.dim() == 2 else y[m0 * R:] for (_, R, _, _), y in zip(mats, outs)]
            for i in range(0, len(mats), 3):
                ops.gemm_f32_multi(mats[i:i + 3], X[m0:m0 + mc], views[i:i + 3], self.gemm_ws)
        return 1

    def embed(self, tok, out=None, name="token_embd.weight"):
        """Row ``tok`` of the token embedding, decoded to fp32 (Engine.embed with q4_embed,
        gpu4.py:100-103, q4.cu:28-32; kq_dequant_rows)."""
        w, R, C, ty = self.w[name]
        if not 0 <= tok < R:
            raise ValueError("Invalid token")
        return self.dequant(name, tok, out)

    def dequant(self, name, row, out=None):
        """One decoded row (kc_dequant, kcpu4.c:341; q4_embed, q4.cu:28-32) into ``out`` or the
        engine's preallocated row buffer (the reference decodes the embedding into its h scratch,
        gpu4.py:100-103), which the next embed/dequant call overwrites."""
        w, R, C, ty = self.w[name]
        if not 0 <= row < R:
            raise ValueError("Invalid row")
        if out is None:
            if C > self.row.numel():
                raise ValueError("row of %d values, the engine holds %d" % (C, self.row.numel()))
            out = self.row[:C]
        ops.dequant_rows(w, R, C, ty, row, 1, out)
        return out
