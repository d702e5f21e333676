"""Host-side pieces: the C ABI library loads and exports what include/*.h declares (no GPU
compute), the synthetic quantizer, the Kindi repack, and argument validation paths."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT


def _declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kq_\w+)\s*\(", text)))


@pytest.mark.parametrize("header,lib", [("kq.h", "libkq.so"), ("kq_host.h", "libkqhost.so")])
def test_library_exports_every_declared_symbol(header, lib):
    from kq import _lib
    path = os.path.join(ROOT, "oxcoder-9b_amd", "kq", lib)
    assert os.path.exists(path), "build the package first"
    so = ctypes.CDLL(path)
    names = _declared(header)
    assert names, header
    for n in names:
        assert hasattr(so, n), n
    table = _lib.KQ_SYMBOLS if lib == "libkq.so" else _lib.KQHOST_SYMBOLS
    assert sorted(table) == names


def test_error_text_and_version_without_gpu():
    """Entry points that touch no device work on a host without a GPU."""
    from kq import _lib
    lib = _lib.kq()
    assert lib.kq_version() >> 16 == 1
    assert lib.kq_last_error() == b""


@pytest.mark.parametrize("args,msg", [
    ((None, 16, 512, 12), "w is NULL"),
    ((16, 12, 512, 12), "R=12"),
    ((16, 16, 500, 12), "C=500"),
    ((16, 16, 512, 13), "type 13"),
    ((8, 16, 512, 12), "16-byte aligned"),
])
def test_argument_errors_raise_before_launch(args, msg):
    """Bad shapes return KQ_ERR_ARG with a message and launch nothing (host-only path)."""
    from kq import _lib
    lib = _lib.kq()
    w, R, C, ty = args
    rc = lib.kq_gemv_q8k(ctypes.c_void_p(w), R, C, ty, ctypes.c_void_p(64), 1, ctypes.c_void_p(64), R, None)
    assert rc == _lib.KQ_ERR_ARG
    assert msg in lib.kq_last_error().decode()
    with pytest.raises(ValueError, match=re.escape(msg)):
        _lib.check(rc)


def test_batch_limit():
    from kq import _lib
    lib = _lib.kq()
    rc = lib.kq_gemv_q8k(ctypes.c_void_p(256), 16, 512, 12, ctypes.c_void_p(64), 17, ctypes.c_void_p(64), 16, None)
    assert rc == _lib.KQ_ERR_ARG and "N=17" in lib.kq_last_error().decode()


@pytest.mark.parametrize("ty", [12, 14])
def test_tile_round_trip_and_addressing(ty):
    from kq import formats, quantize as kqq
    R, C = 24, 768
    rng = np.random.default_rng(ty)
    raw = rng.integers(0, 256, R * (C // 256) * formats.BLOCK[ty], dtype=np.uint8)
    t_np = formats.tile(raw, R, C, ty)
    t_nat = kqq.tile(raw, R, C, ty)
    np.testing.assert_array_equal(t_np, t_nat)
    np.testing.assert_array_equal(formats.untile(t_np, R, C, ty), raw)
    np.testing.assert_array_equal(kqq.untile(t_nat, R, C, ty), raw)
    bs = formats.BLOCK[ty]
    G = C // 256
    for r, g in [(0, 0), (7, 2), (8, 1), (23, 2)]:
        off = formats.block_offset(R, C, ty, r, g)
        np.testing.assert_array_equal(t_np[off:off + bs], raw[(r * G + g) * bs:(r * G + g + 1) * bs])


def test_shape_validation():
    from kq import formats
    for R, C, ty in [(12, 512, 12), (16, 500, 12), (16, 512, 0), (0, 512, 14)]:
        with pytest.raises(ValueError):
            formats.check_shape(R, C, ty)


@pytest.mark.parametrize("ty", [12, 14])
def test_quantizer_round_trip(orc, ty):
    """Quantize N(0, 0.02) weights and decode with the oracle: per-weight error within the
    quantization step of its sub-block, and small RMS error."""
    from kq import quantize as kqq
    R, C = 64, 2048
    w = kqq.synthetic_fp32(R, C, seed=3)
    W = kqq.tile(kqq.quantize(w, ty), R, C, ty)
    deq = orc.dequant(W, R, C, ty)
    err = np.abs(deq - w)
    rms = np.sqrt(np.mean(err ** 2)) / 0.02
    assert rms < (0.12 if ty == 12 else 0.03), rms
    # step bound: Q4_K step = range/15 of a 32-block (<= 2*max|x|/15); Q6_K step = max|x|/31
    blocks = w.reshape(R, -1, 32 if ty == 12 else 16)
    amax = np.abs(blocks).max(-1, keepdims=True)
    step = 2 * amax / 15 if ty == 12 else amax / 31
    bound = np.broadcast_to(step, blocks.shape).reshape(R, C)
    assert np.all(err <= 1.1 * bound + 1e-6)


def test_quantizer_zero_and_constant_blocks(orc):
    from kq import quantize as kqq
    w = np.zeros((8, 512), np.float32)
    w[1] = 0.5
    w[2, :256] = -0.25
    for ty in (12, 14):
        W = kqq.tile(kqq.quantize(w, ty), 8, 512, ty)
        deq = orc.dequant(W, 8, 512, ty)
        np.testing.assert_allclose(deq, w, atol=0.5 / 31)
        assert not deq[0].any() and not deq[3:].any()


def test_producer_argument_errors():
    """kq_rms_q8k / kq_swiglu_q8k validate shapes and pointers before any launch."""
    from kq import _lib
    lib = _lib.kq()
    p = ctypes.c_void_p(256)
    rc = lib.kq_rms_q8k(p, None, 0, p, 300, 1, 300, None, p, None)
    assert rc == _lib.KQ_ERR_ARG and "D=300" in lib.kq_last_error().decode()
    rc = lib.kq_rms_q8k(p, None, 1, p, 256, 1, 256, None, p, None)
    assert rc == _lib.KQ_ERR_ARG and "residual is NULL" in lib.kq_last_error().decode()
    rc = lib.kq_rms_q8k(p, None, 0, p, 512, 1, 256, None, p, None)
    assert rc == _lib.KQ_ERR_ARG and "ld=256" in lib.kq_last_error().decode()
    rc = lib.kq_swiglu_q8k(p, p, 256, 0, 256, None, p, None)
    assert rc == _lib.KQ_ERR_ARG and "N=0" in lib.kq_last_error().decode()
    rc = lib.kq_swiglu_q8k(p, None, 256, 1, 256, None, p, None)
    assert rc == _lib.KQ_ERR_ARG and "up is NULL" in lib.kq_last_error().decode()


def test_source_hash_is_the_built_sources():
    """kq_source_hash names the sources the loaded library was built from."""
    import importlib.util
    from kq import _lib
    spec = importlib.util.spec_from_file_location("kq_build", os.path.join(ROOT, "oxcoder-9b_amd", "build.py"))
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    h = _lib.kq().kq_source_hash().decode()
    assert len(h) == 16 and h == b.source_hash()


def _split_rule(R, C, M):
    """The K-split rule kq_gemm_q8k_ws documents: tiles of 64 rows x 128 tokens; S = floor(512 /
    tiles), at most 8 and at most G/4; a 2- or 3-way split only when G >= 32."""
    G = C // 256
    tiles = -(-R // 64) * -(-M // 128)
    S = 1
    if tiles < 512:
        want = 512 // tiles
        if want < 4 and G < 32:
            want = 1
        S = max(1, min(want, 8, G // 4))
    gps = -(-G // S)
    return -(-G // gps)


def test_gemm_workspace_follows_the_split_rule():
    """kq_gemm_q8k_workspace (host only, no GPU): fragment bytes (M rounded up to 256 rows of C
    bytes, 256-byte aligned) plus S * M * R * 4 when K is split; 0 for invalid sizes."""
    from kq import _lib
    lib = _lib.kq()
    rng = np.random.default_rng(3)
    shapes = [(12288, 4096, 512), (4096, 12288, 512), (4096, 12288, 64), (4096, 4096, 64), (1024, 4096, 1),
              (12288, 4096, 2048), (8, 256, 1), (136, 256, 300), (2048, 4352, 130), (151936, 4096, 16)]
    shapes += [(8 * int(rng.integers(1, 3000)), 256 * int(rng.integers(1, 60)), int(rng.integers(1, 4000)))
               for _ in range(300)]
    for R, C, M in shapes:
        S = _split_rule(R, C, M)
        frag = -(-M // 256) * 256 * C
        want = -(-frag // 256) * 256 + (S * M * R * 4 if S > 1 else 0)
        assert lib.kq_gemm_q8k_workspace(R, C, M) == want, (R, C, M, S)
    for R, C, M in [(0, 4096, 8), (12, 4096, 8), (64, 0, 8), (64, 300, 8), (64, 4096, 0)]:
        assert lib.kq_gemm_q8k_workspace(R, C, M) == 0, (R, C, M)


def test_grouped_gemm_workspace_and_argument_checks():
    """kq_gemm_q8k_multi_workspace / kq_gemm_f32_multi_workspace (host only): the fragment copy once
    plus each matrix's own partial planes (the f32 form adds the chunk's Q8_K rows, 256-byte
    aligned, in front); invalid sizes give 0; bad calls return KQ_ERR_ARG before any launch."""
    from kq import _lib
    lib = _lib.kq()
    I3 = ctypes.c_int * 3
    for Rs, C, M in [((4096, 1024, 1024), 4096, 256), ((12288, 12288, 12288), 4096, 300),
                     ((4096, 8, 136), 12288, 130), ((2048, 2048, 2048), 2048, 2048)]:
        frag = -(-(-(-M // 256) * 256 * C) // 256) * 256
        want = frag + sum(lib.kq_gemm_q8k_workspace(R, C, M) - frag for R in Rs)
        assert lib.kq_gemm_q8k_multi_workspace(3, I3(*Rs), C, M) == want
        q8k = -(-M * (C // 256) * 292 // 256) * 256
        assert lib.kq_gemm_f32_multi_workspace(3, I3(*Rs), C, M) == q8k + want
        assert lib.kq_gemm_q8k_multi_workspace(1, I3(*Rs), C, M) == lib.kq_gemm_q8k_workspace(Rs[0], C, M)
    for n, Rs, C, M in [(0, (8, 8, 8), 256, 1), (4, (8, 8, 8), 256, 1), (2, (8, 12, 8), 256, 1),
                        (1, (8, 8, 8), 300, 1), (1, (8, 8, 8), 256, 0)]:
        assert lib.kq_gemm_q8k_multi_workspace(n, I3(*Rs), C, M) == 0
        assert lib.kq_gemm_f32_multi_workspace(n, I3(*Rs), C, M) == 0
    P = ctypes.c_void_p * 3
    L = ctypes.c_int64 * 3
    w, y = P(4096, 4096, 4096), P(4096, 4096, 4096)
    R, T, ld = I3(64, 64, 64), I3(12, 14, 12), L(64, 64, 64)
    cases = [
        (lambda: lib.kq_gemm_q8k_multi_ws(4, w, R, 256, T, ctypes.c_void_p(4096), 8, y, ld, ctypes.c_void_p(4096),
                                          1 << 20, None), "n=4"),
        (lambda: lib.kq_gemm_q8k_multi_ws(2, None, R, 256, T, ctypes.c_void_p(4096), 8, y, ld,
                                          ctypes.c_void_p(4096), 1 << 20, None), "NULL array"),
        (lambda: lib.kq_gemm_q8k_multi_ws(3, w, R, 256, I3(12, 13, 12), ctypes.c_void_p(4096), 8, y, ld,
                                          ctypes.c_void_p(4096), 1 << 20, None), "type 13"),
        (lambda: lib.kq_gemm_q8k_multi_ws(3, w, R, 256, T, ctypes.c_void_p(4096), 8, y, ld, ctypes.c_void_p(4100),
                                          1 << 20, None), "256-byte aligned"),
        (lambda: lib.kq_gemm_q8k_multi_ws(3, w, R, 256, T, ctypes.c_void_p(4096), 8, y, ld, ctypes.c_void_p(4096),
                                          16, None), "workspace of 16 bytes"),
        (lambda: lib.kq_gemm_f32_multi(3, w, R, 256, T, ctypes.c_void_p(4096), 100, 8, y, ld, ctypes.c_void_p(4096),
                                       1 << 20, None), "ldx=100"),
        (lambda: lib.kq_gemm_f32_multi(3, w, R, 256, T, None, 256, 8, y, ld, ctypes.c_void_p(4096), 1 << 20, None),
         "x is NULL"),
        (lambda: lib.kq_gemm_f32_multi(3, w, R, 256, T, ctypes.c_void_p(4096), 256, 8, y, L(64, 8, 64),
                                       ctypes.c_void_p(4096), 1 << 20, None), "ldy=8"),
    ]
    for call, msg in cases:
        assert call() == _lib.KQ_ERR_ARG, msg
        assert msg in lib.kq_last_error().decode(), (msg, lib.kq_last_error())


def test_static_gemm_limit_checked_on_the_host():
    """kq_gemm_q8k_static rejects a GEMM whose workspace exceeds its static array before touching a
    device (host only); a 256-token chunk of every 9B-model matrix fits the array."""
    from kq import _lib
    lib = _lib.kq()
    m = re.search(r"#define KQ_GEMM_STATIC_SCRATCH_BYTES \((\d+)u << (\d+)\)",
                  open(os.path.join(ROOT, "include", "kq.h")).read())
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.KQ_GEMM_STATIC_SCRATCH_BYTES
    for R, C in [(4096, 4096), (1024, 4096), (12288, 4096), (4096, 12288), (8192, 4096)]:
        assert lib.kq_gemm_q8k_workspace(R, C, 256) <= _lib.KQ_GEMM_STATIC_SCRATCH_BYTES, (R, C)
    R, C, M = 4096, 12288, 4096
    assert lib.kq_gemm_q8k_workspace(R, C, M) > _lib.KQ_GEMM_STATIC_SCRATCH_BYTES
    p = ctypes.c_void_p(4096)
    rc = lib.kq_gemm_q8k_static(p, R, C, 14, p, M, p, R, None)
    assert rc == _lib.KQ_ERR_ARG
    assert "static scratch" in lib.kq_last_error().decode()


def test_missing_library_raises(monkeypatch):
    """No fallback: without the built library every entry point raises."""
    from kq import _lib, ops
    monkeypatch.setattr(_lib, "LIBKQ", "/nonexistent/libkq.so")
    with pytest.raises(RuntimeError, match="not built"):
        _lib.kq()
    with pytest.raises(RuntimeError, match="not built"):
        ops.gemm_workspace_bytes(4096, 4096, 512)


@pytest.mark.parametrize("args,code,text", [
    (["--gpus", "2"], 2, "measures one GPU"),
    (["--gpus", "8"], 2, "measures one GPU"),
    (["--steps", "0"], 2, "--steps and --copies must be positive"),
    (["--warmup", "-1"], 2, "--warmup not negative"),
])
def test_bench_refuses_what_it_does_not_measure(args, code, text):
    """bench.py exits before touching a GPU: more than one GPU (no multi-GPU path) or counts that
    cannot be timed."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == code, (r.returncode, r.stderr)
    assert text in r.stderr
    assert r.stdout == ""


def test_argmax_workspace_size_in_the_docs():
    """The argmax workspace size that the header and the integration guide state is what the
    library asks for: a caller who sizes the buffer from the documents gets enough bytes."""
    from kq import _lib
    n = int(_lib.kq().kq_argmax_workspace())
    for doc in ("include/kq.h", "INTEGRATION.md"):
        text = open(os.path.join(ROOT, doc)).read()
        stated = {int(v) for v in re.findall(r"kq_argmax_workspace\(\)`? bytes \((\d+)", text)}
        assert stated == {n}, (doc, stated, n)


def test_integration_table_lists_every_entry_point():
    """The integration guide's ABI table has a row for every function include/kq.h declares, and
    names no function the header lacks."""
    names = set(_declared("kq.h"))
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    listed = set()
    for line in text.splitlines():
        if line.startswith("| `kq_"):
            listed |= set(re.findall(r"(kq_\w+)\(", line.split("|")[1]))
    assert listed == names, (sorted(names - listed), sorted(listed - names))


@pytest.mark.parametrize("n,C,x,xq,msg", [
    (0, 4096, 64, None, "n=0 must be 1..3"),
    (1, 4096, 8, None, "x must be 16-byte aligned"),
    (1, 4096, 64, 2, "xq must be 4-byte aligned"),
    (1, 8192, 64, None, "C=8192 > 4096 needs the xq buffer"),
])
def test_gemv_q8k_x_argument_errors(n, C, x, xq, msg):
    """kq_gemv_q8k_x checks its count, the activation and Q8_K buffer alignment, and the xq buffer that
    more than one column pass needs, before any launch (host-only path; the pointers are never read)."""
    from kq import _lib
    lib = _lib.kq()
    W = (ctypes.c_void_p * 1)(16)
    R = (ctypes.c_int * 1)(16)
    T = (ctypes.c_int * 1)(12)
    Y = (ctypes.c_void_p * 1)(64)
    rc = lib.kq_gemv_q8k_x(n, W, R, C, T, ctypes.c_void_p(x), Y, None if xq is None else ctypes.c_void_p(xq), None)
    assert rc == _lib.KQ_ERR_ARG
    assert msg in lib.kq_last_error().decode()
