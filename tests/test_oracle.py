"""Pins the CPU oracle (oracle/kq_oracle.c) before anything is checked against it.

* Decode and the fp32-activation matvec: bit-exact against outputs of the reference's own CPU
  path (kc_dequant / kc_matvec, kcpu4.c:337-341) -- committed fixtures always, and the live
  reference build (oracle/_ref) on fresh random inputs when it is present.
* The reference unit test's own tolerance (test_quant.py:32).
* Q8_K (GGML semantics, not in the reference): closed-form blocks that fix rounding, sign
  convention, tie-breaking and the zero block, plus invariants; a planted-mistake check shows each
  closed form rejects a plausible wrong variant.
* Integer sub-block sums and their epilogue: against an fp64 dense product of the reference's
  decode (exact for d = dmin = fp16(0.013) inputs) and the dequantized Q8_K activations.
"""
import numpy as np
import pytest

from helpers import reference_unit_inputs

CASES = [("tq", 12), ("tq", 14), ("syn", 12), ("syn", 14)]


@pytest.mark.parametrize("tag,ty", CASES)
def test_golden_decode_bit_exact(orc, golden, tag, ty):
    k = "%s_%d_" % (tag, ty)
    R, C, _ = golden[k + "shape"]
    W = golden[k + "w"]
    for i, r in enumerate(golden[k + "rows"]):
        np.testing.assert_array_equal(orc.dequant_row(W, R, C, ty, int(r)), golden[k + "deq"][i])


@pytest.mark.parametrize("tag,ty", CASES)
def test_golden_matvec_bit_exact(orc, golden, tag, ty):
    """The restated q4_dot lane order reproduces kc_matvec bit for bit."""
    k = "%s_%d_" % (tag, ty)
    R, C, _ = golden[k + "shape"]
    y = orc.matvec_f32(golden[k + "w"], R, C, ty, golden[k + "x"])
    np.testing.assert_array_equal(y, golden[k + "y"])


def _random_blocks(rng, R, C, ty, d_choices):
    bs = {12: 144, 14: 210}[ty]
    raw = rng.integers(0, 256, (R, C // 256, bs), dtype=np.uint8)
    d = rng.choice(np.array(d_choices, dtype="<f2"), size=(R, C // 256, 2 if ty == 12 else 1))
    if ty == 12:
        raw[:, :, 0:4] = d.view(np.uint8).reshape(R, C // 256, 4)
    else:
        raw[:, :, 208:210] = d.view(np.uint8).reshape(R, C // 256, 2)
    return raw.reshape(R // 8, 8, C // 256, bs).transpose(0, 2, 1, 3).copy().reshape(-1)


@pytest.mark.parametrize("ty", [12, 14])
def test_live_reference_bit_exact(orc, ty):
    """Fresh inputs through the compiled reference: zero, subnormal, negative and large scales."""
    if not orc.ref_available():
        pytest.skip("reference library not built (needs the reference sources)")
    rng = np.random.default_rng(101 + ty)
    R, C = 24, 1536
    W = _random_blocks(rng, R, C, ty, [0.0, -0.0, 1e-7, 3e-5, 0.013, -0.25, 1.5, 60000.0])
    x = rng.normal(size=C).astype(np.float32)
    np.testing.assert_array_equal(orc.matvec_f32(W, R, C, ty, x), orc.ref_matvec(W, R, C, ty, x))
    for r in (0, 5, 8, 23):
        np.testing.assert_array_equal(orc.dequant_row(W, R, C, ty, r), orc.ref_dequant_row(W, R, C, ty, r))


@pytest.mark.parametrize("ty", [12, 14])
def test_reference_unit_tolerance(orc, ty):
    """tests/kindi_q4/test_quant.py:30-32 with its own tolerance."""
    W, x, R, C = reference_unit_inputs()[ty]
    dense = orc.dequant(W, R, C, ty).astype(np.float64)
    y = orc.matvec_f32(W, R, C, ty, x)
    np.testing.assert_allclose(y, dense @ x.astype(np.float64), atol=0.00015, rtol=0.00001)


def test_q4k_closed_form_block(orc):
    """A hand-built Q4_K block: d=1, dmin=0.5, sc_k = k+1, m_k = 2k, q_j = j % 16.

    The 12 scale bytes follow GGML's packing: bytes 0..3 hold sc_0..3 (low 6 bits) and the top
    two bits of sc_4..7; bytes 4..7 hold m_0..3 and the top bits of m_4..7; bytes 8..11 hold the
    low nibbles of sc_4..7 (low) and m_4..7 (high).  Expected w = (k+1)*q - k.
    """
    sc = [1, 2, 3, 4, 5, 6, 7, 8]
    m = [0, 2, 4, 6, 8, 10, 12, 14]
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([1.0], "<f2").view(np.uint8)
    b[2:4] = np.array([0.5], "<f2").view(np.uint8)
    for j in range(4):
        b[4 + j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        b[8 + j] = m[j] | ((m[j + 4] >> 4) << 6)
        b[12 + j] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    q = np.arange(32) % 16
    for p in range(4):   # qs[32p + j]: low nibble -> sub-block 2p, high nibble -> 2p+1
        b[16 + 32 * p:48 + 32 * p] = q | (((q + 1) % 16) << 4)
    y = orc.decode_block(b, 12)
    for k in range(8):
        qk = q if k % 2 == 0 else (q + 1) % 16
        np.testing.assert_array_equal(y[32 * k:32 * k + 32], (k + 1) * qk.astype(np.float32) - k)


def test_q4k_high_scale_bits(orc):
    """sc, m >= 16 for k >= 4 exercise the 2-bit carries (sc = 48 + k, m = 33 + k)."""
    sc = [10, 11, 12, 13, 52, 53, 54, 55]
    m = [20, 21, 22, 23, 37, 38, 39, 40]
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([0.25], "<f2").view(np.uint8)
    b[2:4] = np.array([0.125], "<f2").view(np.uint8)
    for j in range(4):
        b[4 + j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        b[8 + j] = m[j] | ((m[j + 4] >> 4) << 6)
        b[12 + j] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    b[16:144] = 0xF3            # low nibble 3, high nibble 15
    y = orc.decode_block(b, 12)
    for k in range(8):
        q = 3 if k % 2 == 0 else 15
        np.testing.assert_array_equal(y[32 * k:32 * k + 32], np.float32(0.25 * sc[k] * q - 0.125 * m[k]))


def test_q6k_closed_form_block(orc):
    """Q6_K extremes: q6 = 0 -> -32, 63 -> 31; sc = -128 and 127; element layout of q4kernels.h:26-28."""
    b = np.zeros(210, np.uint8)
    b[208:210] = np.array([0.5], "<f2").view(np.uint8)
    sc = np.array([(-128 if t % 2 else 127) for t in range(16)], np.int8)
    b[192:208] = sc.view(np.uint8)
    u = np.array([(e * 7) % 64 for e in range(256)])
    for e in range(256):
        h, k, j = e // 128, (e % 128) // 32, e % 32
        b[h * 64 + (k % 2) * 32 + j] |= (u[e] & 15) << ((k // 2) * 4)
        b[128 + h * 32 + j] |= (u[e] >> 4) << (2 * k)
    y = orc.decode_block(b, 14)
    expect = np.array([0.5 * sc[e // 16] * (u[e] - 32) for e in range(256)], np.float32)
    np.testing.assert_array_equal(y, expect)


# ------------------------------------------------------------------------------------------ Q8_K
def _fields(orc, x):
    return orc.q8k_fields(orc.quantize_q8k(np.asarray(x, np.float32).reshape(1, -1)))


def q8k_closed_form_failures(quantize):
    """Runs the closed-form Q8_K cases through `quantize(x[256]) -> (d, qs, bsums)`; returns the
    names of the cases it gets wrong (empty for a correct GGML quantize_row_q8_K_ref)."""
    bad = []
    d, qs, bs = quantize(np.zeros(256, np.float32))
    if not (d == 0 and not qs.any() and not bs.any()):
        bad.append("zero block")
    # max = -127 -> iscale = 1 exactly: quants are round-half-even of x itself
    x = np.zeros(256, np.float32)
    x[0] = -127
    x[1:9] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.4999999, 126.5]
    d, qs, bs = quantize(x)
    if not (d == 1.0 and list(qs[:9]) == [-127, 2, 4, -2, -4, 0, 0, 1, 126]):
        bad.append("round half even")
    # positive max maps to -127 and d is negative
    x = np.full(256, 0.01, np.float32)
    x[5] = 2.0
    d, qs, bs = quantize(x)
    if not (qs[5] == -127 and d == np.float32(1) / (np.float32(-127) / np.float32(2.0))):
        bad.append("sign convention")
    # equal |x| at indexes 3 (negative) and 10 (positive): the first one is max
    x = np.zeros(256, np.float32)
    x[3], x[10] = -5.0, 5.0
    d, qs, bs = quantize(x)
    if not (qs[3] == -127 and qs[10] == 127):
        bad.append("first max wins")
    # bsums are the sums of 16 consecutive quants
    x = np.linspace(-3, 2, 256).astype(np.float32)
    d, qs, bs = quantize(x)
    if not np.array_equal(bs, qs.reshape(16, 16).astype(np.int32).sum(1)):
        bad.append("bsums")
    return bad


def test_q8k_closed_forms(orc):
    def q(x):
        d, qs, bs = _fields(orc, x)
        return d[0, 0], qs[0, 0], bs[0, 0]
    assert q8k_closed_form_failures(q) == []


def test_q8k_closed_forms_reject_planted_mistakes():
    """Each plausible mistake, planted in a small Python quantizer, fails a closed form."""
    def make(mistake):
        def quantize(x):
            x = np.asarray(x, np.float32)
            ax = np.abs(x)
            amax = ax.max()
            if amax == 0:
                return np.float32(0), np.zeros(256, np.int8), np.zeros(16, np.int16)
            i = int(np.argmax(ax)) if mistake != "last max" else int(255 - np.argmax(ax[::-1]))
            mx = x[i] if mistake != "positive max" else amax
            iscale = np.float32(-127) / mx if mistake != "positive scale" else np.float32(127) / mx
            t = (iscale * x).astype(np.float32)
            qf = np.rint(t) if mistake != "half away" else np.sign(t) * np.floor(np.abs(t) + 0.5)
            qs = np.minimum(127, qf).astype(np.int8)
            bs = qs.reshape(16, 16).astype(np.int32).sum(1).astype(np.int16)
            if mistake == "bsum stride":
                bs = qs.reshape(16, 16).astype(np.int32).sum(0).astype(np.int16)
            return np.float32(1) / iscale, qs, bs
        return quantize
    assert q8k_closed_form_failures(make(None)) == []
    for mistake in ("half away", "positive max", "positive scale", "last max", "bsum stride"):
        assert q8k_closed_form_failures(make(mistake)), mistake


def test_q8k_invariants_random(orc):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((8, 4096)) * rng.choice([1e-3, 1.0, 300.0], size=(8, 1))).astype(np.float32)
    x[3, 256:512] = 0
    d, qs, bs = orc.q8k_fields(orc.quantize_q8k(x))
    xb = x.reshape(8, 16, 256)
    assert np.all(np.abs(qs.astype(np.int32)) <= 127)
    np.testing.assert_array_equal(bs, qs.reshape(8, 16, 16, 16).astype(np.int32).sum(-1))
    err = np.abs(xb - d[..., None].astype(np.float64) * qs)
    assert np.all(err <= np.abs(d[..., None]) * (0.5 + 1e-5) + 1e-30)
    first = np.argmax(np.abs(xb), axis=-1)
    np.testing.assert_array_equal(np.take_along_axis(qs, first[..., None], -1)[..., 0][d != 0], -127)
    assert d[3, 1] == 0 and not qs[3, 1].any()


# ---------------------------------------------------------------------- integer dot and epilogue
@pytest.mark.parametrize("ty", [12, 14])
def test_int_sums_match_exact_dense_product(orc, ty):
    """sum_g epilogue(S) == dense fp64 product of the reference decode and dequantized Q8_K.

    With d = dmin = fp16(0.013) the reference's fp32 decode is exact for Q4_K, so the two sides
    are the same real number; Q6_K's (d*sc)*(q-32) can round once per weight (relative 2^-24).
    """
    W, _, R, C = reference_unit_inputs()[ty]
    rng = np.random.default_rng(11)
    x = rng.standard_normal((5, C)).astype(np.float32)
    x[4, :256] = 0
    xq = orc.quantize_q8k(x)
    d, qs, _ = orc.q8k_fields(xq)
    xd = (d[..., None].astype(np.float64) * qs).reshape(5, C)
    dense = orc.dequant(W, R, C, ty).astype(np.float64)
    want = xd @ dense.T
    got = orc.gemv_q8k(W, R, C, ty, xq, 5)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= (1e-12 if ty == 12 else 1e-6) * scale


@pytest.mark.parametrize("ty", [12, 14])
def test_subblock_sums_isolated(orc, ty):
    """Activations confined to one sub-block s isolate S_s.  For every row the decoded weights of
    that sub-block must then satisfy  w_s . q8 = a*S_s + b*sum(q8)  with one (a, b) per row
    (a = d*sc, b = -dmin*m; Q6_K has b = 0 since its -32 offset is inside S); a fit over four
    independent activations leaves no residual only if S_s holds exactly the right elements."""
    W, _, R, C = reference_unit_inputs()[ty]
    nsub = 8 if ty == 12 else 16
    width = 256 // nsub
    rng = np.random.default_rng(3)
    dense = orc.dequant(W, R, C, ty).astype(np.float64)
    for s in (0, 1, nsub // 2, nsub - 1):
        lo = 256 + s * width
        S, B, L = [], [], []
        for _ in range(4):
            x = np.zeros((1, C), np.float32)
            x[0, lo:lo + width] = rng.standard_normal(width)
            xq = orc.quantize_q8k(x)
            Sk = orc.subblock_sums(W, R, C, ty, xq, 1)[0]
            assert not Sk[:, 0].any() and not np.delete(Sk[:, 1], s, axis=1).any()
            q8 = orc.q8k_fields(xq)[1].reshape(C).astype(np.float64)
            S.append(Sk[:, 1, s].astype(np.float64))
            B.append(q8[lo:lo + width].sum())
            L.append(dense[:, lo:lo + width] @ q8[lo:lo + width])
        S, L = np.array(S), np.array(L)
        for r in range(R):
            A = np.stack([S[:, r], np.array(B)], 1) if ty == 12 else S[:, r:r + 1]
            coef = np.linalg.lstsq(A, L[:, r], rcond=None)[0]
            resid = np.abs(A @ coef - L[:, r]).max()
            assert resid <= (1e-9 if ty == 12 else 1e-5) * max(1.0, np.abs(L[:, r]).max()), (s, r)


def test_ggml_fp32_order_within_tolerance(orc):
    from kq import quantize as kqq
    for ty in (12, 14):
        R, C = 64, 4096
        W = kqq.synthetic_matrix(R, C, ty, seed=ty)
        xq = orc.quantize_q8k(kqq.synthetic_activations(2, C, seed=ty))
        ref = orc.gemv_q8k(W, R, C, ty, xq, 2)
        g = orc.gemv_q8k_ggml(W, R, C, ty, xq, 2)
        assert np.abs(g - ref).max() <= 1e-5 * np.abs(ref).max()
