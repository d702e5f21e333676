"""The oracle's producers of the GEMV inputs (RMSNorm, SwiGLU, their exp), pinned by what the
mathematics fixes: exp against the exact value and its special cases, RMSNorm against closed
forms and the reference CPU engine's summation order, SwiGLU against its limits and exact
scalings.  Each check is shown to reject a plausible mistake planted in a small Python copy."""
import math

import numpy as np
import pytest

F32 = np.float32


def ulp_dist(a, b):
    """Distance in binary32 ulps between float32 arrays a and b (same sign region)."""
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7fffffff), ia)
    ib = np.where(ib < 0, -(ib & 0x7fffffff), ib)
    return np.abs(ia - ib)


def exp_sweep():
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.uniform(-103.9, 88.7, 400000), rng.uniform(-1, 1, 100000),
                        rng.uniform(-87.5, -86.0, 20000), np.linspace(-0.5, 0.5, 10001)]).astype(F32)
    return x


def exp_max_ulp(fn, x):
    got = fn(x)
    want = np.array([math.exp(float(v)) for v in x], np.float64)
    normal = want >= np.finfo(np.float32).tiny
    err = ulp_dist(got[normal], want[normal].astype(F32))
    # subnormal results: within one unit of the smallest subnormal
    sub_err = np.abs(got[~normal].astype(np.float64) - want[~normal]) / 2.0 ** -149
    return int(err.max()), float(sub_err.max()) if sub_err.size else 0.0


def py_expf(x, mistake=None):
    """numpy float32 copy of the oracle's exp steps, with an optional planted mistake."""
    x = np.asarray(x, F32)
    n = np.rint(x * F32(1.4426950216293335)).astype(F32)
    hi, lo = F32(0.693145751953125), F32(1.4286067653e-06)
    if mistake == "no low part":
        lo = F32(0)
    r = ((x - n * hi) - n * lo).astype(F32)
    c = [F32(1 / 5040), F32(1 / 720), F32(1 / 120), F32(1 / 24), F32(1 / 6), F32(0.5), F32(1), F32(1)]
    if mistake == "degree 5":
        c = c[2:]
    if mistake == "wrong coefficient":
        c[4] = F32(1 / 8)
    p = c[0]
    for ck in c[1:]:
        p = (p * r + ck).astype(F32)
    return (p * np.exp2(n.astype(np.float64))).astype(F32)


def test_expf_within_two_ulp_of_exp(orc):
    x = exp_sweep()
    e, sub = exp_max_ulp(orc.expf, x)
    assert e <= 2, e
    assert sub <= 1.0, sub


def test_expf_special_values(orc):
    sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 88.72283, 88.72284, -103.97207, -103.98, 1.0], F32)
    y = orc.expf(sp)
    assert y[0] == 1.0 and y[1] == 1.0
    assert y[2] == np.inf and y[3] == 0.0 and np.isnan(y[4])
    assert np.isfinite(y[5]) and y[5] > 3.4e38 and y[6] == np.inf
    assert y[7] > 0.0 and y[8] == 0.0
    assert ulp_dist(y[9:10], np.array([math.e], F32))[0] <= 1


@pytest.mark.parametrize("mistake", ["no low part", "degree 5", "wrong coefficient"])
def test_expf_check_rejects_planted_mistakes(mistake):
    x = exp_sweep()[::20]
    assert exp_max_ulp(py_expf, x)[0] <= 2                     # the copy without a mistake passes
    assert exp_max_ulp(lambda v: py_expf(v, mistake), x)[0] > 2, mistake


# ---------------------------------------------------------------------------------- RMSNorm
def rms_closed_form_failures(rms):
    """rms(h [N][D], w [D], residual or None) -> (h_out, xn).  Closed forms of q4_rms."""
    bad = []
    D = 4096
    w1 = np.ones(D, F32)
    for c in (1e-3, 0.1, 1.0, 37.5):                          # constant rows: s = 1/sqrt(c^2 + 1e-6)
        h = np.full((1, D), c, F32)
        _, xn = rms(h, w1, None)
        want = F32(c) / math.sqrt(float(F32(c)) ** 2 + 1e-6)
        if ulp_dist(xn[0], np.full(D, want, F32)).max() > 2:
            bad.append("constant %g" % c)
    rng = np.random.default_rng(2)
    h = rng.standard_normal((3, D)).astype(F32)
    r = rng.standard_normal((3, D)).astype(F32)
    w = (1 + 0.1 * rng.standard_normal(D)).astype(F32)
    h_out, xn = rms(h.copy(), w, r)
    if not np.array_equal(h_out, (h + r).astype(F32)):
        bad.append("residual add")
    hs = (h + r).astype(np.float64)
    s = 1.0 / np.sqrt((hs * hs).mean(axis=1, keepdims=True) + 1e-6)
    if np.abs(xn - hs * s * w).max() > 4e-7 * np.abs(hs * s * w).max():
        bad.append("scale")
    return bad


def py_rms(mistake=None):
    def rms(h, w, res):
        h = np.array(h, F32)
        if res is not None and mistake != "no add":
            h = (h + res).astype(F32)
        D = h.shape[1]
        if mistake == "float sum":
            acc = np.zeros(h.shape[0], F32)
            for i in range(D):
                acc = (acc + h[:, i] * h[:, i]).astype(F32)
            acc = acc.astype(np.float64)
        else:
            acc = (h.astype(np.float64) ** 2).sum(axis=1)
        div = D - 1 if mistake == "D-1" else D
        eps = F32(1e-5) if mistake == "eps" else F32(1e-6)
        s = (F32(1) / np.sqrt((acc / div).astype(F32) + eps)).astype(F32)
        return h, ((h * s[:, None]).astype(F32) * w).astype(F32)
    return rms


def test_rms_norm_closed_forms(orc):
    assert rms_closed_form_failures(lambda h, w, r: orc.rms_norm(h, w, r)) == []


@pytest.mark.parametrize("mistake", ["no add", "float sum", "D-1", "eps"])
def test_rms_closed_forms_reject_planted_mistakes(mistake):
    assert rms_closed_form_failures(py_rms()) == []
    assert rms_closed_form_failures(py_rms(mistake)), mistake


def test_rms_norm_orders_agree(orc):
    """q4.cu's strided-tree double sum and kcpu4.c's sequential one give the same floats."""
    rng = np.random.default_rng(9)
    for D in (256, 4096, 12288):
        h = (rng.standard_normal((16, D)) * rng.choice([1e-3, 1.0, 50.0], (16, 1))).astype(F32)
        w = rng.standard_normal(D).astype(F32)
        a = orc.rms_norm(h, w, order=0)[1]
        b = orc.rms_norm(h, w, order=1)[1]
        np.testing.assert_array_equal(a, b)


# ---------------------------------------------------------------------------------- SwiGLU
def swiglu_failures(sw):
    bad = []
    rng = np.random.default_rng(4)
    g = np.concatenate([rng.standard_normal(20000) * 4, [0.0, -0.0, 100.0, -100.0, 30.0, -30.0]]).astype(F32)
    u = rng.standard_normal(g.size).astype(F32)
    y = sw(g, u)
    gd = g.astype(np.float64)
    want = gd / (1 + np.exp(-gd)) * u
    if np.abs(y - want).max() > 4 * 2.0 ** -24 * np.abs(want).max():
        bad.append("value")
    ones = np.ones_like(g)
    y1 = sw(g, ones)
    if not (y1[-6] == 0 and y1[-4] == 100.0 and y1[-3] == 0.0):
        bad.append("limits")
    if not np.array_equal(sw(g, (2 * u).astype(F32)), (2 * y).astype(F32)):
        bad.append("scaling")
    return bad


def py_swiglu(mistake=None):
    def sw(g, u):
        g = np.asarray(g, F32)
        e = np.exp(-g.astype(np.float64)).astype(F32)
        if mistake == "sigmoid only":
            return (F32(1) / (F32(1) + e) * u).astype(F32)
        if mistake == "exp(+g)":
            e = np.exp(g.astype(np.float64)).astype(F32)
        return ((g / (F32(1) + e)).astype(F32) * u).astype(F32)
    return sw


def test_swiglu_closed_forms(orc):
    assert swiglu_failures(orc.swiglu) == []


@pytest.mark.parametrize("mistake", ["sigmoid only", "exp(+g)"])
def test_swiglu_check_rejects_planted_mistakes(mistake):
    with np.errstate(over="ignore"):
        assert swiglu_failures(py_swiglu()) == []
        assert swiglu_failures(py_swiglu(mistake)), mistake


# ---------------------------------------------------------------------------------- greedy pick
def argmax_failures(am):
    """am(y) -> index.  The rule of k_argmax: largest value, smallest index among equals, NaN never
    chosen, nothing above -1e30 -> 0."""
    bad = []
    rng = np.random.default_rng(8)
    y = rng.standard_normal(151936).astype(F32)
    if am(y) != int(np.argmax(y)):
        bad.append("random")
    t = y.copy()
    t[[700, 90000, 150000]] = 9.0                         # three equal maxima
    if am(t) != 700:
        bad.append("ties")
    t[5] = np.nan
    t[6] = np.inf
    if am(t) != 6:
        bad.append("inf")
    t[6] = 0.0
    if am(t) != 700:
        bad.append("nan")
    if am(np.full(3000, -np.inf, F32)) != 0 or am(np.full(5, -2e30, F32)) != 0:
        bad.append("nothing above -1e30")
    neg = (-1 - rng.random(5000)).astype(F32)
    if am(neg) != int(np.argmax(neg)):
        bad.append("all negative")
    if am(np.array([1.0], F32)) != 0 or am(np.array([-1e30, -1e29], F32)) != 1:
        bad.append("small")
    return bad


def py_argmax(mistake=None):
    def am(y):
        y = np.asarray(y, F32)
        bv, bi = (F32(0) if mistake == "start at 0" else F32(-1e30)), 0
        for i, v in enumerate(y):
            if (v >= bv) if mistake == "last max" else (v > bv or (mistake == "nan wins" and np.isnan(v))):
                bv, bi = v, i
        return bi
    return am


def test_argmax_rule(orc):
    assert argmax_failures(orc.argmax) == []


@pytest.mark.parametrize("mistake", ["start at 0", "last max", "nan wins"])
def test_argmax_check_rejects_planted_mistakes(mistake):
    assert argmax_failures(py_argmax()) == []
    assert argmax_failures(py_argmax(mistake)), mistake
