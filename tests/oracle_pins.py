"""Pins of the oracle's quantizers and activation rounding points, written against a ctypes handle of any build of
oracle/rda_oracle.c (oracle.load(path)), so that the same checks run on the oracle itself (tests/test_oracle_pins.py,
which expects no failures) and on copies of it with one planted mistake each (tests/test_oracle_mutants.py, which
expects the matching check to fail).

What fixes each function, independently of the oracle's own formula:

* rint quantizers (int8-QK Q/K codes, hip_attention.hip:85-91, 183-193; W4A4 activations, int8_gemm.hip:71, 84):
  rows built so that every quotient x / s is exactly k + 1/2 (s a power of two), checked against round-half-to-even
  done in exact rational arithmetic; random rows against numpy's IEEE float32 division and np.rint; zero rows
  against the scale floors 1e-30 (int8) and 1e-10 / 7 (int4).
* floor(x / s + 1/2) quantizer of the rotated int8 path (int8_gemm.hip:38, 53): the same exact-tie rows, checked
  against rational round-half-up.
  The rotated rows reach the quantizer through the oracle's block Hadamard: inputs are x = H y / 16 for an integer
  vector y with few non-zeros, so every butterfly is exact and the rotated row is y itself (H H = 256 I).
* SwiGLU, sigmoid gate (int8_gemm.hip:130-137): r16(r16(f(g)) * u) where f is silu or sigmoid. For every input
  whose float64 f(g) lies farther than 2^-18 (relative) from an fp16 rounding midpoint -- beyond the few-ulp error
  of the fp32 exp chain -- the inner fp16 value is the correctly rounded f(g), the product with u is exact, and the
  result is fp16 of that exact product. The check also counts inputs where a single rounding of f(g) * u gives
  another result, so that it is known to see that mistake.
* situ (int8_gemm.hip:124-127): one fp16 rounding of the fp32 product chain: for inputs farther than 2^-14 from a
  midpoint (the chain's soft tanh loses a few bits to cancellation near |x| = 0.02), the result is fp16 of the
  float64 value.
* modulate (int8_gemm.hip:140-143): r16(r16(r16(x rstd (w + 1)) s) + t): the first rounding is the correctly
  rounded float64 product (2^-19 margin), the second is exact fp16 of an exact product, the last fp16 of the
  IEEE float32 sum.
"""
import ctypes
import math
from fractions import Fraction

import numpy as np

import oracle


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _rhe(fr):
    """Round half to even of a Fraction."""
    fl = math.floor(fr)
    rem = fr - fl
    if rem > Fraction(1, 2):
        return fl + 1
    if rem < Fraction(1, 2):
        return fl
    return fl if fl % 2 == 0 else fl + 1


def _half_up(fr):
    return math.floor(fr + Fraction(1, 2))


def _quant_rows_rint(L, x):
    x = np.ascontiguousarray(x, np.float16)
    R, D = x.shape
    q = np.empty((R, D), np.int8)
    s = np.empty(R, np.float32)
    L.orc_quant_rows_rint(R, D, _ptr(x), D, _ptr(q), _ptr(s))
    return q, s


def _rot_quant(L, x, i4):
    x = np.ascontiguousarray(x, np.float16)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    rot = np.empty((M, K), np.uint16)
    L.orc_rot_quant_rows(0, int(i4), 256, M, K, _ptr(x), K, None, None, None, None, 1, 0.0, _ptr(q), _ptr(s), _ptr(rot))
    return q, s, rot.view(np.float16)


# ---------------------------------------------------------------------------------------- rint quantizers ---

def rint_failures(L):
    """orc_quant_rows_rint (Q/K codes of the int8-QK attention)."""
    bad = []
    D = 128
    rows, expect_q, expect_s = [], [], []
    # Scales m 2^e (absmax 127 m 2^e): every quotient is exactly k + 1/2. With m = 7 or 13 the fp32 reciprocal of the
    # scale is off by ~2^-24.4, enough to move a product x (1 / s) off the tie when k + 1/2 is near 127.
    for m in (1, 3, 5, 7, 11, 13):
        kmax = min(126, (2047 // m - 1) // 2)  # (2k + 1) m must fit fp16's 11-bit significand
        for e in range(-14, 9):
            if 127 * m * 2.0 ** e > 65504:
                continue
            sign = -1 if (e + m) % 2 else 1
            ks = [((j * 37 + e * 11) % (2 * kmax + 1)) - kmax for j in range(1, D)]  # k in [-kmax, kmax]
            row = [sign * 127 * m * 2.0 ** e] + [(k + 0.5) * m * 2.0 ** e for k in ks]
            rows.append(row)
            expect_s.append(np.float32(m * 2.0 ** e))
            expect_q.append([sign * 127] + [_rhe(Fraction(k) + Fraction(1, 2)) for k in ks])
    x = np.array(rows, np.float64).astype(np.float16)
    assert np.array_equal(x.astype(np.float64), np.array(rows)), "tie rows must be exact in fp16"
    q, s = _quant_rows_rint(L, x)
    if not np.array_equal(s, np.array(expect_s, np.float32)):
        bad.append("tie-row scales")
    if not np.array_equal(q.astype(np.int64), np.array(expect_q)):
        bad.append(f"exact k+1/2 quotients: {int((q != np.array(expect_q)).sum())} codes differ from round-half-even")
    # Random rows against IEEE float32 division and numpy's round-half-even.
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((64, D)) * 10.0 ** rng.uniform(-4, 3.5, (64, 1))).astype(np.float16)
    q, s = _quant_rows_rint(L, x)
    mx = np.abs(x.astype(np.float32)).max(1)
    es = np.maximum(mx / np.float32(127), np.float32(1e-30)).astype(np.float32)
    eq = np.rint(x.astype(np.float32) / es[:, None]).astype(np.int64)
    if not np.array_equal(s, es):
        bad.append("random-row scales")
    if not np.array_equal(q.astype(np.int64), eq):
        bad.append("random-row codes")
    # Zero rows: the 1e-30 floor, all codes 0.
    q, s = _quant_rows_rint(L, np.zeros((2, D), np.float16))
    if not (np.all(s == np.float32(1e-30)) and np.all(q == 0)):
        bad.append("zero-row floor")
    return bad


def _tie_rows(scale_exp, top, ks_list, rng):
    """Rows x = H y / 16 whose rotation is exactly y: y[p0] = +-top (the absmax), y[p] = (k + 1/2) 2^scale_exp."""
    H = oracle.hadamard_matrix(256)
    xs, ys = [], []
    for r, ks in enumerate(ks_list):
        y = np.zeros(256, np.int64)
        pos = rng.choice(256, len(ks) + 1, replace=False)
        y[pos[0]] = top if r % 2 == 0 else -top
        for p, k in zip(pos[1:], ks):
            y[p] = (2 * k + 1) * 2 ** (scale_exp - 1)
        x = H @ y
        assert np.all(x % 16 == 0) and np.abs(x // 16).max() <= 2048
        xs.append(x // 16)
        ys.append(y)
    return np.array(xs, np.float64).astype(np.float16), np.array(ys)


def i4_failures(L):
    """quant_row_i4 of the W4A4 activations (rint, clamp 7, scale max(absmax, 1e-10) / 7)."""
    bad = []
    rng = np.random.default_rng(11)
    ks_list = [[int(k) for k in rng.integers(-7, 7, 15)] for _ in range(24)]  # k + 1/2 in [-6.5, 6.5]
    x, y = _tie_rows(5, 224, ks_list, rng)  # absmax 224: scale 224 / 7 = 32 exactly
    q, s, rot = _rot_quant(L, x, True)
    if not np.array_equal(rot.astype(np.int64), y):
        bad.append("tie rows: rotation is not y")
    if not np.all(s == np.float32(32)):
        bad.append("tie-row scales")
    expect = np.array([[_rhe(Fraction(int(v), 32)) for v in row] for row in y])
    if not np.array_equal(q.astype(np.int64), expect):
        bad.append(f"exact k+1/2 quotients: {int((q != expect).sum())} codes differ from round-half-even")
    q, s, _ = _rot_quant(L, np.zeros((2, 256), np.float16), True)
    if not (np.all(s == np.float32(1e-10) / np.float32(7)) and np.all(q == 0)):
        bad.append("zero-row floor")
    return bad


def i8_rot_failures(L):
    """quant_row of the rotated int8 path (floor(x / s + 1/2), clamp [-128, 127], scale max(absmax / 127, 1e-30))."""
    bad = []
    rng = np.random.default_rng(13)
    ks_list = [[int(k) for k in rng.integers(-40, 40, 15)] for _ in range(24)]
    x, y = _tie_rows(5, 4064, ks_list, rng)  # absmax 4064 = 127 x 32: scale 32 exactly
    q, s, rot = _rot_quant(L, x, False)
    if not np.array_equal(rot.astype(np.int64), y):
        bad.append("tie rows: rotation is not y")
    if not np.all(s == np.float32(32)):
        bad.append("tie-row scales")
    expect = np.array([[_half_up(Fraction(int(v), 32)) for v in row] for row in y])
    if not np.array_equal(q.astype(np.int64), expect):
        bad.append(f"exact k+1/2 quotients: {int((q != expect).sum())} codes differ from round-half-up")
    q, s, _ = _rot_quant(L, np.zeros((2, 256), np.float16), False)
    if not (np.all(s == np.float32(1e-30)) and np.all(q == 0)):
        bad.append("zero-row floor")
    return bad


# ------------------------------------------------------------------------------ activation rounding points ---

def _midpoint_distance(v):
    """Relative distance of float64 values v from the nearest fp16 rounding midpoint (inf where |v| >= 65520)."""
    v = np.asarray(v, np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        h = v.astype(np.float16)
        up = np.nextafter(h, np.float16(np.inf)).astype(np.float64)
        dn = np.nextafter(h, np.float16(-np.inf)).astype(np.float64)
        hv = h.astype(np.float64)
        mid = np.where(v >= hv, (hv + up) / 2, (hv + dn) / 2)
        d = np.abs(v - mid) / np.maximum(np.abs(v), 2.0 ** -25)
    return np.where(np.isfinite(hv), d, np.inf)


def _fp16_grid(lo, hi):
    """Every finite fp16 value in [lo, hi], as float64."""
    h = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float64)
    h = h[np.isfinite(h)]
    return np.unique(h[(h >= lo) & (h <= hi)])


def _call(L, name, *cols):
    f = getattr(L, name)
    return np.array([f(*[float(c[i]) for c in cols]) for i in range(len(cols[0]))], np.float64)


def _gated_product_failures(L, name, inner64, g, other, min_single_differs):
    """r16(r16(inner) * other) checks for SwiGLU / sigmoid gate (see the module docstring)."""
    bad = []
    sure = _midpoint_distance(inner64) > 2.0 ** -18
    inner = inner64.astype(np.float16).astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        expect = (inner * other).astype(np.float16).astype(np.float64)  # exact product, one rounding
        single = (inner64 * other).astype(np.float16).astype(np.float64)
    got = _call(L, name, *((g, other) if name == "orc_swiglu" else (other, g)))
    mism = sure & ~((got == expect) | (np.isnan(got) & np.isnan(expect)))
    if mism.any():
        i = int(np.argmax(mism))
        bad.append(f"{name}: {int(mism.sum())} of {int(sure.sum())} sure inputs differ, e.g. g={g[i]} other={other[i]}: {got[i]} vs {expect[i]}")
    differs = int((sure & (single != expect)).sum())
    if differs < min_single_differs:
        bad.append(f"{name}: only {differs} inputs tell double from single rounding")
    return bad


def swiglu_failures(L):
    rng = np.random.default_rng(17)
    g = _fp16_grid(-30.0, 30.0)
    u = (rng.standard_normal(g.size) * 3).astype(np.float16).astype(np.float64)
    silu = g / (1.0 + np.exp(-g))
    return _gated_product_failures(L, "orc_swiglu", silu, g, u, g.size // 50)


def sigmoid_gate_failures(L):
    rng = np.random.default_rng(19)
    g = _fp16_grid(-16.0, 16.0)
    x = (rng.standard_normal(g.size) * 3).astype(np.float16).astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-g))
    return _gated_product_failures(L, "orc_sigmoid_gate", sig, g, x, g.size // 50)


def _tanh_fp32_args(a):
    """tanh of |a| as the soft tanh defines it: the logistic form (1 - 2^(-c a)) / (1 + 2^(-c a)) with c the fp32
    constant 2 / ln 2, and its Taylor polynomial (the series of tanh) below 0.02."""
    c = float(np.float32(2.885390082))
    t = np.exp2(-c * a)
    return np.where(a < 0.02, np.tanh(a), (1 - t) / (1 + t))


def situ_failures(L):
    bad = []
    rng = np.random.default_rng(23)
    n = 20000
    g = (rng.standard_normal(n) * 4).astype(np.float16).astype(np.float64)
    h = (rng.standard_normal(n) * 20).astype(np.float16).astype(np.float64)
    c_sig = float(np.float32(1.442695041))
    c_h = float(np.float32(0.04))
    ga, ha = np.abs(g * 0.25), np.abs(h * c_h)
    v = 4 * np.sign(g) * _tanh_fp32_args(ga) / (1 + np.exp2(-c_sig * g)) * 25 * np.sign(h) * _tanh_fp32_args(ha)
    sure = _midpoint_distance(v) > 2.0 ** -14
    got = _call(L, "orc_situ", h, g)
    expect = v.astype(np.float16).astype(np.float64)
    mism = sure & (got != expect)
    if mism.any():
        i = int(np.argmax(mism))
        bad.append(f"orc_situ: {int(mism.sum())} of {int(sure.sum())} sure inputs differ, e.g. h={h[i]} g={g[i]}: {got[i]} vs {expect[i]}")
    if sure.sum() < n // 2:
        bad.append("orc_situ: too few sure inputs")
    return bad


def modulate_failures(L):
    bad = []
    rng = np.random.default_rng(29)
    n = 20000
    x = (rng.standard_normal(n) * 2).astype(np.float16).astype(np.float64)
    rstd = rng.uniform(0.3, 3.0, n).astype(np.float32).astype(np.float64)
    w = (rng.standard_normal(n) * 0.1).astype(np.float32).astype(np.float64)
    s = (1 + rng.standard_normal(n) * 0.3).astype(np.float16).astype(np.float64)
    t = (rng.standard_normal(n) * 0.3).astype(np.float16).astype(np.float64)
    v = x * rstd * (1 + w)
    sure = _midpoint_distance(v) > 2.0 ** -19
    a = v.astype(np.float16).astype(np.float64)
    b = (a * s).astype(np.float16)  # a s is exact in float64 (and float32): one rounding
    expect = (b.astype(np.float32) + t.astype(np.float32)).astype(np.float16).astype(np.float64)
    got = _call(L, "orc_modulate", x, rstd, w, s, t)
    mism = sure & (got != expect)
    if mism.any():
        i = int(np.argmax(mism))
        bad.append(f"orc_modulate: {int(mism.sum())} of {int(sure.sum())} sure inputs differ, e.g. x={x[i]}: {got[i]} vs {expect[i]}")
    no_mid = ((a * s).astype(np.float32) + t.astype(np.float32)).astype(np.float16).astype(np.float64)
    if int((sure & (no_mid != expect)).sum()) < n // 100:
        bad.append("orc_modulate: too few inputs tell the middle rounding apart")
    return bad


CHECKS = {
    "rint": rint_failures,
    "i4": i4_failures,
    "i8_rot": i8_rot_failures,
    "swiglu": swiglu_failures,
    "sigmoid_gate": sigmoid_gate_failures,
    "situ": situ_failures,
    "modulate": modulate_failures,
}
