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
* GEMM epilogue (int8_gemm.hip:382-383): y = ((float)acc * as) * ws, left to right, each step one IEEE fp32
  rounding, then + bias and fp16. Evaluated in exact rationals with a rounding to fp32 after every operation.
  The accumulators are chosen so that y lands within an fp32 ulp of an fp16 rounding midpoint, where the
  association acc * (as * ws) gives another fp16 result; the check counts those inputs.
* gated residual (int8_gemm.hip:394-400): C = fp16(R + fp16(G[m / L] * y)), contraction off: exact rationals,
  with the inner fp16 rounding, against inputs where dropping it changes C.
* RoPE (rms_norm.hip:55-57): a = fp16(fma(m1, x1, fp32(m0 x0))), c likewise with m2, m3: exact rationals, with
  rotation matrices built so that the exact value lies near an fp16 midpoint, where evaluating with two separate
  fp32 roundings, or in one exact step, gives another result.
* W4A8 epilogue (no reference counterpart): y = fma((float)p_g, gs[n][g], y) over the groups in order, then
  fp16(y * as (+ bias)): exact rationals with one fp32 rounding per fma and per operation.
"""
import ctypes
import math
from fractions import Fraction

import numpy as np

import oracle


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


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


# ------------------------------------------------------------------- exact binary rounding (no numpy floats) ---

def _round_binary(fr, p, emin, emax):
    """fr rounded to the nearest binary float with p significant bits, normal exponents emin..emax and subnormals
    below 2^emin, ties to even; magnitudes that round to 2^(emax + 1) or beyond become +-inf. Exact arithmetic."""
    if fr == 0:
        return Fraction(0)
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    elif Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = Fraction(2) ** (max(e, emin) - p + 1)
    r = _rhe(a / ulp) * ulp
    if r >= Fraction(2) ** (emax + 1):
        return math.inf if fr > 0 else -math.inf
    return r if fr > 0 else -r


def _r32(fr):
    return _round_binary(fr, 24, -126, 127)


def _r16(fr):
    return _round_binary(fr, 11, -14, 15)


def _fr(v):
    return Fraction(float(v))


def _as_f64(frs):
    return np.array([float(v) for v in frs], np.float64)


def _epilogue(L, acc, a_s, w_s, bias=None, R=None, G=None, Lg=1):
    acc = np.ascontiguousarray(acc, np.int32)
    M, N = acc.shape
    out = np.empty((M, N), np.uint16)
    a_s = np.ascontiguousarray(a_s, np.float32)
    w_s = np.ascontiguousarray(w_s, np.float32)
    args = [None if t is None else np.ascontiguousarray(t, np.float16) for t in (bias, R, G)]
    L.orc_gemm_epilogue(M, N, _ptr(acc), _ptr(a_s), _ptr(w_s), *[_ptr(t) for t in args], Lg, _ptr(out))
    return out.view(np.float16).astype(np.float64)


def _midpoint_accumulators(rng, a_s, w_s, lo, hi, offset=None):
    """acc[m, n] = the integer nearest (mid - offset[n]) / (as[m] ws[n]) for a random fp16 rounding midpoint mid in
    [lo, hi]: with |acc| >= 2^23 the exact product plus the offset lies within about an fp32 ulp of the midpoint."""
    grid = _fp16_grid(lo, hi)
    M, N = a_s.size, w_s.size
    h = grid[rng.integers(0, grid.size - 1, (M, N))]
    up = np.nextafter(h.astype(np.float16), np.float16(np.inf)).astype(np.float64)
    mid = (h + up) / 2 * np.where(rng.random((M, N)) < 0.5, -1, 1)
    if offset is not None:
        mid = mid - np.asarray(offset, np.float64)[None]
    acc = np.rint(mid / (a_s.astype(np.float64)[:, None] * w_s.astype(np.float64)[None]))
    assert np.abs(acc).max() < 2 ** 31 and np.abs(acc).min() >= 2 ** 23
    return acc.astype(np.int32)


def epilogue_failures(L):
    """((float)acc * as) * ws (+ bias) -> fp16, left to right."""
    bad = []
    rng = np.random.default_rng(31)
    M, N = 48, 64
    a_s = rng.uniform(2e-5, 1e-4, M).astype(np.float32)
    w_s = rng.uniform(1e-3, 3e-3, N).astype(np.float32)
    bias = rng.uniform(-2, 2, N).astype(np.float16)
    for with_bias in (False, True):
        acc = _midpoint_accumulators(rng, a_s, w_s, 6.0, 16.0, bias.astype(np.float64) if with_bias else None)
        got = _epilogue(L, acc, a_s, w_s, bias if with_bias else None)
        expect, other = [], 0
        for m in range(M):
            for n in range(N):
                a, x, w = _r32(Fraction(int(acc[m, n]))), _fr(a_s[m]), _fr(w_s[n])
                y = _r32(_r32(a * x) * w)
                y2 = _r32(a * _r32(x * w))
                if with_bias:
                    y, y2 = _r32(y + _fr(bias[n])), _r32(y2 + _fr(bias[n]))
                expect.append(_r16(y))
                other += _r16(y2) != _r16(y)
        expect = _as_f64(expect).reshape(M, N)
        tag = "epilogue with bias" if with_bias else "epilogue"
        if not np.array_equal(got, expect):
            bad.append(f"{tag}: {int((got != expect).sum())} of {M * N} outputs differ from the left-to-right fp32 chain")
        if other < M * N // 50:
            bad.append(f"{tag}: only {other} inputs tell acc * (as * ws) apart")
    return bad


def gated_residual_failures(L):
    """C = fp16(R + fp16(G[m / L] * y)) after the epilogue, with L tokens per gate row."""
    bad = []
    rng = np.random.default_rng(37)
    M, N, Lg = 32, 64, 4
    acc = rng.integers(-2 ** 22, 2 ** 22, (M, N)).astype(np.int32)
    a_s = rng.uniform(1e-3, 1e-2, M).astype(np.float32)
    w_s = rng.uniform(1e-3, 3e-3, N).astype(np.float32)
    y = _epilogue(L, acc, a_s, w_s)
    R = (rng.standard_normal((M, N)) * np.abs(y) * 2).astype(np.float16)
    G = (rng.standard_normal((M // Lg, N)) * 2).astype(np.float16)
    got = _epilogue(L, acc, a_s, w_s, R=R, G=G, Lg=Lg)
    expect, single = [], 0
    for m in range(M):
        for n in range(N):
            r, g, yv = _fr(R[m, n]), _fr(G[m // Lg, n]), Fraction(float(y[m, n]))
            c = _r16(_r32(r + _r16(_r32(g * yv))))
            expect.append(c)
            single += _r16(_r32(r + _r32(g * yv))) != c
    expect = _as_f64(expect).reshape(M, N)
    if not np.array_equal(got, expect):
        bad.append(f"gated residual: {int((got != expect).sum())} of {M * N} outputs differ")
    if single < M * N // 50:
        bad.append(f"gated residual: only {single} inputs tell a single rounding apart")
    return bad


def rope_failures(L):
    """rms_norm_rope's rotation of each (x0, x1) pair of the normalised row."""
    bad = []
    rng = np.random.default_rng(41)
    Lr, D = 24, 128
    x = rng.standard_normal((Lr, D)).astype(np.float16)
    w = (rng.standard_normal(D) * 0.1).astype(np.float32)

    def norm(freqs):
        y = np.empty((Lr, D), np.uint16)
        L.orc_rms_norm(1, 1, Lr, D, _ptr(x), Lr * D, Lr * D, D, _ptr(w), np.float32(1e-6), _ptr(freqs), 0, _ptr(y))
        return y.view(np.float16).astype(np.float64)

    y = norm(None)
    grid = _fp16_grid(0.25, 8.0)
    f = rng.standard_normal((Lr, D // 2, 4)).astype(np.float32)
    for l in range(Lr):
        for p in range(D // 2):
            x0, x1 = y[l, 2 * p], y[l, 2 * p + 1]
            if x1 == 0:
                continue
            for i in (0, 2):  # second entry of each matrix row chosen so the row's result sits near a midpoint
                h = grid[rng.integers(0, grid.size - 1)]
                mid = (h + float(np.nextafter(np.float16(h), np.float16(np.inf)))) / 2 * (1 if rng.random() < .5 else -1)
                f[l, p, i + 1] = np.float32((mid - float(f[l, p, i]) * x0) / x1)
    got = norm(f)
    expect, sep, once = [], 0, 0
    for l in range(Lr):
        for p in range(D // 2):
            x0, x1 = Fraction(float(y[l, 2 * p])), Fraction(float(y[l, 2 * p + 1]))
            for i in (0, 2):
                m0, m1 = _fr(f[l, p, i]), _fr(f[l, p, i + 1])
                v = _r16(_r32(m1 * x1 + _r32(m0 * x0)))
                expect.append(v)
                sep += _r16(_r32(_r32(m1 * x1) + _r32(m0 * x0))) != v
                once += _r16(m1 * x1 + m0 * x0) != v
    expect = _as_f64(expect).reshape(Lr, D)
    if not np.array_equal(got, expect):
        bad.append(f"rope: {int((got != expect).sum())} of {Lr * D} outputs differ from fp16(fma(m1, x1, fp32(m0 x0)))")
    if sep < Lr * D // 50 or once < Lr * D // 50:
        bad.append(f"rope: only {sep} / {once} inputs tell separate roundings / one exact step apart")
    return bad


def w4a8_epilogue_failures(L):
    """y = fma((float)p_g, gs[n][g], y) in group order, then fp16(y * as (+ bias))."""
    bad = []
    rng = np.random.default_rng(43)
    Gs, M, N = 6, 8, 32
    parts = rng.integers(-2 ** 18, 2 ** 18, (Gs, M, N)).astype(np.int32)
    a_s = rng.uniform(1e-4, 1e-2, M).astype(np.float32)
    gs = rng.uniform(5e-3, 2e-2, (N, Gs)).astype(np.float16)
    bias = rng.standard_normal(N).astype(np.float16)
    for with_bias in (False, True):
        out = np.empty((M, N), np.uint16)
        L.orc_w4a8_epilogue(M, N, Gs, _ptr(parts), _ptr(a_s), _ptr(gs), _ptr(bias) if with_bias else None, _ptr(out))
        got = out.view(np.float16).astype(np.float64)
        expect = []
        for m in range(M):
            for n in range(N):
                yv = Fraction(0)
                for g in range(Gs):
                    yv = _r32(Fraction(int(parts[g, m, n])) * _fr(gs[n, g]) + yv)
                t = _r32(yv * _fr(a_s[m]))
                if with_bias:
                    t = _r32(t + _fr(bias[n]))
                expect.append(_r16(t))
        expect = _as_f64(expect).reshape(M, N)
        if not np.array_equal(got, expect):
            bad.append(f"w4a8 epilogue{' with bias' if with_bias else ''}: {int((got != expect).sum())} outputs differ")
    return bad


CHECKS = {
    "rint": rint_failures,
    "i4": i4_failures,
    "i8_rot": i8_rot_failures,
    "swiglu": swiglu_failures,
    "sigmoid_gate": sigmoid_gate_failures,
    "situ": situ_failures,
    "modulate": modulate_failures,
    "epilogue": epilogue_failures,
    "gated_residual": gated_residual_failures,
    "rope": rope_failures,
    "w4a8_epilogue": w4a8_epilogue_failures,
}
