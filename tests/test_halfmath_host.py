"""CPU pins of the oracle's canonical half arithmetic (oracle/halfmath.h),
which the fp16 rasterizer's kernels share: add / sub / mul / div against
numpy's float16 arithmetic (correctly rounded), fma against exact rational
arithmetic, exp2 against a 40-digit decimal evaluation, the directed
conversion against its definition, all with subnormal, overflow and signed
zero cases; and the method the device uses to round exact double sums to
half (through float rounded toward odd)."""
import decimal
from fractions import Fraction

import numpy as np


def _halves(rng, n):
    """Random half bit patterns, NaN / inf excluded, subnormals included."""
    b = rng.integers(0, 1 << 16, n).astype(np.uint16)
    return b[(b & 0x7c00) != 0x7c00]


def _f(bits):
    return bits.view(np.float16).astype(np.float64)


def test_basic_ops_correctly_rounded(orc):
    rng = np.random.default_rng(0)
    a = _halves(rng, 300000)
    b = _halves(rng, a.size)
    m = min(a.size, b.size)
    a, b = a[:m], b[:m]
    ha, hb = a.view(np.float16), b.view(np.float16)
    with np.errstate(all="ignore"):
        for op, want in ((3, ha * hb), (4, ha + hb), (9, ha - hb), (5, ha / hb)):
            got = orc.half_op(op, a, b)
            w = want.view(np.uint16)
            ok = (got == w) | (np.isnan(want) & np.isnan(got.view(np.float16)))
            assert ok.all(), (op, np.nonzero(~ok)[0][:5])


def _round_fraction_to_half(x: Fraction) -> float:
    """Correct RNE rounding of a rational to binary16 (finite results)."""
    if x == 0:
        return 0.0
    neg = x < 0
    a = -x if neg else x
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    qe = max(e - 10, -24)
    q = Fraction(2) ** qe
    m = a / q
    fl = m.numerator // m.denominator
    frac = m - fl
    up = frac > Fraction(1, 2) or (frac == Fraction(1, 2) and fl % 2 == 1)
    r = float((fl + up) * q)
    if r > 65504:
        r = float("inf")
    return -r if neg else r


def test_fma_correctly_rounded(orc):
    rng = np.random.default_rng(1)
    n = 60000
    a, b, c = _halves(rng, n)[:20000], _halves(rng, n)[:20000], _halves(rng, n)[:20000]
    # products near sums and halfway cases: c = -round(a b) plus tiny offsets
    with np.errstate(over="ignore"):
        ab = (a.view(np.float16).astype(np.float32) * b.view(np.float16).astype(np.float32)).astype(np.float16)
    near = np.isfinite(ab[::3])
    c[::3] = np.where(near, (-ab[::3]).view(np.uint16), c[::3])
    got = orc.half_op(2, a, b, c).view(np.float16).astype(np.float64)
    for i in range(a.size):
        x = Fraction(float(_f(a[i:i + 1])[0])) * Fraction(float(_f(b[i:i + 1])[0])) + Fraction(float(_f(c[i:i + 1])[0]))
        want = _round_fraction_to_half(x)
        if np.isinf(want):
            assert np.isinf(got[i]) and np.sign(got[i]) == np.sign(want), i
            continue
        if want == 0 and got[i] == 0:
            continue
        assert got[i] == want, (i, a[i], b[i], c[i], got[i], want)


def test_exp2_correctly_rounded_all_inputs(orc):
    x = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = x[(x & 0x7c00) != 0x7c00]
    got = orc.half_op(0, x)
    decimal.getcontext().prec = 40
    ln2 = decimal.Decimal(2).ln()
    fx = _f(x)
    for i in range(x.size):
        v = float(fx[i])
        if v > 16.0 or v < -25.0:   # overflow / underflow to zero, checked below
            continue
        e = (decimal.Decimal(v) * ln2).exp()
        want = _round_fraction_to_half(Fraction(e))
        assert float(got[i:i + 1].view(np.float16)[0]) == want, (v, got[i], want)
    assert np.all(got[fx > 16.0].view(np.float16) == np.inf)
    assert np.all(got[fx < -25.0].view(np.float16) == 0)


def test_directed_conversion(orc):
    rng = np.random.default_rng(2)
    f = np.concatenate([rng.normal(0, 1, 50000), rng.uniform(-70000, 70000, 20000), rng.uniform(-1e-5, 1e-5, 20000),
                        [0.0, -0.0, 65504.0, 65519.0, 65520.0, -65520.0, 6e-8, -6e-8]]).astype(np.float32)
    rn = orc.half_op(7, f)
    with np.errstate(over="ignore"):
        assert np.array_equal(rn, f.astype(np.float16).view(np.uint16))
    rd = orc.half_op(8, f).view(np.float16).astype(np.float64)
    assert np.all(rd <= f.astype(np.float64))
    # the largest half not above f: the next half up exceeds f
    nxt = np.nextafter(rd.astype(np.float16), np.float16(np.inf)).astype(np.float64)
    assert np.all((nxt > f) | np.isinf(rd))


def _round_to_odd_f32(s):
    """Round float64 values to float32 toward odd: truncate toward zero, then
    set the last bit when inexact (the device's half_of_double_sum)."""
    f = s.astype(np.float32)
    inexact = f.astype(np.float64) != s
    u = f.view(np.uint32).copy()
    away = np.abs(f.astype(np.float64)) > np.abs(s)
    u[inexact & away] -= 1
    u[inexact] |= 1
    return u.view(np.float32)


def test_double_sum_rounding_method():
    """The method of half_of_double_sum (tinygs_amd/csrc/halfmath.h): round
    an exact double sum of halves to float toward odd, then to nearest half,
    equals the direct nearest half (numpy's double -> half conversion,
    correctly rounded), while rounding to nearest float first does not:
    near half midpoints (m + k 2^-24, |k| <= 40, at every binade a sum of
    halves can reach) and on random multiples of 2^-24."""
    rng = np.random.default_rng(5)
    e = rng.integers(-13, 16, 100000)
    q = rng.integers(1 << 10, 1 << 11, 100000)
    mid = (2 * q + 1).astype(np.float64) * np.exp2(e - 11.0)
    k = rng.integers(-40, 41, 100000)
    near = np.concatenate([mid + k * 2.0 ** -24, -(mid + k * 2.0 ** -24), mid])
    rand = (rng.integers(-(1 << 52), 1 << 52, 1 << 18) >> rng.integers(0, 52, 1 << 18)).astype(np.float64)
    s = np.concatenate([near, rand * 2.0 ** -24, [0.0, 2.0 ** -24, 65504.0, 65519.0, 65520.0, -65520.0]])
    with np.errstate(over="ignore"):
        want = s.astype(np.float16).view(np.uint16)
        odd = _round_to_odd_f32(s).astype(np.float16).view(np.uint16)
        nearest = s.astype(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(odd, want)
    assert np.count_nonzero(nearest != want) > 100   # the double rounding it avoids
