"""The oracle's binary64 (the generic path's f64 ops) pinned without itself.

The reference computes f64 with integer soft-float kernels
(StablehloMlx/Kernels/SoftFloat.lean): IEEE binary64, round to nearest even,
with arm64's NaN rules.  The oracle restates that on the host's binary64.
Two independent checks pin it:

* exact rational arithmetic (Python's Fraction), rounded once to binary64 by
  float(), and to binary32 by the rounding written out below, on random,
  subnormal, near-overflow and integer operands;
* the special cases SoftFloat.lean states: which NaN propagates, the default
  NaN of invalid operations, signed zeros, floor of negatives, the saturating
  conversion to int64, and the NaN payloads of the conversions."""
import math
import struct
from fractions import Fraction

import numpy as np
import pytest

NAN64 = 0x7FF8000000000000
Q64 = 0x0008000000000000
I64_MAX, I64_MIN = 0x7FFFFFFFFFFFFFFF, 0x8000000000000000


def d(bits):
    return struct.unpack("<d", struct.pack("<Q", bits))[0]


def b(x):
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def one(oracle, op, x, y=0):
    return int(oracle.f64_ew(op, np.array([x], np.uint64), np.array([y], np.uint64))[0])


def test_nan_rules(oracle):
    qa, sb = 0x7FF8000000000123, 0xFFF0000000000456  # a quiet NaN, a negative signalling NaN
    for op in range(4):
        assert one(oracle, op, qa, sb) == qa  # the first NaN operand
        assert one(oracle, op, b(1.5), sb) == sb | Q64  # quieted, sign kept (subtract too)
        assert one(oracle, op, sb, b(2.0)) == sb | Q64
    inf, ninf, z, nz = b(math.inf), b(-math.inf), 0, 1 << 63
    for op, x, y in ((0, inf, ninf), (1, inf, inf), (2, inf, z), (2, nz, inf), (3, z, nz), (3, ninf, inf)):
        assert one(oracle, op, x, y) == NAN64, (op, hex(x), hex(y))
    assert one(oracle, 4, sb) == sb | Q64
    assert one(oracle, 5, qa) == 0 and one(oracle, 5, sb) == 0


def test_signed_zeros_and_floor(oracle):
    nz = 1 << 63
    assert one(oracle, 0, nz, nz) == nz
    assert one(oracle, 0, nz, 0) == 0
    assert one(oracle, 1, b(3.25), b(3.25)) == 0
    assert one(oracle, 1, nz, 0) == nz
    assert one(oracle, 2, b(-1.0), 0) == nz
    assert one(oracle, 3, b(1.0), nz) == b(-math.inf)
    assert one(oracle, 3, b(-1.0), b(math.inf)) == nz
    for x, want in ((-0.0, -0.0), (-0.5, -1.0), (0.5, 0.0), (-1e300, -1e300), (-2.5, -3.0),
                    (2.0 ** 52 + 1, 2.0 ** 52 + 1), (-(2.0 ** -1074), -1.0), (math.inf, math.inf)):
        assert one(oracle, 4, b(x)) == b(want), x


def test_to_int64(oracle):
    cases = [(2.0 ** 63, I64_MAX), (-(2.0 ** 63), I64_MIN), (1e19, I64_MAX), (-1e19, I64_MIN),
             (math.inf, I64_MAX), (-math.inf, I64_MIN), (-0.9, 0), (-1.5, (1 << 64) - 1),
             (2.0 ** 63 - 1024, 2 ** 63 - 1024), (-(2.0 ** 62) - 0.5, (1 << 64) - 2 ** 62), (0.0, 0)]
    for x, want in cases:
        assert one(oracle, 5, b(x)) == want, x


def test_maxmin(oracle):
    nz, q = 1 << 63, 0x7FF8000000000777
    a = np.array([0, nz, 0, nz, q, b(1.0), q, b(-2.0), b(3.0)], np.uint64)
    c = np.array([nz, 0, 0, nz, b(1.0), q | (1 << 63), 0xFFF0000000000001, b(-2.0), b(-3.0)], np.uint64)
    mx = oracle.f64_maxmin(True, a, c)
    mn = oracle.f64_maxmin(False, a, c)
    assert [int(v) for v in mx] == [0, 0, 0, nz, q, q | (1 << 63), q, b(-2.0), b(3.0)]
    assert [int(v) for v in mn] == [nz, nz, 0, nz, q, q | (1 << 63), q, b(-2.0), b(-3.0)]


def test_conversions_special(oracle):
    f = np.array([0x7F800001, 0xFFC00000, 0x00000001, 0x80000000, 0x7F7FFFFF], np.uint32).view(np.float32)
    w = oracle.f64_of_f32(f)
    assert [int(v) for v in w] == [0x7FF0000020000000, 0xFFF8000000000000, b(2.0 ** -149), 1 << 63,
                                   b(float(np.float32(3.4028234663852886e38)))]
    dd = np.array([0x7FF0000000000001, 0xFFF8000000000000, 0x7FF0000020000000, b(2.0 ** 128),
                   b(2.0 ** -150), b(3 * 2.0 ** -151), b((2 - 2.0 ** -24) * 2.0 ** 127),
                   b(-(2.0 ** -149) * 0.75)], np.uint64)
    assert [int(v) for v in oracle.f32_of_f64(dd)] == [0x7FC00000, 0xFFC00000, 0x7FC00001, 0x7F800000,
                                                        0, 1, 0x7F800000, 0x80000001]


def rand_doubles(rng, n):
    kind = rng.integers(0, 5, n)
    bits = rng.integers(0, 1 << 63, n, dtype=np.uint64) | (rng.integers(0, 2, n, dtype=np.uint64) << 63)
    out = bits.copy()
    # subnormals and the smallest normals
    sub = kind == 1
    out[sub] = (bits[sub] & np.uint64(0x801FFFFFFFFFFFFF))
    # near overflow
    big = kind == 2
    out[big] = (bits[big] & np.uint64(0x800FFFFFFFFFFFFF)) | np.uint64(0x7FE0000000000000)
    # small integers and halves
    it = kind == 3
    vals = (rng.integers(-(1 << 20), 1 << 20, int(it.sum())) / 2.0).astype(np.float64)
    out[it] = vals.view(np.uint64)
    # moderate magnitudes
    mid = kind == 4
    out[mid] = (rng.standard_normal(int(mid.sum())) * 1e3).view(np.uint64)
    out = out[(out & np.uint64(0x7FF0000000000000)) != np.uint64(0x7FF0000000000000)]  # finite only
    return out


def exact_round64(q):
    try:
        return b(float(q))
    except OverflowError:
        return b(math.inf if q > 0 else -math.inf)


def round_to_f32_bits(q):
    """Round an exact rational to binary32 (nearest, ties to even, subnormals,
    overflow to infinity), written out independently of any float type."""
    if q == 0:
        return 0
    s = 0x80000000 if q < 0 else 0
    a = abs(q)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)  # subnormal range: fixed quantum 2^-149
    quantum = Fraction(2) ** (e - 23)
    m = a / quantum
    n = math.floor(m)
    r = m - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    if n == 1 << 24:
        n >>= 1
        e += 1
    if e > 127:
        return s | 0x7F800000
    if n < (1 << 23):
        return s | n  # subnormal
    return s | ((e + 127) << 23) | (n - (1 << 23))


def test_arithmetic_against_exact_rationals(oracle):
    rng = np.random.default_rng(11)
    a = rand_doubles(rng, 6000)
    c = rand_doubles(rng, 6000)
    n = min(a.size, c.size)
    a, c = a[:n], c[:n]
    res = [oracle.f64_ew(op, a, c) for op in range(4)]
    fl = oracle.f64_ew(4, a)
    ti = oracle.f64_ew(5, a)
    for i in range(n):
        x, y = Fraction(d(int(a[i]))), Fraction(d(int(c[i])))
        assert int(res[0][i]) == exact_round64(x + y) or (x + y == 0), i
        assert int(res[1][i]) == exact_round64(x - y) or (x - y == 0), i
        assert int(res[2][i]) == exact_round64(x * y) or (x * y == 0), i
        if y != 0:
            assert int(res[3][i]) == exact_round64(x / y) or (x == 0), i
        assert int(fl[i]) == b(float(math.floor(x))) or x == 0 or (x < 0 and math.floor(x) == 0), i
        t = int(x)  # toward zero
        t = max(min(t, 2 ** 63 - 1), -(2 ** 63))
        assert int(ti[i]) == t % (1 << 64), i


def test_narrowing_against_exact_rationals(oracle):
    rng = np.random.default_rng(12)
    e = rng.integers(-160, 130, 20000)
    m = rng.random(20000) + 1.0
    x = (np.sign(rng.standard_normal(20000)) * m * np.exp2(e.astype(np.float64))).astype(np.float64)
    got = oracle.f32_of_f64(x)
    for i in range(x.size):
        assert int(got[i]) == round_to_f32_bits(Fraction(float(x[i]))), x[i]
    f = x.astype(np.float32)
    f = f[np.isfinite(f)]
    w = oracle.f64_of_f32(f)
    assert np.array_equal(w.view(np.float64), f.astype(np.float64))


@pytest.mark.parametrize("planted", [0])
def test_exact_rational_rounding_sanity(planted):
    """The checker's own rounding catches a wrong rounding: a value one
    quarter-ulp above a binary32 midpoint must round up."""
    half = Fraction(1) + Fraction(1, 2 ** 24)
    assert round_to_f32_bits(half) == 0x3F800000  # tie, even
    assert round_to_f32_bits(half + Fraction(1, 2 ** 26)) == 0x3F800001
