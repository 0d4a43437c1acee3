"""The softmax denominator's exactness tests, checked on the CPU.

ggml_vec_soft_max_f32 adds the rows' binary32 group parts (all >= 0) to a
binary64 sum strictly in order.  The GPU kernel shortens that chain wherever
no addition in it can round: for a run s + p_1 + ... + p_n whose values are
all multiples of u (the smallest ulp among s and the nonzero parts), a
computed total t <= (1 - 2^-20) 2^53 u proves the exact total below 2^53 u,
and then every partial sum in every order is exact.  It applies the test to
the whole row first (a wave's tree sum), then to 16-part segments walked in
order, adding a failing segment's parts one by one.

The final (float)(1.0/S) hides almost every binary64 difference, so the
claims are checked here at the binary64 level: over random and adversarial
part arrays (wide exponent spreads, subnormals, zeros, totals at the
threshold), a row that passes has chain == tree in every lane's order, and
the segment walk equals the in-order chain on every array, passing or not.
"""
import numpy as np

LANES = 64


def part_ulp_exp(parts):
    bits = np.asarray(parts, np.float32).view(np.uint32) & 0x7FFFFFFF
    e = (bits >> 23).astype(np.int64)
    return np.where(bits == 0, 255, np.maximum(e, 1))


def sum_ulp_exp(s):
    """ulp(s) = 2^(D - 1075) = 2^(e - 150) for exponent field D: e = D - 925."""
    return int(np.float64(s).view(np.uint64) >> np.uint64(52)) - 925 if s > 0 else 255


def limit(e):
    """(1 - 2^-20) 2^53 u for u = 2^(e - 150), from its bits as the kernel
    builds it: exponent field e + 925, the top 19 fraction bits set."""
    return np.uint64(((int(e) + 925) << 52) | (((1 << 19) - 1) << 33)).view(np.float64)


def limit_of_sum(s):
    """limit(sum_ulp_exp(s)) as the kernel builds it from s's high word:
    (hi & 0xFFF00000) | 0x000FFFFE, low word zero."""
    hi = int(np.float64(s).view(np.uint64) >> np.uint64(32))
    return np.uint64(((hi & 0xFFF00000) | 0x000FFFFE) << 32).view(np.float64)


def chain(parts):
    s = 0.0
    for p in np.asarray(parts, np.float32).astype(np.float64):
        s = s + p
    return s


def wave_sums(parts):
    """Each lane's sum of its parts (g = lane + 64 j, ascending j), then the
    xor butterfly over 32, 16, ..., 1: the sum every lane ends with."""
    ls = np.zeros(LANES)
    for g, p in enumerate(parts):
        ls[g % LANES] = ls[g % LANES] + np.float64(p)
    for o in (32, 16, 8, 4, 2, 1):
        ls = ls + ls[np.arange(LANES) ^ o]
    return ls


def row16_sum(seg):
    """The kernel's DPP grouping over one 16-lane row: quad_perm [1,0,3,2],
    quad_perm [2,3,0,1], row_half_mirror (i <-> 7 - i in each half), row_mirror."""
    v = np.zeros(16)
    v[:len(seg)] = np.asarray(seg, np.float32).astype(np.float64)
    i = np.arange(16)
    for src in (i ^ 1, i ^ 2, (i & 8) | (7 - (i & 7)), 15 - i):
        v = v + v[src]
    return v[0]


def walk(parts):
    """The kernel's order for a row that fails the whole-row test."""
    s = 0.0
    fast = slow = 0
    for q in range(0, len(parts), 16):
        seg = parts[q:q + 16]
        t = s + row16_sum(seg)
        if t <= limit(int(part_ulp_exp(seg).min())) and (s == 0.0 or t <= limit_of_sum(s)):
            s, fast = t, fast + 1
        else:
            slow += 1
            for p in np.asarray(seg, np.float32).astype(np.float64):
                s = s + p
    return s, fast, slow


def check(parts):
    """Both paths against the in-order chain; returns (row test passed,
    the chain rounds somewhere (differs from the tree sum), walk stats)."""
    parts = np.asarray(parts, np.float32)
    le = int(part_ulp_exp(parts).min()) if len(parts) else 255
    t = wave_sums(parts)
    passed = t <= limit(le)
    assert passed.all() or not passed.any(), "the test must be wave-uniform"
    c = chain(parts)
    if passed[0]:
        assert np.all(t.view(np.uint64) == np.float64(c).view(np.uint64)), (c, t[0])
    w, fast, slow = walk(parts)
    assert np.float64(w).view(np.uint64) == np.float64(c).view(np.uint64), (w, c)
    return bool(passed[0]), c != t[0], fast, slow


def inv_of(x):
    """(float)(1.0 / x) for a binary64 x: IEEE division, then round to nearest."""
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.float32(np.float64(1.0) / np.float64(x))


def kernel_inv(parts):
    """The kernel's decision for a row's inv, and which path gave it."""
    parts = np.asarray(parts, np.float32)
    le = int(part_ulp_exp(parts).min()) if len(parts) else 255
    t = wave_sums(parts)[0]
    if t <= limit(le):
        return inv_of(t), "exact"
    d = t * 2.0 ** -40
    lo, hi = inv_of(t + d), inv_of(t - d)
    if lo == hi:
        return lo, "interval"
    return inv_of(walk(parts)[0]), "walk"


def near_boundary(offset, count, k0=1 << 21, k1=3 << 21):
    """Floats P = 1 + k 2^-23 whose S = P + offset has (float)(1/x) differing
    at the two ends of S (1 -+ 2^-40): 1/S within about 2^-40 of a binary32
    rounding boundary."""
    k = np.arange(k0, k1, dtype=np.int64)
    P = 1.0 + k * 2.0 ** -23
    S = P + offset
    d = S * 2.0 ** -40
    with np.errstate(divide="ignore"):
        hit = (1.0 / (S + d)).astype(np.float32) != (1.0 / (S - d)).astype(np.float32)
    return P[hit][:count].astype(np.float32)


def random_parts(rng, n, spread):
    """Parts like exp(x - max) group sums: values 2^-spread .. 4, a few zeros."""
    x = rng.uniform(-spread, 2.0, n)
    p = np.exp2(x).astype(np.float32)
    p[rng.random(n) < 0.05] = 0.0
    return p


def test_random_rows():
    rng = np.random.default_rng(5)
    n_pass = n_fail_rounded = fast = slow = 0
    for _ in range(1500):
        n = int(rng.choice([4, 63, 256, 1027]))
        spread = float(rng.uniform(0, 80))
        passed, differs, f, s = check(random_parts(rng, n, spread))
        n_pass += passed
        if not passed:
            n_fail_rounded += differs
            fast, slow = fast + f, slow + s
    assert n_pass > 300 and n_fail_rounded > 100, (n_pass, n_fail_rounded)
    assert fast > 300 and slow > 1000, (fast, slow)


def test_softmax_like_rows():
    """Rows shaped like a causal softmax over N(0, 4) logits: the row test
    fails on a few, and most of their segments still pass."""
    rng = np.random.default_rng(8)
    fails = fast = slow = 0
    for _ in range(400):
        x = rng.normal(0, 4, 1024).astype(np.float32)
        e = np.exp(x - x.max()).astype(np.float32).reshape(256, 4)
        parts = ((e[:, 0] + e[:, 1]) + (e[:, 2] + e[:, 3])).astype(np.float32)
        passed, _, f, s = check(parts)
        if not passed:
            fails, fast, slow = fails + 1, fast + f, slow + s
    assert fails > 0 and fast > slow, (fails, fast, slow)


def test_subnormal_and_zero_parts():
    rng = np.random.default_rng(6)
    for n in (1, 5, 64, 300):
        sub = (rng.integers(1, 1 << 23, n).astype(np.uint32)).view(np.float32)  # subnormal parts
        check(sub)
        mixed = sub.copy()
        mixed[0] = np.float32(1.0)
        passed, _, _, _ = check(mixed)
        assert passed == (n == 1)  # 1 next to multiples of 2^-149 needs 150 bits
        check(np.zeros(n, np.float32))


def test_totals_at_the_threshold():
    """One part of ulp u = 2^-40 (p = 2^-17) beside parts of 1.0: the row
    test passes while the total stays below 2^53 u = 2^13 and fails from there."""
    small = np.float32(2.0 ** -17)
    for k in (4095, 4096, 8190, 8191, 8192, 8200):
        parts = np.concatenate([np.ones(k, np.float32), [small]]).astype(np.float32)
        passed, _, _, _ = check(parts)
        assert passed == (k + 2.0 ** -17 < 2.0 ** 13), (k, passed)
    # at 2^53 u the chain really rounds: 2^13 + 2^-40 is not a binary64 number
    parts = np.concatenate([np.full(8192, 1.0, np.float32), [np.float32(2.0 ** -40)]]).astype(np.float32)
    passed, _, _, _ = check(parts)
    assert not passed and chain(parts) == 8192.0


def test_ulp_exponents_and_limit():
    p = np.array([0.0, 1.0, 1.5, 2.0 ** -126, 2.0 ** -149, 3.9999998], np.float32)
    assert list(part_ulp_exp(p)) == [255, 127, 127, 1, 1, 128]
    # ulp(1.0f) = 2^-23 = 2^(127 - 150); the binary64 1.0 has ulp 2^-52 = 2^(98 - 150)
    assert sum_ulp_exp(1.0) == 98 and sum_ulp_exp(0.0) == 255 and sum_ulp_exp(3.0) == 99
    assert limit(127) == 2.0 ** 30 * (1 - 2.0 ** -20)
    rng = np.random.default_rng(9)
    for v in np.concatenate([rng.uniform(0, 5000, 200), 2.0 ** rng.integers(-140, 40, 200), [1.0, 2.0 ** -149]]):
        assert limit_of_sum(v) == limit(sum_ulp_exp(v)), v
    assert limit(1) == 2.0 ** -96 * (1 - 2.0 ** -20)


def test_interval_and_walk_paths():
    """Rows whose 1/S lies within 2^-40 of a binary32 rounding boundary fail
    the interval test and take the walk; every path's inv equals
    (float)(1.0 / in-order sum).  Parts: one P in [1, 2) first, then tiny
    parts (the chain absorbs them: S = P), or moderate parts and one tiny part
    last (S = P + 254 m, the last segment walked part by part)."""
    tiny = np.float32(2.0 ** -100)
    m = np.float32(2.0 ** -20)
    paths = {}
    for P in near_boundary(0.0, 20):
        parts = np.concatenate([[P], np.full(255, tiny, np.float32)]).astype(np.float32)
        inv, path = kernel_inv(parts)
        assert inv == inv_of(chain(parts)) and path == "walk", (P, path)
        paths[path] = paths.get(path, 0) + 1
    for P in near_boundary(254 * float(m), 20):
        parts = np.concatenate([[P], np.full(254, m, np.float32), [tiny]]).astype(np.float32)
        assert chain(parts) == float(P) + 254 * float(m)
        inv, path = kernel_inv(parts)
        assert inv == inv_of(chain(parts)) and path == "walk", (P, path)
        _, fast, slow = walk(parts)
        assert fast == 15 and slow == 1
    rng = np.random.default_rng(10)
    for _ in range(800):
        parts = random_parts(rng, int(rng.choice([64, 256, 1027])), float(rng.uniform(0, 120)))
        inv, path = kernel_inv(parts)
        assert inv == inv_of(chain(parts)), path
        paths[path] = paths.get(path, 0) + 1
    assert paths.get("exact", 0) > 100 and paths.get("interval", 0) > 100, paths


def row16_sums(parts):
    """The fused attention kernel's order for rows of 16 n groups on 16 lanes:
    lane i sums the parts g = i + 16 j in ascending j, then the row's DPP
    grouping (row16_sum's four steps) over the 16 lane sums."""
    ls = np.zeros(16)
    for g, p in enumerate(np.asarray(parts, np.float32)):
        ls[g % 16] = ls[g % 16] + np.float64(p)
    i = np.arange(16)
    for src in (i ^ 1, i ^ 2, (i & 8) | (7 - (i & 7)), 15 - i):
        ls = ls + ls[src]
    assert np.all(ls == ls[0])
    return ls[0]


def kernel_inv16(parts):
    parts = np.asarray(parts, np.float32)
    le = int(part_ulp_exp(parts).min()) if len(parts) else 255
    t = row16_sums(parts)
    if t <= limit(le):
        assert np.float64(t).view(np.uint64) == np.float64(chain(parts)).view(np.uint64)
        return inv_of(t), "exact"
    d = t * 2.0 ** -40
    lo, hi = inv_of(t + d), inv_of(t - d)
    if lo == hi:
        return lo, "interval"
    return inv_of(walk(parts)[0]), "walk"


def test_sixteen_lane_rows():
    """The 16-lane order (rows of 256 and 512 columns in the fused attention
    kernel): a row that passes has tree == chain, and every path's inv is
    (float)(1.0 / in-order sum), over random, softmax-like and walk rows."""
    rng = np.random.default_rng(11)
    paths = {}
    for _ in range(1200):
        n = int(rng.choice([64, 128]))
        parts = random_parts(rng, n, float(rng.uniform(0, 120)))
        inv, path = kernel_inv16(parts)
        assert inv == inv_of(chain(parts)), path
        paths[path] = paths.get(path, 0) + 1
    for _ in range(200):
        x = rng.normal(0, 4, 512).astype(np.float32)
        e = np.exp(x - x.max()).astype(np.float32).reshape(128, 4)
        parts = ((e[:, 0] + e[:, 1]) + (e[:, 2] + e[:, 3])).astype(np.float32)
        inv, path = kernel_inv16(parts)
        assert inv == inv_of(chain(parts)), path
        paths[path] = paths.get(path, 0) + 1
    tiny = np.float32(2.0 ** -100)
    for n in (64, 128):
        for P in near_boundary(0.0, 10):
            parts = np.concatenate([[P], np.full(n - 1, tiny, np.float32)]).astype(np.float32)
            inv, path = kernel_inv16(parts)
            assert inv == inv_of(chain(parts)) and path == "walk", (P, path)
            paths[path] = paths.get(path, 0) + 1
    assert all(paths.get(k, 0) > 15 for k in ("exact", "interval", "walk")), paths
