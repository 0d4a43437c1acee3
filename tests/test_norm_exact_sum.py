"""norm's mean: the kernel's three ways to ggml's in-order binary64 sum, on the CPU.

ggml norm adds the row's elements (any signs) to a binary64 sum in element
order, then mean = (float)sum / (float)cols.  The GPU kernel (one wave per
row, lane l holding the elements of groups g = l + 64 j, a butterfly
reduction) takes the tree sum t when a <= (1 - 2^-20) 2^53 u (a = the tree sum
of |x_i|, u = the smallest ulp among the nonzero x_i), accepts the mean the
interval t -+ a (cols + 4 J + 8) 2^-52 fixes when both ends agree (J groups
per lane; twice the bound on |chain - t|), and otherwise adds the elements in
order.  These tests restate that decision and check it against
the in-order chain over random, cancelling, wide-spread and constructed rows:
a row the exactness test passes has t equal to the chain bit for bit, and a
row the interval passes has the chain's mean.  (The variance's sum of
non-negative parts shares softmax's code, checked in test_softmax_exact_sum.)
"""
import numpy as np

from test_softmax_exact_sum import limit, part_ulp_exp

LANES = 64
F32 = np.float32


def chain(x):
    s = 0.0
    with np.errstate(all="ignore"):
        for v in np.asarray(x, F32).astype(np.float64):
            s = s + v
    return s


def wave_sums(x):
    """Lane l adds its groups' elements in order, then the xor butterfly."""
    x = np.asarray(x, F32).astype(np.float64)
    ls = np.zeros(LANES)
    la = np.zeros(LANES)
    with np.errstate(all="ignore"):
        for i, v in enumerate(x):
            l = (i // 4) % LANES
            ls[l] = ls[l] + v
            la[l] = la[l] + abs(v)
        for o in (32, 16, 8, 4, 2, 1):
            ls = ls + ls[np.arange(LANES) ^ o]
            la = la + la[np.arange(LANES) ^ o]
    return ls[0], la[0]


def low_bit_exp(s):
    """The biased exponent (2^(e-150)) of the lowest set bit of binary64 s; 255 for 0."""
    b = int(np.float64(s).view(np.uint64)) & 0x7FFFFFFFFFFFFFFF
    if b == 0:
        return 255
    E, m = b >> 52, b & ((1 << 52) - 1)
    sig = (m | (1 << 52)) if E else m
    ctz = (sig & -sig).bit_length() - 1
    return (E if E else 1) - 1075 + ctz + 150


def seg_sums(q):
    """A 16-lane segment's tree sums as the kernel forms them: per lane
    (x + y) + (z + w), then the DPP row reduction."""
    from test_softmax_exact_sum import row16_sum
    q = np.asarray(q, F32).reshape(-1, 4).astype(np.float64)
    with np.errstate(all="ignore"):
        lane = (q[:, 0] + q[:, 1]) + (q[:, 2] + q[:, 3])
        lane_a = (np.abs(q[:, 0]) + np.abs(q[:, 1])) + (np.abs(q[:, 2]) + np.abs(q[:, 3]))
    return row16_sum_d(lane), row16_sum_d(lane_a)


def row16_sum_d(v):
    w = np.zeros(16)
    w[:len(v)] = v
    i = np.arange(16)
    with np.errstate(all="ignore"):
        for src in (i ^ 1, i ^ 2, (i & 8) | (7 - (i & 7)), 15 - i):
            w = w + w[src]
    return w[0]


def walk_mean_sum(x):
    """The kernel's segmented walk: 64 consecutive elements at a time."""
    x = np.asarray(x, F32)
    G = len(x) // 4
    body, tail = x[:4 * G], x[4 * G:]
    s, fast, slow = 0.0, 0, 0
    for q0 in range(0, 4 * G, 64):
        seg = body[q0:q0 + 64]
        ssum, sabs = seg_sums(seg)
        e_min = min(int(part_ulp_exp(seg).min()), low_bit_exp(s))
        with np.errstate(all="ignore"):
            ok = abs(s) + sabs <= limit(e_min)
        if ok:
            s, fast = s + ssum, fast + 1
        else:
            slow += 1
            with np.errstate(all="ignore"):
                for v in seg.astype(np.float64):
                    s = s + v
    with np.errstate(all="ignore"):
        for v in tail.astype(np.float64):
            s = s + v
    return s, fast, slow


def mean_of(s, cols):
    with np.errstate(all="ignore"):
        return F32(F32(s) / F32(cols))


def kernel_mean(x):
    """The kernel's mean and the path that decided it."""
    x = np.asarray(x, F32)
    t, a = wave_sums(x)
    u = int(part_ulp_exp(x).min()) if len(x) else 255
    if a <= limit(u):
        return mean_of(t, len(x)), "exact", t
    J = max(1, -(-(len(x) // 4) // LANES))
    with np.errstate(all="ignore"):
        d = a * ((len(x) + 4 * J + 8) * 2.0 ** -52)
        lo, hi = mean_of(t - d, len(x)), mean_of(t + d, len(x))
    if lo == hi:
        return lo, "interval", t
    return mean_of(walk_mean_sum(x)[0], len(x)), "walk", t


def same(a, b):
    return np.asarray(a, F32).view(np.uint32) == np.asarray(b, F32).view(np.uint32)


def check(x):
    m, path, t = kernel_mean(x)
    c = chain(x)
    if path == "exact":
        assert np.float64(t).view(np.uint64) == np.float64(c).view(np.uint64), (t, c)
    assert same(m, mean_of(c, len(x))), (path, m, mean_of(c, len(x)))
    return path


def test_random_rows():
    rng = np.random.default_rng(11)
    paths = {}
    for _ in range(600):
        cols = int(rng.choice([4, 63, 512, 1024, 4096]))
        x = rng.normal(0, float(rng.uniform(0.01, 100)), cols).astype(F32)
        if rng.random() < 0.5:  # one tiny element: the exactness test fails
            x[rng.integers(cols)] = F32(rng.normal() * 2.0 ** -float(rng.uniform(30, 120)))
        p = check(x)
        paths[p] = paths.get(p, 0) + 1
    assert paths.get("exact", 0) > 100 and paths.get("interval", 0) > 100, paths


def test_cancelling_rows():
    """Rows summing to (nearly) zero: pairs +v, -v with one small remainder."""
    rng = np.random.default_rng(12)
    for _ in range(300):
        v = rng.normal(0, 10, 256).astype(F32)
        x = np.concatenate([v, -v[::-1]]).astype(F32)
        x[rng.integers(512)] += F32(rng.normal() * 1e-3)
        check(x)


def test_wide_spreads_and_subnormals():
    rng = np.random.default_rng(13)
    for _ in range(300):
        cols = int(rng.choice([8, 100, 512]))
        e = rng.uniform(-149, 100, cols)
        x = (np.sign(rng.normal(size=cols)) * np.exp2(e)).astype(F32)
        x[rng.random(cols) < 0.1] = 0.0
        check(x)


def test_constructed_walk_row():
    """1, 2^-53, 2^-24, 2^-53 in lanes 0..3: the chain and the tree round to
    different means, the interval straddles, and the walk gives the chain's."""
    x = np.zeros(512, F32)
    x[0], x[4], x[8], x[12] = 1.0, 2.0 ** -53, 2.0 ** -24, 2.0 ** -53
    m, path, t = kernel_mean(x)
    assert path == "walk"
    assert not same(mean_of(t, 512), mean_of(chain(x), 512))
    assert same(m, mean_of(chain(x), 512))


def test_special_values():
    for bad in (np.nan, np.inf, -np.inf):
        x = np.ones(64, F32)
        x[5] = bad
        m, path, _ = kernel_mean(x)
        assert path == "walk" and np.isnan(m) == np.isnan(mean_of(chain(x), 64))
    x = np.ones(64, F32)
    x[3], x[9] = np.inf, -np.inf
    assert kernel_mean(x)[1] == "walk"
    assert check(np.zeros(16, F32)) == "exact"
    assert check(-np.zeros(16, F32)) == "exact"


def test_segment_walk_equals_chain():
    """The segmented walk's sum equals the in-order chain bit for bit on
    every row, passing segments or not: rows with one tiny element, wide
    exponent spreads, cancellation, and ties built to round."""
    rng = np.random.default_rng(14)
    fast = slow = 0
    rows = []
    for _ in range(300):
        cols = int(rng.choice([64, 512, 1024, 1027]))
        x = rng.normal(0, 1, cols).astype(F32)
        k = int(rng.integers(0, 4))
        if k == 1:
            x[rng.integers(cols)] = F32(rng.normal() * 2.0 ** -float(rng.uniform(30, 140)))
        elif k == 2:
            x = (np.sign(rng.normal(size=cols)) * np.exp2(rng.uniform(-140, 60, cols))).astype(F32)
        elif k == 3:
            x[: cols // 2] = np.round(x[: cols // 2] * 1024) / 1024
            x[cols // 2:] = -x[: cols - cols // 2][::-1]
            x[rng.integers(cols)] = F32(2.0 ** -53)
        rows.append(x)
    walk_row = np.zeros(512, F32)
    walk_row[0], walk_row[4], walk_row[8], walk_row[12] = 1.0, 2.0 ** -53, 2.0 ** -24, 2.0 ** -53
    rows.append(walk_row)
    for x in rows:
        w, f, sl = walk_mean_sum(x)
        c = chain(x)
        assert np.float64(w).view(np.uint64) == np.float64(c).view(np.uint64), (w, c)
        fast, slow = fast + f, slow + sl
    assert fast > 1000 and slow > 50, (fast, slow)
