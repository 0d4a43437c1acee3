"""dot_general on special values, through every dot kernel family.

ggml-cpu (arm64, FPCR.FZ = 0) computes each of its 16 chains with IEEE fused
multiply-adds that keep binary32 subnormals, then a fixed tree of IEEE adds
and the serial tail (StablehloMlx/Kernels/Shaders.lean:69-90).  The matrix
kernels map each chain onto v_mfma_f32_32x32x1_2b_f32 (one fused multiply-add
per output and instruction).  These tests check, bit for bit against the
oracle, that the mapping keeps IEEE semantics where it is easiest to lose:

* subnormal operands, products that underflow into the subnormal range and
  accumulators that cross between normal and subnormal values;
* signed zeros: products that underflow to -0 or +0, so each chain ends with
  the sign of its last product, and the tree adds +0 and -0;
* products and sums that overflow to +-inf, inf - inf and inf * 0;
* NaN operands (quiet and signalling, both signs, random payloads) and
  infinities in chosen rows and columns.

NaN outputs are compared by NaN-ness only.  A NaN's sign and payload are the
platform's: x86's invalid operations return the negative default NaN
0xFFC00000 where arm64 and gfx950 return 0x7FC00000, and which NaN operand
propagates differs between instruction sets.  Every other output must have
the oracle's exact bits.

Each case runs eager and compiled (graph-captured and replayed launches) in
both tail flavours when K % 16 != 0, and asserts which kernel the shape
selected, so a change in the dispatch cannot silently drop a family."""
import zlib

import numpy as np
import pytest

F32_EXP_BIAS = 127


def _bits(sign, biased_exp, frac):
    return ((sign.astype(np.uint32) << 31) | (biased_exp.astype(np.uint32) << 23) |
            frac.astype(np.uint32)).view(np.float32)


def _scaled(rng, n, lo, hi):
    """Random signs and mantissas, exponents uniform in [lo, hi]."""
    e = rng.integers(lo, hi + 1, n) + F32_EXP_BIAS
    assert e.min() >= 1 and e.max() <= 254
    return _bits(rng.integers(0, 2, n), e, rng.integers(0, 1 << 23, n))


def special_values(rng, shape, cls, side, period=8):
    """One operand of a class (side 0: lhs [B, N, K]; side 1: rhs [B, K, M])."""
    n = int(np.prod(shape))
    if cls == "tiny":  # products 2^-160 .. 2^-120: subnormal products and sums
        v = _scaled(rng, n, -80, -60)
    elif cls == "subnormal_in":  # lhs subnormal (or the smallest normals), rhs near 1
        if side == 0:
            e = (rng.random(n) < 0.3).astype(np.int64)  # biased exponent 0 (subnormal) or 1
            v = _bits(rng.integers(0, 2, n), e, rng.integers(0, 1 << 23, n))
        else:
            v = _scaled(rng, n, -2, 3)
    elif cls == "zeros":
        # Products about 2^-160: each fused multiply-add underflows to the
        # sign of its product, so a chain ends with its last product's sign.
        # Every 4th lhs row (counted over the batch) is all negative and every
        # 4th rhs column all positive, so at their crossings every product,
        # chain and tree sum is -0; elsewhere +0 and -0 mix.
        v = _scaled(rng, n, -82, -78)
        z = rng.random(n) < 0.2
        v[z] = np.where(rng.integers(0, 2, int(z.sum())) == 1, np.float32(-0.0), np.float32(0.0))
        v = v.reshape(shape)
        rows = v.reshape(-1, shape[2]) if side == 0 else np.ascontiguousarray(v.transpose(0, 2, 1)).reshape(-1, shape[1])
        rows[::4] = -np.abs(rows[::4]) if side == 0 else np.abs(rows[::4])
        if side == 0:
            return rows.reshape(shape)
        return np.ascontiguousarray(rows.reshape(shape[0], shape[2], shape[1]).transpose(0, 2, 1))
    elif cls == "overflow":  # products up to 2^130: a few overflow, sums overflow, inf - inf
        v = _scaled(rng, n, 40, 64)
    elif cls == "specials":  # N(0,1), with +-0, subnormals, huge values; inf / NaN in chosen rows / columns
        v = rng.standard_normal(n).astype(np.float32)
        r = rng.random(n)
        v[r < 0.05] = np.where(rng.integers(0, 2, int((r < 0.05).sum())) == 1, np.float32(-0.0), np.float32(0.0))
        sub = (r >= 0.05) & (r < 0.07)
        v[sub] = _bits(rng.integers(0, 2, int(sub.sum())), np.zeros(int(sub.sum()), np.int64),
                       rng.integers(1, 1 << 23, int(sub.sum())))
        big = (r >= 0.07) & (r < 0.08)
        v[big] = _scaled(rng, int(big.sum()), 60, 70)
        v = v.reshape(shape)
        # inf and NaN only in every `period`-th row of the lhs (rows counted
        # over the batch) and column of the rhs
        Bx = shape[0]
        rows = v.reshape(-1, shape[2]) if side == 0 else np.ascontiguousarray(v.transpose(0, 2, 1)).reshape(-1, shape[1])
        sel = rows[(1 if side == 0 else 2)::period]
        flat = sel.reshape(-1).copy()
        r2 = rng.random(flat.size)
        inf = r2 < 0.02
        flat[inf] = np.where(rng.integers(0, 2, int(inf.sum())) == 1, np.float32(-np.inf), np.float32(np.inf))
        nan = (r2 >= 0.02) & (r2 < 0.03)
        k = int(nan.sum())
        flat[nan] = _bits(rng.integers(0, 2, k), np.full(k, 255), rng.integers(1, 1 << 23, k))  # quiet and signalling
        rows[(1 if side == 0 else 2)::period] = flat.reshape(sel.shape)
        if side == 0:
            return rows.reshape(shape)
        return np.ascontiguousarray(rows.reshape(Bx, shape[2], shape[1]).transpose(0, 2, 1))
    else:
        raise ValueError(cls)
    return v.reshape(shape)


CLASSES = ["tiny", "subnormal_in", "zeros", "overflow", "specials"]


def dot_layout_module(B, N, K, M, lhs_layout, rhs_layout):
    """A module computing out[b, n, m] = sum_k lhs[b, n, k] rhs[b, k, m] from
    operands stored as:
      lhs "nk": [B, N, K];  "kn": [B, K, N], transposed in the module (read
      along the free dim);
      rhs "km": [B, K, M];  "mk": [B, M, K] (contracted on its last dim);
      "strided": [B, K, 2M], every other column sliced out (no unit stride).
    The batch dim is left out when B == 1."""
    from shlo_hip.configs import t
    bat = B > 1
    pre = (lambda *d: (B,) + d) if bat else (lambda *d: d)
    lines = []
    if lhs_layout == "nk":
        a_in = t(pre(N, K))
        lhs = "%a0"
    else:
        a_in = t(pre(K, N))
        perm = "0, 2, 1" if bat else "1, 0"
        lines.append(f'    %lt = "stablehlo.transpose"(%a0) {{permutation = array<i64: {perm}>}} : ({a_in}) -> {t(pre(N, K))}')
        lhs = "%lt"
    if rhs_layout == "km":
        b_in = t(pre(K, M))
        rhs, rt, rc = "%a1", t(pre(K, M)), 1 if bat else 0
    elif rhs_layout == "mk":
        b_in = t(pre(M, K))
        rhs, rt, rc = "%a1", t(pre(M, K)), 2 if bat else 1
    else:
        b_in = t(pre(K, 2 * M))
        st = "0, 0, 0" if bat else "0, 0"
        li = f"{B}, {K}, {2 * M}" if bat else f"{K}, {2 * M}"
        sd = "1, 1, 2" if bat else "1, 2"
        lines.append(f'    %rs = "stablehlo.slice"(%a1) {{start_indices = array<i64: {st}>, limit_indices = '
                     f'array<i64: {li}>, strides = array<i64: {sd}>}} : ({b_in}) -> {t(pre(K, M))}')
        rhs, rt, rc = "%rs", t(pre(K, M)), 1 if bat else 0
    o = t(pre(N, M))
    lc = 2 if bat else 1
    bd = "lhs_batching_dimensions = [0], rhs_batching_dimensions = [0], " if bat else ""
    dn = f"#stablehlo.dot<{bd}lhs_contracting_dimensions = [{lc}], rhs_contracting_dimensions = [{rc}]>"
    lines.append(f'    %0 = "stablehlo.dot_general"({lhs}, {rhs}) {{dot_dimension_numbers = {dn}}} : '
                 f'({t(pre(N, K))}, {rt}) -> {o}')
    body = "\n".join(lines)
    return (f"module {{\n  func.func public @main(%a0: {a_in}, %a1: {b_in}) -> ({o}) {{\n{body}\n"
            f"    func.return %0 : {o}\n  }}\n}}\n")


def physical(lhs, rhs_bkm, lhs_layout, rhs_layout, rng):
    """The stored operands for dot_layout_module (B == 1 drops the batch dim)."""
    B = lhs.shape[0]
    a = lhs if lhs_layout == "nk" else lhs.transpose(0, 2, 1)
    if rhs_layout == "km":
        b = rhs_bkm
    elif rhs_layout == "mk":
        b = rhs_bkm.transpose(0, 2, 1)
    else:
        Bk, K, M = rhs_bkm.shape
        b = np.empty((Bk, K, 2 * M), np.float32)
        b[:, :, 0::2] = rhs_bkm
        b[:, :, 1::2] = np.float32(np.nan)  # never read: a wrong stride shows up as NaN
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    if B == 1:
        a, b = a[0], b[0]
    return a, b


def same_or_both_nan(got, want):
    g = np.ascontiguousarray(got).view(np.uint32)
    w = np.ascontiguousarray(want).view(np.uint32)
    gn = (g & 0x7FFFFFFF) > 0x7F800000
    wn = (w & 0x7FFFFFFF) > 0x7F800000
    return got.shape == want.shape and np.array_equal(gn, wn) and np.array_equal(g[~gn], w[~wn])


# (name, lhs layout, rhs layout, B, N, K, M, the kernel the shape selects)
CASES = [
    ("direct8_colquad", "nk", "km", 1, 64, 640, 64, "dot_mfma8d_k<RowVecB,ColQuadB,128,8>"),
    ("direct8_rowvec_kc128", "nk", "mk", 1, 64, 640, 128, "dot_mfma8d_k<RowVecB,RowVecB,128,8>"),
    ("direct8_rowvec_kc64", "nk", "mk", 1, 128, 576, 64, "dot_mfma8d_k<RowVecB,RowVecB,64,8>"),
    ("direct4_colquad", "nk", "km", 1, 64, 256, 128, "dot_mfma8d_k<RowVecB,ColQuadB,64,4>"),
    ("direct4_rowvec_batched", "nk", "mk", 3, 64, 64, 64, "dot_mfma8d_k<RowVecB,RowVecB,64,4>"),
    ("staged_rowvec_colquad", "nk", "km", 1, 40, 260, 64, "dot_mfma8_k<RowVec,ColQuad>"),
    ("staged_rowvec_colvec", "nk", "km", 1, 40, 260, 66, "dot_mfma8_k<RowVec,ColVec>"),
    ("staged_scalar_colquad", "nk", "km", 1, 33, 37, 68, "dot_mfma8_k<Scalar,ColQuad>"),
    ("staged_colquad_rowvec", "kn", "mk", 1, 68, 40, 36, "dot_mfma8_k<ColQuad,RowVec>"),
    ("staged_colvec_scalar", "kn", "strided", 1, 35, 45, 30, "dot_mfma8_k<ColVec,Scalar>"),
    ("staged_rowvec_scalar", "nk", "strided", 2, 70, 44, 70, "dot_mfma8_k<RowVec,Scalar>"),
    ("staged_colquadB_rowvecB", "kn", "mk", 1, 64, 136, 64, "dot_mfma8_k<ColQuadB,RowVecB>"),
    ("staged_colquadB_colquadB", "kn", "km", 1, 64, 256, 128, "dot_mfma8_k<ColQuadB,ColQuadB>"),
    # Whole stages of blocks plus a tail (K % 16 != 0): the direct kernel runs
    # the serial tail in its store.
    ("direct_with_tail_colquad", "nk", "km", 1, 64, 132, 64, "dot_mfma8d_k<RowVecB,ColQuadB,64,4>"),
    ("direct_with_tail_rowvec", "nk", "mk", 1, 64, 140, 128, "dot_mfma8d_k<RowVecB,RowVecB,64,4>"),
    # Large products the direct kernel cannot read in place run on padded
    # copies (rows 4-float aligned, row counts multiples of 64): an unaligned
    # K = 263 lhs, a 263-wide rhs, edge tiles in both dims, a batch.
    ("padded_lhs_k263", "nk", "km", 1, 1024, 263, 512, "dot_mfma8d_k<RowVecB,ColQuadB,64,4>"),
    ("padded_rhs_m263", "nk", "km", 1, 1024, 512, 263, "dot_mfma8d_k<RowVecB,ColQuadB,64,4>"),
    ("padded_edges_rowvec", "nk", "mk", 1, 210, 640, 1000, "dot_mfma8d_k<RowVecB,RowVecB,128,8>"),
    ("padded_batched", "nk", "km", 3, 100, 270, 1800, "dot_mfma8d_k<RowVecB,ColQuadB,64,4>"),
    ("one_thread_per_output", "nk", "km", 65536, 1, 37, 2, "dot_ggml_simple<"),
]


@pytest.mark.gpu
@pytest.mark.usefixtures("graph_mode")
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_dot_special_values(oracle, case):
    import shlo_hip
    name, ll, rl, B, N, K, M, kernel = case
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    text = dot_layout_module(B, N, K, M, ll, rl)
    mod = shlo_hip.Module(text)
    flavors = (0, 1) if K % 16 else (0,)
    classes = CLASSES if B < 1000 else ["tiny", "zeros", "specials"]
    for cls in classes:
        lhs = special_values(rng, (B, N, K), cls, 0)
        rhs = special_values(rng, (B, K, M), cls, 1)
        a, b = physical(lhs, rhs, ll, rl, rng)
        ins = [shlo_hip.from_numpy(a), shlo_hip.from_numpy(b)]
        rhs_bmk = np.ascontiguousarray(rhs.transpose(0, 2, 1))
        for flavor in flavors:
            want = oracle.dot_general_bnk(lhs, rhs_bmk, flavor)
            if B == 1:
                want = want[0]
            shlo_hip.set_flavor(flavor)
            try:
                for compile in (False, True):
                    got = mod.prepare(0, compile).call(ins)[0].numpy()
                    if not compile:
                        assert shlo_hip.last_dot_kernel().startswith(kernel), (name, shlo_hip.last_dot_kernel())
                    assert same_or_both_nan(got, want), (name, cls, flavor, compile)
            finally:
                shlo_hip.set_flavor(0)


def test_special_classes_reach_their_ranges(oracle):
    """The classes produce what they are meant to (checked on the oracle's
    outputs, so a generator change cannot quietly weaken the GPU test):
    subnormal and -0 outputs, overflow to inf, and NaN from inf - inf."""
    rng = np.random.default_rng(5)
    B, N, K, M = 1, 32, 48, 32

    def out(cls):
        lhs = special_values(rng, (B, N, K), cls, 0)
        rhs = special_values(rng, (B, K, M), cls, 1)
        return oracle.dot_general_bnk(lhs, np.ascontiguousarray(rhs.transpose(0, 2, 1)))[0]

    y = out("tiny")
    u = y.view(np.uint32) & 0x7FFFFFFF
    assert np.any((u > 0) & (u < 0x00800000)) and np.any(u >= 0x00800000)
    y = out("subnormal_in")
    u = y.view(np.uint32) & 0x7FFFFFFF
    assert np.any((u > 0) & (u < 0x00800000))
    y = out("zeros")
    assert np.all(y == 0) and np.any(np.signbit(y)) and np.any(~np.signbit(y))
    y = out("overflow")
    assert np.any(np.isinf(y)) and np.any(np.isnan(y)) and np.any(np.isfinite(y))
    y = out("specials")
    assert np.any(np.isnan(y)) and np.isfinite(y[0, 0]) and np.isnan(y[1::8, :]).mean() > 0.3
