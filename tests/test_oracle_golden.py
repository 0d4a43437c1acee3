"""The oracle against the reference's golden vectors and against mathematics.

The reference's fixtures are the SHA-256 hashes of every input, output and
graph.txt ref/ggml_ref.c writes (evidence/ref-pinned.sha256, ref-stock.sha256,
copied under tests/golden/).  The oracle must regenerate all of them; each check
below also has a planted mistake (made in the oracle, on the CPU) that it
must catch.
"""
import hashlib
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _hashes(flavor, graphs=False):
    """path -> SHA-256 of the reference's in*.f32 / out.f32 files, or of its
    graph.txt files (ggml's graph per case, "ghlo-graph 1") with graphs=True."""
    res = {}
    with open(os.path.join(ROOT, "tests", "golden", f"ref-{flavor}.sha256")) as f:
        for line in f:
            h, p = line.split()
            if p.endswith("graph.txt") == graphs:
                res[p] = h
    return res


def _sha(path):
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def _mismatches(ref_dir, flavor):
    return sorted(p for p, h in _hashes(flavor).items() if _sha(os.path.join(ref_dir, p)) != h)


def test_pinned_fixtures_bit_exact(ref_pinned):
    """Every in*.f32 and out.f32 of the pinned reference build (96 files)."""
    assert len(_hashes("pinned")) == 96
    assert _mismatches(ref_pinned, "pinned") == []


@pytest.mark.parametrize("flavor", ["pinned", "stock"])
def test_graph_descriptions_bit_exact(ref_pinned, ref_stock, flavor):
    """Every case's graph.txt (ggml's graph as contract-ggml-stablehlo's backend
    describes it, ref/ggml_ref.c:94-134): 38 files per flavour, the same in both."""
    ref = ref_pinned if flavor == "pinned" else ref_stock
    want = _hashes(flavor, graphs=True)
    assert len(want) == 38
    assert sorted(p for p, h in want.items() if _sha(os.path.join(ref, p)) != h) == []


def test_graph_description_catches_a_wrong_op_param(ref_pinned):
    """A planted mistake: the GELU_ERF unary op code one off changes the hash."""
    p = os.path.join(ref_pinned, "gelu_erf_small", "graph.txt")
    lines = open(p).read().splitlines()
    w = lines[2].split()
    assert w[2:4] == ["UNARY", "GELU_ERF"]
    w[27] = str(int(w[27]) - 1)
    text = "\n".join(lines[:2] + [" ".join(w)]) + "\n"
    assert hashlib.sha256(text.encode()).hexdigest() != _hashes("pinned", graphs=True)["gelu_erf_small/graph.txt"]


def test_stock_fixtures_bit_exact_except_platform_erff(ref_stock):
    """The stock build differs only where it calls Apple libsystem_m's erff,
    which is closed code and not restated (gelu_erf_kimodo's output)."""
    assert _mismatches(ref_stock, "stock") == ["gelu_erf_kimodo/out.f32"]


def test_flavours_differ_exactly_where_the_reference_says(ref_pinned, ref_stock):
    """evidence/README.md:48-51: the two builds differ on the mul_mat cases with
    a K tail and on gelu_erf_kimodo."""
    hp, hs = _hashes("pinned"), _hashes("stock")
    differ = sorted(p for p in hp if hp[p] != hs[p])
    assert differ == ["gelu_erf_kimodo/out.f32", "mul_mat_body_in/out.f32", "mul_mat_heading/out.f32",
                      "mul_mat_k2/out.f32", "mul_mat_root_in/out.f32", "mul_mat_small/out.f32"]
    ours = sorted(p for p in hp if p != "gelu_erf_kimodo/out.f32"
                  and _sha(os.path.join(ref_pinned, p)) != _sha(os.path.join(ref_stock, p)))
    assert ours == [p for p in differ if p != "gelu_erf_kimodo/out.f32"]


def _case_io(ref, name):
    meta = {}
    with open(os.path.join(ref, name, "meta.txt")) as f:
        for line in f:
            w = line.split()
            meta[w[0]] = [int(x) for x in w[1:]]
    rd = lambda n: np.fromfile(os.path.join(ref, name, f"{n}.f32"), dtype=np.float32)
    return meta, rd


@pytest.mark.parametrize("tail", [2])
def test_planted_dot_order_changes_hashes(oracle, ref_pinned, tail):
    """Planted: the dot product as a plain sequential sum must miss the hash."""
    meta, rd = _case_io(ref_pinned, "mul_mat_qkv")
    K, M, _, _ = meta["in0"]
    _, R, B, _ = meta["in1"]
    y = oracle.mul_mat(rd("in0"), rd("in1"), K, M, R * B, R, 0, tail)
    assert hashlib.sha256(y.tobytes()).hexdigest() != _hashes("pinned")["mul_mat_qkv/out.f32"]


def test_planted_softmax_float_sum_changes_hash(oracle, ref_pinned):
    meta, rd = _case_io(ref_pinned, "soft_max_kimodo")
    y = oracle.soft_max(rd("in0").reshape(352, 352), float_sum=True)
    assert hashlib.sha256(y.tobytes()).hexdigest() != _hashes("pinned")["soft_max_kimodo/out.f32"]


def test_planted_gelu_tanh_changes_hash(oracle, ref_pinned):
    meta, rd = _case_io(ref_pinned, "gelu_erf_kimodo")
    y = oracle.gelu_erf(rd("in0"), tanh_form=True)
    assert hashlib.sha256(y.tobytes()).hexdigest() != _hashes("pinned")["gelu_erf_kimodo/out.f32"]


def test_dot_within_the_textbook_error_bound(oracle):
    """|dot - exact| <= gamma_K * sum|w x| for any summation order (Higham 3.1)."""
    rng = np.random.default_rng(0)
    for K in (1, 7, 16, 33, 257, 1024):
        w = rng.standard_normal(K).astype(np.float32)
        x = rng.standard_normal(K).astype(np.float32)
        exact = float(np.dot(w.astype(np.float64), x.astype(np.float64)))
        bound = K * 2.0 ** -24 / (1 - K * 2.0 ** -24) * float(np.abs(w.astype(np.float64) * x).sum())
        for tail in (0, 1, 2):
            assert abs(float(oracle.vec_dot(w, x, tail)) - exact) <= bound + 1e-45


def test_dot_exact_on_integers(oracle):
    """Small integers: every partial sum is exact, so every order gives the true dot."""
    rng = np.random.default_rng(1)
    for K in (5, 16, 37, 300):
        w = rng.integers(-8, 8, K).astype(np.float32)
        x = rng.integers(-8, 8, K).astype(np.float32)
        assert float(oracle.vec_dot(w, x)) == float(np.dot(w.astype(np.int64), x.astype(np.int64)))


def test_dot_block_order_is_not_sequential(oracle):
    """A case where ggml's 16-accumulator order and a sequential sum differ:
    1 at lane 0, then 2^25 at lane 1, then -2^25 at lane 2 ... the per-lane
    accumulators keep the 1, a sequential sum loses it."""
    w = np.zeros(32, np.float32)
    x = np.ones(32, np.float32)
    w[0], w[1], w[16] = 2.0 ** 25, 1.0, -(2.0 ** 25)
    # lane 0: fma(-2^25, 1, 2^25) = 0; lane 1: 1; so the tree gives 1, while a
    # sequential sum rounds 2^25 + 1 back to 2^25 and ends at 0.
    seq = np.float32(0)
    for i in range(32):
        seq = np.float32(seq + np.float32(w[i] * x[i]))
    got = oracle.vec_dot(w, x)
    assert float(got) == 1.0 and float(seq) == 0.0


def test_ggml_v_expf_close_to_exp(oracle):
    """ggml_v_expf is within a few ulp of exp over its range; exact at 0; -inf -> +0."""
    xs = np.linspace(-87, 88, 20001, dtype=np.float32)
    for x in xs[::7]:
        got = oracle.ggml_v_expf(x)
        ref = np.float32(np.exp(np.float64(x)))
        ulps = abs(int(np.float32(got).view(np.int32)) - int(ref.view(np.int32)))
        assert ulps <= 2, (x, got, ref)
    assert oracle.ggml_v_expf(0.0) == 1.0
    assert oracle.ggml_v_expf(-np.inf) == 0.0 and not np.signbit(oracle.ggml_v_expf(-np.inf))


def test_expf_erff_correctly_rounded_samples(oracle):
    """CR expf/erff against float64 libm on values where the double result is
    far from a binary32 rounding boundary (where RN(double) must equal CR)."""
    rng = np.random.default_rng(2)
    xs = rng.uniform(-20, 20, 20000).astype(np.float32)
    import math
    for x in xs:
        for f, ref in ((oracle.erff_cr, math.erf), (oracle.expf_cr, math.exp)):
            d = ref(float(x))
            if not math.isfinite(d) or d == 0:
                continue
            r = np.float32(d)
            # distance of d from the binary32 midpoints around r, in units of r's ulp
            up = np.nextafter(r, np.float32(np.inf))
            dn = np.nextafter(r, np.float32(-np.inf))
            mid_gap = min(abs(d - (float(r) + float(up)) / 2), abs(d - (float(r) + float(dn)) / 2))
            if mid_gap > 1e-9 * abs(d):
                assert f(x) == r, (f, x)


def test_erff_chunks_against_mpfr_fixture(oracle):
    """Three 2^24-input chunks of the exhaustive fixture (MPFR-decided) and a
    planted shift by one input that must miss."""
    want = oracle.golden_chunks()
    for c in (0x3F, 0x40, 0xBE):
        base = c << 24
        got = oracle.erff_range(base, 1 << 24)
        assert oracle.checksum_words(got, base) == want[c]
        if c == 0x3F:
            shifted = oracle.erff_range(base + 1, 1 << 24)
            assert oracle.checksum_words(shifted, base) != want[c]


def test_softmax_and_norm_invariants(oracle):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 256)) * 4).astype(np.float32)
    y = oracle.soft_max(x)
    assert np.all(y >= 0) and np.allclose(y.sum(-1, dtype=np.float64), 1.0, atol=1e-5)
    z = oracle.norm(x)
    assert np.allclose(z.mean(-1), 0, atol=1e-5) and np.allclose(z.var(-1), 1, atol=1e-3)
    # causal mask: -inf columns give exactly +0
    m = np.triu(np.ones((64, 256), bool), 1)
    y = oracle.soft_max(np.where(m, np.float32(-np.inf), x))
    assert np.all(y[m] == 0) and not np.any(np.signbit(y[m]))


def test_normal_generator(oracle):
    v, _ = oracle.fill_normal(5, 3.0, 200000)
    assert abs(v.mean()) < 0.03 and abs(v.std() - 3.0) < 0.03
    u, _ = oracle.fill_unif(1, 1.0, 100000)
    assert u.min() >= -1.0 and u.max() < 1.0
