"""GPU parity at the measurement configs: dot_general, softmax
with a causal mask and erf-GELU, each eager and hipGraph-compiled, bit for
bit against the oracle; each with its planted wrong lowering."""
import numpy as np
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("graph_mode")]


def dot_module(N, K, M, batch=0):
    """[N,K] x [K,M] (contract [1]/[0]); with batch > 0, [B,N,K] x [B,K,M]."""
    if batch:
        a, b, o = f"tensor<{batch}x{N}x{K}xf32>", f"tensor<{batch}x{K}x{M}xf32>", f"tensor<{batch}x{N}x{M}xf32>"
        dn = ("#stablehlo.dot<lhs_batching_dimensions = [0], rhs_batching_dimensions = [0], "
              "lhs_contracting_dimensions = [2], rhs_contracting_dimensions = [1]>")
    else:
        a, b, o = f"tensor<{N}x{K}xf32>", f"tensor<{K}x{M}xf32>", f"tensor<{N}x{M}xf32>"
        dn = "#stablehlo.dot<lhs_contracting_dimensions = [1], rhs_contracting_dimensions = [0]>"
    return (f"module {{\n  func.func public @main(%a0: {a}, %a1: {b}) -> ({o}) {{\n"
            f'    %0 = "stablehlo.dot_general"(%a0, %a1) {{dot_dimension_numbers = {dn}}} : ({a}, {b}) -> {o}\n'
            f"    func.return %0 : {o}\n  }}\n}}\n")


def custom_call_module(target, attrs, shape):
    t = "tensor<" + "".join(f"{d}x" for d in shape) + "f32>"
    return (f"module {{\n  func.func public @main(%a0: {t}) -> ({t}) {{\n"
            f'    %0 = "stablehlo.custom_call"(%a0) {{call_target_name = "{target}", backend_config = "{attrs}"}} : ({t}) -> {t}\n'
            f"    func.return %0 : {t}\n  }}\n}}\n")


def run(text, inputs, faults=0, compile=True):
    import shlo_hip
    m = shlo_hip.Module(text)
    f = m.prepare(faults, compile)
    return [o.numpy() for o in f.call([shlo_hip.from_numpy(x) for x in inputs])]


def oracle_dot(oracle, lhs, rhs, tail):
    """out[n, m] = dot(lhs[n, :], rhs[:, m]) in ggml order."""
    return oracle.dot_general_bnk(lhs[None], np.ascontiguousarray(rhs.T)[None], tail)[0]


def same_bits(a, b):
    return a.shape == b.shape and np.array_equal(np.ascontiguousarray(a).view(np.uint32),
                                                 np.ascontiguousarray(b).view(np.uint32))


@pytest.mark.parametrize("flavor", [0, 1])
def test_dot_config1(oracle, flavor):
    """[128,256] x [256,512], uniform[-1,1] from seed 1."""
    import shlo_hip
    N, K, M = 128, 256, 512
    lhs, st = oracle.fill_unif(1, 1.0, N * K)
    rhs, _ = oracle.fill_unif(1, 1.0, K * M, state=st)
    lhs, rhs = lhs.reshape(N, K), rhs.reshape(K, M)
    want = oracle_dot(oracle, lhs, rhs, flavor)
    shlo_hip.set_flavor(flavor)
    try:
        for compile in (True, False):
            got = run(dot_module(N, K, M), [lhs, rhs], compile=compile)[0]
            assert same_bits(got, want), compile
        for fault in ("dot_plain", "dot_builtin"):
            got = run(dot_module(N, K, M), [lhs, rhs], faults=shlo_hip.fault_bits(fault))[0]
            assert not same_bits(got, want), fault
    finally:
        shlo_hip.set_flavor(0)


ODD = [1, 7, 33, 257]


@pytest.mark.parametrize("K", ODD)
def test_dot_odd_shapes(oracle, K):
    """M, N, K in {1, 7, 33, 257}: every tail length and block count, both flavours."""
    import shlo_hip
    for N in ODD:
        for M in ODD:
            lhs, st = oracle.fill_normal(3, 1.0, N * K)
            rhs, _ = oracle.fill_normal(3, 1.0, K * M, state=st)
            lhs, rhs = lhs.reshape(N, K), rhs.reshape(K, M)
            for flavor in (0, 1):
                want = oracle_dot(oracle, lhs, rhs, flavor)
                shlo_hip.set_flavor(flavor)
                try:
                    for compile in (True, False):
                        got = run(dot_module(N, K, M), [lhs, rhs], compile=compile)[0]
                        assert same_bits(got, want), (N, K, M, flavor, compile)
                finally:
                    shlo_hip.set_flavor(0)


def test_dot_batched_small(oracle):
    """A batched dot_general (batch [0]/[0], contract [2]/[1]) at a reduced size."""
    B, N, K, M = 3, 33, 70, 45
    lhs, st = oracle.fill_normal(4, 1.0, B * N * K)
    rhs, _ = oracle.fill_normal(4, 1.0, B * K * M, state=st)
    lhs, rhs = lhs.reshape(B, N, K), rhs.reshape(B, K, M)
    want = np.stack([oracle_dot(oracle, lhs[b], rhs[b], 0) for b in range(B)])
    for compile in (True, False):
        got = run(dot_module(N, K, M, batch=B), [lhs, rhs], compile=compile)[0]
        assert same_bits(got, want)


@pytest.mark.parametrize("B,N,M,K", [(3, 700, 650, 100), (2, 1024, 1024, 512)])
def test_dot_many_tiles(oracle, B, N, M, K):
    """More output tiles than CUs, so workgroups of the short-contraction
    kernel walk several tiles, across batch boundaries: (3,700,650,100) has
    363 tiles with edge tiles, a short last stage and a 4-element tail (plain
    loaders); (2,1024,1024,512) has 512 full tiles on the buffer loaders.
    Both flavours, eager and compiled."""
    import shlo_hip
    lhs, st = oracle.fill_normal(31, 1.0, B * N * K)
    rhs, _ = oracle.fill_normal(31, 1.0, B * K * M, state=st)
    lhs, rhs = lhs.reshape(B, N, K), rhs.reshape(B, K, M)
    for flavor in (0, 1):
        want = oracle.dot_general_bnk(lhs, np.ascontiguousarray(rhs.transpose(0, 2, 1)), flavor)
        shlo_hip.set_flavor(flavor)
        try:
            for compile in (True, False):
                got = run(dot_module(N, K, M, batch=B), [lhs, rhs], compile=compile)[0]
                assert same_bits(got, want), (flavor, compile)
        finally:
            shlo_hip.set_flavor(0)



@pytest.mark.parametrize("B,N,M,K", [(2, 128, 192, 640), (1, 192, 128, 768), (3, 64, 64, 1152),
                                     (5, 512, 512, 128), (3, 512, 704, 384), (1, 128, 64, 256),
                                     (3, 64, 64, 128), (7, 64, 192, 256)])
def test_dot_direct_lds_loads(oracle, B, N, M, K):
    """Contractions in full stages of 128 with the lhs read along k, the rhs
    along its free dim and rows multiples of 64: both operands go from HBM
    straight into LDS.  Long contractions with odd and even stage counts (5,
    6, 9); short ones (four-wave kernel) with more tiles than CUs and 1, 2 and
    3 stages per tile.
    Batched short contractions renumber their workgroups across the 8 XCDs:
    (3,64,64,128) has 6 workgroups (fewer than XCDs) and (7,64,192,256) 42
    (runs of 6 and 5).  Both flavours, eager and compiled."""
    import shlo_hip
    lhs, st = oracle.fill_normal(37, 1.0, B * N * K)
    rhs, _ = oracle.fill_normal(37, 1.0, B * K * M, state=st)
    lhs, rhs = lhs.reshape(B, N, K), rhs.reshape(B, K, M)
    for flavor in (0, 1):
        want = oracle.dot_general_bnk(lhs, np.ascontiguousarray(rhs.transpose(0, 2, 1)), flavor)
        shlo_hip.set_flavor(flavor)
        try:
            for compile in (True, False):
                got = run(dot_module(N, K, M, batch=B), [lhs, rhs], compile=compile)[0]
                assert same_bits(got, want), (flavor, compile)
        finally:
            shlo_hip.set_flavor(0)



def dot_nt_module(B, N, M, K):
    """[B,N,K] x [B,M,K] -> [B,N,M], both operands contiguous along k (Q K^T)."""
    from shlo_hip.configs import t
    a, b, o = t((B, N, K)), t((B, M, K)), t((B, N, M))
    dn = ("#stablehlo.dot<lhs_batching_dimensions = [0], rhs_batching_dimensions = [0], "
          "lhs_contracting_dimensions = [2], rhs_contracting_dimensions = [2]>")
    return (f"module {{\n  func.func public @main(%a0: {a}, %a1: {b}) -> ({o}) {{\n"
            f'    %0 = "stablehlo.dot_general"(%a0, %a1) {{dot_dimension_numbers = {dn}}} : ({a}, {b}) -> {o}\n'
            f"    func.return %0 : {o}\n  }}\n}}\n")


@pytest.mark.parametrize("B,N,M,K", [(2, 128, 192, 64), (3, 192, 128, 192), (8, 256, 320, 64),
                                     (2, 128, 128, 256), (1, 64, 64, 640), (5, 64, 64, 64)])
def test_dot_direct_lds_loads_both_along_k(oracle, B, N, M, K):
    """Both operands contiguous along k, rows multiples of 64: straight into
    LDS in stages of 64 (K = 64, 192; the second with three stages) or of 128
    (K = 256, 640), the rhs stored and read as the lhs.  The batched short ones
    renumber their workgroups across the 8 XCDs: (3,192,128,192) has 36 (runs
    of 5 and 4), (5,64,64,64) 10.  Both flavours, eager and compiled."""
    import shlo_hip
    lhs, st = oracle.fill_normal(41, 1.0, B * N * K)
    rhs, _ = oracle.fill_normal(41, 1.0, B * M * K, state=st)
    lhs, rhs = lhs.reshape(B, N, K), rhs.reshape(B, M, K)
    for flavor in (0, 1):
        want = oracle.dot_general_bnk(lhs, rhs, flavor)
        shlo_hip.set_flavor(flavor)
        try:
            for compile in (True, False):
                got = run(dot_nt_module(B, N, M, K), [lhs, rhs], compile=compile)[0]
                assert same_bits(got, want), (flavor, compile)
        finally:
            shlo_hip.set_flavor(0)


def causal_logits(oracle, rows, cols, sigma=4.0, seed=7):
    x, _ = oracle.fill_normal(seed, sigma, rows * cols)
    x = x.reshape(rows, cols)
    mask = np.triu(np.ones((rows, cols), bool), 1)
    return np.where(mask, np.float32(-np.inf), x).astype(np.float32), mask


def test_softmax_config2(oracle):
    """[4096,1024] softmax, N(0,4) logits with an upper-triangular -inf mask."""
    import shlo_hip
    x, mask = causal_logits(oracle, 4096, 1024)
    want = oracle.soft_max(x)
    text = custom_call_module("ggml.soft_max", "scale = 0x3F800000 : f32", x.shape)
    for compile in (True, False):
        got = run(text, [x], compile=compile)[0]
        assert same_bits(got, want), compile
        assert np.all(got[mask] == 0) and not np.any(np.signbit(got[mask]))
    got = run(text, [x], faults=shlo_hip.fault_bits("soft_max_float_sum"))[0]
    assert not same_bits(got, want)


@pytest.mark.parametrize("cols", [4, 16, 352, 512, 1020, 4096])
def test_softmax_row_lengths(oracle, cols):
    x, _ = oracle.fill_normal(11, 8.0, 64 * cols)
    x = x.reshape(64, cols)
    want = oracle.soft_max(x)
    got = run(custom_call_module("ggml.soft_max", "scale = 0x3F800000 : f32", x.shape), [x])[0]
    assert same_bits(got, want)


@pytest.mark.parametrize("cols", [256, 1024, 4096])
def test_softmax_subnormal_exps(oracle, cols):
    """Rows whose entries sit 80-140 below the row maximum: ggml_v_expf's
    126 < |n| <= 192 branch (subnormal results) and the |n| > 192 branch (+0),
    with -inf entries, next to ordinary ones."""
    rng = np.random.default_rng(cols)
    rows = 64
    x = rng.uniform(-140.0, -80.0, (rows, cols)).astype(np.float32)
    x[:, 0] = 0.0
    x[::3, 1:cols // 4] = rng.normal(0, 2, (len(range(0, rows, 3)), cols // 4 - 1)).astype(np.float32)
    x[::5, -7:] = -np.inf
    x[::7, 2:9] = -250.0
    want = oracle.soft_max(x)
    got = run(custom_call_module("ggml.soft_max", "scale = 0x3F800000 : f32", x.shape), [x])[0]
    assert same_bits(got, want)
    assert np.any((got > 0) & (got < np.float32(1.1754944e-38)))  # subnormal outputs reached


def exact_sum_passes(x):
    """Rows whose group parts pass the kernel's exactness test (tree sum
    <= 2^52 u), estimated with numpy's expf: that decides which of the two
    denominator paths a row takes."""
    e = np.exp(x - x.max(1, keepdims=True)).astype(np.float32)
    p = e.reshape(x.shape[0], -1, 4)
    parts = ((p[..., 0] + p[..., 1]) + (p[..., 2] + p[..., 3])).astype(np.float32)
    bits = parts.view(np.uint32)
    le = np.where(bits == 0, 255, np.maximum(bits >> 23, 1)).min(1).astype(np.int64)
    return parts.astype(np.float64).sum(1) <= np.ldexp(1.0, le - 98)


@pytest.mark.parametrize("cols", [352, 1024, 4096])
def test_softmax_denominator_paths(oracle, cols):
    """Rows spread 4 to 48 below their maximum: the group parts' tree sum
    (exact, so equal to the in-order binary64 sum) on some rows, the in-order
    chain on the others; the planted binary32 denominator on both."""
    import shlo_hip
    rng = np.random.default_rng(100 + cols)
    rows = 96
    spread = np.linspace(4.0, 48.0, rows, dtype=np.float32)[:, None]
    x = (-spread * rng.random((rows, cols), dtype=np.float32)).astype(np.float32)
    x[:, 0] = 0.0
    passes = exact_sum_passes(x)
    assert 0.2 < passes.mean() < 0.8, passes.mean()
    text = custom_call_module("ggml.soft_max", "scale = 0x3F800000 : f32", x.shape)
    want = oracle.soft_max(x)
    for compile in (True, False):
        assert same_bits(run(text, [x], compile=compile)[0], want), compile
    got = run(text, [x], faults=shlo_hip.fault_bits("soft_max_float_sum"))[0]
    assert same_bits(got, oracle.soft_max(x, float_sum=True))


def _find_logit(oracle, P):
    """A logit a <= 0 with fl32(1 + ggml_v_expf(a)) == P, or None."""
    P = np.float32(P)
    a = np.float32(np.log(np.float64(P) - 1.0))
    for _ in range(400):
        v = np.float32(np.float32(1.0) + oracle.ggml_v_expf(a))
        if v == P:
            return a
        a = np.nextafter(a, np.float32(np.inf) if v < P else np.float32(-np.inf), dtype=np.float32)
    return None


def _walk_rows(oracle, cols, count):
    """Rows that fail both fast denominator tests, so the kernel walks their
    parts in order: x = [0, a, -inf, -inf, body..., -70 x 4 (+ tail)] with the
    first part P = fl32(1 + e(a)) chosen so that 1/S lies within 2^-40 of a
    binary32 rounding boundary.  Half the rows have a body of -70 (tiny parts
    the chain absorbs: S = P, every segment walked part by part), half a body
    of logits whose parts m keep 15 segments exact (S = P + 254 m)."""
    from test_softmax_exact_sum import kernel_inv, near_boundary
    e = lambda v: oracle.ggml_v_expf(np.float32(v))
    quad = lambda v: np.float32(np.float32(e(v) + e(v)) + np.float32(e(v) + e(v)))
    G = cols // 4
    v_m = np.float32(-15.25)
    rows = []
    for body in (np.float32(-70.0), v_m):
        offset = 0.0 if body == -70.0 else float(G - 2) * float(quad(v_m))
        found = 0
        for P in near_boundary(offset, 200):
            a = _find_logit(oracle, P)
            if a is None:
                continue
            x = np.full(cols, body, np.float32)
            x[0], x[1], x[2], x[3] = 0.0, a, -np.inf, -np.inf
            x[4 * (G - 1):] = -70.0
            parts = np.array([P] + [quad(body)] * (G - 2) + [quad(-70.0)], np.float32)
            tail = [oracle.expf_cr(np.float32(-70.0))] * (cols % 4)
            inv, path = kernel_inv(np.concatenate([parts, np.array(tail, np.float32)]))
            assert path == "walk", (P, path)
            rows.append(x)
            found += 1
            if found == count:
                break
        assert found == count
    return np.stack(rows)


@pytest.mark.parametrize("cols", [1024, 1023])
def test_softmax_denominator_walk(oracle, cols):
    """Rows whose denominator needs the in-order walk (see _walk_rows), next
    to ordinary rows: bit for bit against the oracle.  cols = 1023 runs the
    row-tail kernel (pinned flavour), whose three tail values follow the parts."""
    import shlo_hip
    walk = _walk_rows(oracle, cols, 6)
    x, _ = oracle.fill_normal(21, 3.0, 20 * cols)
    x = np.concatenate([walk, x.reshape(20, cols)]).astype(np.float32)
    text = custom_call_module("ggml.soft_max", "scale = 0x3F800000 : f32", x.shape)
    want = oracle.soft_max(x)
    shlo_hip.set_flavor(1 if cols % 4 else 0)
    try:
        for compile in (True, False):
            assert same_bits(run(text, [x], compile=compile)[0], want), compile
    finally:
        shlo_hip.set_flavor(0)


@pytest.mark.parametrize("cols", [1, 2, 3, 5, 7, 13, 257, 1021, 4093, 4095])
def test_softmax_row_tails_pinned(oracle, cols):
    """Rows with cols % 4 != 0 in the pinned flavour: the last cols % 4
    elements through the correctly rounded expf, added after the group parts
    (with -inf entries, a scale, and the planted binary32 denominator)."""
    import shlo_hip
    rows = 37
    x, _ = oracle.fill_normal(15, 6.0, rows * cols)
    x = x.reshape(rows, cols)
    if cols > 2:  # masked entries, never a whole row (NaN bits of -inf - -inf are the platform's)
        x[np.arange(rows) % 5 == 0, -1] = -np.inf
        x[np.arange(rows) % 7 == 0, 0] = -np.inf
    text = custom_call_module("ggml.soft_max", "scale = 0x3F000000 : f32", x.shape)
    want = oracle.soft_max(x, scale=0.5)
    shlo_hip.set_flavor(1)
    try:
        for compile in (True, False):
            got = run(text, [x], compile=compile)[0]
            assert same_bits(got, want), (cols, compile)
        if cols > 4:
            got = run(text, [x], faults=shlo_hip.fault_bits("soft_max_float_sum"))[0]
            assert same_bits(got, oracle.soft_max(x, scale=0.5, float_sum=True))
    finally:
        shlo_hip.set_flavor(0)


def test_row_tails_refused_in_stock_flavour(oracle):
    """The stock flavour refuses a row tail, as the reference does
    (Lower.lean:485-486): its expf is Apple libsystem_m's."""
    import shlo_hip
    x, _ = oracle.fill_normal(16, 1.0, 4 * 7)
    x = x.reshape(4, 7)
    for target, attrs in (("ggml.soft_max", "scale = 0x3F800000 : f32"), ("ggml.silu", "")):
        with pytest.raises(shlo_hip.ShloError, match="not carried"):
            run(custom_call_module(target, attrs, x.shape), [x])


@pytest.mark.parametrize("cols", [1, 3, 6, 259, 1023])
def test_silu_row_tails_pinned(oracle, cols):
    import shlo_hip
    rows = 29
    x, _ = oracle.fill_normal(17, 8.0, rows * cols)
    x = x.reshape(rows, cols)
    shlo_hip.set_flavor(1)
    try:
        for compile in (True, False):
            got = run(custom_call_module("ggml.silu", "", x.shape), [x], compile=compile)[0]
            assert same_bits(got, oracle.silu(x)), (cols, compile)
    finally:
        shlo_hip.set_flavor(0)


def test_softmax_scale_attribute(oracle):
    x, _ = oracle.fill_normal(12, 8.0, 32 * 256)
    x = x.reshape(32, 256)
    want = oracle.soft_max(x, scale=0.125)
    got = run(custom_call_module("ggml.soft_max", "scale = 0x3E000000 : f32", x.shape), [x])[0]
    assert same_bits(got, want)


def test_gelu_config2b(oracle):
    """erf-GELU over 64 Mi f32 ~ N(0,3): eager == graph on everything, and
    against the oracle on a 1 Mi prefix and a strided 1 Mi sample."""
    import shlo_hip
    n = 64 << 20
    x = shlo_hip.fill_random((n,), 8, 1, 3.0)
    text = custom_call_module("ggml.gelu_erf", "", (n,))
    m = shlo_hip.Module(text)
    g = m.prepare(0, True).call([x])[0]
    e = m.prepare(0, False).call([x])[0]
    assert shlo_hip.count_nonzero(shlo_hip.binary("ne", shlo_hip.view(g, shlo_hip.U32),
                                                  shlo_hip.view(e, shlo_hip.U32))) == 0
    xs = x.numpy()
    gs = g.numpy()
    for sl in (slice(0, 1 << 20), slice(17, n, 64)):
        want = oracle.gelu_erf(xs[sl])
        assert same_bits(gs[sl], want)
    f = m.prepare(shlo_hip.fault_bits("gelu_tanh"), True).call([x])[0].numpy()
    assert not same_bits(f[:1 << 20], gs[:1 << 20])


@pytest.mark.parametrize("n", [1, 3, 4, 5, 1027, 4096 + 3, 262147, 3 * 1024 * 1024 + 5])
def test_gelu_lengths(oracle, n):
    """Lengths with every n % 4 (the scalar tail), below one block's step and
    spread over many blocks' chunks."""
    x, _ = oracle.fill_normal(13, 3.0, n)
    got = run(custom_call_module("ggml.gelu_erf", "", (n,)), [x])[0]
    assert same_bits(got, oracle.gelu_erf(x))


@pytest.mark.parametrize("off", [1, 2, 3, 4])
def test_gelu_on_offset_view(oracle, off):
    """GELU of a slice starting `off` elements in (a view that is not 16-byte
    aligned unless off % 4 == 0)."""
    n = 70000
    x, _ = oracle.fill_normal(14, 3.0, n + off)
    t_in, t_out = f"tensor<{n + off}xf32>", f"tensor<{n}xf32>"
    text = (f"module {{\n  func.func public @main(%a0: {t_in}) -> ({t_out}) {{\n"
            f'    %0 = "stablehlo.slice"(%a0) {{start_indices = array<i64: {off}>, limit_indices = '
            f"array<i64: {n + off}>, strides = array<i64: 1>}} : ({t_in}) -> {t_out}\n"
            f'    %1 = "stablehlo.custom_call"(%0) {{call_target_name = "ggml.gelu_erf", backend_config = ""}}'
            f" : ({t_out}) -> {t_out}\n    func.return %1 : {t_out}\n  }}\n}}\n")
    for compile in (True, False):
        got = run(text, [x], compile=compile)[0]
        assert same_bits(got, oracle.gelu_erf(x[off:]))


def test_gelu_special_values(oracle):
    specials = np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 1e-38, 3.0, -3.0, 5.5, -5.5, 87.0, -87.0,
                         3.4028235e38, -3.4028235e38], np.float32)
    nan = np.array([0x7FC00000, 0x7F800001, 0xFFC01234, 0x7FBFFFFF, 0xFF800001, 0xFFFFFFFF], np.uint32)
    # random payloads, both signs, quiet and signalling
    rng = np.random.default_rng(5)
    payload = rng.integers(1, 1 << 23, 250, dtype=np.uint32)
    sign = rng.integers(0, 2, 250, dtype=np.uint32) << 31
    nan = np.concatenate([nan, sign | 0x7F800000 | payload]).view(np.float32)
    x = np.concatenate([specials, nan, np.zeros(1, np.float32)])
    want = oracle.gelu_erf(x)
    got = run(custom_call_module("ggml.gelu_erf", "", x.shape), [x])[0]
    assert same_bits(got, want)


def test_norm_and_silu_shapes(oracle):
    import shlo_hip
    for cols in (37, 512, 1024):
        x, _ = oracle.fill_normal(5, 3.0, 96 * cols)
        x = x.reshape(96, cols)
        got = run(custom_call_module("ggml.norm", "eps = 0x3727C5AC : f32", x.shape), [x])[0]
        assert same_bits(got, oracle.norm(x))
    x, _ = oracle.fill_normal(9, 12.0, 64 * 1024)
    x = x.reshape(64, 1024)
    got = run(custom_call_module("ggml.silu", "", x.shape), [x])[0]
    assert same_bits(got, oracle.silu(x))


def test_random_fill_matches_oracle_stream(oracle):
    import shlo_hip
    u = shlo_hip.fill_random((1000,), 1, 0, 1.0).numpy()
    assert same_bits(u, oracle.fill_unif(1, 1.0, 1000)[0])
    v = shlo_hip.fill_random((1000,), 5, 1, 3.0).numpy()
    assert same_bits(v, oracle.fill_normal(5, 3.0, 1000)[0])
    w = shlo_hip.fill_random((500,), 5, 1, 3.0, skip=12 * 500).numpy()
    _, st = oracle.fill_normal(5, 3.0, 500)
    assert same_bits(w, oracle.fill_normal(5, 3.0, 500, state=st)[0])
