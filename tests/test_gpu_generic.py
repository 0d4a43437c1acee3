"""The generic StableHLO path on the GPU: native binary64 with the
reference's rules (Lower.lean:255-298, :350-364, SoftFloat.lean), `while`
unrolled on trace-time scalars (Lower.lean:454-470), `dynamic_slice` with
clamped trace-time starts (:417-428), the 1-D `gather` with clamped indices
(:319-331) and the max `reduce` (:430-439).

Each module runs eager and compiled; binary64 results are compared bit for
bit with the oracle's restatement of SoftFloat.lean (pinned in
tests/test_oracle_f64.py), the rest with numpy (data movement, and maximum,
which is exact in any order).  The planted faults f64AsF32 and whileShort
(Lower.lean:53-69) must change the bits, and the refusals the reference makes
must be made."""
import numpy as np
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("graph_mode")]

SIGN64 = np.uint64(1 << 63)


def run(text, inputs, faults=0, compile=True):
    import shlo_hip
    m = shlo_hip.Module(text)
    return [o.numpy() for o in m.prepare(faults, compile).call([shlo_hip.from_numpy(x) for x in inputs])]


def f64_inputs(rng, n):
    """Random binary64 values with NaNs (quiet and signalling, both signs,
    payloads), infinities, signed zeros, subnormals, int64 boundaries and
    values with more than 24 significant bits."""
    x = rng.standard_normal(n) * 10.0 ** rng.integers(-5, 6, n)
    k = rng.integers(0, 14, n)
    bits = x.view(np.uint64).copy()
    pay = rng.integers(1, 1 << 51, n, dtype=np.uint64)
    sgn = rng.integers(0, 2, n, dtype=np.uint64) << np.uint64(63)
    bits[k == 0] = (np.uint64(0x7FF8000000000000) | pay | sgn)[k == 0]  # quiet NaN
    bits[k == 1] = (np.uint64(0x7FF0000000000000) | pay | sgn)[k == 1]  # signalling NaN
    bits[k == 2] = (np.uint64(0x7FF0000000000000) | sgn)[k == 2]  # +-inf
    bits[k == 3] = sgn[k == 3]  # +-0
    bits[k == 4] = ((pay & np.uint64(0xFFFFFFFFFFFFF)) | sgn)[k == 4]  # subnormal
    spec = np.array([2.0 ** 63, -(2.0 ** 63), 1e19, -1e19, 2.0 ** 63 - 1024, -0.5, -1.5, 0.5, 1.7976931348623157e308,
                     3e38, 3.5e38, 1e-40, 2.0 ** -150, -2.5])
    sel = k == 5
    bits[sel] = spec[rng.integers(0, spec.size, int(sel.sum()))].view(np.uint64)
    return bits.view(np.float64)


def f64_module(n):
    t, ti, tf, tb = (f"tensor<{n}xf64>", f"tensor<{n}xi64>", f"tensor<{n}xf32>", f"tensor<{n}xi1>")
    ops = [("add", 2, t), ("subtract", 2, t), ("multiply", 2, t), ("divide", 2, t), ("floor", 1, t),
           ("maximum", 2, t), ("minimum", 2, t), ("abs", 1, t), ("negate", 1, t)]
    lines = []
    for i, (op, ar, o) in enumerate(ops):
        args = "%a, %b" if ar == 2 else "%a"
        ins = f"{t}, {t}" if ar == 2 else t
        lines.append(f'    %{i} = "stablehlo.{op}"({args}) : ({ins}) -> {o}')
    lines.append(f'    %9 = "stablehlo.convert"(%a) : ({t}) -> {ti}')
    lines.append(f'    %10 = "stablehlo.convert"(%a) : ({t}) -> {tf}')
    for j, dr in enumerate(("EQ", "NE", "LT", "LE", "GT", "GE")):
        lines.append(f'    %{11 + j} = "stablehlo.compare"(%a, %b) {{comparison_direction = '
                     f'#stablehlo<comparison_direction {dr}>}} : ({t}, {t}) -> {tb}')
    outs = ", ".join(f"%{i}" for i in range(17))
    otys = ", ".join([t] * 9 + [ti, tf] + [tb] * 6)
    body = "\n".join(lines)
    return (f"module {{\n  func.func public @main(%a: {t}, %b: {t}) -> ({otys}) {{\n{body}\n"
            f"    func.return {outs} : {otys}\n  }}\n}}\n")


def f64_want(oracle, a, b):
    ab, bb = a.view(np.uint64), b.view(np.uint64)
    w = [oracle.f64_ew(op, ab, bb) for op in range(4)]
    w.append(oracle.f64_ew(4, ab))
    w.append(oracle.f64_maxmin(True, ab, bb))
    w.append(oracle.f64_maxmin(False, ab, bb))
    w.append(ab & ~SIGN64)  # abs: AND ABS64 (Lower.lean:360)
    w.append(ab ^ SIGN64)  # negate: XOR SIGN64 (Lower.lean:361)
    w.append(oracle.f64_ew(5, ab))
    w.append(oracle.f32_of_f64(ab))
    with np.errstate(invalid="ignore"):  # IEEE comparisons (f64Compare, Lower.lean:274-288)
        for cmp in (np.equal, np.not_equal, np.less, np.less_equal, np.greater, np.greater_equal):
            w.append(cmp(a, b))
    return w


def bits_of(x):
    x = np.ascontiguousarray(x)
    if x.dtype == np.bool_:
        return x.astype(np.uint8)
    return x.view({8: np.uint64, 4: np.uint32, 1: np.uint8}[x.dtype.itemsize])


def test_f64_ops_vs_oracle(oracle):
    import shlo_hip
    rng = np.random.default_rng(3)
    n = 4099
    a, b = f64_inputs(rng, n), f64_inputs(rng, n)
    want = f64_want(oracle, a, b)
    text = f64_module(n)
    names = ["add", "sub", "mul", "div", "floor", "max", "min", "abs", "neg", "to_i64", "to_f32",
             "eq", "ne", "lt", "le", "gt", "ge"]
    for compile in (True, False):
        got = run(text, [a, b], compile=compile)
        for nm, g, w in zip(names, got, want):
            assert np.array_equal(bits_of(g), bits_of(w).astype(bits_of(g).dtype)), (nm, compile)
    # binary64 done in binary32 (the planted f64AsF32) changes add..divide
    got = run(text, [a, b], faults=shlo_hip.fault_bits("f64_as_f32"))
    for nm, g, w in zip(names[:4], got[:4], want[:4]):
        assert not np.array_equal(bits_of(g), w), nm


def test_f32_to_f64_vs_oracle(oracle):
    rng = np.random.default_rng(4)
    n = 2053
    u = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    u[:6] = [0x7F800001, 0xFFC00000, 0x00000001, 0x80000000, 0x7F7FFFFF, 0xFF800000]
    x = u.view(np.float32)
    t, o = f"tensor<{n}xf32>", f"tensor<{n}xf64>"
    text = (f"module {{\n  func.func public @main(%a: {t}) -> ({o}) {{\n"
            f'    %0 = "stablehlo.convert"(%a) : ({t}) -> {o}\n    func.return %0 : {o}\n  }}\n}}\n')
    want = oracle.f64_of_f32(x)
    for compile in (True, False):
        assert np.array_equal(run(text, [x], compile=compile)[0].view(np.uint64), want)


def test_f64_kernel_surface(oracle):
    """The reference's f64_ew / f64_of_f32 / f32_of_f64 kernels
    (Run.lean:87-104) through shlo_kernel_apply, on uint64 bit patterns."""
    import shlo_hip
    rng = np.random.default_rng(5)
    n = 1031
    a, b = f64_inputs(rng, n).view(np.uint64), f64_inputs(rng, n).view(np.uint64)
    A, B = shlo_hip.from_numpy(a), shlo_hip.from_numpy(b)
    k = shlo_hip.Kernel("f64_ew")
    for op in range(6):
        y = k.apply([A, B, shlo_hip.u32_arr([n, op])], [(n,)], [shlo_hip.U64])[0].numpy()
        assert np.array_equal(y, oracle.f64_ew(op, a, b)), op
    f = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    y = shlo_hip.Kernel("f64_of_f32").apply([shlo_hip.from_numpy(f), shlo_hip.u32_arr([n])], [(n,)],
                                             [shlo_hip.U64])[0].numpy()
    assert np.array_equal(y, oracle.f64_of_f32(f))
    y = shlo_hip.Kernel("f32_of_f64").apply([A, shlo_hip.u32_arr([n])], [(n,)], [shlo_hip.F32])[0].numpy()
    assert np.array_equal(y.view(np.uint32), oracle.f32_of_f64(a))


def test_f64_refusals():
    import shlo_hip
    t = "tensor<4xf64>"
    for op in ("sqrt", "exponential", "tanh", "logistic"):
        text = (f"module {{\n  func.func public @main(%a: {t}) -> ({t}) {{\n"
                f'    %0 = "stablehlo.{op}"(%a) : ({t}) -> {t}\n    func.return %0 : {t}\n  }}\n}}\n')
        with pytest.raises(shlo_hip.ShloError, match="on f64 is not carried"):
            run(text, [np.zeros(4)], compile=False)
    text = (f"module {{\n  func.func public @main(%a: {t}) -> (tensor<4xi32>) {{\n"
            f'    %0 = "stablehlo.convert"(%a) : ({t}) -> tensor<4xi32>\n    func.return %0 : tensor<4xi32>\n  }}\n}}\n')
    with pytest.raises(shlo_hip.ShloError, match="convert f64 to i32 is not carried"):
        run(text, [np.zeros(4)], compile=False)


WHILE = """module {
  func.func public @main(%x: tensor<5x3xf32>) -> (tensor<5x3xf32>) {
    %c0 = "stablehlo.constant"() {value = dense<0> : tensor<i32>} : () -> tensor<i32>
    %r:2 = "stablehlo.while"(%c0, %x) ({
      ^bb0(%i: tensor<i32>, %v: tensor<5x3xf32>):
        %n = "stablehlo.constant"() {value = dense<6> : tensor<i32>} : () -> tensor<i32>
        %c = "stablehlo.compare"(%i, %n) {comparison_direction = #stablehlo<comparison_direction LT>} : (tensor<i32>, tensor<i32>) -> tensor<i1>
        "stablehlo.return"(%c) : (tensor<i1>) -> ()
    }, {
      ^bb0(%i: tensor<i32>, %v: tensor<5x3xf32>):
        %one = "stablehlo.constant"() {value = dense<1> : tensor<i32>} : () -> tensor<i32>
        %i2 = "stablehlo.add"(%i, %one) : (tensor<i32>, tensor<i32>) -> tensor<i32>
        %sq = "stablehlo.multiply"(%v, %v) : (tensor<5x3xf32>, tensor<5x3xf32>) -> tensor<5x3xf32>
        %h = "stablehlo.constant"() {value = dense<0x3F000000> : tensor<5x3xf32>} : () -> tensor<5x3xf32>
        %hv = "stablehlo.multiply"(%sq, %h) : (tensor<5x3xf32>, tensor<5x3xf32>) -> tensor<5x3xf32>
        %v2 = "stablehlo.subtract"(%v, %hv) : (tensor<5x3xf32>, tensor<5x3xf32>) -> tensor<5x3xf32>
        "stablehlo.return"(%i2, %v2) : (tensor<i32>, tensor<5x3xf32>) -> ()
    }) : (tensor<i32>, tensor<5x3xf32>) -> (tensor<i32>, tensor<5x3xf32>)
    func.return %r#1 : tensor<5x3xf32>
  }
}
"""


def test_while_unrolled(oracle):
    """Six iterations of v <- v - (v*v)*0.5, each op one binary32 rounding
    (numpy float32 computes the same); whileShort stops one short."""
    import shlo_hip
    x, _ = oracle.fill_normal(9, 1.0, 15)
    x = x.reshape(5, 3)
    v = x.copy()
    prev = v
    for _ in range(6):
        prev = v
        v = (v - (v * v) * np.float32(0.5)).astype(np.float32)
    for compile in (True, False):
        assert np.array_equal(run(WHILE, [x], compile=compile)[0].view(np.uint32), v.view(np.uint32))
    got = run(WHILE, [x], faults=shlo_hip.fault_bits("while_short"))[0]
    assert np.array_equal(got.view(np.uint32), prev.view(np.uint32))
    assert not np.array_equal(got.view(np.uint32), v.view(np.uint32))


def test_while_on_data_is_refused():
    import shlo_hip
    text = WHILE.replace('%c0 = "stablehlo.constant"() {value = dense<0> : tensor<i32>} : () -> tensor<i32>',
                         '%c0 = "stablehlo.convert"(%k) : (tensor<i32>) -> tensor<i32>')
    text = text.replace("@main(%x: tensor<5x3xf32>)", "@main(%x: tensor<5x3xf32>, %k: tensor<i32>)")
    with pytest.raises(shlo_hip.ShloError, match="while: the condition depends on data"):
        run(text, [np.zeros((5, 3), np.float32), np.array(0, np.int32)], compile=False)


def dyn_slice_module(r0, c0):
    """dynamic_slice of a [6,5] array at trace-time starts r0 + 1, c0 (sizes 2x3)."""
    return f"""module {{
  func.func public @main(%x: tensor<6x5xf32>) -> (tensor<2x3xf32>) {{
    %a = "stablehlo.constant"() {{value = dense<{r0}> : tensor<i32>}} : () -> tensor<i32>
    %one = "stablehlo.constant"() {{value = dense<1> : tensor<i32>}} : () -> tensor<i32>
    %r = "stablehlo.add"(%a, %one) : (tensor<i32>, tensor<i32>) -> tensor<i32>
    %c = "stablehlo.constant"() {{value = dense<{c0}> : tensor<i32>}} : () -> tensor<i32>
    %d = "stablehlo.dynamic_slice"(%x, %r, %c) {{slice_sizes = array<i64: 2, 3>}} : (tensor<6x5xf32>, tensor<i32>, tensor<i32>) -> tensor<2x3xf32>
    func.return %d : tensor<2x3xf32>
  }}
}}
"""


@pytest.mark.parametrize("r0,c0", [(1, 1), (5, -2), (-7, 9), (2, 2)])
def test_dynamic_slice_clamps(oracle, r0, c0):
    x = np.arange(30, dtype=np.float32).reshape(6, 5) * np.float32(1.5)
    r = max(0, min(r0 + 1, 6 - 2))
    c = max(0, min(c0, 5 - 3))
    for compile in (True, False):
        got = run(dyn_slice_module(r0, c0), [x], compile=compile)[0]
        assert np.array_equal(got, x[r:r + 2, c:c + 3]), (r0, c0)


def test_dynamic_slice_on_data_is_refused():
    import shlo_hip
    text = """module {
  func.func public @main(%x: tensor<6x5xf32>, %s: tensor<i32>) -> (tensor<2x3xf32>) {
    %d = "stablehlo.dynamic_slice"(%x, %s, %s) {slice_sizes = array<i64: 2, 3>} : (tensor<6x5xf32>, tensor<i32>, tensor<i32>) -> tensor<2x3xf32>
    func.return %d : tensor<2x3xf32>
  }
}
"""
    with pytest.raises(shlo_hip.ShloError, match="depends on data"):
        run(text, [np.zeros((6, 5), np.float32), np.array(1, np.int32)], compile=False)


GATHER = """module {
  func.func public @main(%t: tensor<10xf32>, %i: tensor<9xi32>) -> (tensor<9xf32>) {
    %g = "stablehlo.gather"(%t, %i) {dimension_numbers = #stablehlo.gather<offset_dims = [], collapsed_slice_dims = [0], start_index_map = [0], index_vector_dim = 1>, slice_sizes = array<i64: 1>} : (tensor<10xf32>, tensor<9xi32>) -> tensor<9xf32>
    func.return %g : tensor<9xf32>
  }
}
"""


def test_gather1d_clamps(oracle):
    t, _ = oracle.fill_normal(10, 1.0, 10)
    idx = np.array([-3, 0, 9, 12, 5, -2147483648, 2147483647, 4, 1], np.int32)
    want = t[np.clip(idx, 0, 9)]
    for compile in (True, False):
        assert np.array_equal(run(GATHER, [t, idx], compile=compile)[0].view(np.uint32), want.view(np.uint32))


def test_gather_other_forms_refused():
    import shlo_hip
    text = GATHER.replace("collapsed_slice_dims = [0]", "collapsed_slice_dims = [1]")
    with pytest.raises(shlo_hip.ShloError, match="only a 1-D table"):
        run(text, [np.zeros(10, np.float32), np.zeros(9, np.int32)], compile=False)


def reduce_module(dims, init_hex, shape=(4, 6, 5)):
    from shlo_hip.configs import t
    keep = tuple(d for i, d in enumerate(shape) if i not in dims)
    dl = ", ".join(str(d) for d in dims)
    return f"""module {{
  func.func public @main(%x: {t(shape)}) -> ({t(keep)}) {{
    %init = "stablehlo.constant"() {{value = dense<{init_hex}> : tensor<f32>}} : () -> tensor<f32>
    %r = "stablehlo.reduce"(%x, %init) ({{
      ^bb0(%p: tensor<f32>, %q: tensor<f32>):
        %m = "stablehlo.maximum"(%p, %q) : (tensor<f32>, tensor<f32>) -> tensor<f32>
        "stablehlo.return"(%m) : (tensor<f32>) -> ()
    }}) {{dimensions = array<i64: {dl}>}} : ({t(shape)}, tensor<f32>) -> {t(keep)}
    func.return %r : {t(keep)}
  }}
}}
"""


@pytest.mark.parametrize("dims,init", [((1,), 0xFF800000), ((0, 2), 0xFF800000), ((2,), 0x3F800000),
                                       ((0, 1, 2), 0xFF800000)])
def test_reduce_max(oracle, dims, init):
    x, _ = oracle.fill_normal(12, 1.0, 120)
    x = x.reshape(4, 6, 5)
    iv = np.array([init], np.uint32).view(np.float32)[0]
    want = np.maximum(x.max(axis=dims), iv)
    for compile in (True, False):
        got = run(reduce_module(dims, f"0x{init:08X}"), [x], compile=compile)[0]
        assert np.array_equal(np.asarray(got).view(np.uint32), np.asarray(want, np.float32).view(np.uint32))


def test_reduce_refusals():
    import shlo_hip
    text = reduce_module((1,), "0xFF800000").replace('"stablehlo.maximum"', '"stablehlo.add"')
    with pytest.raises(shlo_hip.ShloError, match="only a single-operand maximum"):
        run(text, [np.zeros((4, 6, 5), np.float32)], compile=False)
