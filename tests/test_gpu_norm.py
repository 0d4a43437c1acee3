"""GPU parity of ggml.norm (one wave per row, the binary64 sums proved or
walked in order) and of the LayerNorm affine fused into its store.

The kernel takes each of norm's two binary64 sums as a tree when no addition
in ggml's in-order chain can round, checks an interval when one can, and adds
the row in order when the interval straddles a binary32 rounding boundary.
The rows built here reach each path, including rows whose in-order chain and
tree sum round to different outputs, so only the in-order walk matches the
oracle."""
import numpy as np
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("graph_mode")]

F32 = np.float32
EPS = "eps = 0x3727C5AC : f32"  # 1e-5


def t(shape):
    return "tensor<" + "".join(f"{d}x" for d in shape) + "f32>"


def same_bits(a, b):
    return a.shape == b.shape and np.array_equal(np.ascontiguousarray(a).view(np.uint32),
                                                 np.ascontiguousarray(b).view(np.uint32))


def norm_module(shape, affine=False):
    """ggml.norm over the last dim, then (affine) * g + b with g, b of the last dim."""
    s = t(shape)
    last = len(shape) - 1
    args = [f"%x: {s}"] + ([f"%g: {t(shape[-1:])}", f"%b: {t(shape[-1:])}"] if affine else [])
    body = f'    %0 = "stablehlo.custom_call"(%x) {{call_target_name = "ggml.norm", backend_config = "{EPS}"}} : ({s}) -> {s}\n'
    ret = "%0"
    if affine:
        body += (f'    %gb = "stablehlo.broadcast_in_dim"(%g) {{broadcast_dimensions = array<i64: {last}>}} : '
                 f"({t(shape[-1:])}) -> {s}\n"
                 f'    %1 = "stablehlo.multiply"(%0, %gb) : ({s}, {s}) -> {s}\n'
                 f'    %bb = "stablehlo.broadcast_in_dim"(%b) {{broadcast_dimensions = array<i64: {last}>}} : '
                 f"({t(shape[-1:])}) -> {s}\n"
                 f'    %2 = "stablehlo.add"(%1, %bb) : ({s}, {s}) -> {s}\n')
        ret = "%2"
    return (f"module {{\n  func.func public @main({', '.join(args)}) -> ({s}) {{\n" + body +
            f"    func.return {ret} : {s}\n  }}\n}}\n")


def run(text, inputs, faults=0, compile=True):
    import shlo_hip
    f = shlo_hip.Module(text).prepare(faults, compile)
    return f.call([shlo_hip.from_numpy(np.ascontiguousarray(x)) for x in inputs])[0].numpy()


def check(oracle, x, affine=None):
    want = oracle.norm(x)
    ins = [x]
    if affine is not None:
        g, b = affine
        want = ((want * g).astype(F32) + b).astype(F32)
        ins += [g, b]
    text = norm_module(x.shape, affine is not None)
    for compile in (True, False):
        assert same_bits(run(text, ins, compile=compile), want), compile
    return text, ins, want


def mean_walk_row(cols):
    """Elements 1, 2^-53, 2^-24, 2^-53 at columns 0, 4, 8, 12 (lanes 0..3):
    the in-order chain rounds both 2^-53 away (ties to even) and ends at
    1 + 2^-24, a binary32 tie that rounds to 1; the wave's tree adds the two
    2^-53 first and ends at 1 + 2^-24 + 2^-52, which rounds up."""
    x = np.zeros(cols, F32)
    x[0], x[4], x[8], x[12] = 1.0, 2.0 ** -53, 2.0 ** -24, 2.0 ** -53
    return x


def var_walk_row(cols):
    """Mean exactly 0 and group parts 256, 2^-45, 2^-16, 2^-45 (groups 0..3):
    the in-order sum is 256 + 2^-16 (each 2^-45 a tie rounded away), so with
    cols = 16 var = (float)(S / 16) is the tie 16 + 2^-20, which rounds to 16;
    the tree sum holds 2^-44 more and rounds up, and the difference survives
    sqrtf and the reciprocal into the outputs."""
    x = np.zeros(cols, F32)
    x[0:4] = [8, -8, 8, -8]
    x[4:6] = [2.0 ** -23, -2.0 ** -23]
    x[8:12] = [2.0 ** -9, -2.0 ** -9, 2.0 ** -9, -2.0 ** -9]
    x[12:14] = [2.0 ** -23, -2.0 ** -23]
    return x


def test_walk_rows_differ_from_tree_order(oracle):
    """The constructed rows: the oracle's in-order result differs from the
    tree-order one, and the kernel matches the oracle."""
    m = mean_walk_row(512)
    s_chain = 0.0
    for v in m.astype(np.float64):
        s_chain += v
    s_tree = (1.0 + 2.0 ** -24) + (2.0 ** -53 + 2.0 ** -53)
    assert F32(s_chain) != F32(s_tree)
    v = var_walk_row(16)
    assert F32((256.0 + 2.0 ** -16) / 16) != F32((256.0 + 2.0 ** -16 + 2.0 ** -44) / 16)
    rows = np.stack([mean_walk_row(512), mean_walk_row(512) * F32(3), -mean_walk_row(512)])
    check(oracle, rows)
    check(oracle, np.stack([v, v * F32(0.5), v * F32(2.0 ** 40)]))
    # the same rows inside wider blocks of random rows (other waves of a block)
    x, _ = oracle.fill_normal(17, 1.0, 10 * 512)
    x = x.reshape(10, 512)
    x[3] = mean_walk_row(512)
    x[7, :16] = var_walk_row(16)
    x[7, 16:] = 0.0
    check(oracle, x)


@pytest.mark.parametrize("cols", [4, 16, 512, 1024, 1028, 2052, 4096])
def test_tiny_elements_interval_path(oracle, cols):
    """Rows of N(0,1) with one element around 2^-60: the exactness test fails
    for both sums, the interval decides (or the walk)."""
    x, _ = oracle.fill_normal(23, 1.0, 64 * cols)
    x = x.reshape(64, cols)
    tiny, _ = oracle.fill_normal(24, 2.0 ** -60, 64)
    x[np.arange(64), np.arange(64) % cols] = tiny
    check(oracle, x)


@pytest.mark.parametrize("cols", [1, 2, 3, 5, 37, 255, 257, 1023, 4095])
def test_row_tails(oracle, cols):
    x, _ = oracle.fill_normal(25, 3.0, 40 * cols)
    check(oracle, x.reshape(40, cols))


def same_up_to_nan_bits(a, b):
    """Equal bits everywhere except that a NaN matches any NaN: NaN sign and
    payload are not pinned (the x86 oracle's default NaN is negative, arm64's
    and the GPU's positive, and the GPU's subtract flips a NaN operand's sign)."""
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and same_bits(np.where(na, 0, a), np.where(nb, 0, b))


def test_special_values(oracle):
    """NaN, infinities, zeros of both signs, a constant row, subnormals, and
    sums of |x| beyond binary32: every non-NaN output bit for bit."""
    cols = 512
    x, _ = oracle.fill_normal(26, 1.0, 8 * cols)
    x = x.reshape(8, cols)
    x[0, 5] = np.nan
    x[1, 9] = np.inf
    x[2, 9], x[2, 10] = np.inf, -np.inf
    x[3] = 0.0
    x[4] = -0.0
    x[5] = 7.25  # constant row: variance 0
    x[6, ::3] = F32(1e-42)  # subnormals
    x[7] = F32(3e38) * np.sign(x[7])  # the sum of |x| beyond binary32
    want = oracle.norm(x)
    assert np.isnan(want).any() and not np.isnan(want).all()
    text = norm_module(x.shape)
    for compile in (True, False):
        assert same_up_to_nan_bits(run(text, [x], compile=compile), want), compile


@pytest.mark.parametrize("shape", [(8192, 512), (3, 7, 1024), (100, 1028), (33, 6)])
def test_fused_affine(oracle, shape):
    """norm * g + b: fused for rows of at most 1024 columns, separate ops beyond."""
    x, _ = oracle.fill_normal(27, 1.0, int(np.prod(shape)))
    x = x.reshape(shape)
    g, _ = oracle.fill_normal(28, 0.02, shape[-1])
    b, _ = oracle.fill_normal(29, 0.02, shape[-1])
    check(oracle, x, ((g + F32(1)).astype(F32), b))


@pytest.mark.parametrize("kind", ["slice", "transpose"])
def test_fused_operand_layouts(oracle, kind):
    """norm(x) * y + b where y is a view the fused loads cannot take as
    16-byte groups: a slice starting one element into each row (misaligned)
    or a transposed array (column stride 64); b is an aligned bias."""
    R, C = 64, 512
    x, st = oracle.fill_normal(71, 1.0, R * C)
    x = x.reshape(R, C)
    zsh = (R, C + 4) if kind == "slice" else (C, R)
    z, st = oracle.fill_normal(72, 1.0, zsh[0] * zsh[1], state=st)
    z = z.reshape(zsh)
    b, _ = oracle.fill_normal(73, 0.5, C, state=st)
    y = z[:, 1:C + 1] if kind == "slice" else z.T
    want = ((oracle.norm(x) * y).astype(F32) + b).astype(F32)
    s, zt = t((R, C)), t(zsh)
    if kind == "slice":
        view = (f'    %y = "stablehlo.slice"(%z) {{start_indices = array<i64: 0, 1>, limit_indices = '
                f'array<i64: {R}, {C + 1}>, strides = array<i64: 1, 1>}} : ({zt}) -> {s}\n')
    else:
        view = f'    %y = "stablehlo.transpose"(%z) {{permutation = array<i64: 1, 0>}} : ({zt}) -> {s}\n'
    text = (f"module {{\n  func.func public @main(%x: {s}, %z: {zt}, %b: {t((C,))}) -> ({s}) {{\n" + view +
            f'    %0 = "stablehlo.custom_call"(%x) {{call_target_name = "ggml.norm", backend_config = "{EPS}"}} : ({s}) -> {s}\n'
            f'    %1 = "stablehlo.multiply"(%0, %y) : ({s}, {s}) -> {s}\n'
            f'    %bb = "stablehlo.broadcast_in_dim"(%b) {{broadcast_dimensions = array<i64: 1>}} : ({t((C,))}) -> {s}\n'
            f'    %2 = "stablehlo.add"(%1, %bb) : ({s}, {s}) -> {s}\n'
            f"    func.return %2 : {s}\n  }}\n}}\n")
    for compile in (True, False):
        assert same_bits(run(text, [x, z, b], compile=compile), want), compile


def test_planted_norm_fault_differs(oracle):
    import shlo_hip
    x, _ = oracle.fill_normal(30, 1.0, 64 * 512)
    x = x.reshape(64, 512)
    g, _ = oracle.fill_normal(31, 0.02, 512)
    b, _ = oracle.fill_normal(32, 0.02, 512)
    text, ins, want = check(oracle, x, (g, b))
    got = run(text, ins, faults=shlo_hip.fault_bits("norm_gpu_ops"))
    assert not same_bits(got, want)
