"""GPU runtime semantics: compiled (hipGraph) functions against eager ones,
array immutability across replays, the Run.lean kernel surface, and error
paths (the shim contracts of c/smlx_shim.c:299-386)."""
import numpy as np
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("graph_mode")]


def same_bits(a, b):
    return a.shape == b.shape and np.array_equal(np.ascontiguousarray(a).view(np.uint32),
                                                 np.ascontiguousarray(b).view(np.uint32))


GELU_NORM = """module {
  func.func public @main(%a0: tensor<64x256xf32>) -> (tensor<64x256xf32>, tensor<64x256xf32>) {
    %0 = "stablehlo.custom_call"(%a0) {call_target_name = "ggml.gelu_erf", backend_config = ""} : (tensor<64x256xf32>) -> tensor<64x256xf32>
    %1 = "stablehlo.custom_call"(%0) {call_target_name = "ggml.norm", backend_config = "eps = 0x3727C5AC : f32"} : (tensor<64x256xf32>) -> tensor<64x256xf32>
    func.return %1, %0 : tensor<64x256xf32>, tensor<64x256xf32>
  }
}
"""


def test_held_outputs_survive_the_next_call(oracle):
    import shlo_hip
    x1, st = oracle.fill_normal(21, 2.0, 64 * 256)
    x2, _ = oracle.fill_normal(21, 2.0, 64 * 256, state=st)
    x1, x2 = x1.reshape(64, 256), x2.reshape(64, 256)
    f = shlo_hip.Module(GELU_NORM).prepare(0, True)
    a = f.call([shlo_hip.from_numpy(x1)])
    b = f.call([shlo_hip.from_numpy(x2)])
    assert same_bits(a[0].numpy(), oracle.norm(oracle.gelu_erf(x1)))
    assert same_bits(a[1].numpy(), oracle.gelu_erf(x1))
    assert same_bits(b[0].numpy(), oracle.norm(oracle.gelu_erf(x2)))


def test_iterated_feedback_compiled_equals_eager(oracle):
    import shlo_hip
    x, _ = oracle.fill_normal(22, 2.0, 64 * 256)
    x = x.reshape(64, 256)
    m = shlo_hip.Module(GELU_NORM)
    fc, fe = m.prepare(0, True), m.prepare(0, False)
    xc = xe = shlo_hip.from_numpy(x)
    want = x
    for _ in range(5):
        xc = fc.call([xc])[0]
        xe = fe.call([xe])[0]
        want = oracle.norm(oracle.gelu_erf(want))
    assert same_bits(xc.numpy(), want) and same_bits(xe.numpy(), want)


def test_replays_with_eager_work_between(oracle):
    """A graph replayed several times, with eager launches and syncs between
    the replays; every replay must equal the eager result."""
    import shlo_hip
    x, _ = oracle.fill_normal(23, 2.0, 64 * 256)
    x = x.reshape(64, 256)
    xa = shlo_hip.from_numpy(x)
    m = shlo_hip.Module(GELU_NORM)
    want = m.prepare(0, False).call([xa])[0].numpy()
    f = m.prepare(0, True)
    for i in range(6):
        junk = shlo_hip.binary("add", xa, xa)
        shlo_hip.eval_([junk])
        assert same_bits(f.call([xa])[0].numpy(), want), i


def test_python_traced_function():
    """Mlx.compile over a host function: traced once, replayed as a graph."""
    import shlo_hip
    calls = []

    def fn(args):
        calls.append(1)
        a, b = args
        return [shlo_hip.binary("mul", shlo_hip.binary("add", a, b), b)]

    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    b = np.full((3, 4), 0.5, np.float32)
    fc = shlo_hip.compile_fn(fn, enable=True)
    fe = shlo_hip.compile_fn(fn, enable=False)
    want = (a + b) * b
    for _ in range(3):
        assert same_bits(fc.apply([shlo_hip.from_numpy(a), shlo_hip.from_numpy(b)])[0].numpy(), want)
    assert len(calls) == 1  # traced once for this signature
    assert same_bits(fe.apply([shlo_hip.from_numpy(a), shlo_hip.from_numpy(b)])[0].numpy(), want)
    assert len(calls) == 2


def test_traced_function_error_is_reported():
    import shlo_hip

    def bad(args):
        raise ValueError("boom in trace")

    f = shlo_hip.compile_fn(bad, enable=True)
    with pytest.raises(shlo_hip.ShloError, match="traced function: boom in trace"):
        f.apply([shlo_hip.from_numpy(np.zeros(4, np.float32))])


def test_run_lean_kernel_surface(oracle):
    """kernel_new / kernel_apply with Run.lean's parameter arrays."""
    import shlo_hip
    K, M, R, N = 37, 5, 6, 3  # batch 2 of 3 rows, w shared
    w, st = oracle.fill_unif(1, 1.0, K * M)
    x, _ = oracle.fill_unif(1, 1.0, K * R, state=st)
    want = oracle.mul_mat(w, x, K, M, R, N, 0, oracle.TAIL_STOCK)
    k = shlo_hip.Kernel("mul_mat", ["w", "x", "p"], ["y"], "src", "hdr")
    y = k.apply([shlo_hip.from_numpy(w), shlo_hip.from_numpy(x), shlo_hip.u32_arr([K, M, R, 0, N, 0])],
                [(R * M,)], [shlo_hip.F32], grid=(R * M, 1, 1), threadgroup=(64, 1, 1))[0]
    assert same_bits(y.numpy(), want)
    yp = k.apply([shlo_hip.from_numpy(w), shlo_hip.from_numpy(x), shlo_hip.u32_arr([K, M, R, 0, N, 1])],
                 [(R * M,)], [shlo_hip.F32])[0]
    assert same_bits(yp.numpy(), oracle.mul_mat(w, x, K, M, R, N, 0, oracle.TAIL_PLAIN))
    xs, _ = oracle.fill_normal(2, 4.0, 8 * 16)
    sm = shlo_hip.Kernel("soft_max").apply([shlo_hip.from_numpy(xs), shlo_hip.u32_arr([16, 8, 0x3F800000, 0])],
                                           [(128,)], [shlo_hip.F32])[0]
    assert same_bits(sm.numpy(), oracle.soft_max(xs.reshape(8, 16)).reshape(-1))


def test_shape_and_dtype_errors():
    import shlo_hip
    a = shlo_hip.from_numpy(np.zeros((2, 3), np.float32))
    b = shlo_hip.from_numpy(np.zeros((4,), np.float32))
    with pytest.raises(shlo_hip.ShloError, match="broadcast"):
        shlo_hip.binary("add", a, b)
    with pytest.raises(shlo_hip.ShloError, match="reshape"):
        shlo_hip.reshape(a, (5,))
    with pytest.raises(shlo_hip.ShloError, match="not carried"):
        shlo_hip.Module("""module { func.func public @main(%a0: tensor<4x13xf32>) -> tensor<4x13xf32> {
          %0 = "stablehlo.custom_call"(%a0) {call_target_name = "ggml.soft_max", backend_config = "scale = 0x3F800000 : f32"} : (tensor<4x13xf32>) -> tensor<4x13xf32>
          func.return %0 : tensor<4x13xf32> } }""").prepare().call([shlo_hip.from_numpy(np.zeros((4, 13), np.float32))])
    with pytest.raises(shlo_hip.ShloError, match="decimal float literal"):
        shlo_hip.Module("""module { func.func public @main() -> tensor<f32> {
          %0 = "stablehlo.constant"() {value = dense<1.5> : tensor<f32>} : () -> tensor<f32>
          func.return %0 : tensor<f32> } }""").prepare().call([])


def test_views_and_data_movement():
    import shlo_hip
    a = np.arange(2 * 3 * 4, dtype=np.float32).reshape(2, 3, 4)
    A = shlo_hip.from_numpy(a)
    assert same_bits(shlo_hip.transpose(A, (2, 0, 1)).numpy(), a.transpose(2, 0, 1))
    assert same_bits(shlo_hip.slice_(A, (0, 1, 0), (2, 3, 4), (1, 1, 2)).numpy(), a[:, 1:3, ::2])
    assert same_bits(shlo_hip.broadcast(shlo_hip.from_numpy(a[:, :1, :]), (2, 3, 4)).numpy(),
                     np.broadcast_to(a[:, :1, :], (2, 3, 4)))
    c = shlo_hip.concat([A, shlo_hip.transpose(shlo_hip.transpose(A, (0, 2, 1)), (0, 2, 1))], 1).numpy()
    assert same_bits(c, np.concatenate([a, a], 1))
    idx = shlo_hip.from_numpy(np.array([3, 0, 9, -2], np.int64))
    assert same_bits(shlo_hip.take(A, idx, 2).numpy(), a[:, :, [3, 0, 3, 0]])
    assert same_bits(shlo_hip.max_axis(A, 1).numpy(), a.max(1))
    i32 = shlo_hip.astype(A, shlo_hip.I32).numpy()
    assert np.array_equal(i32, a.astype(np.int32))
    assert np.array_equal(shlo_hip.view(A, shlo_hip.U32).numpy(), a.view(np.uint32))


def test_reshape_keeps_views_where_strides_nest():
    """A reshape of a strided view shares its buffer when every group of
    merged or split dims nests (a slice's rows split into heads, a
    transpose's last dim split), and copies when it does not; the values are
    numpy's either way, and element-wise kernels read the strided result."""
    import shlo_hip
    a = np.arange(4 * 6 * 8, dtype=np.float32).reshape(4, 6, 8)
    A = shlo_hip.from_numpy(a)
    S = shlo_hip.slice_(A, (0, 0, 2), (4, 6, 6), (1, 1, 1))
    s = a[:, :, 2:6]
    T = shlo_hip.transpose(A, (1, 0, 2))
    t = a.transpose(1, 0, 2)
    cases = [(S, s, (24, 4), True), (S, s, (4, 6, 2, 2), True), (S, s, (1, 4, 1, 6, 4, 1), True),
             (S, s, (4, 24), False), (S, s, (96,), False), (T, t, (6, 4, 2, 4), True), (T, t, (24, 8), False),
             (T, t, (6, 32), False)]
    for X, x, shape, view in cases:
        R = shlo_hip.reshape(X, shape)
        assert same_bits(R.numpy(), x.reshape(shape)), shape
        assert (R.data_ptr() == X.data_ptr()) == view, (shape, view)
        assert same_bits(shlo_hip.binary("add", R, R).numpy(), (x + x).reshape(shape)), shape


def test_attention_heads_from_one_projection(oracle):
    """q, k, v as per-head views of one [tokens, 3d] projection (slice,
    reshape, transpose, as the denoiser builds them): the products read them
    in place through two batch strides; both flavours, eager and compiled,
    against the oracle on copied operands."""
    import shlo_hip
    B, T, H, dh = 2, 96, 3, 64
    d, tok = H * dh, B * T
    qkv, _ = oracle.fill_normal(61, 1.0, tok * 3 * d)
    qkv = qkv.reshape(tok, 3 * d)

    def ty(*s):
        return "tensor<" + "".join(f"{x}x" for x in s) + "f32>"

    lines = []
    for i, nm in enumerate("qkv"):
        lines.append(f'    %{nm}s = "stablehlo.slice"(%x) {{start_indices = array<i64: 0, {i * d}>, limit_indices = '
                     f'array<i64: {tok}, {(i + 1) * d}>, strides = array<i64: 1, 1>}} : ({ty(tok, 3 * d)}) -> {ty(tok, d)}\n'
                     f'    %{nm}r = "stablehlo.reshape"(%{nm}s) : ({ty(tok, d)}) -> {ty(B, T, H, dh)}\n'
                     f'    %{nm} = "stablehlo.transpose"(%{nm}r) {{permutation = array<i64: 0, 2, 1, 3>}} : '
                     f"({ty(B, T, H, dh)}) -> {ty(B, H, T, dh)}\n")
    dn_qk = ("#stablehlo.dot<lhs_batching_dimensions = [0, 1], rhs_batching_dimensions = [0, 1], "
             "lhs_contracting_dimensions = [3], rhs_contracting_dimensions = [3]>")
    dn_pv = ("#stablehlo.dot<lhs_batching_dimensions = [0, 1], rhs_batching_dimensions = [0, 1], "
             "lhs_contracting_dimensions = [3], rhs_contracting_dimensions = [2]>")
    text = (f"module {{\n  func.func public @main(%x: {ty(tok, 3 * d)}) -> ({ty(B, H, T, T)}, {ty(B, H, T, dh)}) {{\n" +
            "".join(lines) +
            f'    %s = "stablehlo.dot_general"(%q, %k) {{dot_dimension_numbers = {dn_qk}}} : '
            f"({ty(B, H, T, dh)}, {ty(B, H, T, dh)}) -> {ty(B, H, T, T)}\n"
            f'    %o = "stablehlo.dot_general"(%s, %v) {{dot_dimension_numbers = {dn_pv}}} : '
            f"({ty(B, H, T, T)}, {ty(B, H, T, dh)}) -> {ty(B, H, T, dh)}\n"
            f"    func.return %s, %o : {ty(B, H, T, T)}, {ty(B, H, T, dh)}\n  }}\n}}\n")
    heads = qkv.reshape(B, T, 3, H, dh).transpose(2, 0, 3, 1, 4)  # [3, B, H, T, dh]
    q, k, v = (np.ascontiguousarray(heads[i]).reshape(B * H, T, dh) for i in range(3))
    for flavor in (0, 1):
        s_want = oracle.dot_general_bnk(q, k, flavor)
        o_want = oracle.dot_general_bnk(s_want, np.ascontiguousarray(v.transpose(0, 2, 1)), flavor)
        shlo_hip.set_flavor(flavor)
        try:
            for compile in (True, False):
                got = shlo_hip.Module(text).prepare(0, compile).call([shlo_hip.from_numpy(qkv)])
                assert same_bits(got[0].numpy(), s_want.reshape(B, H, T, T)), (flavor, compile)
                assert same_bits(got[1].numpy(), o_want.reshape(B, H, T, dh)), (flavor, compile)
        finally:
            shlo_hip.set_flavor(0)
