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
