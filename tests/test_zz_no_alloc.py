"""shlo_count_nonzero_noalloc against shlo_count_nonzero, through the C ABI.

The no-allocation variant keeps its partial counts in a static device array
shared by every call on the GPU; two calls in a row, the second on a smaller
input (fewer blocks, so slots the first call wrote stay behind), must both
equal the allocating entry point's count."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _fn():
    import shlo_hip
    lib = shlo_hip.lib_handle()
    f = lib.shlo_count_nonzero_noalloc
    f.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_void_p]
    f.restype = ctypes.c_int
    return f


def _inputs(rng, n, dtype, zero_frac):
    bits = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[np.dtype(dtype).itemsize]
    x = rng.integers(1, np.iinfo(bits).max, n, dtype=bits, endpoint=True)
    x[rng.random(n) < zero_frac] = 0
    return x.view(dtype)


@pytest.mark.parametrize("dtype", [np.float32, np.uint8, np.uint16, np.float64])
def test_noalloc_matches_count_nonzero(dtype):
    import shlo_hip
    f = _fn()
    rng = np.random.default_rng(np.dtype(dtype).itemsize)
    out = shlo_hip.from_numpy(np.full(1, 0xDEADBEEF, np.uint64))
    for n, zf in ((3_000_017, 0.3), (1_001, 0.5)):  # the second call uses fewer blocks than the first
        x = _inputs(rng, n, dtype, zf)
        if dtype == np.float32:
            x[:5] = np.array([-0.0, 0.0, np.nan, -np.inf, 1e-45], np.float32)  # -0.0 has a nonzero bit
        X = shlo_hip.from_numpy(x)
        want = shlo_hip.count_nonzero(X)
        assert want == int(np.count_nonzero(x.view({1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[x.itemsize])))
        rc = f(X.data_ptr(), n, x.itemsize, out.data_ptr())
        assert rc == 0, shlo_hip._lib.shlo_last_error().decode()
        shlo_hip.sync()
        assert int(out.numpy()[0]) == want, (dtype, n)


def test_noalloc_empty_and_refusals():
    import shlo_hip
    f = _fn()
    out = shlo_hip.from_numpy(np.full(1, 7, np.uint64))
    x = shlo_hip.from_numpy(np.ones(1000, np.float32))
    assert f(x.data_ptr(), 0, 4, out.data_ptr()) == 0
    shlo_hip.sync()
    assert int(out.numpy()[0]) == 0
    err = lambda: shlo_hip._lib.shlo_last_error().decode()
    assert f(x.data_ptr(), 1000, 3, out.data_ptr()) != 0 and "elem_bytes" in err()
    assert f(x.data_ptr(), 10 ** 9, 4, out.data_ptr()) != 0 and "overrun" in err()
    host = np.zeros(1, np.uint64)
    assert f(x.data_ptr(), 1000, 4, host.ctypes.data) != 0 and "not a device pointer" in err()
    assert f(x.data_ptr(), 1000, 4, None) != 0 and "NULL" in err()
    assert f(x.data_ptr(), (1 << 40) + 1, 4, out.data_ptr()) != 0 and "at most" in err()
    # nothing was written by the refused calls
    assert f(x.data_ptr(), 1000, 4, out.data_ptr()) == 0
    shlo_hip.sync()
    assert int(out.numpy()[0]) == 1000
