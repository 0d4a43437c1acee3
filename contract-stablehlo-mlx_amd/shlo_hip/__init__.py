"""Python binding of the MI355X StableHLO executor (libshlo_hip.so).

A thin ctypes layer over the C ABI in include/shlo_hip.h, mirroring the
reference's Lean surface: `Arr` (StablehloMlx/Mlx.lean's Arr), the op
functions of Mlx.lean, `Module` for Exec.load / argTys / prepare, and
`Fn.call` for Exec.call.  The library must have been built
(contract-stablehlo-mlx_amd/build.py); importing fails loudly otherwise.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libshlo_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is missing: run contract-stablehlo-mlx_amd/build.py first")

_lib = ctypes.CDLL(LIB_PATH)

_P = ctypes.c_void_p
_PP = ctypes.POINTER(ctypes.c_void_p)
_I64P = ctypes.POINTER(ctypes.c_int64)
_SZ = ctypes.c_size_t

_lib.shlo_last_error.restype = ctypes.c_char_p
_lib.shlo_arr_free.argtypes = [_P]
_lib.shlo_arr_free.restype = None
_lib.shlo_fn_free.argtypes = [_P]
_lib.shlo_fn_free.restype = None
_lib.shlo_module_free.argtypes = [_P]
_lib.shlo_module_free.restype = None
_lib.shlo_kernel_free.argtypes = [_P]
_lib.shlo_kernel_free.restype = None
_lib.shlo_get_flavor.restype = ctypes.c_int

# dtype codes (StablehloMlx/Mlx.lean:28-37) and their numpy types
BOOL, U8, U16, U32, U64, I8, I16, I32, I64, F16, F32, F64 = range(12)
_NP = {BOOL: np.bool_, U8: np.uint8, U16: np.uint16, U32: np.uint32, U64: np.uint64, I8: np.int8,
       I16: np.int16, I32: np.int32, I64: np.int64, F16: np.float16, F32: np.float32, F64: np.float64}
_FROM_NP = {np.dtype(v): k for k, v in _NP.items()}

# Unary and binary op codes (StablehloMlx/Mlx.lean:76-108)
UNARY = dict(neg=0, abs=1, sqrt=2, floor=3, exp=4, erf=5, not_=6, invert=7, rsqrt=8, tanh=9, sigmoid=10)
BINARY = dict(add=0, sub=1, mul=2, div=3, max=4, min=5, and_=6, or_=7, xor=8, shl=9, shr=10, eq=11, ne=12,
              lt=13, le=14, gt=15, ge=16, matmul=17, rem=18, land=19, lor=20)

# Planted faults: one bit per field of Lower.Faults (Lower.lean:53-69)
FAULTS = ["dot_builtin", "dot_plain", "soft_max_float_sum", "norm_gpu_ops", "silu_gpu_ops", "gelu_tanh",
          "divide_builtin", "sqrt_builtin", "binary_half", "broadcast_first", "concat_swap",
          "transpose_identity", "slice_shift", "f64_as_f32", "while_short"]


def fault_bits(*names):
    b = 0
    for n in names:
        b |= 1 << FAULTS.index(n)
    return b


class ShloError(RuntimeError):
    pass


def _check(rc):
    if rc != 0:
        raise ShloError(_lib.shlo_last_error().decode(errors="replace"))


def _i64(seq):
    seq = [int(x) for x in seq]
    return (ctypes.c_int64 * max(len(seq), 1))(*seq), len(seq)


class Arr:
    """A device array (immutable; freed when the Python object goes away)."""

    __slots__ = ("_h",)

    def __init__(self, handle):
        self._h = ctypes.c_void_p(handle) if not isinstance(handle, ctypes.c_void_p) else handle

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value and _lib is not None:
            _lib.shlo_arr_free(h)
            self._h = None

    @property
    def shape(self):
        buf = (ctypes.c_int64 * 16)()
        rank = _SZ()
        _check(_lib.shlo_shape(self._h, buf, _SZ(16), ctypes.byref(rank)))
        return tuple(buf[i] for i in range(rank.value))

    @property
    def dtype(self):
        d = ctypes.c_uint8()
        _check(_lib.shlo_dtype(self._h, ctypes.byref(d)))
        return d.value

    @property
    def nbytes(self):
        n = _SZ()
        _check(_lib.shlo_to_bytes(self._h, None, _SZ(0), ctypes.byref(n)))
        return n.value

    def to_bytes(self):
        n = self.nbytes
        buf = ctypes.create_string_buffer(max(n, 1))
        _check(_lib.shlo_to_bytes(self._h, buf, _SZ(n), None))
        return buf.raw[:n]

    def numpy(self):
        out = np.empty(self.shape, dtype=_NP[self.dtype])
        if out.nbytes:
            _check(_lib.shlo_to_bytes(self._h, out.ctypes.data_as(_P), _SZ(out.nbytes), None))
        return out

    def data_ptr(self):
        p = ctypes.c_void_p()
        _check(_lib.shlo_data_ptr(self._h, ctypes.byref(p)))
        return p.value

    def __repr__(self):
        return f"Arr(shape={self.shape}, dtype={self.dtype})"


def _out():
    return ctypes.c_void_p()


def of_bytes(data: bytes, shape, dtype) -> Arr:
    s, r = _i64(shape)
    h = _out()
    _check(_lib.shlo_of_bytes(data, _SZ(len(data)), s, _SZ(r), ctypes.c_uint8(dtype), ctypes.byref(h)))
    return Arr(h)


def from_numpy(a) -> Arr:
    a = np.ascontiguousarray(a)
    dt = _FROM_NP[a.dtype]
    s, r = _i64(a.shape)
    h = _out()
    _check(_lib.shlo_of_bytes(a.ctypes.data_as(_P), _SZ(a.nbytes), s, _SZ(r), ctypes.c_uint8(dt),
                              ctypes.byref(h)))
    return Arr(h)


def empty() -> Arr:
    h = _out()
    _check(_lib.shlo_empty(ctypes.byref(h)))
    return Arr(h)


def unary(op, a: Arr) -> Arr:
    h = _out()
    _check(_lib.shlo_unary(ctypes.c_uint32(UNARY.get(op, op)), a._h, ctypes.byref(h)))
    return Arr(h)


def binary(op, a: Arr, b: Arr) -> Arr:
    h = _out()
    _check(_lib.shlo_binary(ctypes.c_uint32(BINARY.get(op, op)), a._h, b._h, ctypes.byref(h)))
    return Arr(h)


def where(c, a, b) -> Arr:
    h = _out()
    _check(_lib.shlo_where(c._h, a._h, b._h, ctypes.byref(h)))
    return Arr(h)


def reshape(a, shape) -> Arr:
    s, r = _i64(shape)
    h = _out()
    _check(_lib.shlo_reshape(a._h, s, _SZ(r), ctypes.byref(h)))
    return Arr(h)


def transpose(a, perm) -> Arr:
    s, r = _i64(perm)
    h = _out()
    _check(_lib.shlo_transpose(a._h, s, _SZ(r), ctypes.byref(h)))
    return Arr(h)


def broadcast(a, shape) -> Arr:
    s, r = _i64(shape)
    h = _out()
    _check(_lib.shlo_broadcast(a._h, s, _SZ(r), ctypes.byref(h)))
    return Arr(h)


def slice_(a, start, stop, step) -> Arr:
    s0, n = _i64(start)
    s1, _ = _i64(stop)
    s2, _ = _i64(step)
    h = _out()
    _check(_lib.shlo_slice(a._h, s0, s1, s2, _SZ(n), ctypes.byref(h)))
    return Arr(h)


def concat(xs, axis) -> Arr:
    arr = (ctypes.c_void_p * len(xs))(*[x._h.value for x in xs])
    h = _out()
    _check(_lib.shlo_concat(arr, _SZ(len(xs)), ctypes.c_uint32(axis), ctypes.byref(h)))
    return Arr(h)


def astype(a, dtype) -> Arr:
    h = _out()
    _check(_lib.shlo_astype(a._h, ctypes.c_uint8(dtype), ctypes.byref(h)))
    return Arr(h)


def view(a, dtype) -> Arr:
    h = _out()
    _check(_lib.shlo_view(a._h, ctypes.c_uint8(dtype), ctypes.byref(h)))
    return Arr(h)


def take(a, idx, axis) -> Arr:
    h = _out()
    _check(_lib.shlo_take(a._h, idx._h, ctypes.c_uint32(axis), ctypes.byref(h)))
    return Arr(h)


def max_axis(a, axis) -> Arr:
    h = _out()
    _check(_lib.shlo_max_axis(a._h, ctypes.c_uint32(axis), ctypes.byref(h)))
    return Arr(h)


def contiguous(a) -> Arr:
    h = _out()
    _check(_lib.shlo_contiguous(a._h, ctypes.byref(h)))
    return Arr(h)


def eval_(xs):
    arr = (ctypes.c_void_p * max(len(xs), 1))(*[x._h.value for x in xs])
    _check(_lib.shlo_eval(arr, _SZ(len(xs))))


def count_nonzero(a) -> int:
    n = ctypes.c_uint64()
    _check(_lib.shlo_count_nonzero(a._h, ctypes.byref(n)))
    return n.value


def libm_erff_range(base, count) -> np.ndarray:
    out = np.empty(count, dtype=np.uint32)
    _check(_lib.shlo_libm_erff_range(ctypes.c_uint32(base), ctypes.c_uint32(count), out.ctypes.data_as(_P)))
    return out


def expf_range(base, count) -> np.ndarray:
    """The row tails' correctly rounded expf on the host, as bit patterns."""
    out = np.empty(count, dtype=np.uint32)
    _check(_lib.shlo_expf_range(ctypes.c_uint32(base), ctypes.c_uint32(count), out.ctypes.data_as(_P)))
    return out


class Kernel:
    """A precompiled kernel by name (Kernels/Run.lean's cache of specs)."""

    def __init__(self, name, inputs=(), outputs=(), source="", header=""):
        ins = (ctypes.c_char_p * max(len(inputs), 1))(*[s.encode() for s in inputs])
        outs = (ctypes.c_char_p * max(len(outputs), 1))(*[s.encode() for s in outputs])
        h = _out()
        _check(_lib.shlo_kernel_new(name.encode(), ins, _SZ(len(inputs)), outs, _SZ(len(outputs)),
                                    source.encode(), header.encode(), ctypes.byref(h)))
        self._h = h

    def __del__(self):
        if getattr(self, "_h", None) is not None and self._h.value and _lib is not None:
            _lib.shlo_kernel_free(self._h)

    def apply(self, inputs, out_shapes, out_dtypes, grid=(1, 1, 1), threadgroup=(64, 1, 1)):
        arr = (ctypes.c_void_p * len(inputs))(*[x._h.value for x in inputs])
        flat = [d for s in out_shapes for d in s]
        shp, _ = _i64(flat)
        ranks = (_SZ * len(out_shapes))(*[len(s) for s in out_shapes])
        dts = (ctypes.c_uint8 * len(out_dtypes))(*out_dtypes)
        g, _ = _i64(grid)
        t, _ = _i64(threadgroup)
        outs = (ctypes.c_void_p * len(out_shapes))()
        _check(_lib.shlo_kernel_apply(self._h, arr, _SZ(len(inputs)), shp, ranks, dts, _SZ(len(out_shapes)), g,
                                      _SZ(3), t, _SZ(3), outs))
        return [Arr(ctypes.c_void_p(outs[i])) for i in range(len(out_shapes))]


def u32_arr(words) -> Arr:
    """Kernel parameters, padded to 8 words (Run.lean:51-52)."""
    w = list(words) + [0] * (8 - len(words))
    return from_numpy(np.array(w, dtype=np.uint32))


_TRACED = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p), _SZ,
                           ctypes.POINTER(ctypes.c_void_p), _SZ, ctypes.POINTER(_SZ))


class Fn:
    """A (compiled) function: Mlx.compile / Exec.prepare's result."""

    def __init__(self, handle, keep=None):
        self._h = handle
        self._keep = keep

    def __del__(self):
        if getattr(self, "_h", None) is not None and self._h.value and _lib is not None:
            _lib.shlo_fn_free(self._h)

    def _run(self, entry, inputs, cap=64):
        arr = (ctypes.c_void_p * max(len(inputs), 1))(*[x._h.value for x in inputs])
        outs = (ctypes.c_void_p * cap)()
        n = _SZ()
        _check(entry(self._h, arr, _SZ(len(inputs)), outs, _SZ(cap), ctypes.byref(n)))
        return [Arr(ctypes.c_void_p(outs[i])) for i in range(n.value)]

    def apply(self, inputs):
        return self._run(_lib.shlo_apply, inputs)

    def call(self, inputs):
        """Exec.call: apply, then wait for the outputs."""
        return self._run(_lib.shlo_call, inputs)

    def time(self, inputs, reps):
        """Mean ms per apply over `reps` back-to-back applies (HIP events)."""
        arr = (ctypes.c_void_p * max(len(inputs), 1))(*[x._h.value for x in inputs])
        ms = ctypes.c_float()
        _check(_lib.shlo_time_apply(self._h, arr, _SZ(len(inputs)), ctypes.c_int(reps), ctypes.byref(ms)))
        return ms.value


def compile_fn(pyfn, enable=True) -> Fn:
    """Mlx.compile: wrap a Python function of Arr lists (traced on first apply when enabled)."""

    def tramp(payload, ins, nin, outs, cap, nout):
        try:
            args = [_borrow(ins[i]) for i in range(nin)]
            res = pyfn(args)
            if len(res) > cap:
                raise ShloError("too many outputs")
            for i, r in enumerate(res):
                outs[i] = _dup(r)._release()  # the caller owns these handles
            nout[0] = len(res)
            return 0
        except Exception as e:  # noqa: BLE001
            _lib.shlo_set_error(str(e).encode())
            return 1

    cb = _TRACED(tramp)
    h = _out()
    _check(_lib.shlo_compile(cb, None, None, ctypes.c_int(1 if enable else 0), ctypes.byref(h)))
    return Fn(h, keep=cb)


def _borrow(handle_value) -> Arr:
    """A new owned handle to the array behind a borrowed handle."""
    src = Arr(ctypes.c_void_p(handle_value))
    try:
        shp = src.shape
        return reshape(src, shp)
    finally:
        src._h = None  # the borrowed handle is not ours to free


def _dup(a: Arr) -> Arr:
    return reshape(a, a.shape)


def _arr_release(self):
    h = self._h.value
    self._h = None
    return h


Arr._release = _arr_release


class Module:
    """Exec.load: a parsed module with @main."""

    def __init__(self, text: str):
        b = text.encode()
        h = _out()
        _check(_lib.shlo_module_load(b, _SZ(len(b)), ctypes.byref(h)))
        self._h = h

    def __del__(self):
        if getattr(self, "_h", None) is not None and self._h.value and _lib is not None:
            _lib.shlo_module_free(self._h)

    def arg_types(self):
        """Exec.argTys: [(shape, dtype)] of @main's arguments."""
        n = _SZ()
        _check(_lib.shlo_module_nargs(self._h, ctypes.byref(n)))
        res = []
        for i in range(n.value):
            buf = (ctypes.c_int64 * 16)()
            rank = _SZ()
            dt = ctypes.c_uint8()
            _check(_lib.shlo_module_arg(self._h, _SZ(i), buf, _SZ(16), ctypes.byref(rank), ctypes.byref(dt)))
            res.append((tuple(buf[k] for k in range(rank.value)), dt.value))
        return res

    def prepare(self, faults=0, compile=True) -> Fn:
        """Exec.prepare: @main as a function, hipGraph-compiled when `compile`."""
        h = _out()
        _check(_lib.shlo_module_prepare(self._h, ctypes.c_uint64(faults), ctypes.c_int(1 if compile else 0),
                                        ctypes.byref(h)))
        return Fn(h)


def set_flavor(flavor):
    """0 = stock (the reference's mul_mat kernel tail), 1 = pinned."""
    _check(_lib.shlo_set_flavor(ctypes.c_int(flavor)))


def get_flavor():
    return _lib.shlo_get_flavor()


def set_graph_min_ops(n):
    """Compiled functions traced from now on capture a hipGraph when their
    trace holds at least n launches (shorter ones re-issue the launches).
    Returns the previous value."""
    prev = ctypes.c_int()
    _check(_lib.shlo_set_graph_min_ops(ctypes.c_int(n), ctypes.byref(prev)))
    return prev.value


def fill_random(shape, seed, dist, param, skip=0) -> Arr:
    s, r = _i64(shape)
    h = _out()
    _check(_lib.shlo_fill_random(s, _SZ(r), ctypes.c_uint32(seed), ctypes.c_uint64(skip), ctypes.c_int(dist),
                                 ctypes.c_double(param), ctypes.byref(h)))
    return Arr(h)


def checksum_u32(a, start_index) -> int:
    out = ctypes.c_uint64()
    _check(_lib.shlo_checksum_u32(a._h, ctypes.c_uint64(start_index), ctypes.byref(out)))
    return out.value


def sync():
    _check(_lib.shlo_sync())


class Timer:
    """hipEvent timing on the executor's stream."""

    def start(self):
        _check(_lib.shlo_timer_start())

    def stop(self) -> float:
        ms = ctypes.c_float()
        _check(_lib.shlo_timer_stop(ctypes.byref(ms)))
        return ms.value


def device_info():
    name = ctypes.create_string_buffer(256)
    cus = ctypes.c_int()
    pool = ctypes.c_uint64()
    _check(_lib.shlo_device_info(name, _SZ(256), ctypes.byref(cus), ctypes.byref(pool)))
    return name.value.decode(), cus.value, pool.value


def last_dot_kernel() -> str:
    """The dot kernel (family and template arguments) the last dot_general
    dispatch chose."""
    buf = ctypes.create_string_buffer(256)
    _check(_lib.shlo_last_dot_kernel(buf, _SZ(256)))
    return buf.value.decode()


def lib_handle():
    return _lib
