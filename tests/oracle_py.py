"""ctypes binding of the CPU oracle (oracle/liboracle.so) — test infrastructure.

Only tests, __graft_entry__.smoke() and bench.py's cpu_baseline use this, as
the checker; the product never imports it.
"""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "oracle", "build", "liboracle.so")
_l = ctypes.CDLL(LIB)

_FP = ctypes.POINTER(ctypes.c_float)
_P = ctypes.c_void_p
_l.orc_rnd.restype = ctypes.c_uint32
_l.orc_unif.restype = ctypes.c_float
_l.orc_normal.restype = ctypes.c_float
_l.orc_vec_dot.restype = ctypes.c_float
_l.orc_vec_dot.argtypes = [_P, _P, ctypes.c_int64, ctypes.c_int]
_l.orc_ggml_v_expf.restype = ctypes.c_float
_l.orc_ggml_v_expf.argtypes = [ctypes.c_float]
_l.orc_expf_cr.restype = ctypes.c_float
_l.orc_expf_cr.argtypes = [ctypes.c_float]
_l.orc_erff_cr.restype = ctypes.c_float
_l.orc_erff_cr.argtypes = [ctypes.c_float]
_l.orc_gelu_erf1.restype = ctypes.c_float
_l.orc_gelu_erf1.argtypes = [ctypes.c_float, ctypes.c_int]
_l.orc_checksum_words.restype = ctypes.c_uint64
_l.orc_checksum_words.argtypes = [_P, ctypes.c_size_t, ctypes.c_uint64]
_l.orc_write_case.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int]
_l.orc_case_name.restype = ctypes.c_char_p
_l.orc_f64_ew.restype = ctypes.c_uint64
_l.orc_f64_ew.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64]

TAIL_STOCK, TAIL_PINNED, TAIL_PLAIN = 0, 1, 2
NCPU = min(os.cpu_count() or 1, 16)


def _ptr(a):
    return a.ctypes.data_as(_P)


def fill_unif(seed, a, n, state=None):
    st = ctypes.c_uint32(seed if state is None else state)
    out = np.empty(n, np.float32)
    _l.orc_fill_unif(ctypes.byref(st), ctypes.c_float(a), _ptr(out), ctypes.c_size_t(n))
    return out, st.value


def fill_normal(seed, sigma, n, state=None):
    st = ctypes.c_uint32(seed if state is None else state)
    out = np.empty(n, np.float32)
    _l.orc_fill_normal(ctypes.byref(st), ctypes.c_double(sigma), _ptr(out), ctypes.c_size_t(n))
    return out, st.value


def vec_dot(w, x, tail=TAIL_STOCK):
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    return np.float32(_l.orc_vec_dot(_ptr(w), _ptr(x), ctypes.c_int64(w.size), ctypes.c_int(tail)))


def mul_mat(w, x, K, M, R, N, wbs, tail=TAIL_STOCK, nthreads=NCPU):
    """y[r*M + m] = dot(w row (r/N)*wbs/K + m, x row r) in ggml order."""
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(R * M, np.float32)
    _l.orc_mul_mat(_ptr(w), _ptr(x), _ptr(y), ctypes.c_int64(K), ctypes.c_int64(M), ctypes.c_int64(R),
                   ctypes.c_int64(N), ctypes.c_int64(wbs), ctypes.c_int(tail), ctypes.c_int(nthreads))
    return y


def dot_general_bnk(lhs_bnk, rhs_bmk, tail=TAIL_STOCK, nthreads=NCPU):
    """out[b, n, m] = dot(lhs[b, n, :], rhs[b, m, :]) for [B,N,K] x [B,M,K] operands."""
    B, N, K = lhs_bnk.shape
    M = rhs_bmk.shape[1]
    y = mul_mat(rhs_bmk.reshape(-1), lhs_bnk.reshape(-1), K, M, B * N, N, M * K if B > 1 else 0, tail, nthreads)
    return y.reshape(B, N, M)


def soft_max(x, scale=1.0, float_sum=False, nthreads=NCPU):
    x = np.ascontiguousarray(x, np.float32)
    cols = x.shape[-1]
    rows = x.size // cols
    y = np.empty_like(x)
    _l.orc_soft_max(_ptr(x), _ptr(y), ctypes.c_int64(rows), ctypes.c_int64(cols), ctypes.c_float(scale),
                    ctypes.c_int(int(float_sum)), ctypes.c_int(nthreads))
    return y


def norm(x, eps=1e-5, gpu_ops=False, nthreads=NCPU):
    x = np.ascontiguousarray(x, np.float32)
    cols = x.shape[-1]
    rows = x.size // cols
    y = np.empty_like(x)
    _l.orc_norm(_ptr(x), _ptr(y), ctypes.c_int64(rows), ctypes.c_int64(cols), ctypes.c_float(eps),
                ctypes.c_int(int(gpu_ops)), ctypes.c_int(nthreads))
    return y


def gelu_erf(x, tanh_form=False, nthreads=NCPU):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    _l.orc_gelu_erf(_ptr(x), _ptr(y), ctypes.c_size_t(x.size), ctypes.c_int(int(tanh_form)), ctypes.c_int(nthreads))
    return y


def silu(x):
    x = np.ascontiguousarray(x, np.float32)
    cols = x.shape[-1]
    y = np.empty_like(x)
    _l.orc_silu(_ptr(x), _ptr(y), ctypes.c_int64(x.size // cols), ctypes.c_int64(cols))
    return y


def ggml_v_expf(x):
    return np.float32(_l.orc_ggml_v_expf(ctypes.c_float(x)))


def expf_cr(x):
    return np.float32(_l.orc_expf_cr(ctypes.c_float(x)))


def erff_cr(x):
    return np.float32(_l.orc_erff_cr(ctypes.c_float(x)))


def erff_range(base, count, nthreads=NCPU):
    out = np.empty(count, np.uint32)
    _l.orc_erff_range(ctypes.c_uint32(base), ctypes.c_uint32(count), _ptr(out), ctypes.c_int(nthreads))
    return out


def checksum_words(words, start_index):
    w = np.ascontiguousarray(words, np.uint32)
    return int(_l.orc_checksum_words(_ptr(w), ctypes.c_size_t(w.size), ctypes.c_uint64(start_index)))


def _u64(a):
    return np.ascontiguousarray(np.asarray(a).view(np.uint64) if np.asarray(a).dtype == np.float64
                                else np.asarray(a, np.uint64))


def f64_ew(op, a, b=None):
    """The reference's soft-float binary64 op (0 add, 1 sub, 2 mul, 3 div,
    4 floor, 5 to int64) on arrays of bit patterns (uint64) or float64;
    returns uint64 bit patterns."""
    a = _u64(a)
    bb = None if b is None else _u64(b)
    out = np.empty(a.shape, np.uint64)
    _l.orc_f64_ew_n(ctypes.c_int(op), _ptr(a), None if bb is None else _ptr(bb), _ptr(out), ctypes.c_size_t(a.size))
    return out


def f64_maxmin(is_max, a, b):
    a, b = _u64(a), _u64(b)
    out = np.empty(a.shape, np.uint64)
    _l.orc_f64_maxmin_n(ctypes.c_int(int(is_max)), _ptr(a), _ptr(b), _ptr(out), ctypes.c_size_t(a.size))
    return out


def f64_of_f32(x):
    x = np.ascontiguousarray(np.asarray(x, np.float32).view(np.uint32))
    out = np.empty(x.shape, np.uint64)
    _l.orc_f64_of_f32_n(_ptr(x), _ptr(out), ctypes.c_size_t(x.size))
    return out


def f32_of_f64(d):
    d = _u64(d)
    out = np.empty(d.shape, np.uint32)
    _l.orc_f32_of_f64_n(_ptr(d), _ptr(out), ctypes.c_size_t(d.size))
    return out


def case_names():
    return [_l.orc_case_name(i).decode() for i in range(_l.orc_case_count())]


def golden_chunks(fn="erff"):
    """{chunk: checksum} of an exhaustive fixture (tests/golden/<fn>_chunks.txt:
    erff, or the row tails' expf)."""
    res = {}
    with open(os.path.join(ROOT, "tests", "golden", f"{fn}_chunks.txt")) as f:
        for line in f:
            if line.startswith("#"):
                continue
            c, _, h = line.split()
            res[int(c)] = int(h, 16)
    return res
