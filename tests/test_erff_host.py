"""The executor's erff (the routine its kernels run), evaluated on the host,
against the MPFR-decided fixture on all 2^32 inputs (256 chunk checksums)."""
import ctypes
import os
from multiprocessing import Pool

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "contract-stablehlo-mlx_amd", "shlo_hip", "libshlo_hip.so")
C = np.uint64(0x9E3779B97F4A7C15)


def _checksum(c):
    lib = ctypes.CDLL(LIB)
    out = np.empty(1 << 24, dtype=np.uint32)
    assert lib.shlo_libm_erff_range(ctypes.c_uint32(c << 24), ctypes.c_uint32(1 << 24),
                                    out.ctypes.data_as(ctypes.c_void_p)) == 0
    t = np.arange(c << 24, (c + 1) << 24, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return c, int(np.sum((out.astype(np.uint64) + np.uint64(1)) * (np.uint64(2) * t + np.uint64(1)) * C,
                             dtype=np.uint64))


def test_host_erff_all_inputs(oracle):
    want = oracle.golden_chunks()
    with Pool(min(8, os.cpu_count() or 1)) as p:
        got = dict(p.imap_unordered(_checksum, range(256)))
    assert [c for c in range(256) if got[c] != want[c]] == []
