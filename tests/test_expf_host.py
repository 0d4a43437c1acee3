"""The row tails' correctly rounded expf (the routine the kernels run),
evaluated on the host, against the MPFR-decided fixture on all 2^32 inputs
(256 chunk checksums, tests/golden/expf_chunks.txt)."""
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
    assert lib.shlo_expf_range(ctypes.c_uint32(c << 24), ctypes.c_uint32(1 << 24),
                               out.ctypes.data_as(ctypes.c_void_p)) == 0
    t = np.arange(c << 24, (c + 1) << 24, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return c, int(np.sum((out.astype(np.uint64) + np.uint64(1)) * (np.uint64(2) * t + np.uint64(1)) * C,
                             dtype=np.uint64))


def test_host_expf_all_inputs(oracle):
    want = oracle.golden_chunks("expf")
    with Pool(min(8, os.cpu_count() or 1)) as p:
        got = dict(p.imap_unordered(_checksum, range(256)))
    assert [c for c in range(256) if got[c] != want[c]] == []


def test_host_expf_special_values(oracle):
    """Thresholds and specials against the oracle's expf (libquadmath)."""
    import struct
    pats = [0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x42B17217, 0x42B17218, 0xC2CFF1B4, 0xC2CFF1B5,
            0x3F800000, 0xBF800000, 0x33800000, 0xB3800000, 0x00000001, 0x80000001, 0x42AEAC50, 0xC2AEAC50]
    lib = ctypes.CDLL(LIB)
    for b in pats:
        out = np.empty(1, dtype=np.uint32)
        assert lib.shlo_expf_range(ctypes.c_uint32(b), ctypes.c_uint32(1), out.ctypes.data_as(ctypes.c_void_p)) == 0
        x = struct.unpack("<f", struct.pack("<I", b))[0]
        want = np.float32(oracle.expf_cr(x)).view(np.uint32)
        assert int(out[0]) == int(want), hex(b)
