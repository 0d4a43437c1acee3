"""The oracle's correctly rounded erff (orc_erff_cr: binary64 erf with an
exact rounding-boundary test, erfq at 113 bits near a boundary) against the
MPFR-decided fixture on all 2^32 inputs (tests/golden/erff_chunks.txt)."""
import os
from multiprocessing import Pool

NPROC = min(8, os.cpu_count() or 1)


def _chunk(c):
    import oracle_py as oracle
    return c, oracle.checksum_words(oracle.erff_range(c << 24, 1 << 24, nthreads=1), c << 24)


def test_oracle_erff_all_inputs(oracle):
    want = oracle.golden_chunks()
    with Pool(NPROC) as p:
        got = dict(p.imap_unordered(_chunk, range(256)))
    assert [c for c in range(256) if got[c] != want[c]] == []
