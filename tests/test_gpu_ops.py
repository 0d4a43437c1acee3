"""GPU parity: every ggml_ref case, eager and hipGraph, against the oracle's
fixtures, bit for bit, plus each case's planted wrong lowering (the checks of
the reference's Tests/OpTests.lean:180-222)."""
import numpy as np
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("graph_mode")]


def _tally_case(ref, name, pinned=False):
    import copy

    import shlo_hip
    from shlo_hip import op_tests
    t = op_tests.Tally()
    case = copy.copy([c for c in op_tests.CASES if c.name == name][0])
    if pinned and case.fault == shlo_hip.fault_bits("dot_plain"):
        # With K < 16 the pinned dot product (unfused products added in order
        # to +0) is exactly the sequential sum without FMA, so that planted
        # lowering cannot differ there; the built-in matmul's fused chain does.
        case.fault, case.fault_name = shlo_hip.fault_bits("dot_builtin"), "built-in matmul"
    op_tests.run_case(ref, t, case)
    return t


def _case_names():
    import oracle_py
    return oracle_py.case_names()


CASE_NAMES = [
    "mul_mat_small", "mul_mat_k2", "add_small", "mul_small", "repeat_small", "norm_small", "scale_small",
    "soft_max_small", "soft_max_tail", "gelu_erf_small", "silu_small", "silu_tail", "concat0_small",
    "concat1_small", "concat2_small", "transpose_small", "view_small", "mul_mat_qkv", "mul_mat_ffn2",
    "mul_mat_text", "mul_mat_heading", "mul_mat_root_in", "mul_mat_body_in", "mul_mat_scores", "mul_mat_value",
    "add_kimodo", "mul_kimodo", "repeat_kimodo", "norm_kimodo", "scale_kimodo", "soft_max_kimodo",
    "gelu_erf_kimodo", "silu_kimodo", "concat0_kimodo", "concat1_kimodo", "concat2_kimodo", "transpose_kimodo",
    "view_kimodo",
]


def test_case_list_matches_the_oracle(oracle):
    assert oracle.case_names() == CASE_NAMES


@pytest.mark.parametrize("name", CASE_NAMES)
def test_case_pinned(ref_pinned, name):
    """Pinned flavour: the unfused dot tail and correctly rounded erff."""
    import shlo_hip
    shlo_hip.set_flavor(1)
    try:
        t = _tally_case(ref_pinned, name, pinned=True)
    finally:
        shlo_hip.set_flavor(0)
    bad = [l for ok, l in t.lines if not ok]
    assert bad == [], bad
    assert t.passed >= 1


@pytest.mark.parametrize("name", [n for n in CASE_NAMES if n != "gelu_erf_kimodo"])
def test_case_stock(ref_stock, name):
    """Stock flavour (the reference's own kernel tail); gelu_erf_kimodo's stock
    output comes from Apple's closed erff and is checked in the pinned flavour."""
    import shlo_hip
    assert shlo_hip.get_flavor() == 0
    t = _tally_case(ref_stock, name)
    bad = [l for ok, l in t.lines if not ok]
    assert bad == [], bad


def test_builtin_probes():
    from shlo_hip import op_tests
    t = op_tests.Tally()
    op_tests.builtin_probes(t, n=1 << 18)
    assert [l for ok, l in t.lines if not ok] == []


def test_erff_exhaustive_on_gpu(oracle):
    """The GPU erff on all 2^32 inputs against the MPFR-decided chunk
    checksums; the planted fault (inputs shifted by one) must miss."""
    import shlo_hip
    want = oracle.golden_chunks()
    k = shlo_hip.Kernel("erff_map")
    table = shlo_hip.from_numpy(np.zeros(8, np.float32))
    bad = []
    for c in range(256):
        y = k.apply([table, shlo_hip.u32_arr([c << 24, 1 << 24])], [(1 << 24,)], [shlo_hip.U32])[0]
        if shlo_hip.checksum_u32(y, c << 24) != want[c]:
            bad.append(c)
    assert bad == []
    y = k.apply([table, shlo_hip.u32_arr([(0x3F << 24) + 1, 1 << 24])], [(1 << 24,)], [shlo_hip.U32])[0]
    assert shlo_hip.checksum_u32(y, 0x3F << 24) != want[0x3F]


def test_erff_map_matches_host_routine():
    """A chunk word by word against the host copy (the reference's
    count_nonzero comparison, OpTests.lean:279-288)."""
    import shlo_hip
    base, n = 0x3E800000, 1 << 22
    k = shlo_hip.Kernel("erff_map")
    y = k.apply([shlo_hip.from_numpy(np.zeros(8, np.float32)), shlo_hip.u32_arr([base, n])], [(n,)], [shlo_hip.U32])[0]
    host = shlo_hip.from_numpy(shlo_hip.libm_erff_range(base, n))
    assert shlo_hip.count_nonzero(shlo_hip.binary("ne", y, host)) == 0


def test_expf_exhaustive_on_gpu(oracle):
    """The row tails' expf on the GPU, all 2^32 inputs, against the
    MPFR-decided chunk checksums; inputs shifted by one must miss."""
    import shlo_hip
    want = oracle.golden_chunks("expf")
    k = shlo_hip.Kernel("expf_map")
    bad = []
    for c in range(256):
        y = k.apply([shlo_hip.u32_arr([c << 24, 1 << 24])], [(1 << 24,)], [shlo_hip.U32])[0]
        if shlo_hip.checksum_u32(y, c << 24) != want[c]:
            bad.append(c)
    assert bad == []
    y = k.apply([shlo_hip.u32_arr([(0x3F << 24) + 1, 1 << 24])], [(1 << 24,)], [shlo_hip.U32])[0]
    assert shlo_hip.checksum_u32(y, 0x3F << 24) != want[0x3F]


def test_expf_map_matches_host_routine():
    import shlo_hip
    base, n = 0xC2000000, 1 << 22
    y = shlo_hip.Kernel("expf_map").apply([shlo_hip.u32_arr([base, n])], [(n,)], [shlo_hip.U32])[0]
    host = shlo_hip.from_numpy(shlo_hip.expf_range(base, n))
    assert shlo_hip.count_nonzero(shlo_hip.binary("ne", y, host)) == 0
