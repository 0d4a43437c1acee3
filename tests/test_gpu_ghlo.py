"""The generic path on the GPU (OpTests.lean:303-359 over graph.txt): every
case's ggml graph emitted as a module with a leading ui64 0 and rank-4
tensors, run compiled, bit for bit against the case's out.f32, and with a
planted executor fault that must change it."""
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("graph_mode")]


def _names():
    import oracle_py
    return oracle_py.case_names()


@pytest.mark.parametrize("name", _names())
def test_ghlo_case_pinned(ref_pinned, name):
    import shlo_hip
    from shlo_hip import op_tests
    shlo_hip.set_flavor(1)
    try:
        t = op_tests.Tally()
        op_tests.ghlo_case(ref_pinned, t, name)
    finally:
        shlo_hip.set_flavor(0)
    assert [l for ok, l in t.lines if not ok] == []
    assert t.passed >= 2


@pytest.mark.parametrize("name", [n for n in _names() if n != "gelu_erf_kimodo"])
def test_ghlo_case_stock(ref_stock, name):
    """Stock flavour: row tails are refused (Apple's expf), as the reference
    refuses them; gelu_erf_kimodo's stock output needs Apple's erff and is
    left out."""
    from shlo_hip import op_tests
    t = op_tests.Tally()
    op_tests.ghlo_case(ref_stock, t, name, expect_refusal=name in ("soft_max_tail", "silu_tail"))
    assert [l for ok, l in t.lines if not ok] == []
