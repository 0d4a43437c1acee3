"""The graph.txt emitter on the CPU: every case's graph (written by the oracle,
hash-identical to the reference's) becomes a module that parses, with the
generic path's argument types (a leading ui64, then rank-4 f32 tensors in the
case's input order); unsupported graphs are refused by name."""
import os

import pytest


def _cases(ref):
    return sorted(d for d in os.listdir(ref) if os.path.exists(os.path.join(ref, d, "graph.txt")))


def test_every_case_graph_emits_a_module(ref_pinned):
    import shlo_hip
    from shlo_hip import ghlo, op_tests
    names = _cases(ref_pinned)
    assert len(names) == 38
    for n in names:
        d = os.path.join(ref_pinned, n)
        text, args, outs = ghlo.emit(open(os.path.join(d, "graph.txt")).read())
        assert len(outs) == 1, n
        tys = shlo_hip.Module(text).arg_types()
        ins = [ne for k, ne in op_tests.read_meta(d) if k.startswith("in")]
        assert tys[0] == ((), 4), n  # tensor<ui64>
        assert [t for t, _ in tys[1:]] == [(ne[3], ne[2], ne[1], ne[0]) for ne in ins], n
        assert all(dt == shlo_hip.F32 for _, dt in tys[1:]), n


def test_emitter_refuses_what_it_does_not_carry(ref_pinned):
    from shlo_hip import ghlo
    text = open(os.path.join(ref_pinned, "transpose_small", "graph.txt")).read().replace(" TRANSPOSE ", " PERMUTE ")
    with pytest.raises(ghlo.GraphError, match="PERMUTE"):
        ghlo.emit(text)
    with pytest.raises(ghlo.GraphError, match="ghlo-graph 1"):
        ghlo.emit("ghlo-graph 2\n")
