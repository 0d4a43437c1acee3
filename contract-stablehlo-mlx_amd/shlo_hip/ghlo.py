"""graph.txt ingestion: ggml's graph description turned into a StableHLO module.

The reference's fixture writer describes each case's ggml graph in
`<case>/graph.txt` ("ghlo-graph 1", ref/ggml_ref.c:94-134; the oracle writes
the same files).  The reference's generic path hands that description to an
external emitter (scripts/GhloEmit.lean, contract-ggml-stablehlo) and runs the
module it writes with a leading `ui64 0` argument and rank-4 tensors
(Tests/OpTests.lean:300-359).  This module is our own emitter for the same
input and the same module shape.  Each ggml node maps to the op that
reproduces ggml-cpu's bits:

    MUL_MAT -> stablehlo.dot_general (ggml order in the executor)
    ADD, MUL -> stablehlo.add, stablehlo.multiply
    REPEAT -> stablehlo.broadcast_in_dim
    SCALE -> constant, broadcast, multiply (and add for a nonzero bias)
    NORM, SOFT_MAX, UNARY GELU_ERF / SILU -> the ggml.* custom calls
    CONCAT -> stablehlo.concatenate
    TRANSPOSE -> stablehlo.transpose; VIEW (a sub-block) -> stablehlo.slice
    CONT -> nothing (StableHLO values have no layout)

Anything else is refused by name, never approximated.

A ggml tensor with ne = [ne0, ne1, ne2, ne3] (ne0 fastest) is the StableHLO
tensor<ne3 x ne2 x ne1 x ne0 x f32>; its bytes are the same row-major array.
"""
import struct

__all__ = ["GTensor", "parse", "emit", "GraphError"]


class GraphError(ValueError):
    """A graph.txt line or node this emitter does not carry."""


class GTensor:
    __slots__ = ("idx", "op", "unary", "node", "output", "type", "ne", "nb", "view_src", "view_offs", "src",
                 "params")

    def __init__(self, w):
        if len(w) != 43 or w[0] != "T":
            raise GraphError(f"graph.txt: a tensor line has 43 fields starting with T, got {len(w)}")
        self.idx = int(w[1])
        self.op, self.unary = w[2], w[3]
        self.node, self.output = int(w[4]) != 0, int(w[5]) != 0
        self.type = w[6]
        self.ne = [int(v) for v in w[7:11]]
        self.nb = [int(v) for v in w[11:15]]
        self.view_src, self.view_offs = int(w[15]), int(w[16])
        self.src = [int(v) for v in w[17:27]]
        self.params = [int(v) for v in w[27:43]]

    def dims(self):
        return (self.ne[3], self.ne[2], self.ne[1], self.ne[0])

    def ty(self):
        return "tensor<" + "".join(f"{d}x" for d in self.dims()) + "f32>"


def parse(text):
    """The tensors of a graph.txt, in file order (index = position)."""
    lines = [l for l in text.splitlines() if l.strip()]
    if not lines or lines[0].strip() != "ghlo-graph 1":
        raise GraphError("graph.txt: the first line must be 'ghlo-graph 1'")
    ts = [GTensor(l.split()) for l in lines[1:]]
    for i, t in enumerate(ts):
        if t.idx != i:
            raise GraphError(f"graph.txt: tensor {i} is numbered {t.idx}")
        if t.type != "f32":
            raise GraphError(f"graph.txt: tensor {i} has type {t.type}; f32 only")
        for s in t.src + [t.view_src]:
            if s >= i:
                raise GraphError(f"graph.txt: tensor {i} reads tensor {s}, which is not before it")
    return ts


def _hex32(b):
    return f"0x{b & 0xFFFFFFFF:08X}"


def _contig(t):
    nb, want = [], 4
    for d in range(4):
        nb.append(want)
        want *= t.ne[d]
    return nb


def emit(text):
    """(module text, argument tensor indices, output tensor indices) for a
    graph.txt.  @main takes a leading tensor<ui64> (unused, as the reference's
    generic modules do) and then the graph's arguments in order."""
    ts = parse(text)
    args = [t.idx for t in ts if not t.node]
    outs = [t.idx for t in ts if t.node and t.output]
    if any(not t.node for t in ts[len(args):]):
        raise GraphError("graph.txt: the arguments must come before the nodes")
    if not outs:
        raise GraphError("graph.txt: no output node")
    name = {i: f"%a{k + 1}" for k, i in enumerate(args)}
    body = []
    tmp = [0]

    def fresh():
        tmp[0] += 1
        return f"%v{tmp[0]}"

    def op1(out_name, line):
        body.append(f"    {out_name} = {line}")

    for t in ts[len(args):]:
        s = [ts[i] if i >= 0 else None for i in t.src]
        v = f"%t{t.idx}"
        if t.op not in ("TRANSPOSE", "VIEW") and t.nb != _contig(t):
            raise GraphError(f"graph.txt: node {t.idx} ({t.op}) is not contiguous")
        if t.op == "MUL_MAT":
            w, x = s[0], s[1]
            K, M = w.ne[0], w.ne[1]
            if x.ne[0] != K or t.ne != [M, x.ne[1], x.ne[2], x.ne[3]]:
                raise GraphError(f"MUL_MAT {t.idx}: shapes do not match")
            if w.ne[2] == 1 and w.ne[3] == 1:
                w2 = fresh()
                op1(w2, f'"stablehlo.reshape"({name[w.idx]}) : ({w.ty()}) -> tensor<{M}x{K}xf32>')
                op1(v, f'"stablehlo.dot_general"({name[x.idx]}, {w2}) {{dot_dimension_numbers = #stablehlo.dot<'
                       f'lhs_contracting_dimensions = [3], rhs_contracting_dimensions = [1]>}} : '
                       f"({x.ty()}, tensor<{M}x{K}xf32>) -> {t.ty()}")
            elif w.ne[2] == x.ne[2] and w.ne[3] == x.ne[3]:
                op1(v, f'"stablehlo.dot_general"({name[x.idx]}, {name[w.idx]}) {{dot_dimension_numbers = '
                       f"#stablehlo.dot<lhs_batching_dimensions = [0, 1], rhs_batching_dimensions = [0, 1], "
                       f"lhs_contracting_dimensions = [3], rhs_contracting_dimensions = [3]>}} : "
                       f"({x.ty()}, {w.ty()}) -> {t.ty()}")
            else:
                raise GraphError(f"MUL_MAT {t.idx}: a weight broadcast over groups is not carried")
        elif t.op in ("ADD", "MUL"):
            a, b = s[0], s[1]
            if a.ne != t.ne or b.ne != t.ne:
                raise GraphError(f"{t.op} {t.idx}: operands of different shapes (ggml broadcasting) are not carried")
            n = "stablehlo.add" if t.op == "ADD" else "stablehlo.multiply"
            op1(v, f'"{n}"({name[a.idx]}, {name[b.idx]}) : ({a.ty()}, {b.ty()}) -> {t.ty()}')
        elif t.op == "REPEAT":
            a = s[0]
            if any(a.ne[d] not in (1, t.ne[d]) for d in range(4)):
                raise GraphError(f"REPEAT {t.idx}: tiling a dimension larger than 1 is not carried")
            op1(v, f'"stablehlo.broadcast_in_dim"({name[a.idx]}) {{broadcast_dimensions = array<i64: 0, 1, 2, 3>}}'
                   f" : ({a.ty()}) -> {t.ty()}")
        elif t.op == "SCALE":
            a = s[0]
            c, cb = fresh(), fresh()
            op1(c, f'"stablehlo.constant"() {{value = dense<{_hex32(t.params[0])}> : tensor<f32>}} : () -> tensor<f32>')
            op1(cb, f'"stablehlo.broadcast_in_dim"({c}) {{broadcast_dimensions = array<i64>}} : (tensor<f32>) -> {t.ty()}')
            if t.params[1] & 0x7FFFFFFF:  # ggml_scale_bias: y = x*s + b, two roundings
                m, d, db = fresh(), fresh(), fresh()
                op1(m, f'"stablehlo.multiply"({name[a.idx]}, {cb}) : ({a.ty()}, {t.ty()}) -> {t.ty()}')
                op1(d, f'"stablehlo.constant"() {{value = dense<{_hex32(t.params[1])}> : tensor<f32>}} : () -> tensor<f32>')
                op1(db, f'"stablehlo.broadcast_in_dim"({d}) {{broadcast_dimensions = array<i64>}} : (tensor<f32>) -> {t.ty()}')
                op1(v, f'"stablehlo.add"({m}, {db}) : ({t.ty()}, {t.ty()}) -> {t.ty()}')
            else:
                op1(v, f'"stablehlo.multiply"({name[a.idx]}, {cb}) : ({a.ty()}, {t.ty()}) -> {t.ty()}')
        elif t.op in ("NORM", "SOFT_MAX") or (t.op == "UNARY" and t.unary in ("GELU_ERF", "SILU")):
            a = s[0]
            if t.op == "NORM":
                target, attrs = "ggml.norm", f"eps = {_hex32(t.params[0])} : f32"
            elif t.op == "SOFT_MAX":
                if s[1] is not None or s[2] is not None or t.params[1] & 0x7FFFFFFF:
                    raise GraphError(f"SOFT_MAX {t.idx}: a mask, sinks or max_bias are not carried")
                target, attrs = "ggml.soft_max", f"scale = {_hex32(t.params[0])} : f32"
            else:
                target, attrs = ("ggml.gelu_erf" if t.unary == "GELU_ERF" else "ggml.silu"), ""
            op1(v, f'"stablehlo.custom_call"({name[a.idx]}) {{call_target_name = "{target}", backend_config = '
                   f'"{attrs}"}} : ({a.ty()}) -> {t.ty()}')
        elif t.op == "CONCAT":
            a, b = s[0], s[1]
            dim = t.params[0]
            if not 0 <= dim < 4:
                raise GraphError(f"CONCAT {t.idx}: dimension {dim}")
            op1(v, f'"stablehlo.concatenate"({name[a.idx]}, {name[b.idx]}) {{dimension = {3 - dim} : i64}} : '
                   f"({a.ty()}, {b.ty()}) -> {t.ty()}")
        elif t.op == "TRANSPOSE":
            a = s[0]
            if t.ne != [a.ne[1], a.ne[0], a.ne[2], a.ne[3]] or t.nb != [a.nb[1], a.nb[0], a.nb[2], a.nb[3]]:
                raise GraphError(f"TRANSPOSE {t.idx}: not a swap of the first two dimensions")
            op1(v, f'"stablehlo.transpose"({name[a.idx]}) {{permutation = array<i64: 0, 1, 3, 2>}} : '
                   f"({a.ty()}) -> {t.ty()}")
        elif t.op == "VIEW":
            a = ts[t.view_src]
            if t.view_src != t.src[0] or a.nb != _contig(a) or t.view_offs % 4:
                raise GraphError(f"VIEW {t.idx}: only views of a contiguous argument are carried")
            if any(t.ne[d] > 1 and t.nb[d] != a.nb[d] for d in range(4)) or t.nb[0] != 4:
                raise GraphError(f"VIEW {t.idx}: only a sub-block of its source is carried")
            o, start = t.view_offs // 4, []
            for d in range(4):
                start.append(o % a.ne[d])
                o //= a.ne[d]
            if o or any(start[d] + t.ne[d] > a.ne[d] for d in range(4)):
                raise GraphError(f"VIEW {t.idx}: the block leaves its source")
            lo = [start[d] for d in (3, 2, 1, 0)]
            hi = [start[d] + t.ne[d] for d in (3, 2, 1, 0)]
            op1(v, f'"stablehlo.slice"({name[a.idx]}) {{start_indices = array<i64: {", ".join(map(str, lo))}>, '
                   f'limit_indices = array<i64: {", ".join(map(str, hi))}>, strides = array<i64: 1, 1, 1, 1>}} : '
                   f"({a.ty()}) -> {t.ty()}")
        elif t.op == "CONT":
            a = s[0]
            if a.ne != t.ne:
                raise GraphError(f"CONT {t.idx}: a reshaping cont is not carried")
            name[t.idx] = name[a.idx]
            continue
        else:
            u = f" {t.unary}" if t.unary != "-" else ""
            raise GraphError(f"graph.txt: op {t.op}{u} (tensor {t.idx}) is not carried")
        name[t.idx] = v
    head = ", ".join(["%a0: tensor<ui64>"] + [f"{name[i]}: {ts[i].ty()}" for i in args])
    rets = ", ".join(ts[i].ty() for i in outs)
    text = ("module {\n  func.func public @main(" + head + ") -> (" + rets + ") {\n" + "\n".join(body) + "\n"
            "    func.return " + ", ".join(name[i] for i in outs) + " : " + rets + "\n  }\n}\n")
    return text, args, outs


def f32_bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]
