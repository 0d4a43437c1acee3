"""GPU parity of element-wise chains fused into dot_general's store.

A dot_general whose result flows only through f32 add / subtract / multiply
/ divide / maximum / minimum ops of its shape runs as one kernel that applies
them to each output before storing it.  Each case here runs such a chain,
eager and hipGraph-compiled, against the oracle's dot followed by the same
IEEE operations in numpy (one rounding each, in the same operand order), and
covers the cases the fusion must decline or cut short: more than four ops, an
operand whose strides do not flatten over the output's (batch, row, column)
groups, intermediate values with other uses, and planted faults."""
import numpy as np
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("graph_mode")]

F32 = np.float32


def t(shape):
    return "tensor<" + "".join(f"{d}x" for d in shape) + "f32>"


def same_bits(a, b):
    return a.shape == b.shape and np.array_equal(np.ascontiguousarray(a).view(np.uint32),
                                                 np.ascontiguousarray(b).view(np.uint32))


def np_binary(op, x, y):
    """The binary32 semantics of the op table (one IEEE rounding; maximum and
    minimum propagate NaN as x + y and order -0 below +0)."""
    x, y = np.asarray(x, F32), np.asarray(y, F32)
    with np.errstate(all="ignore"):
        if op == "add":
            return (x + y).astype(F32)
        if op == "subtract":
            return (x - y).astype(F32)
        if op == "multiply":
            return (x * y).astype(F32)
        if op == "divide":
            return (x / y).astype(F32)
        nan = np.isnan(x) | np.isnan(y)
        eq = x == y
        if op == "maximum":
            pick = np.where(eq, np.where(np.signbit(x), y, x), np.where(x > y, x, y))
        else:
            pick = np.where(eq, np.where(np.signbit(x), x, y), np.where(x < y, x, y))
        return np.where(nan, x + y, pick).astype(F32)


class Chain:
    """dot_general of [*batch, N, K] x [*batch, K, M] (or its transposed
    contraction), then ops [(name, arg, how, rev)]: arg is an extra function
    argument; how = None (already the output shape), ("bcast", dims) for a
    broadcast_in_dim, or ("perm", perm) for a transpose; rev puts the running
    value on the right."""

    def __init__(self, batch, N, K, M, ops, rhs_mk=False, extra_returns=()):
        self.batch, self.N, self.K, self.M, self.ops = tuple(batch), N, K, M, ops
        self.rhs_mk, self.extra = rhs_mk, extra_returns

    @property
    def out_shape(self):
        return self.batch + (self.N, self.M)

    def module(self):
        nb = len(self.batch)
        a_sh = self.batch + (self.N, self.K)
        b_sh = self.batch + ((self.M, self.K) if self.rhs_mk else (self.K, self.M))
        o = self.out_shape
        bd = list(range(nb))
        dn = (f"#stablehlo.dot<lhs_batching_dimensions = {bd}, rhs_batching_dimensions = {bd}, "
              f"lhs_contracting_dimensions = [{nb + 1}], rhs_contracting_dimensions = "
              f"[{nb + 1 if self.rhs_mk else nb}]>")
        args = [f"%a: {t(a_sh)}", f"%b: {t(b_sh)}"]
        lines = [f'    %v0 = "stablehlo.dot_general"(%a, %b) {{dot_dimension_numbers = {dn}}} : '
                 f"({t(a_sh)}, {t(b_sh)}) -> {t(o)}\n"]
        cur = "%v0"
        names = ["%v0"]
        for i, (name, arg, how, rev) in enumerate(self.ops):
            if name == "gelu":  # ggml.gelu_erf, no operand
                lines.append(f'    %v{i + 1} = "stablehlo.custom_call"({cur}) {{call_target_name = "ggml.gelu_erf", '
                             f'backend_config = ""}} : ({t(o)}) -> {t(o)}\n')
                cur = f"%v{i + 1}"
                names.append(cur)
                continue
            args.append(f"%x{i}: {t(arg.shape)}")
            other = f"%x{i}"
            if how is not None and how[0] == "bcast":
                dims = ", ".join(str(d) for d in how[1])
                lines.append(f'    %b{i} = "stablehlo.broadcast_in_dim"(%x{i}) {{broadcast_dimensions = '
                             f"array<i64{': ' + dims if dims else ''}>}} : ({t(arg.shape)}) -> {t(o)}\n")
                other = f"%b{i}"
            elif how is not None and how[0] == "perm":
                perm = ", ".join(str(d) for d in how[1])
                lines.append(f'    %b{i} = "stablehlo.transpose"(%x{i}) {{permutation = array<i64: {perm}>}} : '
                             f"({t(arg.shape)}) -> {t(o)}\n")
                other = f"%b{i}"
            l, r = (other, cur) if rev else (cur, other)
            lines.append(f'    %v{i + 1} = "stablehlo.{name}"({l}, {r}) : ({t(o)}, {t(o)}) -> {t(o)}\n')
            cur = f"%v{i + 1}"
            names.append(cur)
        rets = [cur] + [names[k] for k in self.extra]
        sig = ", ".join(t(o) for _ in rets)
        return (f"module {{\n  func.func public @main({', '.join(args)}) -> ({sig}) {{\n" + "".join(lines) +
                f"    func.return {', '.join(rets)} : {sig}\n  }}\n}}\n")

    def expect(self, oracle, a, b, tail):
        B = int(np.prod(self.batch)) if self.batch else 1
        lhs = a.reshape(B, self.N, self.K)
        rhs = b.reshape(B, self.M, self.K) if self.rhs_mk else \
            np.ascontiguousarray(b.reshape(B, self.K, self.M).transpose(0, 2, 1))
        v = oracle.dot_general_bnk(np.ascontiguousarray(lhs), np.ascontiguousarray(rhs), tail)
        v = v.reshape(self.out_shape)
        vals = [v]
        o = self.out_shape
        for name, arg, how, rev in self.ops:
            if name == "gelu":
                v = oracle.gelu_erf(np.ascontiguousarray(v, F32)).reshape(o)
                vals.append(v)
                continue
            if how is None:
                other = arg
            elif how[0] == "bcast":
                shp = [1] * len(o)
                for k, d in enumerate(how[1]):
                    shp[d] = arg.shape[k]
                other = np.broadcast_to(arg.reshape(shp), o)
            else:
                other = arg.transpose(how[1])
            v = np_binary(name, other, v) if rev else np_binary(name, v, other)
            vals.append(v)
        return [v] + [vals[k] for k in self.extra]


def run(text, inputs, faults=0, compile=True):
    import shlo_hip
    f = shlo_hip.Module(text).prepare(faults, compile)
    return [o.numpy() for o in f.call([shlo_hip.from_numpy(np.ascontiguousarray(x)) for x in inputs])]


def normal(oracle, seed, shape, sigma=1.0):
    x, _ = oracle.fill_normal(seed, sigma, int(np.prod(shape)))
    return x.reshape(shape)


def check(oracle, ch, seed=5, flavors=(0, 1)):
    import shlo_hip
    a_sh = ch.batch + (ch.N, ch.K)
    b_sh = ch.batch + ((ch.M, ch.K) if ch.rhs_mk else (ch.K, ch.M))
    a, b = normal(oracle, seed, a_sh), normal(oracle, seed + 1, b_sh)
    ins = [a, b] + [arg for name, arg, _, _ in ch.ops if name != "gelu"]
    text = ch.module()
    for flavor in flavors:
        want = ch.expect(oracle, a, b, flavor)
        shlo_hip.set_flavor(flavor)
        try:
            for compile in (True, False):
                got = run(text, ins, compile=compile)
                assert len(got) == len(want)
                for g, w in zip(got, want):
                    assert same_bits(g, w), (flavor, compile)
        finally:
            shlo_hip.set_flavor(0)
    return text, ins


def scalar(v):
    return np.array(v, F32)


@pytest.mark.parametrize("S,K", [(70, 64), (128, 64), (96, 33)])
def test_attention_scale_and_mask(oracle, S, K):
    """Q K^T [2,3,S,S] (contraction over both operands' last dim), times a
    broadcast scalar, plus a broadcast causal mask [S,S] over dims 2, 3."""
    mask = np.where(np.triu(np.ones((S, S), bool), 1), F32(-np.inf), F32(0))
    ch = Chain((2, 3), S, K, S, [("multiply", scalar(0.125), ("bcast", ()), False),
                                 ("add", mask, ("bcast", (2, 3)), False)], rhs_mk=True)
    check(oracle, ch)


@pytest.mark.parametrize("N,K,M", [(256, 64, 192), (130, 512, 70), (64, 1024, 128), (33, 17, 9)])
def test_bias_and_residual(oracle, N, K, M):
    """x W + bias (broadcast over rows), then a residual on the left (rev):
    the four-wave kernel (K <= 512), the eight-wave kernel, partial tiles and
    row tails."""
    bias = normal(oracle, 9, (M,), 0.5)
    res = normal(oracle, 10, (N, M))
    ch = Chain((), N, K, M, [("add", bias, ("bcast", (1,)), False), ("add", res, None, True)])
    check(oracle, ch)


@pytest.mark.parametrize("name", ["subtract", "divide", "maximum", "minimum"])
@pytest.mark.parametrize("rev", [False, True])
def test_each_op_both_orders(oracle, name, rev):
    """Each fusable op with the dot's value on either side; the other operand
    holds zeros of both signs, infinities, NaN, subnormals and values equal to
    the dot's outputs."""
    N, K, M = 96, 48, 80
    other = normal(oracle, 12, (N, M))
    flat = other.reshape(-1)
    flat[::7] = 0.0
    flat[1::7] = -0.0
    flat[2::11] = np.inf
    flat[3::11] = -np.inf
    flat[4::13] = np.nan
    flat[5::13] = np.float32(1e-40)
    a, b = normal(oracle, 5, (N, K)), normal(oracle, 6, (K, M))
    v = oracle.dot_general_bnk(a[None], np.ascontiguousarray(b.T)[None], 0)[0]
    flat[6::17] = v.reshape(-1)[6::17]  # equal operands (maximum / minimum pick by sign)
    ch = Chain((), N, K, M, [(name, other, None, rev)])
    check(oracle, ch, flavors=(0,))


def test_longer_chain_than_fused(oracle):
    """Six ops: the first four fuse, the rest run as separate kernels."""
    N, K, M = 128, 64, 128
    ops = [("add", normal(oracle, 20, (M,)), ("bcast", (1,)), False),
           ("multiply", scalar(1.5), ("bcast", ()), False),
           ("subtract", normal(oracle, 21, (N, M)), None, True),
           ("maximum", normal(oracle, 22, (N,)), ("bcast", (0,)), False),
           ("divide", normal(oracle, 23, (N, M)), None, False),
           ("minimum", scalar(0.75), ("bcast", ()), True)]
    check(oracle, Chain((), N, K, M, ops))


def test_operand_strides_that_do_not_flatten(oracle):
    """An operand transposed across the two batch dims has no single batch
    stride: the chain stops there and the op runs on its own."""
    B1, B2, N, K, M = 3, 2, 64, 32, 64
    tr = normal(oracle, 30, (B2, B1, N, M))
    ops = [("add", normal(oracle, 31, (M,)), ("bcast", (3,)), False),
           ("add", tr, ("perm", (1, 0, 2, 3)), False),
           ("multiply", normal(oracle, 32, (B1, B2, N, M)), None, True)]
    check(oracle, Chain((B1, B2), N, K, M, ops))


def test_transposed_operand_flattens(oracle):
    """A transposed [M,N] operand over an [N,M] output has strides (1, N): one
    dim per group, so it fuses."""
    N, K, M = 96, 64, 160
    ch = Chain((), N, K, M, [("add", normal(oracle, 32, (M, N)), ("perm", (1, 0)), False)])
    check(oracle, ch)


def test_intermediate_with_another_use(oracle):
    """The first op's result is also returned: the chain ends there."""
    N, K, M = 64, 64, 64
    ops = [("add", normal(oracle, 40, (N, M)), None, False), ("multiply", normal(oracle, 41, (N, M)), None, False)]
    check(oracle, Chain((), N, K, M, ops, extra_returns=(1,)))


def test_dot_result_with_two_uses(oracle):
    """The dot's own value is returned too: nothing fuses."""
    N, K, M = 64, 32, 64
    ops = [("add", normal(oracle, 42, (N, M)), None, False)]
    check(oracle, Chain((), N, K, M, ops, extra_returns=(0,)))


def test_many_batches_simple_kernel(oracle):
    """More than 65535 batches take the one-thread-per-output kernel, which
    applies the same chain."""
    B, N, K, M = 70000, 1, 20, 2
    ops = [("add", normal(oracle, 43, (M,)), ("bcast", (2,)), False),
           ("multiply", normal(oracle, 44, (B,)), ("bcast", (0,)), True)]
    check(oracle, Chain((B,), N, K, M, ops), flavors=(1,))


def test_planted_faults_still_differ(oracle):
    import shlo_hip
    N, K, M = 64, 64, 64
    ch = Chain((), N, K, M, [("add", normal(oracle, 50, (M,)), ("bcast", (1,)), False),
                             ("divide", normal(oracle, 51, (N, M)), None, False)])
    text, ins = check(oracle, ch, flavors=(0,))
    want = ch.expect(oracle, ins[0], ins[1], 0)[0]
    for fault in ("dot_plain", "dot_builtin", "binary_half", "divide_builtin", "broadcast_first"):
        got = run(text, ins, faults=shlo_hip.fault_bits(fault))[0]
        assert not same_bits(got, want), fault


@pytest.mark.parametrize("N,K,M", [(256, 512, 192), (130, 1024, 70), (128, 1024, 128), (33, 33, 9), (64, 16, 64)])
def test_bias_then_gelu(oracle, N, K, M):
    """x W + bias, then ggml.gelu_erf (the FFN's first projection): the
    correctly rounded erff runs in the product's epilogue (table in LDS, or read through the cache in the four-wave kernel);
    the four-wave and eight-wave kernels, partial tiles and tails."""
    bias = normal(oracle, 60, (M,), 0.5)
    check(oracle, Chain((), N, K, M, [("add", bias, ("bcast", (1,)), False), ("gelu", None, None, False)]))


def test_gelu_inside_a_chain(oracle):
    """gelu_erf between binary ops, special values in the operands."""
    N, K, M = 96, 64, 96
    res = normal(oracle, 61, (N, M), 3.0)
    res.reshape(-1)[::17] = np.nan
    res.reshape(-1)[1::19] = np.inf
    ops = [("multiply", scalar(4.0), ("bcast", ()), False), ("gelu", None, None, False),
           ("add", res, None, True), ("gelu", None, None, False)]
    check(oracle, Chain((), N, K, M, ops))


def test_gelu_with_many_batches(oracle):
    """More than 65535 batches: the one-thread-per-output kernel's table."""
    B, N, K, M = 70000, 1, 20, 2
    check(oracle, Chain((B,), N, K, M, [("gelu", None, None, False)]), flavors=(0,))


def test_planted_gelu_fault_still_differs(oracle):
    import shlo_hip
    N, K, M = 64, 64, 64
    ch = Chain((), N, K, M, [("add", normal(oracle, 62, (M,)), ("bcast", (1,)), False), ("gelu", None, None, False)])
    text, ins = check(oracle, ch, flavors=(0,))
    want = ch.expect(oracle, ins[0], ins[1], 0)[0]
    got = run(text, ins, faults=shlo_hip.fault_bits("gelu_tanh"))[0]
    assert not same_bits(got, want)


def _erff_exception_keys():
    """|x| bits of the inputs erff_cr.h decides through its exception table
    (the rounding of its binary64 value is undecided there)."""
    import os
    import re
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "contract-stablehlo-mlx_amd", "csrc",
                        "erff_exceptions.h")
    with open(path) as f:
        return [int(k, 16) for k, _ in re.findall(r"\{0x([0-9A-F]+)u, 0x([0-9A-F]+)u\}", f.read())]


def _gelu_inputs_on_exceptions():
    """GELU inputs x whose erff argument RN(x * SQRT_2_INV) is an exception
    key (both signs): the fused GELU's shared branch into the table."""
    c = np.array([0x3F3504F3], np.uint32).view(F32)[0]
    out = []
    for k in _erff_exception_keys():
        a = np.array([k], np.uint32).view(F32)[0]
        x0 = F32(np.float64(a) / np.float64(c))
        cand = [x0]
        for _ in range(3):
            cand += [np.nextafter(cand[-1], F32(np.inf)), np.nextafter(cand[0], F32(0))]
        for x in cand:
            if F32(x * c) == a:
                out += [x, -x]
                break
    return np.array(out, F32)


@pytest.mark.parametrize("N,K,M,kernel", [(256, 512, 192, "dot_mfma8d_k<RowVecB,ColQuadB,64,4>"),
                                          (128, 132, 128, "dot_mfma8d_k<RowVecB,ColQuadB,64,4>"),
                                          (128, 1024, 192, "dot_mfma8d_k<RowVecB,ColQuadB,128,8>"),
                                          (130, 1024, 70, "dot_mfma8_k<"),
                                          (33, 33, 9, None)])
def test_gelu_on_exception_inputs_and_nan_payloads(oracle, N, K, M, kernel):
    """[x 0, + operand, gelu_erf]: the GELU's input is the operand exactly, so
    every value below reaches it: inputs whose erff takes the exception table,
    NaN payloads (quiet and signalling, both signs), +-inf, +-0, subnormals and
    values past erf's clamp.  The matrix kernels evaluate a lane's eight
    GELUs together (one branch into the table, NaN through the clamp), with
    the erff table staged in LDS after the products (the four-wave direct
    kernel, whole tiles), read from global memory (the same with a tail),
    or staged in LDS from the start (the eight-wave direct kernel, the
    register-staged kernel); the kernel of the last shape evaluates them one
    at a time."""
    exc = _gelu_inputs_on_exceptions()
    assert len(exc) >= 100, len(exc)
    special = np.array([0x7FC00000, 0xFFC00001, 0x7F800001, 0xFF812345, 0x7FFFFFFF, 0x7F800000, 0xFF800000,
                        0x00000000, 0x80000000, 0x00000001, 0x807FFFFF, 0x00400000, 0x7F7FFFFF, 0xC0A00000,
                        0x40800000, 0x3F800000], np.uint32).view(F32)
    res = normal(oracle, 63, (N, M), 2.0)
    flat = res.reshape(-1)
    vals = np.concatenate([exc, special])
    rng = np.random.default_rng(7)
    pos = rng.permutation(flat.size)[:min(flat.size, 3 * vals.size)]
    flat[pos] = np.resize(vals, pos.size)
    ops = [("multiply", scalar(0.0), ("bcast", ()), False), ("add", res, None, False), ("gelu", None, None, False)]
    text, ins = check(oracle, Chain((), N, K, M, ops))
    if kernel is not None:
        import shlo_hip
        run(text, ins, compile=False)
        assert shlo_hip.last_dot_kernel().startswith(kernel), shlo_hip.last_dot_kernel()
