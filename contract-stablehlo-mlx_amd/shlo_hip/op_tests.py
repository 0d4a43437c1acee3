"""op_tests — every ggml op case against ggml-cpu's fixtures, bit for bit, on the GPU.

    python -m shlo_hip.op_tests <ref-dir> [case ...]

The surface of the reference's Tests/OpTests.lean: <ref-dir> holds one
directory per case (in<i>.f32, out.f32, meta.txt, as ref/ggml_ref.c writes
them).  For each case the StableHLO module for that ggml op is built, run
through the executor twice (hipGraph-compiled and eager) and compared word
for word with out.f32; then the case's planted wrong lowering must give
different bits or refuse to run.  Cases whose rows ggml-cpu finishes with
code this executor does not carry must be refused with "not carried".
A missing reference is a FAIL, not a skip.  Prints PASS/FAIL lines and
"N passed, M failed"; exits 0 only if nothing failed.
"""
import os
import struct
import sys
import time

import numpy as np

from . import (F32, FAULTS, Module, ShloError, U32, binary, count_nonzero, fault_bits, from_numpy, get_flavor,
               libm_erff_range, Kernel, set_flavor, u32_arr, unary)


def ty_of(ne):
    """ggml ne (fastest first) as a rank-3 MLIR type (slowest first)."""
    return (ne[2], ne[1], ne[0])


def ty_str(dims, el="f32"):
    return "tensor<" + "".join(f"{d}x" for d in dims) + el + ">"


def hex32(b):
    return f"0x{b & 0xFFFFFFFF:08X}"


def fn_header(args, outs):
    a = ", ".join(f"%a{i}: {ty_str(t)}" for i, t in enumerate(args))
    o = ", ".join(ty_str(t) for t in outs)
    return "module {\n  func.func public @main(" + a + ") -> (" + o + ") {\n"


def fn_footer(r, t):
    return f"    func.return {r} : {ty_str(t)}\n  }}\n}}\n"


def unary_call(target, attrs, t):
    return (fn_header([t], [t]) +
            f'    %0 = "stablehlo.custom_call"(%a0) {{call_target_name = "{target}", backend_config = "{attrs}"}}'
            f" : ({ty_str(t)}) -> {ty_str(t)}\n" + fn_footer("%0", t))


def f32_bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def module_for(op, ins, out):
    """The StableHLO for one ggml op from the case's shapes (OpTests.lean:52-97)."""
    to = ty_of(out)
    if op == "mul_mat":
        w, x = ins[0], ins[1]
        tw, tx = ty_of(w), ty_of(x)
        tr = (x[2], x[1], w[2], w[1])
        return (fn_header([tw, tx], [to]) +
                f'    %0 = "stablehlo.dot_general"(%a1, %a0) {{dot_dimension_numbers = #stablehlo.dot<'
                f"lhs_contracting_dimensions = [2], rhs_contracting_dimensions = [2]>}} : "
                f"({ty_str(tx)}, {ty_str(tw)}) -> {ty_str(tr)}\n"
                f'    %1 = "stablehlo.reshape"(%0) : ({ty_str(tr)}) -> {ty_str(to)}\n' + fn_footer("%1", to))
    if op in ("add", "mul"):
        n = "stablehlo.add" if op == "add" else "stablehlo.multiply"
        return (fn_header([to, to], [to]) +
                f'    %0 = "{n}"(%a0, %a1) : ({ty_str(to)}, {ty_str(to)}) -> {ty_str(to)}\n' + fn_footer("%0", to))
    if op == "repeat":
        ti = ty_of(ins[0])
        return (fn_header([ti], [to]) +
                f'    %0 = "stablehlo.broadcast_in_dim"(%a0) {{broadcast_dimensions = array<i64: 0, 1, 2>}} : '
                f"({ty_str(ti)}) -> {ty_str(to)}\n" + fn_footer("%0", to))
    if op == "scale":
        # Kimodo's attention scale, 1/sqrt(head_width), in binary32 as ggml_ref does
        s = np.float32(1.0) / np.sqrt(np.float32(128.0))
        return (fn_header([to], [to]) +
                f'    %0 = "stablehlo.constant"() {{value = dense<{hex32(f32_bits(s))}> : tensor<f32>}} : () -> tensor<f32>\n'
                f'    %1 = "stablehlo.broadcast_in_dim"(%0) {{broadcast_dimensions = array<i64>}} : (tensor<f32>) -> {ty_str(to)}\n'
                f'    %2 = "stablehlo.multiply"(%a0, %1) : ({ty_str(to)}, {ty_str(to)}) -> {ty_str(to)}\n' +
                fn_footer("%2", to))
    if op == "norm":
        return unary_call("ggml.norm", "eps = 0x3727C5AC : f32", to)  # 1e-5f, Kimodo's eps
    if op == "soft_max":
        return unary_call("ggml.soft_max", "scale = 0x3F800000 : f32", to)
    if op == "gelu_erf":
        return unary_call("ggml.gelu_erf", "", to)
    if op == "silu":
        return unary_call("ggml.silu", "", to)
    if op in ("concat0", "concat1", "concat2"):
        d = 2 - int(op[6:])
        ta, tb = ty_of(ins[0]), ty_of(ins[1])
        return (fn_header([ta, tb], [to]) +
                f'    %0 = "stablehlo.concatenate"(%a0, %a1) {{dimension = {d} : i64}} : '
                f"({ty_str(ta)}, {ty_str(tb)}) -> {ty_str(to)}\n" + fn_footer("%0", to))
    if op == "transpose":
        ti = ty_of(ins[0])
        return (fn_header([ti], [to]) +
                f'    %0 = "stablehlo.transpose"(%a0) {{permutation = array<i64: 0, 2, 1>}} : '
                f"({ty_str(ti)}) -> {ty_str(to)}\n" + fn_footer("%0", to))
    raise ValueError(f"no module builder for {op}")


def view_module(inp, out, off):
    """The view cases need the offset, which the shapes do not carry (OpTests.lean:101-106)."""
    ti, to = ty_of(inp), ty_of(out)
    return (fn_header([ti], [to]) +
            f'    %0 = "stablehlo.slice"(%a0) {{start_indices = array<i64: 0, 0, {off}>, limit_indices = '
            f"array<i64: 1, {out[1]}, {off + out[0]}>, strides = array<i64: 1, 1, 1>}} : "
            f"({ty_str(ti)}) -> {ty_str(to)}\n" + fn_footer("%0", to))


class Case:
    def __init__(self, name, op, fault, fault_name, view_offset=0, expect_refusal=False):
        self.name, self.op, self.fault, self.fault_name = name, op, fault, fault_name
        self.view_offset, self.expect_refusal = view_offset, expect_refusal


def _cases():
    """Every ggml_ref case with its planted fault (OpTests.lean:119-139)."""
    mm = lambda n: Case(n, "mul_mat", fault_bits("dot_builtin"), "built-in matmul")
    mm_plain = lambda n: Case(n, "mul_mat", fault_bits("dot_plain"), "sequential sum without FMA")
    cs = [mm_plain("mul_mat_small"), mm_plain("mul_mat_k2"), mm("mul_mat_qkv"), mm("mul_mat_ffn2"),
          mm("mul_mat_text"), mm_plain("mul_mat_heading"), mm("mul_mat_root_in"), mm("mul_mat_body_in"),
          mm("mul_mat_scores"), mm("mul_mat_value")]
    half = fault_bits("binary_half")
    cs += [Case(n, "add", half, "float16 arithmetic") for n in ("add_small", "add_kimodo")]
    cs += [Case(n, "mul", half, "float16 arithmetic") for n in ("mul_small", "mul_kimodo")]
    cs += [Case(n, "scale", half, "float16 arithmetic") for n in ("scale_small", "scale_kimodo")]
    cs += [Case(n, "repeat", fault_bits("broadcast_first"), "broadcast of the first element")
           for n in ("repeat_small", "repeat_kimodo")]
    cs += [Case(n, "norm", fault_bits("norm_gpu_ops"), "binary32 sums and GPU / and sqrt")
           for n in ("norm_small", "norm_kimodo")]
    cs += [Case(n, "soft_max", fault_bits("soft_max_float_sum"), "binary32 denominator")
           for n in ("soft_max_small", "soft_max_kimodo")]
    # refused as the reference refuses them in the stock flavour; carried with
    # the correctly rounded expf in the pinned flavour
    cs += [Case("soft_max_tail", "soft_max", fault_bits("soft_max_float_sum"), "binary32 denominator",
                expect_refusal="stock")]
    cs += [Case(n, "gelu_erf", fault_bits("gelu_tanh"), "tanh-form GELU") for n in ("gelu_erf_small", "gelu_erf_kimodo")]
    cs += [Case(n, "silu", fault_bits("silu_gpu_ops"), "GPU exp and /") for n in ("silu_small", "silu_kimodo")]
    cs += [Case("silu_tail", "silu", fault_bits("silu_gpu_ops"), "GPU exp and /", expect_refusal="stock")]
    cs += [Case(n, o, fault_bits("concat_swap"), "operands swapped") for n, o in (
        ("concat0_small", "concat0"), ("concat1_small", "concat1"), ("concat2_small", "concat2"),
        ("concat0_kimodo", "concat0"), ("concat1_kimodo", "concat1"), ("concat2_kimodo", "concat2"))]
    cs += [Case(n, "transpose", fault_bits("transpose_identity"), "no permutation")
           for n in ("transpose_small", "transpose_kimodo")]
    cs += [Case("view_small", "view", fault_bits("slice_shift"), "offset one late", view_offset=8),
           Case("view_kimodo", "view", fault_bits("slice_shift"), "offset one late", view_offset=1024 + 3 * 128)]
    return cs


CASES = _cases()


def read_meta(d):
    res = []
    with open(os.path.join(d, "meta.txt")) as f:
        for line in f:
            ws = line.split()
            if ws:
                res.append((ws[0], [int(x) for x in ws[1:]]))
    return res


def diff(a: bytes, b: bytes):
    """Compare as binary32 words: (mismatches, first index)."""
    if len(a) != len(b):
        return max(len(a), len(b)), 0
    x = np.frombuffer(a, dtype=np.uint32)
    y = np.frombuffer(b, dtype=np.uint32)
    ne = np.nonzero(x != y)[0]
    return int(ne.size), (int(ne[0]) if ne.size else None)


def word(b, k):
    return struct.unpack_from("<I", b, 4 * k)[0]


def run_module(text, ins, faults, compile):
    """OpTests.runModule: load, prepare, call, toBytes of the first output."""
    try:
        m = Module(text)
        f = m.prepare(faults, compile)
        outs = f.call(ins)
        return True, outs[0].to_bytes()
    except ShloError as e:
        return False, str(e)


class Tally:
    def __init__(self, out=sys.stdout):
        self.passed, self.failed, self.lines, self.out = 0, 0, [], out

    def note(self, ok, line):
        print(("PASS " if ok else "FAIL ") + line, file=self.out, flush=True)
        self.lines.append((ok, line))
        if ok:
            self.passed += 1
        else:
            self.failed += 1


def load_inputs(d, in_meta):
    ins = []
    for n, ne in in_meta:
        a = np.fromfile(os.path.join(d, f"{n}.f32"), dtype=np.float32).reshape(ty_of(ne))
        ins.append(from_numpy(a))
    return ins


def run_case(ref, t: Tally, c: Case):
    """OpTests.runCase (OpTests.lean:180-222)."""
    d = os.path.join(ref, c.name)
    if not os.path.exists(os.path.join(d, "meta.txt")):
        t.note(False, f"{c.name}: reference missing ({d})")
        return
    md = read_meta(d)
    in_meta = [(n, ne) for n, ne in md if n.startswith("in")]
    out_ne = [ne for n, ne in md if n == "out"]
    if not out_ne:
        t.note(False, f"{c.name}: no out in meta")
        return
    out_ne = out_ne[0]
    text = view_module(in_meta[0][1], out_ne, c.view_offset) if c.op == "view" else \
        module_for(c.op, [ne for _, ne in in_meta], out_ne)
    ins = load_inputs(d, in_meta)
    with open(os.path.join(d, "out.f32"), "rb") as f:
        want = f.read()
    count = len(want) // 4
    if c.expect_refusal is True or (c.expect_refusal == "stock" and get_flavor() == 0):
        ok, r = run_module(text, ins, 0, True)
        if not ok:
            t.note("not carried" in r, f"{c.name}: GAP, refused as expected: {r}")
        else:
            t.note(False, f"{c.name}: ran, but it reaches code this executor does not carry")
        return
    for compile in (True, False):
        mode = "compiled" if compile else "uncompiled"
        t0 = time.perf_counter()
        ok, r = run_module(text, ins, 0, compile)
        ms = (time.perf_counter() - t0) * 1e3
        if not ok:
            t.note(False, f"{c.name} [{mode}]: did not run: {r}")
            continue
        n, first = diff(r, want)
        detail = f" first at {first}: got {hex32(word(r, first))} want {hex32(word(want, first))}" if first is not None else ""
        t.note(n == 0, f"{c.name} [{mode}]: {n} of {count} words differ{detail} ({ms:.3f} ms incl. trace)")
    ok, r = run_module(text, ins, c.fault, True)
    if not ok:
        t.note(True, f"{c.name} planted fault ({c.fault_name}): refused to run: {r[:120]}")
    else:
        n, _ = diff(r, want)
        t.note(n != 0, f"{c.name} planted fault ({c.fault_name}): {n} of {count} words differ (must be > 0)")


# ---- checks with no ggml graph -------------------------------------------------------

def random_normals(n, seed, max_exp=254):
    """Random binary32 bit patterns of finite normal values (OpTests.lean:228-238)."""
    out = np.empty(n, dtype=np.uint32)
    s = seed & 0xFFFFFFFF
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        a = s
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        e = 1 + (s >> 8) % max_exp
        out[i] = (a & 0x807FFFFF) | (e << 23)
    return out


def builtin_probes(t: Tally, n=1 << 20):
    """The exact divide and sqrt against the host's IEEE binary32 (OpTests.lean:240-270)."""
    a = random_normals(n, 7, 200)
    b = random_normals(n, 11, 200)
    fa, fb = a.view(np.float32), b.view(np.float32)
    absa = (a & 0x7FFFFFFF).view(np.float32)
    want_div = (fa / fb).view(np.uint32)
    want_sqrt = np.sqrt(absa).view(np.uint32)
    da, db, dabs = from_numpy(fa), from_numpy(fb), from_numpy(absa)
    exact_div = Kernel("divide").apply([da, db, u32_arr([n])], [(n,)], [F32])[0].numpy().view(np.uint32)
    exact_sqrt = Kernel("sqrt").apply([dabs, u32_arr([n])], [(n,)], [F32])[0].numpy().view(np.uint32)
    d2 = int(np.count_nonzero(exact_div != want_div))
    d4 = int(np.count_nonzero(exact_sqrt != want_sqrt))
    t.note(d2 == 0, f"exact_divide kernel: {d2} of {n} differ from IEEE")
    t.note(d4 == 0, f"exact_sqrt kernel: {d4} of {n} differ from IEEE")
    # planted: the GPU's reciprocal-based / and raw sqrt in place of the exact ones
    approx_div = binary(100, da, db).numpy().view(np.uint32)
    d1 = int(np.count_nonzero(approx_div != want_div))
    t.note(d1 != 0, f"exact_divide planted fault (reciprocal-based /): {d1} of {n} differ (must be > 0)")
    nudged = ((a & 0x7FFFFFFF) ^ 1).view(np.float32)
    d5 = int(np.count_nonzero(
        Kernel("sqrt").apply([from_numpy(nudged), u32_arr([n])], [(n,)], [F32])[0].numpy().view(np.uint32)
        != want_sqrt))
    t.note(d5 != 0, f"exact_sqrt planted fault (input one ulp off): {d5} of {n} differ (must be > 0)")


def erff_exhaustive(t: Tally, chunk_log=24):
    """The GPU erff against the host copy of the same routine, every input (OpTests.lean:273-296)."""
    chunk = 1 << chunk_log
    k = Kernel("erff_map")
    bad, first = 0, None
    t0 = time.perf_counter()
    for c in range((1 << 32) // chunk):
        base = c * chunk
        gpu = k.apply([from_numpy(np.zeros(8, np.float32)), u32_arr([base, chunk])], [(chunk,)], [U32])[0]
        cpu = from_numpy(libm_erff_range(base, chunk))
        nz = count_nonzero(binary("ne", gpu, cpu))
        if nz:
            bad += nz
            first = base if first is None else first
    dt = time.perf_counter() - t0
    where = f" (first in chunk at {hex32(first)})" if first is not None else ""
    t.note(bad == 0, f"erff_exhaustive: {bad} of 4294967296 inputs differ from the host erff{where} ({dt:.1f} s)")
    gpu = k.apply([from_numpy(np.zeros(8, np.float32)), u32_arr([0x3F000000, chunk])], [(chunk,)], [U32])[0]
    cpu = from_numpy(libm_erff_range(0x3F000001, chunk))
    nz = count_nonzero(binary("ne", gpu, cpu))
    t.note(nz != 0, f"erff_exhaustive planted fault (reference shifted by one input): {nz} of {chunk} differ (must be > 0)")


# ---- the generic path: each case's graph.txt through the graph emitter ---------------

# The executor's planted faults a generic module can be broken with, first match
# wins (OpTests.lean:339-349), then the ggml.* kernels' own.
_GHLO_FAULTS = [
    ('"stablehlo.add"', "binary_half", "float16 arithmetic"),
    ('"stablehlo.multiply"', "binary_half", "float16 arithmetic"),
    ('"stablehlo.concatenate"', "concat_swap", "operands swapped"),
    ('"stablehlo.transpose"', "transpose_identity", "no permutation"),
    ('"stablehlo.slice"', "slice_shift", "offset one late"),
    ('"stablehlo.broadcast_in_dim"', "broadcast_first", "broadcast of the first element"),
    ('"stablehlo.dot_general"', "dot_builtin", "built-in matmul"),
    ('"ggml.soft_max"', "soft_max_float_sum", "binary32 denominator"),
    ('"ggml.norm"', "norm_gpu_ops", "binary32 sums and GPU / and sqrt"),
    ('"ggml.gelu_erf"', "gelu_tanh", "tanh-form GELU"),
    ('"ggml.silu"', "silu_gpu_ops", "GPU exp and /"),
]


def ghlo_case(ref, t: Tally, name, expect_refusal=False):
    """OpTests.ghloCase (OpTests.lean:303-359) over graph.txt: the case's graph
    emitted as a generic module (a leading ui64 0, rank-4 tensors), run
    compiled, compared with out.f32, then run with a planted executor fault
    that must change it."""
    from . import ghlo
    d = os.path.join(ref, name)
    gp = os.path.join(d, "graph.txt")
    if not os.path.exists(gp):
        t.note(False, f"ghlo {name}: graph missing ({gp})")
        return
    try:
        text, args, outs = ghlo.emit(open(gp).read())
    except ghlo.GraphError as e:
        t.note(False, f"ghlo {name}: not emitted: {e}")
        return
    md = read_meta(d)
    in_meta = [(n, ne) for n, ne in md if n.startswith("in")]
    if len(in_meta) != len(args):
        t.note(False, f"ghlo {name}: module takes {len(args)} tensors, the case has {len(in_meta)}")
        return
    ins = [from_numpy(np.zeros((), np.uint64))]
    for n, ne in in_meta:
        ins.append(from_numpy(np.fromfile(os.path.join(d, f"{n}.f32"), dtype=np.float32)
                              .reshape(ne[3], ne[2], ne[1], ne[0])))
    with open(os.path.join(d, "out.f32"), "rb") as f:
        want = f.read()
    count = len(want) // 4
    t0 = time.perf_counter()
    ok, r = run_module(text, ins, 0, True)
    ms = (time.perf_counter() - t0) * 1e3
    if expect_refusal:
        t.note(not ok and "not carried" in r, f"ghlo {name}: refused as expected: {r[:160]}" if not ok else
               f"ghlo {name}: ran, but it reaches code this executor does not carry")
        return
    if not ok:
        t.note(False, f"ghlo {name}: did not run: {r[:300]}")
        return
    n, first = diff(r, want)
    detail = f" first at {first}: got {hex32(word(r, first))} want {hex32(word(want, first))}" if first is not None else ""
    t.note(n == 0, f"ghlo {name}: {n} of {count} words differ{detail} ({ms:.3f} ms incl. trace)")
    pick = next(((f, fn) for key, f, fn in _GHLO_FAULTS if key in text), None)
    if pick is not None and pick[0] == "dot_builtin" and get_flavor() == 0:
        # The stock tail with K < 4 is exactly the natural-order FMA chain of the
        # built-in matmul; the unfused sequential sum differs from it for K >= 2.
        pick = ("dot_plain", "sequential sum without FMA")
    if pick is None:
        t.note(False, f"ghlo {name}: no executor fault applies to this module")
        return
    ok, r = run_module(text, ins, fault_bits(pick[0]), True)
    if not ok:
        t.note(True, f"ghlo {name} executor fault ({pick[1]}): refused: {r[:100]}")
    else:
        n, _ = diff(r, want)
        t.note(n != 0, f"ghlo {name} executor fault ({pick[1]}): {n} of {count} differ (must be > 0)")


def main(argv=None):
    argv = list(sys.argv[1:] if argv is None else argv)
    pinned = None
    if "--pinned" in argv:
        k = argv.index("--pinned")
        if k + 1 >= len(argv):
            print("--pinned needs a directory", file=sys.stderr)
            return 2
        pinned = argv[k + 1]
        argv = argv[:k] + argv[k + 2:]
    if not argv:
        print("usage: python -m shlo_hip.op_tests <ref-dir> [--pinned <pinned-ref-dir>] [case ...]", file=sys.stderr)
        return 2
    ref, only = argv[0], argv[1:]
    want = lambda n: not only or n in only
    t = Tally()
    if want("builtin"):
        builtin_probes(t)
    for c in CASES:
        if want(c.name):
            run_case(ref, t, c)
    if pinned is not None:  # the generic path, pinned flavour (OpTests.lean:369-372)
        prev = get_flavor()
        set_flavor(1)
        try:
            for c in CASES:
                if want(c.name):
                    ghlo_case(pinned, t, c.name)
        finally:
            set_flavor(prev)
    if want("erff_exhaustive"):
        erff_exhaustive(t)
    print(f"\n{t.passed} passed, {t.failed} failed")
    return 0 if t.failed == 0 else 1


if __name__ == "__main__":
    sys.exit(main())
