"""The fused attention kernel (attention_k): S = Q K^T with its element-wise
chain, P = ggml.soft_max(S), O = P V in one kernel, S and P in LDS.

The lowering runs a dot_general -> (chain) -> ggml.soft_max -> dot_general
group through it when the shapes and layouts allow (head dim 64, 64 value
columns, keys a multiple of 256 up to 1024, queries a multiple of 32), and
through the separate kernels otherwise.  Either way every output bit must be
the oracle's (dot in ggml order, the chain's IEEE ops, ggml soft_max, dot
again): eager and compiled, graph-captured and replayed."""
import numpy as np
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("graph_mode")]

F32 = np.float32


def t(shape):
    return "tensor<" + "".join(f"{d}x" for d in shape) + "f32>"


def hexf(x):
    return "0x%08X" % int(np.array([x], F32).view(np.uint32)[0])


def attn_module(B, H, NQ, NK, D=64, DV=64, scale=0.125, mask=True, sm_scale=1.0, residual=False):
    q, k, v = t((B, H, NQ, D)), t((B, H, NK, D)), t((B, H, NK, DV))
    s, o, m = t((B, H, NQ, NK)), t((B, H, NQ, DV)), t((NQ, NK))
    qk = ("#stablehlo.dot<lhs_batching_dimensions = [0, 1], rhs_batching_dimensions = [0, 1], "
          "lhs_contracting_dimensions = [3], rhs_contracting_dimensions = [3]>")
    pv = ("#stablehlo.dot<lhs_batching_dimensions = [0, 1], rhs_batching_dimensions = [0, 1], "
          "lhs_contracting_dimensions = [3], rhs_contracting_dimensions = [2]>")
    args = [f"%q: {q}", f"%k: {k}", f"%v: {v}"] + ([f"%mask: {m}"] if mask else []) + ([f"%res: {o}"] if residual else [])
    L = [f'    %0 = "stablehlo.dot_general"(%q, %k) {{dot_dimension_numbers = {qk}}} : ({q}, {k}) -> {s}']
    cur = "%0"
    if scale is not None:
        L += [f'    %c = "stablehlo.constant"() {{value = dense<{hexf(scale)}> : tensor<f32>}} : () -> tensor<f32>',
              f'    %cb = "stablehlo.broadcast_in_dim"(%c) {{broadcast_dimensions = array<i64>}} : (tensor<f32>) -> {s}',
              f'    %1 = "stablehlo.multiply"({cur}, %cb) : ({s}, {s}) -> {s}']
        cur = "%1"
    if mask:
        L += [f'    %mb = "stablehlo.broadcast_in_dim"(%mask) {{broadcast_dimensions = array<i64: 2, 3>}} : ({m}) -> {s}',
              f'    %2 = "stablehlo.add"({cur}, %mb) : ({s}, {s}) -> {s}']
        cur = "%2"
    L += [f'    %3 = "stablehlo.custom_call"({cur}) {{call_target_name = "ggml.soft_max", '
          f'backend_config = "scale = {hexf(sm_scale)} : f32"}} : ({s}) -> {s}',
          f'    %4 = "stablehlo.dot_general"(%3, %v) {{dot_dimension_numbers = {pv}}} : ({s}, {v}) -> {o}']
    ret = "%4"
    if residual:
        L += [f'    %5 = "stablehlo.add"(%res, %4) : ({o}, {o}) -> {o}']
        ret = "%5"
    body = "\n".join(L)
    return (f"module {{\n  func.func public @main({', '.join(args)}) -> ({o}) {{\n{body}\n"
            f"    func.return {ret} : {o}\n  }}\n}}\n")


def inputs(oracle, B, H, NQ, NK, D=64, DV=64, seed=61):
    q, st = oracle.fill_normal(seed, 1.0, B * H * NQ * D)
    k, st = oracle.fill_normal(seed, 1.0, B * H * NK * D, state=st)
    v, _ = oracle.fill_normal(seed, 1.0, B * H * NK * DV, state=st)
    return q.reshape(B, H, NQ, D), k.reshape(B, H, NK, D), v.reshape(B, H, NK, DV)


def causal(NQ, NK):
    return np.where(np.triu(np.ones((NQ, NK), bool), 1 + NK - NQ), F32(-np.inf), F32(0))


def oracle_attn(oracle, q, k, v, mask=None, scale=0.125, sm_scale=1.0, residual=None):
    B, H, NQ, D = q.shape
    NK, DV = k.shape[2], v.shape[3]
    s = oracle.dot_general_bnk(q.reshape(B * H, NQ, D), k.reshape(B * H, NK, D))
    if scale is not None:
        s = (s * F32(scale)).astype(F32)
    if mask is not None:
        s = (s + mask[None]).astype(F32)
    p = oracle.soft_max(s, scale=F32(sm_scale))
    vt = np.ascontiguousarray(v.reshape(B * H, NK, DV).transpose(0, 2, 1))
    o = oracle.dot_general_bnk(p, vt).reshape(B, H, NQ, DV)
    if residual is not None:
        o = (residual + o).astype(F32)
    return o


def bits_equal(a, b, nan_ok=False):
    ua, ub = np.ascontiguousarray(a).view(np.uint32), np.ascontiguousarray(b).view(np.uint32)
    if not nan_ok:
        return a.shape == b.shape and np.array_equal(ua, ub)
    na, nb = (ua & 0x7FFFFFFF) > 0x7F800000, (ub & 0x7FFFFFFF) > 0x7F800000
    return a.shape == b.shape and np.array_equal(na, nb) and np.array_equal(ua[~na], ub[~nb])


def fused_name(NK):
    return f"attention_k<{NK // 256}>"


def run(text, ins, compile=True, faults=0):
    import shlo_hip
    m = shlo_hip.Module(text)
    return m.prepare(faults, compile).call([shlo_hip.from_numpy(np.ascontiguousarray(x)) for x in ins])[0].numpy()


@pytest.mark.parametrize("B,H,NQ,NK", [(2, 2, 256, 256), (1, 3, 512, 512), (2, 1, 96, 768), (1, 2, 64, 1024),
                                       (3, 2, 160, 512)])
def test_fused_attention_vs_oracle(oracle, B, H, NQ, NK):
    import shlo_hip
    q, k, v = inputs(oracle, B, H, NQ, NK)
    mask = causal(NQ, NK)
    want = oracle_attn(oracle, q, k, v, mask)
    text = attn_module(B, H, NQ, NK)
    for compile in (False, True):
        got = run(text, [q, k, v, mask], compile=compile)
        if not compile:
            assert shlo_hip.last_dot_kernel() == fused_name(NK)
        assert bits_equal(got, want), compile


@pytest.mark.parametrize("B,H,NQ,NK", [(1, 29, 288, 256), (1, 13, 2528, 512), (2, 3, 1376, 256)])
def test_fused_attention_runs(oracle, B, H, NQ, NK):
    """More workgroups than two rounds over the CUs, grids not a multiple of
    the XCD count (261, 1027 and 258 workgroups), long query runs."""
    import shlo_hip
    q, k, v = inputs(oracle, B, H, NQ, NK, seed=68)
    i, j = np.arange(NQ)[:, None], np.arange(NK)[None, :]
    mask = np.where(j > i % NK, F32(-np.inf), F32(0))  # causal, repeating: no row wholly masked
    want = oracle_attn(oracle, q, k, v, mask)
    text = attn_module(B, H, NQ, NK)
    for compile in (False, True):
        got = run(text, [q, k, v, mask], compile=compile)
        if not compile:
            assert shlo_hip.last_dot_kernel() == fused_name(NK)
        assert bits_equal(got, want), compile


@pytest.mark.parametrize("variant", ["no_chain", "scale_only", "mask_only", "sm_scale_half", "residual"])
def test_fused_attention_chain_variants(oracle, variant):
    import shlo_hip
    B, H, NQ, NK = 2, 2, 128, 512
    q, k, v = inputs(oracle, B, H, NQ, NK, seed=62)
    mask = causal(NQ, NK)
    kw = dict(scale=0.125, mask=True, sm_scale=1.0, residual=False)
    if variant == "no_chain":
        kw.update(scale=None, mask=False)
    elif variant == "scale_only":
        kw.update(mask=False)
    elif variant == "mask_only":
        kw.update(scale=None)
    elif variant == "sm_scale_half":
        kw.update(sm_scale=0.5)
    else:
        kw.update(residual=True)
    res, _ = oracle.fill_normal(63, 1.0, B * H * NQ * 64)
    res = res.reshape(B, H, NQ, 64)
    want = oracle_attn(oracle, q, k, v, mask if kw["mask"] else None, kw["scale"], kw["sm_scale"],
                       res if kw["residual"] else None)
    ins = [q, k, v] + ([mask] if kw["mask"] else []) + ([res] if kw["residual"] else [])
    text = attn_module(B, H, NQ, NK, **kw)
    for compile in (False, True):
        got = run(text, ins, compile=compile)
        if not compile:
            assert shlo_hip.last_dot_kernel() == fused_name(NK), variant
        assert bits_equal(got, want), (variant, compile)


def test_fused_attention_special_values(oracle):
    """NaN and inf in Q, K and V rows, +-0, huge and subnormal scores, and
    masked entries times an infinite V (0 * inf = NaN, which ggml keeps):
    NaN outputs compared by NaN-ness, everything else bit for bit."""
    import shlo_hip
    B, H, NQ, NK = 1, 2, 64, 256
    q, k, v = inputs(oracle, B, H, NQ, NK, seed=64)
    q[0, 0, 3, 5] = np.nan
    q[0, 1, 7, :] *= F32(1e18)  # huge scores: exp underflows to subnormal and zero probabilities
    k[0, 0, 11, 2] = np.inf
    k[0, 1, 40, :] = 0.0
    k[0, 1, 41, :] = -0.0
    v[0, 0, 200, 9] = np.inf  # masked for the early rows: 0 * inf
    v[0, 1, 5, 3] = -np.inf
    v[0, 1, 6, :] = F32(1e-40)
    mask = causal(NQ, NK)
    want = oracle_attn(oracle, q, k, v, mask)
    text = attn_module(B, H, NQ, NK)
    for compile in (False, True):
        got = run(text, [q, k, v, mask], compile=compile)
        if not compile:
            assert shlo_hip.last_dot_kernel() == fused_name(NK)
        assert bits_equal(got, want, nan_ok=True), compile
    assert np.isnan(want).any() and np.isfinite(want).any()


def heads_module(B, T, H):
    """Q, K, V as per-head views of one [B, T, 3 H 64] projection (slice,
    reshape, transpose: two-level batch strides), then QK^T * 1/8, softmax,
    PV, as the denoiser builds its attention."""
    d = H * 64
    x, s3 = t((B, T, 3 * d)), None
    hv, s, o = t((B, H, T, 64)), t((B, H, T, T)), t((B, H, T, 64))
    L = []
    for i, nm in enumerate("qkv"):
        L.append(f'    %{nm}s = "stablehlo.slice"(%x) {{start_indices = array<i64: 0, 0, {i * d}>, limit_indices = '
                 f'array<i64: {B}, {T}, {(i + 1) * d}>, strides = array<i64: 1, 1, 1>}} : ({x}) -> {t((B, T, d))}')
        L.append(f'    %{nm}r = "stablehlo.reshape"(%{nm}s) : ({t((B, T, d))}) -> {t((B, T, H, 64))}')
        L.append(f'    %{nm} = "stablehlo.transpose"(%{nm}r) {{permutation = array<i64: 0, 2, 1, 3>}} : '
                 f'({t((B, T, H, 64))}) -> {hv}')
    qk = ("#stablehlo.dot<lhs_batching_dimensions = [0, 1], rhs_batching_dimensions = [0, 1], "
          "lhs_contracting_dimensions = [3], rhs_contracting_dimensions = [3]>")
    pv = ("#stablehlo.dot<lhs_batching_dimensions = [0, 1], rhs_batching_dimensions = [0, 1], "
          "lhs_contracting_dimensions = [3], rhs_contracting_dimensions = [2]>")
    L += [f'    %0 = "stablehlo.dot_general"(%q, %k) {{dot_dimension_numbers = {qk}}} : ({hv}, {hv}) -> {s}',
          f'    %c = "stablehlo.constant"() {{value = dense<0x3E000000> : tensor<f32>}} : () -> tensor<f32>',
          f'    %cb = "stablehlo.broadcast_in_dim"(%c) {{broadcast_dimensions = array<i64>}} : (tensor<f32>) -> {s}',
          f'    %1 = "stablehlo.multiply"(%0, %cb) : ({s}, {s}) -> {s}',
          f'    %3 = "stablehlo.custom_call"(%1) {{call_target_name = "ggml.soft_max", '
          f'backend_config = "scale = 0x3F800000 : f32"}} : ({s}) -> {s}',
          f'    %4 = "stablehlo.dot_general"(%3, %v) {{dot_dimension_numbers = {pv}}} : ({s}, {hv}) -> {o}']
    body = "\n".join(L)
    return (f"module {{\n  func.func public @main(%x: {x}) -> ({o}) {{\n{body}\n"
            f"    func.return %4 : {o}\n  }}\n}}\n")


def test_fused_attention_head_views(oracle):
    import shlo_hip
    B, T, H = 2, 256, 3
    x, _ = oracle.fill_normal(65, 1.0, B * T * 3 * H * 64)
    x = x.reshape(B, T, 3 * H * 64)
    heads = x.reshape(B, T, 3, H, 64).transpose(2, 0, 3, 1, 4)
    q, k, v = (np.ascontiguousarray(heads[i]) for i in range(3))
    want = oracle_attn(oracle, q, k, v)
    for compile in (False, True):
        got = run(heads_module(B, T, H), [x], compile=compile)
        if not compile:
            assert shlo_hip.last_dot_kernel() == fused_name(T)
        assert bits_equal(got, want), compile


@pytest.mark.parametrize("B,H,NQ,NK,D", [(2, 2, 128, 128, 64), (1, 2, 40, 256, 64), (1, 2, 64, 256, 40)])
def test_unfused_attention_shapes(oracle, B, H, NQ, NK, D):
    """Shapes the fused kernel does not carry (keys not a multiple of 256,
    queries not a multiple of 32, head dim 40) run the separate kernels."""
    import shlo_hip
    q, k, v = inputs(oracle, B, H, NQ, NK, D=D, DV=64, seed=66)
    mask = causal(NQ, NK)
    want = oracle_attn(oracle, q, k, v, mask)
    for compile in (False, True):
        got = run(attn_module(B, H, NQ, NK, D=D), [q, k, v, mask], compile=compile)
        if not compile:
            assert shlo_hip.last_dot_kernel().startswith("dot_"), shlo_hip.last_dot_kernel()
        assert bits_equal(got, want), compile


def test_planted_faults_still_differ(oracle):
    import shlo_hip
    B, H, NQ, NK = 1, 2, 64, 256
    q, k, v = inputs(oracle, B, H, NQ, NK, seed=67)
    mask = causal(NQ, NK)
    want = oracle_attn(oracle, q, k, v, mask)
    text = attn_module(B, H, NQ, NK)
    assert bits_equal(run(text, [q, k, v, mask]), want)
    for fault in ("dot_plain", "dot_builtin", "soft_max_float_sum", "binary_half", "broadcast_first"):
        got = run(text, [q, k, v, mask], faults=shlo_hip.fault_bits(fault))
        assert not bits_equal(got, want), fault


@pytest.mark.parametrize("NK", [256, 512])
def test_fused_attention_denominator_paths(oracle, NK):
    """Scale 0 makes the chain's output the mask row itself (+-0 + m = m), so
    the mask sets the softmax input exactly: rows whose denominator needs the
    in-order walk (1/S within 2^-40 of a binary32 rounding boundary), rows
    with entries 80-140 below the maximum (ggml_v_expf's subnormal branch and
    its +0 branch), spread over both passes and all four 16-lane rows of a
    wave, beside ordinary rows."""
    import shlo_hip
    from test_gpu_configs import _walk_rows
    B, H, NQ = 1, 2, 64
    q, k, v = inputs(oracle, B, H, NQ, NK, seed=69)
    rng = np.random.default_rng(NK)
    mask = rng.normal(0, 3, (NQ, NK)).astype(F32)
    walk = _walk_rows(oracle, NK, 3)
    for i, r in enumerate((0, 5, 10, 15, 36, 63)):
        mask[r] = walk[i]
    for r in (2, 7, 21, 40, 45):
        mask[r] = rng.uniform(-140.0, -80.0, NK).astype(F32)
        mask[r, r % NK] = 0.0
        mask[r, -3:] = -np.inf
    want = oracle_attn(oracle, q, k, v, mask, scale=0.0)
    text = attn_module(B, H, NQ, NK, scale=0.0)
    for compile in (False, True):
        got = run(text, [q, k, v, mask], compile=compile)
        if not compile:
            assert shlo_hip.last_dot_kernel() == fused_name(NK)
        assert bits_equal(got, want), compile


def chain_module(B, H, NQ, NK, ops):
    """QK^T, then `ops` in order: (op, operand, rev) with operand "c" (the
    scalar constant 0.125 broadcast) or "m" (the [NQ, NK] argument broadcast
    over batch and head); rev puts the running value second.  Then softmax, PV."""
    q, k, v = t((B, H, NQ, 64)), t((B, H, NK, 64)), t((B, H, NK, 64))
    s, o, m = t((B, H, NQ, NK)), t((B, H, NQ, 64)), t((NQ, NK))
    qk = ("#stablehlo.dot<lhs_batching_dimensions = [0, 1], rhs_batching_dimensions = [0, 1], "
          "lhs_contracting_dimensions = [3], rhs_contracting_dimensions = [3]>")
    pv = ("#stablehlo.dot<lhs_batching_dimensions = [0, 1], rhs_batching_dimensions = [0, 1], "
          "lhs_contracting_dimensions = [3], rhs_contracting_dimensions = [2]>")
    L = [f'    %s0 = "stablehlo.dot_general"(%q, %k) {{dot_dimension_numbers = {qk}}} : ({q}, {k}) -> {s}',
         f'    %c = "stablehlo.constant"() {{value = dense<0x3E000000> : tensor<f32>}} : () -> tensor<f32>',
         f'    %cb = "stablehlo.broadcast_in_dim"(%c) {{broadcast_dimensions = array<i64>}} : (tensor<f32>) -> {s}',
         f'    %mb = "stablehlo.broadcast_in_dim"(%mask) {{broadcast_dimensions = array<i64: 2, 3>}} : ({m}) -> {s}']
    cur = "%s0"
    for i, (op, operand, rev) in enumerate(ops):
        w = "%cb" if operand == "c" else "%mb"
        a, b = (w, cur) if rev else (cur, w)
        L.append(f'    %s{i + 1} = "stablehlo.{op}"({a}, {b}) : ({s}, {s}) -> {s}')
        cur = f"%s{i + 1}"
    L += [f'    %p = "stablehlo.custom_call"({cur}) {{call_target_name = "ggml.soft_max", '
          f'backend_config = "scale = 0x3F800000 : f32"}} : ({s}) -> {s}',
          f'    %o = "stablehlo.dot_general"(%p, %v) {{dot_dimension_numbers = {pv}}} : ({s}, {v}) -> {o}']
    body = "\n".join(L)
    return (f"module {{\n  func.func public @main(%q: {q}, %k: {k}, %v: {v}, %mask: {m}) -> ({o}) {{\n"
            f"{body}\n    func.return %o : {o}\n  }}\n}}\n")


_NP = {"add": np.add, "subtract": np.subtract, "multiply": np.multiply, "divide": np.divide,
       "maximum": np.maximum, "minimum": np.minimum}


@pytest.mark.parametrize("ops", [
    [("divide", "c", False), ("subtract", "m", True)],
    [("subtract", "m", False), ("divide", "c", True)],
    [("multiply", "c", True), ("maximum", "m", False)],
    [("minimum", "m", True), ("add", "c", False)],
    [("multiply", "c", False), ("add", "m", False), ("maximum", "m", True)],
], ids=["div_rsub", "sub_rdiv", "rmul_max", "rmin_add", "three_ops"])
def test_fused_attention_chain_ops(oracle, ops):
    """Every chain op and operand order in the fused kernel, with NaN and inf
    in Q (NaN scores: the row's P and O are NaN, compared by NaN-ness) and
    +-inf and large finite mask entries; maximum and minimum decide NaN-ness by
    their own rule.  The third op of three_ops runs after the two early ones."""
    import shlo_hip
    B, H, NQ, NK = 1, 2, 64, 256
    q, k, v = inputs(oracle, B, H, NQ, NK, seed=70)
    q[0, 0, 3, 7] = np.nan
    q[0, 1, 9, :] *= F32(1e30)  # inf * finite scores
    rng = np.random.default_rng(71)
    mask = rng.normal(0, 2, (NQ, NK)).astype(F32)
    mask[5, 10] = np.nan
    mask[6, :100] = -np.inf
    mask[7, 3] = np.inf
    mask[8, 1::2] = F32(3e38)
    s = oracle.dot_general_bnk(q.reshape(B * H, NQ, 64), k.reshape(B * H, NK, 64))
    with np.errstate(all="ignore"):
        for op, operand, rev in ops:
            w = np.broadcast_to(F32(0.125), s.shape) if operand == "c" else np.broadcast_to(mask[None], s.shape)
            a, b = (w, s) if rev else (s, w)
            s = _NP[op](a, b).astype(F32)
        p = oracle.soft_max(s)
    vt = np.ascontiguousarray(v.reshape(B * H, NK, 64).transpose(0, 2, 1))
    want = oracle.dot_general_bnk(p, vt).reshape(B, H, NQ, 64)
    text = chain_module(B, H, NQ, NK, ops)
    for compile in (False, True):
        got = run(text, [q, k, v, mask], compile=compile)
        if not compile:
            assert shlo_hip.last_dot_kernel() == fused_name(NK)
        assert bits_equal(got, want, nan_ok=True), compile
    assert np.isnan(want).any() and np.isfinite(want).any()


@pytest.mark.parametrize("sm_scale", [1.0, 0.5, -1.0])
def test_fused_attention_masked_slices(oracle, sm_scale):
    """A 64-column slice that is -inf on all four rows of a pass is set to
    +0 without computing it; the rows here check where that must not happen:
    a wholly -inf row (its maximum is -inf: NaN throughout), a NaN inside
    an otherwise -inf slice (the row is NaN), +inf among -inf, and a negative
    softmax scale (which turns -inf into +inf).  Scale 0 makes the mask row
    the softmax input; NaN outputs compare by NaN-ness."""
    import shlo_hip
    B, H, NQ, NK = 1, 2, 32, 512
    q, k, v = inputs(oracle, B, H, NQ, NK, seed=72)
    rng = np.random.default_rng(73)
    mask = rng.normal(0, 3, (NQ, NK)).astype(F32)
    mask[:, 128:] = -np.inf           # slices 2 .. 7 masked on every row
    mask[3, :] = -np.inf              # a wholly masked row
    mask[9, 300] = np.nan             # NaN in a masked slice
    mask[18, 450] = np.inf            # +inf in a masked slice
    mask[27, 64:128] = -np.inf        # one more masked slice on one row only
    want = oracle_attn(oracle, q, k, v, mask, scale=0.0, sm_scale=sm_scale)
    text = attn_module(B, H, NQ, NK, scale=0.0, sm_scale=sm_scale)
    for compile in (False, True):
        got = run(text, [q, k, v, mask], compile=compile)
        if not compile:
            assert shlo_hip.last_dot_kernel() == fused_name(NK)
        assert bits_equal(got, want, nan_ok=True), compile
    assert np.isnan(want[0, :, 3]).all() and np.isnan(want[0, :, 9]).all()
    # a negative scale turns the masked -inf into +inf: every row is NaN
    assert np.isfinite(want[0, :, 0]).all() == (sm_scale > 0)


def test_fused_attention_zero_slice_after_negative_zero(oracle):
    """Zero products still count: a chain at -0 plus a +0 product is +0, so
    P V cannot drop a slice whose P is +0 on every row while an accumulator
    holds -0 (any such shortcut must check for it).  Row 5 here
    has P = 2^-149 on keys 0..15 (V = -0.25 there: each chain's first
    product underflows to -0), P = 1 on key 16 (V = -0), then zeros with
    negative V (the chains stay -0) and, in the masked last slice, zeros with
    positive V: ggml's chains end at +0, so O[5] is +0, where dropping the
    slice would leave -0.  Scale 0 makes the mask row the softmax input."""
    import shlo_hip
    B, H, NQ, NK = 1, 1, 32, 256
    q, k, _ = inputs(oracle, B, H, NQ, NK, seed=74)
    rng = np.random.default_rng(75)
    mask = rng.normal(0, 1, (NQ, NK)).astype(F32)
    mask[:, 192:] = -np.inf
    # x with ggml_v_expf(x) = 2^-149, the smallest subnormal
    lo, hi = np.float32(-104.0), np.float32(-103.0)
    tiny = np.float32(2.0 ** -149)
    xs = np.sort(np.arange(np.float32(hi).view(np.int32), np.float32(lo).view(np.int32) + 1, dtype=np.int32).view(np.float32))
    hits = [x for x in xs if oracle.ggml_v_expf(np.float32(x)) == tiny]
    assert hits
    mask[5, :] = -np.inf
    mask[5, :16] = hits[len(hits) // 2]
    mask[5, 16] = 0.0
    v = np.empty((B, H, NK, 64), F32)
    v[..., :16, :] = -0.25
    v[..., 16, :] = -0.0
    v[..., 17:192, :] = -rng.uniform(0.5, 1.5, (B, H, 175, 64)).astype(F32)
    v[..., 192:, :] = rng.uniform(0.5, 1.5, (B, H, 64, 64)).astype(F32)
    want = oracle_attn(oracle, q, k, v, mask, scale=0.0)
    assert np.all(want[0, 0, 5].view(np.uint32) == 0)  # +0 in ggml's order
    text = attn_module(B, H, NQ, NK, scale=0.0)
    for compile in (False, True):
        got = run(text, [q, k, v, mask], compile=compile)
        if not compile:
            assert shlo_hip.last_dot_kernel() == fused_name(NK)
        assert bits_equal(got, want), compile


@pytest.mark.parametrize("NK", [256, 512])
@pytest.mark.parametrize("case", ["plain", "v_inf", "v_nan", "neg_zero"])
def test_fused_attention_pv_zero_suffix(oracle, NK, case):
    """Under a square causal mask each block of 32 query rows has P = +0 on
    all its rows from some 64-key slice on, and P V leaves those products out
    when the wave's value columns are finite there and no chain is at -0.
    Here they are, or a masked value is +-inf or NaN (0 * inf is NaN: those
    columns turn NaN), or every chain is at -0 where the products would stop
    (Q = 0 makes P = 1 / (row + 1), and V = -2^-149 on the first half of the
    keys underflows each product to -0) while V is positive further on:
    ggml's +0 products there turn the chains, and O, into +0."""
    import shlo_hip
    B, H, NQ = 1, 2, NK
    q, k, v = inputs(oracle, B, H, NQ, NK, seed=77)
    if case == "v_inf":
        v[0, 0, NK - 1, 7] = np.inf
        v[0, 1, NK - 70, 40] = -np.inf
    elif case == "v_nan":
        v[0, 1, NK - 1, 63] = np.nan
        v[0, 0, 100, 0] = np.nan
    elif case == "neg_zero":
        q[:] = 0.0
        v[..., : NK // 2, 5] = -(2.0 ** -149)
        v[..., NK // 2 :, 5] = 1.0
    mask = causal(NQ, NK)
    with np.errstate(all="ignore"):
        want = oracle_attn(oracle, q, k, v, mask)
    text = attn_module(B, H, NQ, NK)
    for compile in (False, True):
        got = run(text, [q, k, v, mask], compile=compile)
        if not compile:
            assert shlo_hip.last_dot_kernel() == fused_name(NK)
        assert bits_equal(got, want, nan_ok=True), (case, compile)
    if case == "plain":
        assert np.isfinite(want).all()
    elif case == "v_inf":
        assert np.isnan(want[0, 0, : NK - 1, 7]).all() and np.isnan(want[0, 1, : NK - 70, 40]).all()
    elif case == "v_nan":
        assert np.isnan(want[0, 1, :, 63]).all() and np.isnan(want[0, 0, :, 0]).all()
    else:
        # Rows 15 .. NK/2 - 1: every chain is -0 up to key NK/2 (each product
        # underflows), then the masked keys' +0 * 1 products make it +0;
        # leaving those products out would give -0.
        col = want[..., 5].view(np.uint32)
        assert (col[:, :, 15 : NK // 2] == 0).all()


@pytest.mark.parametrize("NK", [256, 512])
@pytest.mark.parametrize("case", ["plain", "k_huge_masked", "k_nan_masked", "q_inf", "near_limit", "over_limit",
                                  "scale_inf", "mask_only"])
def test_fused_attention_masked_tiles(oracle, NK, case):
    """Key tiles whose mask is -inf on all 32 rows of a block skip their
    products when Q, K and the scale bound every score and its scaled value
    below overflow (then the chain gives -inf whatever the score is).  Here
    the bound holds, or fails by a hair, or fails through inf, NaN or
    overflowing scores that sit only in masked tiles (they turn whole rows
    NaN); NaN outputs compare by NaN-ness."""
    import shlo_hip
    B, H, NQ = 1, 2, 64
    q, k, v = inputs(oracle, B, H, NQ, NK, seed=76)
    scale, mask_arg = 0.125, True
    if case == "k_huge_masked":
        k[0, 0, 200, :] = F32(3e38)      # masked for every query row: scores overflow there
        k[0, 1, 100, ::2] = F32(-3e38)
    elif case == "k_nan_masked":
        k[0, 1, 150, 7] = np.nan
    elif case == "q_inf":
        q[0, 0, 40, 3] = np.inf
    elif case == "near_limit":  # |q|, |k| < 2^60 with c = 2^-3: eq + ek + ec + 10 = 126
        q = (np.sign(q) * F32(2.0 ** 59)).astype(F32)
        k = (np.sign(k) * F32(2.0 ** 59)).astype(F32)
    elif case == "over_limit":  # 2^62: the bound fails and the scores overflow to +-inf
        q = (np.sign(q) * F32(2.0 ** 62)).astype(F32)
        k = (np.sign(k) * F32(2.0 ** 62)).astype(F32)
    elif case == "scale_inf":
        scale = float("inf")
    elif case == "mask_only":
        scale = None
    mask = causal(NQ, NK)
    with np.errstate(all="ignore"):  # the overflowing cases overflow in the oracle too
        want = oracle_attn(oracle, q, k, v, mask, scale=scale)
    text = attn_module(B, H, NQ, NK, scale=scale)
    for compile in (False, True):
        got = run(text, [q, k, v, mask], compile=compile)
        if not compile:
            assert shlo_hip.last_dot_kernel() == fused_name(NK)
        assert bits_equal(got, want, nan_ok=True), (case, compile)
    if case in ("plain", "near_limit", "mask_only"):
        assert np.isfinite(want).all()
    if case in ("k_nan_masked", "q_inf", "over_limit", "scale_inf"):
        assert np.isnan(want).any()


@pytest.mark.parametrize("case", ["plain", "v_inf"])
def test_fused_attention_unaligned_v(oracle, case):
    """V as a view whose rows are not 16-byte aligned (columns 1 .. 64 of a
    65-wide argument, read in place): attn_prep_k's finiteness check and P V's
    buffer loads at odd offsets.  With an infinite value among the masked keys
    P V must not leave those products out."""
    import shlo_hip
    B, H, NQ, NK = 2, 2, 256, 256
    q, k, v = inputs(oracle, B, H, NQ, NK, seed=79)
    if case == "v_inf":
        v[1, 0, NK - 3, 17] = np.inf
    wide = np.concatenate([np.full((B, H, NK, 1), F32(5.0)), v], axis=3)
    text = attn_module(B, H, NQ, NK)
    vw = t((B, H, NK, 65))
    text = text.replace(f"%v: {t((B, H, NK, 64))}", f"%vw: {vw}", 1)
    text = text.replace(
        "    %0 = ",
        f'    %v = "stablehlo.slice"(%vw) {{start_indices = array<i64: 0, 0, 0, 1>, limit_indices = '
        f"array<i64: {B}, {H}, {NK}, 65>, strides = array<i64: 1, 1, 1, 1>}} : ({vw}) -> {t((B, H, NK, 64))}\n"
        "    %0 = ", 1)
    mask = causal(NQ, NK)
    with np.errstate(all="ignore"):
        want = oracle_attn(oracle, q, k, v, mask)
    for compile in (False, True):
        got = run(text, [q, k, wide, mask], compile=compile)
        if not compile:
            assert shlo_hip.last_dot_kernel() == fused_name(NK)
        assert bits_equal(got, want, nan_ok=True), (case, compile)
    if case == "v_inf":
        assert np.isnan(want[1, 0, : NK - 3, 17]).all()
