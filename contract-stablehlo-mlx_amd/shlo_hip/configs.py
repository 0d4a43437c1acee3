"""StableHLO modules of the measurement configs, as text.

Each builder returns generic-form module text that the executor's parser and
op table run unchanged, the same way the reference's shlo_mlx runs a
module.mlir (Main.lean:16-48).  Binary32 constants are hex bit patterns,
as the reference's lowering requires (Lower.lean:113-125).
"""
import struct


def t(dims, el="f32"):
    return "tensor<" + "".join(f"{d}x" for d in dims) + el + ">"


def hexf(x):
    return "0x%08X" % struct.unpack("<I", struct.pack("<f", x))[0]


def dot_module(N, K, M, batch=0):
    """dot_general [N,K] x [K,M] (contract [1]/[0]); with batch > 0,
    [B,N,K] x [B,K,M] (batch [0]/[0], contract [2]/[1])."""
    if batch:
        a, b, o = t((batch, N, K)), t((batch, K, M)), t((batch, N, M))
        dn = ("#stablehlo.dot<lhs_batching_dimensions = [0], rhs_batching_dimensions = [0], "
              "lhs_contracting_dimensions = [2], rhs_contracting_dimensions = [1]>")
    else:
        a, b, o = t((N, K)), t((K, M)), t((N, M))
        dn = "#stablehlo.dot<lhs_contracting_dimensions = [1], rhs_contracting_dimensions = [0]>"
    return (f"module {{\n  func.func public @main(%a0: {a}, %a1: {b}) -> ({o}) {{\n"
            f'    %0 = "stablehlo.dot_general"(%a0, %a1) {{dot_dimension_numbers = {dn}}} : ({a}, {b}) -> {o}\n'
            f"    func.return %0 : {o}\n  }}\n}}\n")


def custom_call(res, arg, target, attrs, ty):
    return (f'    {res} = "stablehlo.custom_call"({arg}) {{call_target_name = "{target}", backend_config = "{attrs}"}}'
            f" : ({ty}) -> {ty}\n")


def unary_module(target, attrs, dims):
    ty = t(dims)
    return (f"module {{\n  func.func public @main(%a0: {ty}) -> ({ty}) {{\n" + custom_call("%0", "%a0", target, attrs, ty) +
            f"    func.return %0 : {ty}\n  }}\n}}\n")


SOFTMAX_SCALE1 = "scale = 0x3F800000 : f32"


def unary_many_module(target, attrs, dims, n):
    """n independent applications of one ggml.* custom call, argument i to
    result i (a cold stream: each launch reads its own input)."""
    ty = t(dims)
    args = ", ".join(f"%a{i}: {ty}" for i in range(n))
    body = "".join(custom_call(f"%{i}", f"%a{i}", target, attrs, ty) for i in range(n))
    rets, tys = ", ".join(f"%{i}" for i in range(n)), ", ".join(ty for _ in range(n))
    return f"module {{\n  func.func public @main({args}) -> ({tys}) {{\n{body}    func.return {rets} : {tys}\n  }}\n}}\n"


def hot_path_module(rows=4096, cols=1024, n_gelu=64 << 20):
    """ggml.soft_max over [rows, cols] and ggml.gelu_erf
    over n_gelu elements, one module (one graph)."""
    ts, tg = t((rows, cols)), t((n_gelu,))
    return (f"module {{\n  func.func public @main(%a0: {ts}, %a1: {tg}) -> ({ts}, {tg}) {{\n" +
            custom_call("%0", "%a0", "ggml.soft_max", SOFTMAX_SCALE1, ts) +
            custom_call("%1", "%a1", "ggml.gelu_erf", "", tg) +
            f"    func.return %0, %1 : {ts}, {tg}\n  }}\n}}\n")


def attention_module(B=8, H=8, S=512, D=64, scale=0.125):
    """QK^T dot_general, scale, causal mask add, ggml.soft_max,
    PV dot_general.  Arguments: Q, K, V [B,H,S,D] and the mask [S,S] (0 / -inf)."""
    q, s, m = t((B, H, S, D)), t((B, H, S, S)), t((S, S))
    qk = ("#stablehlo.dot<lhs_batching_dimensions = [0, 1], rhs_batching_dimensions = [0, 1], "
          "lhs_contracting_dimensions = [3], rhs_contracting_dimensions = [3]>")
    pv = ("#stablehlo.dot<lhs_batching_dimensions = [0, 1], rhs_batching_dimensions = [0, 1], "
          "lhs_contracting_dimensions = [3], rhs_contracting_dimensions = [2]>")
    return (f"module {{\n  func.func public @main(%q: {q}, %k: {q}, %v: {q}, %mask: {m}) -> ({q}) {{\n"
            f'    %0 = "stablehlo.dot_general"(%q, %k) {{dot_dimension_numbers = {qk}}} : ({q}, {q}) -> {s}\n'
            f'    %c = "stablehlo.constant"() {{value = dense<{hexf(scale)}> : tensor<f32>}} : () -> tensor<f32>\n'
            f'    %cb = "stablehlo.broadcast_in_dim"(%c) {{broadcast_dimensions = array<i64>}} : (tensor<f32>) -> {s}\n'
            f'    %1 = "stablehlo.multiply"(%0, %cb) : ({s}, {s}) -> {s}\n'
            f'    %mb = "stablehlo.broadcast_in_dim"(%mask) {{broadcast_dimensions = array<i64: 2, 3>}} : ({m}) -> {s}\n'
            f'    %2 = "stablehlo.add"(%1, %mb) : ({s}, {s}) -> {s}\n' +
            custom_call("%3", "%2", "ggml.soft_max", SOFTMAX_SCALE1, s) +
            f'    %4 = "stablehlo.dot_general"(%3, %v) {{dot_dimension_numbers = {pv}}} : ({s}, {q}) -> {q}\n'
            f"    func.return %4 : {q}\n  }}\n}}\n")


def attention_flops(B=8, H=8, S=512, D=64):
    return 2 * (2 * B * H * S * S * D)


# ---- the synthetic motion denoiser ---------------------------------

class Denoiser:
    """A pre-LayerNorm transformer over motion frames, as one StableHLO module.

    x [B, T, F] (motion features) is projected to d_model, the sinusoidal
    timestep embedding temb [B, d] is added, then `layers` blocks of
      a = LN(h)*g1 + b1; qkv = a Wqkv + bqkv; per-head softmax(q k^T / sqrt(dh)) v;
      h = h + (o Wo + bo); f = LN(h)*g2 + b2; h = h + (gelu_erf(f W1 + bf1) W2 + bf2)
    and a final LN and projection back to F.  LN is ggml.norm (eps 1e-5) followed
    by the affine multiply and add; softmax is ggml.soft_max; GELU ggml.gelu_erf;
    every matmul a dot_general.  Weights are arguments (the reference passes
    them as .bin files); temb is computed on the host because sin and cos are
    not in the op table (Lower.lean:186-194).
    """

    def __init__(self, layers=8, d=512, heads=8, ffn=2048, frames=256, feats=263, batch=32):
        self.L, self.d, self.H, self.ffn, self.T, self.F, self.B = layers, d, heads, ffn, frames, feats, batch
        self.dh = d // heads
        assert self.dh * heads == d

    def args(self):
        """[(name, shape, kind)] in argument order; kind: 'x', 'temb', 'w' (N(0,0.02)),
        'g' (1 + N(0,0.02))."""
        B, T, F, d, ffn = self.B, self.T, self.F, self.d, self.ffn
        a = [("x", (B, T, F), "x"), ("temb", (B, d), "temb"), ("w_in", (F, d), "w"), ("b_in", (d,), "w")]
        for i in range(self.L):
            a += [(f"g1_{i}", (d,), "g"), (f"be1_{i}", (d,), "w"), (f"wqkv_{i}", (d, 3 * d), "w"),
                  (f"bqkv_{i}", (3 * d,), "w"), (f"wo_{i}", (d, d), "w"), (f"bo_{i}", (d,), "w"),
                  (f"g2_{i}", (d,), "g"), (f"be2_{i}", (d,), "w"), (f"w1_{i}", (d, ffn), "w"),
                  (f"bf1_{i}", (ffn,), "w"), (f"w2_{i}", (ffn, d), "w"), (f"bf2_{i}", (d,), "w")]
        a += [("gf", (d,), "g"), ("bef", (d,), "w"), ("w_out", (d, F), "w"), ("b_out", (F,), "w")]
        return a

    def flops(self):
        B, T, F, d, H, dh, ffn = self.B, self.T, self.F, self.d, self.H, self.dh, self.ffn
        tok = B * T
        per_layer = 2 * tok * d * 3 * d + 2 * 2 * B * H * T * T * dh + 2 * tok * d * d + 2 * 2 * tok * d * ffn
        return self.L * per_layer + 2 * 2 * tok * F * d

    def module(self):
        B, T, F, d, H, dh, ffn = self.B, self.T, self.F, self.d, self.H, self.dh, self.ffn
        tok = B * T
        lines = []
        n = [0]

        def v():
            n[0] += 1
            return f"%v{n[0]}"

        def op(text):
            r = v()
            lines.append(f"    {r} = {text}\n")
            return r

        def matmul(a, w, K, Mo, bias):  # a [tok, K] x w [K, Mo] + bias [Mo]
            y = op(f'"stablehlo.dot_general"({a}, {w}) {{dot_dimension_numbers = #stablehlo.dot<'
                   f'lhs_contracting_dimensions = [1], rhs_contracting_dimensions = [0]>}} : '
                   f"({t((tok, K))}, {t((K, Mo))}) -> {t((tok, Mo))}")
            bb = op(f'"stablehlo.broadcast_in_dim"({bias}) {{broadcast_dimensions = array<i64: 1>}} : '
                    f"({t((Mo,))}) -> {t((tok, Mo))}")
            return op(f'"stablehlo.add"({y}, {bb}) : ({t((tok, Mo))}, {t((tok, Mo))}) -> {t((tok, Mo))}')

        def layer_norm(h, g, be):
            z = op(f'"stablehlo.custom_call"({h}) {{call_target_name = "ggml.norm", backend_config = '
                   f'"eps = 0x3727C5AC : f32"}} : ({t((tok, d))}) -> {t((tok, d))}')
            gb = op(f'"stablehlo.broadcast_in_dim"({g}) {{broadcast_dimensions = array<i64: 1>}} : '
                    f"({t((d,))}) -> {t((tok, d))}")
            z = op(f'"stablehlo.multiply"({z}, {gb}) : ({t((tok, d))}, {t((tok, d))}) -> {t((tok, d))}')
            bb = op(f'"stablehlo.broadcast_in_dim"({be}) {{broadcast_dimensions = array<i64: 1>}} : '
                    f"({t((d,))}) -> {t((tok, d))}")
            return op(f'"stablehlo.add"({z}, {bb}) : ({t((tok, d))}, {t((tok, d))}) -> {t((tok, d))}')

        def add(a, b, shape):
            return op(f'"stablehlo.add"({a}, {b}) : ({t(shape)}, {t(shape)}) -> {t(shape)}')

        def heads(x, start):  # x [tok, 3d] -> slice -> [B, H, T, dh]
            s = op(f'"stablehlo.slice"({x}) {{start_indices = array<i64: 0, {start}>, limit_indices = '
                   f"array<i64: {tok}, {start + d}>, strides = array<i64: 1, 1>}} : ({t((tok, 3 * d))}) -> {t((tok, d))}")
            r = op(f'"stablehlo.reshape"({s}) : ({t((tok, d))}) -> {t((B, T, H, dh))}')
            return op(f'"stablehlo.transpose"({r}) {{permutation = array<i64: 0, 2, 1, 3>}} : '
                      f"({t((B, T, H, dh))}) -> {t((B, H, T, dh))}")

        argl = self.args()
        names = {nm: f"%{nm}" for nm, _, _ in argl}
        sig = ", ".join(f"%{nm}: {t(shape)}" for nm, shape, _ in argl)
        x2 = op(f'"stablehlo.reshape"(%x) : ({t((B, T, F))}) -> {t((tok, F))}')
        h = matmul(x2, names["w_in"], F, d, names["b_in"])
        tb = op(f'"stablehlo.broadcast_in_dim"(%temb) {{broadcast_dimensions = array<i64: 0, 2>}} : '
                f"({t((B, d))}) -> {t((B, T, d))}")
        tb = op(f'"stablehlo.reshape"({tb}) : ({t((B, T, d))}) -> {t((tok, d))}')
        h = add(h, tb, (tok, d))
        scale = op(f'"stablehlo.constant"() {{value = dense<{hexf(1.0 / (dh ** 0.5))}> : tensor<f32>}} : () -> tensor<f32>')
        s4 = (B, H, T, T)
        scb = op(f'"stablehlo.broadcast_in_dim"({scale}) {{broadcast_dimensions = array<i64>}} : (tensor<f32>) -> {t(s4)}')
        for i in range(self.L):
            a = layer_norm(h, names[f"g1_{i}"], names[f"be1_{i}"])
            qkv = matmul(a, names[f"wqkv_{i}"], d, 3 * d, names[f"bqkv_{i}"])
            q, k, vv = heads(qkv, 0), heads(qkv, d), heads(qkv, 2 * d)
            sc = op(f'"stablehlo.dot_general"({q}, {k}) {{dot_dimension_numbers = #stablehlo.dot<'
                    f"lhs_batching_dimensions = [0, 1], rhs_batching_dimensions = [0, 1], "
                    f"lhs_contracting_dimensions = [3], rhs_contracting_dimensions = [3]>}} : "
                    f"({t((B, H, T, dh))}, {t((B, H, T, dh))}) -> {t(s4)}")
            sc = op(f'"stablehlo.multiply"({sc}, {scb}) : ({t(s4)}, {t(s4)}) -> {t(s4)}')
            p = op(f'"stablehlo.custom_call"({sc}) {{call_target_name = "ggml.soft_max", backend_config = '
                   f'"scale = 0x3F800000 : f32"}} : ({t(s4)}) -> {t(s4)}')
            o = op(f'"stablehlo.dot_general"({p}, {vv}) {{dot_dimension_numbers = #stablehlo.dot<'
                   f"lhs_batching_dimensions = [0, 1], rhs_batching_dimensions = [0, 1], "
                   f"lhs_contracting_dimensions = [3], rhs_contracting_dimensions = [2]>}} : "
                   f"({t(s4)}, {t((B, H, T, dh))}) -> {t((B, H, T, dh))}")
            o = op(f'"stablehlo.transpose"({o}) {{permutation = array<i64: 0, 2, 1, 3>}} : '
                   f"({t((B, H, T, dh))}) -> {t((B, T, H, dh))}")
            o = op(f'"stablehlo.reshape"({o}) : ({t((B, T, H, dh))}) -> {t((tok, d))}')
            o = matmul(o, names[f"wo_{i}"], d, d, names[f"bo_{i}"])
            h = add(h, o, (tok, d))
            f = layer_norm(h, names[f"g2_{i}"], names[f"be2_{i}"])
            f = matmul(f, names[f"w1_{i}"], d, ffn, names[f"bf1_{i}"])
            f = op(f'"stablehlo.custom_call"({f}) {{call_target_name = "ggml.gelu_erf", backend_config = ""}} : '
                   f"({t((tok, ffn))}) -> {t((tok, ffn))}")
            f = matmul(f, names[f"w2_{i}"], ffn, d, names[f"bf2_{i}"])
            h = add(h, f, (tok, d))
        h = layer_norm(h, names["gf"], names["bef"])
        y = matmul(h, names["w_out"], d, F, names["b_out"])
        y = op(f'"stablehlo.reshape"({y}) : ({t((tok, F))}) -> {t((B, T, F))}')
        return (f"module @denoiser {{\n  func.func public @main({sig}) -> ({t((B, T, F))}) {{\n" + "".join(lines) +
                f"    func.return {y} : {t((B, T, F))}\n  }}\n}}\n")


def timestep_embedding(ts, d):
    """Sinusoidal embedding [len(ts), d]: sin at even, cos at odd positions,
    frequencies 10000^(-2i/d), evaluated in binary64 (math.sin/cos) and rounded."""
    import math

    import numpy as np
    out = np.empty((len(ts), d), np.float32)
    for b, tv in enumerate(ts):
        for i in range(d // 2):
            w = tv / (10000.0 ** (2.0 * i / d))
            out[b, 2 * i] = math.sin(w)
            out[b, 2 * i + 1] = math.cos(w)
    return out


def denoiser_arg_seed(i):
    """splitmix32 seed of the i-th denoiser argument (weights N(0, 0.02))."""
    return 100 + i


def denoiser_device_args(shlo, D, timesteps=None):
    """The denoiser's arguments generated on the device (fill_random: the
    splitmix32 Irwin-Hall normal); x ~ N(0,1), weights N(0,0.02), LayerNorm
    gains 1 + N(0,0.02), temb from `timesteps` (default 10*b + 1)."""
    import numpy as np
    out = []
    ts = timesteps if timesteps is not None else [10 * b + 1 for b in range(D.B)]
    one = shlo.from_numpy(np.ones((D.d,), np.float32))
    for i, (nm, shape, kind) in enumerate(D.args()):
        if kind == "x":
            out.append(shlo.fill_random(shape, 1000, 1, 1.0))
        elif kind == "temb":
            out.append(shlo.from_numpy(timestep_embedding(ts, D.d)))
        elif kind == "g":
            out.append(shlo.binary("add", one, shlo.fill_random(shape, denoiser_arg_seed(i), 1, 0.02)))
        else:
            out.append(shlo.fill_random(shape, denoiser_arg_seed(i), 1, 0.02))
    return out
