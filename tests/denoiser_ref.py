"""The synthetic denoiser's forward pass on the CPU oracle — test infrastructure.

The same op sequence as shlo_hip.configs.Denoiser.module(), written directly
against the oracle's ggml routines (dot in ggml order, ggml norm, soft_max,
gelu_erf) and numpy's binary32 elementwise arithmetic (one IEEE rounding per
element), so a GPU run can be compared bit for bit.
"""
import numpy as np

import oracle_py as oracle

F32 = np.float32


def host_args(D, timesteps=None):
    """Host copies of denoiser_device_args (same streams, same bits)."""
    from shlo_hip import configs
    ts = timesteps if timesteps is not None else [10 * b + 1 for b in range(D.B)]
    out = []
    for i, (nm, shape, kind) in enumerate(D.args()):
        n = int(np.prod(shape))
        if kind == "x":
            a = oracle.fill_normal(1000, 1.0, n)[0]
        elif kind == "temb":
            a = configs.timestep_embedding(ts, D.d)
        elif kind == "g":
            a = (F32(1) + oracle.fill_normal(configs.denoiser_arg_seed(i), 0.02, n)[0]).astype(F32)
        else:
            a = oracle.fill_normal(configs.denoiser_arg_seed(i), 0.02, n)[0]
        out.append(np.ascontiguousarray(a, F32).reshape(shape))
    return out


def forward(D, args, tail=oracle.TAIL_STOCK):
    B, T, F, d, H, dh, ffn = D.B, D.T, D.F, D.d, D.H, D.dh, D.ffn
    tok = B * T
    A = {nm: a for (nm, _, _), a in zip(D.args(), args)}

    def matmul(a, w, bias):
        y = oracle.dot_general_bnk(np.ascontiguousarray(a)[None], np.ascontiguousarray(w.T)[None], tail)[0]
        return (y + bias[None, :]).astype(F32)

    def ln(h, g, be):
        z = oracle.norm(h, eps=F32(1e-5))
        return ((z * g[None, :]).astype(F32) + be[None, :]).astype(F32)

    def heads(qkv, start):
        return np.ascontiguousarray(qkv[:, start:start + d].reshape(B, T, H, dh).transpose(0, 2, 1, 3))

    scale = F32(1.0 / (dh ** 0.5))
    h = matmul(A["x"].reshape(tok, F), A["w_in"], A["b_in"])
    h = (h + np.broadcast_to(A["temb"][:, None, :], (B, T, d)).reshape(tok, d)).astype(F32)
    for i in range(D.L):
        a = ln(h, A[f"g1_{i}"], A[f"be1_{i}"])
        qkv = matmul(a, A[f"wqkv_{i}"], A[f"bqkv_{i}"])
        q, k, v = heads(qkv, 0), heads(qkv, d), heads(qkv, 2 * d)
        s = oracle.dot_general_bnk(q.reshape(B * H, T, dh), k.reshape(B * H, T, dh), tail)
        s = (s * scale).astype(F32)
        p = oracle.soft_max(s)
        vt = np.ascontiguousarray(v.reshape(B * H, T, dh).transpose(0, 2, 1))
        o = oracle.dot_general_bnk(p, vt, tail).reshape(B, H, T, dh).transpose(0, 2, 1, 3).reshape(tok, d)
        o = matmul(o, A[f"wo_{i}"], A[f"bo_{i}"])
        h = (h + o).astype(F32)
        f = ln(h, A[f"g2_{i}"], A[f"be2_{i}"])
        f = matmul(f, A[f"w1_{i}"], A[f"bf1_{i}"])
        f = oracle.gelu_erf(f)
        f = matmul(f, A[f"w2_{i}"], A[f"bf2_{i}"])
        h = (h + f).astype(F32)
    h = ln(h, A["gf"], A["bef"])
    return matmul(h, A["w_out"], A["b_out"]).reshape(B, T, F)
