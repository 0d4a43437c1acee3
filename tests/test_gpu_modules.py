"""GPU parity of whole modules: the attention chain through
the parser, op table and hipGraph, against the oracle running the same op
sequence on the CPU."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    return a.shape == b.shape and np.array_equal(np.ascontiguousarray(a).view(np.uint32),
                                                 np.ascontiguousarray(b).view(np.uint32))


def attention_inputs(oracle, B, H, S, D):
    q, st = oracle.fill_normal(41, 1.0, B * H * S * D)
    k, st = oracle.fill_normal(41, 1.0, B * H * S * D, state=st)
    v, _ = oracle.fill_normal(41, 1.0, B * H * S * D, state=st)
    mask = np.where(np.triu(np.ones((S, S), bool), 1), np.float32(-np.inf), np.float32(0))
    sh = (B, H, S, D)
    return q.reshape(sh), k.reshape(sh), v.reshape(sh), mask


def attention_oracle(oracle, q, k, v, mask, scale=np.float32(0.125)):
    B, H, S, D = q.shape
    s = oracle.dot_general_bnk(q.reshape(B * H, S, D), k.reshape(B * H, S, D))
    s = (s * scale).astype(np.float32)
    s = (s + mask[None]).astype(np.float32)
    p = oracle.soft_max(s)
    vt = np.ascontiguousarray(v.reshape(B * H, S, D).transpose(0, 2, 1))
    return oracle.dot_general_bnk(p, vt).reshape(B, H, S, D)


@pytest.mark.parametrize("shape", [(2, 2, 128, 64), (1, 3, 96, 40)])
def test_attention_chain_vs_oracle(oracle, shape):
    import shlo_hip
    from shlo_hip import configs
    q, k, v, mask = attention_inputs(oracle, *shape)
    want = attention_oracle(oracle, q, k, v, mask)
    m = shlo_hip.Module(configs.attention_module(*shape))
    ins = [shlo_hip.from_numpy(x) for x in (q, k, v, mask)]
    for compile in (True, False):
        got = m.prepare(0, compile).call(ins)[0].numpy()
        assert same_bits(got, want), compile
    for fault in ("dot_builtin", "soft_max_float_sum", "broadcast_first", "binary_half"):
        got = m.prepare(shlo_hip.fault_bits(fault), True).call(ins)[0].numpy()
        assert not same_bits(got, want), fault


def test_attention_config4_graph_equals_eager_and_one_head(oracle):
    """B=8, H=8, S=512, D=64: graph == eager on the whole output, and one
    (batch, head) slice against the oracle."""
    import shlo_hip
    from shlo_hip import configs
    B, H, S, D = 8, 8, 512, 64
    q, k, v, mask = attention_inputs(oracle, B, H, S, D)
    m = shlo_hip.Module(configs.attention_module(B, H, S, D))
    ins = [shlo_hip.from_numpy(x) for x in (q, k, v, mask)]
    g = m.prepare(0, True).call(ins)[0].numpy()
    e = m.prepare(0, False).call(ins)[0].numpy()
    assert same_bits(g, e)
    bh = (5, 3)
    one = attention_oracle(oracle, q[bh[0]:bh[0] + 1, bh[1]:bh[1] + 1], k[bh[0]:bh[0] + 1, bh[1]:bh[1] + 1],
                           v[bh[0]:bh[0] + 1, bh[1]:bh[1] + 1], mask)
    assert same_bits(g[bh[0], bh[1]], one[0, 0])


def test_dot_config3_slices_vs_oracle(oracle):
    """Batched [16,1024,4096] x [16,4096,4096]: two output rows of two batches
    against the oracle (full-size operands on the GPU)."""
    import shlo_hip
    from shlo_hip import configs
    B, N, K, M = 16, 1024, 4096, 4096
    a = shlo_hip.fill_random((B, N, K), 31, 1, 1.0)
    b = shlo_hip.fill_random((B, K, M), 32, 1, 1.0)
    y = shlo_hip.Module(configs.dot_module(N, K, M, B)).prepare(0, True).call([a, b])[0]
    for bi, rows in ((0, (0, 777)), (11, (1023, 64))):
        bs = shlo_hip.slice_(b, (bi, 0, 0), (bi + 1, K, M), (1, 1, 1)).numpy()[0]
        for n in rows:
            arow = shlo_hip.slice_(a, (bi, n, 0), (bi + 1, n + 1, K), (1, 1, 1)).numpy()[0]
            want = oracle.dot_general_bnk(arow[None], np.ascontiguousarray(bs.T)[None])[0]
            got = shlo_hip.slice_(y, (bi, n, 0), (bi + 1, n + 1, M), (1, 1, 1)).numpy()[0]
            assert same_bits(got, want), (bi, n)


@pytest.mark.parametrize("dims", [dict(layers=2, d=128, heads=2, ffn=256, frames=32, feats=263, batch=2),
                                  dict(layers=1, d=512, heads=8, ffn=2048, frames=64, feats=263, batch=2)])
def test_denoiser_vs_oracle(oracle, dims):
    """The denoiser module at reduced sizes against the oracle, graph and
    eager, with planted faults in LayerNorm, GELU and dot_general."""
    import denoiser_ref
    import shlo_hip
    from shlo_hip import configs
    D = configs.Denoiser(**dims)
    host = denoiser_ref.host_args(D)
    dev = configs.denoiser_device_args(shlo_hip, D)
    for h, g in zip(host, dev):
        assert same_bits(g.numpy(), h)
    want = denoiser_ref.forward(D, host)
    m = shlo_hip.Module(D.module())
    for compile in (True, False):
        got = m.prepare(0, compile).call(dev)[0].numpy()
        assert same_bits(got, want), compile
    for fault in ("norm_gpu_ops", "gelu_tanh", "dot_plain"):
        got = m.prepare(shlo_hip.fault_bits(fault), True).call(dev)[0].numpy()
        assert not same_bits(got, want), fault


def test_denoiser_config5_graph_equals_eager():
    """The full config: 8 layers, d 512, 8 heads, FFN 2048, 256 frames x 263
    features, batch 32; the compiled module repeated (--repeat) gives the same
    bits every call, equal to the eager run."""
    import shlo_hip
    from shlo_hip import configs
    D = configs.Denoiser()
    dev = configs.denoiser_device_args(shlo_hip, D)
    m = shlo_hip.Module(D.module())
    e = m.prepare(0, False).call(dev)[0]
    f = m.prepare(0, True)
    for _ in range(3):
        g = f.call(dev)[0]
        assert shlo_hip.count_nonzero(shlo_hip.binary("ne", shlo_hip.view(g, shlo_hip.U32),
                                                      shlo_hip.view(e, shlo_hip.U32))) == 0
    y = e.numpy()
    assert y.shape == (32, 256, 263) and np.all(np.isfinite(y))
