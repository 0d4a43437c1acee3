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


def test_attention_config4_all_heads_vs_oracle(oracle):
    """B=8, H=8, S=512, D=64: graph == eager on the whole
    output, and every (batch, head) against the oracle."""
    import shlo_hip
    from shlo_hip import configs
    B, H, S, D = 8, 8, 512, 64
    q, k, v, mask = attention_inputs(oracle, B, H, S, D)
    m = shlo_hip.Module(configs.attention_module(B, H, S, D))
    ins = [shlo_hip.from_numpy(x) for x in (q, k, v, mask)]
    g = m.prepare(0, True).call(ins)[0].numpy()
    e = m.prepare(0, False).call(ins)[0].numpy()
    assert same_bits(g, e)
    want = attention_oracle(oracle, q, k, v, mask)
    assert same_bits(g, want)


def test_dot_config3_strips_vs_oracle(oracle):
    """Batched [16,1024,4096] x [16,4096,4096] against the
    oracle on whole tiles: the first 64-row strip (every column tile) of
    batches 0 and 11, the last 64-row strip of batch 15 and its last 64-column
    strip (every row tile)."""
    import shlo_hip
    from shlo_hip import configs
    B, N, K, M = 16, 1024, 4096, 4096
    a = shlo_hip.fill_random((B, N, K), 31, 1, 1.0)
    b = shlo_hip.fill_random((B, K, M), 32, 1, 1.0)
    y = shlo_hip.Module(configs.dot_module(N, K, M, B)).prepare(0, True).call([a, b])[0]

    def sl(arr, start, stop):
        return shlo_hip.slice_(arr, start, stop, (1, 1, 1)).numpy()[0]

    for bi, n0 in ((0, 0), (11, 0), (15, N - 64)):
        bt = np.ascontiguousarray(sl(b, (bi, 0, 0), (bi + 1, K, M)).T)  # [M, K]
        arows = sl(a, (bi, n0, 0), (bi + 1, n0 + 64, K))
        want = oracle.dot_general_bnk(arows[None], bt[None])[0]
        assert same_bits(sl(y, (bi, n0, 0), (bi + 1, n0 + 64, M)), want), (bi, n0)
    bi = 15
    bcols = np.ascontiguousarray(sl(b, (bi, 0, M - 64), (bi + 1, K, M)).T)  # [64, K]
    want = oracle.dot_general_bnk(sl(a, (bi, 0, 0), (bi + 1, N, K))[None], bcols[None])[0]
    assert same_bits(sl(y, (bi, 0, M - 64), (bi + 1, N, M)), want)


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


def test_denoiser_config5_vs_oracle():
    """The full config (8 layers, d 512, 8 heads, FFN 2048, 256 frames x 263
    features, batch 32): the compiled module repeated (--repeat) gives the
    same bits every call, equal to the eager run, and batch elements 0 and 31
    equal the oracle's forward pass of that element alone (every op of the
    module computes each output from one batch element, in an order that does
    not depend on the batch size)."""
    import denoiser_ref
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
    host = denoiser_ref.host_args(D)
    names = [nm for nm, _, _ in D.args()]
    D1 = configs.Denoiser(batch=1)
    for bi in (0, 31):
        one = [h[bi:bi + 1] if nm in ("x", "temb") else h for nm, h in zip(names, host)]
        want = denoiser_ref.forward(D1, one)
        assert same_bits(y[bi:bi + 1], want), bi
