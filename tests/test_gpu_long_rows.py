"""ggml.soft_max and ggml.norm on rows longer than 4096 columns.

The reference's kernels loop over any row length (StablehloMlx/Kernels/
Shaders.lean:100-166) and refuse only a softmax row tail in the stock flavour
(Lower.lean:485-486).  Rows that do not fit one wave's registers stream
through soft_max_long_k / norm_long_k, whose binary64 sums are decided with an
interval re-derived for the row length (ordered_sum_long).  Bit for bit
against the oracle, eager and compiled: random rows with masks and scales,
row tails (pinned flavour), rows built so that only the in-order walk matches
the oracle, and the planted faults."""
import numpy as np
import pytest

from test_gpu_configs import _walk_rows, custom_call_module, same_bits
from test_gpu_norm import check as norm_check, mean_walk_row, norm_module, var_walk_row

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("graph_mode")]

F32 = np.float32


def run(text, inputs, faults=0, compile=True):
    import shlo_hip
    m = shlo_hip.Module(text)
    return m.prepare(faults, compile).call([shlo_hip.from_numpy(np.ascontiguousarray(x)) for x in inputs])[0].numpy()


def masked_logits(oracle, rows, cols, seed, sigma=4.0):
    x, _ = oracle.fill_normal(seed, sigma, rows * cols)
    x = x.reshape(rows, cols)
    # a causal-style mask over the first columns of every other row (never a whole row)
    for r in range(0, rows, 2):
        x[r, cols // 2 + r:] = -np.inf
    return x


@pytest.mark.parametrize("cols", [4100, 4352, 8192, 32768, 100004])
def test_softmax_long_rows(oracle, cols):
    """9 rows (the last block of four waves partly empty), scale 0.5, masks;
    the planted binary32 denominator must differ."""
    import shlo_hip
    x = masked_logits(oracle, 9, cols, 51)
    text = custom_call_module("ggml.soft_max", "scale = 0x3F000000 : f32", x.shape)
    want = oracle.soft_max(x, scale=0.5)
    for compile in (True, False):
        assert same_bits(run(text, [x], compile=compile), want), (cols, compile)
    got = run(text, [x], faults=shlo_hip.fault_bits("soft_max_float_sum"))
    assert same_bits(got, oracle.soft_max(x, scale=0.5, float_sum=True))
    assert not same_bits(got, want)


@pytest.mark.parametrize("cols", [4097, 4099, 8195, 40003])
def test_softmax_long_row_tails_pinned(oracle, cols):
    """Row tails through the correctly rounded expf, after the group parts."""
    import shlo_hip
    x = masked_logits(oracle, 6, cols, 52, sigma=6.0)
    x[1, -1] = -np.inf
    text = custom_call_module("ggml.soft_max", "scale = 0x3F800000 : f32", x.shape)
    want = oracle.soft_max(x)
    shlo_hip.set_flavor(1)
    try:
        for compile in (True, False):
            assert same_bits(run(text, [x], compile=compile), want), (cols, compile)
        got = run(text, [x], faults=shlo_hip.fault_bits("soft_max_float_sum"))
        assert same_bits(got, oracle.soft_max(x, float_sum=True))
    finally:
        shlo_hip.set_flavor(0)
    with pytest.raises(shlo_hip.ShloError, match="not carried"):
        run(text, [x], compile=False)  # the stock flavour refuses the tail


@pytest.mark.parametrize("cols", [8200, 16384, 8198])
def test_softmax_long_denominator_walk(oracle, cols):
    """Rows whose denominator fails the exactness and interval tests (1/S
    within 2^-40 of a binary32 rounding boundary, which also lies inside the
    long kernel's wider interval), next to ordinary rows."""
    import shlo_hip
    walk = _walk_rows(oracle, cols, 3)
    x, _ = oracle.fill_normal(53, 3.0, 5 * cols)
    x = np.concatenate([walk, x.reshape(5, cols)]).astype(F32)
    text = custom_call_module("ggml.soft_max", "scale = 0x3F800000 : f32", x.shape)
    want = oracle.soft_max(x)
    shlo_hip.set_flavor(1 if cols % 4 else 0)
    try:
        for compile in (True, False):
            assert same_bits(run(text, [x], compile=compile), want), compile
    finally:
        shlo_hip.set_flavor(0)


@pytest.mark.parametrize("cols", [4100, 8192, 32768, 100000, 4097, 10001])
def test_norm_long_rows(oracle, cols):
    import shlo_hip
    x, _ = oracle.fill_normal(54, 3.0, 7 * cols)
    x = x.reshape(7, cols)
    x[2] += F32(1000.0)  # a large mean: the mean's sum fails the exactness test
    text, ins, want = norm_check(oracle, x)
    got = run(text, ins, faults=shlo_hip.fault_bits("norm_gpu_ops"))
    assert not same_bits(got, want)


@pytest.mark.parametrize("cols", [8192, 16384])
def test_norm_long_walk(oracle, cols):
    """Rows whose in-order sums round differently from a tree sum (the mean's
    and the variance's), and rows with one tiny element, among random rows."""
    x, _ = oracle.fill_normal(55, 1.0, 9 * cols)
    x = x.reshape(9, cols)
    x[1] = mean_walk_row(cols)
    x[4] = var_walk_row(cols)
    x[6] = -mean_walk_row(cols) * F32(3)
    tiny, _ = oracle.fill_normal(56, 2.0 ** -60, 9)
    x[7, 5] = tiny[0]
    # the in-order and tree results differ for these rows
    s_chain = 0.0
    for v in x[1].astype(np.float64):
        s_chain += v
    assert F32(s_chain) != F32((1.0 + 2.0 ** -24) + (2.0 ** -53 + 2.0 ** -53))
    norm_check(oracle, x)
