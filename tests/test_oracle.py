"""Pins of the FP64 oracle (CPU only).

Each oracle function is checked against something it does not share code
with: torch's float64 CPU operators, numpy, scipy/mpmath erf, closed forms,
brute force on tiny inputs, and the known answers the reference's own tests
hold (stem KAT, tests/cpp/test_cuda.cpp:449-479; FFN integer-pattern test,
336-393). Every pin is paired with a planted mistake in a copy of the oracle's
inputs or call (a transposed operand, a dropped term, a shifted index) that
the same check must reject, so a pin cannot pass vacuously.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")
import torch.nn.functional as F  # noqa: E402

from cutriton_amd import workloads  # noqa: E402
from oracle import oracle  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def _built():
    oracle.build()


def rng(seed: int = 0) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(workloads.SEED + seed))


CONV_CASES = [
    # (n, c, h, w, k, r, s, strides, pads [t, l, b, r], dilations)
    (1, 3, 9, 11, 4, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1)),
    (2, 5, 13, 10, 6, 7, 7, (2, 2), (3, 3, 3, 3), (1, 1)),
    (1, 8, 8, 8, 16, 1, 1, (2, 2), (0, 0, 0, 0), (1, 1)),
    (2, 4, 12, 12, 3, 3, 3, (1, 2), (2, 0, 1, 2), (2, 1)),
    (1, 2, 5, 5, 2, 5, 5, (1, 1), (0, 0, 0, 0), (1, 1)),
]


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv2d_matches_torch_float64(case):
    n, c, h, w, k, r, s, st, pd, dl = case
    g = rng(1)
    x = g.standard_normal((n, c, h, w))
    wt = g.standard_normal((k, c, r, s))
    got = oracle.conv2d(x, wt, st, pd, dl)
    xp = F.pad(torch.from_numpy(x), (pd[1], pd[3], pd[0], pd[2]))
    want = F.conv2d(xp, torch.from_numpy(wt), stride=st, dilation=dl).numpy()
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    # Planted: transposed spatial kernel must be caught (non-symmetric weights).
    if r > 1 or s > 1:
        bad = oracle.conv2d(x, np.ascontiguousarray(wt[:, :, ::-1, ::-1]), st, pd, dl)
        assert not np.allclose(bad, want, rtol=1e-6, atol=1e-6)


def test_conv2d_brute_force_tiny():
    g = rng(2)
    x = g.standard_normal((1, 2, 4, 5))
    wt = g.standard_normal((3, 2, 2, 3))
    st, pd, dl = (2, 1), (1, 0, 0, 1), (1, 2)
    got = oracle.conv2d(x, wt, st, pd, dl)
    oh = (4 + 1 + 0 - 1 * (2 - 1) - 1) // 2 + 1
    ow = (5 + 0 + 1 - 2 * (3 - 1) - 1) // 1 + 1
    want = np.zeros((1, 3, oh, ow))
    for k in range(3):
        for p in range(oh):
            for q in range(ow):
                acc = 0.0
                for c in range(2):
                    for i in range(2):
                        for j in range(3):
                            ih, iw = p * st[0] - pd[0] + i * dl[0], q * st[1] - pd[1] + j * dl[1]
                            if 0 <= ih < 4 and 0 <= iw < 5:
                                acc += x[0, c, ih, iw] * wt[k, c, i, j]
                want[0, k, p, q] = acc
    np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-13)


def test_batch_norm_matches_torch_float64():
    g = rng(3)
    x = g.standard_normal((2, 6, 5, 7))
    gamma, beta = g.uniform(0.5, 1.5, 6), g.normal(0, 0.1, 6)
    mu, var = g.normal(0, 0.1, 6), g.uniform(0.5, 1.5, 6)
    got = oracle.batch_norm(x, gamma, beta, mu, var, 1e-5)
    want = F.batch_norm(torch.from_numpy(x), torch.from_numpy(mu), torch.from_numpy(var), torch.from_numpy(gamma),
                        torch.from_numpy(beta), training=False, eps=1e-5).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    # Planted: epsilon outside the square root.
    bad = (x - mu[None, :, None, None]) / np.sqrt(var)[None, :, None, None] * gamma[None, :, None, None] \
        + beta[None, :, None, None]
    assert not np.allclose(bad, want, rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("kernel,strides,pads", [((3, 3), (2, 2), (1, 1, 1, 1)), ((2, 2), None, (0, 0, 0, 0)),
                                                 ((3, 2), (1, 2), (1, 0, 1, 1))])
def test_max_pool_bit_exact_vs_torch(kernel, strides, pads):
    g = rng(4)
    x = g.standard_normal((2, 3, 9, 10))
    got = oracle.max_pool(x, kernel, strides, pads)
    st = strides or kernel
    xp = F.pad(torch.from_numpy(x), (pads[1], pads[3], pads[0], pads[2]), value=-math.inf)
    want = F.max_pool2d(xp, kernel, stride=st).numpy()
    assert np.array_equal(got, want)
    # Invariant: every output is one of the inputs (selection, no arithmetic).
    assert np.isin(got, x).all()


def test_max_pool_padding_is_minus_infinity():
    # All-negative input: a zero pad would win at the borders.
    x = -np.ones((1, 1, 4, 4)) - np.arange(16).reshape(1, 1, 4, 4)
    got = oracle.max_pool(x, (3, 3), (2, 2), (1, 1, 1, 1))
    assert (got < 0).all()
    assert got[0, 0, 0, 0] == x[0, 0, :2, :2].max()


def test_max_pool_special_values():
    """NaN never wins (the window max of the numbers, -inf for an all-NaN
    window), +0 beats -0 in either order, infinities order as numbers."""
    nan, inf = math.nan, math.inf
    x = np.array([[nan, 1.0, -inf, nan],
                  [nan, nan, -0.0, 0.0],
                  [inf, -1.0, 0.0, -0.0],
                  [-inf, -inf, -0.0, -0.0]]).reshape(1, 1, 4, 4)
    got = oracle.max_pool(x, (2, 2), (2, 2))[0, 0]
    assert got[0, 0] == 1.0                        # NaNs skipped
    assert got[0, 1] == 0.0 and not math.copysign(1.0, got[0, 1]) < 0   # -inf, nan, -0, +0 -> +0
    assert got[1, 0] == inf
    assert got[1, 1] == 0.0 and not math.copysign(1.0, got[1, 1]) < 0   # +0 first, then -0 -> +0
    allnan = oracle.max_pool(np.full((1, 1, 2, 2), nan), (2, 2), (2, 2))
    assert allnan[0, 0, 0, 0] == -inf
    negzero = oracle.max_pool(np.full((1, 1, 2, 2), -0.0), (2, 2), (2, 2))
    assert negzero[0, 0, 0, 0] == 0.0 and math.copysign(1.0, negzero[0, 0, 0, 0]) < 0
    # Brute force on a random mix: nanmax of each window (NaN windows: -inf),
    # with the zero tie resolved to +0.
    g = rng(11)
    pool = np.array([nan, inf, -inf, 0.0, -0.0, 1.5, -2.0])
    x = g.choice(pool, size=(2, 3, 7, 8))
    got = oracle.max_pool(x, (3, 3), (2, 2), (1, 1, 1, 1))
    for (b, ch, oh, ow), v in np.ndenumerate(got):
        window = [x[b, ch, ih, iw] for ih in range(2 * oh - 1, 2 * oh + 2) for iw in range(2 * ow - 1, 2 * ow + 2)
                  if 0 <= ih < 7 and 0 <= iw < 8 and not math.isnan(x[b, ch, ih, iw])]
        want = max(window, default=-inf)
        if want == 0.0:
            want = 0.0 if any(math.copysign(1.0, z) > 0 for z in window if z == 0.0) else -0.0
        assert v == want and math.copysign(1.0, v) == math.copysign(1.0, want), (b, ch, oh, ow)


def test_global_average_pool_and_gemm_vs_numpy():
    g = rng(5)
    x = g.standard_normal((3, 7, 7, 7))
    np.testing.assert_allclose(oracle.global_average_pool(x)[:, :, 0, 0], x.mean(axis=(2, 3)), rtol=1e-13, atol=1e-14)
    a, b, bias = g.standard_normal((9, 33)), g.standard_normal((33, 5)), g.standard_normal(5)
    np.testing.assert_allclose(oracle.gemm(a, b), a @ b, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.gemm(a, b, bias), a @ b + bias, rtol=1e-12, atol=1e-12)
    # Planted: a transposed right operand (square case) is caught.
    sq = g.standard_normal((33, 33))
    assert not np.allclose(oracle.gemm(a, sq), a @ sq.T)


def test_gelu_erf_form():
    from scipy.special import erf

    x = np.linspace(-6, 6, 1001)
    got = oracle.gelu(x)
    np.testing.assert_allclose(got, 0.5 * x * (1 + erf(x / math.sqrt(2))), rtol=1e-14, atol=1e-15)
    want_t = F.gelu(torch.from_numpy(x), approximate="none").numpy()
    np.testing.assert_allclose(got, want_t, rtol=1e-13, atol=1e-15)
    mpmath = pytest.importorskip("mpmath")
    for v in (-3.7, -0.5, 0.0, 0.3, 1.0, 2.5):
        ref = 0.5 * v * (1 + float(mpmath.erf(mpmath.mpf(v) / mpmath.sqrt(2))))
        assert abs(oracle.gelu(np.array([v]))[0] - ref) <= 1e-15 * max(1.0, abs(ref))
    # Planted: the tanh approximation differs by more than the FP16 bound allows to go unnoticed at 1e-4.
    tanh_form = F.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    assert np.abs(tanh_form - got).max() > 1e-4


def test_layer_norm_two_pass_vs_torch():
    g = rng(6)
    x = g.standard_normal((5, 96)) * 3 + 40  # large mean: a one-pass variance would lose digits
    res = g.standard_normal((5, 96))
    gamma, beta = g.uniform(0.5, 1.5, 96), g.normal(0, 0.1, 96)
    got = oracle.layer_norm(x, gamma, beta, 1e-5)
    want = F.layer_norm(torch.from_numpy(x), (96,), torch.from_numpy(gamma), torch.from_numpy(beta), 1e-5).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-10)
    got_skip = oracle.layer_norm(x, gamma, beta, 1e-5, residual=res)
    want_skip = F.layer_norm(torch.from_numpy(x + res), (96,), torch.from_numpy(gamma), torch.from_numpy(beta),
                             1e-5).numpy()
    np.testing.assert_allclose(got_skip, want_skip, rtol=1e-10, atol=1e-10)
    # Planted: dropping the residual is caught.
    assert not np.allclose(got, want_skip, atol=1e-3)


def test_softmax_last_axis():
    from scipy.special import softmax as scipy_softmax

    g = rng(8)
    x = g.uniform(-50, 50, (5, 37))
    got = oracle.softmax(x)
    np.testing.assert_allclose(got, torch.softmax(torch.from_numpy(x), dim=-1).numpy(), rtol=1e-12, atol=1e-300)
    np.testing.assert_allclose(got, scipy_softmax(x, axis=-1), rtol=1e-12, atol=1e-300)
    # Invariants: rows sum to one; a per-row shift changes nothing.
    np.testing.assert_allclose(got.sum(axis=-1), 1.0, rtol=1e-14)
    np.testing.assert_allclose(oracle.softmax(x + g.uniform(-5, 5, (5, 1))), got, rtol=1e-12, atol=1e-300)
    # Closed form: two entries give the logistic function of their difference,
    # also where exp alone would overflow (the row max is subtracted first).
    for a, b in ((0.3, -1.2), (1000.0, 1000.0 - math.log(2.0)), (-700.0, -705.0)):
        want = [1.0 / (1.0 + math.exp(b - a)), 1.0 / (1.0 + math.exp(a - b))]
        np.testing.assert_allclose(oracle.softmax(np.array([[a, b]])), [want], rtol=1e-14)
    # -inf entries get 0; a row of -inf gives NaN, as in the reference.
    masked = oracle.softmax(np.array([[0.0, -np.inf, 0.0], [-np.inf, -np.inf, -np.inf]]))
    np.testing.assert_allclose(masked[0], [0.5, 0.0, 0.5], rtol=1e-15)
    assert np.isnan(masked[1]).all()
    # Planted: the softmax over the other axis is caught.
    assert not np.allclose(oracle.softmax(x.T).T, got, atol=1e-3)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("s_q,s_k", [(7, 7), (5, 11), (9, 4)])
def test_attention_vs_torch_sdpa(causal, s_q, s_k):
    """Against torch's float64 scaled_dot_product_attention (upper-left
    causal mask), default and explicit scale."""
    g = rng(10)
    q, k, v = (g.standard_normal((2, 3, s, 16)) for s in (s_q, s_k, s_k))
    tq, tk, tv = (torch.from_numpy(a) for a in (q, k, v))
    want = F.scaled_dot_product_attention(tq, tk, tv, is_causal=causal).numpy()
    np.testing.assert_allclose(oracle.attention(q, k, v, causal=causal), want, rtol=1e-12, atol=1e-13)
    want_scaled = F.scaled_dot_product_attention(tq, tk, tv, is_causal=causal, scale=0.3).numpy()
    np.testing.assert_allclose(oracle.attention(q, k, v, 0.3, causal), want_scaled, rtol=1e-12, atol=1e-13)
    # Planted: the bottom-right causal alignment or a dropped scale is caught.
    if causal and s_q != s_k:
        shift = s_k - s_q
        mask = np.tril(np.ones((s_q, s_k), bool), k=shift)
        bottom_right = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=torch.from_numpy(mask)).numpy()
        assert not np.allclose(bottom_right, want, atol=1e-3)
    assert not np.allclose(oracle.attention(q, k, v, 1.0, causal), want, atol=1e-3)


def test_attention_closed_forms():
    g = rng(11)
    v = g.standard_normal((1, 1, 6, 4))
    # Identical keys: uniform weights, the mean of the values (causal: of the
    # values up to each query).
    q = g.standard_normal((1, 1, 6, 4))
    k = np.ones((1, 1, 6, 4))
    np.testing.assert_allclose(oracle.attention(np.zeros_like(q), k, v)[0, 0], np.tile(v[0, 0].mean(0), (6, 1)),
                               rtol=1e-13)
    causal = oracle.attention(np.zeros_like(q), k, v, causal=True)[0, 0]
    np.testing.assert_allclose(causal, np.cumsum(v[0, 0], 0) / np.arange(1, 7)[:, None], rtol=1e-13)
    # One key far ahead of the others: its value row.
    k = np.zeros((1, 1, 6, 4))
    k[0, 0, 3, 0] = 1.0
    q = np.zeros((1, 1, 2, 4))
    q[..., 0] = 1000.0
    np.testing.assert_allclose(oracle.attention(q, k, v, scale=1.0)[0, 0], np.tile(v[0, 0, 3], (2, 1)), rtol=1e-12)


def test_stem_known_answer():
    """Reference stem KAT (tests/cpp/test_cuda.cpp:449-479): one-hot 7x7 weights,
    identity BatchNorm; the logits have a closed form."""
    graph, x, expected = workloads.stem_kat()
    got = oracle.evaluate(graph, {"input": x})["output"]
    np.testing.assert_allclose(got, expected, rtol=1e-7, atol=1e-9)
    # The closed form itself is not vacuous: logits are non-trivial.
    assert np.abs(expected).max() > 1e-3


def test_ffn_integer_pattern_vs_torch_float64():
    """The reference's FFN tokens=17 inputs (tests/cpp/test_cuda.cpp:336-358),
    through the oracle's graph walk, against torch float64 of the same graph."""
    graph, feeds = workloads.ffn_pattern()
    got = oracle.evaluate(graph, feeds)["output"]
    x = torch.from_numpy(feeds["x"].astype(np.float64))
    r = torch.from_numpy(feeds["residual"].astype(np.float64))
    w = torch.from_numpy(graph.constants["weight"][0].astype(np.float64))
    gamma = torch.from_numpy(graph.constants["scale"][0].astype(np.float64))
    beta = torch.from_numpy(graph.constants["bias"][0].astype(np.float64))
    want = F.layer_norm(F.gelu(x @ w) + r, (512,), gamma, beta, 1e-5).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-10)


def test_resnet_graph_walk_matches_torch_float64():
    """A reduced ResNet-50 (bs1, 64x64 image) through the oracle's graph walk
    (fused ops as the passes build them are exercised by the GPU tests; here the
    plain ONNX-style graph) vs the same graph in torch float64."""
    from oracle import torch_cpu

    graph = workloads.resnet50(1)
    graph.inputs["input"] = ((1, 3, 64, 64), "float32", "NCHW")
    x = rng(7).standard_normal((1, 3, 64, 64)).astype(np.float32)
    got = oracle.evaluate(graph, {"input": x})["output"]
    consts = torch_cpu.prepare(graph, dtype=torch.float64)
    want = torch_cpu.run(graph, consts, {"input": torch.from_numpy(x.astype(np.float64))})["output"].numpy()
    np.testing.assert_allclose(got, want, rtol=1e-9, atol=1e-9 * max(1.0, float(np.abs(want).max())))
