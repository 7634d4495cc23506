"""Closed-form and brute-force checks of the CPU oracle (CPU tests).

These pin what the golden vectors leave open, chosen so that a plausible
slip -- a dropped decay term, an off-by-one in the retention exponent, a
transposed operand, a wrong knot vector -- fails at least one of them.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import expansion, mixer, scans


def test_constant_stream_closed_form():
    """q = k = v = 1, static alpha: out_t = (1 - a^(t+1)) / (1 - a)
    (the reference's closed form, tests/test_scan_chunk.py:140-221)."""
    T = 50
    ones = torch.ones(1, 2, T, 1, dtype=torch.float64)
    la = torch.log(torch.tensor([0.9, 0.5], dtype=torch.float64))
    out = scans.linattn_naive(ones, ones, ones, scans.as_stream(la, ones))
    t = torch.arange(T, dtype=torch.float64)
    for h, a in enumerate((0.9, 0.5)):
        expected = (1 - a ** (t + 1)) / (1 - a)
        assert torch.allclose(out[0, h, :, 0], expected, rtol=1e-13, atol=0)


def test_hand_computed_three_tokens():
    """out_2 = q2 . (a2 a1 k0 v0 + a2 k1 v1 + k2 v2) with scalar features."""
    q = torch.tensor([1.0, 2.0, 3.0], dtype=torch.float64).view(1, 1, 3, 1)
    k = torch.tensor([0.5, -1.0, 2.0], dtype=torch.float64).view(1, 1, 3, 1)
    v = torch.tensor([4.0, 1.0, -2.0], dtype=torch.float64).view(1, 1, 3, 1)
    a = torch.tensor([0.3, 0.7, 0.2], dtype=torch.float64)
    out = scans.linattn_naive(q, k, v, a.log().view(1, 1, 3, 1))
    s0 = 0.5 * 4.0
    s1 = 0.7 * s0 + (-1.0) * 1.0
    s2 = 0.2 * s1 + 2.0 * -2.0
    assert torch.allclose(out.view(3), torch.tensor([1 * s0, 2 * s1, 3 * s2], dtype=torch.float64))


def test_quad_equals_naive_brute_force():
    g = torch.Generator().manual_seed(3)
    q, k = torch.randn(2, 3, 21, 4, generator=g, dtype=torch.float64), torch.randn(2, 3, 21, 4, generator=g, dtype=torch.float64)
    v = torch.randn(2, 3, 21, 5, generator=g, dtype=torch.float64)
    decay = -torch.rand(2, 3, 21, 1, generator=g, dtype=torch.float64)
    assert torch.allclose(scans.linattn_quad(q, k, v, decay), scans.linattn_naive(q, k, v, decay), atol=1e-12)
    assert torch.allclose(scans.linattn_cumsum(q, k, v, decay), scans.linattn_naive(q, k, v, decay), atol=1e-10)


def test_cumsum_clamp_fails_exactly_where_documented():
    """Beyond exp(-60) accumulated decay the reference's cumsum form loses the
    leading terms (scan_cumsum.py:4, 15-19); the naive loop does not."""
    T = 100
    ones = torch.ones(1, 1, T, 1, dtype=torch.float64)
    decay = torch.full((1, 1, T, 1), -1.0, dtype=torch.float64)
    naive = scans.linattn_naive(ones, ones, ones, decay)
    cum = scans.linattn_cumsum(ones, ones, ones, decay)
    assert torch.allclose(naive[..., :59, :], cum[..., :59, :], rtol=1e-10)
    assert not torch.allclose(naive[..., 90:, :], cum[..., 90:, :], rtol=1e-3)


def test_ema_cumsum_is_the_unit_query_scan():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 3, 30, 6, generator=g, dtype=torch.float64)
    la = torch.log(torch.tensor([0.9, 0.5, 0.99], dtype=torch.float64))
    ones = torch.ones(2, 3, 30, 1, dtype=torch.float64)
    assert torch.allclose(scans.ema_cumsum(x, la), scans.linattn_naive(ones, ones, x, scans.as_stream(la, x)))


def test_bspline_matches_library_basis_and_partition_of_unity():
    scipy_interp = pytest.importorskip("scipy.interpolate")
    n_basis, degree, bound = 8, 3, 3.0
    inner = np.linspace(-bound, bound, n_basis - degree + 1)[1:-1]
    knots = np.concatenate([[-bound] * (degree + 1), inner, [bound] * (degree + 1)])
    xs = np.linspace(-2.999, 2.999, 301)
    got = mixer.bspline_basis(torch.tensor(xs).view(1, 1, -1, 1), n_basis, degree, bound).view(-1, n_basis)
    for j in range(n_basis):
        coef = np.zeros(n_basis)
        coef[j] = 1.0
        ref = scipy_interp.BSpline(knots, coef, degree)(xs)
        assert np.allclose(got[:, j].numpy(), ref, atol=1e-12), j
    assert torch.allclose(got.sum(-1), torch.ones(len(xs), dtype=torch.float64))
    assert int((got > 0).sum(-1).max()) <= degree + 1
    # the right endpoint maps onto the last basis function
    end = mixer.bspline_basis(torch.tensor([[[[bound]]]], dtype=torch.float64), n_basis, degree, bound)
    assert float(end[..., -1]) == pytest.approx(1.0)


def test_relu2_ridge_is_a_simplex_with_uniform_fallback():
    pre = torch.tensor([[[[1.0, -2.0, 3.0, 0.5]], [[-1.0, -2.0, -3.0, -0.5]]]], dtype=torch.float64)
    f = mixer.relu2_ridge(pre)
    assert torch.allclose(f[0, 0, 0], torch.tensor([1.0, 0.0, 9.0, 0.25], dtype=torch.float64) / 10.25)
    assert torch.allclose(f[0, 1, 0], torch.full((4,), 0.25, dtype=torch.float64))


def test_rope_relative_dot_identity():
    """<R_s x, R_t y> depends only on t - s (tests/test_feature_rope.py:300-337)."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(8, generator=g, dtype=torch.float64)
    y = torch.randn(8, generator=g, dtype=torch.float64)
    T = 20
    xs = mixer.apply_rope(x.expand(1, 1, T, 8).clone(), "full", 1.0, 100.0)
    ys = mixer.apply_rope(y.expand(1, 1, T, 8).clone(), "full", 1.0, 100.0)
    d1 = (xs[0, 0, 3] * ys[0, 0, 7]).sum()
    d2 = (xs[0, 0, 10] * ys[0, 0, 14]).sum()
    assert torch.allclose(d1, d2, rtol=1e-12)


def test_expansion_map_magnitudes():
    m = expansion.row_map((1, 24, 12), "k", "w1-expand-layer-0")
    assert torch.allclose(m.abs(), torch.full_like(m, 1.0 / math.sqrt(12)))
    assert not torch.equal(m, expansion.row_map((1, 24, 12), "k2", "w1-expand-layer-0"))


def _streams(T=37, Dk=5, Dv=4, seed=20260725):
    """B=2, H=3 streams and log-retentions [-0.05, -0.4, -2.0], the shapes of
    the reference's scan fixture (tests/test_scan_chunk.py:15-24)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(2, 3, T, Dk, generator=g, dtype=torch.float64)
    k = torch.randn(2, 3, T, Dk, generator=g, dtype=torch.float64)
    v = torch.randn(2, 3, T, Dv, generator=g, dtype=torch.float64)
    la = torch.tensor([-0.05, -0.4, -2.0], dtype=torch.float64)
    stream = -torch.rand(2, 3, T, 1, generator=g, dtype=torch.float64)
    return q, k, v, la, stream


@pytest.mark.parametrize("chunk", [1, 3, 8, 64, 128])
@pytest.mark.parametrize("retention", ["none", "static", "stream"])
def test_chunk_oracle_equals_naive(chunk, retention):
    """The tiled oracle against the recurrence at 1e-12 for chunks that divide
    T, leave a ragged last tile, or exceed T (tests/test_scan_chunk.py:55-123)."""
    q, k, v, la, stream = _streams()
    decay = {"none": None, "static": scans.as_stream(la, q), "stream": stream}[retention]
    got = scans.linattn_chunk(q, k, v, decay, chunk=chunk)
    ref = scans.linattn_naive(q, k, v, decay)
    assert torch.allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_chunk_oracle_gradients_equal_naive():
    q, k, v, la, stream = _streams(T=29)
    args = [t.clone().requires_grad_(True) for t in (q, k, v, stream)]
    dy = torch.randn(2, 3, 29, 4, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    grads = []
    for fn in (lambda *a: scans.linattn_chunk(*a, chunk=8), scans.linattn_naive):
        for t in args:
            t.grad = None
        (fn(*args) * dy).sum().backward()
        grads.append([t.grad.clone() for t in args])
    for a, b in zip(*grads):
        assert torch.allclose(a, b, rtol=1e-10, atol=1e-12)


def test_final_state_closed_form_and_one_hot_reads():
    """final_state_naive equals N_T = sum_i w_i k_i v_i^T, w_i = prod_{i<j<=T-1} a_j,
    and reading it with one-hot queries reproduces the last output row of the
    recurrence (out_{T-1} = q_{T-1} S_{T-1})."""
    q, k, v, la, stream = _streams(T=23)
    for decay in (None, scans.as_stream(la, q), stream):
        S = scans.final_state_naive(k, v, decay)
        if decay is None:
            w = torch.ones(2, 3, 23, dtype=torch.float64)
        else:
            L = decay[..., 0]
            # weight of token i at the end: exp(sum_{j>i} log a_j)
            w = (L.sum(-1, keepdim=True) - L.cumsum(-1)).exp()
        closed = torch.einsum("bht,bhtk,bhtv->bhkv", w, k, v)
        assert torch.allclose(S, closed, rtol=1e-12, atol=1e-12)
        eye = torch.eye(5, dtype=torch.float64).expand(2, 3, 5, 5)
        # queries e_j at the last step read row j of S_{T-1}
        qq = torch.zeros(2, 3, 23, 5, dtype=torch.float64)
        for j in range(5):
            qq[:, :, -1] = eye[:, :, j]
            out = scans.linattn_naive(qq, k, v, decay)
            assert torch.allclose(out[:, :, -1], S[:, :, j], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("case", ["kernel_softmax_bank_fast", "kernel_relu2_threshold_feature_mass_ema"])
def test_kernel_final_states_equal_the_recurrence(case):
    """oracle.mixer.kernel_final_states (closed form per view) equals the
    naive recurrence's final state on the mixer's own write streams, view by
    view (the plain sum or ema stream, then each recency branch)."""
    import torch.nn.functional as F

    from oracle import mixer
    from tests.test_oracle_golden import load_case

    pub, params, _, arrays = load_case(case)
    c = mixer.core_config(pub)
    x = arrays["x"]
    finals = mixer.kernel_final_states(c, params, x)
    _, streams, _, _, _, decay = mixer._write_side(c, params, x)
    keys, vals = streams["la2"][0]
    ones = torch.ones(*keys.shape[:3], 1, dtype=keys.dtype)
    decays = [decay]
    if c["read_fade"]:
        raw = params["fade_alpha"]
        raw = raw.unsqueeze(0) if raw.ndim == 1 else raw
        decays += [scans.as_stream(-F.softplus(-raw[j]), keys) for j in range(c["fade_branches"])]
    assert len(finals) == len(decays)
    for (N, D), dec in zip(finals, decays):
        S = scans.final_state_naive(keys, torch.cat([vals, ones], -1), dec)
        assert torch.allclose(N, S[..., :-1], rtol=1e-10, atol=1e-12)
        assert torch.allclose(D, S[..., -1], rtol=1e-10, atol=1e-12)
