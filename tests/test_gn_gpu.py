"""HIP GN write payloads (ts_gn_write_fwd/bwd) against the oracle (fp64, CPU).

The oracle's write_streams (a restatement of engine.py:117-340, pinned by the
reference's GN mixer vectors in tests/golden) gives h, s*lam and g for a
depth-1 ReLU^2 memory; its autograd gives every gradient the HIP backward
must reproduce: dx (through h, lam and g), dv, dW1, dW2 and the per-feature
threshold.
"""
from __future__ import annotations

import pytest
import torch

from oracle import mixer
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def _cfg(learn_thresh):
    return {"write_rule": "gn", "nonlin": "relu2", "depth": 1, "fast_w1": True, "write_iters": 1,
            "learn_thresh": learn_thresh, "value_centers": 0}


def _case(B, H, T, d, m, learn_thresh, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(B, H, T, d, generator=g, dtype=torch.float64)
    k = k / k.norm(dim=-1, keepdim=True)
    v = torch.randn(B, H, T, d, generator=g, dtype=torch.float64)
    w1 = torch.randn(H, m, d, generator=g, dtype=torch.float64) / d ** 0.5
    w2 = torch.randn(H, d, m, generator=g, dtype=torch.float64) * 0.3
    wg = (torch.randn(H, m, 1, generator=g, dtype=torch.float64) * 0.3) if learn_thresh else None
    rnd = lambda t: None if t is None else t.to(dtype).to(torch.float64)  # noqa: E731
    return rnd(k), rnd(v), rnd(w1), rnd(w2), rnd(wg)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d,m,learn_thresh,T", [(16, 48, False, 70), (64, 128, False, 150), (32, 96, True, 64),
                                               (16, 16, True, 33), (128, 64, False, 40)])
def test_gn_write_matches_oracle(cuda, dtype, d, m, learn_thresh, T):
    from thetascan_amd._core.ops import gn

    B, H = 2, 3
    k, v, w1, w2, wg = _case(B, H, T, d, m, learn_thresh, 100 * d + m + T, dtype)
    c = _cfg(learn_thresh)
    # oracle forward + backward (fp64)
    rk, rv, rw1, rw2 = (t.clone().requires_grad_(True) for t in (k, v, w1, w2))
    rwg = wg.clone().requires_grad_(True) if learn_thresh else None
    st = mixer.write_streams([(rw1, rw2, rwg)], c, rk, rv, None, {})
    (xk, g_ref), = st["la1"]
    (h_ref, lam_ref), = st["la2"]
    gen = torch.Generator().manual_seed(7)
    dh = torch.randn(h_ref.shape, generator=gen, dtype=torch.float64)
    dl = torch.randn(lam_ref.shape, generator=gen, dtype=torch.float64)
    dg = torch.randn(g_ref.shape, generator=gen, dtype=torch.float64) * 0.1
    torch.autograd.backward([h_ref, lam_ref, g_ref], [dh, dl, dg])

    dev = lambda t: None if t is None else t.to(cuda, dtype).requires_grad_(True)  # noqa: E731
    x_, v_, w1_, w2_ = dev(k), dev(v), dev(w1), dev(w2)
    tau_ = dev(wg[..., 0].contiguous()) if learn_thresh else None
    h, lam, g = gn.write(x_, v_, w1_, w2_, tau_)
    torch.autograd.backward([h, lam, g], [dh.to(cuda, dtype), dl.to(cuda, dtype), dg.to(cuda, dtype)])

    tol = 2e-3 if dtype == torch.float32 else 3e-2
    for name, a, e in (("h", h, h_ref), ("lam", lam, lam_ref), ("g", g, g_ref)):
        assert rel_err(a, e) < tol, (name, d, m, learn_thresh)
    gtol = 5e-3 if dtype == torch.float32 else 6e-2
    grads = [("dx", x_.grad, rk.grad), ("dv", v_.grad, rv.grad), ("dW1", w1_.grad, rw1.grad),
             ("dW2", w2_.grad, rw2.grad)]
    if learn_thresh:
        grads.append(("dtau", tau_.grad, rwg.grad[..., 0]))
    for name, a, e in grads:
        assert rel_err(a, e) < gtol, (name, d, m, learn_thresh, rel_err(a, e))


def test_gn_write_rejects_unsupported_widths(cuda):
    from thetascan_amd._core.ops import gn

    x = torch.zeros(1, 1, 8, 24, device=cuda)
    w1 = torch.zeros(1, 32, 24, device=cuda)
    w2 = torch.zeros(1, 24, 32, device=cuda)
    with pytest.raises(NotImplementedError):
        gn.write(x, x, w1, w2)
