"""The static-retention gradient summed pair by pair (ts_retention_grad,
GPU tests) against float64 autograd of the tiled oracle scan.

dL/dlog_alpha = sum_t sum_{i<=t} (t-i) alpha^(t-i) (q_t.k_i)(dO_t.v_i + dm_t):
checked for ragged and tile-multiple T, one and several segments, key widths
with a 16-wide tail block (16, 48, 80) and without, key widths that split
(192 = 128 + 64), value widths up to eight 16-column blocks per call and
wider ones that split (200), with and without the key-mass column, against the oracle at rel 1e-3 per head (bf16 inputs; the kernel's
own operands are hi/lo bf16 pairs; measured at most 5.1e-5), and through the bank
mixer's backward at T=4096, where the former sum_t t (q.dq - k.dk) in bf16
was 16% off.
"""
from __future__ import annotations

import pytest
import torch

from oracle import scans as oracle
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def _oracle_grad(q, k, v, dO, dm, la):
    """float64 autograd of the tiled scan: d sum(out . dO (+ mass dm)) / d log_alpha [H]."""
    lr = la.clone().requires_grad_(True)
    vv = v if dm is None else torch.cat([v, torch.ones(*v.shape[:3], 1, dtype=v.dtype)], -1)
    out = oracle.linattn_chunk(q, k, vv, oracle.as_stream(lr, q))
    loss = (out[..., :v.shape[-1]] * dO).sum()
    if dm is not None:
        loss = loss + (out[..., -1] * dm).sum()
    (g,) = torch.autograd.grad(loss, lr)
    return g


@pytest.mark.parametrize("T,dk,dv,mass,seg_tiles", [
    (1, 64, 64, False, 0), (63, 64, 64, True, 0), (64, 32, 16, True, 1), (65, 64, 64, True, 1),
    (300, 128, 64, True, 2), (300, 192, 80, False, 0), (1000, 64, 64, True, 0), (4096, 64, 64, True, 0),
    (130, 48, 112, True, 1), (200, 16, 200, True, 0), (129, 128, 120, False, 1), (777, 80, 56, True, 3),
])
def test_retention_grad_matches_float64_autograd(cuda, T, dk, dv, mass, seg_tiles):
    from thetascan_amd._core.ops import scan_hip

    B, H = 2, 3
    g = torch.Generator().manual_seed(T + dk + dv)
    bf = lambda t: t.to(torch.bfloat16).double()  # noqa: E731
    q = bf(torch.rand(B, H, T, dk, generator=g, dtype=torch.float64) / dk ** 0.5)
    k = bf(torch.rand(B, H, T, dk, generator=g, dtype=torch.float64) / dk ** 0.5)
    v = bf(torch.randn(B, H, T, dv, generator=g, dtype=torch.float64))
    dO = bf(torch.randn(B, H, T, dv, generator=g, dtype=torch.float64))
    dm = torch.randn(B, H, T, generator=g, dtype=torch.float64).float().double() if mass else None
    la = torch.log(torch.tensor([0.9, 0.99, 0.999], dtype=torch.float64))
    want = _oracle_grad(q, k, v, dO, dm, la)
    dev = lambda t: t.to(cuda, torch.bfloat16)  # noqa: E731
    got = scan_hip.retention_grad(dev(q), dev(k), dev(v), dev(dO), None if dm is None else dm.to(cuda, torch.float32),
                                  la.to(cuda, torch.float32), seg_tiles=seg_tiles).sum(0)
    print(f"retention grad T={T} dk={dk} dv={dv} mass={mass}: {got.tolist()} vs {want.tolist()}", flush=True)
    # every head on its own (the heads' gradients differ by orders of magnitude)
    for h in range(H):
        assert rel_err(got[h], want[h]) < 1e-3, (h, got.tolist(), want.tolist())


def test_bank_retention_gradient_at_T4096_in_bf16(cuda):
    """The fast-view retention gradient of a bf16 multi-view scan at T=4096
    (plain sum + two static retentions) against float64 autograd."""
    from thetascan_amd._core.ops import scan_hip

    B, H, T, D = 2, 4, 4096, 64
    g = torch.Generator().manual_seed(4097)
    q, k, v = (torch.randn(B, H, T, D, generator=g, dtype=torch.float64).to(torch.bfloat16).double() / 8
               for _ in range(3))
    dOs = [torch.randn(B, H, T, D, generator=g, dtype=torch.float64).to(torch.bfloat16).double() for _ in range(3)]
    las = [torch.log(torch.rand(H, generator=g, dtype=torch.float64) * 0.099 + 0.9) for _ in range(2)]
    wants = [_oracle_grad(q, k, v, dO, None, la) for dO, la in zip(dOs[1:], las)]
    qd, kd, vd = (t.to(cuda, torch.bfloat16).requires_grad_(True) for t in (q, k, v))
    rets = [None] + [la.to(cuda, torch.float32).requires_grad_(True) for la in las]
    outs = scan_hip.linattn_views(qd, kd, vd, tuple(rets))
    sum((o.float() * dO.to(cuda, torch.float32)).sum() for o, dO in zip(outs, dOs)).backward()
    for r, want in zip(rets[1:], wants):
        for h in range(H):
            assert rel_err(r.grad[h], want[h]) < 1e-3, (h, r.grad.tolist(), want.tolist())
