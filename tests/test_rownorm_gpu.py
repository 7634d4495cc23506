"""RMS-normed rows with the rotary turn and per-head gain (ts_rownorm_fwd /
ts_rownorm_bwd) against float64 autograd of the torch composition the hybrid
language model otherwise runs: F.rms_norm (its default eps, the fp32 machine
epsilon also for bf16 rows), the half-split rotation of hybrid_lm._rotate and
the query gain.

Widths 64 (attention heads) and 512 (the residual stream), strided views (a
transposed projection), with and without the turn and the gain, bf16 and
fp32, ragged row counts.  Tolerances: rel 1e-5 (fp32) and 2e-2 (bf16, one
rounding of the output) on y, dx and the gain's gradient (max-abs error over
max-abs reference).
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def reference(x, cos, sin, gain, eps):
    n = F.rms_norm(x, (x.shape[-1],), eps=eps)
    if cos is not None:
        h = x.shape[-1] // 2
        n1, n2 = n[..., :h], n[..., h:]
        c, s = cos[None, None], sin[None, None]
        n = torch.cat([n1 * c + n2 * s, n2 * c - n1 * s], -1)
    if gain is not None:
        n = n * gain[None, :, None, None]
    return n


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("W,H,rope,with_gain", [(64, 8, True, True), (64, 4, True, False), (64, 3, False, False),
                                               (512, 1, False, False), (16, 2, True, True), (128, 2, True, False)])
def test_rows_match_float64(cuda, dtype, tol, W, H, rope, with_gain):
    from thetascan_amd._core.ops import rownorm

    B, T = 2, 77
    g = torch.Generator().manual_seed(W + H)
    # a projection's [B, T, H, W] output seen as [B, H, T, W] (strided rows)
    base = (torch.randn(B, T, H, W, generator=g) * 3).to(dtype)
    x = base.to(cuda).transpose(1, 2).requires_grad_(True)
    ang = torch.outer(torch.arange(T, dtype=torch.float32), torch.rand(W // 2, generator=g))
    cos, sin = (ang.cos(), ang.sin()) if rope else (None, None)
    gain = (torch.rand(H, generator=g) + 0.5) if with_gain else None
    dy = torch.randn(B, H, T, W, generator=g).to(dtype)
    eps = float(torch.finfo(torch.float32).eps)  # F.rms_norm's default, bf16 rows included

    x64 = base.double().transpose(1, 2).clone().requires_grad_(True)
    g64 = gain.double().clone().requires_grad_(True) if with_gain else None
    ref = reference(x64, None if cos is None else cos.double(), None if sin is None else sin.double(), g64, eps)
    ref.backward(dy.double())

    gd = gain.to(cuda).requires_grad_(True) if with_gain else None
    y = rownorm.rms_rows(x, None if cos is None else cos.to(cuda), None if sin is None else sin.to(cuda), gd)
    y.backward(dy.to(cuda))
    torch.cuda.synchronize()
    assert y.dtype == dtype and y.shape == (B, H, T, W)
    errs = {"y": rel_err(y.float(), ref), "dx": rel_err(x.grad.float(), x64.grad)}
    if with_gain:
        errs["dgain"] = rel_err(gd.grad, g64.grad)
    print(f"rownorm W={W} H={H} rope={rope} gain={with_gain} {dtype}: {errs}", flush=True)
    for name, e in errs.items():
        assert e < tol, (name, e)


def test_default_eps_is_the_one_rms_norm_uses(cuda):
    """Small rows (mean square far below bf16's machine epsilon) normalize as
    F.rms_norm does by default."""
    from thetascan_amd._core.ops import rownorm

    x = (torch.randn(2, 1, 33, 64, generator=torch.Generator().manual_seed(5)) * 0.01).to(torch.bfloat16)
    ref = F.rms_norm(x.double(), (64,), eps=float(torch.finfo(torch.float32).eps))
    assert rel_err(rownorm.rms_rows(x.to(cuda)).float(), ref) < 2e-2


def test_rows_refuse_unsupported_widths(cuda):
    from thetascan_amd._core.ops import rownorm

    x = torch.zeros(1, 1, 4, 48, device=cuda)
    assert not rownorm.supported(x)
    with pytest.raises(NotImplementedError):
        rownorm.rms_rows(x)


def test_hybrid_lm_uses_the_row_kernel(cuda):
    """The LM's attention prologue and residual norms run ts_rownorm and agree
    with the torch composition (bf16 model, loose bar: the composition rounds
    to bf16 between its steps)."""
    from thetascan_amd import _lib, hybrid_lm as lm

    torch.manual_seed(0)
    model = lm.HybridLM().to(cuda, torch.bfloat16)
    attn = model.blocks[0].attn
    x = torch.randn(2, 64, lm.D_MODEL, device=cuda, dtype=torch.bfloat16)
    with _lib.record_launches() as recs:
        y = attn(lm._rms(x))
        torch.cuda.synchronize()
    names = {r[0] for r in recs}
    assert "ts_rownorm_fwd" in names
    B, T, D = x.shape
    xn = F.rms_norm(x, (D,))
    q = attn.c_q(xn).view(B, T, attn.heads, attn.hd).transpose(1, 2)
    k = attn.c_k(xn).view(B, T, attn.kv_heads, attn.hd).transpose(1, 2)
    v = attn.c_v(xn).view(B, T, attn.kv_heads, attn.hd).transpose(1, 2)
    cos, sin = attn.rotary(T, cuda)
    q = lm._rotate(F.rms_norm(q, (attn.hd,)), cos, sin) * attn.q_gain.to(q.dtype)[None, :, None, None]
    k = lm._rotate(F.rms_norm(k, (attn.hd,)), cos, sin)
    rep = attn.heads // attn.kv_heads
    o = lm.attention(q.contiguous(), k.repeat_interleave(rep, 1).contiguous(), v.repeat_interleave(rep, 1).contiguous())
    ref = attn.proj(o.transpose(1, 2).reshape(B, T, D))
    # the output projection starts at zero: compare the attention output itself
    with torch.no_grad():
        attn.proj.weight.normal_(0, 0.05)
        y = attn(lm._rms(x))
        ref = attn.proj(o.transpose(1, 2).reshape(B, T, D))
    assert rel_err(y.float(), ref.float()) < 5e-2
