"""Row glue of the hybrid language model (ts_scale_add_*, ts_relu2_*) against
float64 autograd of the torch expressions it replaces: y = a x + b u with
per-channel factors (gradients of x, u, a and b; fp32 1e-6, bf16 one
rounding), and relu(z)^2, whose bf16 forward and backward equal the torch
chain bit for bit (the square of a bf16 value and its product with 2 g are
exact in fp32 before the one rounding)."""
from __future__ import annotations

import pytest
import torch

from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-6), (torch.bfloat16, 1e-2)])
@pytest.mark.parametrize("shape,fa,fb", [((3, 77, 512), True, True), ((2, 5, 64), False, True),
                                         ((1, 1, 960), True, False), ((4, 33, 16), False, False)])
def test_scale_add_matches_float64(cuda, dtype, tol, shape, fa, fb):
    from thetascan_amd import _lib
    from thetascan_amd._core.ops import rowglue

    g = torch.Generator().manual_seed(shape[1])
    W = shape[-1]
    x, u, dy = (torch.randn(shape, generator=g).to(dtype).double() for _ in range(3))
    a = (torch.randn(W, generator=g) + 1).to(dtype).double() if fa else None
    b = (torch.randn(W, generator=g) * 0.5).to(dtype).double() if fb else None
    leaves = [t if t is None else t.clone().requires_grad_(True) for t in (x, u, a, b)]
    lx, lu, la, lb = leaves
    ref = (lx if la is None else la * lx) + (lu if lb is None else lb * lu)
    ref.backward(dy)
    dev = [t if t is None else t.to(cuda, dtype).requires_grad_(True) for t in (x, u, a, b)]
    with _lib.record_launches() as recs:
        y = rowglue.scale_add(*dev)
        y.backward(dy.to(cuda, dtype))
        torch.cuda.synchronize()
    assert {"ts_scale_add_fwd", "ts_scale_add_bwd"} <= {r[0] for r in recs}
    errs = {"y": rel_err(y.float(), ref)}
    for name, t, l in zip("xuab", dev, leaves):
        if t is not None:
            errs["d" + name] = rel_err(t.grad.float(), l.grad)
    print(f"scale_add {shape} {dtype}: {errs}", flush=True)
    for k, e in errs.items():
        assert e < tol, (k, e)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_relu2_equals_the_torch_chain(cuda, dtype):
    from thetascan_amd._core.ops import rowglue

    g = torch.Generator().manual_seed(4)
    z = torch.randn(3, 50, 960, generator=g).to(cuda, dtype)
    dy = torch.randn(3, 50, 960, generator=g).to(cuda, dtype)
    z1, z2 = z.clone().requires_grad_(True), z.clone().requires_grad_(True)
    h1 = rowglue.relu2(z1)
    h1.backward(dy)
    h2 = torch.relu(z2).square()
    h2.backward(dy)
    torch.cuda.synchronize()
    assert torch.equal(h1, h2)
    if dtype == torch.bfloat16:
        assert torch.equal(z1.grad, z2.grad)
    else:
        assert rel_err(z1.grad, z2.grad) < 1e-6


def test_hybrid_lm_blocks_use_the_row_glue(cuda):
    """The LM's residual mixes, scaled adds and MLP activation run the row
    glue, and one training step's loss and gradients agree with the torch
    expressions within 2e-2 (bf16 model; the glue rounds once where torch
    rounds after each product; measured worst 7.1e-3)."""
    from thetascan_amd import _lib, hybrid_lm as lm
    from thetascan_amd._core.ops import rowglue

    torch.manual_seed(0)
    model = lm.HybridLM().to(cuda, torch.bfloat16)
    g = torch.Generator().manual_seed(1)
    idx = torch.randint(0, lm.VOCAB, (2, 128), generator=g).to(cuda)
    tgt = torch.randint(0, lm.VOCAB, (2, 128), generator=g).to(cuda)
    with torch.no_grad():
        for p in model.parameters():
            if float(p.abs().max()) == 0.0:
                p.normal_(0, 0.02)

    def run():
        model.zero_grad(set_to_none=True)
        with _lib.record_launches() as recs:
            loss = model(idx, tgt)
            loss.backward()
            torch.cuda.synchronize()
        return float(loss), {n: p.grad.float().clone() for n, p in model.named_parameters()}, recs

    l1, g1, recs = run()
    names = {r[0] for r in recs}
    assert {"ts_scale_add_fwd", "ts_scale_add_bwd", "ts_relu2_fwd", "ts_relu2_bwd"} <= names
    saved = rowglue.supported
    rowglue.supported = lambda *t: False
    try:
        l0, g0, _ = run()
    finally:
        rowglue.supported = saved
    assert abs(l1 - l0) < 1e-2 * abs(l0)
    errs = {n: rel_err(g1[n], g0[n]) for n in g0 if float(g0[n].abs().max()) > 0}
    worst = max(errs, key=errs.get)
    print(f"LM row glue: loss {l1:.5f} vs {l0:.5f}, worst gradient {worst} {errs[worst]:.3g}", flush=True)
    assert errs[worst] < 2e-2


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("rows,W,cap", [(300, 1024, 30.0), (77, 64, 2.0), (5, 2048, 5.0), (33, 8, 1.5)])
def test_softcap_cross_entropy_matches_float64(cuda, dtype, tol, rows, W, cap):
    """mean_r cross_entropy(cap tanh(z / cap), target) and its gradient in z
    against float64 autograd (the loss within 1e-5 relative for both dtypes,
    since it is an fp32 reduction of the given logits; dz fp32 1e-5, bf16 one
    rounding)."""
    from thetascan_amd import _lib
    from thetascan_amd._core.ops import rowglue

    g = torch.Generator().manual_seed(rows + W)
    z = (torch.randn(rows, W, generator=g) * 4).to(dtype)
    target = torch.randint(0, W, (rows,), generator=g)
    z64 = z.double().requires_grad_(True)
    ref = torch.nn.functional.cross_entropy(cap * torch.tanh(z64 / cap), target)
    ref.backward(torch.tensor(0.7, dtype=torch.float64))
    zd = z.to(cuda).requires_grad_(True)
    with _lib.record_launches() as recs:
        loss = rowglue.softcap_cross_entropy(zd, target.to(cuda), cap)
        loss.backward(torch.tensor(0.7, device=cuda))
        torch.cuda.synchronize()
    assert {"ts_softcap_xent_fwd", "ts_softcap_xent_bwd"} <= {r[0] for r in recs}
    e_loss = abs(float(loss) - float(ref)) / abs(float(ref))
    e_dz = rel_err(zd.grad.float(), z64.grad)
    print(f"softcap xent rows {rows} W {W} cap {cap} {dtype}: loss {e_loss:.3g} dz {e_dz:.3g}", flush=True)
    assert e_loss < 1e-5 and e_dz < tol


def test_softcap_cross_entropy_flags_targets_out_of_range(cuda):
    """A target outside [0, W) has no logit: its row's loss is NaN (the
    kernels have no ignored index), the other rows are unaffected."""
    from thetascan_amd import _lib
    from thetascan_amd._core.ops import rowglue

    z = torch.randn(4, 64, device=cuda)
    target = torch.tensor([1, 64, 3, -100], device=cuda)
    desc = _lib.RowsDesc(4, 64, _lib.TS_F32)
    loss = torch.empty(4, device=cuda)
    lse = torch.empty(4, device=cuda)
    lib = _lib.load()
    import ctypes
    assert lib.ts_softcap_xent_fwd(ctypes.byref(desc), z.data_ptr(), target.data_ptr(), 30.0, loss.data_ptr(),
                                   lse.data_ptr(), _lib.stream_handle(z.device)) == 0
    torch.cuda.synchronize()
    assert torch.isnan(loss[1]) and torch.isnan(loss[3])
    ref = torch.nn.functional.cross_entropy(30 * torch.tanh(z.double() / 30), torch.tensor([1, 0, 3, 0], device=cuda),
                                            reduction="none")
    assert torch.allclose(loss[[0, 2]].double(), ref[[0, 2]], rtol=1e-5)
    assert rowglue.xent_supported(z, target)
