"""Key features that also write the forward scan's segment summaries
(ts_feature_fwd_summary, then ts_scan_fwd with states_in = 3).

The memory's forward scan sum_i <phi(q_t), phi(k_i)> v_i (with the key-mass
ones column when the read is normalized) folds each segment's writes into a
summary before its prefix pass.  The key feature kernel can emit those
summaries itself while phi(k) is still in LDS, so the scan never re-reads
phi(k) and v for them.  The summaries are computed with the scan summary
pass's own MFMA sequence, so the features, the scan outputs, the key mass and
the kept segment states must equal those of the two separate calls bit for
bit (ragged T, one and many segments, both kernel maps, RoPE and tau).
"""
from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

CASES = [
    # B, H, T, seg_chunks, kind, in_rot, feat_rot, tau, normalize
    (2, 4, 300, 0, "relu2", 0, 0, True, True),
    (1, 3, 1000, 2, "softmax", 32, 32, False, True),
    (2, 2, 777, 3, "softmax", 64, 0, True, False),
    (1, 2, 4096, 8, "relu2", 0, 32, True, True),
    (1, 1, 65, 1, "relu2", 0, 0, False, True),
    (2, 8, 4096, 0, "softmax", 32, 0, True, True),
]


def _proj(B, T, H, d, dtype, device, gen):
    """q, k, v as [B,H,T,d] strided views of one [B,T,3*H*d] projection."""
    P = torch.randn(B, T, 3 * H * d, generator=gen).to(device=device, dtype=dtype)
    views = P.view(B, T, 3, H, d).permute(2, 0, 3, 1, 4)
    return P, views[0], views[1], views[2]


@pytest.mark.parametrize("case", CASES)
def test_summaries_from_the_feature_kernel_match_the_scan(cuda, case):
    from thetascan_amd import _lib
    from thetascan_amd._core.ops import fused, scan_hip

    B, H, T, seg_chunks, kind, in_rot, feat_rot, has_tau, normalize = case
    d = m = 64
    dt = torch.bfloat16
    gen = torch.Generator().manual_seed(T + H)
    _, q, k, v = _proj(B, T, H, d, dt, cuda, gen)
    w1 = (torch.randn(H, m, d, generator=gen) / 8).to(cuda, dt)
    w2 = (torch.randn(H, d, m, generator=gen) / 8).to(cuda, dt)
    tau = (torch.randn(H, generator=gen) * 0.1).to(cuda) if has_tau else None
    code = _lib.FEAT_RELU2 if kind == "relu2" else _lib.FEAT_SOFTMAX
    spec = fused.FeatureSpec(code, m, 8.0, in_rot, feat_rot, 10000.0, 0.5)
    phi_q, _ = fused.feature_fwd(spec, q, w1, w2, tau, True)

    results = []
    for summ in (False, True):
        ws = scan_hip.workspace_for(k, k, v, seg_chunks=seg_chunks, v_ext=normalize)
        if ws is None:
            pytest.skip("one segment: no summaries")
        ws.zero_()
        if summ:
            phi_k = fused.feature_fwd_summary(spec, k, w1, tau, v, normalize, seg_chunks, ws)
        else:
            phi_k, _ = fused.feature_fwd(spec, k, w1, None, tau, False)
        out, mass, _ = scan_hip.scan_launch(phi_q, phi_k, v, v_ext="ones" if normalize else None,
                                           want_ext_out=normalize, seg_chunks=seg_chunks, workspace=ws,
                                           states_in=3 if summ else 0)
        torch.cuda.synchronize()
        results.append((phi_k, out, mass, ws))
    (pa, oa, ma, wa), (pb, ob, mb, wb) = results
    assert torch.equal(pa, pb)
    assert torch.equal(oa, ob)
    if normalize:
        assert torch.equal(ma, mb)
    assert torch.equal(wa, wb), "kept segment states differ"


def test_summary_mode_rejects_what_it_does_not_cover(cuda):
    """fp32 features, another width, a retention or a final state are refused
    with an error instead of writing summaries the scan would misread."""
    from thetascan_amd import _lib
    from thetascan_amd._core.ops import fused

    lib = _lib.load()
    B, H, T = 1, 2, 512
    gen = torch.Generator().manual_seed(1)
    spec = fused.FeatureSpec(_lib.FEAT_RELU2, 64, 8.0, 0, 0, 10000.0, 0.5)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device=cuda)

    def call(x, v, **over):
        fields = dict(B=B, H=H, T=T, dk=64, dv=64, dtype=_lib.dtype_code(x.dtype), retention=_lib.RET_NONE,
                      reverse=0, q_ext=0, k_ext=0, v_ext=_lib.EXT_ONES, out_mode=_lib.OUT_STORE, out_scale=1.0,
                      seg_chunks=2, want_final=0, value_split=0, states_in=3, init_state=0)
        fields.update(over)
        sdesc = _lib.ScanDesc(**fields)
        w1 = torch.zeros(H, 64, x.shape[-1], dtype=x.dtype, device=cuda)
        phi = torch.empty(B, H, T, 64, dtype=x.dtype, device=cuda)
        io = _lib.FeatureIO(_lib.strided(x), w1.data_ptr(), None, None, None, None, None, None,
                            _lib.strided(phi), _lib.strided(None))
        desc = spec.desc(x, False)
        return lib.ts_feature_fwd_summary(ctypes.byref(desc), ctypes.byref(io), _lib.strided(v),
                                          ctypes.byref(sdesc), ws.data_ptr(), ws.numel(),
                                          _lib.stream_handle(cuda))

    xb = torch.randn(B, H, T, 64, generator=gen).to(cuda, torch.bfloat16)
    vb = torch.randn(B, H, T, 64, generator=gen).to(cuda, torch.bfloat16)
    assert call(xb, vb) == _lib.TS_OK
    assert call(xb.float(), vb.float()) != _lib.TS_OK
    assert call(xb, vb, retention=_lib.RET_STATIC) != _lib.TS_OK
    assert call(xb, vb, want_final=1) != _lib.TS_OK
    assert call(xb, vb, k_ext=_lib.EXT_ONES, q_ext=_lib.EXT_ONES) != _lib.TS_OK
    x32 = torch.randn(B, H, T, 32, generator=gen).to(cuda, torch.bfloat16)
    assert call(x32, vb) != _lib.TS_OK
    torch.cuda.synchronize()
