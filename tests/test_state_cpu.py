"""The streaming state object on the CPU: size, copies and serialization."""
from __future__ import annotations

import io

import torch

import thetascan_amd as ts


def _state():
    g = torch.Generator().manual_seed(0)
    carries = ([torch.randn(2, 4, 16, 17, generator=g)], [torch.randn(2, 4, 16, 16, generator=g)] * 2,
               torch.randn(2, 4, 16, generator=g))
    return ts.ThetaScanState(fingerprint="f" * 32, position=7, batch=2, carries=carries)


def test_size_copies_and_round_trip():
    st = _state()
    assert st.nbytes == 4 * (2 * 4 * 16 * 17 + 2 * 2 * 4 * 16 * 16 + 2 * 4 * 16)
    c = st.clone()
    c.carries[0][0].add_(1.0)
    assert not torch.equal(c.carries[0][0], st.carries[0][0])
    buf = io.BytesIO()
    torch.save(st.state_dict(), buf)
    buf.seek(0)
    back = ts.ThetaScanState.from_state_dict(torch.load(buf, weights_only=True))
    assert (back.fingerprint, back.position, back.batch) == (st.fingerprint, 7, 2)
    assert len(back.carries) == 3
    for a, b in zip(back._tensors(), st._tensors()):
        assert torch.equal(a, b)


def test_initial_state_and_config_identity():
    a = ts.ThetaScan(ts.ThetaScanConfig(d_model=64, n_heads=2, family="kernel"))
    b = ts.ThetaScan(ts.ThetaScanConfig(d_model=64, n_heads=2, family="gn"))
    sa, sb = a.initial_state(), b.initial_state()
    assert sa.position == 0 and sa.nbytes == 0 and sa.carries == ()
    assert sa.fingerprint == a.initial_state().fingerprint != sb.fingerprint
