"""Decode steps replayed from a captured HIP graph (thetascan_amd.DecodeGraph)
against the eager continuation (GPU tests).

For the benchmark layouts and every golden reference configuration, in fp32
and bf16: a prompt is run eagerly into a state, then six one-token steps are
taken eagerly (``mixer(x_t, state=s)``) and by graph replays from the same
state, with eager work and device synchronisations between the replays (a
graph node that only behaves on its first replay is caught).  The carried
states must agree bit for bit and the fp32 outputs too; bf16 outputs within
2e-2 (the library GEMMs may pick another solution for a captured call; the
measured differences are one bf16 rounding step, <= 6.4e-3).  The eager
continuation itself is checked against the float64 whole-sequence oracle in
tests/test_stream_gpu.py.
"""
from __future__ import annotations

import pytest
import torch

from tests.conftest import rel_err
from tests.test_stream_gpu import CASES, _module

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("name", ["headline_2a", "headline_2b"] + sorted(CASES))
def test_decode_graph_replays_the_eager_steps(cuda, name, dtype):
    import thetascan_amd as ts

    module, pub = _module(name, cuda)
    module = module.to(dtype)
    D = pub["d_model"]
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 70, D, generator=g).to(cuda, dtype)
    xs = torch.randn(2, 6, D, generator=g).to(cuda, dtype)
    with torch.no_grad():
        _, st = module(x, state=module.initial_state())
        s, expected = st.clone(), []
        for t in range(6):
            y, s = module(xs[:, t:t + 1], state=s)
            expected.append(y)
        dec = ts.DecodeGraph(module, st)
        errs = []
        for t in range(6):
            y = dec.step(xs[:, t:t + 1]).clone()
            module(x[:, :9])  # eager work between replays
            torch.cuda.synchronize()
            errs.append(rel_err(y, expected[t]))
        fin = dec.state()
    print(f"{name} {dtype}: max rel err {max(errs):.3g}", flush=True)
    assert fin.position == st.position + 6 and fin.fingerprint == st.fingerprint
    for a, b in zip(fin._tensors(), s._tensors()):
        assert torch.equal(a, b), name
    if dtype == torch.float32:
        assert max(errs) == 0.0, name
    else:
        assert max(errs) < 2e-2, name
    # the state handed back is independent of the graph's buffers
    before = [t.clone() for t in fin._tensors()]
    with torch.no_grad():
        dec.step(xs[:, :1])
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(fin._tensors(), before))


def test_decode_graph_spans_rope_blocks_and_several_tokens(cuda):
    """Steps of three tokens across a 1024-position block boundary of the
    RoPE tables (phases formed on the device from the position counter)."""
    import thetascan_amd as ts

    module, pub = _module("headline_2a", cuda)
    D = pub["d_model"]
    g = torch.Generator().manual_seed(8)
    x = torch.randn(1, 1020, D, generator=g).to(cuda)
    xs = torch.randn(1, 9, D, generator=g).to(cuda)
    with torch.no_grad():
        _, st = module(x, state=module.initial_state())
        s, expected = st.clone(), []
        for t in range(0, 9, 3):
            y, s = module(xs[:, t:t + 3], state=s)
            expected.append(y)
        dec = ts.DecodeGraph(module, st, tokens=3)
        got = [dec.step(xs[:, t:t + 3]).clone() for t in range(0, 9, 3)]
    torch.cuda.synchronize()
    for a, b in zip(got, expected):
        assert torch.equal(a, b)
    assert dec.state().position == 1029


@pytest.mark.parametrize("name", ["headline_2b", "kernel_softmax_bank_fast"])
def test_decode_graph_with_tiled_steps(cuda, name):
    """Steps of sixteen tokens take the tiled scan passes (summary, prefix and
    main) under capture, their final states written in place: fp32 replays
    equal the eager continuation bit for bit."""
    import thetascan_amd as ts

    module, pub = _module(name, cuda)
    D = pub["d_model"]
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 100, D, generator=g).to(cuda)
    xs = torch.randn(2, 48, D, generator=g).to(cuda)
    with torch.no_grad():
        _, st = module(x, state=module.initial_state())
        s, expected = st.clone(), []
        for t in range(0, 48, 16):
            y, s = module(xs[:, t:t + 16], state=s)
            expected.append(y)
        dec = ts.DecodeGraph(module, st, tokens=16)
        got = []
        for t in range(0, 48, 16):
            got.append(dec.step(xs[:, t:t + 16]).clone())
            torch.cuda.synchronize()
        fin = dec.state()
    for a, b in zip(got, expected):
        assert torch.equal(a, b), name
    for a, b in zip(fin._tensors(), s._tensors()):
        assert torch.equal(a, b), name
    assert fin.position == 148


def test_decode_graph_rejects_bad_use(cuda):
    import thetascan_amd as ts

    module, pub = _module("headline_2a", cuda)
    with pytest.raises(ValueError, match="seen tokens"):
        ts.DecodeGraph(module, module.initial_state())
    x = torch.randn(2, 4, pub["d_model"], device=cuda)
    with torch.no_grad():
        _, st = module(x, state=module.initial_state())
        dec = ts.DecodeGraph(module, st)
        with pytest.raises(ValueError, match="shape"):
            dec.step(x)
        # an in-place parameter update is seen by the next replay; a replaced
        # parameter is refused before any replay
        w = module._core.proj_out.weight
        w.mul_(2.0)
        y_eager, _ = module(x[:, :1], state=dec.state())
        assert torch.equal(dec.step(x[:, :1]), y_eager)
        w.data = w.data.clone()
        with pytest.raises(RuntimeError, match="replaced"):
            dec.step(x[:, :1])
