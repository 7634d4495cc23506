"""Decode steps of a mixer replayed from one captured HIP graph.

A decode step at a small batch is launch-bound: one token per sequence gives
every kernel of the step (projections, feature maps, the scan's token-by-token
recurrence, the read, the output projection) a few microseconds of work, while
issuing its twenty-odd launches through Python costs several times that.
:class:`DecodeGraph` records one step once -- with the carried state in fixed
buffers that the step updates in place and the position (RoPE phases) held in
a device counter -- and replays it::

    with torch.no_grad():
        _, state = mixer(prompt, state=mixer.initial_state())   # prefill, eager
    dec = DecodeGraph(mixer, state)
    for t in range(n):
        y = dec.step(x_t)            # [B, 1, D]; overwritten by the next step
    state = dec.state()              # an ordinary ThetaScanState again

Each replay computes what ``mixer(x_t, state=state)`` computes (the same
kernels on the same buffers; RoPE phases formed from the same exact fp32
integer positions).  The recorded step reads the mixer's parameters in
place: in-place updates (an optimizer step) are seen, while a parameter whose
storage was replaced (``.to()``, assignment to ``.data``) makes the next step
raise instead of reading memory the graph no longer owns.  The batch size and
tokens per step are fixed at capture.  Nothing is allocated per step.
"""
from __future__ import annotations

import torch

from ._core.ops import stream
from .state import ThetaScanState


class DecodeGraph:
    """One captured decode step of ``mixer`` continuing ``state``.

    ``mixer`` is a :class:`thetascan_amd.ThetaScan` (or its core module);
    ``state`` a state that has seen at least one token (the prefill call
    creates its buffers); ``tokens`` the tokens per sequence of each step.
    """

    def __init__(self, mixer, state: ThetaScanState, tokens: int = 1, warmup: int = 2):
        if not state.carries:
            raise ValueError("DecodeGraph continues a state that has seen tokens: run the prompt through "
                             "mixer(x, state=mixer.initial_state()) first")
        if tokens < 1:
            raise ValueError("tokens per step must be >= 1")
        core = getattr(mixer, "_core", mixer)
        tensors = list(state._tensors())
        device = tensors[0].device
        if device.type != "cuda":
            raise ValueError("DecodeGraph records a HIP graph: the state must live on the GPU")
        weight = core.proj_out.weight
        self.mixer = mixer
        self.batch, self.tokens = int(state.batch), int(tokens)
        self.fingerprint = state.fingerprint
        self.position = int(state.position)
        self.x = torch.zeros(self.batch, self.tokens, core.cfg.d_model, device=device, dtype=weight.dtype)
        self._state = state.clone()
        self._pos = torch.full((), self.position, dtype=torch.int64, device=device)
        # the storage every recorded launch reads (checked before each replay)
        self._tensors = [t for t in list(core.parameters()) + list(core.buffers())]
        self._ptrs = [t.data_ptr() for t in self._tensors]

        with torch.no_grad():
            # warm-up calls on a side stream set up library handles, plans and
            # workspaces (their results are discarded; the buffers are unchanged)
            side = torch.cuda.Stream(device=device)
            side.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(side), stream.positions_on_device(self._pos):
                for _ in range(max(1, warmup)):
                    mixer(self.x, state=self._state)
            torch.cuda.current_stream(device).wait_stream(side)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                # the scans update their state blocks in place; any other
                # carried row is copied back into its buffer
                with stream.positions_on_device(self._pos), stream.in_place_updates():
                    y, new = mixer(self.x, state=self._state)
                for dst, src in zip(self._state._tensors(), new._tensors()):
                    if dst.data_ptr() != src.data_ptr():
                        dst.copy_(src)
                self._pos.add_(self.tokens)
        self.y = y

    def step(self, x: torch.Tensor) -> torch.Tensor:
        """Advance every sequence by ``x`` [B, tokens, D]; returns the mixer
        output, a fixed buffer that the next step overwrites."""
        if tuple(x.shape) != tuple(self.x.shape):
            raise ValueError(f"this decode graph takes inputs of shape {tuple(self.x.shape)}; got {tuple(x.shape)}")
        for t, ptr in zip(self._tensors, self._ptrs):
            if t.data_ptr() != ptr:
                raise RuntimeError("a parameter of the mixer was replaced after this decode step was recorded "
                                   "(moved, cast or reassigned); record a new DecodeGraph")
        self.x.copy_(x)
        self.graph.replay()
        self.position += self.tokens
        return self.y

    def state(self) -> ThetaScanState:
        """An independent copy of the carried state after the steps so far."""
        snap = ThetaScanState(fingerprint=self.fingerprint, position=self.position, batch=self.batch,
                              carries=self._state.carries)
        return snap.clone()
