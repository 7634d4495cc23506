"""HIP entry points as autograd nodes, for eager callers and for torch.compile.

Each HIP operation of the mixer is a pair (forward, backward) of Python
functions that launch the kernels through ctypes.  :class:`HipOp` exposes such
a pair two ways:

* as a ``torch.library`` custom op ``thetascan_hip::<name>`` with a fake
  (shape-only) implementation and an autograd formula whose backward is the
  custom op ``thetascan_hip::<name>_backward``.  TorchDynamo records each as one
  opaque call, so a compiled mixer traces to one graph (the ctypes launches
  never enter it);
* as a ``torch.autograd.Function`` for eager execution.  The custom-op
  dispatcher costs about 0.1 ms of host time per forward and backward, which
  a GPU-bound training step would otherwise pay per operation.

Where autograd records nothing (grad mode off, or no input that requires
grad) the forward function runs alone, with no node around it.  All paths run
the same forward and backward functions, so their results are bit-identical.  ``setup`` and ``backward`` follow the ``register_autograd``
convention (``setup(ctx, inputs, output)``; ``backward(ctx, grads, bwd)``
returns one gradient per input, a list for a list input), where ``bwd`` is
the backward custom op under compilation and the plain backward function in
eager mode.  Outputs that receive no gradient arrive as None in both modes.
"""
from __future__ import annotations

import threading

import torch

_EAGER = threading.local()


def eager_forward() -> bool:
    """True inside a forward that the eager autograd.Function runs (its setup
    follows on the same thread), False under the custom-op dispatcher."""
    return getattr(_EAGER, "active", False)


def _tensor_slots(args):
    """(argument index, list index or None) of every tensor in ``args``."""
    slots = []
    for i, a in enumerate(args):
        if isinstance(a, torch.Tensor):
            slots.append((i, None))
        elif isinstance(a, (list, tuple)):
            slots.extend((i, j) for j, t in enumerate(a) if isinstance(t, torch.Tensor))
    return slots


class _Eager(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hip_op, args, *tensors):
        ctx.set_materialize_grads(False)
        _EAGER.active = True
        try:
            out = hip_op.forward(*args)
        finally:
            _EAGER.active = False
        hip_op.setup(ctx, args, out)
        ctx.hip_op = hip_op
        ctx.slots = _tensor_slots(args)
        ctx.multi = isinstance(out, (list, tuple))
        return tuple(out) if ctx.multi else out

    @staticmethod
    def backward(ctx, *grads):
        hip_op = ctx.hip_op
        res = hip_op.backward(ctx, list(grads) if ctx.multi else grads[0], hip_op.backward_impl)
        flat = []
        for i, j in ctx.slots:
            g = res[i]
            flat.append(g if j is None else (None if g is None else g[j]))
        return (None, None, *flat)


class HipOp:
    """One HIP operation with its backward (see the module docstring)."""

    def __init__(self, name: str, *, forward, forward_fake, backward_impl, backward_fake, setup, backward):
        self.name = name
        self.forward, self.backward_impl = forward, backward_impl
        self.setup, self.backward = setup, backward
        self.op = torch.library.custom_op(f"thetascan_hip::{name}", forward, mutates_args=())
        self.op.register_fake(forward_fake)
        self.bwd_op = torch.library.custom_op(f"thetascan_hip::{name}_backward", backward_impl, mutates_args=())
        self.bwd_op.register_fake(backward_fake)
        self.op.register_autograd(lambda ctx, grads: backward(ctx, grads, self.bwd_op), setup_context=setup)

    def __call__(self, *args):
        if torch.compiler.is_compiling():
            return self.op(*args)
        tensors = [args[i] if j is None else args[i][j] for i, j in _tensor_slots(args)]
        if not torch.is_grad_enabled() or not any(t.requires_grad for t in tensors):
            # nothing to record (inference, streaming continuation): the
            # forward alone, without an autograd node around it
            return self.forward(*args)
        out = _Eager.apply(self, args, *tensors)
        return list(out) if isinstance(out, tuple) else out
