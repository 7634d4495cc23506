"""Continuation of one causal sequence across forward calls.

A mixer forward is a fixed sequence of causal scans and decayed prefixes
(every other operation is per token).  While a :class:`Carry` is active, each
of them starts from the state the same scan left at the end of the previous
call -- taken in call order -- and leaves its final state for the next one;
RoPE phases start at the number of tokens already seen.  The carries are the
fp32 scan states N = sum_i w_i k_i v_i^T (with the key-mass column where the
read normalizes) and the fp32 last rows of the decayed prefixes, i.e. exactly
what a recurrence S_t = a_t S_{t-1} + k_t v_t^T (scan_naive.py:5-18) keeps
between tokens.  Continuation runs without autograd.
"""
from __future__ import annotations

import contextlib
import contextvars

import torch

_ACTIVE: contextvars.ContextVar = contextvars.ContextVar("thetascan_carry", default=None)


class Carry:
    """The states one forward call consumes (``inp``, in call order; empty
    for a fresh sequence) and produces (``out``), and the position of its
    first token."""

    def __init__(self, carries=(), position: int = 0):
        self.inp = list(carries)
        self.out: list = []
        self.position = int(position)
        self.memo: dict = {}  # per-call values shared by the call's scans (RoPE rows)

    def take(self):
        """The state the next scan or prefix starts from (None: zero)."""
        i = len(self.out)
        return self.inp[i] if i < len(self.inp) else None

    def put(self, state) -> None:
        self.out.append(state)


def active() -> Carry | None:
    """The carry of the current call (None outside one, and in a traced
    forward: continuation is an eager, no-autograd mode)."""
    if torch.compiler.is_compiling():
        return None
    return _ACTIVE.get()


def position() -> int:
    """Absolute position of the current call's first token (0 outside a carry)."""
    carry = active()
    return 0 if carry is None else carry.position


_DEVICE_POSITION: contextvars.ContextVar = contextvars.ContextVar("thetascan_device_position", default=None)


def device_position() -> torch.Tensor | None:
    """The int64 device tensor holding the position of the current call's
    first token while a captured decode step is recorded (None otherwise):
    RoPE phases are then formed on the device from it, so one recorded step
    serves every position."""
    if active() is None:
        return None
    return _DEVICE_POSITION.get()


_IN_PLACE: contextvars.ContextVar = contextvars.ContextVar("thetascan_in_place", default=False)


def updates_in_place() -> bool:
    """Whether the current call's scans write their final states into the
    carried state tensors they start from (a captured decode step owns its
    state buffers; an ordinary call never mutates the state it is given)."""
    return active() is not None and _IN_PLACE.get()


@contextlib.contextmanager
def in_place_updates():
    token = _IN_PLACE.set(True)
    try:
        yield
    finally:
        _IN_PLACE.reset(token)


@contextlib.contextmanager
def positions_on_device(pos: torch.Tensor):
    token = _DEVICE_POSITION.set(pos)
    try:
        yield pos
    finally:
        _DEVICE_POSITION.reset(token)


@contextlib.contextmanager
def carrying(carry: Carry):
    if torch.is_grad_enabled():
        raise RuntimeError("streaming continuation runs without autograd: call it under torch.no_grad() "
                           "or torch.inference_mode()")
    token = _ACTIVE.set(carry)
    try:
        yield carry
    finally:
        _ACTIVE.reset(token)
