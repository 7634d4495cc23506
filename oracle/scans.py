"""CPU restatements of the reference scan backends (test infrastructure only).

Pinning (tests/test_oracle_golden.py, tests/test_oracle_closed_forms.py):
* ``naive``  -- golden vectors written from the reference (tests/golden),
  the constant-stream closed form (1 - a^(t+1)) / (1 - a), a hand-computed
  3-token case, and agreement with the independent ``quad`` formulation.
* ``quad``   -- golden vectors + agreement with ``naive`` (brute force).
* ``cumsum`` -- golden vectors + agreement with ``naive`` inside the CLAMP
  range and the documented clamp failure outside it.
* ``ema_cumsum`` / ``causal_prefix_sum`` -- closed forms and the unit-query
  scan identity (a discounted prefix equals a scan with q = k = 1).
"""
from __future__ import annotations

import torch

CLAMP = 60.0  # scan_cumsum.CLAMP (src/thetascan/_core/ops/scan_cumsum.py:4)


def linattn_naive(q, k, v, decay=None):
    """Sequential recurrence S_t = a_t S_{t-1} + k_t v_t^T, out_t = q_t S_t.

    Follows src/thetascan/_core/ops/scan_naive.py:5-18 (decay multiplies the
    state before the current token is added; scalar [B,H,T,1] or per-channel
    [B,H,T,Dk] log-decay).
    """
    B, H, T, Dk = k.shape
    Dv = v.shape[-1]
    S = q.new_zeros(B, H, Dk, Dv)
    if T == 0:
        return q.new_zeros(B, H, 0, Dv)
    # rows are collected and stacked once: in-place row writes would make
    # autograd's backward copy the whole output per step (O(T^2))
    rows = []
    for t in range(T):
        if decay is not None:
            S = S * decay[:, :, t].exp().unsqueeze(-1)
        S = S + k[:, :, t].unsqueeze(-1) * v[:, :, t].unsqueeze(-2)
        rows.append(torch.einsum("bhk,bhkv->bhv", q[:, :, t], S))
    return torch.stack(rows, dim=2)


def final_state_naive(k, v, decay=None):
    """State after the last token of the naive recurrence (scan_naive.py:10-16)."""
    B, H, T, Dk = k.shape
    S = k.new_zeros(B, H, Dk, v.shape[-1])
    for t in range(T):
        if decay is not None:
            S = S * decay[:, :, t].exp().unsqueeze(-1)
        S = S + k[:, :, t].unsqueeze(-1) * v[:, :, t].unsqueeze(-2)
    return S


def linattn_chunk(q, k, v, decay=None, chunk=64):
    """Tiled exact form of the recurrence (src/thetascan/_core/ops/scan_chunk.py:246-339).

    Tiles of ``min(chunk, T)`` tokens, the last one zero-padded
    (scan_chunk.py:158-167, 274-275).  Inside a tile the score block is
    weighted by exp(min(L_i - L_j, 0)) with L the tile-local cumulative log of
    ``decay`` (scan_chunk.py:122-155); across tiles the state entering tile n
    is S_n = S_{n-1} exp(L_last) + U_{n-1}, U = sum_j exp(L_last - L_j) k_j v_j^T
    (scan_chunk.py:170-212, 318-334); the entering state reaches position i
    with weight exp(L_i).  A static [H] retention is passed as its [B,H,T,1]
    stream (``as_stream``).  Same mathematics as ``linattn_naive`` with a cost
    linear in T, so the float64 oracle reaches long sequences; pinned against
    ``linattn_naive`` at 1e-12 for several chunks, retentions and ragged tiles
    (tests/test_oracle_closed_forms.py), as the reference pins its chunk
    backend (tests/test_scan_chunk.py:55-123).
    """
    B, H, T, Dk = q.shape
    Dv = v.shape[-1]
    if T == 0:
        return q.new_zeros(B, H, 0, Dv)
    if decay is not None and decay.shape[-1] != 1:
        raise NotImplementedError("chunk backend: scalar decay only (v1)")
    C = min(int(chunk), T)
    NT = -(-T // C)
    pad = NT * C - T

    def tiles(x):
        if pad:
            x = torch.cat([x, x.new_zeros(*x.shape[:2], pad, *x.shape[3:])], dim=2)
        return x.reshape(B, H, NT, C, x.shape[-1])

    qt, kt, vt = tiles(q), tiles(k), tiles(v)
    causal = torch.ones(C, C, dtype=torch.bool).tril()
    if decay is None:
        w = causal.to(q.dtype)
        key_w = close = enter = None
    else:
        L = tiles(decay.to(q.dtype)).squeeze(-1).cumsum(-1)        # [B,H,NT,C]
        w = (L.unsqueeze(-1) - L.unsqueeze(-2)).clamp(max=0.0).exp() * causal
        key_w = (L[..., -1:] - L).exp()                            # weight of key j leaving the tile
        close = L[..., -1].exp()                                   # whole-tile retention
        enter = L.exp()                                            # entering state at position i
    out = ((qt @ kt.transpose(-1, -2)) * w) @ vt                   # intra-tile part
    keys = kt if key_w is None else kt * key_w.unsqueeze(-1)
    U = keys.transpose(-1, -2) @ vt                                # [B,H,NT,Dk,Dv]
    S = q.new_zeros(B, H, Dk, Dv)
    states = []
    for n in range(NT):
        states.append(S)
        S = (S if close is None else S * close[:, :, n, None, None]) + U[:, :, n]
    cross = qt @ torch.stack(states, dim=2)
    out = out + (cross if enter is None else cross * enter.unsqueeze(-1))
    return out.reshape(B, H, NT * C, Dv)[:, :, :T]


def linattn_quad(q, k, v, decay=None):
    """Masked O(T^2) dual form (src/thetascan/_core/ops/scan_quad.py:5-16)."""
    T = q.shape[2]
    att = q @ k.transpose(-1, -2)
    if decay is not None:
        if decay.shape[-1] != 1:
            raise NotImplementedError("quad backend: scalar decay only (v1)")
        L = decay.squeeze(-1).cumsum(-1)
        att = att * (L.unsqueeze(-1) - L.unsqueeze(-2)).clamp(max=0.0).exp()
    mask = torch.ones(T, T, dtype=torch.bool).tril()
    return att.masked_fill(~mask, 0.0) @ v


def linattn_cumsum(q, k, v, decay=None):
    """Prefix-sum form over the materialised outer products.

    Follows src/thetascan/_core/ops/scan_cumsum.py:7-19 (CLAMP=60 guard on the
    cumulative log).  This is the CPU baseline algorithm.
    """
    if decay is None:
        S = (k.unsqueeze(-1) * v.unsqueeze(-2)).cumsum(2)
        return torch.einsum("bhtk,bhtkv->bhtv", q, S)
    if decay.shape[-1] != 1:
        raise NotImplementedError("cumsum backend: scalar decay only (v1)")
    L = decay.squeeze(-1).cumsum(-1)
    w = (-L).clamp(max=CLAMP).exp().unsqueeze(-1)
    S = ((k * w).unsqueeze(-1) * v.unsqueeze(-2)).cumsum(2)
    out = torch.einsum("bhtk,bhtkv->bhtv", q, S)
    return out * L.clamp(min=-CLAMP).exp().unsqueeze(-1)


def as_stream(log_alpha: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    """Widen a static [H] log-retention to [B,H,T,1] (interface.py:110-117)."""
    B, H, T = like.shape[:3]
    return log_alpha.to(like.dtype).view(1, H, 1, 1).expand(B, H, T, 1)


def linattn_views_naive(q, k, v, retentions):
    """Multi-view scan by separate naive scans (interface.py:178-182)."""
    return tuple(
        linattn_naive(q, k, v, None if r is None else (as_stream(r, q) if r.ndim == 1 else r))
        for r in retentions
    )


def causal_prefix_sum(x):
    """Plain prefix sum along T (src/thetascan/_core/ops/interface.py:96-107)."""
    return x.cumsum(2)


def ema_cumsum(x, log_alpha):
    """Discounted prefix z_t = sum_{i<=t} alpha^(t-i) x_i, static alpha[H].

    Restates src/thetascan/_core/ops/interface.py:58-93 as the direct sum
    (the reference's chunking changes rounding only).
    """
    B, H, T = x.shape[:3]
    la = log_alpha.to(x.dtype).view(1, H, 1, 1) if x.dim() == 4 else log_alpha.to(x.dtype).view(1, H, 1)
    if T == 0:
        return torch.zeros_like(x)
    z = torch.zeros_like(x[:, :, 0])
    alpha = la.exp().squeeze(2)
    rows = []
    for t in range(T):
        z = z * alpha + x[:, :, t]
        rows.append(z)
    return torch.stack(rows, dim=2)
