"""Rotary position tables and interleaved-pair rotation
(src/thetascan/_core/modules/rope.py:7-72).

Phases are formed in fp32 (fp64 for fp64 streams) so positions above the
bf16 integer range never alias, then cast once to the stream dtype.
"""
from __future__ import annotations

from functools import lru_cache

import torch


def _tables(T: int, rot_dim: int, base: float, device, dtype: torch.dtype, start: int = 0):
    phase_dtype = torch.float64 if dtype == torch.float64 else torch.float32
    inv = 1.0 / (base ** (torch.arange(0, rot_dim, 2, device=device, dtype=phase_dtype) / rot_dim))
    f = torch.outer(torch.arange(start, start + T, device=device, dtype=phase_dtype), inv)
    return f.cos().to(dtype=dtype), f.sin().to(dtype=dtype)


@lru_cache(maxsize=32)
def _rope_cache_cached(T: int, rot_dim: int, base: float, device_type: str, device_index, dtype: torch.dtype):
    device = torch.device(device_type) if device_index is None else torch.device(device_type, device_index)
    return _tables(T, rot_dim, base, device, dtype)


def rope_cache(T: int, rot_dim: int, base: float, device, dtype):
    """cos/sin of the current call's positions: 0 .. T-1, or, while a
    sequence is continued across calls, from the number of tokens seen."""
    from ..ops import stream

    start = stream.position()
    if start:
        return _tables(T, rot_dim, base, torch.device(device), dtype, start)
    resolved = torch.device(device)
    index = resolved.index
    if resolved.type == "cuda" and index is None:
        index = torch.cuda.current_device()
    return _rope_cache_cached(T, rot_dim, float(base), resolved.type, index, dtype)


def rotated_width(width: int, mode: str, frac: float) -> int:
    """Rotated channel count: all pairs for 'full', else max(2, floor(width*frac) to even)."""
    max_rot = width // 2 * 2
    if mode == "none" or max_rot == 0:
        return 0
    if mode == "full":
        return max_rot
    return min(max_rot, max(2, int(width * frac) // 2 * 2))


def apply_rope(x: torch.Tensor, mode: str, frac: float, base: float) -> torch.Tensor:
    """x [B,H,T,d]: rotate the first rot channels pairwise (2i, 2i+1)."""
    rot = rotated_width(x.shape[-1], mode, frac)
    if rot == 0:
        return x
    cos, sin = rope_cache(x.shape[2], rot, base, x.device, x.dtype)
    x1, x2 = x[..., :rot:2], x[..., 1:rot:2]
    out = torch.stack((x1 * cos - x2 * sin, x1 * sin + x2 * cos), dim=-1).flatten(-2)
    return torch.cat((out, x[..., rot:]), dim=-1)
