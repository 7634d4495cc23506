"""Rotary position tables and interleaved-pair rotation
(src/thetascan/_core/modules/rope.py:7-72).

Phases are formed in fp32 (fp64 for fp64 streams) so positions above the
bf16 integer range never alias, then cast once to the stream dtype.
"""
from __future__ import annotations

from functools import lru_cache

import torch

# Tables of captured decode steps, keyed by shape, base, device and dtype
_DEVICE_TABLES: dict = {}


def _tables(T: int, rot_dim: int, base: float, device, dtype: torch.dtype, start=0):
    """cos/sin [T, rot_dim/2] of positions start .. start+T-1; ``start`` may
    be an int64 device tensor (a captured decode step)."""
    phase_dtype = torch.float64 if dtype == torch.float64 else torch.float32
    if isinstance(start, torch.Tensor):
        # a captured step: frequencies and offsets kept for the life of the
        # process (the graph reads them in place), the positions in one launch
        # (integers below 2^24 are exact in fp32: the values of
        # (start + arange(T)) converted)
        key = (T, rot_dim, float(base), str(device), phase_dtype)
        hit = _DEVICE_TABLES.get(key)
        if hit is None:
            hit = _DEVICE_TABLES[key] = (
                1.0 / (base ** (torch.arange(0, rot_dim, 2, device=device, dtype=phase_dtype) / rot_dim)),
                torch.arange(T, device=device, dtype=phase_dtype))
        inv, offsets = hit
        f = torch.outer(offsets + start, inv)
        return f.cos().to(dtype=dtype), f.sin().to(dtype=dtype)
    inv = 1.0 / (base ** (torch.arange(0, rot_dim, 2, device=device, dtype=phase_dtype) / rot_dim))
    pos = torch.arange(start, start + T, device=device, dtype=phase_dtype)
    f = torch.outer(pos, inv)
    return f.cos().to(dtype=dtype), f.sin().to(dtype=dtype)


@lru_cache(maxsize=32)
def _rope_cache_cached(T: int, rot_dim: int, base: float, device_type: str, device_index, dtype: torch.dtype):
    device = torch.device(device_type) if device_index is None else torch.device(device_type, device_index)
    return _tables(T, rot_dim, base, device, dtype)


POSITION_BLOCK = 1024


@lru_cache(maxsize=32)
def _rope_block_cached(start: int, rot_dim: int, base: float, device_type: str, device_index, dtype: torch.dtype):
    device = torch.device(device_type) if device_index is None else torch.device(device_type, device_index)
    return _tables(POSITION_BLOCK, rot_dim, base, device, dtype, start)


def rope_cache(T: int, rot_dim: int, base: float, device, dtype):
    """cos/sin of the current call's positions: 0 .. T-1, or, while a
    sequence is continued across calls, from the number of tokens seen."""
    from ..ops import stream

    dev_pos = stream.device_position()
    if dev_pos is not None:
        # a captured decode step: rows formed on the device once per call
        memo = stream.active().memo
        key = ("rope", T, rot_dim, float(base), str(device), dtype)
        if key not in memo:
            memo[key] = _tables(T, rot_dim, base, torch.device(device), dtype, dev_pos)
        return memo[key]
    start = stream.position()
    resolved = torch.device(device)
    index = resolved.index
    if resolved.type == "cuda" and index is None:
        index = torch.cuda.current_device()
    if start:
        # rows of a cached block of positions (bit-equal to forming them
        # directly while positions are exact fp32 integers, below 2^24)
        b0 = start - start % POSITION_BLOCK
        if start + T > b0 + POSITION_BLOCK or b0 + POSITION_BLOCK > 1 << 24:
            return _tables(T, rot_dim, base, resolved, dtype, start)
        cos, sin = _rope_block_cached(b0, rot_dim, float(base), resolved.type, index, dtype)
        return cos[start - b0:start - b0 + T], sin[start - b0:start - b0 + T]
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
