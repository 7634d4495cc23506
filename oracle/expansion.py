"""Fixed random-feature expansion maps (test infrastructure only).

Restates the SHAKE256 sign maps of src/thetascan/_core/modules/block.py:49-133
with the standard library's ``hashlib``.  Pinned by golden vectors
(tests/golden/features.npz: row maps and the 40-byte checkpoint fingerprint)
and by the +-1/sqrt(width) magnitude closed form.
"""
from __future__ import annotations

import hashlib
import math

import torch

DOMAIN = "thetascan-expansion-v1"
MAGIC = b"TSXF"
SCHEMA = 1


def domain(shape, key: str, role: str) -> bytes:
    """block.py:67-74"""
    return f"{DOMAIN}\0{key}\0{role}\0{','.join(str(x) for x in shape)}".encode("utf-8")


def rademacher(shape, key: str, role: str) -> torch.Tensor:
    """Low bit of each SHAKE256 output byte -> +-1 (block.py:49-64)."""
    count = math.prod(shape)
    raw = hashlib.shake_256(domain(shape, key, role)).digest(count)
    bits = torch.tensor(list(raw), dtype=torch.int64) & 1
    return (bits.to(torch.float32) * 2.0 - 1.0).reshape(shape)


def row_map(shape, key: str, role: str, row_norm: float = 1.0) -> torch.Tensor:
    """Uncentred unit-norm rows, computed in float32 (block.py:117-133)."""
    matrix = rademacher(shape, key, role)
    norm = matrix.norm(dim=-1, keepdim=True)
    fallback = rademacher(shape, key, f"{role}-fallback")
    matrix = torch.where(norm > 0.0, matrix, fallback)
    return matrix * (float(row_norm) / matrix.norm(dim=-1, keepdim=True))


def fingerprint(key: str, effective_hidden: int, feature_expansion: int, depth: int) -> bytes:
    """40-byte checkpoint identity ``TSXF || u32 schema || sha256`` (block.py:77-114)."""
    base = effective_hidden // feature_expansion
    digest = hashlib.sha256()
    digest.update(b"thetascan-expansion-checkpoint\0")
    digest.update(DOMAIN.encode("ascii"))
    for layer in range(depth):
        for desc in (
            domain((1, effective_hidden, base), key, f"w1-expand-layer-{layer}"),
            domain((1, base, effective_hidden), key, f"w2-expand-layer-{layer}"),
        ):
            digest.update(len(desc).to_bytes(8, "big"))
            digest.update(desc)
    return MAGIC + SCHEMA.to_bytes(4, "big") + digest.digest()
