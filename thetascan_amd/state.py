"""The persistent fast-memory state of a ThetaScan mixer (streaming).

``ThetaScan.forward(x)`` reads a fresh memory.  Passing a state continues one
causal sequence across calls::

    state = mixer.initial_state()
    with torch.no_grad():
        y1, state = mixer(x[:, :1000], state=state)
        y2, state = mixer(x[:, 1000:], state=state)     # == mixer(x)[:, 1000:]
        y3, state = mixer(x_next_token, state=state)     # one-token decode

The concatenated outputs equal the full-sequence call (to fp32 rounding: the
scans' tilings differ) for every family, temporal view, normalization and
expansion setting, and the chunk boundaries do not change causal results.
This is the persistent streaming state the reference lists as its largest
missing feature (ROADMAP.md:7-22); its semantics:

* contents: the number of tokens already seen (RoPE phases continue from
  it) and, per causal scan of the forward in call order, the fp32 state
  N = sum_i w_i k_i v_i^T [B,H,dk,dv] (with the key-mass column D = sum_i w_i
  k_i where the read normalizes; wide widths as blocks of at most 128
  columns), plus the fp32 last row of every decayed prefix (feature-mass
  reads).  ``nbytes`` is its memory cost; it does not grow with T.
* device and dtype: fp32 tensors on the mixer's device, whatever the
  activation dtype; ``to(device)`` moves them.
* autograd: continuation runs under ``torch.no_grad()``; the state holds no
  graph.  ``detach()`` and ``clone()`` return independent copies.
* reset: start again from ``initial_state()`` (or call without a state).
* serialization: ``state_dict()`` / ``ThetaScanState.from_state_dict`` (plain
  tensors; ``torch.save`` / ``torch.load(weights_only=True)`` round-trip it).
  A state is tied to the configuration that made it: its fingerprint is
  checked on use.
"""
from __future__ import annotations

import dataclasses
import hashlib
import json

import torch


def config_fingerprint(core_config) -> str:
    """Identity of the configuration a state belongs to."""
    fields = dataclasses.asdict(core_config)
    text = json.dumps(fields, sort_keys=True, default=str)
    return hashlib.sha256(text.encode("utf-8")).hexdigest()[:32]


@dataclasses.dataclass
class ThetaScanState:
    """Carried memory of one mixer after ``position`` tokens of a sequence."""

    fingerprint: str
    position: int = 0
    batch: int | None = None
    carries: tuple = ()

    # ---------------------------------------------------------------- info

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self._tensors())

    def _tensors(self):
        for c in self.carries:
            if isinstance(c, torch.Tensor):
                yield c
            else:
                yield from c

    # ---------------------------------------------------------------- copies

    def _map(self, fn) -> "ThetaScanState":
        carries = tuple(fn(c) if isinstance(c, torch.Tensor) else [fn(t) for t in c] for c in self.carries)
        return dataclasses.replace(self, carries=carries)

    def detach(self) -> "ThetaScanState":
        return self._map(lambda t: t.detach().clone())

    def clone(self) -> "ThetaScanState":
        return self._map(lambda t: t.clone())

    def to(self, device) -> "ThetaScanState":
        return self._map(lambda t: t.to(device))

    # ---------------------------------------------------------------- serialization

    def state_dict(self) -> dict:
        out = {"fingerprint": torch.tensor(list(self.fingerprint.encode("ascii")), dtype=torch.uint8),
               "position": torch.tensor(self.position, dtype=torch.int64),
               "batch": torch.tensor(-1 if self.batch is None else self.batch, dtype=torch.int64)}
        for i, c in enumerate(self.carries):
            if isinstance(c, torch.Tensor):
                out[f"carry.{i}"] = c
            else:
                for j, t in enumerate(c):
                    out[f"carry.{i}.{j}"] = t
        return out

    @classmethod
    def from_state_dict(cls, d: dict) -> "ThetaScanState":
        fingerprint = bytes(d["fingerprint"].tolist()).decode("ascii")
        batch = int(d["batch"])
        groups: dict = {}
        for key, t in d.items():
            if not key.startswith("carry."):
                continue
            parts = key.split(".")
            i = int(parts[1])
            if len(parts) == 2:
                groups[i] = t
            else:
                groups.setdefault(i, {})[int(parts[2])] = t
        carries = tuple(groups[i] if isinstance(groups[i], torch.Tensor)
                        else [groups[i][j] for j in sorted(groups[i])] for i in sorted(groups))
        return cls(fingerprint=fingerprint, position=int(d["position"]), batch=None if batch < 0 else batch,
                   carries=carries)
