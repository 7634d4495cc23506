"""Public module (drop-in for src/thetascan/api.py:13-48)."""
from __future__ import annotations

from copy import deepcopy

import torch
import torch.nn as nn

from ._core.modules.block import ThetaScan as _CoreThetaScan
from .state import ThetaScanState
from .config import ThetaScanConfig


class ThetaScan(nn.Module):
    """A token mixer with the ``[batch, time, channels]`` contract, on MI355X."""

    def __init__(self, config: ThetaScanConfig):
        super().__init__()
        self.config = deepcopy(config)
        self.config.validate()
        self._core_config = self.config._to_core_config()
        self._core = _CoreThetaScan(self._core_config)
        if self.config.family == "kernel" and not self.config.kernel.feature_parameters_trainable:
            frozen = list(self._core.key_query_feature_parameters())
            for parameter in frozen:
                parameter.requires_grad_(False)
            if not frozen:
                raise RuntimeError("could not locate kernel feature parameters to freeze")

    def forward(self, x: torch.Tensor, state: ThetaScanState | None = None):
        """``y`` [B,T,D]; with ``state`` (see :mod:`thetascan_amd.state`) the
        causal sequence continues from it and ``(y, new_state)`` is returned."""
        if state is None:
            return self._core(x)
        return self._core(x, state)

    def initial_state(self) -> ThetaScanState:
        """The state of a sequence with no tokens yet."""
        return self._core.initial_state()

    def zero_output_projection_(self) -> "ThetaScan":
        nn.init.zeros_(self._core.proj_out.weight)
        return self

    def regularization_loss(self) -> torch.Tensor:
        return self._core.ortho_loss()
