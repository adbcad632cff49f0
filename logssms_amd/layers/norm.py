"""``RMSNormGated`` (reference ``python/logssms/layers/norm.py:42-53``): the
output norm ``GatedDeltaNet.output`` applies to the core output
(``python/logssms/layers/gated_delta.py:133-139``)."""

from __future__ import annotations

import torch

from ..kernel.norm import rms_norm_gated


class RMSNormGated:
    def __init__(self, size: int, eps: float) -> None:
        self.eps = eps
        self.weight = torch.ones(size, dtype=torch.float32)

    def forward(self, hidden_states: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        return rms_norm_gated(hidden_states, gate, self.weight, self.eps)


__all__ = ["RMSNormGated"]
