"""``GatedDeltaConfig`` (reference ``python/logssms/layers/gated_delta.py:15-31``)."""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class GatedDeltaConfig:
    num_k_heads: int
    num_v_heads: int
    head_k_dim: int
    head_v_dim: int
    conv_dim: int
    state_len: int
    layer_idx: int

    @property
    def key_dim(self) -> int:
        return self.num_k_heads * self.head_k_dim

    @property
    def value_dim(self) -> int:
        return self.num_v_heads * self.head_v_dim


__all__ = ["GatedDeltaConfig"]
