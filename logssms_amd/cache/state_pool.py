"""``LinearStatePool`` (reference ``python/logssms/cache/radix/state_pool.py:12-41``).

Layout (same as the reference, so the slot tables and kernels index it the
same way): ``conv_state[slot, layer, conv_dim, W-1]`` in the model dtype and
``recurrent_state[slot, layer, HV, dk, dv]``.  The reference keeps both in the
model dtype; here the recurrent state defaults to fp32 (the carried state of
the chunked prefill and the decode updates is fp32 either way, and an fp32
pool keeps it so between launches).  Pass ``state_dtype=dtype`` for the
reference's single-dtype pool.
"""

from __future__ import annotations

import torch


class LinearStatePool:
    def __init__(self, num_slots: int, num_linear_layers: int, conv_dim: int, kernel_size: int,
                 num_v_heads: int, head_k_dim: int, head_v_dim: int, device: torch.device,
                 dtype: torch.dtype, state_dtype: torch.dtype | None = torch.float32) -> None:
        self.conv_state = torch.zeros(num_slots, num_linear_layers, conv_dim, kernel_size - 1,
                                      device=device, dtype=dtype)
        self.recurrent_state = torch.zeros(num_slots, num_linear_layers, num_v_heads, head_k_dim, head_v_dim,
                                           device=device, dtype=state_dtype or dtype)
        self._device = torch.device(device)
        self._dtype = dtype

    @property
    def device(self) -> torch.device:
        return self._device

    @property
    def dtype(self) -> torch.dtype:
        return self._dtype


__all__ = ["LinearStatePool"]
