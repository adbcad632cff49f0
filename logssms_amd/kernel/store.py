"""``store_state`` (drop-in for the reference's
``python/logssms/kernel/store.py:69-83`` -> ``csrc/jit/store.cu:143-252``)."""

from __future__ import annotations

import torch

from .. import _lib


def store_state(pool: torch.Tensor, indices: torch.Tensor, states: torch.Tensor) -> None:
    """``pool[indices[i]] = states[i]`` for every ``indices[i] >= 0`` (a byte
    copy of whole rows; int32 or int64 indices)."""
    assert pool.device == states.device == indices.device
    assert pool.dtype == states.dtype
    num_slots = pool.shape[0]
    pool2 = pool.view(num_slots, -1)
    states2 = states.view(states.shape[0], -1)
    assert pool2.shape[1] == states2.shape[1]
    assert pool2.stride(1) == 1 and states2.stride(1) == 1
    row_bytes = pool2.shape[1] * pool2.element_size()
    assert row_bytes % 128 == 0
    assert indices.shape == (states2.shape[0],)
    if states2.shape[0] == 0:
        return
    _lib.call(
        "gdn_store_state",
        pool2.data_ptr(), pool2.stride(0) * pool2.element_size(), indices.data_ptr(), _lib.index_code(indices),
        states2.data_ptr(), states2.stride(0) * states2.element_size(), states2.shape[0], row_bytes,
        _lib.stream_of(pool2),
    )


__all__ = ["store_state"]
