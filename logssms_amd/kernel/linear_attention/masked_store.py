"""LogState snapshot stores that skip inactive (negative) slots (drop-in for
``python/logssms/kernel/linear_attention/masked_store.py``)."""

from __future__ import annotations

import torch

from ... import _lib


def _frames(pool):
    storage = pool.storage
    assert storage.is_contiguous()
    return storage, storage.numel() * storage.element_size() // pool.frame_bytes


def store_states(pool, slots: torch.Tensor, layer: int, values: torch.Tensor) -> None:
    """masked_store.py:45-55: ``values[i]`` ([HV, dk, dv], converted to the
    pool dtype) to the state heads of layer ``layer`` of ``slots[i]``
    (``gdn_logstate_store_states``); rows with ``slots[i] < 0`` are skipped."""
    assert slots.is_cuda and values.is_cuda
    if not len(slots):
        return
    storage, num_frames = _frames(pool)
    layout = pool.layout
    HV = layout.num_value_heads
    width = layout.head_k_dim * layout.head_v_dim
    values = values.to(pool.dtype).reshape(len(slots), HV, width).contiguous()
    slots = slots.contiguous()
    table = pool.payload_frame_table.contiguous()
    _lib.call(
        "gdn_logstate_store_states",
        storage.data_ptr(), table.data_ptr(), _lib.index_code(table), table.shape[0], table.shape[1],
        pool.frame_bytes, pool.head_payload_bytes, num_frames, slots.data_ptr(), _lib.index_code(slots), len(slots),
        layer, HV, width * pool.dtype.itemsize, values.data_ptr(), _lib.stream_of(storage),
    )


def store_conv(pool, slots: torch.Tensor, granules: torch.Tensor, layer: int, values: torch.Tensor) -> None:
    """masked_store.py:58-72: ``values[i]`` ([conv_dim, state_len], converted
    to the pool dtype) to layer ``layer`` of the (``slots[i]``,
    ``granules[i]``) conv snapshot (``gdn_logstate_store_conv``); rows with
    ``slots[i] < 0`` are skipped."""
    assert slots.is_cuda and granules.is_cuda and values.is_cuda
    assert granules.shape == slots.shape
    if not len(slots):
        return
    storage, num_frames = _frames(pool)
    layout = pool.layout
    width = layout.conv_dim * layout.state_len
    values = values.to(pool.dtype).reshape(len(slots), width).contiguous()
    slots, granules = slots.contiguous(), granules.contiguous()
    table = pool.conv_frame_table
    assert table.ndim == 3 and table.is_contiguous()
    _lib.call(
        "gdn_logstate_store_conv",
        storage.data_ptr(), table.data_ptr(), _lib.index_code(table), table.shape[0], table.shape[1], table.shape[2],
        pool.frame_bytes, num_frames, slots.data_ptr(), _lib.index_code(slots), granules.data_ptr(),
        _lib.index_code(granules), len(slots), layer, width * pool.dtype.itemsize, values.data_ptr(),
        _lib.stream_of(storage),
    )


__all__ = ["store_conv", "store_states"]
