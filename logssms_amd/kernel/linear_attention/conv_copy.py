"""LogState conv snapshot copy (drop-in for
``python/logssms/kernel/linear_attention/conv_copy.py``)."""

from __future__ import annotations

import torch

from ... import _lib


def copy_conv_snapshots(pool, source_slots: torch.Tensor, source_granules: torch.Tensor,
                        output_slots: torch.Tensor, output_granules: torch.Tensor) -> None:
    """conv_copy.py:31-52: every layer's conv window of (``source_slots[i]``,
    ``source_granules[i]``) to (``output_slots[i]``, ``output_granules[i]``)
    through ``pool.conv_frame_table`` [slots, granules, frames per snapshot]
    (``gdn_logstate_copy_conv``).  Pairs with a negative slot are skipped."""
    count = source_slots.numel()
    assert source_granules.numel() == output_slots.numel() == output_granules.numel() == count
    if count == 0:
        return
    storage = pool.storage
    assert all(t.device == storage.device for t in (source_slots, source_granules, output_slots, output_granules))
    assert storage.is_contiguous()
    layout = pool.layout
    table = pool.conv_frame_table
    assert table.ndim == 3 and table.is_contiguous()
    snapshot_bytes = layout.num_linear_layers * layout.conv_dim * layout.state_len * pool.dtype.itemsize
    num_frames = storage.numel() * storage.element_size() // pool.frame_bytes
    src, sg = source_slots.contiguous(), source_granules.contiguous()
    dst, dg = output_slots.contiguous(), output_granules.contiguous()
    _lib.call(
        "gdn_logstate_copy_conv",
        storage.data_ptr(), table.data_ptr(), _lib.index_code(table), table.shape[0], table.shape[1],
        table.shape[2], pool.frame_bytes, num_frames, snapshot_bytes, src.data_ptr(), _lib.index_code(src),
        sg.data_ptr(), _lib.index_code(sg), dst.data_ptr(), _lib.index_code(dst), dg.data_ptr(),
        _lib.index_code(dg), count, _lib.stream_of(storage),
    )


__all__ = ["copy_conv_snapshots"]
