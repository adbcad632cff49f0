"""State-pool descriptors of the chunked prefill (reference
``python/logssms/kernel/linear_attention/state_io.py:15-39``)."""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class ChunkStateIO:
    """state_io.py:15-28.  ``storage`` is ``[slots, layers, HV, dk, dv]``
    (any slot/layer/head strides, inner dims contiguous), or, with
    ``payload_frames`` set (the LogState layout), the frame storage
    ``[num_frames, frame_bytes / itemsize]`` in the state dtype: head h of
    layer ``layer`` in slot s starts at logical byte ``(layer HV + h)
    head_payload_bytes`` of the slot, and logical byte x lies in frame
    ``payload_frames[s, x // frame_bytes]`` at offset ``x % frame_bytes``
    (``layout.py:11-26``)."""

    storage: torch.Tensor
    read_slots: torch.Tensor
    chunk_write_slots: torch.Tensor
    final_write_slots: torch.Tensor | None = None
    payload_frames: torch.Tensor | None = None
    frame_bytes: int = 0
    head_payload_bytes: int = 0
    layer: int = 0
    num_layers: int = 1
    granularity: int = 64
    page_size: int = 64


@dataclass(frozen=True)
class ChunkLogIO:
    """state_io.py:31-39: the LogState token log.  ``slots`` / ``token_offsets``
    [T] give each token's log slot (-1: none) and position in its page;
    ``gate`` [1, T, HV] is the prepared (natural-log) gate; ``decay_frames``
    [slots, 2] the {frame, record} of each slot's decay record of
    ``decay_record_bytes``; ``num_key_heads`` the key heads the log keeps."""

    slots: torch.Tensor
    token_offsets: torch.Tensor
    decay_frames: torch.Tensor
    gate: torch.Tensor
    page_size: int
    decay_record_bytes: int
    num_key_heads: int


__all__ = ["ChunkStateIO", "ChunkLogIO"]
