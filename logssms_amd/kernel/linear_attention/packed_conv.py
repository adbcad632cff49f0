"""Packed varlen causal conv1d (drop-in for
``logssms.kernel.linear_attention.packed_conv``, reference file
``python/logssms/kernel/linear_attention/packed_conv.py``)."""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ... import _lib


@dataclass(frozen=True)
class PackedConvStateIO:
    """packed_conv.py:11-20.  Standard mode: ``storage [slots, layers, C,
    W-1]`` indexed by ``slots``.  LogState mode (``frame_table`` set): the
    windows go to the (slot, granule) conv snapshots of the frame storage
    ``[num_frames, frame_bytes / itemsize]`` in the io dtype, with
    ``frame_table [slots, granules, frames per snapshot]``."""

    storage: torch.Tensor
    slots: torch.Tensor
    granules: torch.Tensor | None = None
    final_slots: torch.Tensor | None = None
    frame_table: torch.Tensor | None = None
    frame_bytes: int = 0
    layer: int = 0


def conv_input_scale_args(channels, boundaries, scales):
    """packed_conv.py:33-38."""
    if boundaries is None:
        assert tuple(scales) == (1.0, 1.0, 1.0)
        boundaries = (channels, channels)
    assert len(scales) == 3 and 0 <= boundaries[0] <= boundaries[1] <= channels
    return (int(boundaries[0]), int(boundaries[1]), *[float(s) for s in scales])


def packed_causal_conv1d(
    x: torch.Tensor,
    weight: torch.Tensor,
    history: torch.Tensor,
    cu_seqlens: torch.Tensor,
    chunk_indices: torch.Tensor | None = None,
    bias: torch.Tensor | None = None,
    *,
    state_io: PackedConvStateIO | None = None,
    input_boundaries: tuple[int, int] | None = None,
    input_scales: tuple[float, float, float] = (1.0, 1.0, 1.0),
) -> torch.Tensor:
    """packed_conv.py:143-192: ``y = SiLU(round(sum_tap w x + b))`` per packed
    sequence, inputs before a sequence taken from ``history``; with
    ``state_io`` the raw window ``[x_{t-W+2}..x_t]`` goes to
    ``storage[slots[t], layer]`` for ``slots[t] >= 0`` (and to
    ``final_slots[n]`` for each sequence's last token).

    ``chunk_indices`` is accepted for signature compatibility; the kernel tiles
    packed tokens directly, so it is not read.
    """
    del chunk_indices
    total_tokens, channels = x.shape
    kernel_size = weight.shape[-1]
    state_len = kernel_size - 1
    assert history.shape == (len(cu_seqlens) - 1, channels, state_len)
    assert weight.shape == (channels, 1, kernel_size)
    direct = state_io is not None
    if direct and state_io.frame_table is not None:
        return _packed_conv_logstate(x, weight, history, cu_seqlens, bias, state_io, input_boundaries, input_scales)
    if direct:
        assert state_io.granules is None, "conv granules need a frame table"
        assert state_io.slots.shape == (total_tokens,)
        assert state_io.storage.dtype == x.dtype and state_io.storage.device == x.device
        assert state_io.storage.ndim == 4 and state_io.storage.shape[2:] == (channels, state_len)
        assert state_io.storage.stride(3) == 1 and state_io.storage.stride(2) == state_len
        if state_io.final_slots is not None:
            assert state_io.final_slots.shape == (len(cu_seqlens) - 1,)
    output = torch.empty((total_tokens, channels), device=x.device, dtype=x.dtype)
    if total_tokens == 0:
        return output
    history = history.to(x.dtype).contiguous()
    weight = weight.contiguous()
    if bias is not None:
        bias = bias.to(x.dtype).contiguous()
    scale_args = conv_input_scale_args(channels, input_boundaries, input_scales)
    storage = state_io.storage if direct else None
    final = state_io.final_slots if direct else None
    _lib.call(
        "gdn_packed_causal_conv1d",
        x.data_ptr(), x.stride(0), x.stride(1), _lib.dtype_code(x.dtype),
        weight.data_ptr(), _lib.ptr(bias), history.data_ptr(),
        cu_seqlens.data_ptr(), _lib.index_code(cu_seqlens), len(cu_seqlens) - 1,
        total_tokens, channels, kernel_size, output.data_ptr(),
        _lib.ptr(storage), storage.stride(0) if direct else 0, storage.stride(1) if direct else 0,
        state_io.layer if direct else 0,
        _lib.ptr(state_io.slots) if direct else None,
        _lib.index_code(state_io.slots) if direct else 0,
        _lib.ptr(final), _lib.index_code(final) if final is not None else 0,
        *scale_args, _lib.stream_of(x),
    )
    return output


def _packed_conv_logstate(x, weight, history, cu_seqlens, bias, state_io, input_boundaries, input_scales):
    """LogState mode of ``packed_causal_conv1d`` (``packed_conv.py:160-189``):
    the conv itself, then the windows through the conv frame table."""
    output = packed_causal_conv1d(x, weight, history, cu_seqlens, None, bias, input_boundaries=input_boundaries,
                                  input_scales=input_scales)
    conv_windows_logstate(x, history, cu_seqlens, state_io, weight.shape[-1], input_boundaries, input_scales)
    return output


def conv_windows_logstate(x, history, cu_seqlens, state_io: PackedConvStateIO, kernel_size: int,
                          input_boundaries=None, input_scales=(1.0, 1.0, 1.0)) -> None:
    """The state writes of ``packed_causal_conv1d`` with a LogState
    ``state_io`` (``packed_conv.py:75-133`` with LOGSTATE): the raw window
    ending at each packed row t (inputs scaled as the conv reads them, rows
    before a sequence from ``history``) to the conv snapshot
    (``slots[t]``, ``granules[t]``) when that slot is >= 0, and each sequence's
    last window to granule 0 of ``final_slots`` (``gdn_conv_windows_logstate``)."""
    total_tokens, channels = x.shape
    scale_args = conv_input_scale_args(channels, input_boundaries, input_scales)
    table = state_io.frame_table
    assert history.shape == (len(cu_seqlens) - 1, channels, kernel_size - 1)
    assert state_io.granules is not None and state_io.granules.shape == (total_tokens,)
    assert state_io.slots.shape == (total_tokens,)
    assert state_io.frame_bytes % x.element_size() == 0
    assert table.ndim == 3 and table.is_contiguous()
    storage = state_io.storage
    assert storage.dtype == x.dtype and storage.device == x.device and storage.is_contiguous()
    if state_io.final_slots is not None:
        assert state_io.final_slots.shape == (len(cu_seqlens) - 1,)
    if total_tokens == 0:
        return
    history = history.to(x.dtype).contiguous()
    slots, granules = state_io.slots.contiguous(), state_io.granules.contiguous()
    final = state_io.final_slots.contiguous() if state_io.final_slots is not None else None
    num_frames = storage.numel() * storage.element_size() // state_io.frame_bytes
    _lib.call(
        "gdn_conv_windows_logstate",
        x.data_ptr(), x.stride(0), x.stride(1), _lib.dtype_code(x.dtype), history.data_ptr(),
        cu_seqlens.data_ptr(), _lib.index_code(cu_seqlens), len(cu_seqlens) - 1, total_tokens, channels,
        kernel_size, storage.data_ptr(), table.data_ptr(), _lib.index_code(table), table.shape[0], table.shape[1],
        table.shape[2], state_io.frame_bytes, num_frames, state_io.layer, slots.data_ptr(), _lib.index_code(slots),
        granules.data_ptr(), _lib.index_code(granules), _lib.ptr(final),
        _lib.index_code(final) if final is not None else 0, *scale_args, _lib.stream_of(x),
    )


__all__ = ["PackedConvStateIO", "conv_windows_logstate", "packed_causal_conv1d"]
