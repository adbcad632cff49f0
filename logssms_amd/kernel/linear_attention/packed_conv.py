"""Packed varlen causal conv1d (drop-in for
``logssms.kernel.linear_attention.packed_conv``, reference file
``python/logssms/kernel/linear_attention/packed_conv.py``)."""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ... import _lib


@dataclass(frozen=True)
class PackedConvStateIO:
    """packed_conv.py:11-20.  Standard slot mode only: ``granules``,
    ``frame_table`` and ``frame_bytes`` belong to the LogState cache and raise
    ``NotImplementedError`` when set."""

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
    if direct:
        if state_io.frame_table is not None or state_io.granules is not None:
            raise NotImplementedError("LogState conv frames are not supported by the MI355X backend")
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


__all__ = ["PackedConvStateIO", "packed_causal_conv1d"]
