"""Single-token conv update (drop-in for
``logssms.kernel.linear_attention.conv_decode``, reference file
``python/logssms/kernel/linear_attention/conv_decode.py``)."""

from __future__ import annotations

import torch

from ... import _lib
from .packed_conv import conv_input_scale_args


def conv_decode(
    mixed_qkv: torch.Tensor,
    weight: torch.Tensor,
    config,
    *,
    bias: torch.Tensor | None = None,
    split_qkv: bool = False,
    round_conv: bool = False,
    read_slots: torch.Tensor,
    write_slots: torch.Tensor,
    standard_state: torch.Tensor | None = None,
    pool=None,
    read_granules: torch.Tensor | None = None,
    write_granules: torch.Tensor | None = None,
    work_slots: torch.Tensor | None = None,
    input_boundaries: tuple[int, int] | None = None,
    input_scales: tuple[float, float, float] = (1.0, 1.0, 1.0),
):
    """conv_decode.py:293-352: ``y = SiLU(sum_j w_j [window, x]_j (+ b))``.

    Standard mode: the window is ``standard_state[read_slots, layer]`` and the
    shifted window ``[window[1:], x]`` goes to
    ``standard_state[write_slots, layer]`` (in place when equal).

    LogState mode (``pool``): the window is the conv snapshot of
    (``read_slots``, ``read_granules``) in the pool's frame storage
    (``pool.conv_frame_table``); the shifted window goes to (``write_slots``,
    ``write_granules``) and to granule 0 of ``work_slots``
    (``gdn_conv_decode_logstate``).

    Returns ``(q [B,1,H,dk], k, v [B,1,HV,dv])`` when ``split_qkv`` else
    ``y [B, C]``.
    """
    assert mixed_qkv.is_cuda and mixed_qkv.ndim == 2
    assert 1 <= config.state_len <= 5
    bs, channels = mixed_qkv.shape
    if pool is not None:
        return _conv_decode_logstate(mixed_qkv, weight, config, bias, split_qkv, round_conv, read_slots,
                                     write_slots, pool, read_granules, write_granules, work_slots,
                                     input_boundaries, input_scales)
    assert standard_state is not None
    assert channels == config.conv_dim
    assert read_slots.shape == write_slots.shape == (bs,)
    assert standard_state.stride(3) == 1 and standard_state.stride(2) == config.state_len
    if split_qkv:
        q = torch.empty((bs, 1, config.num_k_heads, config.head_k_dim),
                        dtype=mixed_qkv.dtype, device=mixed_qkv.device)
        k = torch.empty_like(q)
        v = torch.empty((bs, 1, config.num_v_heads, config.head_v_dim),
                        dtype=mixed_qkv.dtype, device=mixed_qkv.device)
    else:
        q = torch.empty((bs, channels), dtype=mixed_qkv.dtype, device=mixed_qkv.device)
        k = v = q
    if bs:
        weight = weight.contiguous()
        if bias is not None:
            bias = bias.to(mixed_qkv.dtype).contiguous()
        scale_args = conv_input_scale_args(channels, input_boundaries, input_scales)
        _lib.call(
            "gdn_conv_decode",
            mixed_qkv.data_ptr(), mixed_qkv.stride(0), mixed_qkv.stride(1), _lib.dtype_code(mixed_qkv.dtype),
            weight.data_ptr(), _lib.ptr(bias), config.state_len + 1, bs, channels,
            standard_state.data_ptr(), standard_state.stride(0), standard_state.stride(1), config.layer_idx,
            read_slots.data_ptr(), read_slots.stride(0), _lib.index_code(read_slots),
            write_slots.data_ptr(), write_slots.stride(0), _lib.index_code(write_slots),
            q.data_ptr(), k.data_ptr(), v.data_ptr(), config.key_dim if split_qkv else 0,
            int(split_qkv), int(round_conv), *scale_args, _lib.stream_of(mixed_qkv),
        )
    return (q, k, v) if split_qkv else q


def _outputs(mixed_qkv, config, split_qkv):
    bs, channels = mixed_qkv.shape
    if split_qkv:
        q = torch.empty((bs, 1, config.num_k_heads, config.head_k_dim), dtype=mixed_qkv.dtype,
                        device=mixed_qkv.device)
        k = torch.empty_like(q)
        v = torch.empty((bs, 1, config.num_v_heads, config.head_v_dim), dtype=mixed_qkv.dtype,
                        device=mixed_qkv.device)
        return q, k, v
    q = torch.empty((bs, channels), dtype=mixed_qkv.dtype, device=mixed_qkv.device)
    return q, q, q


def _conv_decode_logstate(mixed_qkv, weight, config, bias, split_qkv, round_conv, read_slots, write_slots, pool,
                          read_granules, write_granules, work_slots, input_boundaries, input_scales):
    """The LogState mode of ``conv_decode`` (``conv_decode.py:320-345``)."""
    assert read_granules is not None and write_granules is not None and work_slots is not None
    bs, channels = mixed_qkv.shape
    scale_args = conv_input_scale_args(channels, input_boundaries, input_scales)
    assert channels == config.conv_dim
    assert read_slots.shape == write_slots.shape == read_granules.shape == write_granules.shape == (bs,)
    assert work_slots.shape == (bs,)
    read_slots, write_slots, work_slots = read_slots.contiguous(), write_slots.contiguous(), work_slots.contiguous()
    read_granules, write_granules = read_granules.contiguous(), write_granules.contiguous()
    table = pool.conv_frame_table
    assert table.ndim == 3 and table.is_contiguous()
    q, k, v = _outputs(mixed_qkv, config, split_qkv)
    if bs:
        weight = weight.contiguous()
        if bias is not None:
            bias = bias.to(mixed_qkv.dtype).contiguous()
        storage = pool.storage
        assert storage.is_contiguous() and storage.device == mixed_qkv.device
        num_frames = storage.numel() * storage.element_size() // pool.frame_bytes
        _lib.call(
            "gdn_conv_decode_logstate",
            mixed_qkv.data_ptr(), mixed_qkv.stride(0), mixed_qkv.stride(1), _lib.dtype_code(mixed_qkv.dtype),
            weight.data_ptr(), _lib.ptr(bias), config.state_len + 1, bs, channels,
            storage.data_ptr(), table.data_ptr(), _lib.index_code(table), table.shape[0], table.shape[1],
            table.shape[2], pool.frame_bytes, num_frames, config.layer_idx,
            read_slots.data_ptr(), _lib.index_code(read_slots), read_granules.data_ptr(),
            _lib.index_code(read_granules), write_slots.data_ptr(), _lib.index_code(write_slots),
            write_granules.data_ptr(), _lib.index_code(write_granules), work_slots.data_ptr(),
            _lib.index_code(work_slots), q.data_ptr(), k.data_ptr(), v.data_ptr(),
            config.key_dim if split_qkv else 0, int(split_qkv), int(round_conv), *scale_args,
            _lib.stream_of(mixed_qkv),
        )
    return (q, k, v) if split_qkv else q


__all__ = ["conv_decode"]
