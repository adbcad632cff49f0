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
    """conv_decode.py:293-352 (standard-state mode):
    ``y = SiLU(sum_j w_j [window, x]_j (+ b))`` from
    ``standard_state[read_slots, layer]``; the shifted window
    ``[window[1:], x]`` is written to ``standard_state[write_slots, layer]``
    (in place when equal).  ``pool``/granules/``work_slots`` are the LogState
    mode and raise ``NotImplementedError``.

    Returns ``(q [B,1,H,dk], k, v [B,1,HV,dv])`` when ``split_qkv`` else
    ``y [B, C]``.
    """
    assert mixed_qkv.is_cuda and mixed_qkv.ndim == 2
    assert 1 <= config.state_len <= 5
    if pool is not None or read_granules is not None or write_granules is not None or work_slots is not None:
        raise NotImplementedError("LogState conv pools are not supported by the MI355X backend")
    assert standard_state is not None
    bs, channels = mixed_qkv.shape
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


__all__ = ["conv_decode"]
