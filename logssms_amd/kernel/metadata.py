"""``copy_metadata`` / ``pad_metadata``: the interface of the reference's
``python/logssms/kernel/metadata.py:108-150`` (same arguments, results and
``ValueError`` conditions).  On the device a whole group of small index
tensors moves in one launch (``gdn_metadata_copy`` / ``gdn_metadata_pad``,
``csrc/metadata.hip``): the per-field pointers, lengths and strides travel as
a kernel argument table.  Host tensors take plain torch copies."""

from __future__ import annotations

import ctypes

import torch

from .. import _lib


def _table(ctype, values):
    """A ctypes array of ``values`` and a pointer to it (keep both alive)."""
    arr = (ctype * len(values))(*values)
    return ctypes.cast(arr, ctypes.c_void_p), arr


def _element_stride(t: torch.Tensor) -> int:
    """Stride of a tensor read as a flat vector: 1 when contiguous, its own
    stride when it is 1-D; anything else cannot be read that way."""
    if t.is_contiguous():
        return 1
    if t.ndim == 1:
        return t.stride(0)
    raise ValueError("metadata copies require contiguous tensors or strided vectors")


def copy_metadata(sources, outputs) -> None:
    """``outputs[i][...] = sources[i]`` for each pair of equally long tensors
    (contiguous, or vectors of any stride)."""
    pairs = list(zip(sources, outputs))
    if not outputs or len(pairs) != len(sources) or len(pairs) != len(outputs):
        raise ValueError("metadata copies require equally sized nonempty source/output groups")
    lengths = [dst.numel() for dst in outputs]
    if any(src.numel() != n for (src, _), n in zip(pairs, lengths)):
        raise ValueError("metadata copies require matching source/output tensor lengths")
    if not any(lengths):
        return
    if not outputs[0].is_cuda:
        for src, dst in pairs:
            dst.copy_(src)
        return
    src_strides = [_element_stride(src) for src, _ in pairs]
    dst_strides = [_element_stride(dst) for _, dst in pairs]
    if any(src.dtype != dst.dtype or src.device != dst.device for src, dst in pairs):
        raise ValueError("metadata copies require matching dtypes and devices")
    src_ptrs = _table(ctypes.c_void_p, [src.data_ptr() for src, _ in pairs])
    dst_ptrs = _table(ctypes.c_void_p, [dst.data_ptr() for _, dst in pairs])
    sizes = _table(ctypes.c_int, [dst.element_size() for _, dst in pairs])
    _lib.call("gdn_metadata_copy", src_ptrs[0], dst_ptrs[0], _lib.i64_array(lengths), _lib.i64_array(src_strides),
              _lib.i64_array(dst_strides), sizes[0], len(pairs), _lib.stream_of(outputs[0]))


def pad_metadata(sources, outputs, fills, chunk_tails) -> None:
    """``outputs[i][:len(sources[i])] = sources[i]``; the rows after it get
    ``fills[i]``, or, for a flattened (request, chunk) pair table
    (``chunk_tails[i] >= 0``), the pair ``(0, chunk_tails[i])``."""
    if not outputs:
        return
    jobs = list(zip(sources, outputs, fills, chunk_tails))
    if not outputs[0].is_cuda:
        for src, dst, fill, tail in jobs:
            if tail >= 0:
                dst.view(-1, 2).copy_(torch.tensor([0, tail], dtype=dst.dtype))
            else:
                dst.fill_(fill)
            dst[:src.shape[0]] = src
        return
    if any(src.dtype != dst.dtype or not (src.is_contiguous() and dst.is_contiguous()) for src, dst, _, _ in jobs):
        raise ValueError("metadata padding requires contiguous tensors of one dtype")
    src_ptrs = _table(ctypes.c_void_p, [src.data_ptr() for src, _, _, _ in jobs])
    dst_ptrs = _table(ctypes.c_void_p, [dst.data_ptr() for _, dst, _, _ in jobs])
    sizes = _table(ctypes.c_int, [dst.element_size() for _, dst, _, _ in jobs])
    _lib.call("gdn_metadata_pad", src_ptrs[0], dst_ptrs[0], _lib.i64_array([src.numel() for src, _, _, _ in jobs]),
              _lib.i64_array([dst.numel() for _, dst, _, _ in jobs]), _lib.i64_array([f for _, _, f, _ in jobs]),
              _lib.i64_array([t for _, _, _, t in jobs]), sizes[0], len(jobs), _lib.stream_of(outputs[0]))


def make_logstate_prefill_writes(logs: torch.Tensor, offsets: torch.Tensor, plan: torch.Tensor, granularity: int):
    """metadata.py:150-178: from the per-token log slots ``logs``, page
    offsets ``offsets`` and the int32 host plan ``[conv slot | conv granule |
    log enabled]`` (conv slot -2: the token's own log slot), the
    ``(log write slots, conv token slots, conv token granules)`` of a LogState
    prefill (``gdn_logstate_prefill_writes`` on the device; host tensors take
    the same torch expressions)."""
    count = logs.numel()
    output = torch.empty((3, count), dtype=logs.dtype, device=logs.device)
    if not logs.is_cuda:
        conv, granules, enabled = plan[:3 * count].view(3, count)
        output[0] = torch.where(enabled != 0, logs, -1)
        output[1] = torch.where(conv == -2, logs, conv)
        output[2] = torch.where(conv == -2, offsets // granularity, granules)
        return output.unbind(0)
    assert plan.dtype == torch.int32 and plan.is_contiguous() and plan.numel() >= 3 * count
    logs, offsets = logs.contiguous(), offsets.contiguous()
    _lib.call("gdn_logstate_prefill_writes", logs.data_ptr(), _lib.index_code(logs), offsets.data_ptr(),
              _lib.index_code(offsets), plan.data_ptr(), output.data_ptr(), count, granularity,
              _lib.stream_of(logs))
    return output.unbind(0)


__all__ = ["copy_metadata", "make_logstate_prefill_writes", "pad_metadata"]
