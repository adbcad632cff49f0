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
    prefill (``gdn_logstate_prefill_writes``)."""
    count = logs.numel()
    output = torch.empty((3, count), dtype=logs.dtype, device=logs.device)
    assert logs.is_cuda and offsets.device == plan.device == logs.device
    assert plan.dtype == torch.int32 and plan.is_contiguous() and plan.numel() >= 3 * count
    logs, offsets = logs.contiguous(), offsets.contiguous()
    _lib.call("gdn_logstate_prefill_writes", logs.data_ptr(), _lib.index_code(logs), offsets.data_ptr(),
              _lib.index_code(offsets), plan.data_ptr(), output.data_ptr(), count, granularity,
              _lib.stream_of(logs))
    return output.unbind(0)


def gather_linear_slots(indices, state_table: torch.Tensor, *, work_table: torch.Tensor | None = None,
                        out_loc: torch.Tensor | None = None, page_size: int = 1) -> torch.Tensor:
    """metadata.py:266-320: decode slots from the engine's prepared batch
    packet (``indices.table_ids``, ``indices.cached_lens``) in one launch
    (``gdn_gather_linear_slots``), with no host copy of the tables.

    Standard pool: int64 ``[count, 2]`` of (read, write) slots,
    ``state_table[row, cached - 1]`` (the row's last column for cached 0) and
    ``state_table[row, cached]``.  LogState (``work_table`` given): int32
    ``[4, count]`` of (work slot, log slot, ``out_loc mod page_size``, 0)."""
    tables, cached = indices.table_ids, indices.cached_lens
    count = tables.numel()
    assert cached.numel() == count and state_table.ndim == 2 and state_table.stride(1) == 1
    assert tables.is_cuda and cached.device == tables.device == state_table.device
    logstate = work_table is not None
    if logstate:
        assert out_loc is not None and out_loc.numel() >= count and page_size > 0
        assert work_table.ndim == 2 and work_table.device == state_table.device
        output = torch.empty((4, count), dtype=torch.int32, device=state_table.device)
    else:
        output = torch.empty((count, 2), dtype=torch.int64, device=state_table.device)
    if count == 0:
        return output
    tables, cached = tables.contiguous(), cached.contiguous()
    loc = out_loc.contiguous() if logstate else None
    _lib.call("gdn_gather_linear_slots", tables.data_ptr(), _lib.index_code(tables), cached.data_ptr(),
              _lib.index_code(cached), state_table.data_ptr(), _lib.index_code(state_table), state_table.shape[0],
              state_table.shape[1], state_table.stride(0), _lib.ptr(work_table),
              _lib.index_code(work_table) if logstate else 0, work_table.shape[0] if logstate else 0,
              work_table.stride(0) if logstate else 0, _lib.ptr(loc), _lib.index_code(loc) if logstate else 0,
              page_size, output.data_ptr(), count, _lib.stream_of(state_table))
    return output


__all__ = ["copy_metadata", "gather_linear_slots", "make_logstate_prefill_writes", "pad_metadata"]
