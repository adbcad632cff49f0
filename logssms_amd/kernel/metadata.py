"""``copy_metadata`` / ``pad_metadata`` (drop-ins for the reference's
``python/logssms/kernel/metadata.py:108-150``): one launch moves a group of
small index tensors (``gdn_metadata_copy`` / ``gdn_metadata_pad``,
``csrc/metadata.hip``).  CPU tensors take the same plain torch path as the
reference's host branch."""

from __future__ import annotations

import ctypes

import torch

from .. import _lib


def _ptrs(values):
    arr = (ctypes.c_void_p * len(values))(*values)
    return ctypes.cast(arr, ctypes.c_void_p), arr


def _i64(values):
    return (ctypes.c_int64 * len(values))(*[int(v) for v in values])


def _i32(values):
    arr = (ctypes.c_int * len(values))(*[int(v) for v in values])
    return ctypes.cast(arr, ctypes.c_void_p), arr


def copy_metadata(sources, outputs) -> None:
    """``outputs[i][:] = sources[i]`` for equally sized tensors; contiguous
    tensors or strided vectors (``metadata.py:108-134``)."""
    if not outputs or len(sources) != len(outputs):
        raise ValueError("metadata copies require equally sized nonempty source/output groups")
    counts = tuple(output.numel() for output in outputs)
    if any(source.numel() != count for source, count in zip(sources, counts)):
        raise ValueError("metadata copies require matching source/output tensor lengths")
    if max(counts) == 0:
        return
    if not outputs[0].is_cuda:
        for source, output in zip(sources, outputs, strict=True):
            output.copy_(source)
        return

    def stride(tensor):
        if tensor.is_contiguous():
            return 1
        if tensor.ndim == 1:
            return tensor.stride(0)
        raise ValueError("metadata copies require contiguous tensors or strided vectors")

    for src, dst in zip(sources, outputs):
        if src.dtype != dst.dtype or src.device != dst.device:
            raise ValueError("metadata copies require matching dtypes and devices")
    srcs, dsts = _ptrs([s.data_ptr() for s in sources]), _ptrs([d.data_ptr() for d in outputs])
    sizes = _i32([d.element_size() for d in outputs])
    _lib.call("gdn_metadata_copy", srcs[0], dsts[0], _i64(counts), _i64([stride(s) for s in sources]),
              _i64([stride(d) for d in outputs]), sizes[0], len(outputs), _lib.stream_of(outputs[0]))


def pad_metadata(sources, outputs, fills, chunk_tails) -> None:
    """``outputs[i][:len(sources[i])] = sources[i]``, the rest ``fills[i]``, or
    for a flattened pair table (``chunk_tails[i] >= 0``) the pairs
    ``(0, chunk_tails[i])`` (``metadata.py:137-150``)."""
    if not outputs:
        return
    if not outputs[0].is_cuda:
        for src, dst, fill, tail in zip(sources, outputs, fills, chunk_tails):
            dst.fill_(fill)
            if tail >= 0:
                dst[:, 1] = tail
            dst[:len(src)].copy_(src)
        return
    for src, dst in zip(sources, outputs):
        if src.dtype != dst.dtype or not src.is_contiguous() or not dst.is_contiguous():
            raise ValueError("metadata padding requires contiguous tensors of one dtype")
    srcs, dsts = _ptrs([s.data_ptr() for s in sources]), _ptrs([d.data_ptr() for d in outputs])
    sizes = _i32([d.element_size() for d in outputs])
    _lib.call("gdn_metadata_pad", srcs[0], dsts[0], _i64([s.numel() for s in sources]),
              _i64([d.numel() for d in outputs]), _i64(fills), _i64(chunk_tails), sizes[0], len(outputs),
              _lib.stream_of(outputs[0]))


__all__ = ["copy_metadata", "pad_metadata"]
