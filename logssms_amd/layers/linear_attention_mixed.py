"""Fixed-capacity metadata for mixed prefill/decode graph buckets (reference
``python/logssms/layers/linear_attention_backend/mixed.py:1-197``).

Ordinary metadata is prepared with the actual token lengths first and then
normalised outside capture: the per-chunk and per-token tables are padded to
the bucket's capacity (padded chunk pairs point past the packed tokens,
padded write slots are -1, so padded entries write nothing), decode slots
become int64.  ``MixedLinearCopyPlan`` then copies fresh metadata into the
tensors a graph captured, after checking that nothing but tensor contents
changed.  No device tensor is read on the host.  Only the standard
(radix-pool) metadata is handled; the LogState variant is not part of this
build."""

from __future__ import annotations

from dataclasses import fields, is_dataclass, replace

import torch

from ..kernel.metadata import copy_metadata, pad_metadata
from .linear_attention_backend import LinearAttnMetadata, PackedLinearIndices


class _MetadataPadding:
    """Collects (source, padded output, fill, pair tail) and pads them all in
    one launch (``mixed.py:23-38``)."""

    def __init__(self):
        self.copies = []

    def __call__(self, tensor, capacity, value=0, *, chunk_tail=-1):
        if tensor.shape[0] > capacity:
            raise ValueError("metadata exceeds mixed graph capacity")
        output = tensor.new_empty((capacity, *tensor.shape[1:]))
        self.copies.append((tensor.contiguous(), output, value, chunk_tail))
        return output

    def finish(self):
        if self.copies:
            sources, outputs, fills, tails = zip(*self.copies)
            pad_metadata(sources, outputs, fills, tails)


def _packed_pad(indices: PackedLinearIndices, capacity: int, requests: int, chunk_size: int,
                pad: _MetadataPadding) -> PackedLinearIndices:
    """``mixed.py:41-56``: the most chunks positive lengths summing to
    ``capacity`` can have, for the chunk and conv-chunk pair tables."""
    chunks = requests + (capacity - requests) // chunk_size
    conv_chunks = requests + (capacity - requests) // 64

    def pad_chunks(source: torch.Tensor, count: int) -> torch.Tensor:
        return pad(source, count, chunk_tail=capacity)

    return replace(indices, chunk_indices=pad_chunks(indices.chunk_indices, chunks),
                   conv_chunks=pad_chunks(indices.conv_chunks, conv_chunks))


def prepare_mixed_linear_metadata(prefill, decode, prefill_capacity: int):
    """Normalise already-prepared metadata, install it, and return both
    (``mixed.py:59-124``).  The prefill forward then takes exactly
    ``prefill_capacity`` input rows, of which the first
    ``sum(req.extend_len)`` are meaningful; request-level arrays and
    ``cu_seqlens`` keep their actual values and shapes."""
    pm, dm = prefill.linear_attn_metadata, decode.linear_attn_metadata
    if not isinstance(pm, LinearAttnMetadata):
        raise TypeError("mixed prefill requires prepared linear metadata")
    if type(dm) is not type(pm) or pm.phase != "prefill" or dm.phase != "decode":
        raise ValueError("mixed metadata requires matching prefill/decode backends")
    lengths = [req.extend_len for req in prefill.reqs]
    if not lengths or any(length <= 0 for length in lengths):
        raise ValueError("mixed prefill requires nonempty positive request lengths")
    if prefill_capacity < sum(lengths):
        raise ValueError("actual prefill length exceeds mixed graph capacity")
    indices = pm.prefill_indices
    if indices is None or len(indices.cu_seqlens) != len(lengths) + 1:
        raise ValueError("prepare ordinary actual-length metadata before normalization")
    pad = _MetadataPadding()
    packed = _packed_pad(indices, prefill_capacity, len(lengths), 64, pad)
    chunk_capacity = len(packed.chunk_indices)
    if pm.chunk_write_slots is None or pm.conv_token_slots is None:
        raise ValueError("mixed prefill requires direct-write metadata")
    updates = dict(
        prefill_indices=packed,
        chunk_write_slots=pad(pm.chunk_write_slots, chunk_capacity, -1),
        conv_token_slots=pad(pm.conv_token_slots, prefill_capacity, -1),
    )
    # at most one checkpoint per chunk; padded entries read the first real
    # row and write nothing (slot -1)
    for name in ("checkpoint_slots", "checkpoint_chunks", "snapshot_rows", "snapshot_reqs"):
        tensor = getattr(pm, name)
        if tensor is None:
            raise ValueError(f"missing prefill {name}")
        updates[name] = pad(tensor, chunk_capacity, -1 if name == "checkpoint_slots" else 0)
    decode_updates = {}
    for name in ("slots", "read_slots", "write_slots"):
        tensor = getattr(dm, name)
        if tensor is not None:
            decode_updates[name] = tensor.to(torch.int64)
    pad.finish()
    normalized = replace(pm, **updates), replace(dm, **decode_updates)
    prefill.linear_attn_metadata, decode.linear_attn_metadata = normalized
    return normalized


class MixedLinearCopyPlan:
    """Copies fresh normalised metadata into the tensors of ``destination``
    (the structure a graph captured), after validating that only tensor
    contents changed (``mixed.py:127-197``).  Contiguous device tensors (and
    strided vectors) go in one batched launch per device; the rest use
    ``copy_``.  Nothing is written if validation fails."""

    def __init__(self, destination):
        self.tensors = []
        self.constants = []
        self.structures = []

        def visit(dst, getter):
            if isinstance(dst, torch.Tensor):
                self.tensors.append((getter, dst, (dst.shape, dst.dtype, dst.device)))
            elif is_dataclass(dst):
                self.structures.append((getter, type(dst), None))
                for field in fields(dst):
                    visit(getattr(dst, field.name), lambda root, get=getter, name=field.name: getattr(get(root), name))
            elif isinstance(dst, (tuple, list, dict)):
                keys = tuple(dst) if isinstance(dst, dict) else tuple(range(len(dst)))
                self.structures.append((getter, type(dst), keys if isinstance(dst, dict) else len(dst)))
                for key in keys:
                    visit(dst[key], lambda root, get=getter, key=key: get(root)[key])
            else:
                self.constants.append((getter, dst))

        visit(destination, lambda root: root)
        groups = {}
        self.fallback = []
        for index, (_, dst, _) in enumerate(self.tensors):
            if dst.numel() == 0:
                continue
            if dst.is_cuda and (dst.is_contiguous() or dst.ndim == 1):
                groups.setdefault(dst.device, []).append(index)
            else:
                self.fallback.append(index)
        self.groups = [(tuple(indices), tuple(self.tensors[i][1] for i in indices)) for indices in groups.values()]

    def copy(self, source) -> None:
        try:
            for get, kind, size in self.structures:
                value = get(source)
                if type(value) is not kind:
                    raise ValueError("mixed metadata structure changed")
                if size is not None and (tuple(value) if kind is dict else len(value)) != size:
                    raise ValueError("mixed metadata sequence/dictionary changed")
            for get, expected in self.constants:
                if get(source) != expected:
                    raise ValueError("mixed metadata non-tensor value changed")
            sources = tuple(get(source) for get, _, _ in self.tensors)
            for src, (_, _, layout) in zip(sources, self.tensors):
                if not isinstance(src, torch.Tensor) or (src.shape, src.dtype, src.device) != layout:
                    raise ValueError("mixed metadata tensor shape/dtype/device changed")
            for indices, _ in self.groups:
                if any(not sources[i].is_contiguous() and sources[i].ndim != 1 for i in indices):
                    raise ValueError("mixed metadata source strides changed")
        except (AttributeError, KeyError, IndexError, TypeError) as error:
            raise ValueError("mixed metadata structure changed") from error
        for indices, outputs in self.groups:
            copy_metadata(tuple(sources[i] for i in indices), outputs)
        for i in self.fallback:
            self.tensors[i][1].copy_(sources[i])


__all__ = ["MixedLinearCopyPlan", "prepare_mixed_linear_metadata"]
