"""Fixed-capacity metadata for mixed prefill/decode graph buckets.

Interface of the reference's
``python/logssms/layers/linear_attention_backend/mixed.py:59-197``
(``prepare_mixed_linear_metadata``, ``MixedLinearCopyPlan``): the same names,
arguments, padding rules and errors; the bodies are this library's own.

A bucket fixes the prefill request count and token capacity.  Metadata is
first prepared at the actual lengths and then normalised, outside capture,
to shapes that depend on the bucket only:

* per-token tables are ``capacity`` rows long, per-chunk tables
  ``chunk_capacity(requests, capacity)`` rows long;
* padded write slots are -1 (the kernels skip them), padded index entries are
  0 (they read the first real row), padded chunk pairs are ``(0, capacity)``
  (a chunk starting past the packed tokens, which the kernels clamp away);
* decode slot tables of the standard backend become int64.

Both backends' metadata are handled: the standard (radix / Marconi pool)
``LinearAttnMetadata`` with 64-token chunks, and the LogState
``LogStateLinearAttnMetadata`` with chunks of the pool's granularity and its
per-token log / snapshot tables (``mixed.py:90-121``).  All padding of one
bucket is one ``gdn_metadata_pad`` launch; no device tensor is read on the
host.
"""

from __future__ import annotations

from dataclasses import fields, is_dataclass, replace

import torch

from ..core import get_global_ctx
from ..kernel.metadata import copy_metadata, pad_metadata
from .linear_attention_backend import LinearAttnMetadata
from .linear_attention_logstate import LogStateLinearAttnMetadata

# standard prefill tables padded to the bucket's chunk capacity (at most one
# checkpoint per chunk), and their fill values: padded index entries read the
# first real row, padded destinations are -1 (skipped)
_CHUNK_TABLE_FILLS = {"checkpoint_slots": -1, "checkpoint_chunks": 0, "snapshot_rows": 0, "snapshot_reqs": 0}
# LogState per-token tables padded to the token capacity
_LOGSTATE_TOKEN_FILLS = {"log_slots": -1, "token_offsets": 0, "log_write_slots": -1, "conv_token_granules": 0}
_DECODE_SLOT_TABLES = ("slots", "read_slots", "write_slots")


def chunk_capacity(requests: int, capacity: int, chunk: int = 64) -> int:
    """Most chunks ``requests`` positive lengths summing to at most
    ``capacity`` can need: a length l takes ceil(l / chunk) = 1 + (l - 1) //
    chunk chunks, and the (l - 1) sum to at most capacity - requests."""
    return requests + (capacity - requests) // chunk


class _Padding:
    """Pending padded copies, run together in one launch by ``flush``."""

    def __init__(self):
        self._jobs: list[tuple[torch.Tensor, torch.Tensor, int, int]] = []

    def add(self, tensor: torch.Tensor, rows: int, fill: int = 0, pair_tail: int = -1) -> torch.Tensor:
        if tensor.shape[0] > rows:
            raise ValueError("metadata exceeds mixed graph capacity")
        padded = torch.empty((rows, *tensor.shape[1:]), dtype=tensor.dtype, device=tensor.device)
        self._jobs.append((tensor.contiguous(), padded, fill, pair_tail))
        return padded

    def flush(self) -> None:
        if self._jobs:
            pad_metadata(*(list(column) for column in zip(*self._jobs)))
            self._jobs = []


def prepare_mixed_linear_metadata(prefill, decode, prefill_capacity: int):
    """Normalise the actual-length metadata of ``prefill`` and ``decode`` to
    the bucket of ``prefill_capacity`` tokens, install the results on the two
    batches and return them.  The prefill forward then reads exactly
    ``prefill_capacity`` input rows, of which the first ``sum(extend_len)``
    are real; ``cu_seqlens`` and request-level arrays keep their actual
    values.  The input metadata objects are left unmodified."""
    pm, dm = prefill.linear_attn_metadata, decode.linear_attn_metadata
    if not isinstance(pm, (LinearAttnMetadata, LogStateLinearAttnMetadata)):
        raise TypeError("mixed prefill requires prepared linear metadata")
    if type(dm) is not type(pm) or (pm.phase, dm.phase) != ("prefill", "decode"):
        raise ValueError("mixed metadata requires matching prefill/decode backends")
    lengths = [req.extend_len for req in prefill.reqs]
    if not lengths or min(lengths) <= 0:
        raise ValueError("mixed prefill requires nonempty positive request lengths")
    if sum(lengths) > prefill_capacity:
        raise ValueError("actual prefill length exceeds mixed graph capacity")
    indices = pm.prefill_indices
    if indices is None or indices.cu_seqlens.shape[0] != len(lengths) + 1:
        raise ValueError("prepare ordinary actual-length metadata before normalization")
    if pm.chunk_write_slots is None or pm.conv_token_slots is None:
        raise ValueError("mixed prefill requires direct-write metadata")
    logstate = isinstance(pm, LogStateLinearAttnMetadata)
    per_token, per_chunk = (_LOGSTATE_TOKEN_FILLS, {}) if logstate else ({}, _CHUNK_TABLE_FILLS)
    missing = [name for name in (*per_token, *per_chunk) if getattr(pm, name) is None]
    if missing:
        raise ValueError(f"missing prefill {missing[0]}")
    # LogState chunks are the pool's checkpoint granularity (mixed.py:90-93)
    chunk = get_global_ctx().linear_state.layout.granularity if logstate else 64

    chunks = chunk_capacity(len(lengths), prefill_capacity, chunk)
    padding = _Padding()
    packed = replace(
        indices,
        chunk_indices=padding.add(indices.chunk_indices, chunks, pair_tail=prefill_capacity),
        conv_chunks=padding.add(indices.conv_chunks, chunk_capacity(len(lengths), prefill_capacity, 64),
                                pair_tail=prefill_capacity))
    prefill_tables = {"chunk_write_slots": padding.add(pm.chunk_write_slots, chunks, -1),
                      "conv_token_slots": padding.add(pm.conv_token_slots, prefill_capacity, -1)}
    prefill_tables.update({name: padding.add(getattr(pm, name), chunks, fill) for name, fill in per_chunk.items()})
    prefill_tables.update({name: padding.add(getattr(pm, name), prefill_capacity, fill)
                           for name, fill in per_token.items()})
    if logstate:
        prefill_tables["cu_seqlens"] = packed.cu_seqlens
    decode_tables = {name: getattr(dm, name).to(torch.int64) for name in _DECODE_SLOT_TABLES
                     if isinstance(dm, LinearAttnMetadata) and getattr(dm, name) is not None}
    padding.flush()
    normalized = (replace(pm, prefill_indices=packed, **prefill_tables), replace(dm, **decode_tables))
    prefill.linear_attn_metadata, decode.linear_attn_metadata = normalized
    return normalized


def _leaves(obj, path=()):
    """Flattens a metadata structure into (kind, path, payload) entries in a
    fixed order: ("tensor", path, tensor), ("node", path, shape signature)
    for dataclasses / dicts / lists / tuples, ("const", path, value) for
    anything else."""
    if isinstance(obj, torch.Tensor):
        yield "tensor", path, obj
    elif is_dataclass(obj) and not isinstance(obj, type):
        yield "node", path, (type(obj), None)
        for f in fields(obj):
            yield from _leaves(getattr(obj, f.name), path + (f.name,))
    elif isinstance(obj, dict):
        yield "node", path, (dict, tuple(obj))
        for key, value in obj.items():
            yield from _leaves(value, path + (key,))
    elif isinstance(obj, (list, tuple)):
        yield "node", path, (type(obj), len(obj))
        for i, value in enumerate(obj):
            yield from _leaves(value, path + (i,))
    else:
        yield "const", path, obj


def _layout(t: torch.Tensor):
    return t.shape, t.dtype, t.device


def _vector_or_dense(t: torch.Tensor) -> bool:
    return t.is_contiguous() or t.ndim == 1


class MixedLinearCopyPlan:
    """Refreshes the tensors a graph captured (``destination``) from fresh
    normalised metadata of the same structure.  ``copy`` first checks that
    nothing but tensor contents changed -- same dataclass / container types,
    keys and lengths, equal non-tensor values, same tensor shapes, dtypes and
    devices -- and writes nothing if any check fails.  Device tensors that
    are contiguous or vectors (any stride) are refreshed in one launch per
    device; the rest with ``copy_``."""

    def __init__(self, destination):
        entries = list(_leaves(destination))
        self._structure = [(kind, path, payload) for kind, path, payload in entries if kind != "tensor"]
        self._targets = [(path, tensor, _layout(tensor)) for kind, path, tensor in entries if kind == "tensor"]
        by_device: dict[torch.device, list[int]] = {}
        self._eager: list[int] = []
        for i, (_, tensor, _) in enumerate(self._targets):
            if tensor.numel() == 0:
                continue
            if tensor.is_cuda and _vector_or_dense(tensor):
                by_device.setdefault(tensor.device, []).append(i)
            else:
                self._eager.append(i)
        self._launches = list(by_device.values())

    def _sources(self, source) -> list[torch.Tensor]:
        entries = list(_leaves(source))
        structure = [(kind, path, payload) for kind, path, payload in entries if kind != "tensor"]
        tensors = [(path, tensor) for kind, path, tensor in entries if kind == "tensor"]
        if len(structure) != len(self._structure) or len(tensors) != len(self._targets):
            raise ValueError("mixed metadata structure changed")
        for (kind, path, payload), (want_kind, want_path, want) in zip(structure, self._structure):
            if (kind, path) != (want_kind, want_path):
                raise ValueError("mixed metadata structure changed")
            if kind == "node" and payload != want:
                raise ValueError("mixed metadata sequence/dictionary changed")
            if kind == "const" and payload != want:
                raise ValueError("mixed metadata non-tensor value changed")
        for (path, tensor), (want_path, _, layout) in zip(tensors, self._targets):
            if path != want_path or _layout(tensor) != layout:
                raise ValueError("mixed metadata tensor shape/dtype/device changed")
        sources = [tensor for _, tensor in tensors]
        for group in self._launches:
            if not all(_vector_or_dense(sources[i]) for i in group):
                raise ValueError("mixed metadata source strides changed")
        return sources

    def copy(self, source) -> None:
        sources = self._sources(source)  # validates everything before any write
        for group in self._launches:
            copy_metadata([sources[i] for i in group], [self._targets[i][1] for i in group])
        for i in self._eager:
            self._targets[i][1].copy_(sources[i])


__all__ = ["MixedLinearCopyPlan", "chunk_capacity", "prepare_mixed_linear_metadata"]
