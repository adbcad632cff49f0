"""Minimal engine-side records the GDN backend reads (mirrors of the fields the
reference's ``python/logssms/core.py`` ``Context`` / ``Batch`` / ``Request``
expose to ``layers/linear_attention_backend``).  The engine, scheduler and
cache managers that fill them in are outside this library."""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Literal

import torch


@dataclass
class Request:
    table_idx: int
    cached_len: int
    device_len: int

    @property
    def extend_len(self) -> int:
        return self.device_len - self.cached_len


@dataclass
class MarconiCacheMetadata:
    """cache/marconi/metadata.py:6-9."""

    checkpoint_writes: list[list[tuple[int, int]]] | None = None
    checkpoint_copies: list[tuple[int, int]] = field(default_factory=list)


@dataclass
class LogStateCacheMetadata:
    """cache/logstate/metadata.py:6-10 (with cache/metadata.py:5-6): the
    replay count of each decode request, the page offset of each prefill
    request's first token, the checkpoint writes (global token row, slot) and
    the (request, begin, end) position ranges whose tokens are not logged."""

    replay_counts: list[int] | None = None
    first_offsets: list[int] | None = None
    checkpoint_writes: list[tuple[int, int]] = field(default_factory=list)
    checkpoint_ranges: list[tuple[int, int, int]] = field(default_factory=list)


@dataclass
class BatchIndices:
    """utils/batch.py:9-32: the fields of the engine's prepared batch packet
    (``Batch.prepared_indices``) that the linear-attention backends read, all
    int32 device tensors: per request its table row, cached length, previous
    position (cached length - 1) and replay count; per token its table row
    (``token_table_ids``, set by the engine after ``make_batch_mapping``)."""

    table_ids: torch.Tensor
    cached_lens: torch.Tensor
    previous_positions: torch.Tensor
    replay_counts: torch.Tensor
    token_table_ids: torch.Tensor | None = None

    @classmethod
    def make(cls, batch: "Batch", device, replay_counts=None) -> "BatchIndices":
        """The packet of ``batch.padded_reqs`` in one host-to-device copy
        (utils/batch.py:43-121 builds the same per-request vectors)."""
        reqs = batch.padded_reqs
        n = len(reqs)
        counts = list(replay_counts) if replay_counts is not None else [0] * n
        assert len(counts) == n
        host = torch.tensor([r.table_idx for r in reqs] + [r.cached_len for r in reqs] +
                            [r.cached_len - 1 for r in reqs] + counts, dtype=torch.int32)
        packet = host.to(device)
        tables, cached, previous, replay = packet.split(n)
        return cls(tables, cached, previous, replay)


@dataclass
class Batch:
    reqs: list[Request]
    phase: Literal["prefill", "decode", "verify", "mixed"]
    padded_reqs: list[Request] | None = None
    cache_metadata: Any = None
    linear_attn_metadata: Any = None
    # mixed batches (core.py:117-127): the prefill requests first, then the decode
    # ones; mixed_parts = (prefill batch, decode batch); the prefill inputs take
    # prefill_token_capacity rows (0: exactly the prefill tokens)
    num_prefill_reqs: int = 0
    mixed_parts: tuple | None = None
    prefill_token_capacity: int = 0
    # token positions and KV locations of the batch rows (core.py Batch.positions
    # / out_loc), read by the LogState metadata
    positions: torch.Tensor | None = None
    out_loc: torch.Tensor | None = None
    # the engine's prepared batch packet (core.py:132), or None
    prepared_indices: BatchIndices | None = None

    def __post_init__(self):
        if self.padded_reqs is None:
            self.padded_reqs = self.reqs

    @property
    def is_mixed(self) -> bool:
        return self.phase == "mixed"

    @property
    def prefill_count(self) -> int:
        return self.size if self.is_prefill else self.num_prefill_reqs

    @property
    def prefill_reqs(self) -> list[Request]:
        return self.reqs[:self.prefill_count]

    @property
    def decode_reqs(self) -> list[Request]:
        return self.reqs[self.prefill_count:] if not self.is_verify else []

    @property
    def prefill_tokens(self) -> int:
        return sum(req.extend_len for req in self.prefill_reqs)

    @property
    def is_prefill(self) -> bool:
        return self.phase == "prefill"

    @property
    def is_decode(self) -> bool:
        return self.phase == "decode"

    @property
    def is_verify(self) -> bool:
        return self.phase == "verify"

    @property
    def size(self) -> int:
        return len(self.reqs)

    @property
    def padded_size(self) -> int:
        return len(self.padded_reqs)


@dataclass
class Context:
    page_size: int
    linear_state: Any = None
    state_table: torch.Tensor | None = None
    work_state_table: torch.Tensor | None = None
    page_table: torch.Tensor | None = None
    batch: Any = None  # the batch being run (GatedDeltaNet.attend reads it)
    _backend: Any = field(default=None, repr=False)

    @property
    def linear_attn_backend(self):
        """The GDN backend bound to this context (created on first use)."""
        if self._backend is None:
            from .layers.linear_attention_backend import GatedDeltaBackend

            self._backend = GatedDeltaBackend(self)
        return self._backend


_GLOBAL_CTX: Context | None = None


def set_global_ctx(ctx: Context) -> None:
    global _GLOBAL_CTX
    _GLOBAL_CTX = ctx


def clear_global_ctx() -> None:
    global _GLOBAL_CTX
    _GLOBAL_CTX = None


def get_global_ctx() -> Context:
    assert _GLOBAL_CTX is not None, "no global context set"
    return _GLOBAL_CTX


__all__ = ["Batch", "BatchIndices", "Context", "LogStateCacheMetadata", "MarconiCacheMetadata", "Request", "clear_global_ctx",
           "get_global_ctx", "set_global_ctx"]
