"""Marconi hybrid block pool and checkpoint placement, the state side of the
reference's shared KV/state block storage.

Interface (names, fields, views and semantics) of the reference's
``python/logssms/cache/marconi/layout.py:5-38``,
``cache/marconi/block_pool.py:13-110`` and the ``prepare_batch`` /
``after_forward`` steps of ``cache/marconi/manager.py:248-278``; the
implementation is this library's own:

* ``HybridBlockLayout`` -- the block format arithmetic (fixed by the format).
* ``HybridBlockPool`` -- block storage ``[lanes, blocks, layer_elements]``;
  free blocks are a bitmap searched for runs with a sliding-window count;
  state slots are recycled lowest id first; the lane-strided
  ``recurrent_state`` / ``conv_state`` views the kernels index with
  (start block, lane); ``copy_state`` / ``zero_state`` / ``copy_blocks`` are
  one gfx950 launch each (``gdn_copy_rows`` / ``gdn_zero_rows``), and
  ``map_metadata`` is one device gather per slot table through a column
  that ends in a -1 sentinel.
* ``MarconiRequestState`` / ``MarconiCheckpointer`` -- where a prefill writes
  its states (branch checkpoints, the last page boundary, the output slot of
  the double-buffered live states) and the checkpoint copies after the
  forward, all of a step's copies in one launch.

The prefix tree, eviction tuning and block allocation policy of the
reference's ``MarconiCacheManager`` are engine-side and not part of this
library.
"""

from __future__ import annotations

import heapq
from dataclasses import dataclass, field, replace
from math import prod

import numpy as np
import torch

from .. import _lib
from ..core import MarconiCacheMetadata


def _ceil_div(a: int, b: int) -> int:
    return -(-a // b)


@dataclass(frozen=True)
class HybridBlockLayout:
    """``cache/marconi/layout.py:5-38``: a block holds ``block_size`` tokens
    of K and V for one attention layer per lane (``layers_per_group`` lanes);
    a linear layer's state plus conv window spans ``state_blocks_per_group``
    consecutive blocks of one lane, and the linear layers are split into
    ``state_groups`` groups of ``layers_per_group`` layers."""

    block_size: int
    layers_per_group: int
    state_groups: int
    state_blocks_per_group: int
    layer_elements: int
    kv_heads: int
    head_dim: int
    state_shape: tuple[int, int, int]
    conv_shape: tuple[int, int]

    @classmethod
    def make(cls, attention_layers, linear_spec, kv_heads, head_dim, block_size=128):
        if attention_layers < 1:
            raise ValueError("Marconi requires at least one full-attention layer")
        if block_size < 0 or block_size % 64:
            raise ValueError("Marconi block size must be zero (auto) or a multiple of 64")
        per_token = 2 * kv_heads * head_dim  # K and V elements of one token in one lane
        state = prod(linear_spec.state_shape) + prod(linear_spec.conv_shape)
        if block_size == 0:  # smallest multiple of 64 tokens whose block holds a whole state
            block_size = 64 * _ceil_div(state, 64 * per_token)
        layer_elements = block_size * per_token
        return cls(block_size=block_size, layers_per_group=attention_layers,
                   state_groups=_ceil_div(linear_spec.num_layers, attention_layers),
                   state_blocks_per_group=_ceil_div(state, layer_elements), layer_elements=layer_elements,
                   kv_heads=kv_heads, head_dim=head_dim, state_shape=tuple(linear_spec.state_shape),
                   conv_shape=tuple(linear_spec.conv_shape))

    @property
    def state_blocks(self) -> int:
        return self.state_groups * self.state_blocks_per_group

    def block_bytes(self, itemsize: int) -> int:
        return self.layers_per_group * self.layer_elements * itemsize


class _FreeBlocks:
    """Free-block bitmap.  ``take_run`` returns the lowest block starting
    ``width`` consecutive free blocks and marks them used."""

    def __init__(self, num_blocks: int):
        self._free = np.ones(num_blocks, dtype=bool)

    @property
    def free(self) -> list[int]:
        return np.flatnonzero(self._free).tolist()

    def take_run(self, width: int) -> int:
        window = np.convolve(self._free.astype(np.int32), np.ones(width, dtype=np.int32), mode="valid")
        starts = np.flatnonzero(window == width)
        if starts.size == 0:
            raise RuntimeError("Marconi reservation exhausted")
        start = int(starts[0])
        self._free[start:start + width] = False
        return start

    def give_back(self, blocks) -> None:
        self._free[np.asarray(blocks, dtype=np.int64)] = True


# LinearAttnMetadata fields holding logical state slots (map_metadata maps them)
_SLOT_FIELDS = ("read_slots", "write_slots", "baseline_slots", "checkpoint_slots", "chunk_write_slots",
                "conv_token_slots")


class HybridBlockPool:
    def __init__(self, layout: HybridBlockLayout, num_blocks: int, device, dtype):
        if num_blocks < layout.state_blocks:
            raise ValueError("Insufficient blocks for a complete State")
        self.layout = layout
        self.num_blocks = num_blocks
        self._device, self._dtype = torch.device(device), dtype
        self.allocator = _FreeBlocks(num_blocks)
        self.storage = torch.zeros(layout.layers_per_group, num_blocks, layout.layer_elements, device=device,
                                   dtype=dtype)
        # slot -> all its blocks (state_groups runs of state_blocks_per_group), and its reference count
        self.state_blocks: dict[int, tuple[int, ...]] = {}
        self.state_refs: dict[int, int] = {}
        self._free_ids = list(range(num_blocks))  # a heap: lowest free slot id first
        # slot -> start block of each group's run (what the kernels address)
        self.group_table = torch.zeros(num_blocks, layout.state_groups, device=device, dtype=torch.int64)
        self.recurrent_state = self._lane_view(layout.state_shape, 0)
        self.conv_state = self._lane_view(layout.conv_shape, prod(layout.state_shape))

    def _lane_view(self, inner_shape, offset: int) -> torch.Tensor:
        """``[start block, lane, *inner_shape]`` over the storage: a state that
        starts at block b of lane l begins ``offset`` elements into it and
        runs on contiguously (across block ends when it spans several)."""
        lane_stride, block_stride, _ = self.storage.stride()
        inner = [1]
        for n in reversed(inner_shape[1:]):
            inner.insert(0, inner[0] * n)
        starts = self.num_blocks - self.layout.state_blocks_per_group + 1
        return self.storage.as_strided((starts, self.layout.layers_per_group, *inner_shape),
                                       (block_stride, lane_stride, *inner), storage_offset=offset)

    @property
    def device(self):
        return self._device

    @property
    def dtype(self):
        return self._dtype

    @property
    def num_layers(self):
        return self.layout.layers_per_group

    # ------------------------------------------------------------ slots
    def allocate_state(self) -> int:
        width = self.layout.state_blocks_per_group
        if not self._free_ids:
            raise RuntimeError("Marconi reservation exhausted")
        starts = []
        try:
            for _ in range(self.layout.state_groups):
                starts.append(self.allocator.take_run(width))
        except RuntimeError:
            for s in starts:
                self.allocator.give_back(range(s, s + width))
            raise
        slot = heapq.heappop(self._free_ids)
        self.state_blocks[slot] = tuple(b for s in starts for b in range(s, s + width))
        self.state_refs[slot] = 1
        self.group_table[slot] = torch.tensor(starts, dtype=torch.int64)
        return slot

    def retain_state(self, slot: int) -> None:
        self.state_refs[slot] += 1

    def release_state(self, slot: int) -> None:
        self.state_refs[slot] -= 1
        if self.state_refs[slot] > 0:
            return
        del self.state_refs[slot]
        self.allocator.give_back(self.state_blocks.pop(slot))
        heapq.heappush(self._free_ids, slot)

    def _starts(self, slot: int) -> tuple[int, ...]:
        return self.state_blocks[slot][::self.layout.state_blocks_per_group]

    # ------------------------------------------------------------ state I/O
    def _row_geometry(self):
        """(bytes between start blocks, bytes of one state row, bytes between lanes)."""
        size = self.storage.element_size()
        lane_stride, block_stride, _ = self.storage.stride()
        row = prod(self.layout.state_shape) + prod(self.layout.conv_shape)
        return block_stride * size, row * size, lane_stride * size

    def copy_blocks(self, src_blocks, dst_blocks) -> None:
        """State rows (state + conv window, every lane) of start blocks
        ``src_blocks[i]`` -> ``dst_blocks[i]``, all in one launch.  Host
        sequences; the destinations must be distinct and none of them a
        source, because the copies of one launch run in no fixed order (the
        reference copies one after another, ``block_pool.py:90-94``)."""
        src = [int(b) for b in src_blocks]
        dst = [int(b) for b in dst_blocks]
        if len(src) != len(dst):
            raise ValueError("copy_blocks: source and destination counts differ")
        if not src:
            return
        if len(set(dst)) != len(dst) or set(dst) & set(src):
            raise ValueError("copy_blocks: a destination block repeats or is also a source")
        pairs = torch.tensor([src, dst], dtype=torch.int64).to(self.device)
        row_stride, row_bytes, lane_bytes = self._row_geometry()
        base = self.storage.data_ptr()
        _lib.call("gdn_copy_rows", base, row_stride, pairs[1].data_ptr(), _lib.I64_CODE, base, row_stride,
                  pairs[0].data_ptr(), _lib.I64_CODE, len(src), self.layout.layers_per_group, row_bytes, lane_bytes,
                  _lib.stream_of(self.storage))

    def copy_states(self, pairs) -> None:
        """``copy_state`` for every (source, target) slot pair, one launch."""
        src, dst = [], []
        for source, target in pairs:
            src.extend(self._starts(source))
            dst.extend(self._starts(target))
        self.copy_blocks(src, dst)

    def copy_state(self, source: int, target: int) -> None:
        """``block_pool.py:90-94``: every group's state and conv window, all
        lanes, from ``source``'s blocks to ``target``'s."""
        self.copy_states([(source, target)])

    def zero_state(self, slot: int) -> None:
        """``block_pool.py:96-99``."""
        starts = torch.tensor(self._starts(slot), dtype=torch.int64).to(self.device)
        row_stride, row_bytes, lane_bytes = self._row_geometry()
        _lib.call("gdn_zero_rows", self.storage.data_ptr(), row_stride, starts.data_ptr(), _lib.I64_CODE,
                  starts.numel(), self.layout.layers_per_group, row_bytes, lane_bytes, _lib.stream_of(self.storage))

    def map_metadata(self, metadata, layer: int):
        """``block_pool.py:101-110``: logical slots -> the start block of the
        layer's group; negative slots map to -1.  Returns (metadata, lane).
        Device-side only (no host read), so it may run under capture."""
        group, lane = divmod(layer, self.layout.layers_per_group)
        column = torch.cat([self.group_table[:, group], self.group_table.new_full((1,), -1)])

        def mapped(slots):
            # index -1 is the sentinel appended above; every negative slot goes there
            return None if slots is None else column[slots.long().clamp_min(-1)]

        return replace(metadata, **{name: mapped(getattr(metadata, name)) for name in _SLOT_FIELDS}), lane


# ---------------------------------------------------------------- checkpoint placement

@dataclass
class MarconiRequestState:
    """What checkpoint placement reads of a request (the reference's
    ``MarconiRequest``, ``cache/marconi/manager.py:70-85``): two live state
    slots used alternately page by page, and planned checkpoints
    {token end: slot}."""

    states: tuple[int, int]
    checkpoints: dict[int, int] = field(default_factory=dict)

    def state_at(self, end: int, page_size: int) -> int:
        """Live slot holding the state after ``end`` tokens: pages alternate."""
        return self.states[((end - 1) // page_size) & 1]


class MarconiCheckpointer:
    """``prepare_batch`` / ``after_forward`` of the reference's
    ``MarconiCacheManager`` (``cache/marconi/manager.py:248-278``) over
    ``requests`` (``table_idx`` -> ``MarconiRequestState``).

    For each prefill request extending ``cached_len`` -> ``device_len``, the
    forward writes the state after ``end - cached_len`` of its tokens to a
    slot, for every ``end`` in:

    * a planned checkpoint strictly inside (cached_len, device_len): its slot;
    * the last page boundary inside it: the live slot of that page, and when
      a checkpoint is planned there too, that checkpoint instead receives a
      copy of the live slot after the forward;
    * device_len: the live slot of the last page, copied after the forward to
      a checkpoint planned at device_len.
    """

    def __init__(self, pool: HybridBlockPool, page_size: int):
        self.pool = pool
        self.page_size = page_size
        self.requests: dict[int, MarconiRequestState] = {}

    def plan(self, entry: MarconiRequestState, cached_len: int, device_len: int):
        """(sorted [(end - cached_len, slot)], [(source slot, checkpoint slot)])."""
        ps = self.page_size
        writes = {end - cached_len: slot for end, slot in entry.checkpoints.items() if cached_len < end < device_len}
        copies = []
        last = entry.state_at(device_len, ps)
        writes[device_len - cached_len] = last
        if device_len in entry.checkpoints:
            copies.append((last, entry.checkpoints[device_len]))
        boundary = device_len - device_len % ps
        if cached_len < boundary < device_len:
            live = entry.state_at(boundary, ps)
            writes[boundary - cached_len] = live
            if boundary in entry.checkpoints:
                copies.append((live, entry.checkpoints[boundary]))
        return sorted(writes.items()), copies

    def prepare_batch(self, batch) -> None:
        if not batch.is_prefill:
            return
        metadata = MarconiCacheMetadata(checkpoint_writes=[])
        for req in batch.reqs:
            writes, copies = self.plan(self.requests[req.table_idx], req.cached_len, req.device_len)
            metadata.checkpoint_writes.append(writes)
            metadata.checkpoint_copies.extend(copies)
        batch.cache_metadata = metadata

    def after_forward(self, batch) -> None:
        """All checkpoint copies of the batch (of both parts of a mixed
        batch) in one ``copy_rows`` launch."""
        parts = batch.mixed_parts if batch.is_mixed else (batch,)
        pairs = [pair for part in parts if isinstance(part.cache_metadata, MarconiCacheMetadata)
                 for pair in part.cache_metadata.checkpoint_copies]
        self.pool.copy_states(pairs)


__all__ = ["HybridBlockLayout", "HybridBlockPool", "MarconiCheckpointer", "MarconiRequestState"]
