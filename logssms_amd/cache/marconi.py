"""Marconi hybrid block pool: the state side of the reference's shared KV/state
block storage (``python/logssms/cache/marconi/layout.py:5-38``,
``python/logssms/cache/marconi/block_pool.py:13-110``).

Only what the GDN path touches is here: the layout arithmetic, the strided
``recurrent_state`` / ``conv_state`` views the kernels index with
(physical block, lane), slot allocation bookkeeping (a first-fit contiguous
allocator standing in for the reference's interval allocator), and the state
I/O -- ``copy_state`` / ``zero_state`` run as one gfx950 row-copy / row-zero
launch each instead of a Python loop of per-block ``.copy_()`` calls, and
``map_metadata`` stays device-side torch indexing (graph-capturable).
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, replace
from math import prod

import torch

from .. import _lib


@dataclass(frozen=True)
class HybridBlockLayout:
    """layout.py:5-38."""

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
        """layout.py:17-32: blocks hold one attention layer's KV for
        ``block_size`` tokens per lane; a linear layer's state (+ conv window)
        spans ``state_blocks_per_group`` consecutive blocks."""
        if attention_layers < 1:
            raise ValueError("Marconi requires at least one full-attention layer")
        state_elements = prod(linear_spec.state_shape) + prod(linear_spec.conv_shape)
        token_elements = 2 * kv_heads * head_dim
        minimum = -(-state_elements // (token_elements * 64)) * 64
        if block_size < 0 or block_size % 64:
            raise ValueError("Marconi block size must be zero (auto) or a multiple of 64")
        block_size = block_size or minimum
        layer_elements = block_size * token_elements
        return cls(block_size, attention_layers, -(-linear_spec.num_layers // attention_layers),
                   -(-state_elements // layer_elements), layer_elements, kv_heads, head_dim,
                   tuple(linear_spec.state_shape), tuple(linear_spec.conv_shape))

    @property
    def state_blocks(self) -> int:
        return self.state_groups * self.state_blocks_per_group

    def block_bytes(self, itemsize: int) -> int:
        return self.layers_per_group * self.layer_elements * itemsize


class _ContiguousAllocator:
    """First-fit allocator of runs of consecutive blocks."""

    def __init__(self, num_blocks: int):
        self.free = list(range(num_blocks))

    def allocate_run(self, width: int) -> int:
        free = sorted(self.free)
        run = 0
        for i, b in enumerate(free):
            run = run + 1 if i and b == free[i - 1] + 1 else 1
            if run == width:
                start = b - width + 1
                for x in range(start, start + width):
                    self.free.remove(x)
                return start
        raise RuntimeError("Marconi reservation exhausted")

    def release(self, blocks):
        self.free.extend(blocks)


class HybridBlockPool:
    def __init__(self, layout: HybridBlockLayout, num_blocks: int, device, dtype):
        self.layout = layout
        self._device, self._dtype = torch.device(device), dtype
        self.allocator = _ContiguousAllocator(num_blocks)
        self.storage = torch.zeros(layout.layers_per_group, num_blocks, layout.layer_elements, device=device,
                                   dtype=dtype)
        self.num_blocks = num_blocks
        if num_blocks < layout.state_blocks:
            raise ValueError("Insufficient blocks for a complete State")
        self.state_blocks: dict[int, tuple[int, ...]] = {}
        self.state_refs: dict[int, int] = {}
        self._state_ids = deque(range(num_blocks))
        self.group_table = torch.zeros(num_blocks, layout.state_groups, device=device, dtype=torch.int64)
        lane_stride, block_stride, _ = self.storage.stride()
        state_starts = num_blocks - layout.state_blocks_per_group + 1
        # block_pool.py:32-41: per (start block, lane) views of state and conv window
        self.recurrent_state = self.storage.as_strided(
            (state_starts, layout.layers_per_group, *layout.state_shape),
            (block_stride, lane_stride, layout.state_shape[1] * layout.state_shape[2], layout.state_shape[2], 1))
        self.conv_state = self.storage.as_strided(
            (state_starts, layout.layers_per_group, *layout.conv_shape),
            (block_stride, lane_stride, layout.conv_shape[1], 1), storage_offset=prod(layout.state_shape))

    @property
    def device(self):
        return self._device

    @property
    def dtype(self):
        return self._dtype

    @property
    def num_layers(self):
        return self.layout.layers_per_group

    def allocate_state(self) -> int:
        """block_pool.py:72-79."""
        width = self.layout.state_blocks_per_group
        starts = [self.allocator.allocate_run(width) for _ in range(self.layout.state_groups)]
        blocks = tuple(b for s in starts for b in range(s, s + width))
        slot = self._state_ids.popleft()
        self.state_blocks[slot] = blocks
        self.state_refs[slot] = 1
        self.group_table[slot] = torch.tensor(blocks[::width], device=self.device)
        return slot

    def retain_state(self, slot):
        self.state_refs[slot] += 1

    def release_state(self, slot):
        self.state_refs[slot] -= 1
        if self.state_refs[slot] == 0:
            self.allocator.release(self.state_blocks.pop(slot))
            del self.state_refs[slot]
            self._state_ids.append(slot)

    def _row_geometry(self):
        esize = self.storage.element_size()
        lane_stride, block_stride, _ = self.storage.stride()
        row = prod(self.layout.state_shape) + prod(self.layout.conv_shape)
        return block_stride * esize, row * esize, lane_stride * esize

    def copy_state(self, source, target):
        """block_pool.py:90-94: every group's state + conv window, all lanes,
        from ``source``'s blocks to ``target``'s -- one launch."""
        width = self.layout.state_blocks_per_group
        src = torch.tensor(self.state_blocks[source][::width], dtype=torch.int64).to(self.device)
        dst = torch.tensor(self.state_blocks[target][::width], dtype=torch.int64).to(self.device)
        self.copy_blocks(src, dst)

    def copy_blocks(self, src: torch.Tensor, dst: torch.Tensor):
        """Batched form: state rows of start blocks ``src[i]`` -> ``dst[i]``
        (negative entries skipped), e.g. all of a batch's checkpoint copies."""
        if src.numel() == 0:
            return
        row_stride, row_bytes, lane_bytes = self._row_geometry()
        base = self.storage.data_ptr()
        _lib.call("gdn_copy_rows", base, row_stride, dst.data_ptr(), _lib.index_code(dst), base, row_stride,
                  src.data_ptr(), _lib.index_code(src), src.numel(), self.layout.layers_per_group, row_bytes,
                  lane_bytes, _lib.stream_of(self.storage))

    def zero_state(self, slot):
        """block_pool.py:96-99."""
        blocks = torch.tensor(self.state_blocks[slot][::self.layout.state_blocks_per_group],
                              dtype=torch.int64).to(self.device)
        row_stride, row_bytes, lane_bytes = self._row_geometry()
        _lib.call("gdn_zero_rows", self.storage.data_ptr(), row_stride, blocks.data_ptr(), _lib.index_code(blocks),
                  blocks.numel(), self.layout.layers_per_group, row_bytes, lane_bytes, _lib.stream_of(self.storage))

    def map_metadata(self, metadata, layer):
        """block_pool.py:101-110: logical slots -> physical start blocks of the
        layer's group; negative slots stay -1.  Returns (metadata, lane)."""
        group, lane = divmod(layer, self.layout.layers_per_group)

        def mapped(value):
            if value is None:
                return None
            result = self.group_table[:, group][value.clamp_min(0).long()]
            return torch.where(value >= 0, result, -1)

        names = ("read_slots", "write_slots", "baseline_slots", "checkpoint_slots", "chunk_write_slots",
                 "conv_token_slots")
        return replace(metadata, **{name: mapped(getattr(metadata, name)) for name in names}), lane


__all__ = ["HybridBlockLayout", "HybridBlockPool"]
