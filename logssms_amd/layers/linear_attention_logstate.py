"""``GatedDeltaLogStateBackend`` -- the LogState variant of the GDN backend,
drop-in for the reference's
``python/logssms/layers/linear_attention_backend/{logstate,gdn_logstate}.py``.

In the LogState cache a request keeps one *work slot* (its running state and
conv window) and writes per-token *logs* (key, v' residual, gate) into the
frames of its pages; decode rebuilds the state from the work slot plus the
tokens logged since its last write-back (at most 16).  The forward passes
here are the reference's, on this library's kernels:

* prefill (``gdn_logstate.py:85-172``): conv history read through the pool,
  packed conv with window snapshots to (slot, granule) frames and the final
  window to the work slot, ``prepare_gdn``, the chunked rule with frame-table
  states (read from and finally written to the work slot, checkpoints every
  ``granularity`` tokens) and the token log;
* decode (``gdn_logstate.py:174-224``): conv decode through the conv frame
  table, then the replayed recurrence with its log rows.

The pool is the process-global ``ctx.linear_state`` (or the context bound at
construction) and must provide what ``cache/logstate/frame_pool.py``'s pool
provides: ``storage`` (uint8 frames), ``dtype``, ``frame_bytes``,
``head_payload_bytes``, ``page_size``, ``payload_frame_table``,
``decay_frame_table``, ``conv_frame_table``, ``layout`` and ``read_conv``.
``prepare_metadata`` (``logstate.py:92-272``) builds the metadata from the
context's ``state_table`` (the log slot of each position), ``work_state_table``
and ``page_table``, the batch's ``positions`` / ``out_loc`` and its
``LogStateCacheMetadata`` (replay counts, checkpoint writes and unlogged
ranges, which the LogState cache manager plans); the pool's ``allocator``
tells work slots from others.  Speculative verify raises
``NotImplementedError``, as in the reference.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ..core import LogStateCacheMetadata, get_global_ctx
from ..kernel.fused import prepare_gdn
from ..kernel.metadata import copy_metadata, make_logstate_prefill_writes
from ..kernel.linear_attention.conv_decode import conv_decode
from ..kernel.linear_attention.gdn import (
    chunk_gated_delta_rule_to_cache,
    fused_recurrent_gated_delta_rule_to_logstate,
)
from ..kernel.linear_attention.packed_conv import PackedConvStateIO, packed_causal_conv1d
from ..kernel.linear_attention.state_io import ChunkLogIO, ChunkStateIO
from .linear_attention_backend import PackedLinearIndices


@dataclass
class LogStateLinearAttnMetadata:
    """logstate.py:21-35."""

    phase: str
    work_slots: torch.Tensor
    log_slots: torch.Tensor
    token_offsets: torch.Tensor
    conv_read_slots: torch.Tensor
    conv_read_granules: torch.Tensor
    replay_counts: torch.Tensor
    cu_seqlens: torch.Tensor | None = None
    prefill_indices: PackedLinearIndices | None = None
    chunk_write_slots: torch.Tensor | None = None
    log_write_slots: torch.Tensor | None = None
    conv_token_slots: torch.Tensor | None = None
    conv_token_granules: torch.Tensor | None = None


@dataclass
class LogStateLinearAttnCaptureData:
    """logstate.py:38-61: decode capture buffers, one int32 entry per
    sequence of the largest captured batch."""

    work_slots: torch.Tensor
    log_slots: torch.Tensor
    token_offsets: torch.Tensor
    conv_read_slots: torch.Tensor
    conv_read_granules: torch.Tensor
    replay_counts: torch.Tensor

    @classmethod
    def make(cls, max_bs: int, device) -> "LogStateLinearAttnCaptureData":
        return cls(*(torch.zeros(max_bs, dtype=torch.int32, device=device) for _ in range(6)))


_CAPTURED = ("work_slots", "log_slots", "token_offsets", "conv_read_slots", "conv_read_granules", "replay_counts")


class GatedDeltaLogStateBackend:
    def __init__(self, ctx=None, *, enable_eager_state: bool = False) -> None:
        self._ctx = ctx
        self.enable_eager_state = enable_eager_state
        self.capture: LogStateLinearAttnCaptureData | None = None
        self.capture_bs: list[int] = []

    @property
    def ctx(self):
        return self._ctx if self._ctx is not None else get_global_ctx()

    # ------------------------------------------------------------ metadata
    def prepare_metadata(self, batch) -> None:
        """logstate.py:92-212 (the table path; the reference's prepared-packet
        shortcut gathers the same slots)."""
        if batch.cache_metadata is None:
            batch.cache_metadata = LogStateCacheMetadata()
        assert isinstance(batch.cache_metadata, LogStateCacheMetadata)
        if batch.is_verify:
            raise NotImplementedError("LogState speculative verify is not implemented yet.")
        ctx = self.ctx
        pool = ctx.linear_state
        state_table, work_table = ctx.state_table, ctx.work_state_table
        assert state_table is not None and work_table is not None and ctx.page_table is not None
        assert work_table.shape[1] == 1
        assert batch.positions is not None and batch.out_loc is not None
        device = pool.storage.device
        reqs = batch.padded_reqs if batch.is_decode else batch.reqs
        table_indices = torch.tensor([r.table_idx for r in reqs], dtype=torch.int64, device=state_table.device)
        if batch.is_decode:
            row_table_indices = table_indices
        else:
            row_table_indices = torch.tensor([r.table_idx for r in reqs for _ in range(r.extend_len)],
                                             dtype=torch.int64, device=state_table.device)
        work_slots = work_table[table_indices, 0]
        positions = batch.positions
        assert len(positions) == len(row_table_indices)
        log_slots = state_table[row_table_indices, positions.long()]
        token_offsets = batch.out_loc.remainder(pool.page_size).to(torch.int32)
        if batch.is_decode:
            counts = batch.cache_metadata.replay_counts
            if counts is None:
                counts = [0] * len(reqs)
            assert len(counts) == len(reqs)
            replay_counts = torch.tensor(counts, dtype=torch.int32, device=device)
            conv_read_slots = work_slots
            conv_read_granules = torch.zeros_like(work_slots)
        else:
            replay_counts = torch.empty(0, dtype=torch.int32, device=device)
            previous = torch.tensor([r.cached_len - 1 for r in reqs], dtype=torch.int64, device=state_table.device)
            previous_slots = state_table[table_indices, previous.clamp_min(0)]
            previous_kv = ctx.page_table[table_indices, previous.clamp_min(0)]
            mapped = (previous >= 0) & (previous_slots >= 0)
            conv_read_slots = torch.where(mapped, previous_slots, work_slots)
            conv_read_granules = torch.where(
                mapped, previous_kv.remainder(pool.page_size) // pool.layout.granularity, 0).to(torch.int32)
        metadata = LogStateLinearAttnMetadata(
            phase=batch.phase, work_slots=work_slots, log_slots=log_slots, token_offsets=token_offsets,
            conv_read_slots=conv_read_slots, conv_read_granules=conv_read_granules, replay_counts=replay_counts)
        if batch.is_prefill:
            self._prepare_direct_prefill(batch, metadata, pool)
        batch.linear_attn_metadata = metadata

    @staticmethod
    def _prepare_direct_prefill(batch, metadata, pool) -> None:
        """logstate.py:214-272: the packed-sequence indices, the chunk
        checkpoint slots, and per token the log write slot (none inside an
        unlogged range) and the conv snapshot target: the token's own log
        slot and granule at each granule end and at the sequence end, or a
        checkpoint slot (granule 0 of a work slot, else the last granule)."""
        lengths = [r.extend_len for r in batch.reqs]
        granularity = pool.layout.granularity
        device = pool.storage.device
        metadata.prefill_indices = PackedLinearIndices.from_lengths(lengths, device, granularity)
        metadata.cu_seqlens = metadata.prefill_indices.cu_seqlens
        first_offsets = batch.cache_metadata.first_offsets
        if first_offsets is None:
            first_offsets = metadata.token_offsets.index_select(0, metadata.cu_seqlens[:-1]).tolist()
        total = sum(lengths)
        chunks = len(metadata.prefill_indices.chunk_indices)
        host = torch.empty(3 * total + chunks, dtype=torch.int32, pin_memory=device.type == "cuda")
        conv_slots, conv_granules, log_mask = host[:3 * total].view(3, total).numpy()
        chunk_writes = host[3 * total:].numpy()
        conv_slots.fill(-1)
        conv_granules.fill(0)
        log_mask.fill(1)
        chunk_writes.fill(-1)
        checkpoints = iter(sorted(batch.cache_metadata.checkpoint_writes))
        checkpoint = next(checkpoints, None)
        ranges: dict[int, list[tuple[int, int]]] = {}
        for req, begin, end in batch.cache_metadata.checkpoint_ranges:
            ranges.setdefault(req, []).append((begin, end))
        token_begin = chunk_begin = 0
        for i, req in enumerate(batch.reqs):
            length, first = lengths[i], first_offsets[i]
            token_end = token_begin + length
            conv_slots[token_begin + granularity - 1 - first % granularity:token_end:granularity] = -2
            if length:
                conv_slots[token_end - 1] = -2
            for begin, end in ranges.get(i, ()):
                begin = max(0, begin - req.cached_len)
                end = min(length, end - req.cached_len)
                if begin < end:
                    log_mask[token_begin + begin:token_begin + end] = 0
                    conv_slots[token_begin + begin:token_begin + end] = -1
            while checkpoint is not None and checkpoint[0] < token_end:
                global_row, slot = checkpoint
                row = global_row - token_begin
                assert row >= 0
                if (first + row + 1) % granularity == 0 or row + 1 == length:
                    conv_slots[global_row] = slot
                    conv_granules[global_row] = (
                        0 if pool.allocator.slot(slot).kind == "work" else pool.layout.num_granules - 1)
                    chunk_writes[chunk_begin + row // granularity] = slot
                checkpoint = next(checkpoints, None)
            token_begin += length
            chunk_begin += (length + granularity - 1) // granularity
        packet = host.to(device, non_blocking=device.type == "cuda")
        metadata.chunk_write_slots = packet[3 * total:]
        metadata.log_write_slots, metadata.conv_token_slots, metadata.conv_token_granules = (
            make_logstate_prefill_writes(metadata.log_slots, metadata.token_offsets, packet, granularity))

    # ------------------------------------------------------------ decode graphs
    def init_capture_graph(self, max_seq_len: int, bs_list: list[int]) -> None:
        del max_seq_len
        assert self.capture is None, "Capture already initialized."
        self.capture_bs = sorted(bs_list)
        self.capture = LogStateLinearAttnCaptureData.make(max(bs_list), self.ctx.linear_state.storage.device)

    def prepare_for_capture(self, batch) -> None:
        """logstate.py:285-292: the batch's metadata, copied into the capture
        buffers, which the captured decode then reads."""
        assert self.capture is not None and batch.size in self.capture_bs
        self.prepare_metadata(batch)
        batch.linear_attn_metadata = self._copy_to_capture(batch.linear_attn_metadata, batch.size)

    def prepare_for_replay(self, batch) -> None:
        """logstate.py:294-299: the fresh metadata of ``batch`` into the
        capture buffers."""
        bs = batch.padded_size
        assert self.capture is not None and bs in self.capture_bs
        self._copy_to_capture(batch.linear_attn_metadata, bs)

    def _copy_to_capture(self, metadata, bs: int) -> "LogStateLinearAttnMetadata":
        """logstate.py:301-329: one batched copy of the six decode fields."""
        assert self.capture is not None and isinstance(metadata, LogStateLinearAttnMetadata)
        copy_metadata(tuple(getattr(metadata, name).to(torch.int32) for name in _CAPTURED),
                      tuple(getattr(self.capture, name)[:bs] for name in _CAPTURED))
        return LogStateLinearAttnMetadata(phase="decode",
                                          **{name: getattr(self.capture, name)[:bs] for name in _CAPTURED})

    # ------------------------------------------------------------ forward
    def forward(self, mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, batch, out=None):
        """gdn_logstate.py:19-59."""
        metadata = batch.linear_attn_metadata
        assert isinstance(metadata, LogStateLinearAttnMetadata)
        assert metadata.phase == batch.phase
        if batch.is_prefill:
            return self._forward_prefill(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, metadata, out)
        if batch.is_verify:
            raise NotImplementedError("LogState speculative verify is not implemented yet.")
        return self._forward_decode(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, metadata, out)

    @staticmethod
    def _split_qkv(mixed_qkv, config):
        """gdn_logstate.py:61-83."""
        query, key, value = torch.split(mixed_qkv, [config.key_dim, config.key_dim, config.value_dim], dim=-1)
        seq_len = mixed_qkv.shape[1]
        return (query.reshape(mixed_qkv.shape[0], seq_len, -1, config.head_k_dim),
                key.reshape(mixed_qkv.shape[0], seq_len, -1, config.head_k_dim),
                value.reshape(mixed_qkv.shape[0], seq_len, -1, config.head_v_dim))

    def _forward_prefill(self, mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, metadata, out=None):
        """gdn_logstate.py:85-172."""
        pool = self.ctx.linear_state
        layer = config.layer_idx
        assert metadata.cu_seqlens is not None and metadata.prefill_indices is not None
        assert metadata.chunk_write_slots is not None
        assert metadata.conv_token_slots is not None and metadata.conv_token_granules is not None
        assert metadata.log_write_slots is not None
        storage = pool.storage.view(pool.dtype)
        history = pool.read_conv(metadata.conv_read_slots, metadata.conv_read_granules, layer)
        mixed = packed_causal_conv1d(
            mixed_qkv, conv_weight, history, metadata.cu_seqlens, metadata.prefill_indices.conv_chunks,
            state_io=PackedConvStateIO(storage=storage, slots=metadata.conv_token_slots,
                                       granules=metadata.conv_token_granules, final_slots=metadata.work_slots,
                                       frame_table=pool.conv_frame_table, frame_bytes=pool.frame_bytes,
                                       layer=layer),
        ).unsqueeze(0)
        query, key, value = self._split_qkv(mixed, config)
        query, key, value, prepared_gate, prepared_beta = prepare_gdn(query, key, value, gate.unsqueeze(0),
                                                                      beta.unsqueeze(0), A_log, dt_bias)
        layout = pool.layout
        output, _ = chunk_gated_delta_rule_to_cache(
            query, key, value, prepared_gate, prepared_beta,
            ChunkStateIO(storage=storage, read_slots=metadata.work_slots,
                         chunk_write_slots=metadata.chunk_write_slots, final_write_slots=metadata.work_slots,
                         payload_frames=pool.payload_frame_table, frame_bytes=pool.frame_bytes,
                         head_payload_bytes=pool.head_payload_bytes, layer=layer,
                         num_layers=layout.num_linear_layers, granularity=layout.granularity,
                         page_size=pool.page_size),
            metadata.cu_seqlens,
            chunk_size=layout.granularity,
            log_io=ChunkLogIO(slots=metadata.log_write_slots, token_offsets=metadata.token_offsets,
                              decay_frames=pool.decay_frame_table, gate=prepared_gate, page_size=pool.page_size,
                              decay_record_bytes=layout.log_decay_bytes, num_key_heads=layout.num_key_heads),
            out=None if out is None else out.unsqueeze(0),
            return_v_new=False,  # v' goes to the log only
        )
        return output.squeeze(0)

    def _forward_decode(self, mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, metadata, out=None):
        """gdn_logstate.py:174-224."""
        pool = self.ctx.linear_state
        layer = config.layer_idx
        query, key, value = conv_decode(
            mixed_qkv, conv_weight, config, split_qkv=True,
            read_slots=metadata.conv_read_slots, read_granules=metadata.conv_read_granules,
            write_slots=metadata.log_slots, write_granules=metadata.token_offsets // pool.layout.granularity,
            work_slots=metadata.work_slots, pool=pool,
        )
        output = fused_recurrent_gated_delta_rule_to_logstate(
            query, key, value, gate.unsqueeze(1), beta.unsqueeze(1), A_log, dt_bias, pool,
            metadata.work_slots, metadata.log_slots, metadata.token_offsets, layer, metadata.replay_counts,
            enable_eager_state=self.enable_eager_state, out=None if out is None else out.unsqueeze(1),
        )
        return output.squeeze(1)


__all__ = ["GatedDeltaLogStateBackend", "LogStateLinearAttnCaptureData", "LogStateLinearAttnMetadata"]
