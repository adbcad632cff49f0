"""``GatedDeltaLogStateBackend``: the Gated DeltaNet backend over a LogState
cache, drop-in for the reference's
``python/logssms/layers/linear_attention_backend/{logstate,gdn_logstate}.py``
(same class, dataclass and method names and fields, same slot plan).

In a LogState cache a request owns one *work slot* (its running state and
conv window) and logs every token (key, v' residual, gate) into the frames of
the log slot of the page the token lands in; decode rebuilds the state from
the work slot plus the at most 16 tokens logged since its last write-back.

Metadata (``prepare_metadata``), from the context's ``state_table`` (the log
slot of every position), ``work_state_table`` and ``page_table``:

* decode: work slot, log slot at the new position, the position's page
  offset and the replay count per request -- gathered on the device from the
  engine's prepared packet when the batch carries one (``gdn_gather_linear_
  slots``), else from the tables with one host upload;
* prefill: the same per token, the conv history source of each request (the
  log slot and granule of its previous position, else its work slot), and
  the write plan -- per token the conv snapshot target and the log write
  slot, per ``granularity``-token chunk the checkpoint slot.  The plan's host
  part is built vectorised in numpy (``logstate_prefill_plan``) from the
  ``LogStateCacheMetadata`` the cache manager fills in (first page offsets,
  checkpoint writes, unlogged ranges) and finished on the device
  (``make_logstate_prefill_writes``).

Forward, on this library's kernels:

* prefill (``gdn_logstate.py:85-172``'s results): the conv history is read
  through the pool (``read_conv``); one front-end pass computes the packed
  conv + SiLU, the q/k/v split and ``prepare_gdn``
  (``gdn_prefill_frontend``) where the reference runs two ops; the raw conv
  windows go to their (slot, granule) snapshots and each request's last one
  to its work slot; the chunked rule runs at the pool's granularity on
  frame-table states with the v' rows written into the log by the chunk
  kernel, and the log store adds keys and gates;
* decode (``gdn_logstate.py:174-224``): the conv decode through the conv
  frame table, then the replayed recurrence.

The pool is the process-global ``ctx.linear_state`` (or that of the context
bound at construction) and provides what the reference's
``cache/logstate/frame_pool.py`` pool provides: ``storage`` (uint8 frames),
``dtype``, ``frame_bytes``, ``head_payload_bytes``, ``page_size``,
``payload_frame_table``, ``decay_frame_table``, ``conv_frame_table``,
``layout``, ``allocator`` and ``read_conv``.  Speculative verify raises
``NotImplementedError``, as in the reference.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import NamedTuple

import numpy as np
import torch

from ..core import LogStateCacheMetadata, get_global_ctx
from ..kernel.linear_attention.conv_decode import conv_decode
from ..kernel.linear_attention.fused_backend import prefill_frontend
from ..kernel.linear_attention.gdn import (
    chunk_gated_delta_rule_to_cache,
    fused_recurrent_gated_delta_rule_to_logstate,
)
from ..kernel.linear_attention.packed_conv import PackedConvStateIO, conv_windows_logstate
from ..kernel.linear_attention.state_io import ChunkLogIO, ChunkStateIO
from ..kernel.metadata import copy_metadata, gather_linear_slots, make_logstate_prefill_writes
from .linear_attention_backend import MixedForward, PackedLinearIndices


@dataclass
class LogStateLinearAttnMetadata:
    """logstate.py:21-35 (field names and meaning are the interface)."""

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


# the per-request fields a captured decode reads (all int32)
_DECODE_FIELDS = ("work_slots", "log_slots", "token_offsets", "conv_read_slots", "conv_read_granules",
                  "replay_counts")


@dataclass
class LogStateLinearAttnCaptureData:
    """logstate.py:38-61: the decode capture buffers, one int32 entry per
    request of the largest captured batch."""

    work_slots: torch.Tensor
    log_slots: torch.Tensor
    token_offsets: torch.Tensor
    conv_read_slots: torch.Tensor
    conv_read_granules: torch.Tensor
    replay_counts: torch.Tensor

    @classmethod
    def make(cls, max_bs: int, device) -> "LogStateLinearAttnCaptureData":
        block = torch.zeros(len(_DECODE_FIELDS), max_bs, dtype=torch.int32, device=device)
        return cls(*block.unbind(0))

    def view(self, bs: int) -> LogStateLinearAttnMetadata:
        """Decode metadata reading the first ``bs`` entries of the buffers."""
        return LogStateLinearAttnMetadata(phase="decode", **{f: getattr(self, f)[:bs] for f in _DECODE_FIELDS})


def logstate_prefill_plan(lengths, cached_lens, first_offsets, checkpoint_writes, checkpoint_ranges,
                          granularity: int, num_granules: int, work_slot) -> np.ndarray:
    """The host part of the LogState prefill write plan
    (``logstate.py:215-272``), one int32 vector ``[conv slot (T) | conv
    granule (T) | log enabled (T) | chunk write slot (chunks)]`` for T packed
    tokens and ``sum(ceil(length / granularity))`` chunks.

    Conv slot -2 marks a token whose snapshot goes to its own log slot (at a
    granule end, ``(first + row + 1) % granularity == 0``, and at its
    request's last token); tokens inside an unlogged range ``(request, begin,
    end)`` (positions; ``begin - cached_len`` .. ``end - cached_len`` clipped
    to the request) are not logged and take no snapshot.  A checkpoint
    ``(global row, slot)`` whose token is a marked one makes that token's
    snapshot and its chunk's state write go to ``slot`` (granule 0 when
    ``work_slot(slot)``, else the last granule); among checkpoints on one
    token or one chunk the last in sorted ``(row, slot)`` order wins, and the
    rest are ignored."""
    g = int(granularity)
    lens = np.asarray(lengths, dtype=np.int64)
    n = lens.size
    tok_start = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(lens, out=tok_start[1:])
    chunk_start = np.zeros(n + 1, dtype=np.int64)
    np.cumsum((lens + g - 1) // g, out=chunk_start[1:])
    T, chunks = int(tok_start[-1]), int(chunk_start[-1])
    owner = np.repeat(np.arange(n, dtype=np.int64), lens)
    row = np.arange(T, dtype=np.int64) - tok_start[owner]
    first = np.asarray(first_offsets, dtype=np.int64).reshape(n)
    marked = ((first[owner] + row + 1) % g == 0) | (row + 1 == lens[owner])

    plan = np.empty(3 * T + chunks, dtype=np.int32)
    conv, gran, logged, chunk = plan[:T], plan[T:2 * T], plan[2 * T:3 * T], plan[3 * T:]
    conv[:] = np.where(marked, -2, -1)
    gran[:] = 0
    logged[:] = 1
    chunk[:] = -1

    if len(checkpoint_ranges):
        spans = np.asarray(checkpoint_ranges, dtype=np.int64).reshape(-1, 3)
        spans = spans[(spans[:, 0] >= 0) & (spans[:, 0] < n)]  # ranges of other batches' requests: none
        req = spans[:, 0]
        cached = np.asarray(cached_lens, dtype=np.int64).reshape(n)[req]
        lo = np.maximum(0, spans[:, 1] - cached)
        hi = np.minimum(lens[req], spans[:, 2] - cached)
        keep = lo < hi
        edges = np.zeros(T + 1, dtype=np.int64)  # +1 at a range's first token, -1 after its last
        np.add.at(edges, tok_start[req[keep]] + lo[keep], 1)
        np.add.at(edges, tok_start[req[keep]] + hi[keep], -1)
        unlogged = np.cumsum(edges[:T]) > 0
        logged[unlogged] = 0
        conv[unlogged] = -1

    if len(checkpoint_writes):
        writes = np.asarray(sorted(checkpoint_writes), dtype=np.int64).reshape(-1, 2)
        assert (writes[:, 0] >= 0).all(), "checkpoint rows are packed token indices"
        writes = writes[writes[:, 0] < T]  # rows past the batch are never reached
        writes = writes[marked[writes[:, 0]]]
        if len(writes):
            tok, slot = writes[:, 0], writes[:, 1]
            kind = np.asarray([0 if work_slot(int(s)) else num_granules - 1 for s in slot], dtype=np.int64)
            target = chunk_start[owner[tok]] + row[tok] // g

            def last_of(keys):  # index of the last entry of each distinct key (entries in sorted order)
                _, from_end = np.unique(keys[::-1], return_index=True)
                return len(keys) - 1 - from_end

            t_last = last_of(tok)
            conv[tok[t_last]] = slot[t_last]
            gran[tok[t_last]] = kind[t_last]
            c_last = last_of(target)
            chunk[target[c_last]] = slot[c_last]
    return plan


class _Tables(NamedTuple):
    pool: object
    state: torch.Tensor  # [rows, positions]: the log slot of every position
    work: torch.Tensor   # [rows, 1]
    page: torch.Tensor   # [rows, positions]: KV locations

    @classmethod
    def of(cls, ctx) -> "_Tables":
        assert ctx.state_table is not None and ctx.work_state_table is not None and ctx.page_table is not None
        assert ctx.work_state_table.shape[1] == 1
        return cls(ctx.linear_state, ctx.state_table, ctx.work_state_table, ctx.page_table)


def _upload(values: np.ndarray, device) -> torch.Tensor:
    """One host-to-device copy of an index vector (pinned, asynchronous)."""
    host = torch.from_numpy(np.ascontiguousarray(values))
    device = torch.device(device)
    if device.type != "cuda":
        return host.to(device)
    return host.pin_memory().to(device, non_blocking=True)


class GatedDeltaLogStateBackend(MixedForward):
    def __init__(self, ctx=None, *, enable_eager_state: bool = False) -> None:
        self._ctx = ctx
        self.enable_eager_state = enable_eager_state
        self.capture: LogStateLinearAttnCaptureData | None = None
        self.capture_bs: list[int] = []
        self._sequence_ids: torch.Tensor | None = None  # 0, 1, 2, ... on the pool's device

    @property
    def ctx(self):
        return self._ctx if self._ctx is not None else get_global_ctx()

    # ------------------------------------------------------------ metadata
    def prepare_metadata(self, batch) -> None:
        if batch.cache_metadata is None:
            batch.cache_metadata = LogStateCacheMetadata()
        assert isinstance(batch.cache_metadata, LogStateCacheMetadata)
        if batch.is_verify:
            raise NotImplementedError("LogState speculative verify is not implemented yet.")
        assert batch.positions is not None and batch.out_loc is not None
        tables = _Tables.of(self.ctx)
        if batch.is_decode:
            batch.linear_attn_metadata = self._decode_metadata(batch, tables)
        else:
            batch.linear_attn_metadata = self._prefill_metadata(batch, tables)

    @staticmethod
    def _decode_metadata(batch, t: _Tables) -> LogStateLinearAttnMetadata:
        reqs = batch.padded_reqs
        packet = batch.prepared_indices
        if packet is not None and t.state.is_cuda:
            work, logs, offsets, granules = gather_linear_slots(
                packet, t.state, work_table=t.work, out_loc=batch.out_loc, page_size=t.pool.page_size).unbind(0)
            counts = packet.replay_counts
        else:
            replay = batch.cache_metadata.replay_counts
            replay = [0] * len(reqs) if replay is None else list(replay)
            assert len(replay) == len(reqs)
            host = np.asarray([[r.table_idx for r in reqs], replay], dtype=np.int64)
            rows, counts = _upload(host, t.state.device).unbind(0)
            work = t.work[rows, 0]
            assert len(batch.positions) == len(reqs)
            logs = t.state[rows, batch.positions.long()]
            offsets = batch.out_loc.remainder(t.pool.page_size).to(torch.int32)
            granules = torch.zeros_like(work)
            counts = counts.to(torch.int32)
        return LogStateLinearAttnMetadata(phase=batch.phase, work_slots=work, log_slots=logs, token_offsets=offsets,
                                          conv_read_slots=work, conv_read_granules=granules, replay_counts=counts)

    def _prefill_metadata(self, batch, t: _Tables) -> LogStateLinearAttnMetadata:
        pool = t.pool
        reqs = batch.reqs
        lengths = np.asarray([r.extend_len for r in reqs], dtype=np.int64)
        cached = np.asarray([r.cached_len for r in reqs], dtype=np.int64)
        packet = batch.prepared_indices
        if packet is not None and packet.token_table_ids is not None:
            req_rows, token_rows, previous = packet.table_ids, packet.token_table_ids, packet.previous_positions
        else:
            ids = np.asarray([r.table_idx for r in reqs], dtype=np.int64)
            req_rows, token_rows, previous = _upload(
                np.concatenate([ids, np.repeat(ids, lengths), cached - 1]), t.state.device).split(
                    [len(reqs), int(lengths.sum()), len(reqs)])
        assert len(batch.positions) == len(token_rows)
        work = t.work[req_rows, 0]
        logs = t.state[token_rows, batch.positions.long()]
        offsets = batch.out_loc.remainder(pool.page_size).to(torch.int32)
        # the conv history: the snapshot at the previous position when it is logged, else the work slot's window
        before = previous.clamp_min(0)
        before_slots = t.state[req_rows, before]
        before_granules = t.page[req_rows, before].remainder(pool.page_size) // pool.layout.granularity
        logged_before = (previous >= 0) & (before_slots >= 0)
        conv_read_slots = torch.where(logged_before, before_slots, work)
        conv_read_granules = torch.where(logged_before, before_granules, 0).to(torch.int32)

        gran = pool.layout.granularity
        indices = PackedLinearIndices.from_lengths(lengths, pool.storage.device, gran)
        cm = batch.cache_metadata
        first = cm.first_offsets
        if first is None:  # read back from the device (a sync, as in the reference)
            first = offsets.index_select(0, indices.cu_seqlens[:-1]).tolist()
        plan = _upload(logstate_prefill_plan(lengths, cached, first, cm.checkpoint_writes, cm.checkpoint_ranges,
                                             gran, pool.layout.num_granules,
                                             lambda s: pool.allocator.slot(s).kind == "work"),
                       pool.storage.device)
        T = int(lengths.sum())
        log_writes, conv_slots, conv_granules = make_logstate_prefill_writes(logs, offsets, plan, gran)
        return LogStateLinearAttnMetadata(
            phase=batch.phase, work_slots=work, log_slots=logs, token_offsets=offsets,
            conv_read_slots=conv_read_slots, conv_read_granules=conv_read_granules,
            replay_counts=torch.empty(0, dtype=torch.int32, device=pool.storage.device),
            cu_seqlens=indices.cu_seqlens, prefill_indices=indices, chunk_write_slots=plan[3 * T:],
            log_write_slots=log_writes, conv_token_slots=conv_slots, conv_token_granules=conv_granules)

    # ------------------------------------------------------------ decode graphs
    def init_capture_graph(self, max_seq_len: int, bs_list: list[int]) -> None:
        del max_seq_len
        assert self.capture is None, "Capture already initialized."
        self.capture_bs = sorted(bs_list)
        self.capture = LogStateLinearAttnCaptureData.make(max(bs_list), self.ctx.linear_state.storage.device)

    def _refresh_capture(self, metadata: LogStateLinearAttnMetadata, bs: int) -> LogStateLinearAttnMetadata:
        """The six decode fields of ``metadata`` into the first ``bs`` capture
        entries (one launch); returns the metadata that reads them."""
        assert self.capture is not None and bs in self.capture_bs
        assert isinstance(metadata, LogStateLinearAttnMetadata)
        target = self.capture.view(bs)
        copy_metadata([getattr(metadata, f).to(torch.int32) for f in _DECODE_FIELDS],
                      [getattr(target, f) for f in _DECODE_FIELDS])
        return target

    def prepare_for_capture(self, batch) -> None:
        """logstate.py:285-292."""
        self.prepare_metadata(batch)
        batch.linear_attn_metadata = self._refresh_capture(batch.linear_attn_metadata, batch.size)

    def prepare_for_replay(self, batch) -> None:
        """logstate.py:294-299."""
        self._refresh_capture(batch.linear_attn_metadata, batch.padded_size)

    # ------------------------------------------------------------ forward
    def forward(self, mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, batch, out=None):
        """gdn_logstate.py:19-59."""
        metadata = batch.linear_attn_metadata
        assert isinstance(metadata, LogStateLinearAttnMetadata) and metadata.phase == batch.phase
        if batch.is_verify:
            raise NotImplementedError("LogState speculative verify is not implemented yet.")
        run = self._prefill if batch.is_prefill else self._decode
        return run(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, metadata, out)

    def _sequence_index(self, n: int, device) -> torch.Tensor:
        """0..n-1 (int32) on ``device``, from a cached vector."""
        ids = self._sequence_ids
        if ids is None or ids.numel() < n or ids.device != torch.device(device):
            ids = self._sequence_ids = torch.arange(max(n, 64), dtype=torch.int32, device=device)
        return ids[:n]

    def _prefill(self, mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, m, out=None):
        pool = self.ctx.linear_state
        layout, layer = pool.layout, config.layer_idx
        assert m.prefill_indices is not None and m.chunk_write_slots is not None
        assert m.conv_token_slots is not None and m.conv_token_granules is not None and m.log_write_slots is not None
        frames16 = pool.storage.view(pool.dtype)
        cu = m.cu_seqlens
        assert cu is not None
        history = pool.read_conv(m.conv_read_slots, m.conv_read_granules, layer).contiguous()
        # conv + SiLU + split + prepare_gdn in one pass, the history read as a pool of one slot per sequence
        q, k, v, g, b = prefill_frontend(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config,
                                         history.unsqueeze(1), cu,
                                         self._sequence_index(history.shape[0], history.device), layer=0)
        conv_windows_logstate(
            mixed_qkv, history, cu,
            PackedConvStateIO(storage=frames16, slots=m.conv_token_slots, granules=m.conv_token_granules,
                              final_slots=m.work_slots, frame_table=pool.conv_frame_table,
                              frame_bytes=pool.frame_bytes, layer=layer),
            conv_weight.shape[-1])
        states = ChunkStateIO(storage=frames16, read_slots=m.work_slots, chunk_write_slots=m.chunk_write_slots,
                              final_write_slots=m.work_slots, payload_frames=pool.payload_frame_table,
                              frame_bytes=pool.frame_bytes, head_payload_bytes=pool.head_payload_bytes, layer=layer,
                              num_layers=layout.num_linear_layers, granularity=layout.granularity,
                              page_size=pool.page_size)
        log = ChunkLogIO(slots=m.log_write_slots, token_offsets=m.token_offsets, decay_frames=pool.decay_frame_table,
                         gate=g, page_size=pool.page_size, decay_record_bytes=layout.log_decay_bytes,
                         num_key_heads=layout.num_key_heads)
        o, _ = chunk_gated_delta_rule_to_cache(q, k, v, g, b, states, cu, chunk_size=layout.granularity,
                                               log_io=log, out=None if out is None else out.unsqueeze(0),
                                               return_v_new=False)
        return o.squeeze(0)

    def _decode(self, mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, m, out=None):
        pool = self.ctx.linear_state
        q, k, v = conv_decode(mixed_qkv, conv_weight, config, split_qkv=True, read_slots=m.conv_read_slots,
                              read_granules=m.conv_read_granules, write_slots=m.log_slots,
                              write_granules=m.token_offsets // pool.layout.granularity, work_slots=m.work_slots,
                              pool=pool)
        o = fused_recurrent_gated_delta_rule_to_logstate(
            q, k, v, gate.unsqueeze(1), beta.unsqueeze(1), A_log, dt_bias, pool, m.work_slots, m.log_slots,
            m.token_offsets, config.layer_idx, m.replay_counts, enable_eager_state=self.enable_eager_state,
            out=None if out is None else out.unsqueeze(1))
        return o.squeeze(1)


__all__ = ["GatedDeltaLogStateBackend", "LogStateLinearAttnCaptureData", "LogStateLinearAttnMetadata",
           "logstate_prefill_plan"]
