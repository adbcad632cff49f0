"""``GatedDeltaBackend`` and its host metadata -- drop-in for the reference's
``python/logssms/layers/linear_attention_backend/{standard,gdn}.py``.

Host side (integers, bit-exact with the reference):
  * ``PackedLinearIndices.from_lengths`` (standard.py:42-73)
  * ``GatedDeltaBackend.prepare_metadata`` prefill / decode / verify branches
    (standard.py:112-250): baseline slots, checkpoint placement, chunk write
    slots, conv snapshot rows, decode read/write slots, verify length groups
  * decode graph capture buffers (standard.py:85-97, 252-281)
Device side, one fused gfx950 pass per phase (``kernel.linear_attention.fused_backend``):
  * prefill: front end (conv history gather + packed conv + snapshots + split +
    prepare) then the chunked rule with pool I/O (gdn.py:74-149)
  * decode: conv + recurrent step in one kernel (gdn.py:222-265)
  * verify: per length group, conv + T recurrent steps with per-step conv
    windows and states written straight to the reserve slots (gdn.py:151-220)

Like the reference, the backend reads the pool and slot tables from the
process-global context (``logssms_amd.core.set_global_ctx``) unless one is
bound at construction (``Context.linear_attn_backend`` binds its own).
"""

from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np
import torch

from ..core import MarconiCacheMetadata, get_global_ctx
from ..kernel.linear_attention.fused_backend import decode_step, prefill_frontend, prefill_fused, verify_group
from ..kernel.linear_attention.gdn import chunk_gated_delta_rule_to_cache
from ..kernel.linear_attention.state_io import ChunkStateIO
from ..kernel.metadata import gather_linear_slots


@dataclass
class LinearAttnMetadata:
    """standard.py:16-31."""

    phase: str
    slots: torch.Tensor | None = None
    read_slots: torch.Tensor | None = None
    write_slots: torch.Tensor | None = None
    verify_groups: dict[int, tuple[torch.Tensor, torch.Tensor, torch.Tensor]] | None = None
    prefill_indices: "PackedLinearIndices | None" = None
    baseline_slots: torch.Tensor | None = None
    checkpoint_slots: torch.Tensor | None = None
    checkpoint_chunks: torch.Tensor | None = None
    chunk_write_slots: torch.Tensor | None = None
    snapshot_rows: torch.Tensor | None = None
    snapshot_reqs: torch.Tensor | None = None
    conv_token_slots: torch.Tensor | None = None


@dataclass
class PackedLinearIndices:
    """standard.py:34-73."""

    cu_seqlens: torch.Tensor
    chunk_indices: torch.Tensor
    chunk_offsets: torch.Tensor
    endings: torch.Tensor
    conv_chunks: torch.Tensor

    @classmethod
    def from_lengths(cls, lengths, device, chunk_size: int) -> "PackedLinearIndices":
        lens = np.asarray(lengths, dtype=np.int64)
        assert (lens > 0).all()
        n_chunks = (lens + chunk_size - 1) // chunk_size
        n_conv = (lens + 63) // 64
        offsets = np.concatenate([[0], np.cumsum(lens)])
        chunk_offsets = np.concatenate([[0], np.cumsum(n_chunks)])
        endings = chunk_offsets[1:] - 1

        def pairs(counts):
            req = np.repeat(np.arange(len(counts), dtype=np.int64), counts)
            starts = np.repeat(np.concatenate([[0], np.cumsum(counts)[:-1]]), counts)
            return np.stack([req, np.arange(req.size, dtype=np.int64) - starts], 1)

        vectors = [offsets, pairs(n_chunks).ravel(), chunk_offsets, endings, pairs(n_conv).ravel()]
        sizes = [v.size for v in vectors]
        device = torch.device(device)
        host = torch.from_numpy(np.concatenate(vectors))
        if device.type == "cuda":
            host = host.pin_memory()
        packet = host.to(device, non_blocking=device.type == "cuda")
        cu, chunks, chunk_offs, ends, conv = packet.split(sizes)
        return cls(cu_seqlens=cu, chunk_indices=chunks.view(-1, 2), chunk_offsets=chunk_offs, endings=ends,
                   conv_chunks=conv.view(-1, 2))

    def fla_kwargs(self) -> dict[str, torch.Tensor]:
        return {"chunk_indices": self.chunk_indices, "chunk_offsets": self.chunk_offsets}


@dataclass
class LinearAttnCaptureData:
    """standard.py:76-97."""

    slots: torch.Tensor

    @property
    def read_slots(self) -> torch.Tensor:
        return self.slots[:, 0]

    @property
    def write_slots(self) -> torch.Tensor:
        return self.slots[:, 1]

    @classmethod
    def make(cls, max_bs: int, device) -> "LinearAttnCaptureData":
        return cls(slots=torch.zeros(max_bs, 2, dtype=torch.int64, device=device))


def _gather(table: torch.Tensor, rows, cols) -> torch.Tensor:
    r = torch.as_tensor(np.asarray(rows, dtype=np.int64), device=table.device)
    c = torch.as_tensor(np.asarray(cols, dtype=np.int64), device=table.device)
    return table[r, c].to(torch.int64)


class MixedForward:
    """``forward_mixed`` of the reference's ``BaseLinearAttnBackend``
    (``base.py:20-42``) for the GDN backends here: a mixed batch's prefill
    part (its first ``prefill_token_capacity`` rows, or the prefill tokens)
    and decode part (the remaining rows), each through ``forward`` into slices
    of one output."""

    def forward_mixed(self, batch, token_inputs: dict[str, torch.Tensor], **kwargs) -> torch.Tensor:
        assert batch.mixed_parts is not None
        split = batch.prefill_token_capacity or batch.prefill_tokens
        example = next(iter(token_inputs.values()))
        config = kwargs["config"]
        output = torch.empty(len(example), config.num_v_heads, config.head_v_dim, dtype=example.dtype,
                             device=example.device)
        for part, begin, end in ((batch.mixed_parts[0], 0, split), (batch.mixed_parts[1], split, len(example))):
            self.forward(**{name: tensor[begin:end] for name, tensor in token_inputs.items()}, **kwargs,
                         batch=part, out=output[begin:end])
        return output


class GatedDeltaBackend(MixedForward):
    def __init__(self, ctx=None) -> None:
        self._ctx = ctx
        self.capture: LinearAttnCaptureData | None = None
        self.capture_bs: list[int] = []

    @property
    def ctx(self):
        return self._ctx if self._ctx is not None else get_global_ctx()

    # ------------------------------------------------------------ metadata
    def prepare_metadata(self, batch) -> None:
        ctx = self.ctx
        state_table = ctx.state_table
        assert state_table is not None
        metadata = LinearAttnMetadata(phase=batch.phase)
        if batch.is_decode:
            packet = batch.prepared_indices
            if packet is not None and state_table.is_cuda:
                # standard.py:114-117: the engine's packet, gathered on the device
                metadata.slots = gather_linear_slots(packet, state_table)
            else:
                reqs = batch.padded_reqs
                t = [r.table_idx for r in reqs]
                c = np.asarray([r.cached_len for r in reqs], dtype=np.int64)
                # cached_len - 1 = -1 wraps to the row's last entry, as torch indexing does
                read = _gather(state_table, t, np.where(c - 1 < 0, c - 1 + state_table.shape[1], c - 1))
                write = _gather(state_table, t, c)
                metadata.slots = torch.stack([read, write], 1)
            metadata.read_slots = metadata.slots[:, 0]
            metadata.write_slots = metadata.slots[:, 1]
        elif batch.is_prefill:
            self._prefill_metadata(batch, metadata)
        elif batch.is_verify:
            self._verify_metadata(batch, metadata)
        batch.linear_attn_metadata = metadata

    def _prefill_metadata(self, batch, metadata) -> None:
        ctx = self.ctx
        state_table = ctx.state_table
        dev = state_table.device
        page = ctx.page_size
        assert page % 64 == 0
        reqs = batch.reqs
        lengths = np.asarray([r.extend_len for r in reqs], dtype=np.int64)
        cached = np.asarray([r.cached_len for r in reqs], dtype=np.int64)
        tables = np.asarray([r.table_idx for r in reqs], dtype=np.int64)
        metadata.prefill_indices = PackedLinearIndices.from_lengths(lengths, dev, 64)
        prev = cached - 1
        base = _gather(state_table, tables, np.maximum(prev, 0))
        metadata.baseline_slots = torch.where(torch.as_tensor(prev >= 0, device=dev), base, -1)
        sparse = (batch.cache_metadata.checkpoint_writes
                  if isinstance(batch.cache_metadata, MarconiCacheMetadata) else None)
        grouped = hasattr(ctx.linear_state, "group_table")
        ends_per_req, explicit = [], []
        for i, r in enumerate(reqs):
            ext = int(lengths[i])
            if sparse is None and grouped:
                ends = np.asarray([ext], dtype=np.int64)
            elif sparse is None:
                assert cached[i] % 64 == 0
                ends = np.append(np.arange(page, ext, page, dtype=np.int64), ext)
            else:
                ends = np.asarray([e for e, _ in sparse[i]], dtype=np.int64)
                explicit.extend(s for _, s in sparse[i])
                assert all(e == ext or e % 64 == 0 for e in ends.tolist())
            ends_per_req.append(ends)
        counts = np.asarray([e.size for e in ends_per_req], dtype=np.int64)
        all_ends = np.concatenate(ends_per_req) if ends_per_req else np.zeros(0, np.int64)
        req_of = np.repeat(np.arange(len(reqs), dtype=np.int64), counts)
        chunk_off = np.concatenate([[0], np.cumsum((lengths + 63) // 64)])
        tok_off = np.concatenate([[0], np.cumsum(lengths)])
        if sparse is None:
            metadata.checkpoint_slots = _gather(state_table, tables[req_of], cached[req_of] + all_ends - 1)
        else:
            metadata.checkpoint_slots = torch.tensor(explicit, dtype=torch.int64, device=dev)
        metadata.checkpoint_chunks = torch.as_tensor(chunk_off[req_of] + (all_ends - 1) // 64, device=dev)
        metadata.chunk_write_slots = torch.full((int(chunk_off[-1]),), -1, dtype=torch.int64, device=dev)
        metadata.chunk_write_slots.index_copy_(0, metadata.checkpoint_chunks, metadata.checkpoint_slots)
        metadata.snapshot_rows = torch.as_tensor(tok_off[req_of] + all_ends - 1, device=dev)
        metadata.snapshot_reqs = torch.as_tensor(req_of, device=dev)
        metadata.conv_token_slots = torch.full((int(tok_off[-1]),), -1, dtype=torch.int64, device=dev)
        metadata.conv_token_slots.index_copy_(0, metadata.snapshot_rows, metadata.checkpoint_slots)

    def _verify_metadata(self, batch, metadata) -> None:
        ctx = self.ctx
        state_table, work = ctx.state_table, ctx.work_state_table
        assert work is not None
        by_len: dict[int, list[tuple[int, int, int]]] = {}
        offset = 0
        for r in batch.reqs:
            by_len.setdefault(r.extend_len, []).append((r.table_idx, r.cached_len - 1, offset))
            offset += r.extend_len
        groups = {}
        dev = state_table.device
        for seq_len, entries in by_len.items():
            starts = np.asarray([s for _, _, s in entries], dtype=np.int64)
            rows = (starts[:, None] + np.arange(seq_len, dtype=np.int64)[None, :]).ravel()
            tables = [t for t, _, _ in entries]
            base = _gather(state_table, tables, [p for _, p, _ in entries])
            writes = work[torch.as_tensor(tables, dtype=torch.int64, device=work.device), :seq_len]
            groups[seq_len] = (torch.as_tensor(rows, device=dev), base, writes)
        metadata.verify_groups = groups

    # ------------------------------------------------------------ decode graph capture
    def init_capture_graph(self, max_seq_len: int, bs_list: list[int]) -> None:
        del max_seq_len
        assert self.capture is None, "Capture already initialized."
        self.capture = LinearAttnCaptureData.make(max(bs_list), self.ctx.linear_state.device)
        self.capture_bs = sorted(bs_list)

    def prepare_for_capture(self, batch) -> None:
        bs = batch.size
        assert self.capture is not None and bs in self.capture_bs
        self.prepare_metadata(batch)
        metadata = batch.linear_attn_metadata
        self.capture.slots[:bs].copy_(metadata.slots)
        batch.linear_attn_metadata = LinearAttnMetadata(
            phase="decode", slots=self.capture.slots[:bs], read_slots=self.capture.read_slots[:bs],
            write_slots=self.capture.write_slots[:bs])

    def prepare_for_replay(self, batch) -> None:
        metadata = batch.linear_attn_metadata
        bs = batch.padded_size
        assert self.capture is not None and bs in self.capture_bs
        self.capture.slots[:bs].copy_(metadata.slots)

    # ------------------------------------------------------------ forward
    def forward(self, mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, batch, out=None):
        """gdn.py:20-49."""
        metadata = batch.linear_attn_metadata
        pool = self.ctx.linear_state
        if hasattr(pool, "group_table"):
            metadata, lane = pool.map_metadata(metadata, config.layer_idx)
            config = replace(config, layer_idx=lane)
        assert metadata.phase == batch.phase
        if metadata.phase == "prefill":
            return self._forward_prefill(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, metadata, out)
        if metadata.phase == "verify":
            return self._forward_verify(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, metadata)
        return self._forward_decode(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, metadata, out)

    def _forward_prefill(self, mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, metadata, out=None):
        pool = self.ctx.linear_state
        idx = metadata.prefill_indices
        o = prefill_fused(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, pool.conv_state,
                          pool.recurrent_state, idx.cu_seqlens, metadata.baseline_slots, metadata.chunk_write_slots,
                          metadata.snapshot_rows, metadata.checkpoint_slots, out=out)
        if o is not None:
            return o
        q, k, v, g, b = prefill_frontend(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, pool.conv_state,
                                         idx.cu_seqlens, metadata.baseline_slots, metadata.snapshot_rows,
                                         metadata.checkpoint_slots)
        io = ChunkStateIO(storage=pool.recurrent_state, read_slots=metadata.baseline_slots,
                          chunk_write_slots=metadata.chunk_write_slots, layer=config.layer_idx)
        o, _ = chunk_gated_delta_rule_to_cache(q, k, v, g, b, io, idx.cu_seqlens, out=None if out is None else
                                               out.unsqueeze(0), return_v_new=False)
        return o.squeeze(0)

    def _forward_decode(self, mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, metadata, out=None):
        pool = self.ctx.linear_state
        return decode_step(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, pool.conv_state,
                           pool.recurrent_state, metadata.read_slots, metadata.write_slots, out=out)

    def _forward_verify(self, mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, metadata):
        pool = self.ctx.linear_state
        output = torch.empty(mixed_qkv.shape[0], config.num_v_heads, config.head_v_dim, dtype=mixed_qkv.dtype,
                             device=mixed_qkv.device)
        for seq_len, (rows, baseline, writes) in metadata.verify_groups.items():
            verify_group(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, pool.conv_state,
                         pool.recurrent_state, rows, baseline, writes.to(torch.int64), output)
        return output


__all__ = ["GatedDeltaBackend", "LinearAttnCaptureData", "LinearAttnMetadata", "MixedForward", "PackedLinearIndices"]
