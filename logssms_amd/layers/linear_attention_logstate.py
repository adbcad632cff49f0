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
Building the metadata is the LogState cache manager's work (its page and
work-slot tables); the backend takes it from ``batch.linear_attn_metadata``.
Speculative verify raises ``NotImplementedError``, as in the reference.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ..core import get_global_ctx
from ..kernel.fused import prepare_gdn
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

    # ------------------------------------------------------------ decode graphs
    def init_capture_graph(self, max_seq_len: int, bs_list: list[int]) -> None:
        del max_seq_len
        self.capture_bs = sorted(bs_list)
        self.capture = LogStateLinearAttnCaptureData.make(max(bs_list), self.ctx.linear_state.storage.device)

    def prepare_for_capture(self, batch) -> None:
        """The captured decode reads the capture buffers (their first
        ``batch.size`` entries)."""
        assert self.capture is not None and batch.is_decode
        bs = batch.size
        cap = self.capture
        batch.linear_attn_metadata = LogStateLinearAttnMetadata(
            phase="decode", **{name: getattr(cap, name)[:bs] for name in _CAPTURED})

    def prepare_for_replay(self, batch) -> None:
        """Copies the fresh metadata of ``batch`` into the capture buffers
        (padding entries keep what they held)."""
        assert self.capture is not None
        metadata = batch.linear_attn_metadata
        for name in _CAPTURED:
            src = getattr(metadata, name)
            getattr(self.capture, name)[:src.shape[0]].copy_(src)

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
