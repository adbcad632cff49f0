"""LogState slot-state construction and log stores (drop-in for
``python/logssms/kernel/linear_attention/logstate.py``):

* ``restore_log_state_chains`` -- states rebuilt from a base state and logged
  token segments (``logstate.py:59-88``, ``gdn_logstate_restore``);
* ``store_log_states`` -- token log rows and gates (``logstate.py:91-115``,
  ``gdn_store_chunk_log``);
* ``copy_states`` -- whole slot states (``logstate.py:118-128``,
  ``gdn_logstate_copy_states``).

``pool`` provides what ``cache/logstate/frame_pool.py``'s pool does:
``storage`` (uint8 frames), ``dtype``, ``frame_bytes``, ``head_payload_bytes``,
``page_size``, ``payload_frame_table``, ``decay_frame_table`` and ``layout``
(``num_linear_layers``, ``num_value_heads``, ``num_key_heads``,
``head_k_dim``, ``head_v_dim``, ``granularity``, ``log_decay_bytes``).
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from ... import _lib


def _vectors(groups, device) -> list[torch.Tensor]:
    """The int32 vectors of ``groups`` on ``device`` from one packed host
    copy (one transfer instead of one per vector)."""
    sizes = [len(g) for g in groups]
    host = torch.tensor([v for g in groups for v in g], dtype=torch.int32)
    if torch.device(device).type == "cuda":
        host = host.pin_memory()
    return list(host.to(device, non_blocking=True).split(sizes))


def _common(pool):
    storage = pool.storage
    frames = pool.payload_frame_table.contiguous()
    assert storage.is_contiguous()
    num_frames = storage.numel() * storage.element_size() // pool.frame_bytes
    return storage, frames, num_frames


def restore_log_state_chains(pool, chains: Sequence[tuple[int | None, Sequence[tuple[int, int, int]], int]]) -> None:
    """For each ``(base, segments, output)``: the state of slot ``base``
    (zero for None), then the logged tokens ``begin .. end - 1`` of each
    ``(log_slot, begin, end)`` segment in order, ``S <- e^g S + k v'^T``,
    written to slot ``output`` for every layer and value head."""
    if not chains:
        return
    allocator = getattr(pool, "allocator", None)
    if allocator is not None and hasattr(allocator, "slot"):
        assert all(allocator.slot(output).kind != "log" for _base, _logs, output in chains), "State output required"
    storage, frames, num_frames = _common(pool)
    layout = pool.layout
    segments = [entry for _base, logs, _out in chains for entry in logs]
    offsets = [0]
    for _base, logs, _out in chains:
        offsets.append(offsets[-1] + len(logs))
    base, seg_offsets, seg_slots, seg_begin, seg_end, outputs = _vectors([
        [-1 if b is None else b for b, _logs, _out in chains],
        offsets,
        [slot for slot, _b, _e in segments] or [0],
        [b for _s, b, _e in segments] or [0],
        [e for _s, _b, e in segments] or [0],
        [out for _b, _logs, out in chains],
    ], storage.device)
    decay = pool.decay_frame_table.contiguous()
    _lib.call(
        "gdn_logstate_restore",
        storage.data_ptr(), frames.data_ptr(), _lib.index_code(frames), min(frames.shape[0], decay.shape[0]),
        frames.shape[1], pool.frame_bytes,
        pool.head_payload_bytes, num_frames, decay.data_ptr(), _lib.index_code(decay), layout.log_decay_bytes,
        layout.num_linear_layers, layout.num_value_heads, layout.num_key_heads, layout.head_k_dim,
        layout.head_v_dim, layout.granularity, pool.page_size, _lib.dtype_code(pool.dtype),
        base.data_ptr(), seg_offsets.data_ptr(), seg_slots.data_ptr(), seg_begin.data_ptr(), seg_end.data_ptr(),
        outputs.data_ptr(), len(chains), _lib.stream_of(storage),
    )


def store_log_states(pool, slots: torch.Tensor, token_offsets: torch.Tensor, keys: torch.Tensor,
                     residual_values: torch.Tensor, decays: torch.Tensor, layer: int) -> None:
    """Token ``t``'s residual ``residual_values[t, h]``, key (``keys[t]``
    holds one row per value head or per key head) and gate ``decays[t, h]``
    into the log at ``token_offsets[t]`` of ``slots[t]`` (``slots[t] < 0``:
    none)."""
    if len(slots) == 0:
        return
    storage, frames, num_frames = _common(pool)
    assert keys.is_cuda and keys.device == storage.device
    layout = pool.layout
    T = len(slots)
    HV, dv = layout.num_value_heads, layout.head_v_dim
    keys = keys.reshape(T, -1, layout.head_k_dim).to(pool.dtype).contiguous()
    residual = residual_values.reshape(T, HV, dv).to(pool.dtype).contiguous()
    gates = decays.float().reshape(T, HV).contiguous()
    decay = pool.decay_frame_table.contiguous()
    _lib.call(
        "gdn_store_chunk_log",
        storage.data_ptr(), frames.data_ptr(), _lib.index_code(frames), min(frames.shape[0], decay.shape[0]),
        frames.shape[1], pool.frame_bytes,
        num_frames, slots.contiguous().data_ptr(), _lib.index_code(slots), token_offsets.contiguous().data_ptr(),
        _lib.index_code(token_offsets), T, residual.data_ptr(), keys.data_ptr(), keys.shape[1], HV,
        layout.head_k_dim, dv, layout.num_key_heads, gates.data_ptr(), decay.data_ptr(), _lib.index_code(decay),
        layout.log_decay_bytes, layer, layout.num_linear_layers, layout.granularity, pool.page_size,
        _lib.stream_of(storage),
    )


def copy_states(pool, sources: Sequence[int], destinations: Sequence[int]) -> None:
    """The state of every layer and value head of ``sources[i]`` to
    ``destinations[i]``."""
    if not sources:
        return
    assert len(sources) == len(destinations)
    storage, frames, num_frames = _common(pool)
    layout = pool.layout
    src, dst = _vectors([list(sources), list(destinations)], storage.device)
    _lib.call(
        "gdn_logstate_copy_states",
        storage.data_ptr(), frames.data_ptr(), _lib.index_code(frames), frames.shape[0], frames.shape[1],
        pool.frame_bytes,
        pool.head_payload_bytes, num_frames, layout.num_linear_layers, layout.num_value_heads, layout.head_k_dim,
        layout.head_v_dim, _lib.dtype_code(pool.dtype), src.data_ptr(), dst.data_ptr(), len(src),
        _lib.stream_of(storage),
    )


__all__ = ["copy_states", "restore_log_state_chains", "store_log_states"]
