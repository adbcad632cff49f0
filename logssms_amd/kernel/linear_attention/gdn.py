"""Gated delta rule operators (drop-in for the reference's vendored FLA entry
points, ``python/logssms/kernel/linear_attention/vendor/fla/__init__.py``):

* ``chunk_gated_delta_rule_to_cache``  -- ``vendor/fla/gated_delta.py:15-82``
* ``fused_recurrent_gated_delta_rule_to_slots`` -- ``vendor/fla/fused_recurrent.py:396-458``
* ``fused_recurrent_gated_delta_rule`` -- ``vendor/fla/fused_recurrent.py:461-550``

All run one hand-written gfx950 kernel each (``libgdn_mi355x.so``).
"""

from __future__ import annotations

import torch

from ... import _lib
from .state_io import ChunkLogIO, ChunkStateIO


def _check_state_storage(storage: torch.Tensor, hv: int, dk: int, dv: int) -> None:
    assert storage.ndim == 5 and tuple(storage.shape[2:]) == (hv, dk, dv), storage.shape
    assert storage.stride(4) == 1 and storage.stride(3) == dv, "state rows must be contiguous"


@torch.compiler.disable
def chunk_gated_delta_rule_to_cache(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    gate: torch.Tensor,
    beta: torch.Tensor,
    state_io: ChunkStateIO,
    cu_seqlens: torch.Tensor,
    chunk_size: int = 64,
    chunk_indices: torch.Tensor | None = None,
    chunk_offsets: torch.Tensor | None = None,
    *,
    log_io: ChunkLogIO | None = None,
    out: torch.Tensor | None = None,
    return_v_new: bool = True,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Chunked gated delta rule over packed sequences with pool I/O
    (``gated_delta.py:15-82``): initial state of sequence n from
    ``storage[read_slots[n], layer]`` (zero if negative), checkpoint states to
    ``storage[chunk_write_slots[c], layer]`` for every ``chunk_size``-token
    interval ``c`` (global numbering, the last interval of a sequence possibly
    shorter) with a non-negative slot, optional final states to
    ``final_write_slots``.  With ``state_io.payload_frames`` the same states
    live in the LogState frame storage (``state_io.py:42-80``).  ``gate`` is
    the natural-log decay and ``beta`` the prepared write strength
    (``prepare_gdn`` outputs).  Returns ``(o, v_new)``; ``v_new`` is
    ``u - w h`` (None when ``return_v_new=False``).

    The kernel always solves 64-token chunks; ``chunk_size`` 16 or 32 sets
    where checkpoints are taken (the results do not depend on it beyond
    rounding).  ``chunk_indices``/``chunk_offsets`` are accepted for signature
    compatibility (the kernel derives interval boundaries from
    ``cu_seqlens``).  With ``log_io`` (frame storage only) every logged
    token's v' rows, key rows and gates then go into its log slot
    (``state_io.py:83-126``, ``gdn_store_chunk_log``).  With
    ``return_v_new=False`` as well, the chunk kernel writes the v' rows into
    the log itself (``gdn_chunk_gated_delta_rule_logged``; v' never makes an
    HBM round trip) and ``v_new`` is None.
    """
    del chunk_offsets
    assert query.shape[0] == key.shape[0] == value.shape[0] == 1
    assert chunk_size in (16, 32, 64)
    assert cu_seqlens.ndim == 1
    assert len(cu_seqlens) == len(state_io.read_slots) + 1
    _, T, H, dk = query.shape
    HV, dv = value.shape[2:]
    assert key.shape == query.shape and value.shape[:2] == query.shape[:2]
    assert HV % H == 0
    assert gate.shape == beta.shape == (1, T, HV)
    storage = state_io.storage
    frames = state_io.payload_frames
    if frames is None:
        _check_state_storage(storage, HV, dk, dv)
        strides = (storage.stride(0), storage.stride(1), storage.stride(2))
        frame_args = (None, 0, 0, 0, 0, 0, 0)
    else:
        assert storage.ndim == 2 and storage.is_contiguous()
        assert state_io.frame_bytes > 0 and state_io.head_payload_bytes > 0
        assert storage.shape[1] * storage.element_size() == state_io.frame_bytes
        assert frames.ndim == 2 and frames.is_contiguous() and frames.device == storage.device
        strides = (0, 0, 0)
        # slots past the table's rows (and past the decay table's, when logging) are unmapped
        rows = frames.shape[0] if log_io is None else min(frames.shape[0], log_io.decay_frames.shape[0])
        frame_args = (frames, _lib.index_code(frames), rows, frames.shape[1], state_io.frame_bytes,
                      state_io.head_payload_bytes, storage.shape[0])
    if log_io is not None:
        assert frames is not None, "the token log lives in the LogState frame storage"
        assert log_io.slots.shape == log_io.token_offsets.shape == (T,)
        assert log_io.gate.numel() == T * HV and log_io.num_key_heads > 0
        assert H % log_io.num_key_heads == 0 and HV % log_io.num_key_heads == 0
        assert storage.dtype == value.dtype, "log rows are stored in the io dtype"
    if dv != 32 and dv % 64:
        raise NotImplementedError("head_v_dim must be 32 or a multiple of 64 on the MI355X backend")
    assert storage.device == query.device
    if chunk_indices is not None:
        assert state_io.chunk_write_slots.shape == (len(chunk_indices),)
    if state_io.final_write_slots is not None:
        assert state_io.final_write_slots.shape == state_io.read_slots.shape
    query, key, value = query.contiguous(), key.contiguous(), value.contiguous()
    gate = gate.float().contiguous()
    beta = beta.float().contiguous()
    o = torch.empty_like(value) if out is None else out
    assert o.shape == value.shape and o.dtype == value.dtype and o.is_contiguous()
    # v' straight into the log when the caller does not want v_new back
    direct_log = (log_io is not None and not return_v_new and state_io.frame_bytes % (2 * min(dv, 64)) == 0)
    v_new = torch.empty_like(value) if (return_v_new or (log_io is not None and not direct_log)) else None
    if T and direct_log:
        fw = state_io.final_write_slots
        _lib.call(
            "gdn_chunk_gated_delta_rule_logged",
            query.data_ptr(), key.data_ptr(), value.data_ptr(), _lib.dtype_code(value.dtype),
            gate.data_ptr(), beta.data_ptr(), cu_seqlens.data_ptr(), _lib.index_code(cu_seqlens),
            len(cu_seqlens) - 1, T, H, HV, dk, dv,
            storage.data_ptr(), _lib.dtype_code(storage.dtype), state_io.layer,
            state_io.read_slots.data_ptr(), _lib.index_code(state_io.read_slots),
            state_io.chunk_write_slots.data_ptr(), _lib.index_code(state_io.chunk_write_slots),
            _lib.ptr(fw), _lib.index_code(fw) if fw is not None else 0, chunk_size,
            _lib.ptr(frame_args[0]), *frame_args[1:],
            log_io.slots.data_ptr(), _lib.index_code(log_io.slots),
            log_io.token_offsets.data_ptr(), _lib.index_code(log_io.token_offsets),
            log_io.num_key_heads, state_io.num_layers, log_io.page_size,
            o.data_ptr(), float(dk) ** -0.5, _lib.stream_of(query),
        )
    elif T:
        fw = state_io.final_write_slots
        _lib.call(
            "gdn_chunk_gated_delta_rule",
            query.data_ptr(), key.data_ptr(), value.data_ptr(), _lib.dtype_code(value.dtype),
            gate.data_ptr(), beta.data_ptr(), cu_seqlens.data_ptr(), _lib.index_code(cu_seqlens),
            len(cu_seqlens) - 1, T, H, HV, dk, dv,
            storage.data_ptr(), _lib.dtype_code(storage.dtype), *strides, state_io.layer,
            state_io.read_slots.data_ptr(), _lib.index_code(state_io.read_slots),
            state_io.chunk_write_slots.data_ptr(), _lib.index_code(state_io.chunk_write_slots),
            _lib.ptr(fw), _lib.index_code(fw) if fw is not None else 0, chunk_size,
            _lib.ptr(frame_args[0]), *frame_args[1:],
            o.data_ptr(), _lib.ptr(v_new), float(dk) ** -0.5, _lib.stream_of(query),
        )
    if T and log_io is not None:
        log_gate = log_io.gate.float().contiguous()
        _lib.call(
            "gdn_store_chunk_log",
            storage.data_ptr(), frames.data_ptr(), _lib.index_code(frames), frame_args[2], frames.shape[1],
            state_io.frame_bytes, storage.shape[0],
            log_io.slots.data_ptr(), _lib.index_code(log_io.slots),
            log_io.token_offsets.data_ptr(), _lib.index_code(log_io.token_offsets), T,
            _lib.ptr(None if direct_log else v_new), key.data_ptr(), H, HV, dk, dv, log_io.num_key_heads,
            log_gate.data_ptr(), log_io.decay_frames.data_ptr(), _lib.index_code(log_io.decay_frames),
            log_io.decay_record_bytes, state_io.layer, state_io.num_layers, state_io.granularity,
            log_io.page_size, _lib.stream_of(query),
        )
    return o, v_new if return_v_new else None


def _gates(gate: torch.Tensor, beta: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor):
    A_log = A_log.contiguous()
    dt_bias = dt_bias.contiguous()
    return gate, beta, A_log, dt_bias


@torch.compiler.disable
def fused_recurrent_gated_delta_rule_to_slots(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    gate: torch.Tensor,
    beta: torch.Tensor,
    A_log: torch.Tensor,
    dt_bias: torch.Tensor,
    state_pool: torch.Tensor,
    read_slots: torch.Tensor,
    write_slots: torch.Tensor,
    layer: int,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """fused_recurrent.py:396-458: one decode step per sequence with the state
    read from ``state_pool[read_slots[b], layer]`` and written to
    ``state_pool[write_slots[b], layer]`` (in place when equal).  Raw inputs:
    q/k are L2-normalised, ``g = -exp(A_log) softplus(gate + dt_bias)`` and
    ``beta = sigmoid(beta)`` inside the kernel."""
    batch_size, seq_len, num_k_heads, head_k_dim = query.shape
    num_v_heads, head_v_dim = value.shape[2:]
    assert seq_len == 1 and state_pool.ndim == 5
    assert read_slots.shape == write_slots.shape == (batch_size,)
    assert tuple(state_pool.shape[2:]) == (num_v_heads, head_k_dim, head_v_dim)
    assert num_v_heads % num_k_heads == 0
    _check_state_storage(state_pool, num_v_heads, head_k_dim, head_v_dim)
    output = torch.empty_like(value) if out is None else out
    assert output.shape == value.shape and output.dtype == value.dtype and output.is_contiguous()
    if batch_size == 0:
        return output
    query, key, value = query.contiguous(), key.contiguous(), value.contiguous()
    gate, beta, A_log, dt_bias = _gates(gate, beta, A_log, dt_bias)
    _lib.call(
        "gdn_fused_recurrent",
        query.data_ptr(), key.data_ptr(), value.data_ptr(), _lib.dtype_code(value.dtype),
        gate.data_ptr(), gate.stride(0), gate.stride(1), gate.stride(2), _lib.dtype_code(gate.dtype),
        beta.data_ptr(), beta.stride(0), beta.stride(1), beta.stride(2), _lib.dtype_code(beta.dtype),
        A_log.data_ptr(), _lib.dtype_code(A_log.dtype), dt_bias.data_ptr(), _lib.dtype_code(dt_bias.dtype),
        batch_size, 1, num_k_heads, num_v_heads, head_k_dim, head_v_dim,
        state_pool.data_ptr(), _lib.dtype_code(state_pool.dtype), state_pool.stride(0), state_pool.stride(1),
        state_pool.stride(2), int(layer),
        read_slots.data_ptr(), read_slots.stride(0), _lib.index_code(read_slots),
        write_slots.data_ptr(), write_slots.stride(0), 0, _lib.index_code(write_slots),
        None, None, output.data_ptr(), float(head_k_dim) ** -0.5, _lib.stream_of(query),
    )
    return output


@torch.compiler.disable
def fused_recurrent_gated_delta_rule(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    gate: torch.Tensor,
    beta: torch.Tensor,
    A_log: torch.Tensor,
    dt_bias: torch.Tensor,
    initial_state: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """fused_recurrent.py:461-550: T recurrent steps from ``initial_state``
    [B, HV, dk, dv]; returns ``(o [B, T, HV, dv], states [B, T, HV, dk, dv])``
    with every per-step state kept (the reference verify path)."""
    assert query.is_cuda and key.is_cuda and value.is_cuda
    assert query.ndim == key.ndim == value.ndim == 4
    batch_size, seq_len, num_k_heads, head_k_dim = query.shape
    num_v_heads, head_v_dim = value.shape[2:]
    assert key.shape == query.shape
    assert value.shape[:2] == (batch_size, seq_len)
    assert num_v_heads % num_k_heads == 0
    assert gate.shape == beta.shape == (batch_size, seq_len, num_v_heads)
    assert initial_state.shape == (batch_size, num_v_heads, head_k_dim, head_v_dim)
    query, key, value = query.contiguous(), key.contiguous(), value.contiguous()
    initial_state = initial_state.contiguous()
    output = torch.empty_like(value)
    states = torch.empty(batch_size, seq_len, num_v_heads, head_k_dim, head_v_dim,
                         dtype=initial_state.dtype, device=initial_state.device)
    if batch_size == 0 or seq_len == 0:
        return output, states
    gate, beta, A_log, dt_bias = _gates(gate, beta, A_log, dt_bias)
    _lib.call(
        "gdn_fused_recurrent",
        query.data_ptr(), key.data_ptr(), value.data_ptr(), _lib.dtype_code(value.dtype),
        gate.data_ptr(), gate.stride(0), gate.stride(1), gate.stride(2), _lib.dtype_code(gate.dtype),
        beta.data_ptr(), beta.stride(0), beta.stride(1), beta.stride(2), _lib.dtype_code(beta.dtype),
        A_log.data_ptr(), _lib.dtype_code(A_log.dtype), dt_bias.data_ptr(), _lib.dtype_code(dt_bias.dtype),
        batch_size, seq_len, num_k_heads, num_v_heads, head_k_dim, head_v_dim,
        None, _lib.dtype_code(initial_state.dtype), 0, 0, 0, 0,
        None, 0, 0, None, 0, 0, 0,
        initial_state.data_ptr(), states.data_ptr(), output.data_ptr(), float(head_k_dim) ** -0.5,
        _lib.stream_of(query),
    )
    return output, states


@torch.compiler.disable
def fused_recurrent_gated_delta_rule_to_logstate(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    gate: torch.Tensor,
    beta: torch.Tensor,
    A_log: torch.Tensor,
    dt_bias: torch.Tensor,
    pool,
    work_slots: torch.Tensor,
    log_slots: torch.Tensor,
    token_offsets: torch.Tensor,
    layer: int,
    replay_counts: torch.Tensor,
    enable_eager_state: bool = False,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """fused_recurrent.py:292-394: one LogState decode step per sequence.
    The state is the work slot's state in the pool's frame storage plus,
    unless ``enable_eager_state``, the ``replay_counts[b]`` (<= 16) tokens
    logged since it, replayed from the log (``gdn_replay.py:17-148``); the
    step's v' row, key row and gate go into the log at ``token_offsets[b]`` of
    ``log_slots[b]``; the new state goes to the work slot every step (eager) or
    at the end of each 16-token replay window.  Raw inputs as
    ``fused_recurrent_gated_delta_rule_to_slots``.  ``pool`` carries
    ``storage``, ``payload_frame_table``, ``decay_frame_table``,
    ``frame_bytes``, ``head_payload_bytes``, ``page_size`` and ``layout``
    (``head_k_dim``, ``head_v_dim``, ``num_value_heads``,
    ``num_linear_layers``, ``granularity``, ``log_decay_bytes``), as
    ``cache/logstate/frame_pool.py``'s pool does."""
    batch_size, seq_len, num_k_heads, head_k_dim = query.shape
    num_v_heads, head_v_dim = value.shape[2:]
    layout = pool.layout
    assert seq_len == 1
    assert head_k_dim == layout.head_k_dim and head_v_dim == layout.head_v_dim
    assert num_v_heads == layout.num_value_heads and num_v_heads % num_k_heads == 0
    # the step's key rows go to the log at the prefill's key-head layout
    assert getattr(layout, "num_key_heads", num_k_heads) == num_k_heads, "log key heads != query key heads"
    assert replay_counts.shape == work_slots.shape == log_slots.shape == token_offsets.shape == (batch_size,)
    assert pool.frame_bytes % pool.head_payload_bytes == 0 or pool.head_payload_bytes % pool.frame_bytes == 0
    output = torch.empty_like(value) if out is None else out
    assert output.shape == value.shape and output.dtype == value.dtype and output.is_contiguous()
    if batch_size == 0:
        return output
    storage = pool.storage
    frames = pool.payload_frame_table.contiguous()
    decay = pool.decay_frame_table.contiguous()
    assert storage.is_contiguous() and storage.device == query.device
    num_frames = storage.numel() * storage.element_size() // pool.frame_bytes
    query, key, value = query.contiguous(), key.contiguous(), value.contiguous()
    gate, beta, A_log, dt_bias = _gates(gate, beta, A_log, dt_bias)
    slots = [t.contiguous() for t in (work_slots, log_slots, token_offsets, replay_counts)]
    _lib.call(
        "gdn_recurrent_logstate",
        query.data_ptr(), key.data_ptr(), value.data_ptr(), _lib.dtype_code(value.dtype),
        gate.data_ptr(), gate.stride(0), gate.stride(2), _lib.dtype_code(gate.dtype),
        beta.data_ptr(), beta.stride(0), beta.stride(2), _lib.dtype_code(beta.dtype),
        A_log.data_ptr(), _lib.dtype_code(A_log.dtype), dt_bias.data_ptr(), _lib.dtype_code(dt_bias.dtype),
        batch_size, num_k_heads, num_v_heads, head_k_dim, head_v_dim,
        storage.data_ptr(), frames.data_ptr(), _lib.index_code(frames), min(frames.shape[0], decay.shape[0]),
        frames.shape[1], pool.frame_bytes, pool.head_payload_bytes, num_frames, decay.data_ptr(), _lib.index_code(decay), layout.log_decay_bytes,
        slots[0].data_ptr(), _lib.index_code(slots[0]), slots[1].data_ptr(), _lib.index_code(slots[1]),
        slots[2].data_ptr(), _lib.index_code(slots[2]), slots[3].data_ptr(), _lib.index_code(slots[3]),
        layer, layout.num_linear_layers, layout.granularity, pool.page_size, int(enable_eager_state),
        output.data_ptr(), float(head_k_dim) ** -0.5, _lib.stream_of(query),
    )
    return output


__all__ = [
    "ChunkLogIO",
    "ChunkStateIO",
    "chunk_gated_delta_rule_to_cache",
    "fused_recurrent_gated_delta_rule",
    "fused_recurrent_gated_delta_rule_to_logstate",
    "fused_recurrent_gated_delta_rule_to_slots",
]
