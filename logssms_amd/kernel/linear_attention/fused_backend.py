"""Backend-level fused operators: the three phases of
``GatedDeltaBackend.forward`` (reference
``python/logssms/layers/linear_attention_backend/gdn.py:74-265``) each as the
smallest number of gfx950 kernels.

* ``prefill_fused`` -- the whole prefill (``gdn.py:100-150``): a q/k pass,
  then the chunk kernel computing the v conv + SiLU and the gates in its
  staging waves and writing the conv windows once the histories are read.
* ``prefill_frontend`` -- conv-history gather + packed conv + split +
  ``prepare_gdn`` in one pass over ``mixed_qkv`` (``gdn.py:100-132``), then
  the window snapshots, for shapes outside the fused kernel.
* ``decode_step`` -- ``conv_decode`` + slotted recurrent update in one kernel
  (``gdn.py:222-265``).
* ``verify_group`` -- one verify length group: conv over the drafts, conv
  snapshots and per-step states straight into the write slots, outputs at the
  group's rows (``gdn.py:165-218``; replaces the torch conv, ``index_copy_``
  snapshots, the temporary ``states`` tensor and ``store_state``).
"""

from __future__ import annotations

import torch

from ... import _lib


def _check_pools(conv_state: torch.Tensor, recurrent_state: torch.Tensor | None, config) -> None:
    assert conv_state.ndim == 4 and tuple(conv_state.shape[2:]) == (config.conv_dim, config.state_len)
    assert conv_state.stride(3) == 1 and conv_state.stride(2) == config.state_len
    if recurrent_state is not None:
        assert recurrent_state.ndim == 5
        assert tuple(recurrent_state.shape[2:]) == (config.num_v_heads, config.head_k_dim, config.head_v_dim)
        assert recurrent_state.stride(4) == 1 and recurrent_state.stride(3) == config.head_v_dim


def prefill_frontend(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, conv_state, cu_seqlens,
                     baseline_slots, snapshot_rows=None, snapshot_slots=None, *, layer=None):
    """Returns ``(q [1,T,H,dk], k, v [1,T,HV,dv], g [1,T,HV] fp32, beta fp32)``
    exactly as ``prepare_gdn(split(packed_causal_conv1d(...)))`` would, with
    the conv history read from ``conv_state[baseline_slots, layer]`` (zeros for
    negative slots).  The window of packed row ``snapshot_rows[i]`` then goes
    to ``conv_state[snapshot_slots[i]]`` (negative slots skipped) in a second
    launch, after every history has been read: a window slot may equal a
    baseline slot (a prefill resuming mid-page writes its checkpoint to the
    page it resumed from), and the reference reads all histories before any
    window is written (``gdn.py:107-112`` gathers them with ``index_select``).
    ``layer`` (default ``config.layer_idx``) is the conv pool's layer read."""
    T, C = mixed_qkv.shape
    assert C == config.conv_dim == 2 * config.key_dim + config.value_dim
    assert gate.shape == beta.shape == (T, config.num_v_heads)
    _check_pools(conv_state, None, config)
    if snapshot_rows is not None:
        assert snapshot_slots is not None and snapshot_rows.shape == snapshot_slots.shape and snapshot_rows.ndim == 1
    dev, dt = mixed_qkv.device, mixed_qkv.dtype
    q = torch.empty(1, T, config.num_k_heads, config.head_k_dim, device=dev, dtype=dt)
    k = torch.empty_like(q)
    v = torch.empty(1, T, config.num_v_heads, config.head_v_dim, device=dev, dtype=dt)
    g = torch.empty(1, T, config.num_v_heads, device=dev, dtype=torch.float32)
    b = torch.empty_like(g)
    if T == 0:
        return q, k, v, g, b
    weight = conv_weight.contiguous()
    A_log = A_log.contiguous()
    dt_bias = dt_bias.contiguous()
    _lib.call(
        "gdn_prefill_frontend",
        mixed_qkv.data_ptr(), mixed_qkv.stride(0), mixed_qkv.stride(1), _lib.dtype_code(dt),
        weight.data_ptr(), None, config.state_len + 1, cu_seqlens.data_ptr(), _lib.index_code(cu_seqlens),
        len(cu_seqlens) - 1, T, config.num_k_heads, config.num_v_heads, config.head_k_dim, config.head_v_dim,
        conv_state.data_ptr(), conv_state.stride(0), conv_state.stride(1),
        config.layer_idx if layer is None else layer, baseline_slots.data_ptr(), _lib.index_code(baseline_slots),
        gate.data_ptr(), gate.stride(0), gate.stride(1), _lib.dtype_code(gate.dtype),
        beta.data_ptr(), beta.stride(0), beta.stride(1), _lib.dtype_code(beta.dtype),
        A_log.data_ptr(), _lib.dtype_code(A_log.dtype), dt_bias.data_ptr(), _lib.dtype_code(dt_bias.dtype),
        q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), b.data_ptr(), _lib.stream_of(mixed_qkv),
    )
    if snapshot_rows is not None:
        conv_snapshots(mixed_qkv, config, conv_state, cu_seqlens, baseline_slots, snapshot_rows, snapshot_slots)
    return q, k, v, g, b


def conv_snapshots(mixed_qkv, config, conv_state, cu_seqlens, baseline_slots, rows, slots):
    """``conv_state[slots[i], layer] <- `` the raw conv window ending at packed
    row ``rows[i]`` (history from ``baseline_slots`` before the sequence start;
    negative slots skipped).  16-bit inputs with unit column stride."""
    if not rows.numel():
        return
    assert mixed_qkv.stride(1) == 1 and mixed_qkv.dtype in (torch.bfloat16, torch.float16)
    _lib.call("gdn_conv_snapshots", mixed_qkv.data_ptr(), mixed_qkv.stride(0), _lib.dtype_code(mixed_qkv.dtype),
              cu_seqlens.data_ptr(), _lib.index_code(cu_seqlens), len(cu_seqlens) - 1, mixed_qkv.shape[0],
              mixed_qkv.shape[1], config.state_len + 1, conv_state.data_ptr(), conv_state.stride(0),
              conv_state.stride(1), config.layer_idx, baseline_slots.data_ptr(), _lib.index_code(baseline_slots),
              rows.data_ptr(), _lib.index_code(rows), slots.data_ptr(), _lib.index_code(slots), rows.numel(),
              _lib.stream_of(mixed_qkv))


def _aligned16(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0


def _fused_covered(mixed_qkv, config, conv_state, recurrent_state) -> bool:
    """The shapes ``gdn_prefill_qk`` and ``gdn_prefill_fused`` take (checked
    before the first launch, so an uncovered shape launches nothing and the
    two-step path runs instead): conv width 4, d_k in {32, 64, 128}, d_v a
    multiple of 64, 16-bit io with unit-stride 16-byte-aligned rows (row
    stride below 2^24 elements), a
    16-byte-aligned conv pool whose slot and layer strides keep that
    alignment, and an fp32 or io-typed state pool."""
    return (config.state_len == 3 and config.head_k_dim in (32, 64, 128) and config.head_v_dim % 64 == 0
            and mixed_qkv.dtype in (torch.bfloat16, torch.float16) and mixed_qkv.stride(1) == 1
            and mixed_qkv.stride(0) % 8 == 0 and 0 < mixed_qkv.stride(0) < (1 << 24)
            and _aligned16(mixed_qkv) and _aligned16(conv_state)
            and conv_state.stride(0) % 8 == 0 and conv_state.stride(1) % 8 == 0
            and conv_state.dtype == mixed_qkv.dtype
            and recurrent_state.dtype in (torch.float32, mixed_qkv.dtype))


def prefill_fused(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, conv_state, recurrent_state,
                  cu_seqlens, baseline_slots, chunk_write_slots, snapshot_rows, snapshot_slots, out=None,
                  chunk_events=None):
    """``gdn.py:100-150`` in two launches: the q/k pass writes normalised
    q and k (their conv is shared by all the v heads and d_v slices of a key
    head) and the prepared gates; the chunk kernel's staging waves compute
    the v conv + SiLU of each 64-token chunk from ``mixed_qkv`` (no v round
    trip through HBM), and its side waves write the conv windows of
    ``snapshot_rows`` to ``conv_state[snapshot_slots]`` once their loops
    (and every read of the histories) are done.  Conv history and initial state come
    from ``baseline_slots``; chunk-end states go to ``chunk_write_slots``.
    Results equal ``prefill_frontend`` + ``chunk_gated_delta_rule_to_cache``
    + ``conv_snapshots`` bit for bit.  Returns o [T, HV, dv], or None (nothing launched) when the
    shapes are outside the fused kernel -- conv width 4, d_k in {32, 64, 128},
    d_v % 64 == 0, 16-byte aligned rows, fp32 or io-typed state -- and the
    two-step path has to be used.  ``chunk_events``: optional (start, end)
    ``torch.cuda.Event`` pair recorded around the chunk-kernel launch."""
    T, C = mixed_qkv.shape
    assert C == config.conv_dim == 2 * config.key_dim + config.value_dim
    assert gate.shape == beta.shape == (T, config.num_v_heads)
    _check_pools(conv_state, recurrent_state, config)
    assert snapshot_rows.shape == snapshot_slots.shape and snapshot_rows.ndim == 1
    weight = conv_weight.contiguous()
    if not (_fused_covered(mixed_qkv, config, conv_state, recurrent_state) and _aligned16(weight)):
        return None
    if out is None:
        out = torch.empty(T, config.num_v_heads, config.head_v_dim, device=mixed_qkv.device, dtype=mixed_qkv.dtype)
    assert out.shape == (T, config.num_v_heads, config.head_v_dim) and out.is_contiguous()
    A_log = A_log.contiguous()
    dt_bias = dt_bias.contiguous()
    # q, k as the chunk kernel's f16 MFMA operands; prepared gates
    q = torch.empty(T, config.num_k_heads, config.head_k_dim, device=mixed_qkv.device, dtype=torch.float16)
    k = torch.empty_like(q)
    g = torch.empty(config.num_v_heads, T, device=mixed_qkv.device, dtype=torch.float32)  # head-major
    b = torch.empty_like(g)
    stream = _lib.stream_of(mixed_qkv)
    N = len(cu_seqlens) - 1
    try:
        _lib.call("gdn_prefill_qk", mixed_qkv.data_ptr(), mixed_qkv.stride(0), _lib.dtype_code(mixed_qkv.dtype),
                  weight.data_ptr(), 4, cu_seqlens.data_ptr(), _lib.index_code(cu_seqlens), N, T,
                  config.num_k_heads, config.head_k_dim, conv_state.data_ptr(), conv_state.stride(0),
                  conv_state.stride(1), config.layer_idx, baseline_slots.data_ptr(), _lib.index_code(baseline_slots),
                  q.data_ptr(), k.data_ptr(), _lib.F16_CODE, config.num_v_heads,
                  gate.data_ptr(), gate.stride(0), gate.stride(1), _lib.dtype_code(gate.dtype),
                  beta.data_ptr(), beta.stride(0), beta.stride(1), _lib.dtype_code(beta.dtype),
                  A_log.data_ptr(), _lib.dtype_code(A_log.dtype), dt_bias.data_ptr(), _lib.dtype_code(dt_bias.dtype),
                  g.data_ptr(), b.data_ptr(), stream)
    except NotImplementedError:
        return None
    if chunk_events is not None:
        chunk_events[0].record()
    prefill_chunk_fused(q, k, g, b, mixed_qkv, weight, config, conv_state, recurrent_state, cu_seqlens,
                        baseline_slots, chunk_write_slots, out, snapshot_rows, snapshot_slots)
    if chunk_events is not None:
        chunk_events[1].record()
    return out


def prefill_fused_noalloc(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, conv_state, recurrent_state,
                          cu_seqlens, baseline_slots, chunk_write_slots, snapshot_rows, snapshot_slots, out):
    """``prefill_fused`` through ``gdn_prefill_fused_noalloc``: the same
    two launches, with the q/k operands and prepared gates staged in the
    library's per-GPU device array, so nothing is allocated (``out`` [T, HV,
    dv] is the caller's).  Raises ``RuntimeError`` when T exceeds what the
    array holds and ``NotImplementedError`` for shapes outside the fused
    kernel; calls that overlap on one GPU race on the shared array."""
    T, C = mixed_qkv.shape
    assert C == config.conv_dim == 2 * config.key_dim + config.value_dim
    assert gate.shape == beta.shape == (T, config.num_v_heads)
    _check_pools(conv_state, recurrent_state, config)
    assert snapshot_rows.shape == snapshot_slots.shape and snapshot_rows.ndim == 1
    assert out.shape == (T, config.num_v_heads, config.head_v_dim) and out.is_contiguous()
    assert conv_weight.is_contiguous() and A_log.is_contiguous() and dt_bias.is_contiguous()
    _lib.call(
        "gdn_prefill_fused_noalloc",
        mixed_qkv.data_ptr(), mixed_qkv.stride(0), _lib.dtype_code(mixed_qkv.dtype), conv_weight.data_ptr(),
        config.state_len + 1, cu_seqlens.data_ptr(), _lib.index_code(cu_seqlens), len(cu_seqlens) - 1, T,
        config.num_k_heads, config.num_v_heads, config.head_k_dim, config.head_v_dim,
        conv_state.data_ptr(), conv_state.stride(0), conv_state.stride(1),
        gate.data_ptr(), gate.stride(0), gate.stride(1), _lib.dtype_code(gate.dtype),
        beta.data_ptr(), beta.stride(0), beta.stride(1), _lib.dtype_code(beta.dtype),
        A_log.data_ptr(), _lib.dtype_code(A_log.dtype), dt_bias.data_ptr(), _lib.dtype_code(dt_bias.dtype),
        recurrent_state.data_ptr(), _lib.dtype_code(recurrent_state.dtype), recurrent_state.stride(0),
        recurrent_state.stride(1), recurrent_state.stride(2), config.layer_idx,
        baseline_slots.data_ptr(), _lib.index_code(baseline_slots),
        chunk_write_slots.data_ptr(), _lib.index_code(chunk_write_slots),
        snapshot_rows.data_ptr(), _lib.index_code(snapshot_rows), snapshot_slots.data_ptr(),
        _lib.index_code(snapshot_slots), snapshot_rows.numel(),
        out.data_ptr(), float(config.head_k_dim) ** -0.5, _lib.stream_of(mixed_qkv),
    )
    return out


def prefill_chunk_fused(q, k, g, b, mixed_qkv, weight, config, conv_state, recurrent_state, cu_seqlens,
                        baseline_slots, chunk_write_slots, out, snapshot_rows=None, snapshot_slots=None):
    """The chunk-kernel launch of ``prefill_fused`` (q, k, g, beta from the q/k
    pass, g and beta head-major ``[HV, T]``; v computed from ``mixed_qkv`` inside).
    The conv windows of ``snapshot_rows`` go to ``conv_state[snapshot_slots]``
    in the same launch, after the histories are read (none when omitted)."""
    T = mixed_qkv.shape[0]
    count = 0 if snapshot_rows is None else snapshot_rows.numel()
    if count:
        assert snapshot_slots is not None and snapshot_slots.shape == snapshot_rows.shape
        assert snapshot_rows.is_contiguous() and snapshot_slots.is_contiguous()
    _lib.call(
        "gdn_prefill_fused",
        q.data_ptr(), k.data_ptr(), mixed_qkv.data_ptr(), mixed_qkv.stride(0), _lib.dtype_code(mixed_qkv.dtype),
        weight.data_ptr(), 4, cu_seqlens.data_ptr(), _lib.index_code(cu_seqlens), len(cu_seqlens) - 1, T,
        config.num_k_heads, config.num_v_heads, config.head_k_dim, config.head_v_dim,
        conv_state.data_ptr(), conv_state.stride(0), conv_state.stride(1), g.data_ptr(), b.data_ptr(),
        recurrent_state.data_ptr(), _lib.dtype_code(recurrent_state.dtype), recurrent_state.stride(0),
        recurrent_state.stride(1), recurrent_state.stride(2), config.layer_idx,
        baseline_slots.data_ptr(), _lib.index_code(baseline_slots),
        chunk_write_slots.data_ptr(), _lib.index_code(chunk_write_slots), None, 0,
        snapshot_rows.data_ptr() if count else None, _lib.index_code(snapshot_rows) if count else 0,
        snapshot_slots.data_ptr() if count else None, _lib.index_code(snapshot_slots) if count else 0, count,
        out.data_ptr(), float(config.head_k_dim) ** -0.5, _lib.stream_of(mixed_qkv),
    )
    return out


def _fused(mixed, row_index, gate, beta, conv_weight, A_log, dt_bias, config, conv_state, recurrent_state,
           read_slots, write_slots, batch, steps, write_b, write_t, out):
    weight = conv_weight.contiguous()
    A_log = A_log.contiguous()
    dt_bias = dt_bias.contiguous()
    _lib.call(
        "gdn_fused_conv_recurrent",
        mixed.data_ptr(), mixed.stride(0), mixed.stride(1), _lib.dtype_code(mixed.dtype),
        _lib.ptr(row_index), _lib.index_code(row_index) if row_index is not None else 0,
        weight.data_ptr(), None, config.state_len + 1,
        gate.data_ptr(), gate.stride(0), gate.stride(1), _lib.dtype_code(gate.dtype),
        beta.data_ptr(), beta.stride(0), beta.stride(1), _lib.dtype_code(beta.dtype),
        A_log.data_ptr(), _lib.dtype_code(A_log.dtype), dt_bias.data_ptr(), _lib.dtype_code(dt_bias.dtype),
        batch, steps, config.num_k_heads, config.num_v_heads, config.head_k_dim, config.head_v_dim,
        conv_state.data_ptr(), conv_state.stride(0), conv_state.stride(1),
        recurrent_state.data_ptr(), _lib.dtype_code(recurrent_state.dtype), recurrent_state.stride(0),
        recurrent_state.stride(1), recurrent_state.stride(2), config.layer_idx,
        read_slots.data_ptr(), read_slots.stride(0), _lib.index_code(read_slots),
        write_slots.data_ptr(), write_b, write_t, _lib.index_code(write_slots),
        out.data_ptr(), float(config.head_k_dim) ** -0.5, _lib.stream_of(mixed),
    )


# limits of gdn_fused_conv_recurrent: drafts per launch, v-heads per key head
_MAX_FUSED_STEPS = 16
_MAX_FUSED_GROUP = 4


def _stepwise(mixed, row_index, gate, beta, conv_weight, A_log, dt_bias, config, conv_state, recurrent_state,
              read_slots, write_slots, batch, steps, out):
    """Decode/verify for head groups wider than the fused kernel takes (more
    than 4 v-heads per key head): per step, ``conv_decode`` (split, rounded
    before SiLU for verify as in its torch conv) then the slotted recurrence
    (``fused_recurrent_gated_delta_rule_to_slots``); step t reads the conv
    window and state step t-1 wrote, step 0 those of ``read_slots``."""
    from .conv_decode import conv_decode
    from .gdn import fused_recurrent_gated_delta_rule_to_slots
    dev = mixed.device
    rows = (row_index.view(batch, steps).long() if row_index is not None
            else torch.arange(batch * steps, device=dev).view(batch, steps))
    writes = write_slots.view(batch, 1) if write_slots.ndim == 1 else write_slots
    for t in range(steps):
        r = rows[:, t]
        read = read_slots if t == 0 else writes[:, t - 1]
        q, k, v = conv_decode(mixed.index_select(0, r), conv_weight, config, split_qkv=True, round_conv=steps > 1,
                              read_slots=read, write_slots=writes[:, t], standard_state=conv_state)
        o = fused_recurrent_gated_delta_rule_to_slots(q, k, v, gate.index_select(0, r)[:, None],
                                                      beta.index_select(0, r)[:, None], A_log, dt_bias,
                                                      recurrent_state, read, writes[:, t], config.layer_idx)
        out.index_copy_(0, r, o[:, 0])


def decode_step(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, conv_state, recurrent_state,
                read_slots, write_slots, out=None):
    """``gdn.py:222-265`` in one kernel: conv window of ``read_slots`` -> SiLU
    (unrounded pre-activation, like ``conv_decode`` in GDN mode) -> recurrent
    step; windows and states go to ``write_slots`` (in place when equal).
    Returns o [B, HV, dv]."""
    B, C = mixed_qkv.shape
    assert C == config.conv_dim
    assert read_slots.shape == write_slots.shape == (B,)
    _check_pools(conv_state, recurrent_state, config)
    if out is None:
        out = torch.empty(B, config.num_v_heads, config.head_v_dim, device=mixed_qkv.device, dtype=mixed_qkv.dtype)
    assert out.shape == (B, config.num_v_heads, config.head_v_dim) and out.is_contiguous()
    if B and config.num_v_heads // config.num_k_heads > _MAX_FUSED_GROUP:
        _stepwise(mixed_qkv, None, gate, beta, conv_weight, A_log, dt_bias, config, conv_state, recurrent_state,
                  read_slots, write_slots, B, 1, out)
    elif B:
        _fused(mixed_qkv, None, gate, beta, conv_weight, A_log, dt_bias, config, conv_state, recurrent_state,
               read_slots, write_slots, B, 1, write_slots.stride(0), 0, out)
    return out


def verify_group(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, conv_state, recurrent_state,
                 row_indices, baseline_slots, write_slots, output):
    """One verify length group (``gdn.py:165-218``): B sequences of T drafts at
    rows ``row_indices`` (``[B*T]``, or None for rows ``0..B*T-1``) of
    ``mixed_qkv``/``gate``/``beta``.  Step t's conv window and state go to
    ``write_slots[b, t]``; outputs land in ``output[row]`` ([rows, HV, dv]).
    Groups of more than 16 drafts run as 16-step segments (each resuming from
    the slot the previous segment's last step wrote, so those write slots must
    be valid); more than 4 v-heads per key head take ``_stepwise``."""
    B, T = write_slots.shape
    assert baseline_slots.shape == (B,)
    assert T >= 1
    _check_pools(conv_state, recurrent_state, config)
    assert output.is_contiguous() and output.shape[1:] == (config.num_v_heads, config.head_v_dim)
    if row_indices is not None:
        assert row_indices.shape == (B * T,)
    if B and config.num_v_heads // config.num_k_heads > _MAX_FUSED_GROUP:
        _stepwise(mixed_qkv, row_indices, gate, beta, conv_weight, A_log, dt_bias, config, conv_state,
                  recurrent_state, baseline_slots, write_slots, B, T, output)
    elif B and T > _MAX_FUSED_STEPS:
        # segments of at most 16 drafts; each resumes from the conv window and
        # state the previous segment's last step wrote
        rows = (row_indices.view(B, T) if row_indices is not None
                else torch.arange(B * T, device=mixed_qkv.device).view(B, T))
        for s0 in range(0, T, _MAX_FUSED_STEPS):
            s1 = min(s0 + _MAX_FUSED_STEPS, T)
            base = baseline_slots if s0 == 0 else write_slots[:, s0 - 1]
            verify_group(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, config, conv_state, recurrent_state,
                         rows[:, s0:s1].reshape(-1), base, write_slots[:, s0:s1], output)
    elif B:
        _fused(mixed_qkv, row_indices, gate, beta, conv_weight, A_log, dt_bias, config, conv_state,
               recurrent_state, baseline_slots, write_slots, B, T, write_slots.stride(0), write_slots.stride(1),
               output)
    return output


__all__ = ["conv_snapshots", "decode_step", "prefill_chunk_fused", "prefill_frontend", "prefill_fused",
           "prefill_fused_noalloc", "verify_group"]
