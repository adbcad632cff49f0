"""CPU restatement of the LogState frame-table state addressing.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Paths are relative to
the reference repository root (``python/logssms/...``).

In the LogState cache a slot owns a row of frame numbers
(``payload_frames[slot, :]``) and its recurrent states live in those frames
of a byte storage ``[num_frames, frame_bytes]``.  Head ``h`` of layer ``l``
starts at logical byte ``(l HV + h) head_bytes`` of the slot; logical byte
``x`` lies in frame ``payload_frames[slot, x // frame_bytes]`` at offset
``x % frame_bytes`` (``kernel/linear_attention/layout.py:11-26``,
``cache/logstate/frame_pool.py:181-199``).  ``head_bytes`` is the state size
or its power-of-two padding (``cache/logstate/layout.py:64-71``).

The token log of the chunked prefill (``store_chunk_log``) uses the same
frame tables for its rows and a per-slot decay record for the gates
(``kernel/linear_attention/state_io.py:83-126``, ``layout.py:29-80``).

Pinning (``tests/test_oracle_frames.py``): with the identity table
``payload_frames[s, i] = s fps + i`` the storage is one contiguous pool, so
``read_frame_states`` must equal a plain reshape of the storage (heads inside
one frame, heads spanning frames, padded heads), and ``store_chunk_log`` must
write each row where a reshape of the slot's log payload as
``[granule, layer, keys | values]`` puts it; relabelling frames (moving frame
f's bytes to frame p(f) and the table entries with them) leaves every read
and write unchanged; and ``chunk_gated_delta_rule_to_frames`` on the identity
table must equal ``gdn.chunk_gated_delta_rule_to_cache`` on the reshaped pool
bit for bit.  ``restore_log_state_chains`` must rebuild, from a copied base
state and the rows that eager decode steps logged, the state those steps left
in the work slot (any split into segments or chained restores), a None base
must equal a zeroed one, and a bf16 restore must round the suffix-scaled v'
before the product; ``copy_states`` must move every layer of the named slots
and no other byte.
"""

from __future__ import annotations

import torch

from .gdn import _scale_inputs, chunk_gated_delta_rule_to_cache, l2norm, softplus_decode


def frame_state_index(frames, slots, layer, HV, dk, dv, itemsize, frame_bytes, head_bytes):
    """Element indices ``[len(slots), HV, dk dv]`` into the flat storage (viewed
    in the state dtype) of every state element of ``slots`` at ``layer``
    (``frame_pool.py:181-199``: one frame per head when ``head_bytes <=
    frame_bytes``, a frame per element otherwise)."""
    slots = torch.as_tensor(slots, dtype=torch.int64)
    heads = torch.arange(HV, dtype=torch.int64)
    elems = torch.arange(dk * dv, dtype=torch.int64)
    frames = frames.to(torch.int64)
    frame_elems = frame_bytes // itemsize
    if head_bytes <= frame_bytes:
        logical = (layer * HV + heads) * head_bytes  # [HV]
        fr = frames[slots[:, None], (logical // frame_bytes)[None, :]]  # [S, HV]
        base = fr * frame_elems + (logical % frame_bytes)[None, :] // itemsize
        return base[:, :, None] + elems[None, None, :]
    logical = (layer * HV + heads[:, None]) * head_bytes + elems[None, :] * itemsize  # [HV, E]
    fr = frames[slots[:, None, None], (logical // frame_bytes)[None]]  # [S, HV, E]
    return fr * frame_elems + (logical % frame_bytes)[None] // itemsize


def read_frame_states(storage, frames, slots, layer, HV, dk, dv, frame_bytes, head_bytes):
    """States ``[len(slots), HV, dk, dv]`` of ``slots`` from the frame storage
    ``[num_frames, frame_bytes / itemsize]`` (``frame_pool.py:201-205``)."""
    idx = frame_state_index(frames, slots, layer, HV, dk, dv, storage.element_size(), frame_bytes, head_bytes)
    return storage.reshape(-1)[idx].reshape(len(idx), HV, dk, dv)


def write_frame_states(storage, frames, slots, layer, values, frame_bytes, head_bytes):
    """``storage[...] = values`` for the slots >= 0 (``frame_pool.py:207-227``,
    host branch); ``storage`` is modified in place."""
    slots = torch.as_tensor(slots, dtype=torch.int64)
    keep = slots >= 0
    slots, values = slots[keep], values[keep]
    if not len(slots):
        return
    HV, dk, dv = values.shape[1:]
    idx = frame_state_index(frames, slots, layer, HV, dk, dv, storage.element_size(), frame_bytes, head_bytes)
    flat = storage.view(-1)
    flat[idx.reshape(-1)] = values.to(storage.dtype).reshape(-1)


def chunk_gated_delta_rule_to_frames(query, key, value, gate, beta, storage, frames, frame_bytes, head_bytes,
                                     read_slots, chunk_write_slots, cu_seqlens, *, layer=0,
                                     final_write_slots=None, chunk_size=64, dtype=torch.float32):
    """``chunk_gated_delta_rule_to_cache`` with the states in a LogState frame
    storage (``vendor/fla/chunk_delta_h.py:89-139,226-284`` with
    ``LOGSTATE=True``): the states of every slot the call names are read
    through the frame table into a compact pool, the chunk pipeline runs on
    it, and the written slots go back through the table.  Requires the slots
    to map to disjoint bytes (distinct frames), as the reference pool
    guarantees.  ``storage`` is modified in place."""
    _, _, HV, dv = value.shape
    dk = query.shape[-1]
    named = [int(s) for s in read_slots] + [int(s) for s in chunk_write_slots]
    if final_write_slots is not None:
        named += [int(s) for s in final_write_slots]
    used = sorted({s for s in named if s >= 0})
    compact = {s: i for i, s in enumerate(used)}
    pool = torch.zeros(len(used), 1, HV, dk, dv, dtype=storage.dtype)
    if used:
        pool[:, 0] = read_frame_states(storage, frames, used, layer, HV, dk, dv, frame_bytes, head_bytes)

    def remap(t):
        return None if t is None else torch.tensor([compact.get(int(s), -1) for s in t], dtype=torch.int64)

    writes = remap(chunk_write_slots)
    finals = remap(final_write_slots)
    o, v_new = chunk_gated_delta_rule_to_cache(query, key, value, gate, beta, pool, remap(read_slots), writes,
                                               cu_seqlens, layer=0, final_write_slots=finals,
                                               chunk_size=chunk_size, dtype=dtype)
    written = sorted({int(s) for s in writes if s >= 0} | ({int(s) for s in finals if s >= 0} if finals is not None
                                                              else set()))
    if written:
        write_frame_states(storage, frames, [used[i] for i in written], layer, pool[written, 0], frame_bytes,
                           head_bytes)
    return o, v_new


def log_element_index(frames, slots, positions, index, columns, layer, layers, granularity, key_heads, HV, dk, dv,
                      frame_bytes, value, itemsize=2):
    """Flat 16-bit element indices into the frame storage of log rows
    (``kernel/linear_attention/layout.py:29-80``, ``log_pointer``): slot
    ``slots[i]``, page position ``positions[i]``, row ``index[i]`` (a value
    head, or a logged key head), element ``columns``.  The slot's log holds,
    from logical byte 0, granule (position // granularity), layer, keys
    ``[key_heads, granularity, dk]`` then values ``[HV, granularity, dv]``.
    Every element is placed through its own byte offset, which equals the
    reference's per-row placement whenever a row fits one frame.  The
    reference's log elements are 16-bit (``itemsize`` 2); other sizes serve
    the oracle's own fp32 checks."""
    slots = torch.as_tensor(slots, dtype=torch.int64)[:, None]
    positions = torch.as_tensor(positions, dtype=torch.int64)[:, None]
    index = torch.as_tensor(index, dtype=torch.int64)[:, None]
    columns = torch.as_tensor(columns, dtype=torch.int64)[None, :]
    key_size = granularity * key_heads * dk
    layer_size = key_size + granularity * HV * dv
    dim = dv if value else dk
    elem = ((positions // granularity * layers + layer) * layer_size + (key_size if value else 0)
            + (index * granularity + positions % granularity) * dim + columns)
    byte = itemsize * elem
    fr = frames.to(torch.int64)[slots, byte // frame_bytes]
    return (fr * frame_bytes + byte % frame_bytes) // itemsize


def store_chunk_log(storage, frames, frame_bytes, log_slots, token_offsets, v_new, key, gate, decay_frames,
                    decay_record_bytes, *, layer, layers, granularity, page_size, key_heads):
    """The token-log stores of the chunked prefill (``state_io.py:83-126``):
    for every token t with ``log_slots[t] >= 0`` and every value head h,
    ``v_new[t, h]`` goes to value row h, ``key[t, h // (HV // H)]`` to key row
    ``h // (HV // key_heads)`` when ``h % (HV // key_heads) == 0``, and
    ``gate[t, h]`` (fp32) to float ``(layer page_size + position) HV + h`` of
    the slot's decay record.  ``storage`` ([num_frames, frame_bytes / 2],
    16-bit) is modified in place; v_new [T, HV, dv], key [T, H, dk] in its
    dtype, gate [T, HV]."""
    T, HV, dv = v_new.shape
    H, dk = key.shape[1:]
    flat = storage.view(-1)
    as_bytes = storage.view(torch.uint8).view(-1)
    group = HV // key_heads
    for t in range(T):
        slot, pos = int(log_slots[t]), int(token_offsets[t])
        if slot < 0 or not 0 <= pos < page_size:
            continue
        heads = list(range(HV))
        idx = log_element_index(frames, [slot] * HV, [pos] * HV, heads, range(dv), layer, layers, granularity,
                                key_heads, HV, dk, dv, frame_bytes, True)
        flat[idx.reshape(-1)] = v_new[t].reshape(-1).to(storage.dtype)
        logged = [h for h in heads if h % group == 0]
        kidx = log_element_index(frames, [slot] * len(logged), [pos] * len(logged), [h // group for h in logged],
                                 range(dk), layer, layers, granularity, key_heads, HV, dk, dv, frame_bytes, False)
        flat[kidx.reshape(-1)] = key[t, [h // (HV // H) for h in logged]].reshape(-1).to(storage.dtype)
        frame, record = int(decay_frames[slot, 0]), int(decay_frames[slot, 1])
        base = frame * frame_bytes + record * decay_record_bytes + 4 * ((layer * page_size + pos) * HV)
        as_bytes[base:base + 4 * HV] = gate[t].to(torch.float32).contiguous().view(torch.uint8)


# ----------------------------------------------------------------- LogState decode

def conv_element_index(conv_frames, slots, granules, layer, C, S, frame_elems):
    """Flat element indices ``[len(slots), C S]`` of the conv windows of
    (slot, granule) at ``layer`` (``layout.py:104-112``, ``conv_pointer``):
    element ``layer C S + ch S + s`` of the (slot, granule) snapshot lies in
    frame ``conv_frames[slot, granule, e // frame_elems]`` at ``e % frame_elems``
    (one frame per snapshot: ``conv_frames[slot, granule, 0]`` plus e)."""
    slots = torch.as_tensor(slots, dtype=torch.int64)[:, None]
    granules = torch.as_tensor(granules, dtype=torch.int64)[:, None]
    elem = layer * C * S + torch.arange(C * S, dtype=torch.int64)[None, :]
    table = conv_frames.to(torch.int64)
    if table.shape[2] == 1:
        return table[slots, granules, 0] * frame_elems + elem
    return table[slots, granules, elem // frame_elems] * frame_elems + elem % frame_elems


def conv_decode_logstate(x, weight, storage, conv_frames, frame_bytes, layer, read_slots, read_granules,
                         write_slots, write_granules, work_slots, *, round_conv=False, input_boundaries=None,
                         input_scales=(1.0, 1.0, 1.0)):
    """``conv_decode`` with the LogState pool (``conv_decode.py:293-352`` with
    ``pool=``, kernel ``:25-289``): the window is read from (read slot, read
    granule), and the shifted window goes to (write slot, write granule) and to
    granule 0 of the work slot.  ``storage`` ([num_frames, frame elements], the
    io dtype) is modified in place.  The input is scaled per channel range
    (``conv_decode.py:142``, ``_scale_conv_input``) before the conv and the
    window.  Returns y [B, C]."""
    B, C = x.shape
    x = _scale_inputs(x, torch.arange(C)[None, :], input_boundaries or (C, C), input_scales)
    W = weight.shape[-1]
    S = W - 1
    fe = frame_bytes // storage.element_size()
    flat = storage.view(-1)
    idx = conv_element_index(conv_frames, read_slots, read_granules, layer, C, S, fe)
    windows = flat[idx].view(B, C, S)
    acc_t = torch.float64 if x.dtype == torch.float64 else torch.float32
    full = torch.cat([windows, x[:, :, None]], -1).to(acc_t)
    acc = (full * weight.reshape(C, W).to(acc_t)[None]).sum(-1)
    if round_conv:
        acc = acc.to(x.dtype).to(acc_t)
    y = (acc / (1.0 + torch.exp(-acc))).to(x.dtype)
    new = torch.cat([windows[:, :, 1:], x[:, :, None]], -1).to(storage.dtype).reshape(B, C * S)
    for slots, granules in ((write_slots, write_granules), (work_slots, torch.zeros(B, dtype=torch.int64))):
        out = conv_element_index(conv_frames, slots, granules, layer, C, S, fe)
        flat[out.reshape(-1)] = new.reshape(-1)
    return y


def fused_recurrent_to_logstate(query, key, value, gate, beta, A_log, dt_bias, storage, payload_frames,
                                decay_frames, frame_bytes, head_bytes, record_bytes, work_slots, log_slots,
                                token_offsets, replay_counts, *, layer, layers, granularity, page_size,
                                eager=False, window=16, dtype=torch.float32):
    """LogState decode (``vendor/fla/fused_recurrent.py:292-394``, kernels
    ``:31-288`` with DIRECT_STORE and ``gdn_replay.py:17-148``).  Per sequence
    b with work slot w, log slot l, page position p and replay count n:

    * state: the work slot's state, and unless ``eager`` the n tokens logged
      since it (positions p - n .. p - 1) replayed onto it,
      S = e^{sum g} S_w + sum_i k_i (e^{sum_{j > i} g_j} v'_i)^T, the scaled
      logged values rounded to the io dtype (``replay.py``);
    * step (raw inputs, q / k L2-normalised, g = -exp(A_log) softplus(gate +
      dt_bias), beta = sigmoid(beta)): eager as ``fused_recurrent``; otherwise
      delta = (v - e^g S^T k) beta, o = e^g S^T q + delta (k . q);
    * logs at position p of slot l: v' row = delta, key row = k (for v-heads
      h with h % (HV / H) == 0), decay = g;
    * the work slot receives the new state every step when ``eager``, else
      only when (p + 1) % window == 0.

    query/key [B, 1, H, dk], value [B, 1, HV, dv], gate/beta [B, 1, HV].
    ``storage`` ([num_frames, frame elements], the io dtype) is modified in
    place.  Returns o [B, 1, HV, dv]."""
    B, _, H, dk = query.shape
    HV, dv = value.shape[2:]
    group = HV // H
    io = value.dtype
    item = storage.element_size()
    flat = storage.view(-1)
    as_bytes = storage.view(torch.uint8).view(-1)
    scale = dk ** -0.5
    q_all = l2norm(query[:, 0].to(dtype)) * scale
    k_all = l2norm(key[:, 0].to(dtype))
    g_all = -torch.exp(A_log.to(dtype))[None] * softplus_decode(gate[:, 0].to(dtype) + dt_bias.to(dtype))
    b_all = torch.sigmoid(beta[:, 0].to(dtype))
    out = torch.empty(B, 1, HV, dv, dtype=io)
    for b in range(B):
        w, lslot, pos, n = int(work_slots[b]), int(log_slots[b]), int(token_offsets[b]), int(replay_counts[b])
        state = read_frame_states(storage, payload_frames, [w], layer, HV, dk, dv, frame_bytes,
                                  head_bytes)[0].to(dtype)
        frame, record = int(decay_frames[lslot, 0]), int(decay_frames[lslot, 1])
        rec = frame * frame_bytes + record * record_bytes
        if not eager and n > 0:
            positions = list(range(pos - n, pos))
            g_log = torch.stack([as_bytes[rec + 4 * (layer * page_size + t) * HV:
                                          rec + 4 * ((layer * page_size + t) * HV + HV)].view(torch.float32)
                                 for t in positions]).to(dtype)  # [n, HV]
            heads = list(range(HV))
            keys = torch.stack([flat[log_element_index(payload_frames, [lslot] * HV, [t] * HV,
                                                       [h // group for h in heads], range(dk), layer, layers,
                                                       granularity, H, HV, dk, dv, frame_bytes, False, item)]
                                for t in positions]).to(dtype)  # [n, HV, dk]
            vals = torch.stack([flat[log_element_index(payload_frames, [lslot] * HV, [t] * HV, heads, range(dv),
                                                       layer, layers, granularity, H, HV, dk, dv, frame_bytes,
                                                       True, item)]
                                for t in positions]).to(dtype)  # [n, HV, dv]
            total = g_log.sum(0)
            suffix = torch.exp(total[None] - torch.cumsum(g_log, 0))
            scaled = (vals * suffix[..., None]).to(io).to(dtype)
            state = state * torch.exp(total)[:, None, None] + torch.einsum('thk,thv->hkv', keys, scaled)
        q = q_all[b].repeat_interleave(group, 0)  # [HV, dk]
        k = k_all[b].repeat_interleave(group, 0)
        g, bt = g_all[b], b_all[b]
        v = value[b, 0].to(dtype)
        decay = torch.exp(g)
        if eager:
            state = state * decay[:, None, None]
            delta = (v - (state * k[:, :, None]).sum(1)) * bt[:, None]
            state = state + k[:, :, None] * delta[:, None, :]
            o = (state * q[:, :, None]).sum(1)
            new_state = state
        else:
            sk = (state * k[:, :, None]).sum(1) * decay[:, None]
            sq = (state * q[:, :, None]).sum(1) * decay[:, None]
            delta = (v - sk) * bt[:, None]
            o = sq + delta * (k * q).sum(-1, keepdim=True)
            new_state = state * decay[:, None, None] + k[:, :, None] * delta[:, None, :]
        out[b, 0] = o.to(io)
        if lslot >= 0 and 0 <= pos < page_size:
            heads = list(range(HV))
            vidx = log_element_index(payload_frames, [lslot] * HV, [pos] * HV, heads, range(dv), layer, layers,
                                     granularity, H, HV, dk, dv, frame_bytes, True, item)
            flat[vidx.reshape(-1)] = delta.to(io).reshape(-1)
            logged = [h for h in heads if h % group == 0]
            kidx = log_element_index(payload_frames, [lslot] * len(logged), [pos] * len(logged),
                                     [h // group for h in logged], range(dk), layer, layers, granularity, H, HV, dk,
                                     dv, frame_bytes, False, item)
            flat[kidx.reshape(-1)] = k[logged].to(io).reshape(-1)
            base = rec + 4 * (layer * page_size + pos) * HV
            as_bytes[base:base + 4 * HV] = g.to(torch.float32).contiguous().view(torch.uint8)
        if w >= 0 and (eager or (pos + 1) % window == 0):
            write_frame_states(storage, payload_frames, [w], layer, new_state[None], frame_bytes, head_bytes)
    return out


def read_conv_windows(storage, conv_frames, frame_bytes, slots, granules, layer, C, S):
    """The pool's ``read_conv`` (``cache/logstate/frame_pool.py:229-257``):
    windows [len(slots), C, S] of the (slot, granule) snapshots; a negative
    slot reads zeros."""
    slots = torch.as_tensor(slots, dtype=torch.int64)
    granules = torch.as_tensor(granules, dtype=torch.int64)
    out = torch.zeros(len(slots), C, S, dtype=storage.dtype)
    keep = slots >= 0
    if keep.any():
        idx = conv_element_index(conv_frames, slots[keep], granules[keep], layer, C, S,
                                 frame_bytes // storage.element_size())
        out[keep] = storage.reshape(-1)[idx].view(-1, C, S)
    return out


def forward_prefill_logstate(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, storage, payload_frames,
                             decay_frames, conv_frames, frame_bytes, head_bytes, record_bytes, *, layer, layers,
                             granularity, page_size, cu_seqlens, work_slots, conv_read_slots, conv_read_granules,
                             conv_token_slots, conv_token_granules, chunk_write_slots, log_write_slots,
                             token_offsets, num_k_heads, head_k_dim, num_v_heads, head_v_dim, dtype=torch.float32):
    """The LogState prefill (``layers/linear_attention_backend/gdn_logstate.py:85-172``):
    conv history from the (read slot, read granule) snapshots, packed conv
    with windows to (``conv_token_slots``, ``conv_token_granules``) and each
    sequence's last window to granule 0 of its work slot, ``prepare_gdn``, the
    chunked rule from and to the work slots with checkpoints every
    ``granularity`` tokens, and the token log.  ``storage`` (the io dtype) is
    modified in place; returns o [T, HV, dv]."""
    from .gdn import packed_causal_conv1d, prepare_gdn, split_qkv
    N = len(cu_seqlens) - 1
    C = mixed_qkv.shape[1]
    S = conv_weight.shape[-1] - 1
    fe = frame_bytes // storage.element_size()
    flat = storage.view(-1)
    history = read_conv_windows(storage, conv_frames, frame_bytes, conv_read_slots, conv_read_granules, layer, C, S)
    cu = [int(v) for v in cu_seqlens]
    token_slots = [int(x) for x in conv_token_slots]
    rows = sorted({t for t, s in enumerate(token_slots) if s >= 0} | {cu[n + 1] - 1 for n in range(N)
                                                                      if cu[n + 1] > cu[n]})
    y, windows = packed_causal_conv1d(mixed_qkv, conv_weight, history, cu_seqlens, window_rows=rows)
    where = {t: i for i, t in enumerate(rows)}
    for t, s in enumerate(token_slots):
        if s >= 0:
            idx = conv_element_index(conv_frames, [s], [int(conv_token_granules[t])], layer, C, S, fe)
            flat[idx.reshape(-1)] = windows[where[t]].reshape(-1).to(storage.dtype)
    for n in range(N):
        if cu[n + 1] > cu[n] and int(work_slots[n]) >= 0:
            idx = conv_element_index(conv_frames, [int(work_slots[n])], [0], layer, C, S, fe)
            flat[idx.reshape(-1)] = windows[where[cu[n + 1] - 1]].reshape(-1).to(storage.dtype)
    q, k, v = split_qkv(y[None], num_k_heads, head_k_dim, num_v_heads, head_v_dim)
    q, k, v, g, b = prepare_gdn(q, k, v, gate[None], beta[None], A_log, dt_bias)
    o, v_new = chunk_gated_delta_rule_to_frames(q, k, v, g, b, storage, payload_frames, frame_bytes, head_bytes,
                                                work_slots, chunk_write_slots, cu_seqlens, layer=layer,
                                                final_write_slots=work_slots, chunk_size=granularity, dtype=dtype)
    store_chunk_log(storage, payload_frames, frame_bytes, log_write_slots, token_offsets, v_new[0], k[0], g[0],
                    decay_frames, record_bytes, layer=layer, layers=layers, granularity=granularity,
                    page_size=page_size, key_heads=num_k_heads)
    return o[0]


# ----------------------------------------------------------------- LogState construction

def read_log_segment(storage, payload_frames, decay_frames, frame_bytes, record_bytes, slot, begin, end, *, layer,
                     layers, granularity, page_size, key_heads, HV, dk, dv):
    """The logged tokens ``begin .. end - 1`` of log slot ``slot`` at
    ``layer``: gates [n, HV] (fp32), key rows [n, HV, dk] (value head h reads
    key row h // (HV / key_heads)) and v' rows [n, HV, dv], in the storage
    dtype (``logstate_construction.cuh:137-190``)."""
    flat = storage.view(-1)
    as_bytes = storage.view(torch.uint8).view(-1)
    item = storage.element_size()
    group = HV // key_heads
    positions = list(range(begin, end))
    frame, record = int(decay_frames[slot, 0]), int(decay_frames[slot, 1])
    rec = frame * frame_bytes + record * record_bytes
    gates = torch.stack([as_bytes[rec + 4 * (layer * page_size + t) * HV:rec + 4 * ((layer * page_size + t) * HV + HV)]
                         .view(torch.float32) for t in positions])
    heads = list(range(HV))
    keys = torch.stack([flat[log_element_index(payload_frames, [slot] * HV, [t] * HV, [h // group for h in heads],
                                               range(dk), layer, layers, granularity, key_heads, HV, dk, dv,
                                               frame_bytes, False, item)] for t in positions])
    vals = torch.stack([flat[log_element_index(payload_frames, [slot] * HV, [t] * HV, heads, range(dv), layer, layers,
                                               granularity, key_heads, HV, dk, dv, frame_bytes, True, item)]
                        for t in positions])
    return gates, keys, vals


def restore_log_state_chains(storage, payload_frames, decay_frames, frame_bytes, head_bytes, record_bytes, chains, *,
                             layers, HV, key_heads, dk, dv, granularity, page_size, dtype=torch.float32):
    """``restore_log_state_chains`` (``kernel/linear_attention/logstate.py:59-88``,
    kernel ``logstate_construction.cuh:290-393``): for each ``(base, segments,
    output)`` and every layer and value head, S = the state of slot ``base``
    (zero for None), then per segment ``(slot, begin, end)``
    S <- e^{sum g} S + sum_t k_t (e^{sum_{j > t} g_j} v'_t)^T over its tokens,
    the scaled v' rounded to the storage dtype; S goes to slot ``output``.
    Chains are taken in order; ``storage`` is modified in place."""
    io = storage.dtype
    for base, segments, output in chains:
        for layer in range(layers):
            if base is None:
                state = torch.zeros(HV, dk, dv, dtype=dtype)
            else:
                state = read_frame_states(storage, payload_frames, [base], layer, HV, dk, dv, frame_bytes,
                                          head_bytes)[0].to(dtype)
            for slot, begin, end in segments:
                if end <= begin:
                    continue
                g, keys, vals = read_log_segment(storage, payload_frames, decay_frames, frame_bytes, record_bytes,
                                                 slot, begin, end, layer=layer, layers=layers,
                                                 granularity=granularity, page_size=page_size, key_heads=key_heads,
                                                 HV=HV, dk=dk, dv=dv)
                g = g.to(dtype)
                total = g.sum(0)
                suffix = torch.exp(total[None] - torch.cumsum(g, 0))
                scaled = (vals.to(dtype) * suffix[..., None]).to(io).to(dtype)
                state = state * torch.exp(total)[:, None, None] + torch.einsum('thk,thv->hkv', keys.to(dtype), scaled)
            write_frame_states(storage, payload_frames, [output], layer, state[None], frame_bytes, head_bytes)


def copy_states(storage, payload_frames, frame_bytes, head_bytes, sources, destinations, *, layers, HV, dk, dv):
    """``copy_states`` (``logstate.py:118-128``, ``logstate_construction.cuh:397-414``):
    every layer's states of ``sources[i]`` to ``destinations[i]``."""
    for src, dst in zip(sources, destinations):
        for layer in range(layers):
            state = read_frame_states(storage, payload_frames, [src], layer, HV, dk, dv, frame_bytes, head_bytes)
            write_frame_states(storage, payload_frames, [dst], layer, state, frame_bytes, head_bytes)


def store_states(storage, payload_frames, frame_bytes, head_bytes, slots, layer, values):
    """``store_states`` (``kernel/linear_attention/masked_store.py:11-55``):
    ``values[i]`` [HV, dk, dv] to layer ``layer`` of ``slots[i]``, negative
    slots skipped; the values are rounded to the storage dtype."""
    write_frame_states(storage, payload_frames, slots, layer, values, frame_bytes, head_bytes)


def store_conv(storage, conv_frames, frame_bytes, slots, granules, layer, values):
    """``store_conv`` (``masked_store.py:34-72``): ``values[i]`` [C, S] to
    layer ``layer`` of the (slots[i], granules[i]) conv snapshot, negative
    slots skipped."""
    n, C, S = values.shape
    flat = storage.view(-1)
    fe = frame_bytes // storage.element_size()
    for i in range(n):
        if int(slots[i]) < 0:
            continue
        idx = conv_element_index(conv_frames, [int(slots[i])], [int(granules[i])], layer, C, S, fe)
        flat[idx.reshape(-1)] = values[i].reshape(-1).to(storage.dtype)


def copy_conv_snapshots(storage, conv_frames, frame_bytes, source_slots, source_granules, output_slots,
                        output_granules, *, layers, C, S):
    """``copy_conv_snapshots`` (``kernel/linear_attention/conv_copy.py:7-52``):
    every layer's window of (source slot, granule) to (output slot, granule),
    pairs with a negative slot skipped (the pairs must not overlap)."""
    flat = storage.view(-1)
    fe = frame_bytes // storage.element_size()
    for s, sg, o, og in zip(source_slots, source_granules, output_slots, output_granules):
        if int(s) < 0 or int(o) < 0:
            continue
        for layer in range(layers):
            src = conv_element_index(conv_frames, [int(s)], [int(sg)], layer, C, S, fe).reshape(-1)
            dst = conv_element_index(conv_frames, [int(o)], [int(og)], layer, C, S, fe).reshape(-1)
            flat[dst] = flat[src].clone()
