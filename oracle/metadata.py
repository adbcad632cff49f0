"""Bit-exact restatement of the reference's host-side integer logic for the
GDN path, written as plain Python loops.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Pinned by the known
answers in the reference's own tests (``tests/test_oracle_metadata.py`` lists
each one with its source line).
"""

from __future__ import annotations


def from_lengths(lengths, chunk_size=64):
    """layers/linear_attention_backend/standard.py:42-73
    (``PackedLinearIndices.from_lengths``).

    Returns dict of python lists: cu_seqlens [N+1], chunk_indices [[req, chunk]],
    chunk_offsets [N+1], endings [N] (last global chunk of each request) and
    conv_chunks [[req, chunk]] (always 64-token chunks).
    """
    offsets, chunk_offsets = [0], [0]
    chunks, conv_chunks, endings = [], [], []
    for req, length in enumerate(lengths):
        assert length > 0
        offsets.append(offsets[-1] + length)
        n = (length + chunk_size - 1) // chunk_size
        chunk_offsets.append(chunk_offsets[-1] + n)
        chunks.extend([req, c] for c in range(n))
        conv_chunks.extend([req, c] for c in range((length + 63) // 64))
        endings.append(chunk_offsets[-1] - 1)
    return dict(cu_seqlens=offsets, chunk_indices=chunks, chunk_offsets=chunk_offsets,
                endings=endings, conv_chunks=conv_chunks)


def prepare_chunk_indices(cu_seqlens, chunk_size):
    """vendor/fla/index.py:28-36."""
    out = []
    for n in range(len(cu_seqlens) - 1):
        length = cu_seqlens[n + 1] - cu_seqlens[n]
        out.extend([n, c] for c in range((length + chunk_size - 1) // chunk_size))
    return out


def prepare_chunk_offsets(cu_seqlens, chunk_size):
    """vendor/fla/index.py:39-46."""
    out = [0]
    for n in range(len(cu_seqlens) - 1):
        length = cu_seqlens[n + 1] - cu_seqlens[n]
        out.append(out[-1] + (length + chunk_size - 1) // chunk_size)
    return out


def decode_slots(state_table, reqs):
    """standard.py:112-128 -- ``read = table[t, cached-1]``, ``write = table[t, cached]``.

    ``reqs`` = list of (table_idx, cached_len).  ``state_table`` = list of rows.
    """
    read = [state_table[t][c - 1] for t, c in reqs]
    write = [state_table[t][c] for t, c in reqs]
    return read, write


def prefill_metadata(state_table, reqs, page_size, *, sparse=None, group_table=False):
    """standard.py:129-209 (prefill branch).

    ``reqs`` = list of (table_idx, cached_len, extend_len).  ``sparse`` =
    Marconi ``checkpoint_writes`` (list per request of (end, slot)), or None.
    ``group_table`` mimics a pool with a ``group_table`` attribute (final-only
    checkpoints).  Returns dict of python lists.
    """
    assert page_size % 64 == 0
    baseline = []
    for t, cached, _ in reqs:
        prev = cached - 1
        baseline.append(state_table[t][max(prev, 0)] if prev >= 0 else -1)
    ck_slots, ck_chunks, rows, snap_reqs = [], [], [], []
    chunk_offset = token_offset = 0
    for i, (t, cached, ext) in enumerate(reqs):
        if sparse is None and group_table:
            ends = [ext]
            slots = [state_table[t][cached + ext - 1]]
        elif sparse is None:
            assert cached % 64 == 0
            ends = list(range(page_size, ext, page_size)) + [ext]
            slots = [state_table[t][cached + e - 1] for e in ends]
        else:
            ends = [e for e, _ in sparse[i]]
            slots = [s for _, s in sparse[i]]
            assert all(e == ext or e % 64 == 0 for e in ends)
        for e, s in zip(ends, slots):
            ck_slots.append(s)
            ck_chunks.append(chunk_offset + (e - 1) // 64)
            rows.append(token_offset + e - 1)
            snap_reqs.append(i)
        chunk_offset += (ext + 63) // 64
        token_offset += ext
    chunk_write = [-1] * chunk_offset
    for c, s in zip(ck_chunks, ck_slots):
        chunk_write[c] = s
    conv_tokens = [-1] * token_offset
    for r, s in zip(rows, ck_slots):
        conv_tokens[r] = s
    return dict(baseline_slots=baseline, checkpoint_slots=ck_slots,
                checkpoint_chunks=ck_chunks, chunk_write_slots=chunk_write,
                snapshot_rows=rows, snapshot_reqs=snap_reqs, conv_token_slots=conv_tokens)


def verify_groups(state_table, work_state_table, reqs):
    """standard.py:210-250 -- group by draft length.

    ``reqs`` = list of (table_idx, cached_len, extend_len).  Returns
    {seq_len: (row_indices, baseline_slots, write_slots[B][seq_len])} in
    first-seen order of lengths.
    """
    by_len = {}
    offset = 0
    for t, cached, ext in reqs:
        by_len.setdefault(ext, []).append((t, cached - 1, offset))
        offset += ext
    groups = {}
    for seq_len, entries in by_len.items():
        rows = [r for _, _, start in entries for r in range(start, start + seq_len)]
        base = [state_table[t][p] for t, p, _ in entries]
        writes = [list(work_state_table[t][:seq_len]) for t, _, _ in entries]
        groups[seq_len] = (rows, base, writes)
    return groups


def marconi_layout(attention_layers, num_layers, state_shape, conv_shape, kv_heads, head_dim,
                   block_size=128):
    """cache/marconi/layout.py:17-32 (``HybridBlockLayout.make``)."""
    if attention_layers < 1:
        raise ValueError("Marconi requires at least one full-attention layer")
    state_elements = state_shape[0] * state_shape[1] * state_shape[2] + conv_shape[0] * conv_shape[1]
    token_elements = 2 * kv_heads * head_dim
    minimum = ((state_elements + token_elements * 64 - 1) // (token_elements * 64)) * 64
    if block_size < 0 or block_size % 64:
        raise ValueError("Marconi block size must be zero (auto) or a multiple of 64")
    block_size = block_size or minimum
    layer_elements = block_size * token_elements
    return dict(block_size=block_size, layers_per_group=attention_layers,
                state_groups=(num_layers + attention_layers - 1) // attention_layers,
                state_blocks_per_group=(state_elements + layer_elements - 1) // layer_elements,
                layer_elements=layer_elements)


def map_slots(group_table, values, layer, layers_per_group):
    """cache/marconi/block_pool.py:101-110 -- logical slot -> physical block of
    the layer's group; negative stays -1.  Returns (mapped, lane)."""
    group, lane = divmod(layer, layers_per_group)
    return [group_table[v][group] if v >= 0 else -1 for v in values], lane


def state_at(states, end, page_size):
    """cache/marconi/manager.py:84-85 -- alternating live state slots."""
    return states[((end - 1) // page_size) % 2]


def marconi_checkpoint_writes(requests, page_size):
    """cache/marconi/manager.py:248-270 (``prepare_batch``).

    ``requests`` = list of dicts with cached_len, device_len, states (2-tuple)
    and checkpoints ({end: slot}).  Returns (checkpoint_writes per request
    [(end - cached, slot)] sorted, checkpoint_copies [(source, target)]).
    """
    writes, copies = [], []
    for r in requests:
        cached, device = r["cached_len"], r["device_len"]
        extend = device - cached
        ck = r["checkpoints"]
        targets = [(end - cached, slot) for end, slot in ck.items() if cached < end < device]
        boundary = device // page_size * page_size
        if cached < boundary < device:
            targets.append((boundary - cached, state_at(r["states"], boundary, page_size)))
        output = state_at(r["states"], device, page_size)
        targets.append((extend, output))
        if device in ck:
            copies.append((output, ck[device]))
        if boundary in ck and cached < boundary < device:
            targets.remove((boundary - cached, ck[boundary]))
            copies.append((state_at(r["states"], boundary, page_size), ck[boundary]))
        writes.append(sorted(targets))
    return writes, copies


def commit_speculative(state_table, work_state_table, uid, C, num_sampled, page_size):
    """cache/radix/manager.py:248-268 -- verify commit by slot remap.  Mutates
    both tables (lists of lists) in place; no state bytes move."""
    C_end = C + num_sampled
    for page in range(C // page_size, (C_end - 1) // page_size + 1):
        last = min(C_end, (page + 1) * page_size) - 1
        cand = last - C
        live_pos = page * page_size
        live = state_table[uid][live_pos]
        verify = work_state_table[uid][cand]
        assert live >= 0 and verify >= 0
        row = state_table[uid]
        for p in range(live_pos, min(live_pos + page_size, len(row))):
            row[p] = verify
        work_state_table[uid][cand] = live


def logstate_prefill_plan(lengths, cached_lens, first_offsets, checkpoint_writes, checkpoint_ranges, granularity,
                          num_granules, work_slots):
    """layers/linear_attention_backend/logstate.py:215-272 -- the host part of
    the LogState prefill write plan, token by token.

    ``lengths`` / ``cached_lens`` / ``first_offsets`` per request (the page
    offset of its first new token); ``checkpoint_writes`` = (global token
    row, slot) pairs; ``checkpoint_ranges`` = (request, begin, end) position
    ranges whose tokens are not logged; ``work_slots`` = the set of slots of
    kind "work".  Returns dict of python lists: ``conv_slots`` (per token: -1
    none, -2 the token's own log slot, else a checkpoint slot),
    ``conv_granules``, ``log_enabled`` (0 / 1) and ``chunk_writes`` (per
    ``granularity``-token chunk of each request, -1 or a checkpoint slot).

    Per request: every token at a granule end ((first + row + 1) %
    granularity == 0) and its last token are marked -2; a token inside an
    unlogged range (positions relative to cached_len, clipped to the request)
    gets log_enabled 0 and conv slot -1; then, in sorted order, a checkpoint
    whose row lies in this request and sits at a granule end or at the
    request's last token sets the token's conv slot and granule (0 for a work
    slot, else the last granule) and its chunk's write slot.  Later
    checkpoints overwrite earlier ones; checkpoints elsewhere are ignored.
    """
    total = sum(lengths)
    conv_slots = [-1] * total
    conv_granules = [0] * total
    log_enabled = [1] * total
    chunk_writes = [-1] * sum((n + granularity - 1) // granularity for n in lengths)
    pending = sorted(checkpoint_writes)
    k = 0
    token_begin = chunk_begin = 0
    for i, length in enumerate(lengths):
        first = first_offsets[i]
        token_end = token_begin + length
        for row in range(length):
            if (first + row + 1) % granularity == 0 or row + 1 == length:
                conv_slots[token_begin + row] = -2
        for req, begin, end in checkpoint_ranges:
            if req != i:
                continue
            for row in range(max(0, begin - cached_lens[i]), min(length, end - cached_lens[i])):
                log_enabled[token_begin + row] = 0
                conv_slots[token_begin + row] = -1
        while k < len(pending) and pending[k][0] < token_end:
            global_row, slot = pending[k]
            row = global_row - token_begin
            assert row >= 0
            if (first + row + 1) % granularity == 0 or row + 1 == length:
                conv_slots[global_row] = slot
                conv_granules[global_row] = 0 if slot in work_slots else num_granules - 1
                chunk_writes[chunk_begin + row // granularity] = slot
            k += 1
        token_begin = token_end
        chunk_begin += (length + granularity - 1) // granularity
    return dict(conv_slots=conv_slots, conv_granules=conv_granules, log_enabled=log_enabled,
                chunk_writes=chunk_writes)


def logstate_prefill_writes(log_slots, token_offsets, plan, granularity):
    """kernel/metadata.py:150-178 (make_logstate_prefill_writes) -- the device
    half of the plan: per token, the log write slot (its log slot where
    logging is enabled, else -1), the conv snapshot slot (its log slot where
    the plan says -2) and granule (its page offset // granularity there)."""
    log_writes, conv_slots, conv_granules = [], [], []
    for t, slot in enumerate(log_slots):
        conv = plan["conv_slots"][t]
        log_writes.append(slot if plan["log_enabled"][t] else -1)
        conv_slots.append(slot if conv == -2 else conv)
        conv_granules.append(token_offsets[t] // granularity if conv == -2 else plan["conv_granules"][t])
    return log_writes, conv_slots, conv_granules


def logstate_decode_slots(work_table, state_table, reqs, out_loc, page_size):
    """logstate.py:128-175 (decode branch) and kernel/metadata.py:290-300
    (gather_linear_slots, LogState) -- per decode request (table_idx,
    cached_len): the work slot, the log slot at the new position, the page
    offset of its KV location, and conv read granule 0."""
    work = [work_table[t][0] for t, _ in reqs]
    logs = [state_table[t][c] for t, c in reqs]
    offsets = [loc % page_size for loc in out_loc]
    return work, logs, offsets, [0] * len(reqs)
