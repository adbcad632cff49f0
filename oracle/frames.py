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

Pinning (``tests/test_oracle.py``): with the identity table
``payload_frames[s, i] = s fps + i`` the storage is one contiguous pool, so
``read_frame_states`` must equal a plain reshape of the storage (heads inside
one frame, heads spanning frames, padded heads); relabelling frames (moving
frame f's bytes to frame p(f) and the table entries with them) leaves every
read unchanged; and ``chunk_gated_delta_rule_to_frames`` on the identity
table must equal ``gdn.chunk_gated_delta_rule_to_cache`` on the reshaped
pool bit for bit.
"""

from __future__ import annotations

import torch

from .gdn import chunk_gated_delta_rule_to_cache


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
