"""Spec-decode verify commit.

``commit_speculative`` restates the reference's host-side commit by slot
remap (``python/logssms/cache/radix/manager.py:248-268``): for every page the
accepted tokens cross, the live state-table entries are pointed at the verify
slot holding the state after the page's last accepted token, and that verify
slot's old live slot goes back to the reserve.  No state bytes move.

``commit_accepted`` is the device-side alternative for callers that keep one
fixed live slot per sequence: it copies the accepted step's recurrent state and
conv window from the verify write slots into the live slots for one layer, in
one launch, reading the accepted counts on the device (graph-capturable).
"""

from __future__ import annotations

import torch

from .. import _lib


def commit_speculative(state_table: torch.Tensor, work_state_table: torch.Tensor, uid: int, C: int,
                       num_sampled: int, page_size: int) -> None:
    """manager.py:248-268 (host integers; tables may live on any device)."""
    reserve = work_state_table
    assert num_sampled <= reserve.shape[1]
    C_end = C + num_sampled
    for page in range(C // page_size, (C_end - 1) // page_size + 1):
        last_position = min(C_end, (page + 1) * page_size) - 1
        candidate = last_position - C
        live_position = page * page_size
        live_slot = int(state_table[uid, live_position])
        verify_slot = int(reserve[uid, candidate])
        assert live_slot >= 0 and verify_slot >= 0
        state_table[uid, live_position:live_position + page_size] = verify_slot
        reserve[uid, candidate] = live_slot


def commit_accepted(recurrent_state: torch.Tensor, conv_state: torch.Tensor, layer: int, live_slots: torch.Tensor,
                    write_slots: torch.Tensor, accepted: torch.Tensor) -> None:
    """For each sequence b with ``1 <= accepted[b] <= T``:
    ``pool[live_slots[b], layer] <- pool[write_slots[b, accepted[b] - 1], layer]``
    for both pools.  ``recurrent_state`` [slots, L, HV, dk, dv] and
    ``conv_state`` [slots, L, C, W-1] must have contiguous per-(slot, layer) rows."""
    B, T = write_slots.shape
    assert live_slots.shape == accepted.shape == (B,)
    rs, cs = recurrent_state, conv_state
    assert rs[0, 0].is_contiguous() and cs[0, 0].is_contiguous()
    _lib.call("gdn_commit_accepted", rs.data_ptr(), rs.stride(0) * rs.element_size(),
              layer * rs.stride(1) * rs.element_size(), rs[0, 0].numel() * rs.element_size(), cs.data_ptr(),
              cs.stride(0) * cs.element_size(), layer * cs.stride(1) * cs.element_size(),
              cs[0, 0].numel() * cs.element_size(), live_slots.data_ptr(), _lib.index_code(live_slots),
              write_slots.data_ptr(), write_slots.stride(0), write_slots.stride(1), _lib.index_code(write_slots),
              accepted.data_ptr(), _lib.index_code(accepted), B, T, _lib.stream_of(rs))


__all__ = ["commit_accepted", "commit_speculative"]
