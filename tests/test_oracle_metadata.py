"""Pins ``oracle/metadata.py`` with the known answers of the reference's own tests."""

import pytest

from oracle import metadata as md


def test_decode_capture_known_answer():
    """tests/layers/test_linear_attention_backend.py:100-129."""
    table = [[3] * 64 + [4] * 64, [5] * 64 + [6] * 64, [9] * 128]
    read, write = md.decode_slots(table, [(0, 64), (2, 0)])
    assert read == [3, 9] and write == [4, 9]


def test_verify_groups_known_answer():
    """tests/layers/test_linear_attention_backend.py:203-237."""
    table = [[11] * 64 + [12] * 64 + [13] * 64, [20] * 64 + [21] * 64 + [22] * 64]
    work = [[100, 101, 102], [110, 111, 112]]
    groups = md.verify_groups(table, work, [(0, 62, 3), (1, 128, 2)])
    assert groups[3] == ([0, 1, 2], [11], [[100, 101, 102]])
    assert groups[2] == ([3, 4], [21], [[110, 111]])
    assert list(groups) == [3, 2]


@pytest.mark.parametrize("block_size, width", [(0, 1), (64, 7), (128, 4), (256, 2), (448, 1), (512, 1)])
def test_marconi_layout_table(block_size, width):
    """tests/hybrid/test_marconi.py:17-30."""
    lay = md.marconi_layout(16, 48, (24, 128, 128), (5120, 3), 2, 256, block_size)
    assert lay["block_size"] == (block_size or 448)
    assert lay["state_blocks_per_group"] == width
    assert lay["state_groups"] * width == 3 * width
    block_bytes = lay["layers_per_group"] * lay["layer_elements"] * 2
    assert lay["state_groups"] * width * block_bytes == 3 * width * 16 * lay["block_size"] * 2048


def test_marconi_layout_rejects_bad_block_size():
    for size in (-64, 16, 32, 65):
        with pytest.raises(ValueError):
            md.marconi_layout(16, 48, (24, 128, 128), (5120, 3), 2, 256, size)


def test_from_lengths_known_answer_and_fla_agreement():
    """standard.py:42-73 vs the independent FLA helpers (vendor/fla/index.py)."""
    r = md.from_lengths([17, 31, 33, 65], 32)
    assert r["cu_seqlens"] == [0, 17, 48, 81, 146]
    assert r["chunk_offsets"] == [0, 1, 2, 4, 7]
    assert r["endings"] == [0, 1, 3, 6]
    assert r["chunk_indices"] == [[0, 0], [1, 0], [2, 0], [2, 1], [3, 0], [3, 1], [3, 2]]
    assert r["conv_chunks"] == [[0, 0], [1, 0], [2, 0], [3, 0], [3, 1]]
    for chunk in (16, 32, 64):
        lengths = [1, 63, 64, 65, 200]
        r = md.from_lengths(lengths, chunk)
        assert r["chunk_indices"] == md.prepare_chunk_indices(r["cu_seqlens"], chunk)
        assert r["chunk_offsets"] == md.prepare_chunk_offsets(r["cu_seqlens"], chunk)


def test_prefill_checkpoint_placement_radix_pages():
    """standard.py:157-209: every page end + the final token; chunk = offset + (end-1)//64."""
    page = 128
    table = [list(range(1000, 1000 + 512)), list(range(2000, 2000 + 512))]
    # request 0: fresh, 300 tokens; request 1: cached 128, extends 64.
    r = md.prefill_metadata(table, [(0, 0, 300), (1, 128, 64)], page)
    assert r["baseline_slots"] == [-1, table[1][127]]
    assert r["checkpoint_chunks"] == [1, 3, 4, 5]
    assert r["snapshot_rows"] == [127, 255, 299, 363]
    assert r["checkpoint_slots"] == [table[0][127], table[0][255], table[0][299], table[1][191]]
    cw = [-1] * 6
    for c, s in zip(r["checkpoint_chunks"], r["checkpoint_slots"]):
        cw[c] = s
    assert r["chunk_write_slots"] == cw
    assert sum(s >= 0 for s in r["conv_token_slots"]) == 4
    assert len(r["conv_token_slots"]) == 364


def test_prefill_checkpoint_placement_marconi_sparse():
    """standard.py:166-169 with Marconi checkpoint_writes (ends % 64 == 0 or final)."""
    table = [[7] * 256]
    r = md.prefill_metadata(table, [(0, 0, 200)], 64, sparse=[[(64, 11), (128, 12), (200, 13)]])
    assert r["chunk_write_slots"] == [11, 12, -1, 13]
    assert [i for i, s in enumerate(r["conv_token_slots"]) if s >= 0] == [63, 127, 199]
    with pytest.raises(AssertionError):
        md.prefill_metadata(table, [(0, 0, 200)], 64, sparse=[[(65, 11), (200, 13)]])


def test_marconi_branch_checkpoint_known_answer():
    """tests/hybrid/test_marconi.py:226-268: checkpoint ends [ps, ps + 12];
    the branch slot receives a copy of the boundary state after the forward."""
    ps = 128
    req = dict(cached_len=0, device_len=ps + 12, states=(5, 6), checkpoints={ps: 9})
    writes, copies = md.marconi_checkpoint_writes([req], ps)
    assert [end for end, _ in writes[0]] == [ps, ps + 12]
    assert writes[0] == [(ps, 5), (ps + 12, 6)]
    assert copies == [(5, 9)]


@pytest.mark.parametrize("end", [1, 127, 128, 129, 255, 256, 257, 384, 385])
def test_double_state_parity(end):
    """tests/hybrid/test_marconi.py:163-224: with the row filled from
    ``states[page_parity]``, decode read != write exactly when (pos-1) % ps == 0."""
    ps = 128
    states = (40, 41)
    row = [states[(i // ps) % 2] for i in range(512)]
    for position in range(2, end + 1):
        read, write = row[position - 2], row[position - 1]
        assert (read != write) == ((position - 1) % ps == 0)
        assert write == md.state_at(states, position, ps)


def test_map_slots_keeps_sentinels():
    """cache/marconi/block_pool.py:101-110."""
    group_table = [[10, 20], [11, 21], [12, 22]]
    mapped, lane = md.map_slots(group_table, [2, -1, 0], layer=5, layers_per_group=4)
    assert mapped == [22, -1, 20] and lane == 1


def test_commit_speculative_remaps_pages():
    """cache/radix/manager.py:248-268: accepted positions inside one page move
    the reserve slot into the live row; crossing a page remaps each page."""
    ps = 4
    table = [[1] * 4 + [2] * 4 + [3] * 4]
    work = [[100, 101, 102, 103, 104]]
    md.commit_speculative(table, work, 0, C=6, num_sampled=3, page_size=ps)
    # positions 6,7 are on page 1 (last = 7 -> cand 1); position 8 on page 2 (cand 2)
    assert table[0] == [1] * 4 + [101] * 4 + [102] * 4
    assert work[0] == [100, 2, 3, 103, 104]


def test_logstate_prefill_plan_known_answer():
    """layers/linear_attention_backend/logstate.py:215-272 worked by hand on a
    granularity-4 page: request 0 (6 tokens from page offset 1, nothing
    cached), request 1 (3 tokens from offset 2 after 5 cached).

    Marks (-2): request 0 at rows whose offset closes a granule ((1 + row + 1)
    % 4 == 0: row 2) and its last row 5; request 1 at row 1 and its last row
    2 (global 7, 8).  The unlogged range (1, 5, 7) covers positions 5, 6 =
    rows 0, 1 of request 1 (global 6, 7): not logged, no snapshot.
    Checkpoints, sorted: (1, 10) sits at no mark: ignored.  (5, 11) at the
    last row of request 0: slot 11 (a work slot: granule 0), chunk 5 // 4 = 1.
    (7, 12) at a granule end inside the unlogged range: the snapshot goes to
    slot 12 (granule 3 = the last of 4) while the token stays unlogged; its
    chunk is chunk 0 of request 1 = global chunk 2.  (8, 9) and then (8, 13)
    at request 1's last row, the same token and chunk: 13 wins.  (20, 14)
    lies past the batch: never reached."""
    plan = md.logstate_prefill_plan(
        [6, 3], [0, 5], [1, 2], [(8, 13), (1, 10), (5, 11), (7, 12), (8, 9), (20, 14)], [(1, 5, 7)],
        granularity=4, num_granules=4, work_slots={11})
    assert plan["conv_slots"] == [-1, -1, -2, -1, -1, 11, -1, 12, 13]
    assert plan["conv_granules"] == [0, 0, 0, 0, 0, 0, 0, 3, 3]
    assert plan["log_enabled"] == [1, 1, 1, 1, 1, 1, 0, 0, 1]
    assert plan["chunk_writes"] == [-1, 11, 13]


def test_logstate_prefill_plan_unlogged_range_clipping():
    """A range reaching before the cached prefix and past the request is
    clipped to the request's own rows; ranges of other requests do nothing."""
    plan = md.logstate_prefill_plan([5], [10], [2], [], [(0, 4, 12), (3, 0, 100)], granularity=4,
                                    num_granules=2, work_slots=set())
    # positions 10..14 are rows 0..4; the range [4, 12) covers rows 0, 1
    assert plan["log_enabled"] == [0, 0, 1, 1, 1]
    # marks: (2 + row + 1) % 4 == 0 at row 1 (cleared by the range), last row 4
    assert plan["conv_slots"] == [-1, -1, -1, -1, -2]
    assert plan["chunk_writes"] == [-1, -1]


def test_logstate_prefill_writes_known_answer():
    """kernel/metadata.py:150-178: -2 resolves to the token's log slot at
    granule offset // granularity; disabled tokens get no log write."""
    plan = {"conv_slots": [-2, -2, 5, -1], "conv_granules": [0, 0, 2, 0], "log_enabled": [1, 0, 1, 1]}
    writes, conv, granules = md.logstate_prefill_writes([7, 7, 7, 8], [3, 7, 11, 12], plan, 4)
    assert writes == [7, -1, 7, 8]
    assert conv == [7, 7, 5, -1]
    assert granules == [0, 1, 2, 0]


def test_logstate_decode_slots_known_answer():
    """tests/layers/test_logstate_linear_attention_backend.py:74-96: a decode
    at position 20 of a row whose first page logs to slot 0, work slot 2."""
    state = [[0] * 64 + [1] * 64, [1] * 128]
    work = [[2], [3]]
    assert md.logstate_decode_slots(work, state, [(0, 20)], [20], 64) == ([2], [0], [20], [0])
