"""Host side of the backend: metadata, capture buffers, Marconi layout/mapping
and the speculative commit remap, checked bit-exactly against ``oracle/metadata``
(itself pinned by the reference's known answers) and the reference tests'
own expected values.  CPU only."""

import random
from types import SimpleNamespace

import pytest
import torch

from logssms_amd.cache import HybridBlockLayout, HybridBlockPool, LinearStatePool, commit_speculative
from logssms_amd.core import Batch, Context, MarconiCacheMetadata, Request, clear_global_ctx, set_global_ctx
from logssms_amd.layers.linear_attention_backend import GatedDeltaBackend, PackedLinearIndices
from oracle import metadata as md


def _tables(seed, rows, cols, low=-1, high=500):
    rng = random.Random(seed)
    return [[rng.randrange(low, high) for _ in range(cols)] for _ in range(rows)]


@pytest.mark.parametrize("chunk_size", [16, 32, 64])
def test_packed_indices_match_oracle(chunk_size):
    rng = random.Random(chunk_size)
    for _ in range(20):
        lengths = [rng.choice([1, 2, 63, 64, 65, 127, 128, 129, rng.randrange(1, 700)])
                   for _ in range(rng.randrange(1, 9))]
        got = PackedLinearIndices.from_lengths(lengths, torch.device("cpu"), chunk_size)
        want = md.from_lengths(lengths, chunk_size)
        assert got.cu_seqlens.tolist() == want["cu_seqlens"]
        assert got.chunk_indices.tolist() == want["chunk_indices"]
        assert got.chunk_offsets.tolist() == want["chunk_offsets"]
        assert got.endings.tolist() == want["endings"]
        assert got.conv_chunks.tolist() == want["conv_chunks"]
        assert got.fla_kwargs()["chunk_indices"] is got.chunk_indices
        assert got.chunk_indices.tolist() == md.prepare_chunk_indices(want["cu_seqlens"], chunk_size)
        assert got.chunk_offsets.tolist() == md.prepare_chunk_offsets(want["cu_seqlens"], chunk_size)


def test_decode_graph_metadata_uses_capture_buffers():
    """tests/layers/test_linear_attention_backend.py:100-129 (same tables and answer)."""
    backend = GatedDeltaBackend()
    ctx = Context(page_size=64)
    ctx.linear_state = SimpleNamespace(device=torch.device("cpu"))
    ctx.state_table = torch.tensor([[3] * 64 + [4] * 64, [5] * 64 + [6] * 64, [9] * 128], dtype=torch.int32)
    real = Request(0, 64, 65)
    dummy = Request(2, 0, 1)
    batch = Batch(reqs=[real], phase="decode", padded_reqs=[real, dummy])
    capture = Batch(reqs=[dummy, dummy], phase="decode")
    set_global_ctx(ctx)
    try:
        backend.init_capture_graph(max_seq_len=128, bs_list=[2])
        backend.prepare_for_capture(capture)
        assert capture.linear_attn_metadata.read_slots.data_ptr() == backend.capture.read_slots.data_ptr()
        backend.prepare_metadata(batch)
        backend.prepare_for_replay(batch)
    finally:
        clear_global_ctx()
    assert backend.capture.read_slots.tolist() == [3, 9]
    assert backend.capture.write_slots.tolist() == [4, 9]


def test_decode_slots_match_oracle():
    table = _tables(1, 6, 96)
    ctx = Context(page_size=64, state_table=torch.tensor(table, dtype=torch.int32))
    reqs = [(t, c) for t, c in [(0, 1), (3, 95), (5, 64), (2, 0), (1, 30)]]
    batch = Batch(reqs=[Request(t, c, c + 1) for t, c in reqs], phase="decode")
    ctx.linear_attn_backend.prepare_metadata(batch)
    read, write = md.decode_slots(table, reqs)
    meta = batch.linear_attn_metadata
    assert meta.read_slots.tolist() == read and meta.write_slots.tolist() == write
    assert meta.read_slots.dtype == torch.int64 and meta.slots.shape == (5, 2)


def test_verify_metadata_uses_live_baseline_and_reserve():
    """tests/layers/test_linear_attention_backend.py:203-237."""
    ctx = Context(page_size=64)
    ctx.state_table = torch.tensor([[11] * 64 + [12] * 64 + [13] * 64, [20] * 64 + [21] * 64 + [22] * 64],
                                   dtype=torch.int32)
    ctx.work_state_table = torch.tensor([[100, 101, 102], [110, 111, 112]], dtype=torch.int32)
    batch = Batch(reqs=[Request(0, 62, 65), Request(1, 128, 130)], phase="verify")
    ctx.linear_attn_backend.prepare_metadata(batch)
    groups = batch.linear_attn_metadata.verify_groups
    assert list(groups) == [3, 2]
    rows3, reads3, writes3 = groups[3]
    rows2, reads2, writes2 = groups[2]
    assert rows3.tolist() == [0, 1, 2] and reads3.tolist() == [11] and writes3.tolist() == [[100, 101, 102]]
    assert rows2.tolist() == [3, 4] and reads2.tolist() == [21] and writes2.tolist() == [[110, 111]]


def test_verify_groups_match_oracle():
    table = _tables(2, 8, 200, low=0)
    work = _tables(3, 8, 16, low=0)
    rng = random.Random(4)
    reqs = [(t, rng.randrange(1, 180), rng.choice([1, 2, 4, 8, 16])) for t in range(8)]
    ctx = Context(page_size=64, state_table=torch.tensor(table), work_state_table=torch.tensor(work))
    batch = Batch(reqs=[Request(t, c, c + e) for t, c, e in reqs], phase="verify")
    ctx.linear_attn_backend.prepare_metadata(batch)
    got = batch.linear_attn_metadata.verify_groups
    want = md.verify_groups(table, work, reqs)
    assert list(got) == list(want)
    for n, (rows, base, writes) in want.items():
        assert got[n][0].tolist() == rows and got[n][1].tolist() == base and got[n][2].tolist() == writes


def _prefill(ctx, reqs, cache_metadata=None):
    batch = Batch(reqs=[Request(t, c, c + e) for t, c, e in reqs], phase="prefill", cache_metadata=cache_metadata)
    ctx.linear_attn_backend.prepare_metadata(batch)
    return batch.linear_attn_metadata


_FIELDS = ("baseline_slots", "checkpoint_slots", "checkpoint_chunks", "chunk_write_slots", "snapshot_rows",
           "snapshot_reqs", "conv_token_slots")


@pytest.mark.parametrize("page", [64, 128, 256])
def test_prefill_metadata_matches_oracle(page):
    table = _tables(page, 6, 1200)
    reqs = [(0, 0, 1), (1, 64 * 3, 700), (2, 0, page), (3, page, page + 1), (4, 128, 63), (5, 0, 1000)]
    ctx = Context(page_size=page, state_table=torch.tensor(table))
    meta = _prefill(ctx, reqs)
    want = md.prefill_metadata(table, reqs, page)
    for name in _FIELDS:
        assert getattr(meta, name).tolist() == want[name], name
    idx = meta.prefill_indices
    assert idx.cu_seqlens.tolist() == md.from_lengths([e for _, _, e in reqs])["cu_seqlens"]


def test_prefill_metadata_page_checkpoints_known_layout():
    """Two pages of 64 plus a 16-token tail, one page already cached: one
    checkpoint per page boundary plus the final one, each at the chunk holding
    the boundary's last token and the token row before it."""
    table = [[7] * 64 + [8] * 64 + [9] * 64 + [10] * 64]
    ctx = Context(page_size=64, state_table=torch.tensor(table))
    meta = _prefill(ctx, [(0, 64, 144)])
    assert meta.baseline_slots.tolist() == [7]
    assert meta.checkpoint_slots.tolist() == [8, 9, 10]
    assert meta.checkpoint_chunks.tolist() == [0, 1, 2]
    assert meta.chunk_write_slots.tolist() == [8, 9, 10]
    assert meta.snapshot_rows.tolist() == [63, 127, 143]
    assert meta.conv_token_slots[[63, 127, 143]].tolist() == [8, 9, 10]
    assert (meta.conv_token_slots >= 0).sum().item() == 3


def test_prefill_metadata_sparse_and_grouped_match_oracle():
    table = _tables(9, 3, 900)
    reqs = [(0, 0, 300), (1, 128, 256), (2, 64, 5)]
    sparse = [[(64, 41), (256, 42), (300, 43)], [(256, 44)], [(5, 45)]]
    ctx = Context(page_size=128, state_table=torch.tensor(table))
    meta = _prefill(ctx, reqs, MarconiCacheMetadata(checkpoint_writes=sparse))
    want = md.prefill_metadata(table, reqs, 128, sparse=sparse)
    for name in _FIELDS:
        assert getattr(meta, name).tolist() == want[name], name
    ctx.linear_state = SimpleNamespace(group_table=None)
    meta = _prefill(ctx, reqs)
    want = md.prefill_metadata(table, reqs, 128, group_table=True)
    for name in _FIELDS:
        assert getattr(meta, name).tolist() == want[name], name


def test_prefill_rejects_unaligned_resume():
    ctx = Context(page_size=64, state_table=torch.zeros(1, 256, dtype=torch.int64))
    with pytest.raises(AssertionError):
        _prefill(ctx, [(0, 30, 10)])


@pytest.mark.parametrize("block_size, width", [(0, 1), (64, 7), (128, 4), (256, 2), (448, 1), (512, 1)])
def test_hybrid_layout_matches_reference_table(block_size, width):
    """tests/hybrid/test_marconi.py:17-30 (Qwen3.5-like: 16 attention layers,
    48 linear layers, state (24,128,128), conv window (5120,3), 2x256 KV)."""
    spec = SimpleNamespace(num_layers=48, state_shape=(24, 128, 128), conv_shape=(5120, 3))
    lay = HybridBlockLayout.make(16, spec, 2, 256, block_size)
    want = md.marconi_layout(16, 48, (24, 128, 128), (5120, 3), 2, 256, block_size)
    assert lay.block_size == want["block_size"] == (block_size or 448)
    assert lay.state_blocks_per_group == want["state_blocks_per_group"] == width
    assert lay.state_groups == want["state_groups"] == 3
    assert lay.layer_elements == want["layer_elements"]
    assert lay.state_blocks * lay.block_bytes(2) == 3 * width * 16 * lay.block_size * 2048


def test_hybrid_layout_rejects_bad_sizes():
    spec = SimpleNamespace(num_layers=4, state_shape=(2, 8, 8), conv_shape=(40, 3))
    for size in (-64, 16, 65):
        with pytest.raises(ValueError):
            HybridBlockLayout.make(2, spec, 1, 8, size)
    with pytest.raises(ValueError):
        HybridBlockLayout.make(0, spec, 1, 8, 64)


def _small_pool(num_blocks=12):
    spec = SimpleNamespace(num_layers=4, state_shape=(2, 8, 8), conv_shape=(40, 3))
    lay = HybridBlockLayout.make(2, spec, 1, 2, 64)  # 256 elements per lane-block, state 248 -> 1 block
    return HybridBlockPool(lay, num_blocks, "cpu", torch.float32)


def test_hybrid_pool_views_address_the_block_storage():
    pool = _small_pool()
    lay = pool.layout
    assert pool.recurrent_state.shape == (12 - lay.state_blocks_per_group + 1, 2, 2, 8, 8)
    pool.recurrent_state[5, 1, 1, 3, 4] = 1.5
    pool.conv_state[5, 1, 39, 2] = 2.5
    flat = pool.storage[1, 5]
    assert flat[1 * 64 + 3 * 8 + 4].item() == 1.5
    assert flat[128 + 39 * 3 + 2].item() == 2.5
    assert flat.count_nonzero().item() == 2


def test_hybrid_pool_allocate_release_and_map():
    pool = _small_pool()
    a, b = pool.allocate_state(), pool.allocate_state()
    assert a != b
    groups = pool.group_table.tolist()
    assert len(set(groups[a] + groups[b])) == 2 * pool.layout.state_groups
    pool.retain_state(a)
    pool.release_state(a)
    assert a in pool.state_blocks
    pool.release_state(a)
    assert a not in pool.state_blocks
    rng = random.Random(5)
    values = [rng.choice([-1, b, -3, b]) for _ in range(9)]
    from logssms_amd.layers.linear_attention_backend import LinearAttnMetadata

    meta = LinearAttnMetadata(phase="prefill", baseline_slots=torch.tensor(values),
                              chunk_write_slots=torch.tensor(values[::-1]))
    for layer in range(4):
        mapped, lane = pool.map_metadata(meta, layer)
        want, want_lane = md.map_slots(groups, values, layer, pool.layout.layers_per_group)
        assert lane == want_lane
        assert mapped.baseline_slots.tolist() == want
        assert mapped.chunk_write_slots.tolist() == md.map_slots(groups, values[::-1], layer, 2)[0]
        assert mapped.read_slots is None


def test_hybrid_pool_exhaustion():
    pool = _small_pool(num_blocks=4)
    pool.allocate_state(), pool.allocate_state()
    with pytest.raises(RuntimeError):
        pool.allocate_state()


def test_commit_speculative_matches_oracle():
    rng = random.Random(6)
    for trial in range(40):
        page = rng.choice([4, 8, 64])
        C = rng.randrange(0, 3 * page)
        n = rng.randrange(1, 9)
        table = [[rng.randrange(0, 1000) for _ in range(4 * page + 8)] for _ in range(2)]
        work = [[rng.randrange(1000, 2000) for _ in range(8)] for _ in range(2)]
        t, w = torch.tensor(table), torch.tensor(work)
        commit_speculative(t, w, 1, C, n, page)
        md.commit_speculative(table, work, 1, C, n, page)
        assert t.tolist() == table and w.tolist() == work, trial


def test_linear_state_pool_layout():
    pool = LinearStatePool(3, 2, 40, 4, 2, 8, 16, "cpu", torch.bfloat16)
    assert pool.conv_state.shape == (3, 2, 40, 3) and pool.conv_state.dtype == torch.bfloat16
    assert pool.recurrent_state.shape == (3, 2, 2, 8, 16) and pool.recurrent_state.dtype == torch.float32
    single = LinearStatePool(3, 2, 40, 4, 2, 8, 16, "cpu", torch.bfloat16, state_dtype=None)
    assert single.recurrent_state.dtype == torch.bfloat16


def _planner(page):
    from logssms_amd.cache import MarconiCheckpointer
    return MarconiCheckpointer(pool=None, page_size=page)


def test_marconi_checkpoint_plan_matches_oracle():
    """``cache/marconi/manager.py:248-270`` placement against the oracle's
    restatement on random requests: planned checkpoints inside and at both
    ends of the extension, page boundaries with and without a checkpoint."""
    from logssms_amd.cache import MarconiRequestState
    rng = random.Random(11)
    for trial in range(400):
        page = rng.choice([64, 128, 256])
        cached = rng.randrange(0, 6) * page
        device = cached + rng.randrange(1, 4 * page)
        candidates = sorted({rng.randrange(cached, device + page) // 64 * 64 for _ in range(rng.randrange(0, 4))})
        checkpoints = {e: 1000 + i for i, e in enumerate(candidates) if e > 0}
        if rng.random() < 0.3:
            checkpoints[device] = 2000
        states = (rng.randrange(0, 50), rng.randrange(50, 100))
        writes, copies = _planner(page).plan(MarconiRequestState(states, dict(checkpoints)), cached, device)
        want_writes, want_copies = md.marconi_checkpoint_writes(
            [dict(cached_len=cached, device_len=device, states=states, checkpoints=dict(checkpoints))], page)
        assert writes == want_writes[0], trial
        assert copies == want_copies, trial


def test_marconi_branch_checkpoint_known_answer():
    """tests/hybrid/test_marconi.py:226-268: a request of ps + 12 tokens with
    a branch checkpoint planned at ps writes [ps, ps + 12] to the two live
    states, and the branch slot receives a copy of the state at ps."""
    from logssms_amd.cache import MarconiRequestState
    from logssms_amd.core import Batch, Request
    ps = 64
    planner = _planner(ps)
    planner.requests[0] = MarconiRequestState(states=(7, 9), checkpoints={ps: 3})
    batch = Batch([Request(0, 0, ps + 12)], "prefill")
    planner.prepare_batch(batch)
    assert batch.cache_metadata.checkpoint_writes == [[(ps, 7), (ps + 12, 9)]]
    assert batch.cache_metadata.checkpoint_copies == [(7, 3)]
    decode = Batch([Request(0, ps + 12, ps + 13)], "decode")
    planner.prepare_batch(decode)
    assert decode.cache_metadata is None


def test_marconi_copy_blocks_rejects_aliasing():
    pool = _small_pool()
    with pytest.raises(ValueError):
        pool.copy_blocks([1, 2], [3, 3])
    with pytest.raises(ValueError):
        pool.copy_blocks([1, 2], [2, 4])
    with pytest.raises(ValueError):
        pool.copy_blocks([1], [2, 4])
    pool.copy_blocks([], [])


def test_chunk_entry_rejects_what_it_does_not_cover():
    """A token log without frame storage is rejected, and head_v_dim other
    than 32 or a multiple of 64 raises NotImplementedError (plain pools at
    any granularity, and frame tables), before anything is launched."""
    from logssms_amd.kernel.linear_attention import ChunkLogIO, ChunkStateIO, chunk_gated_delta_rule_to_cache
    T, H, dk, dv = 4, 1, 32, 48
    q = torch.zeros(1, T, H, dk, dtype=torch.bfloat16)
    v = torch.zeros(1, T, H, dv, dtype=torch.bfloat16)
    g = torch.zeros(1, T, H)
    cu = torch.tensor([0, T])
    slots = torch.tensor([-1])
    pool = torch.zeros(1, 1, H, dk, dv)
    io = ChunkStateIO(pool, slots, torch.tensor([-1]))
    log = ChunkLogIO(slots, torch.zeros(T, dtype=torch.int64), torch.zeros(1, 2, dtype=torch.int32), g, 64, 4, H)
    with pytest.raises(AssertionError):
        chunk_gated_delta_rule_to_cache(q, q, v, g, g, io, cu, log_io=log)
    with pytest.raises(NotImplementedError):
        chunk_gated_delta_rule_to_cache(q, q, v, g, g, ChunkStateIO(pool, slots, torch.tensor([-1])), cu,
                                        chunk_size=32)
    frames = ChunkStateIO(torch.zeros(4, 1024, dtype=torch.bfloat16), slots, torch.tensor([-1]),
                          payload_frames=torch.zeros(1, 1, dtype=torch.int32), frame_bytes=2048,
                          head_payload_bytes=2048)
    with pytest.raises(NotImplementedError):
        chunk_gated_delta_rule_to_cache(q, q, v, g, g, frames, cu)


@pytest.mark.parametrize("granularity", [16, 32, 64])
def test_logstate_prefill_plan_matches_oracle(granularity):
    """The vectorised LogState prefill plan (layers/linear_attention_logstate.py)
    against the oracle's token-by-token statement of logstate.py:215-272:
    random batches with granule-end and off-granule checkpoints (some
    duplicated, some past the batch), work and log checkpoint slots, and
    unlogged ranges (some clipped, some of absent requests)."""
    import numpy as np

    from logssms_amd.layers.linear_attention_logstate import logstate_prefill_plan
    rng = random.Random(granularity)
    for trial in range(60):
        n = rng.randrange(1, 6)
        lengths = [rng.choice([1, granularity - 1, granularity, granularity + 1, rng.randrange(1, 300)])
                   for _ in range(n)]
        cached = [rng.randrange(0, 500) for _ in range(n)]
        first = [rng.randrange(0, 256) for _ in range(n)]
        total = sum(lengths)
        writes = [(rng.randrange(0, total + 5), rng.randrange(0, 40)) for _ in range(rng.randrange(0, 12))]
        starts = np.concatenate([[0], np.cumsum(lengths)])
        for i in range(n):  # checkpoints at the marked rows too
            row = rng.randrange(lengths[i])
            writes.append((int(starts[i]) + lengths[i] - 1, rng.randrange(0, 40)))
            writes.append((int(starts[i]) + row, rng.randrange(0, 40)))
        if writes and rng.random() < 0.5:
            writes.append(writes[0])
        ranges = [(rng.randrange(-1, n + 1), cached[0] + rng.randrange(-20, 200), cached[0] + rng.randrange(0, 400))
                  for _ in range(rng.randrange(0, 4))]
        work = {s for s in range(40) if s % 3 == 0}
        got = logstate_prefill_plan(lengths, cached, first, writes, ranges, granularity, 7, lambda s: s in work)
        want = md.logstate_prefill_plan(lengths, cached, first, writes, ranges, granularity, 7, work)
        assert got.dtype == np.int32
        assert got[:total].tolist() == want["conv_slots"], trial
        assert got[total:2 * total].tolist() == want["conv_granules"], trial
        assert got[2 * total:3 * total].tolist() == want["log_enabled"], trial
        assert got[3 * total:].tolist() == want["chunk_writes"], trial
