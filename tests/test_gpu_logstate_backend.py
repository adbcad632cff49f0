"""GPU tests of the LogState backend around the kernels:

* the reference's capacity-bucket graph test for ``gdn_logstate``
  (``tests/layers/test_mixed_linear_graph.py:27-168``, with and without
  checkpoints): the LogState prefill forward captured once at 128 input rows
  (d_k = d_v = 32, granularity 16, frame-table states), then replayed for
  actual lengths 1..128 after ``MixedLinearCopyPlan`` refreshes the
  metadata, with NaN in every padding row, equals an eager actual-length run
  bit for bit (output rows and the whole frame storage);
* ``forward_mixed`` on LogState metadata equals its two parts run separately;
* the engine's prepared packet (``gdn_gather_linear_slots``) gives the same
  decode / prefill metadata as the table path, standard and LogState,
  including the wrap of cached length 0 to the row's last column;
* every frame-table entry point treats a slot at or past the table's rows as
  it treats a negative slot (no read, no write);
* input scales on the LogState conv pools against the oracle.
"""

from types import SimpleNamespace

import pytest
import torch

from oracle import frames as ofr
from oracle import gdn as ref
from tests.gpu_util import DEV, assert_bf16_close, gen
from tests.test_gpu_logstate import _decode_pool

pytestmark = pytest.mark.gpu


def _device_read_conv(pool, C, S):
    """The pool's ``read_conv`` (cache/logstate/frame_pool.py:229-257) as
    device gathers, graph-capturable: windows [N, C, S] of the (slot,
    granule) snapshots, zeros for a negative slot or an unmapped frame (each
    snapshot sits in one frame here)."""
    fe = pool.frame_bytes // 2
    table = pool.conv_frame_table
    assert table.shape[2] == 1
    elems = torch.arange(C * S, device=DEV)

    def read_conv(slots, granules, layer):
        s = slots.long()
        fr = table[s.clamp_min(0), granules.long(), 0].long()
        ok = (s >= 0) & (fr >= 0)
        idx = (fr.clamp_min(0) * fe + layer * C * S)[:, None] + elems[None, :]
        vals = pool.storage.view(torch.bfloat16).reshape(-1)[idx].view(-1, C, S)
        return torch.where(ok[:, None, None], vals, torch.zeros((), dtype=vals.dtype, device=DEV))

    return read_conv


def _pool(g, slots, work, H, HV, d, page, gran, C, frame_bytes, head_bytes, layers=1):
    storage, payload, decay, conv, record, pool = _decode_pool(g, slots, H, HV, d, d, layers, page, gran, C, 4,
                                                               frame_bytes, head_bytes)
    pool.storage = storage.view(torch.uint8).to(DEV)
    pool.payload_frame_table, pool.decay_frame_table = payload.to(DEV), decay.to(DEV)
    pool.conv_frame_table = conv.to(DEV)
    pool.read_conv = _device_read_conv(pool, C, 3)
    pool.allocator = SimpleNamespace(slot=lambda s: SimpleNamespace(kind="work" if s in work else "log"))
    return pool


LENGTHS = [128, 1, 31, 32, 63, 64, 65, 127, 128]


@pytest.mark.parametrize("checkpoints", [False, True])
def test_logstate_capacity_graph_replay_matches_actual_length_eager(checkpoints):
    from logssms_amd.core import Batch, Context, LogStateCacheMetadata, Request, clear_global_ctx, set_global_ctx
    from logssms_amd.layers import (GatedDeltaConfig, GatedDeltaLogStateBackend, MixedLinearCopyPlan,
                                    prepare_mixed_linear_metadata)
    print(f"LogState capacity graph replay, checkpoints={checkpoints}", flush=True)
    torch.manual_seed(387)
    g = gen(387)
    cfg = GatedDeltaConfig(2, 2, 32, 32, 192, 3, 0)
    channels, heads = cfg.conv_dim, cfg.num_v_heads
    # slots 0, 1 log pages, 2, 3 work slots (tests/layers/test_logstate_linear_attention_backend.py:30-71)
    pool = _pool(g, 4, {2, 3}, 2, 2, 32, 64, 16, channels, 16384, 2048)
    ctx = Context(page_size=64, linear_state=pool,
                  state_table=torch.tensor([[0] * 64 + [1] * 64, [1] * 128], dtype=torch.int32, device=DEV),
                  work_state_table=torch.tensor([[2], [3]], dtype=torch.int32, device=DEV),
                  page_table=torch.arange(128, dtype=torch.int32, device=DEV).repeat(2, 1))
    set_global_ctx(ctx)
    backend = GatedDeltaLogStateBackend(ctx)
    initial = pool.storage.clone()

    def reset():
        pool.storage.copy_(initial)

    def batches(length):
        positions = torch.arange(length, dtype=torch.int32, device=DEV)
        batch = Batch([Request(0, 0, length)], "prefill", cache_metadata=LogStateCacheMetadata(first_offsets=[0]),
                      positions=positions, out_loc=positions)
        if checkpoints and length >= 64:
            batch.cache_metadata.checkpoint_ranges = [(0, 0, 64)]
            batch.cache_metadata.checkpoint_writes = [(63, 3)]
        five = torch.tensor([5], dtype=torch.int32, device=DEV)
        decode = Batch([Request(1, 5, 6)], "decode", positions=five, out_loc=five)
        backend.prepare_metadata(batch)
        backend.prepare_metadata(decode)
        return batch, decode

    x = torch.randn(128, channels, dtype=torch.bfloat16, device=DEV) * .1
    gate = torch.randn(128, heads, dtype=torch.bfloat16, device=DEV) * .1
    beta = torch.randn_like(gate)
    weight = torch.randn(channels, 1, 4, dtype=torch.bfloat16, device=DEV) * .02
    A, bias = (torch.randn(heads, device=DEV) * .1 for _ in range(2))
    static_x, static_gate, static_beta = x.clone(), gate.clone(), beta.clone()

    def forward(batch, inputs):
        a, b, c = inputs
        return backend.forward(a, b, c, weight, A, bias, cfg, batch)

    graph = None
    try:
        capture_batch, decode = batches(128)
        capture_batch.prefill_token_capacity = 128
        captured = prepare_mixed_linear_metadata(capture_batch, decode, 128)
        copy_plan = MixedLinearCopyPlan(captured)
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for _ in range(3):
                reset()
                forward(capture_batch, (static_x, static_gate, static_beta))
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        reset()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            actual = forward(capture_batch, (static_x, static_gate, static_beta))
        torch.cuda.synchronize()
        for length in LENGTHS:
            eager_batch, decode = batches(length)
            reset()
            expected = forward(eager_batch, (x[:length], gate[:length], beta[:length])).clone()
            expected_storage = pool.storage.clone()
            eager_batch.prefill_token_capacity = 128
            fresh = prepare_mixed_linear_metadata(eager_batch, decode, 128)
            copy_plan.copy(fresh)
            for dst, src in ((static_x, x), (static_gate, gate), (static_beta, beta)):
                dst.copy_(src)
                dst[length:].fill_(float("nan"))  # padding must never affect live state
            reset()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(actual[:length], expected), f"checkpoints={checkpoints} L={length}: output"
            assert torch.equal(pool.storage, expected_storage), f"checkpoints={checkpoints} L={length}: storage"
            assert not torch.equal(pool.storage, initial)
    finally:
        if graph is not None:
            graph.reset()
        clear_global_ctx()


def _logstate_world(g, rows=3, page=64, gran=16, d=64, H=2, HV=4):
    """A LogState pool with `rows` requests: row r logs page p to slot
    2 r + p (slots 0 .. 2 rows - 1) and works in slot 2 rows + r."""
    from logssms_amd.core import Context
    C = 2 * H * d + HV * d
    slots = 3 * rows
    pool = _pool(g, slots, set(range(2 * rows, 3 * rows)), H, HV, d, page, gran, C, 65536, HV * d * d * 2 // HV)
    width = 2 * page
    state = torch.tensor([[2 * r + p // page for p in range(width)] for r in range(rows)], dtype=torch.int32)
    ctx = Context(page_size=page, linear_state=pool, state_table=state.to(DEV),
                  work_state_table=torch.arange(2 * rows, 3 * rows, dtype=torch.int32, device=DEV)[:, None],
                  page_table=torch.arange(width, dtype=torch.int32, device=DEV).repeat(rows, 1))
    return ctx, C


def test_logstate_forward_mixed_equals_separate_parts():
    from logssms_amd.core import Batch, LogStateCacheMetadata, Request, clear_global_ctx, set_global_ctx
    from logssms_amd.layers import GatedDeltaConfig, GatedDeltaLogStateBackend, prepare_mixed_linear_metadata
    g = gen(131)
    H, HV, d = 2, 4, 64
    ctx, C = _logstate_world(g, rows=3, d=d, H=H, HV=HV)
    pool = ctx.linear_state
    set_global_ctx(ctx)
    cfg = GatedDeltaConfig(H, HV, d, d, C, 3, 0)
    backend = GatedDeltaLogStateBackend(ctx)
    prefill_reqs = [Request(0, 0, 70), Request(1, 20, 65)]
    decode_reqs = [Request(2, 30, 31)]
    n_pre, capacity = 70 + 45, 128
    rows = capacity + len(decode_reqs)
    mixed = (torch.randn(rows, C, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    gate = torch.randn(rows, HV, generator=g).to(torch.bfloat16).to(DEV)
    beta = torch.randn(rows, HV, generator=g).to(torch.bfloat16).to(DEV)
    weight = (torch.randn(C, 1, 4, generator=g) * 0.3).to(torch.bfloat16).to(DEV)
    A_log, dt_bias = (-torch.rand(HV, generator=g)).to(DEV), (torch.randn(HV, generator=g) * 0.5).to(DEV)

    def parts():
        pos = torch.tensor(list(range(70)) + list(range(20, 65)), dtype=torch.int32, device=DEV)
        # a checkpoint at token 63 of request 0 into log slot 5 (a snapshot target no other token writes)
        pre = Batch(prefill_reqs, "prefill", cache_metadata=LogStateCacheMetadata(checkpoint_writes=[(63, 5)]),
                    positions=pos, out_loc=pos)
        dpos = torch.tensor([30], dtype=torch.int32, device=DEV)
        dec = Batch(decode_reqs, "decode", cache_metadata=LogStateCacheMetadata(replay_counts=[14]),
                    positions=dpos, out_loc=dpos)
        backend.prepare_metadata(pre)
        backend.prepare_metadata(dec)
        return pre, dec

    try:
        initial = pool.storage.clone()
        pre, dec = parts()
        want_pre = backend.forward(mixed[:n_pre], gate[:n_pre], beta[:n_pre], weight, A_log, dt_bias, cfg, pre).clone()
        want_dec = backend.forward(mixed[capacity:], gate[capacity:], beta[capacity:], weight, A_log, dt_bias, cfg,
                                   dec).clone()
        storage_want = pool.storage.clone()
        pool.storage.copy_(initial)
        pre, dec = parts()
        prepare_mixed_linear_metadata(pre, dec, capacity)
        batch = Batch(prefill_reqs + decode_reqs, "mixed", num_prefill_reqs=2, mixed_parts=(pre, dec),
                      prefill_token_capacity=capacity)
        mixed[n_pre:capacity] = float("nan")
        print("LogState forward_mixed: prefill [70, 45 after 20], decode 1 at capacity 128", flush=True)
        got = backend.forward_mixed(batch, {"mixed_qkv": mixed, "gate": gate, "beta": beta}, conv_weight=weight,
                                    A_log=A_log, dt_bias=dt_bias, config=cfg)
        torch.cuda.synchronize()
        assert got.shape == (rows, HV, d)
        assert torch.equal(got[:n_pre], want_pre) and torch.equal(got[capacity:], want_dec)
        assert torch.equal(pool.storage, storage_want)
    finally:
        clear_global_ctx()


def test_prepared_packet_slots_match_table_path():
    """standard.py:114-117 and logstate.py:113-157: the packet path
    (``gdn_gather_linear_slots``) against the table path, bit for bit."""
    from logssms_amd.core import Batch, BatchIndices, Context, LogStateCacheMetadata, Request
    from logssms_amd.kernel.metadata import gather_linear_slots
    from logssms_amd.layers import GatedDeltaLogStateBackend
    from logssms_amd.layers.linear_attention_backend import GatedDeltaBackend
    g = gen(141)
    # ---- standard pool: cached_len 0 wraps to the row's last column
    table = torch.randint(-1, 900, (6, 256), generator=g, dtype=torch.int32)
    ctx = Context(page_size=64, state_table=table.to(DEV))
    backend = GatedDeltaBackend(ctx)
    reqs = [Request(0, 0, 1), Request(1, 255, 256), Request(2, 64, 65), Request(5, 17, 18), Request(3, 1, 2)]
    host = Batch(reqs, "decode")
    backend.prepare_metadata(host)
    packed = Batch(reqs, "decode")
    packed.prepared_indices = BatchIndices.make(packed, DEV)
    backend.prepare_metadata(packed)
    want = torch.tensor([[int(table[r.table_idx, r.cached_len - 1]), int(table[r.table_idx, r.cached_len])]
                         for r in reqs])
    assert torch.equal(host.linear_attn_metadata.slots.cpu(), want)
    assert torch.equal(packed.linear_attn_metadata.slots.cpu(), want)
    assert packed.linear_attn_metadata.slots.dtype == torch.int64
    # rows or positions outside the table give -1
    bad = SimpleNamespace(table_ids=torch.tensor([6, -1, 0], dtype=torch.int32, device=DEV),
                          cached_lens=torch.tensor([0, 3, 256], dtype=torch.int32, device=DEV))
    assert (gather_linear_slots(bad, ctx.state_table) == -1).all()

    # ---- LogState: decode and prefill
    ctx, C = _logstate_world(g, rows=3)
    backend = GatedDeltaLogStateBackend(ctx)
    dreqs = [Request(0, 70, 71), Request(1, 3, 4), Request(2, 127, 128)]
    dpos = torch.tensor([70, 3, 127], dtype=torch.int32, device=DEV)
    counts = [5, 0, 15]
    host = Batch(dreqs, "decode", cache_metadata=LogStateCacheMetadata(replay_counts=counts), positions=dpos,
                 out_loc=dpos)
    backend.prepare_metadata(host)
    packed = Batch(dreqs, "decode", cache_metadata=LogStateCacheMetadata(replay_counts=counts), positions=dpos,
                   out_loc=dpos)
    packed.prepared_indices = BatchIndices.make(packed, DEV, replay_counts=counts)
    backend.prepare_metadata(packed)
    for name in ("work_slots", "log_slots", "token_offsets", "conv_read_slots", "conv_read_granules",
                 "replay_counts"):
        a, b = getattr(host.linear_attn_metadata, name), getattr(packed.linear_attn_metadata, name)
        assert a.dtype == b.dtype == torch.int32 and torch.equal(a, b), name
    assert host.linear_attn_metadata.log_slots.tolist() == [1, 2, 5]
    assert host.linear_attn_metadata.work_slots.tolist() == [6, 7, 8]

    preqs = [Request(0, 0, 70), Request(2, 20, 65)]
    lengths = [70, 45]
    pos = torch.tensor(list(range(70)) + list(range(20, 65)), dtype=torch.int32, device=DEV)
    cache = dict(checkpoint_writes=[(63, 6), (114, 8)], checkpoint_ranges=[(1, 30, 40)])
    host = Batch(preqs, "prefill", cache_metadata=LogStateCacheMetadata(**cache), positions=pos, out_loc=pos)
    backend.prepare_metadata(host)
    packed = Batch(preqs, "prefill", cache_metadata=LogStateCacheMetadata(**cache), positions=pos, out_loc=pos)
    packed.prepared_indices = BatchIndices.make(packed, DEV)
    packed.prepared_indices.token_table_ids = torch.repeat_interleave(
        torch.tensor([0, 2], device=DEV), torch.tensor(lengths, device=DEV))
    backend.prepare_metadata(packed)
    for name in ("work_slots", "log_slots", "token_offsets", "conv_read_slots", "conv_read_granules",
                 "cu_seqlens", "chunk_write_slots", "log_write_slots", "conv_token_slots", "conv_token_granules"):
        a, b = getattr(host.linear_attn_metadata, name), getattr(packed.linear_attn_metadata, name)
        assert torch.equal(a.long(), b.long()), name
    m = host.linear_attn_metadata
    # request 1 resumes at position 20: its history is the snapshot of its previous position 19
    assert m.conv_read_slots.tolist() == [6, 4] and m.conv_read_granules.tolist() == [0, 1]


def _bounds_world(g):
    H, HV, d, page, gran = 2, 4, 64, 64, 32
    C = 2 * H * d + HV * d
    slots = 6
    pool = _pool(g, slots, {0, 1}, H, HV, d, page, gran, C, 65536, 16384)
    return pool, H, HV, d, C, slots


def _twice(pool, run):
    """run(out_of_range) on two copies of the storage: slots past the table
    (out_of_range=True) and -1 in their place.  Returns the two results and
    leaves the first storage in the pool."""
    start = pool.storage.clone()
    first = run(True)
    torch.cuda.synchronize()
    after_oob = pool.storage.clone()
    pool.storage.copy_(start)
    second = run(False)
    torch.cuda.synchronize()
    assert torch.equal(after_oob, pool.storage), "storage differs from the run with -1 slots"
    return first, second


def test_frame_table_slots_past_the_table_are_unmapped():
    """A slot at or past the frame table's rows reads and writes nothing,
    exactly as a negative slot, at every frame-table entry point."""
    from logssms_amd.kernel.linear_attention import ChunkLogIO, ChunkStateIO, chunk_gated_delta_rule_to_cache
    from logssms_amd.kernel.linear_attention.conv_decode import conv_decode
    from logssms_amd.kernel.linear_attention.gdn import fused_recurrent_gated_delta_rule_to_logstate
    from logssms_amd.kernel.linear_attention.logstate import (copy_states, restore_log_state_chains,
                                                             store_log_states)
    from logssms_amd.kernel.linear_attention.packed_conv import PackedConvStateIO, packed_causal_conv1d
    g = gen(151)
    pool, H, HV, d, C, rows = _bounds_world(g)
    pool.allocator = None  # restore's output-kind check would reject the sentinel outputs
    cfg = SimpleNamespace(key_dim=H * d, value_dim=HV * d, head_k_dim=d, head_v_dim=d, layer_idx=0, state_len=3,
                          conv_dim=C, num_k_heads=H, num_v_heads=HV)
    past = [rows, rows + 3, 1 << 20]

    def pick(oob, values):  # None entries become a past-the-table slot or -1
        out, k = [], 0
        for v in values:
            if v is None:
                out.append(past[k % len(past)] if oob else -1)
                k += 1
            else:
                out.append(v)
        return torch.tensor(out, device=DEV)

    frames16 = pool.storage.view(torch.bfloat16)
    # ---- chunked prefill with the token log (frame-table states, granularity 32)
    lengths = [70, 40]
    T = sum(lengths)
    cu = torch.tensor([0, 70, 110], device=DEV)
    q = torch.nn.functional.normalize(torch.randn(1, T, H, d, generator=g), dim=-1).to(torch.bfloat16).to(DEV)
    k = torch.nn.functional.normalize(torch.randn(1, T, H, d, generator=g), dim=-1).to(torch.bfloat16).to(DEV)
    v = torch.randn(1, T, HV, d, generator=g).to(torch.bfloat16).to(DEV)
    gg = (-torch.rand(1, T, HV, generator=g) * 0.3).to(DEV)
    bb = torch.sigmoid(torch.randn(1, T, HV, generator=g)).to(DEV)
    # states go to slots 0-3, the token log to slots 4-5 (a slot's frames hold states or a log, not both)
    logs = [None if t % 7 == 3 else 4 + t // 64 for t in range(T)]

    def chunk(oob):
        # 3 + 2 checkpoint intervals of 32 tokens
        io = ChunkStateIO(frames16, pick(oob, [None, 0]), pick(oob, [None, 1, 2, None, 3]),
                          final_write_slots=pick(oob, [1, None]), payload_frames=pool.payload_frame_table,
                          frame_bytes=pool.frame_bytes, head_payload_bytes=pool.head_payload_bytes, layer=0,
                          num_layers=1, granularity=32, page_size=64)
        log = ChunkLogIO(pick(oob, logs), torch.arange(T, device=DEV) % 64, pool.decay_frame_table, gg, 64,
                         pool.layout.log_decay_bytes, H)
        o, _ = chunk_gated_delta_rule_to_cache(q, k, v, gg, bb, io, cu, chunk_size=32, log_io=log,
                                               return_v_new=False)
        return o

    a, b = _twice(pool, chunk)
    assert torch.equal(a, b)
    # ---- LogState decode (replay) and the conv decode
    B = 3
    x = torch.randn(B, C, generator=g).to(torch.bfloat16).to(DEV)
    weight = (torch.randn(C, 1, 4, generator=g) * 0.3).to(torch.bfloat16).to(DEV)
    a_log, dt = (-torch.rand(HV, generator=g)).to(DEV), torch.zeros(HV, device=DEV)
    gate = torch.randn(B, 1, HV, generator=g).to(torch.bfloat16).to(DEV)
    beta = torch.randn(B, 1, HV, generator=g).to(torch.bfloat16).to(DEV)

    def decode(oob):
        qq, kk, vv = conv_decode(x, weight, cfg, split_qkv=True, read_slots=pick(oob, [None, 2, 3]),
                                 read_granules=torch.tensor([0, 1, 0], device=DEV),
                                 write_slots=pick(oob, [4, None, 5]), write_granules=torch.tensor([1, 0, 1],
                                                                                                  device=DEV),
                                 work_slots=pick(oob, [0, 1, None]), pool=pool)
        o = fused_recurrent_gated_delta_rule_to_logstate(
            qq, kk, vv, gate, beta, a_log, dt, pool, pick(oob, [None, 1, 0]), pick(oob, [2, None, 3]),
            torch.tensor([20, 5, 47], device=DEV), 0, torch.tensor([4, 5, 15], device=DEV))
        return torch.cat([qq.flatten(), kk.flatten(), vv.flatten(), o.flatten()])

    a, b = _twice(pool, decode)
    assert torch.equal(a, b)
    # ---- prefill conv windows to the conv snapshots
    xp = torch.randn(T, C, generator=g).to(torch.bfloat16).to(DEV)
    hist = torch.randn(2, C, 3, generator=g).to(torch.bfloat16).to(DEV)

    # each snapshot (slot, granule) has at most one writer: tokens 3, 40, 90 write (2, 1), (3, 1), (4, 0);
    # tokens 17, 71, 100 get slots past the table (or -1)
    targets = {3: 2, 17: None, 40: 3, 71: None, 90: 4, 100: None}

    def windows(oob):
        io = PackedConvStateIO(storage=frames16, slots=pick(oob, [targets.get(t, -1) for t in range(T)]),
                               granules=torch.tensor([0 if t == 90 else 1 for t in range(T)], device=DEV),
                               final_slots=pick(oob, [None, 1]), frame_table=pool.conv_frame_table,
                               frame_bytes=pool.frame_bytes, layer=0)
        return packed_causal_conv1d(xp, weight, hist, cu, None, state_io=io)

    a, b = _twice(pool, windows)
    assert torch.equal(a, b)
    # ---- log stores, restore chains, state copies
    keys = torch.randn(4, H, d, generator=g).to(torch.bfloat16).to(DEV)
    resid = torch.randn(4, HV, d, generator=g).to(torch.bfloat16).to(DEV)
    decays = (-torch.rand(4, HV, generator=g)).to(DEV)

    def stores(oob):
        store_log_states(pool, pick(oob, [2, None, 3, None]), torch.tensor([1, 2, 3, 4], device=DEV), keys, resid,
                         decays, 0)
        base, seg, out = (rows, rows + 1, rows + 2) if oob else (None, -1, -1)
        restore_log_state_chains(pool, [(base, [(seg, 0, 10), (2, 0, 6)], 0), (1, [(3, 0, 4)], out)])
        copy_states(pool, [rows if oob else -1, 1], [4, rows + 1 if oob else -1])
        return torch.zeros(1)

    _twice(pool, stores)


def test_logstate_conv_input_scales():
    """_conv_input_scale_args on LogState conv pools (packed_conv.py:172-192,
    conv_decode.py:293-352): the scaled, rounded inputs feed the conv and the
    snapshots (history unscaled), against the oracle."""
    from logssms_amd.kernel.linear_attention.conv_decode import conv_decode
    from logssms_amd.kernel.linear_attention.packed_conv import PackedConvStateIO, packed_causal_conv1d
    g = gen(161)
    pool, H, HV, d, C, rows = _bounds_world(g)
    cfg = SimpleNamespace(key_dim=H * d, value_dim=HV * d, head_k_dim=d, head_v_dim=d, layer_idx=0, state_len=3,
                          conv_dim=C, num_k_heads=H, num_v_heads=HV)
    scales, bounds = (0.7, 1.3, 0.45), (H * d, 2 * H * d + 64)
    weight = (torch.randn(C, 1, 4, generator=g) * 0.3).to(torch.bfloat16)
    fe = pool.frame_bytes // 2
    conv_table = pool.conv_frame_table.cpu()
    # ---- prefill: conv output and snapshots at chosen rows
    lengths = [50, 23]
    T = sum(lengths)
    cu = [0, 50, 73]
    x = torch.randn(T, C, generator=g).to(torch.bfloat16)
    hist = torch.randn(2, C, 3, generator=g).to(torch.bfloat16)
    slots = torch.full((T,), -1)
    granules = torch.zeros(T, dtype=torch.int64)
    for t, s, gr in [(0, 2, 0), (31, 3, 1), (49, 4, 0), (60, 5, 1)]:
        slots[t], granules[t] = s, gr
    y_ref, win = ref.packed_causal_conv1d(x, weight, hist, cu, input_boundaries=bounds, input_scales=scales)
    io = PackedConvStateIO(storage=pool.storage.view(torch.bfloat16), slots=slots.to(DEV), granules=granules.to(DEV),
                           final_slots=torch.tensor([0, 1], device=DEV), frame_table=pool.conv_frame_table,
                           frame_bytes=pool.frame_bytes, layer=0)
    y = packed_causal_conv1d(x.to(DEV), weight.to(DEV), hist.to(DEV), torch.tensor(cu, device=DEV), None,
                             state_io=io, input_boundaries=bounds, input_scales=scales)
    torch.cuda.synchronize()
    assert_bf16_close(y, y_ref, rel=1e-2, atol=1e-2)
    host = pool.storage.view(torch.bfloat16).cpu()
    for t, s, gr in [(0, 2, 0), (31, 3, 1), (49, 4, 0), (60, 5, 1), (49, 0, 0), (72, 1, 0)]:
        idx = ofr.conv_element_index(conv_table, [s], [gr], 0, C, 3, fe)
        assert torch.equal(host.reshape(-1)[idx].view(C, 3), win[t]), (t, s)
    # ---- decode from those snapshots
    expected = host.clone()
    xd = torch.randn(2, C, generator=g).to(torch.bfloat16)
    reads, rgr, writes, wgr, works = [3, 4], [1, 0], [2, 5], [1, 0], [0, 1]
    t = lambda v: torch.tensor(v)  # noqa: E731
    y_ref = ofr.conv_decode_logstate(xd, weight, expected, conv_table, pool.frame_bytes, 0, t(reads), t(rgr),
                                     t(writes), t(wgr), t(works), input_boundaries=bounds, input_scales=scales)
    y = conv_decode(xd.to(DEV), weight.to(DEV), cfg, read_slots=t(reads).to(DEV), read_granules=t(rgr).to(DEV),
                    write_slots=t(writes).to(DEV), write_granules=t(wgr).to(DEV), work_slots=t(works).to(DEV),
                    pool=pool, input_boundaries=bounds, input_scales=scales)
    torch.cuda.synchronize()
    assert_bf16_close(y, y_ref, rel=1e-2, atol=1e-2)
    assert torch.equal(pool.storage.view(torch.bfloat16).cpu(), expected)
