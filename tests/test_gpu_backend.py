"""End-to-end parity of ``GatedDeltaBackend`` (prefill / decode / verify through
the slot pools) against the CPU oracle, the reference backend tests'
invariants (packed == per-request, resume from a stored checkpoint), the
Marconi block pool's state I/O and the speculative commit."""

import pytest
import torch

from oracle import gdn as ref
from oracle import metadata as md
from tests.gpu_util import DEV, assert_bf16_close, assert_state_close, gen, rand, randn

pytestmark = pytest.mark.gpu


def _cfg(H=2, HV=4, dk=64, dv=64, width=4, layer=1):
    from logssms_amd.layers import GatedDeltaConfig
    return GatedDeltaConfig(num_k_heads=H, num_v_heads=HV, head_k_dim=dk, head_v_dim=dv,
                            conv_dim=2 * H * dk + HV * dv, state_len=width - 1, layer_idx=layer)


def _pool(cfg, slots, layers=2, g=None, state_dtype=torch.float32):
    from logssms_amd.cache import LinearStatePool
    pool = LinearStatePool(slots, layers, cfg.conv_dim, cfg.state_len + 1, cfg.num_v_heads, cfg.head_k_dim,
                           cfg.head_v_dim, DEV, torch.bfloat16, state_dtype=state_dtype)
    if g is not None:
        pool.conv_state.copy_(randn(*pool.conv_state.shape, g=g, dtype=torch.bfloat16))
        pool.recurrent_state.copy_(randn(*pool.recurrent_state.shape, g=g, std=0.1).to(state_dtype))
    return pool


def _weights(g, cfg, rows):
    return dict(
        mixed=randn(rows, cfg.conv_dim, g=g, dtype=torch.bfloat16),
        gate=randn(rows, cfg.num_v_heads, g=g, dtype=torch.bfloat16),
        beta=randn(rows, cfg.num_v_heads, g=g, dtype=torch.bfloat16),
        weight=randn(cfg.conv_dim, 1, cfg.state_len + 1, g=g, dtype=torch.bfloat16, std=0.3),
        A_log=-rand(cfg.num_v_heads, g=g),
        dt_bias=randn(cfg.num_v_heads, g=g, std=0.5),
    )


def _forward(ctx, batch, w, cfg, rows=None):
    backend = ctx.linear_attn_backend
    backend.prepare_metadata(batch)
    sl = slice(None) if rows is None else rows
    return backend.forward(w["mixed"][sl].to(DEV), w["gate"][sl].to(DEV), w["beta"][sl].to(DEV),
                           w["weight"].to(DEV), w["A_log"].to(DEV), w["dt_bias"].to(DEV), cfg, batch)


@pytest.mark.parametrize("dims", [(64, 64), (128, 128)])
def test_backend_prefill_matches_oracle(dims):
    from logssms_amd.core import Batch, Context, Request
    dk, dv = dims
    g = gen(41)
    cfg = _cfg(H=2, HV=4, dk=dk, dv=dv, layer=1)
    page = 64
    reqs = [(0, 0, 1), (1, 128, 200), (2, 0, 64), (3, 64, 63), (4, 0, 300)]
    slots = 64
    perm = torch.randperm(slots, generator=g).tolist()
    table = [[perm[(10 * i + p // page) % slots] for p in range(640)] for i in range(5)]
    T = sum(e for _, _, e in reqs)
    w = _weights(g, cfg, T)
    pool = _pool(cfg, slots, g=g)
    conv_ref, state_ref = pool.conv_state.cpu(), pool.recurrent_state.cpu()
    meta = md.prefill_metadata(table, reqs, page)
    cu = md.from_lengths([e for _, _, e in reqs])["cu_seqlens"]
    want = ref.forward_prefill(w["mixed"], w["gate"], w["beta"], w["weight"], w["A_log"], w["dt_bias"], conv_ref,
                               state_ref, 1, torch.tensor(cu), meta["baseline_slots"], meta["chunk_write_slots"],
                               meta["conv_token_slots"], 2, dk, 4, dv)
    ctx = Context(page_size=page, linear_state=pool, state_table=torch.tensor(table, device=DEV))
    got = _forward(ctx, Batch(reqs=[Request(t, c, c + e) for t, c, e in reqs], phase="prefill"), w, cfg)
    assert got.shape == (T, 4, dv)
    assert_bf16_close(got, want)
    torch.testing.assert_close(pool.conv_state.cpu(), conv_ref, rtol=0, atol=0)
    assert_state_close(pool.recurrent_state, state_ref)


def _reference_cfg():
    """The configuration of tests/layers/test_linear_attention_backend.py:240-255."""
    from logssms_amd.layers import GatedDeltaConfig
    return GatedDeltaConfig(num_k_heads=2, num_v_heads=2, head_k_dim=32, head_v_dim=32, conv_dim=192, state_len=3,
                            layer_idx=0)


def _reference_inputs(seed, rows, cfg):
    torch.manual_seed(seed)
    return dict(
        mixed=torch.randn(rows, cfg.conv_dim, dtype=torch.bfloat16),
        gate=torch.randn(rows, cfg.num_v_heads, dtype=torch.bfloat16),
        beta=torch.randn(rows, cfg.num_v_heads, dtype=torch.bfloat16),
        weight=torch.randn(cfg.conv_dim, 1, cfg.state_len + 1, dtype=torch.bfloat16) * 0.02,
        A_log=torch.zeros(cfg.num_v_heads),
        dt_bias=torch.zeros(cfg.num_v_heads),
    )


def test_packed_prefill_matches_individual_requests():
    """tests/layers/test_linear_attention_backend.py:240-330, with the bars of
    this build (packed and per-request runs share kernels, so they agree far
    inside the reference's 1e-2 / 5e-2)."""
    from logssms_amd.core import Batch, Context, Request
    cfg = _reference_cfg()
    lengths = [96, 64]
    w = _reference_inputs(11, sum(lengths), cfg)
    table = torch.tensor([[0] * 64 + [1] * 64, [2] * 64 + [-1] * 64], dtype=torch.int32, device=DEV)
    reqs = [Request(i, 0, n) for i, n in enumerate(lengths)]
    packed = _pool(cfg, 4, layers=1)
    ctx = Context(page_size=64, linear_state=packed, state_table=table)
    out = _forward(ctx, Batch(reqs=reqs, phase="prefill"), w, cfg).clone()
    single = _pool(cfg, 4, layers=1)
    ctx1 = Context(page_size=64, linear_state=single, state_table=table)
    parts, offset = [], 0
    for r, n in zip(reqs, lengths):
        parts.append(_forward(ctx1, Batch(reqs=[r], phase="prefill"), w, cfg, slice(offset, offset + n)).clone())
        offset += n
    assert_bf16_close(out, torch.cat(parts))
    torch.testing.assert_close(packed.conv_state[:3], single.conv_state[:3], rtol=0, atol=0)
    assert_state_close(packed.recurrent_state[:3], single.recurrent_state[:3], atol=1e-5)
    assert packed.recurrent_state[1].abs().sum() > 0 and packed.recurrent_state[2].abs().sum() > 0


@pytest.mark.parametrize("split", [64, 128])
def test_chunked_prefill_resumes_from_stored_checkpoint(split):
    """tests/layers/test_linear_attention_backend.py:333-428 (split 64 of 96),
    plus a two-page first half."""
    from logssms_amd.core import Batch, Context, Request
    cfg = _reference_cfg()
    seq_len = split + 32
    w = _reference_inputs(17, seq_len, cfg)
    table = torch.tensor([[0] * 64 + [1] * 64 + [2] * 64 + [3] * 64], dtype=torch.int32, device=DEV)
    full = _pool(cfg, 4, layers=1)
    full_ctx = Context(page_size=64, linear_state=full, state_table=table)
    full_out = _forward(full_ctx, Batch(reqs=[Request(0, 0, seq_len)], phase="prefill"), w, cfg).clone()
    resumed = _pool(cfg, 4, layers=1)
    ctx = Context(page_size=64, linear_state=resumed, state_table=table)
    first = _forward(ctx, Batch(reqs=[Request(0, 0, split)], phase="prefill"), w, cfg, slice(0, split)).clone()
    second = _forward(ctx, Batch(reqs=[Request(0, split, seq_len)], phase="prefill"), w, cfg,
                      slice(split, seq_len)).clone()
    assert_bf16_close(torch.cat([first, second]), full_out)
    last = (seq_len - 1) // 64
    torch.testing.assert_close(full.conv_state[last], resumed.conv_state[last], rtol=0, atol=0)
    assert_state_close(full.recurrent_state[last], resumed.recurrent_state[last], atol=1e-5)


def test_backend_decode_with_capture_matches_oracle():
    from logssms_amd.core import Batch, Context, Request
    g = gen(43)
    cfg = _cfg(H=4, HV=8, dk=128, dv=128, layer=0)
    slots, B = 40, 6
    pool = _pool(cfg, slots, g=g)
    perm = torch.randperm(slots, generator=g).tolist()
    table = [[perm[2 * i + (p >= 100)] for p in range(200)] for i in range(B + 1)]
    cached = [99, 5, 150, 100, 1, 120]
    reqs = [Request(i, c, c + 1) for i, c in enumerate(cached)]
    w = _weights(g, cfg, B)
    ctx = Context(page_size=64, linear_state=pool, state_table=torch.tensor(table, device=DEV))
    backend = ctx.linear_attn_backend
    backend.init_capture_graph(200, [B])
    d = {k: v.to(DEV) for k, v in w.items()}
    out = torch.empty(B, cfg.num_v_heads, cfg.head_v_dim, device=DEV, dtype=torch.bfloat16)
    warm = Batch(reqs=[Request(B, 0, 1)] * B, phase="decode")
    backend.prepare_for_capture(warm)
    conv_before, state_before = pool.conv_state.clone(), pool.recurrent_state.clone()
    backend.forward(d["mixed"], d["gate"], d["beta"], d["weight"], d["A_log"], d["dt_bias"], cfg, warm, out=out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        backend.forward(d["mixed"], d["gate"], d["beta"], d["weight"], d["A_log"], d["dt_bias"], cfg, warm,
                        out=out)
    pool.conv_state.copy_(conv_before)
    pool.recurrent_state.copy_(state_before)
    batch = Batch(reqs=reqs, phase="decode")
    backend.prepare_metadata(batch)
    backend.prepare_for_replay(batch)
    read, write = md.decode_slots(table, [(i, c) for i, c in enumerate(cached)])
    conv_ref, state_ref = conv_before.cpu(), state_before.cpu()
    want = ref.forward_decode(w["mixed"], w["gate"], w["beta"], w["weight"], w["A_log"], w["dt_bias"], conv_ref,
                              state_ref, 0, torch.tensor(read), torch.tensor(write), 4, 128, 8, 128)
    graph.replay()
    torch.cuda.synchronize()
    assert_bf16_close(out, want)
    torch.testing.assert_close(pool.conv_state.cpu(), conv_ref, rtol=0, atol=0)
    assert_state_close(pool.recurrent_state, state_ref)


def test_backend_verify_commit_then_decode():
    """Verify two length groups, commit the accepted drafts by slot remap, then
    decode one token: the decode must read the state after the last accepted
    draft (cache/radix/manager.py:248-268 + gdn.py:151-265)."""
    from logssms_amd.cache import commit_speculative
    from logssms_amd.core import Batch, Context, Request
    g = gen(44)
    cfg = _cfg(H=2, HV=4, dk=64, dv=64, layer=1)
    page, slots = 64, 64
    perm = torch.randperm(slots, generator=g).tolist()
    table = [[perm[3 * i + p // page] for p in range(192)] for i in range(3)]
    work = [perm[40 + 8 * i:40 + 8 * i + 8] for i in range(3)]
    cached = [70, 62, 100]
    drafts = [4, 4, 2]
    pool = _pool(cfg, slots, g=g)
    rows = sum(drafts)
    w = _weights(g, cfg, rows)
    state_table = torch.tensor(table, device=DEV)
    work_table = torch.tensor(work, device=DEV)
    ctx = Context(page_size=page, linear_state=pool, state_table=state_table, work_state_table=work_table)
    conv_ref, state_ref = pool.conv_state.cpu(), pool.recurrent_state.cpu()
    reqs = [(i, c, e) for i, (c, e) in enumerate(zip(cached, drafts))]
    got = _forward(ctx, Batch(reqs=[Request(t, c, c + e) for t, c, e in reqs], phase="verify"), w, cfg)
    want = torch.empty(rows, 4, 64, dtype=torch.float32)
    for n, (row_idx, base, writes) in md.verify_groups(table, work, reqs).items():
        r = torch.tensor(row_idx)
        want[r] = ref.forward_verify(w["mixed"][r], w["gate"][r], w["beta"][r], w["weight"], w["A_log"],
                                     w["dt_bias"], conv_ref, state_ref, 1, torch.tensor(base), torch.tensor(writes),
                                     2, 64, 4, 64).float()
    assert_bf16_close(got, want)
    torch.testing.assert_close(pool.conv_state.cpu(), conv_ref, rtol=0, atol=0)
    assert_state_close(pool.recurrent_state, state_ref)
    # accept 3, 1 and 2 drafts; the sampled token after them is the next decode input
    accepted = [3, 1, 2]
    host_table, host_work = [list(r) for r in table], [list(r) for r in work]
    for uid, (c, n) in enumerate(zip(cached, accepted)):
        commit_speculative(state_table, work_table, uid, c, n, page)
        md.commit_speculative(host_table, host_work, uid, c, n, page)
    assert state_table.tolist() == host_table and work_table.tolist() == host_work
    new_cached = [c + n for c, n in zip(cached, accepted)]
    dec = _weights(gen(45), cfg, 3)
    got = _forward(ctx, Batch(reqs=[Request(i, c, c + 1) for i, c in enumerate(new_cached)], phase="decode"),
                   dec | {k: w[k] for k in ("weight", "A_log", "dt_bias")}, cfg)
    read, write = md.decode_slots(host_table, list(enumerate(new_cached)))
    want = ref.forward_decode(dec["mixed"], dec["gate"], dec["beta"], w["weight"], w["A_log"], w["dt_bias"],
                              conv_ref, state_ref, 1, torch.tensor(read), torch.tensor(write), 2, 64, 4, 64)
    assert_bf16_close(got, want)
    assert_state_close(pool.recurrent_state, state_ref)
    torch.testing.assert_close(pool.conv_state.cpu(), conv_ref, rtol=0, atol=0)


def _hybrid(cfg, layers, num_blocks, block_size=64, dtype=torch.float32):
    from types import SimpleNamespace

    from logssms_amd.cache import HybridBlockLayout, HybridBlockPool
    spec = SimpleNamespace(num_layers=layers, state_shape=(cfg.num_v_heads, cfg.head_k_dim, cfg.head_v_dim),
                           conv_shape=(cfg.conv_dim, cfg.state_len))
    lay = HybridBlockLayout.make(2, spec, 2, 64, block_size)
    return HybridBlockPool(lay, num_blocks, DEV, dtype)


def test_marconi_pool_copy_zero_bit_exact():
    g = gen(46)
    cfg = _cfg(H=2, HV=4, dk=64, dv=64)
    pool = _hybrid(cfg, 4, 40)
    a, b = pool.allocate_state(), pool.allocate_state()
    pool.storage.copy_(randn(*pool.storage.shape, g=g).to(DEV))
    before = pool.storage.clone()
    pool.copy_state(a, b)
    width = pool.layout.state_blocks_per_group
    expect = before.clone()
    row = pool.recurrent_state[0, 0].numel() + pool.conv_state[0, 0].numel()
    for sa, sb in zip(pool.state_blocks[a][::width], pool.state_blocks[b][::width]):
        flat = expect.view(expect.shape[0], -1)
        src = before.view(before.shape[0], -1)
        start_a, start_b = sa * pool.layout.layer_elements, sb * pool.layout.layer_elements
        flat[:, start_b:start_b + row] = src[:, start_a:start_a + row]
    torch.testing.assert_close(pool.storage, expect, rtol=0, atol=0)
    pool.zero_state(a)
    for sa in pool.state_blocks[a][::width]:
        flat = expect.view(expect.shape[0], -1)
        flat[:, sa * pool.layout.layer_elements:sa * pool.layout.layer_elements + row] = 0
    torch.testing.assert_close(pool.storage, expect, rtol=0, atol=0)


def test_marconi_backend_prefill_matches_standard_pool():
    """Prefill through the Marconi block pool (map_metadata + lane-strided
    views) writes the same states and conv windows as the plain slot pool."""
    from logssms_amd.core import Batch, Context, MarconiCacheMetadata, Request
    g = gen(47)
    cfg = _cfg(H=2, HV=4, dk=64, dv=64, layer=3)
    hybrid = _hybrid(cfg, 4, 48, dtype=torch.bfloat16)
    logical = [hybrid.allocate_state() for _ in range(4)]
    plain = _pool(cfg, 48, layers=4, state_dtype=torch.bfloat16)
    reqs = [(0, 0, 200), (1, 0, 64)]
    sparse = [[(128, logical[0]), (200, logical[1])], [(64, logical[2])]]
    w = _weights(g, cfg, 264)
    table = torch.zeros(2, 256, dtype=torch.int64, device=DEV)
    batch_reqs = [Request(t, c, c + e) for t, c, e in reqs]
    out_h = _forward(Context(page_size=64, linear_state=hybrid, state_table=table),
                     Batch(reqs=batch_reqs, phase="prefill",
                           cache_metadata=MarconiCacheMetadata(checkpoint_writes=sparse)), w, cfg).clone()
    out_p = _forward(Context(page_size=64, linear_state=plain, state_table=table),
                     Batch(reqs=batch_reqs, phase="prefill",
                           cache_metadata=MarconiCacheMetadata(checkpoint_writes=sparse)), w, cfg).clone()
    torch.testing.assert_close(out_h, out_p, rtol=0, atol=0)
    group, lane = divmod(cfg.layer_idx, hybrid.layout.layers_per_group)
    for s in logical[:3]:
        blk = int(hybrid.group_table[s, group])
        torch.testing.assert_close(hybrid.recurrent_state[blk, lane], plain.recurrent_state[s, cfg.layer_idx],
                                   rtol=0, atol=0)
        torch.testing.assert_close(hybrid.conv_state[blk, lane], plain.conv_state[s, cfg.layer_idx], rtol=0, atol=0)
        assert hybrid.recurrent_state[blk, lane].abs().sum() > 0


@pytest.mark.parametrize("dims", [(128, 128), (32, 32)], ids=["fused_dv128", "two_step_dv32"])
def test_prefill_resuming_mid_page_writes_windows_after_reading_history(dims):
    """Page size 256 with prefixes cached to 64 and 192 tokens: a short
    extension's only checkpoint lands on the page the prefill resumed from,
    so its window slot is the baseline slot whose history the same prefill
    reads (``gdn.py:107-112`` gathers every history before any window is
    written).  d_v = 128 runs the fused path, d_v = 32 the two-step path."""
    from logssms_amd.core import Batch, Context, Request
    dk, dv = dims
    g = gen(77 + dk)
    cfg = _cfg(H=2, HV=4, dk=dk, dv=dv, layer=1)
    page = 256
    reqs = [(0, 64, 100), (1, 128, 200), (2, 0, 70), (3, 192, 64), (4, 64, 1)]
    slots = 32
    perm = torch.randperm(slots, generator=g).tolist()
    table = [[perm[(3 * i + p // page) % slots] for p in range(1024)] for i in range(5)]
    meta = md.prefill_metadata(table, reqs, page)
    aliased = [n for n, (t, c, e) in enumerate(reqs) if c and table[t][c - 1] == table[t][c + e - 1]]
    assert aliased == [0, 3, 4]
    T = sum(e for _, _, e in reqs)
    w = _weights(g, cfg, T)
    pool = _pool(cfg, slots, g=g)
    conv_ref, state_ref = pool.conv_state.cpu(), pool.recurrent_state.cpu()
    cu = md.from_lengths([e for _, _, e in reqs])["cu_seqlens"]
    want = ref.forward_prefill(w["mixed"], w["gate"], w["beta"], w["weight"], w["A_log"], w["dt_bias"], conv_ref,
                               state_ref, 1, torch.tensor(cu), meta["baseline_slots"], meta["chunk_write_slots"],
                               meta["conv_token_slots"], 2, dk, 4, dv)
    ctx = Context(page_size=page, linear_state=pool, state_table=torch.tensor(table, device=DEV))
    got = _forward(ctx, Batch(reqs=[Request(t, c, c + e) for t, c, e in reqs], phase="prefill"), w, cfg)
    assert_bf16_close(got, want)
    torch.testing.assert_close(pool.conv_state.cpu(), conv_ref, rtol=0, atol=0)
    assert_state_close(pool.recurrent_state, state_ref)


def test_marconi_checkpointer_writes_live_states_and_copies_the_branch():
    """``cache/marconi/manager.py:248-278`` end to end on the block pool: a
    prefill of ps + 12 tokens with a branch checkpoint planned at ps writes
    the states at ps and ps + 12 into the two live slots, and
    ``after_forward`` copies the live state at ps (state and conv window,
    every lane) into the branch slot in one launch.  The live states equal a
    plain slot pool run with the same writes bit for bit."""
    from logssms_amd.cache import MarconiCheckpointer, MarconiRequestState
    from logssms_amd.core import Batch, Context, MarconiCacheMetadata, Request
    g = gen(48)
    cfg = _cfg(H=2, HV=4, dk=64, dv=64, layer=2)
    hybrid = _hybrid(cfg, 4, 48, dtype=torch.bfloat16)
    hybrid.storage.copy_(randn(*hybrid.storage.shape, g=g, std=0.1).to(torch.bfloat16))
    s0, s1, branch = (hybrid.allocate_state() for _ in range(3))
    ps = hybrid.layout.block_size
    planner = MarconiCheckpointer(hybrid, ps)
    planner.requests[0] = MarconiRequestState((s0, s1), {ps: branch})
    T = ps + 12
    w = _weights(g, cfg, T)
    table = torch.zeros(1, 256, dtype=torch.int64, device=DEV)
    batch = Batch([Request(0, 0, T)], "prefill")
    planner.prepare_batch(batch)
    assert batch.cache_metadata.checkpoint_writes == [[(ps, s0), (T, s1)]]
    out_h = _forward(Context(page_size=ps, linear_state=hybrid, state_table=table), batch, w, cfg).clone()
    planner.after_forward(batch)
    plain = _pool(cfg, 48, layers=4, state_dtype=torch.bfloat16)
    sparse = MarconiCacheMetadata(checkpoint_writes=batch.cache_metadata.checkpoint_writes)
    out_p = _forward(Context(page_size=ps, linear_state=plain, state_table=table),
                     Batch([Request(0, 0, T)], "prefill", cache_metadata=sparse), w, cfg)
    torch.testing.assert_close(out_h, out_p, rtol=0, atol=0)
    group, lane = divmod(cfg.layer_idx, hybrid.layout.layers_per_group)
    blk = {s: int(hybrid.group_table[s, group]) for s in (s0, s1, branch)}
    for s in (s0, s1):
        torch.testing.assert_close(hybrid.recurrent_state[blk[s], lane], plain.recurrent_state[s, cfg.layer_idx],
                                   rtol=0, atol=0)
        torch.testing.assert_close(hybrid.conv_state[blk[s], lane], plain.conv_state[s, cfg.layer_idx], rtol=0, atol=0)
    for other_lane in range(hybrid.layout.layers_per_group):
        for g_ in range(hybrid.layout.state_groups):
            a, b = int(hybrid.group_table[s0, g_]), int(hybrid.group_table[branch, g_])
            torch.testing.assert_close(hybrid.recurrent_state[b, other_lane], hybrid.recurrent_state[a, other_lane],
                                       rtol=0, atol=0)
            torch.testing.assert_close(hybrid.conv_state[b, other_lane], hybrid.conv_state[a, other_lane],
                                       rtol=0, atol=0)
