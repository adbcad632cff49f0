"""The fused prefill (``gdn_prefill_fused``: conv + SiLU, q/k L2
normalisation and gates computed by the chunk kernel's staging waves from the
raw projections) against the two-step path (``gdn_prefill_frontend`` writing
q, k, v, g, beta, then ``gdn_chunk_gated_delta_rule``).  Both follow
``layers/linear_attention_backend/gdn.py:100-150``; the fused kernel repeats
the front end's arithmetic and rounding, so outputs, recurrent states and conv
windows must agree bit for bit.  The two-step path itself is checked against
the oracle in test_gpu_chunk.py / test_gpu_backend.py, and the backend (which
now takes the fused path) in test_gpu_backend.py."""

import pytest
import torch

from tests.gpu_util import DEV, gen, rand, randn

pytestmark = pytest.mark.gpu


def _cfg(H, HV, dk, dv, layer=1):
    from logssms_amd.layers import GatedDeltaConfig
    return GatedDeltaConfig(num_k_heads=H, num_v_heads=HV, head_k_dim=dk, head_v_dim=dv,
                            conv_dim=2 * H * dk + HV * dv, state_len=3, layer_idx=layer)


def _setup(cfg, lengths, g, state_dtype=torch.float32, slots=96, layers=2, io=torch.bfloat16):
    """Random pools and inputs; per sequence a baseline (or none), checkpoint
    slots at some chunk ends and at the end, and conv snapshots at the same
    rows plus one skipped (negative) snapshot."""
    from logssms_amd.cache import LinearStatePool
    pool = LinearStatePool(slots, layers, cfg.conv_dim, 4, cfg.num_v_heads, cfg.head_k_dim, cfg.head_v_dim, DEV,
                           io, state_dtype=state_dtype)
    pool.conv_state.copy_(randn(*pool.conv_state.shape, g=g, dtype=io))
    pool.recurrent_state.copy_(randn(*pool.recurrent_state.shape, g=g, std=0.1).to(state_dtype))
    T = sum(lengths)
    free = torch.randperm(slots, generator=g).tolist()
    baseline = [free.pop() if i % 3 != 1 else -1 for i in range(len(lengths))]
    n_chunks = [(n + 63) // 64 for n in lengths]
    chunk_write = [-1] * sum(n_chunks)
    rows, snap_slots = [], []
    c0 = t0 = 0
    for n, nc in zip(lengths, n_chunks):
        for c in range(nc):
            last = c == nc - 1
            if last or c % 2 == 1:
                s = free.pop()
                chunk_write[c0 + c] = s
                rows.append(t0 + (n - 1 if last else 64 * c + 63))
                snap_slots.append(s)
        c0 += nc
        t0 += n
    rows.append(0)
    snap_slots.append(-1)
    cu = torch.tensor([0] + torch.tensor(lengths).cumsum(0).tolist(), dtype=torch.int32)
    w = dict(
        mixed=randn(T, cfg.conv_dim, g=g, dtype=io),
        gate=randn(T, cfg.num_v_heads, g=g, dtype=io),
        beta=randn(T, cfg.num_v_heads, g=g, dtype=io),
        weight=randn(cfg.conv_dim, 1, 4, g=g, dtype=io, std=0.3),
        A_log=-rand(cfg.num_v_heads, g=g),
        dt_bias=randn(cfg.num_v_heads, g=g, std=0.5),
    )
    meta = dict(cu=cu, baseline=torch.tensor(baseline), chunk_write=torch.tensor(chunk_write),
                rows=torch.tensor(rows), snap_slots=torch.tensor(snap_slots))
    return pool, {k: v.to(DEV) for k, v in w.items()}, {k: v.to(DEV) for k, v in meta.items()}


def _two_step(cfg, pool, w, meta):
    from logssms_amd.kernel.linear_attention.fused_backend import prefill_frontend
    from logssms_amd.kernel.linear_attention.gdn import chunk_gated_delta_rule_to_cache
    from logssms_amd.kernel.linear_attention.state_io import ChunkStateIO
    q, k, v, g, b = prefill_frontend(w["mixed"], w["gate"], w["beta"], w["weight"], w["A_log"], w["dt_bias"], cfg,
                                     pool.conv_state, meta["cu"], meta["baseline"], meta["rows"], meta["snap_slots"])
    io = ChunkStateIO(storage=pool.recurrent_state, read_slots=meta["baseline"], chunk_write_slots=meta["chunk_write"],
                      layer=cfg.layer_idx)
    o, _ = chunk_gated_delta_rule_to_cache(q, k, v, g, b, io, meta["cu"], return_v_new=False)
    return o.squeeze(0)


def _fused(cfg, pool, w, meta):
    from logssms_amd.kernel.linear_attention.fused_backend import prefill_fused
    return prefill_fused(w["mixed"], w["gate"], w["beta"], w["weight"], w["A_log"], w["dt_bias"], cfg,
                         pool.conv_state, pool.recurrent_state, meta["cu"], meta["baseline"], meta["chunk_write"],
                         meta["rows"], meta["snap_slots"])


CASES = [
    # H, HV, dk, dv, lengths, state dtype, io dtype
    (2, 4, 128, 128, [1, 2, 3, 63, 64, 65, 130, 257], torch.float32, torch.bfloat16),
    (2, 2, 128, 64, [200, 5, 64, 129], torch.float32, torch.bfloat16),
    (2, 4, 64, 64, [1, 70, 64, 191, 2], torch.float32, torch.bfloat16),
    (4, 4, 32, 64, [33, 128, 3, 100], torch.float32, torch.bfloat16),
    (2, 4, 128, 128, [96, 1, 300], torch.bfloat16, torch.bfloat16),
    (2, 4, 128, 128, [1, 63, 64, 65, 200], torch.float32, torch.float16),
    (2, 4, 64, 64, [70, 3, 129], torch.float16, torch.float16),
]


@pytest.mark.parametrize("case", CASES, ids=[f"H{c[0]}_HV{c[1]}_dk{c[2]}_dv{c[3]}_{str(c[5])[6:]}_{str(c[6])[6:]}"
                                             for c in CASES])
def test_fused_prefill_equals_two_step_path(case):
    H, HV, dk, dv, lengths, sdt, io = case
    print(f"fused prefill case H={H} HV={HV} dk={dk} dv={dv} lengths={lengths} state={sdt} io={io}", flush=True)
    cfg = _cfg(H, HV, dk, dv)
    pool, w, meta = _setup(cfg, lengths, gen(100 + dk + dv + len(lengths)), sdt, io=io)
    conv0, state0 = pool.conv_state.clone(), pool.recurrent_state.clone()
    want = _two_step(cfg, pool, w, meta).clone()
    conv_want, state_want = pool.conv_state.clone(), pool.recurrent_state.clone()
    pool.conv_state.copy_(conv0)
    pool.recurrent_state.copy_(state0)
    got = _fused(cfg, pool, w, meta)
    assert got is not None, "shape should be covered by the fused kernel"
    torch.cuda.synchronize()
    assert torch.equal(got, want), f"output differs: max {float((got.float() - want.float()).abs().max()):.3e}"
    assert torch.equal(pool.recurrent_state, state_want), "recurrent states differ"
    assert torch.equal(pool.conv_state, conv_want), "conv windows differ"
    # the snapshots and checkpoints were written (the comparison is not vacuous)
    written = meta["snap_slots"][meta["snap_slots"] >= 0]
    assert not torch.equal(pool.conv_state[written], conv0[written])
    assert not torch.equal(pool.recurrent_state[written], state0[written])


def test_prefill_pool_offsets_beyond_2gib():
    """Both prefill paths on pool views whose offsets pass 2**31 bytes (the
    reference's conv layer stride of 1,487,011,840 elements, a 512 MiB state
    slot stride) give bit for bit what the fused path gives on compact pools:
    baseline states and conv histories are read from, and checkpoints and
    snapshots written to, the far rows."""
    from types import SimpleNamespace
    cfg = _cfg(2, 4, 128, 128)
    pool, w, meta = _setup(cfg, [70, 3, 130], gen(77), slots=8)
    conv0, state0 = pool.conv_state.clone(), pool.recurrent_state.clone()
    want = _fused(cfg, pool, w, meta).clone()
    conv_want, state_want = pool.conv_state.clone(), pool.recurrent_state.clone()
    slots, layers, C, S = conv0.shape
    ls = 1487011840
    conv_buf = torch.empty(ls * (layers - 1) + slots * C * S, device=DEV, dtype=conv0.dtype)
    ss = (1 << 27) + 64
    per_slot = state0[0].numel()
    state_buf = torch.empty(ss * (slots - 1) + per_slot, device=DEV, dtype=state0.dtype)
    wide = SimpleNamespace(conv_state=conv_buf.as_strided(conv0.shape, (C * S, ls, S, 1)),
                           recurrent_state=state_buf.as_strided(state0.shape, (ss,) + state0.stride()[1:]))
    used = torch.cat([meta["baseline"], meta["chunk_write"]])
    assert int(used.max()) * ss * state0.element_size() >= 1 << 31, "no state slot past 2 GiB is used"
    for path in (_fused, _two_step):
        wide.conv_state.copy_(conv0)
        wide.recurrent_state.copy_(state0)
        got = path(cfg, wide, w, meta)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{path.__name__}: output differs"
        assert torch.equal(wide.recurrent_state, state_want), f"{path.__name__}: states differ"
        assert torch.equal(wide.conv_state, conv_want), f"{path.__name__}: conv windows differ"


def test_fused_prefill_declines_uncovered_shapes():
    """dv = 32 is outside the fused kernel: the wrapper returns None (the
    backend then takes the two-step path) and writes nothing."""
    cfg = _cfg(2, 2, 32, 32)
    pool, w, meta = _setup(cfg, [70, 3], gen(5))
    conv0, state0 = pool.conv_state.clone(), pool.recurrent_state.clone()
    assert _fused(cfg, pool, w, meta) is None
    torch.cuda.synchronize()
    assert torch.equal(pool.conv_state, conv0) and torch.equal(pool.recurrent_state, state0)
