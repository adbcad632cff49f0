"""GPU parity of the HBM-bound kernels against the CPU oracle: conv (prefill and
decode), prepare_gdn, the fused prefill front end, recurrent decode / verify /
plain recurrence, and state-pool row I/O."""

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn as ref
from tests.gpu_util import DEV, assert_bf16_close, assert_state_close, gen, rand, randn

pytestmark = pytest.mark.gpu


def _cfg(H=2, HV=4, dk=32, dv=32, width=4, layer=1):
    from logssms_amd.layers import GatedDeltaConfig
    return GatedDeltaConfig(num_k_heads=H, num_v_heads=HV, head_k_dim=dk, head_v_dim=dv,
                            conv_dim=2 * H * dk + HV * dv, state_len=width - 1, layer_idx=layer)


# ------------------------------------------------------------------ conv decode

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("width", [2, 3, 4, 5, 6])
@pytest.mark.parametrize("slots", [([0, 2], [0, 2]), ([0, 2], [1, 2])])
@pytest.mark.parametrize("fused_input", [False, True])
def test_conv_decode_matches_oracle(dtype, width, slots, fused_input):
    from logssms_amd.kernel.linear_attention import conv_decode
    g = gen(93)
    cfg = _cfg(width=width)
    C = cfg.conv_dim
    x = randn(2, C, g=g, dtype=dtype)
    if fused_input:
        wide = randn(2, C + 40, g=g, dtype=dtype)
        wide[:, :C] = x
    weight = randn(C, 1, width, g=g, dtype=dtype, std=0.1)
    state = randn(3, 2, C, width - 1, g=g, dtype=dtype)
    reads, writes = slots
    expected_state = state.clone()
    want = ref.conv_decode(x, weight, expected_state, 1, reads, writes)
    dev_state = state.to(DEV)
    xin = wide.to(DEV)[:, :C] if fused_input else x.to(DEV)
    q, k, v = conv_decode(xin, weight.to(DEV), cfg, split_qkv=True,
                          read_slots=torch.tensor(reads, device=DEV), write_slots=torch.tensor(writes, device=DEV),
                          standard_state=dev_state)
    got = torch.cat([q.flatten(2), k.flatten(2), v.flatten(2)], -1)[:, 0]
    assert_bf16_close(got, want, rel=1e-2, atol=1e-2)
    torch.testing.assert_close(dev_state.cpu(), expected_state, rtol=0, atol=0)


def test_conv_decode_unsplit_round_and_scales():
    from logssms_amd.kernel.linear_attention import conv_decode
    g = gen(87)
    cfg = _cfg(width=4)
    C = cfg.conv_dim
    x = randn(3, C, g=g, dtype=torch.bfloat16)
    weight = randn(C, 1, 4, g=g, dtype=torch.bfloat16, std=0.2)
    bias = randn(C, g=g, dtype=torch.bfloat16, std=0.1)
    state = randn(4, 2, C, 3, g=g, dtype=torch.bfloat16)
    scales, bounds = (0.7, 0.8, 0.9), (64, 128)
    expected_state = state.clone()
    want = ref.conv_decode(x, weight, expected_state, 1, [0, 1, 2], [3, 1, 0], bias=bias, round_conv=True,
                           input_boundaries=bounds, input_scales=scales)
    dev_state = state.to(DEV)
    y = conv_decode(x.to(DEV), weight.to(DEV), cfg, bias=bias.to(DEV), round_conv=True,
                    read_slots=torch.tensor([0, 1, 2], device=DEV, dtype=torch.int32),
                    write_slots=torch.tensor([3, 1, 0], device=DEV, dtype=torch.int32),
                    standard_state=dev_state, input_boundaries=bounds, input_scales=scales)
    assert_bf16_close(y, want, rel=1e-2, atol=1e-2)
    torch.testing.assert_close(dev_state.cpu(), expected_state, rtol=0, atol=0)


# ------------------------------------------------------------------ packed conv

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("channels", [192, 65])
def test_packed_conv_matches_oracle_with_snapshots(dtype, channels):
    from logssms_amd.kernel.linear_attention import PackedConvStateIO, packed_causal_conv1d
    g = gen(31)
    lengths = [1, 2, 17, 79, 130]
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    T, W = cu[-1], 4
    wide = randn(T, 2 * channels, g=g, dtype=dtype)
    x = wide[:, ::2]
    weight = randn(channels, 1, W, g=g, dtype=dtype, std=0.1)
    history = randn(len(lengths), channels, W - 1, g=g, dtype=dtype)
    bias = randn(channels, g=g, dtype=dtype, std=0.05)
    y_ref, windows = ref.packed_causal_conv1d(x, weight, history, cu, bias)
    rows = [0, 2, 5, 19, 50, 98, 99, 228]
    slots = torch.full((T,), -1, dtype=torch.int32)
    slots[rows] = torch.arange(len(rows), dtype=torch.int32)
    storage = torch.zeros(len(rows) + len(lengths), 2, channels, W - 1, dtype=dtype)
    final = torch.arange(len(rows), len(rows) + len(lengths), dtype=torch.int64)
    dev_storage = storage.to(DEV)
    io = PackedConvStateIO(dev_storage, slots.to(DEV), final_slots=final.to(DEV), layer=1)
    cu_t = torch.tensor(cu, device=DEV)
    got = packed_causal_conv1d(wide.to(DEV)[:, ::2], weight.to(DEV), history.to(DEV), cu_t, None, bias.to(DEV),
                               state_io=io)
    assert_bf16_close(got, y_ref, rel=1e-2, atol=1e-2)
    out = dev_storage.cpu()
    for i, r in enumerate(rows):
        torch.testing.assert_close(out[i, 1], windows[r], rtol=0, atol=0)
    for n in range(len(lengths)):
        torch.testing.assert_close(out[len(rows) + n, 1], windows[cu[n + 1] - 1], rtol=0, atol=0)
    torch.testing.assert_close(out[:, 0], storage[:, 0], rtol=0, atol=0)


def test_packed_conv_input_scales():
    from logssms_amd.kernel.linear_attention import packed_causal_conv1d
    g = gen(88)
    C, W = 512, 4
    lengths = [7, 16]
    cu = [0, 7, 23]
    raw = randn(23, C + 32, g=g, dtype=torch.bfloat16)[:, :C]
    history = randn(2, C, 3, g=g, dtype=torch.bfloat16)
    weight = randn(C, 1, W, g=g, dtype=torch.bfloat16, std=0.2)
    scales, bounds = (0.7, 0.8, 0.9), (256, 384)
    want, _ = ref.packed_causal_conv1d(raw, weight, history, cu, None, input_boundaries=bounds,
                                       input_scales=scales)
    got = packed_causal_conv1d(raw.to(DEV), weight.to(DEV), history.to(DEV), torch.tensor(cu, device=DEV),
                               None, input_boundaries=bounds, input_scales=scales)
    assert_bf16_close(got, want, rel=1e-2, atol=1e-2)
    assert len(lengths) == 2


def test_packed_conv_graph_replay_reads_current_slots():
    """One capture, replays with new token and final snapshot slots: the
    windows land where the slot tensors say at replay time
    (tests/kernel/test_gdn_prefill_direct.py:271-283)."""
    from logssms_amd.kernel.linear_attention import PackedConvStateIO, packed_causal_conv1d
    g = gen(41)
    C, W = 256, 4
    cu = [0, 5, 70, 71]
    T, N = cu[-1], len(cu) - 1
    x = randn(T, C, g=g, dtype=torch.bfloat16)
    weight = randn(C, 1, W, g=g, dtype=torch.bfloat16, std=0.2)
    history = randn(N, C, W - 1, g=g, dtype=torch.bfloat16)
    y_ref, windows = ref.packed_causal_conv1d(x, weight, history, cu)
    storage = torch.zeros(12, 2, C, W - 1, device=DEV, dtype=torch.bfloat16)
    slots = torch.full((T,), -1, device=DEV, dtype=torch.int64)
    final = torch.full((N,), -1, device=DEV, dtype=torch.int64)
    io = PackedConvStateIO(storage, slots, final_slots=final, layer=1)
    args = (x.to(DEV), weight.to(DEV), history.to(DEV), torch.tensor(cu, device=DEV), None)
    out = packed_causal_conv1d(*args, state_io=io)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = packed_causal_conv1d(*args, state_io=io)
    plans = [({3: 0, 40: 1}, [2, 3, 4]), ({0: 5, 63: 6, 69: 7}, [-1, 8, 9]), ({}, [10, -1, 11])]
    for rows, fin in plans:
        storage.zero_()
        slots.fill_(-1)
        for r, s in rows.items():
            slots[r] = s
        final.copy_(torch.tensor(fin, device=DEV))
        graph.replay()
        torch.cuda.synchronize()
        assert_bf16_close(out, y_ref, rel=1e-2, atol=1e-2)
        got = storage.cpu()
        want = torch.zeros_like(got)
        for r, s in rows.items():
            want[s, 1] = windows[r]
        for n, s in enumerate(fin):
            if s >= 0:
                want[s, 1] = windows[cu[n + 1] - 1]
        torch.testing.assert_close(got, want, rtol=0, atol=0)


def test_conv_decode_graph_replay_reads_current_slots():
    """One capture of the single-token conv, replays with new read/write
    slots, including in-place updates (tests/layers/test_conv_decode.py:143-159)."""
    from logssms_amd.kernel.linear_attention import conv_decode
    g = gen(42)
    cfg = _cfg(width=4)
    C = cfg.conv_dim
    x = randn(3, C, g=g, dtype=torch.bfloat16)
    weight = randn(C, 1, 4, g=g, dtype=torch.bfloat16, std=0.2)
    state = randn(8, 2, C, 3, g=g, dtype=torch.bfloat16)
    dev_state = state.to(DEV)
    reads = torch.tensor([0, 1, 2], device=DEV)
    writes = torch.tensor([3, 4, 5], device=DEV)
    args = (x.to(DEV), weight.to(DEV), cfg)
    conv_decode(*args, read_slots=reads, write_slots=writes, standard_state=dev_state)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = conv_decode(*args, read_slots=reads, write_slots=writes, standard_state=dev_state)
    # (a slot written by one sequence is never read by another in the same step)
    for r, w in [([7, 6, 5], [0, 1, 2]), ([1, 3, 5], [1, 3, 5]), ([2, 0, 4], [6, 7, 3])]:
        reads.copy_(torch.tensor(r, device=DEV))
        writes.copy_(torch.tensor(w, device=DEV))
        expected_state = dev_state.cpu()
        want = ref.conv_decode(x, weight, expected_state, 1, r, w)
        graph.replay()
        torch.cuda.synchronize()
        assert_bf16_close(y, want, rel=1e-2, atol=1e-2)
        torch.testing.assert_close(dev_state.cpu(), expected_state, rtol=0, atol=0)


# ------------------------------------------------------------------ prepare_gdn

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("dims", [(32, 64), (128, 128), (64, 256)])
@pytest.mark.parametrize("repeats", [1, 2])
def test_prepare_gdn_strided(dtype, dims, repeats):
    from logssms_amd.kernel import prepare_gdn
    g = gen(11)
    kd, vd = dims
    B, T, H = 2, 17, 3
    HV = H * repeats
    raw = randn(B, T, 2 * H * kd + HV * vd + 8, g=g, dtype=dtype)
    q, k, v, _ = raw.split([H * kd, H * kd, HV * vd, 8], -1)
    q, k = [t.view(B, T, H, kd) for t in (q, k)]
    v = v.view(B, T, HV, vd)
    both = randn(B, T, 2 * HV, g=g, dtype=dtype)
    beta, gate = both.chunk(2, -1)
    a = (randn(2 * HV, g=g) * 0.1)[::2]
    bias = randn(2 * HV, g=g, dtype=dtype)[::2]
    q[:, 0] = 0
    k[:, -1] = 0
    gate[:, 0] = -40
    gate[:, -1] = 40
    beta[:, 0] = -40
    beta[:, -1] = 40
    want = ref.prepare_gdn(q, k, v, gate, beta, a, bias)
    dev_raw = raw.to(DEV)
    dq, dk_, dv_, _ = dev_raw.split([H * kd, H * kd, HV * vd, 8], -1)
    dq, dk_ = [t.view(B, T, H, kd) for t in (dq, dk_)]
    dv_ = dv_.view(B, T, HV, vd)
    dboth = both.to(DEV)
    dbeta, dgate = dboth.chunk(2, -1)
    got = prepare_gdn(dq, dk_, dv_, dgate, dbeta, a.to(DEV), bias.to(DEV))
    tol = 2e-3 if dtype == torch.bfloat16 else 5e-4 if dtype == torch.float16 else 1e-6
    for x, y in zip(got[:2], want[:2]):
        torch.testing.assert_close(x.cpu(), y, rtol=tol, atol=tol)
    torch.testing.assert_close(got[2].cpu(), want[2], rtol=0, atol=0)
    for x, y in zip(got[3:], want[3:]):
        torch.testing.assert_close(x.cpu(), y, rtol=2e-6, atol=1e-7)
        assert x.dtype == torch.float32
    assert all(t.is_contiguous() for t in got)


def test_prepare_gdn_softplus_edges_and_empty():
    from logssms_amd.kernel import prepare_gdn
    edges = torch.tensor([-80, -20, 0, 19.999, 20, 20.001, 80], dtype=torch.float32)
    gate = edges[None, :, None].expand(1, 7, 2).contiguous()
    q = torch.randn(1, 7, 1, 128)
    v = torch.randn(1, 7, 2, 128)
    z = torch.zeros(2)
    want = ref.prepare_gdn(q, q, v, gate, gate, z, z)
    got = prepare_gdn(*[t.to(DEV) for t in (q, q, v, gate, gate, z, z)])
    for x, y in zip(got[3:], want[3:]):
        torch.testing.assert_close(x.cpu(), y, rtol=2e-6, atol=1e-7)
    empty = prepare_gdn(*[t.to(DEV)[:, :0] if t.ndim > 1 else t.to(DEV) for t in (q, q, v, gate, gate)], z.to(DEV),
                        z.to(DEV))
    assert all(t.shape[1] == 0 for t in empty)


# ------------------------------------------------------------------ fused prefill front end

@pytest.mark.parametrize("dk", [32, 64, 128, 256])
def test_prefill_frontend_matches_conv_then_prepare(dk):
    from logssms_amd.kernel.linear_attention.fused_backend import prefill_frontend
    g = gen(5 + dk)
    H, HV = 2, 4
    cfg = _cfg(H=H, HV=HV, dk=dk, dv=dk, layer=1)
    C = cfg.conv_dim
    lengths = [3, 64, 100]
    cu = [0, 3, 67, 167]
    T = cu[-1]
    mixed = randn(T, C + 16, g=g, dtype=torch.bfloat16)[:, :C]
    weight = randn(C, 1, 4, g=g, dtype=torch.bfloat16, std=0.3)
    conv_state = randn(6, 2, C, 3, g=g, dtype=torch.bfloat16)
    gate = randn(T, HV, g=g, dtype=torch.bfloat16)
    beta = randn(T, HV, g=g, dtype=torch.bfloat16)
    A_log = randn(HV, g=g) * 0.5
    dt_bias = randn(HV, g=g) * 0.5
    baseline = torch.tensor([2, -1, 4])
    token_slots = torch.full((T,), -1, dtype=torch.int64)
    token_slots[[2, 66, 130, 166]] = torch.tensor([0, 1, 3, 5])
    # oracle: history gather, conv, snapshots, split, prepare
    hist = torch.zeros(3, C, 3, dtype=torch.bfloat16)
    for n, s in enumerate(baseline.tolist()):
        if s >= 0:
            hist[n] = conv_state[s, 1]
    y, windows = ref.packed_causal_conv1d(mixed, weight, hist, cu)
    q, k, v = ref.split_qkv(y[None], H, dk, HV, dk)
    want = ref.prepare_gdn(q, k, v, gate[None], beta[None], A_log, dt_bias)
    expected_pool = conv_state.clone()
    for t, s in enumerate(token_slots.tolist()):
        if s >= 0:
            expected_pool[s, 1] = windows[t]
    pool = conv_state.to(DEV)
    rows = (token_slots >= 0).nonzero().flatten()
    got = prefill_frontend(mixed.to(DEV), gate.to(DEV), beta.to(DEV), weight.to(DEV), A_log.to(DEV),
                           dt_bias.to(DEV), cfg, pool, torch.tensor(cu, device=DEV), baseline.to(DEV),
                           rows.to(DEV), token_slots[rows].to(DEV))
    for x, w in zip(got[:3], want[:3]):
        assert_bf16_close(x, w, rel=1e-2, atol=1e-2)
    for x, w in zip(got[3:], want[3:]):
        torch.testing.assert_close(x.cpu(), w, rtol=2e-6, atol=1e-7)
    torch.testing.assert_close(pool.cpu(), expected_pool, rtol=0, atol=0)
    assert len(lengths) == 3


# ------------------------------------------------------------------ recurrent

def _rec_inputs(g, B, T, H, HV, dk, dv, dtype=torch.bfloat16):
    return dict(
        query=randn(B, T, H, dk, g=g, dtype=dtype),
        key=randn(B, T, H, dk, g=g, dtype=dtype),
        value=randn(B, T, HV, dv, g=g, dtype=dtype),
        gate=randn(B, T, HV, g=g, dtype=dtype),
        beta=randn(B, T, HV, g=g, dtype=dtype),
        A_log=randn(HV, g=g),
        dt_bias=randn(HV, g=g),
    )


@pytest.mark.parametrize("pool_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dims", [(64, 64), (128, 128)])
@pytest.mark.parametrize("slots", [([1, 3], [1, 3]), ([1, 3], [2, 4])])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_recurrent_to_slots_matches_oracle(pool_dtype, dims, slots, index_dtype):
    from logssms_amd.kernel.linear_attention import fused_recurrent_gated_delta_rule_to_slots as to_slots
    g = gen(7)
    dk, dv = dims
    B, H, HV = 2, 2, 4
    inp = _rec_inputs(g, B, 1, H, HV, dk, dv)
    pool = randn(5, 2, HV, dk, dv, g=g, std=0.5).to(pool_dtype)
    reads, writes = slots
    expected = pool.clone()
    want = ref.fused_recurrent_to_slots(inp["query"], inp["key"], inp["value"], inp["gate"], inp["beta"],
                                        inp["A_log"], inp["dt_bias"], expected, reads, writes, 1)
    dpool = pool.to(DEV)
    d = {k: v.to(DEV) for k, v in inp.items()}
    got = to_slots(d["query"], d["key"], d["value"], d["gate"], d["beta"], d["A_log"], d["dt_bias"], dpool,
                   torch.tensor(reads, device=DEV, dtype=index_dtype),
                   torch.tensor(writes, device=DEV, dtype=index_dtype), 1)
    assert_bf16_close(got, want)
    tol = 1e-3 if pool_dtype == torch.float32 else 2e-2
    assert_state_close(dpool, expected, atol=tol)
    untouched = [s for s in range(5) if s not in writes]
    torch.testing.assert_close(dpool.cpu()[untouched], pool[untouched], rtol=0, atol=0)
    torch.testing.assert_close(dpool.cpu()[:, 0], pool[:, 0], rtol=0, atol=0)


def test_recurrent_to_slots_fused_gate_views():
    """tests/layers/test_linear_attention_backend.py:132-167: gate/beta as
    strided halves of one tensor; direct-store == gather -> recurrence -> scatter."""
    from logssms_amd.kernel.linear_attention import (fused_recurrent_gated_delta_rule,
                                                     fused_recurrent_gated_delta_rule_to_slots)
    g = gen(8)
    B, H, HV, dk = 2, 2, 4, 64
    inp = _rec_inputs(g, B, 1, H, HV, dk, dk)
    both = torch.cat([inp["beta"], inp["gate"]], -1).to(DEV)
    beta, gate = both.chunk(2, -1)
    d = {k: v.to(DEV) for k, v in inp.items()}
    pool = (torch.randn(5, 2, HV, dk, dk, generator=g)).to(torch.bfloat16).to(DEV)
    before = pool.clone()
    reads = torch.tensor([1, 3], device=DEV)
    writes = torch.tensor([2, 3], device=DEV)
    ref_o, ref_states = fused_recurrent_gated_delta_rule(d["query"], d["key"], d["value"], gate.contiguous(),
                                                         beta.contiguous(), d["A_log"], d["dt_bias"],
                                                         pool[:, 1].index_select(0, reads))
    out = fused_recurrent_gated_delta_rule_to_slots(d["query"], d["key"], d["value"], gate, beta, d["A_log"],
                                                    d["dt_bias"], pool, reads, writes, 1)
    expected = before.clone()
    expected[:, 1].index_copy_(0, writes, ref_states[:, 0])
    torch.testing.assert_close(out, ref_o, rtol=0, atol=0)
    torch.testing.assert_close(pool, expected, rtol=0, atol=0)


@pytest.mark.parametrize("T", [1, 5, 20])
def test_plain_recurrence_keeps_every_state(T):
    from logssms_amd.kernel.linear_attention import fused_recurrent_gated_delta_rule
    g = gen(9)
    B, H, HV, dk = 2, 2, 4, 128
    inp = _rec_inputs(g, B, T, H, HV, dk, dk)
    init = randn(B, HV, dk, dk, g=g, std=0.3)
    want_o, want_s = ref.fused_recurrent(inp["query"], inp["key"], inp["value"], inp["gate"], inp["beta"],
                                         inp["A_log"], inp["dt_bias"], init)
    d = {k: v.to(DEV) for k, v in inp.items()}
    o, s = fused_recurrent_gated_delta_rule(d["query"], d["key"], d["value"], d["gate"], d["beta"], d["A_log"],
                                            d["dt_bias"], init.to(DEV))
    assert_bf16_close(o, want_o)
    assert_state_close(s, want_s)


# ------------------------------------------------------------------ fused decode / verify

def _backend_inputs(g, cfg, rows, slots, io=torch.bfloat16):
    C = cfg.conv_dim
    return dict(
        mixed=randn(rows, C, g=g, dtype=io),
        gate=randn(rows, cfg.num_v_heads, g=g, dtype=io),
        beta=randn(rows, cfg.num_v_heads, g=g, dtype=io),
        weight=randn(C, 1, cfg.state_len + 1, g=g, dtype=io, std=0.3),
        A_log=-rand(cfg.num_v_heads, g=g),
        dt_bias=torch.zeros(cfg.num_v_heads),
        conv=randn(slots, 2, C, cfg.state_len, g=g, dtype=io),
        state=randn(slots, 2, cfg.num_v_heads, cfg.head_k_dim, cfg.head_v_dim, g=g, std=0.1),
    )


@pytest.mark.parametrize("in_place", [True, False])
@pytest.mark.parametrize("shape", [(2, 4, 64), (16, 32, 128)])
@pytest.mark.parametrize("io", [torch.bfloat16, torch.float16])
def test_decode_step_matches_oracle(in_place, shape, io):
    from logssms_amd.kernel.linear_attention.fused_backend import decode_step
    H, HV, d = shape
    g = gen(3)
    cfg = _cfg(H=H, HV=HV, dk=d, dv=d, layer=1)
    B, slots = 16, 40
    inp = _backend_inputs(g, cfg, B, slots, io)
    perm = torch.randperm(slots, generator=g)
    reads = perm[:B]
    writes = reads.clone() if in_place else perm[B:2 * B]
    conv_ref, state_ref = inp["conv"].clone(), inp["state"].clone()
    want = ref.forward_decode(inp["mixed"], inp["gate"], inp["beta"], inp["weight"], inp["A_log"], inp["dt_bias"],
                              conv_ref, state_ref, 1, reads, writes, H, d, HV, d)
    conv, state = inp["conv"].to(DEV), inp["state"].to(DEV)
    got = decode_step(inp["mixed"].to(DEV), inp["gate"].to(DEV), inp["beta"].to(DEV), inp["weight"].to(DEV),
                      inp["A_log"].to(DEV), inp["dt_bias"].to(DEV), cfg, conv, state, reads.to(DEV),
                      writes.to(DEV))
    assert_bf16_close(got, want)
    torch.testing.assert_close(conv.cpu(), conv_ref, rtol=0, atol=0)
    assert_state_close(state, state_ref)


def test_decode_step_graph_replay_reads_current_slots():
    from logssms_amd.kernel.linear_attention.fused_backend import decode_step
    g = gen(4)
    cfg = _cfg(H=2, HV=4, dk=64, dv=64, layer=0)
    B, slots = 4, 12
    inp = _backend_inputs(g, cfg, B, slots)
    d = {k: v.to(DEV) for k, v in inp.items()}
    reads = torch.tensor([0, 1, 2, 3], device=DEV)
    writes = torch.tensor([4, 5, 6, 7], device=DEV)
    out = torch.empty(B, cfg.num_v_heads, cfg.head_v_dim, device=DEV, dtype=torch.bfloat16)
    args = (d["mixed"], d["gate"], d["beta"], d["weight"], d["A_log"], d["dt_bias"], cfg, d["conv"], d["state"],
            reads, writes)
    decode_step(*args, out=out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        decode_step(*args, out=out)
    for it in range(3):
        reads.copy_(torch.tensor([8, 9, 10, 11], device=DEV) - it)
        writes.copy_(torch.tensor([0, 1, 2, 3], device=DEV) + it)
        conv_ref, state_ref = d["conv"].cpu(), d["state"].cpu()
        want = ref.forward_decode(inp["mixed"], inp["gate"], inp["beta"], inp["weight"], inp["A_log"],
                                  inp["dt_bias"], conv_ref, state_ref, 0, reads.cpu(), writes.cpu(), 2, 64, 4, 64)
        graph.replay()
        torch.cuda.synchronize()
        assert_bf16_close(out, want)
        torch.testing.assert_close(d["conv"].cpu(), conv_ref, rtol=0, atol=0)
        assert_state_close(d["state"], state_ref)


@pytest.mark.parametrize("permute_rows", [False, True])
@pytest.mark.parametrize("io", [torch.bfloat16, torch.float16])
def test_verify_group_matches_oracle(permute_rows, io):
    from logssms_amd.kernel.linear_attention.fused_backend import verify_group
    g = gen(12)
    H, HV, d = 16, 32, 128
    cfg = _cfg(H=H, HV=HV, dk=d, dv=d, layer=1)
    B, T, slots = 3, 8, 40
    rows = B * T
    inp = _backend_inputs(g, cfg, rows + 5, slots, io)
    perm = torch.randperm(slots, generator=g)
    baseline = perm[:B]
    writes = perm[B:B + B * T].view(B, T)
    row_idx = torch.randperm(rows + 5, generator=g)[:rows] if permute_rows else torch.arange(rows)
    conv_ref, state_ref = inp["conv"].clone(), inp["state"].clone()
    want = ref.forward_verify(inp["mixed"][row_idx], inp["gate"][row_idx], inp["beta"][row_idx], inp["weight"],
                              inp["A_log"], inp["dt_bias"], conv_ref, state_ref, 1, baseline, writes, H, d, HV, d)
    conv, state = inp["conv"].to(DEV), inp["state"].to(DEV)
    out = torch.zeros(rows + 5, HV, d, device=DEV, dtype=io)
    verify_group(inp["mixed"].to(DEV), inp["gate"].to(DEV), inp["beta"].to(DEV), inp["weight"].to(DEV),
                 inp["A_log"].to(DEV), inp["dt_bias"].to(DEV), cfg, conv, state,
                 row_idx.to(DEV) if permute_rows else None, baseline.to(DEV), writes.to(DEV), out)
    assert_bf16_close(out[row_idx.to(DEV)], want)
    torch.testing.assert_close(conv.cpu(), conv_ref, rtol=0, atol=0)
    assert_state_close(state, state_ref)


@pytest.mark.parametrize("shape", [(2, 4, 64, 21), (1, 8, 64, 5), (2, 16, 64, 18)],
                         ids=["T21_segments", "group8_stepwise", "group8_T18"])
def test_verify_beyond_fused_limits_matches_oracle(shape):
    """Verify groups of more than 16 drafts (16-step segments, each resuming
    from the previous segment's last write slot) and head groups of more than
    4 v-heads per key head (conv_decode + slotted recurrence per step) against
    the oracle's verify (the reference's fused_recurrent takes any T and head
    ratio, ``fused_recurrent.py:461-550``)."""
    from logssms_amd.kernel.linear_attention.fused_backend import verify_group
    H, HV, d, T = shape
    g = gen(13 + T)
    cfg = _cfg(H=H, HV=HV, dk=d, dv=d, layer=1)
    B = 3
    slots = B * (T + 1) + 4
    rows = B * T
    inp = _backend_inputs(g, cfg, rows + 3, slots)
    perm = torch.randperm(slots, generator=g)
    baseline = perm[:B]
    writes = perm[B:B + B * T].view(B, T)
    row_idx = torch.randperm(rows + 3, generator=g)[:rows]
    conv_ref, state_ref = inp["conv"].clone(), inp["state"].clone()
    want = ref.forward_verify(inp["mixed"][row_idx], inp["gate"][row_idx], inp["beta"][row_idx], inp["weight"],
                              inp["A_log"], inp["dt_bias"], conv_ref, state_ref, 1, baseline, writes, H, d, HV, d)
    conv, state = inp["conv"].to(DEV), inp["state"].to(DEV)
    out = torch.zeros(rows + 3, HV, d, device=DEV, dtype=torch.bfloat16)
    verify_group(inp["mixed"].to(DEV), inp["gate"].to(DEV), inp["beta"].to(DEV), inp["weight"].to(DEV),
                 inp["A_log"].to(DEV), inp["dt_bias"].to(DEV), cfg, conv, state, row_idx.to(DEV), baseline.to(DEV),
                 writes.to(DEV), out)
    assert_bf16_close(out[row_idx.to(DEV)], want)
    torch.testing.assert_close(conv.cpu(), conv_ref, rtol=0, atol=0)
    assert_state_close(state, state_ref)


def test_decode_step_wide_head_group_matches_oracle():
    from logssms_amd.kernel.linear_attention.fused_backend import decode_step
    H, HV, d = 2, 16, 64
    g = gen(14)
    cfg = _cfg(H=H, HV=HV, dk=d, dv=d, layer=1)
    B, slots = 5, 12
    inp = _backend_inputs(g, cfg, B, slots)
    perm = torch.randperm(slots, generator=g)
    reads, writes = perm[:B], torch.cat([perm[:2], perm[B:B + 3]])
    conv_ref, state_ref = inp["conv"].clone(), inp["state"].clone()
    want = ref.forward_decode(inp["mixed"], inp["gate"], inp["beta"], inp["weight"], inp["A_log"], inp["dt_bias"],
                              conv_ref, state_ref, 1, reads, writes, H, d, HV, d)
    conv, state = inp["conv"].to(DEV), inp["state"].to(DEV)
    got = decode_step(inp["mixed"].to(DEV), inp["gate"].to(DEV), inp["beta"].to(DEV), inp["weight"].to(DEV),
                      inp["A_log"].to(DEV), inp["dt_bias"].to(DEV), cfg, conv, state, reads.to(DEV), writes.to(DEV))
    assert_bf16_close(got, want)
    torch.testing.assert_close(conv.cpu(), conv_ref, rtol=0, atol=0)
    assert_state_close(state, state_ref)


def _wide_pools(conv, state):
    """Device views of `conv` / `state` whose element offsets pass 2**31 bytes:
    a 1 GiB slot stride for the state pool and the reference's conv layer
    stride of 1,487,011,840 elements (tests/layers/test_conv_decode.py:25-55)."""
    slots, layers, C, S = conv.shape
    _, _, HV, dk, dv = state.shape
    ls = 1487011840
    cbuf = torch.empty(ls * (layers - 1) + slots * C * S, device=DEV, dtype=conv.dtype)
    wide_conv = cbuf.as_strided(conv.shape, (C * S, ls, S, 1))
    ss = 1 << 28
    sbuf = torch.empty(ss * (slots - 1) + layers * HV * dk * dv, device=DEV, dtype=state.dtype)
    wide_state = sbuf.as_strided(state.shape, (ss, HV * dk * dv, dk * dv, dv, 1))
    wide_conv.copy_(conv.to(DEV))
    wide_state.copy_(state.to(DEV))
    return wide_conv, wide_state


def test_decode_and_verify_pool_offsets_beyond_2gib():
    """Slot and layer offsets above 2**31 bytes address the right rows: the
    layer-1 conv windows sit 2.97 GB into their buffer and slots >= 2 of the
    state pool past 2 GiB; outputs, windows and states equal the oracle on the
    compact pools."""
    from logssms_amd.kernel.linear_attention.fused_backend import decode_step, verify_group
    g = gen(31)
    H, HV, d = 2, 4, 64
    cfg = _cfg(H=H, HV=HV, dk=d, dv=d, layer=1)
    B, T, slots = 3, 2, 10
    inp = _backend_inputs(g, cfg, B * T, slots)
    reads = torch.tensor([1, 6, 3])
    writes = torch.tensor([7, 6, 2])  # one in place
    conv_ref, state_ref = inp["conv"].clone(), inp["state"].clone()
    want = ref.forward_decode(inp["mixed"][:B], inp["gate"][:B], inp["beta"][:B], inp["weight"], inp["A_log"],
                              inp["dt_bias"], conv_ref, state_ref, 1, reads, writes, H, d, HV, d)
    conv, state = _wide_pools(inp["conv"], inp["state"])
    got = decode_step(inp["mixed"][:B].to(DEV), inp["gate"][:B].to(DEV), inp["beta"][:B].to(DEV),
                      inp["weight"].to(DEV), inp["A_log"].to(DEV), inp["dt_bias"].to(DEV), cfg, conv, state,
                      reads.to(DEV), writes.to(DEV))
    assert_bf16_close(got, want)
    torch.testing.assert_close(conv.cpu(), conv_ref, rtol=0, atol=0)
    assert_state_close(state, state_ref)
    # verify from the decoded pools: per-step windows and states to far slots
    # (written slots disjoint from every baseline slot)
    base = torch.tensor([7, 2, 0])
    vwrites = torch.tensor([[5, 4], [1, 3], [8, 9]])
    want = ref.forward_verify(inp["mixed"], inp["gate"], inp["beta"], inp["weight"], inp["A_log"],
                              inp["dt_bias"], conv_ref, state_ref, 1, base, vwrites, H, d, HV, d)
    out = torch.zeros(B * T, HV, d, device=DEV, dtype=torch.bfloat16)
    verify_group(inp["mixed"].to(DEV), inp["gate"].to(DEV), inp["beta"].to(DEV), inp["weight"].to(DEV),
                 inp["A_log"].to(DEV), inp["dt_bias"].to(DEV), cfg, conv, state, None, base.to(DEV),
                 vwrites.to(DEV), out)
    assert_bf16_close(out, want)
    torch.testing.assert_close(conv.cpu(), conv_ref, rtol=0, atol=0)
    assert_state_close(state, state_ref)


# ------------------------------------------------------------------ state rows

@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_store_state_skips_negative(index_dtype, dtype):
    from logssms_amd.kernel import store_state
    g = gen(21)
    pool = randn(10, 4, 64, 64, g=g).to(dtype)
    states = randn(6, 4, 64, 64, g=g).to(dtype)
    idx = torch.tensor([3, -1, 0, 9, -5, 4], dtype=index_dtype)
    expected = pool.clone()
    ref.store_state(expected, idx, states)
    dpool = pool.to(DEV)
    store_state(dpool, idx.to(DEV), states.to(DEV))
    torch.testing.assert_close(dpool.cpu(), expected, rtol=0, atol=0)


def test_marconi_copy_and_zero_rows_segmented():
    """Row = `lanes` segments at the lane stride (cache/marconi/block_pool.py:32-41)."""
    from logssms_amd import _lib
    g = gen(22)
    lanes, blocks, elems = 3, 8, 1000
    storage = randn(lanes, blocks, elems, g=g)
    dst = torch.tensor([5, -1, 2])
    src = torch.tensor([1, 4, 6])
    expected = storage.clone()
    for d_, s_ in zip(dst.tolist(), src.tolist()):
        if d_ >= 0:
            expected[:, d_, :600] = storage[:, s_, :600]
    dev = storage.to(DEV)
    dst_d, src_d = dst.to(DEV), src.to(DEV)
    _lib.call("gdn_copy_rows", dev.data_ptr(), elems * 4, dst_d.data_ptr(), 1, dev.data_ptr(), elems * 4,
              src_d.data_ptr(), 1, 3, lanes, 600 * 4, blocks * elems * 4, _lib.stream_of(dev))
    torch.testing.assert_close(dev.cpu(), expected, rtol=0, atol=0)
    zero_idx = torch.tensor([7, 0], device=DEV)
    _lib.call("gdn_zero_rows", dev.data_ptr(), elems * 4, zero_idx.data_ptr(), 1, 2, lanes, elems * 4,
              blocks * elems * 4, _lib.stream_of(dev))
    expected[:, 7] = 0
    expected[:, 0] = 0
    torch.testing.assert_close(dev.cpu(), expected, rtol=0, atol=0)


def test_commit_accepted_copies_accepted_step():
    from logssms_amd import _lib
    g = gen(23)
    slots, L, HV, d, C = 12, 2, 4, 32, 96
    state = randn(slots, L, HV, d, d, g=g)
    conv = randn(slots, L, C, 3, g=g, dtype=torch.bfloat16)
    live = torch.tensor([0, 1, 2])
    writes = torch.tensor([[3, 4, 5], [6, 7, 8], [9, 10, 11]])
    accepted = torch.tensor([2, 0, 3], dtype=torch.int32)
    es, ec = state.clone(), conv.clone()
    for b in range(3):
        a = int(accepted[b])
        if 1 <= a <= 3:
            es[live[b], 1] = state[writes[b, a - 1], 1]
            ec[live[b], 1] = conv[writes[b, a - 1], 1]
    ds, dc = state.to(DEV), conv.to(DEV)
    lv, wr, ac = live.to(DEV), writes.to(DEV), accepted.to(DEV)
    _lib.call("gdn_commit_accepted", ds.data_ptr(), ds.stride(0) * 4, ds.stride(1) * 4, HV * d * d * 4,
              dc.data_ptr(), dc.stride(0) * 2, dc.stride(1) * 2, C * 3 * 2, lv.data_ptr(), 1, wr.data_ptr(),
              3, 1, 1, ac.data_ptr(), 0, 3, 3, _lib.stream_of(ds))
    torch.testing.assert_close(ds.cpu(), es, rtol=0, atol=0)
    torch.testing.assert_close(dc.cpu(), ec, rtol=0, atol=0)
    assert F is not None
