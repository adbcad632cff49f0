"""Mixed prefill/decode batches and fixed-capacity graph replay on the GPU.

* ``gdn_metadata_pad`` / ``gdn_metadata_copy`` against the host rules
  (``kernel/metadata.py:108-150``), int32/int64, strided vectors, more fields
  than one launch holds.
* The reference's capacity-bucket test
  (``tests/layers/test_mixed_linear_graph.py:27-168``, radix pool): the
  prefill forward captured once at 128 input rows, then replayed for actual
  lengths 1..128 after ``MixedLinearCopyPlan`` refreshes the metadata, with
  NaN in every padding row, equals an eager actual-length run bit for bit
  (output rows and whole pools).  Run for d_v = 32 (two-step path) and
  d_v = 64 (fused prefill).
* ``forward_mixed`` (prefill part at a padded capacity + decode part) equals
  the two parts run separately, bit for bit."""

import pytest
import torch

from tests.gpu_util import DEV, gen, randn

pytestmark = pytest.mark.gpu


def test_metadata_pad_and_copy_kernels_match_host_rules():
    from logssms_amd.kernel.metadata import copy_metadata, pad_metadata
    g = gen(120)
    srcs, outs_d, outs_h, fills, tails = [], [], [], [], []
    for i in range(21):  # more than one launch's 16 fields
        dtype = torch.int64 if i % 3 else torch.int32
        n = int(torch.randint(0, 300, (1,), generator=g))
        pairs = i % 5 == 0
        src = torch.randint(-5, 1000, (n, 2) if pairs else (n,), generator=g).to(dtype)
        cap = n + int(torch.randint(0, 70, (1,), generator=g))
        shape = (cap, 2) if pairs else (cap,)
        srcs.append(src)
        outs_h.append(torch.empty(shape, dtype=dtype))
        outs_d.append(torch.full(shape, 12345, dtype=dtype, device=DEV))
        fills.append(0 if pairs or i % 2 == 0 else -1)  # pair tables pad with (0, tail), as the callers use them
        tails.append(cap if pairs else -1)
    pad_metadata(srcs, outs_h, fills, tails)
    pad_metadata([s.to(DEV) for s in srcs], outs_d, fills, tails)
    torch.cuda.synchronize()
    for h, d in zip(outs_h, outs_d):
        assert torch.equal(h, d.cpu())
    # strided vector copies (every other element of a guard buffer)
    storage = torch.full((64,), -777, device=DEV)
    source = torch.arange(96, device=DEV)[::3]
    copy_metadata((source, torch.arange(7, device=DEV, dtype=torch.int32)),
                  (storage[::2], torch.zeros(7, device=DEV, dtype=torch.int32)))
    torch.cuda.synchronize()
    assert torch.equal(storage[::2], source) and (storage[1::2] == -777).all()


LENGTHS = [128, 1, 31, 32, 63, 64, 65, 127, 128]


@pytest.mark.parametrize("dv", [32, 64])
def test_capacity_graph_replay_matches_actual_length_eager(dv):
    from logssms_amd.cache import LinearStatePool
    from logssms_amd.core import Batch, Context, Request, clear_global_ctx, set_global_ctx
    from logssms_amd.layers import GatedDeltaConfig, MixedLinearCopyPlan, prepare_mixed_linear_metadata
    from logssms_amd.layers.linear_attention_backend import GatedDeltaBackend
    print(f"capacity graph replay dv={dv}", flush=True)
    torch.manual_seed(387)
    dtype = torch.bfloat16
    cfg = GatedDeltaConfig(2, 2, 32, dv, 128 + 2 * dv, 3, 0)
    channels, heads = cfg.conv_dim, cfg.num_v_heads
    ctx = Context(page_size=64)
    ctx.linear_state = LinearStatePool(8, 1, channels, 4, heads, 32, dv, DEV, dtype)
    ctx.state_table = torch.tensor([[0] * 64 + [1] * 64, [6] * 128], dtype=torch.int32, device=DEV)
    buffers = (ctx.linear_state.conv_state, ctx.linear_state.recurrent_state)
    for tensor in buffers:
        tensor.normal_(0, .01)
    initial = tuple(t.clone() for t in buffers)
    set_global_ctx(ctx)
    backend = GatedDeltaBackend(ctx)

    def reset():
        for dst, src in zip(buffers, initial):
            dst.copy_(src)

    def batches(length):
        batch = Batch([Request(0, 0, length)], "prefill")
        decode = Batch([Request(1, 5, 6)], "decode")
        backend.prepare_metadata(batch)
        backend.prepare_metadata(decode)
        return batch, decode

    x = torch.randn(128, channels, dtype=dtype, device=DEV) * .1
    gate = torch.randn(128, heads, dtype=dtype, device=DEV) * .1
    beta = torch.randn_like(gate)
    weight = torch.randn(channels, 1, 4, dtype=dtype, device=DEV) * .02
    A, bias = (torch.randn(heads, device=DEV) * .1 for _ in range(2))
    static_x, static_gate, static_beta = x.clone(), gate.clone(), beta.clone()

    def forward(batch, inputs):
        a, b, c = inputs
        return backend.forward(a, b, c, weight, A, bias, cfg, batch)

    graph = None
    try:
        capture_batch, decode = batches(128)
        capture_batch.prefill_token_capacity = 128
        backend.prepare_metadata(capture_batch)
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
            expected_buffers = tuple(t.clone() for t in buffers)
            eager_batch.prefill_token_capacity = 128
            backend.prepare_metadata(eager_batch)
            fresh = prepare_mixed_linear_metadata(eager_batch, decode, 128)
            copy_plan.copy(fresh)
            for dst, src in ((static_x, x), (static_gate, gate), (static_beta, beta)):
                dst.copy_(src)
                dst[length:].fill_(float("nan"))  # padding must never affect live state
            reset()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(actual[:length], expected), f"dv={dv} L={length}: output"
            for observed, reference, baseline in zip(buffers, expected_buffers, initial):
                assert torch.equal(observed, reference), f"dv={dv} L={length}: pool"
                untouched = reference == baseline
                assert torch.equal(observed[untouched], baseline[untouched])
    finally:
        if graph is not None:
            graph.reset()
        clear_global_ctx()


def test_forward_mixed_equals_separate_parts():
    from logssms_amd.cache import LinearStatePool
    from logssms_amd.core import Batch, Context, Request, clear_global_ctx, set_global_ctx
    from logssms_amd.layers import GatedDeltaConfig, prepare_mixed_linear_metadata
    from logssms_amd.layers.linear_attention_backend import GatedDeltaBackend
    g = gen(121)
    cfg = GatedDeltaConfig(2, 4, 64, 64, 2 * 2 * 64 + 4 * 64, 3, 1)
    pool = LinearStatePool(40, 2, cfg.conv_dim, 4, 4, 64, 64, DEV, torch.bfloat16)
    pool.conv_state.copy_(randn(*pool.conv_state.shape, g=g, dtype=torch.bfloat16))
    pool.recurrent_state.copy_(randn(*pool.recurrent_state.shape, g=g, std=0.1))
    perm = torch.randperm(40, generator=g).tolist()
    table = torch.tensor([[perm[(5 * i + p // 64) % 40] for p in range(320)] for i in range(5)], device=DEV)
    ctx = Context(page_size=64, linear_state=pool, state_table=table)
    set_global_ctx(ctx)
    backend = GatedDeltaBackend(ctx)
    prefill_reqs = [Request(0, 0, 70), Request(1, 64, 130)]
    decode_reqs = [Request(2, 9, 10), Request(3, 100, 101), Request(4, 64, 65)]
    capacity = 160
    rows = capacity + len(decode_reqs)
    mixed = randn(rows, cfg.conv_dim, g=g, dtype=torch.bfloat16).to(DEV)
    gate = randn(rows, 4, g=g, dtype=torch.bfloat16).to(DEV)
    beta = randn(rows, 4, g=g, dtype=torch.bfloat16).to(DEV)
    weight = randn(cfg.conv_dim, 1, 4, g=g, dtype=torch.bfloat16, std=0.3).to(DEV)
    A_log, dt_bias = -torch.rand(4, generator=g).to(DEV), randn(4, g=g, std=0.5).to(DEV)
    n_pre = sum(r.extend_len for r in prefill_reqs)
    try:
        conv0, state0 = pool.conv_state.clone(), pool.recurrent_state.clone()
        # the two parts on their own (actual lengths)
        pre, dec = Batch(prefill_reqs, "prefill"), Batch(decode_reqs, "decode")
        backend.prepare_metadata(pre)
        backend.prepare_metadata(dec)
        want_pre = backend.forward(mixed[:n_pre], gate[:n_pre], beta[:n_pre], weight, A_log, dt_bias, cfg, pre).clone()
        want_dec = backend.forward(mixed[capacity:], gate[capacity:], beta[capacity:], weight, A_log, dt_bias, cfg,
                                   dec).clone()
        conv_want, state_want = pool.conv_state.clone(), pool.recurrent_state.clone()
        pool.conv_state.copy_(conv0)
        pool.recurrent_state.copy_(state0)
        # one mixed batch: prefill rows padded to the capacity, then the decode rows
        pre, dec = Batch(prefill_reqs, "prefill"), Batch(decode_reqs, "decode")
        backend.prepare_metadata(pre)
        backend.prepare_metadata(dec)
        prepare_mixed_linear_metadata(pre, dec, capacity)
        batch = Batch(prefill_reqs + decode_reqs, "mixed", num_prefill_reqs=2, mixed_parts=(pre, dec),
                      prefill_token_capacity=capacity)
        mixed[n_pre:capacity] = float("nan")
        got = backend.forward_mixed(batch, {"mixed_qkv": mixed, "gate": gate, "beta": beta}, conv_weight=weight,
                                    A_log=A_log, dt_bias=dt_bias, config=cfg)
        torch.cuda.synchronize()
        assert got.shape == (rows, 4, 64)
        assert torch.equal(got[:n_pre], want_pre) and torch.equal(got[capacity:], want_dec)
        assert torch.equal(pool.conv_state, conv_want) and torch.equal(pool.recurrent_state, state_want)
    finally:
        clear_global_ctx()
