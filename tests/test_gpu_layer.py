"""``GatedDeltaNet`` (``layers/gated_delta.py:44-139``) end to end on the GPU:
merged projections split into strided views, the backend prefill and decode
through the global context, the gated RMS norm and the output projection.
The expected output recomputes everything after the projections with the
oracle (``oracle/gdn.py``) from the same projection outputs, so the check
covers the wiring of views, the gate/beta order of ``in_proj_ba`` and the
norm/out-projection, not the library GEMM."""

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn as ref
from oracle import metadata as md
from tests.gpu_util import DEV, assert_bf16_close, assert_state_close, gen, rand, randn

pytestmark = pytest.mark.gpu


def _layer(g, hidden, H, HV, dk, dv, layer_idx):
    from logssms_amd.layers import GatedDeltaNet
    net = GatedDeltaNet(hidden, H, HV, dk, dv, 4, 1e-6, layer_idx, device=DEV, dtype=torch.bfloat16)
    cfg = net.config
    net.in_proj_qkvz_weight.copy_(randn(cfg.conv_dim + cfg.value_dim, hidden, g=g, std=0.15))
    net.in_proj_ba_weight.copy_(randn(2 * HV, hidden, g=g, std=0.15))
    net.conv1d_weight.copy_(randn(cfg.conv_dim, 1, 4, g=g, std=0.3))
    net.dt_bias.copy_(randn(HV, g=g, std=0.5))
    net.A_log.copy_(-rand(HV, g=g))
    net.norm.weight.copy_(1.0 + randn(dv, g=g, std=0.2))
    net.out_proj_weight.copy_(randn(hidden, cfg.value_dim, g=g, std=0.08))
    return net


def _expected_output(net, core, z):
    cfg = net.config
    T = core.shape[0]
    normed = ref.rms_norm_gated(core.to(torch.bfloat16).reshape(T, cfg.num_v_heads, cfg.head_v_dim),
                                z.reshape(T, cfg.num_v_heads, cfg.head_v_dim), net.norm.weight.cpu(), net.norm.eps)
    return F.linear(normed.reshape(T, -1).float(), net.out_proj_weight.cpu().float())


def test_gated_delta_net_prefill_then_decode_matches_oracle():
    from logssms_amd.cache import LinearStatePool
    from logssms_amd.core import Batch, Context, Request, clear_global_ctx, set_global_ctx
    g = gen(90)
    hidden, H, HV, dk, dv, layer_idx = 64, 2, 4, 64, 64, 1
    net = _layer(g, hidden, H, HV, dk, dv, layer_idx)
    cfg = net.config
    page, slots = 64, 48
    pool = LinearStatePool(slots, 2, cfg.conv_dim, 4, HV, dk, dv, DEV, torch.bfloat16)
    pool.conv_state.copy_(randn(*pool.conv_state.shape, g=g, dtype=torch.bfloat16))
    pool.recurrent_state.copy_(randn(*pool.recurrent_state.shape, g=g, std=0.1))
    perm = torch.randperm(slots, generator=g).tolist()
    table = [[perm[(6 * i + p // page) % slots] for p in range(384)] for i in range(3)]
    reqs = [(0, 0, 70), (1, 128, 200), (2, 64, 129)]  # (table row, cached, device_len)
    T = sum(e - c for _, c, e in reqs)
    ctx = Context(page_size=page, linear_state=pool, state_table=torch.tensor(table, device=DEV))
    set_global_ctx(ctx)
    try:
        # ---- prefill
        x = randn(T, hidden, g=g, dtype=torch.bfloat16).to(DEV)
        batch = Batch(reqs=[Request(t, c, e) for t, c, e in reqs], phase="prefill")
        ctx.batch = batch
        ctx.linear_attn_backend.prepare_metadata(batch)
        mixed, z, beta, gate = (t.cpu() for t in net.proj(x))
        conv_ref, state_ref = pool.conv_state.cpu(), pool.recurrent_state.cpu()
        y = net.forward(x)
        torch.cuda.synchronize()
        meta = md.prefill_metadata(table, [(t, c, e - c) for t, c, e in reqs], page)
        cu = md.from_lengths([e - c for _, c, e in reqs])["cu_seqlens"]
        core = ref.forward_prefill(mixed, gate, beta, net.conv1d_weight.cpu(), net.A_log.cpu(), net.dt_bias.cpu(),
                                   conv_ref, state_ref, layer_idx, torch.tensor(cu), meta["baseline_slots"],
                                   meta["chunk_write_slots"], meta["conv_token_slots"], H, dk, HV, dv)
        assert y.shape == (T, hidden) and y.dtype == torch.bfloat16
        assert_bf16_close(y, _expected_output(net, core, z), rel=2e-2, atol=2e-2)
        torch.testing.assert_close(pool.conv_state.cpu(), conv_ref, rtol=0, atol=0)
        assert_state_close(pool.recurrent_state, state_ref)
        # ---- one decode token per request
        x1 = randn(len(reqs), hidden, g=g, dtype=torch.bfloat16).to(DEV)
        batch = Batch(reqs=[Request(t, e, e + 1) for t, _, e in reqs], phase="decode")
        ctx.batch = batch
        ctx.linear_attn_backend.prepare_metadata(batch)
        mixed, z, beta, gate = (t.cpu() for t in net.proj(x1))
        y1 = net.forward(x1)
        torch.cuda.synchronize()
        read, write = md.decode_slots(table, [(t, e) for t, _, e in reqs])
        core = ref.forward_decode(mixed, gate, beta, net.conv1d_weight.cpu(), net.A_log.cpu(), net.dt_bias.cpu(),
                                  conv_ref, state_ref, layer_idx, torch.tensor(read), torch.tensor(write), H, dk,
                                  HV, dv)
        assert_bf16_close(y1, _expected_output(net, core, z), rel=2e-2, atol=2e-2)
        torch.testing.assert_close(pool.conv_state.cpu(), conv_ref, rtol=0, atol=0)
        assert_state_close(pool.recurrent_state, state_ref)
    finally:
        clear_global_ctx()


def test_gated_delta_net_projection_views_are_strided_slices():
    """proj() returns views into the two projection outputs (no copies), with
    beta before gate in in_proj_ba (gated_delta.py:99-105)."""
    g = gen(91)
    net = _layer(g, 32, 2, 4, 32, 32, 0)
    x = randn(5, 32, g=g, dtype=torch.bfloat16).to(DEV)
    mixed, z, beta, gate = net.proj(x)
    cfg = net.config
    assert mixed.shape == (5, cfg.conv_dim) and z.shape == (5, cfg.value_dim)
    assert mixed.stride(0) == cfg.conv_dim + cfg.value_dim and z.data_ptr() == mixed.data_ptr() + 2 * cfg.conv_dim
    ba = F.linear(x, net.in_proj_ba_weight)
    assert torch.equal(beta, ba[:, :4]) and torch.equal(gate, ba[:, 4:])
