"""``gdn_prefill_fused_noalloc`` (the fused prefill with its staging in the
library's per-GPU device array) against ``prefill_fused`` (the same kernels
with caller-allocated staging), bit for bit, on two calls in a row -- the
second smaller, so it runs over what the first left in the array -- and the
size limit it enforces before launching anything."""

import pytest
import torch

from tests.gpu_util import DEV, gen
from tests.test_gpu_fused_prefill import _cfg, _setup

pytestmark = pytest.mark.gpu


def _run_both(cfg, lengths, seed, **pool_args):
    from logssms_amd.kernel.linear_attention.fused_backend import prefill_fused, prefill_fused_noalloc
    pool_a, w, meta = _setup(cfg, lengths, gen(seed), **pool_args)
    pool_b, _, _ = _setup(cfg, lengths, gen(seed), **pool_args)
    assert torch.equal(pool_a.recurrent_state, pool_b.recurrent_state)
    T = sum(lengths)
    args = (w["mixed"], w["gate"], w["beta"], w["weight"].contiguous(), w["A_log"], w["dt_bias"], cfg)
    want = prefill_fused(*args, pool_a.conv_state, pool_a.recurrent_state, meta["cu"], meta["baseline"],
                         meta["chunk_write"], meta["rows"], meta["snap_slots"])
    assert want is not None
    out = torch.empty(T, cfg.num_v_heads, cfg.head_v_dim, device=DEV, dtype=w["mixed"].dtype)
    got = prefill_fused_noalloc(*args, pool_b.conv_state, pool_b.recurrent_state, meta["cu"], meta["baseline"],
                                meta["chunk_write"], meta["rows"], meta["snap_slots"], out)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(pool_b.recurrent_state, pool_a.recurrent_state)
    assert torch.equal(pool_b.conv_state, pool_a.conv_state)


def test_noalloc_prefill_equals_allocating_entry_point_twice():
    cfg = _cfg(2, 4, 128, 128)
    print("noalloc call 1: lengths [300, 64, 5, 130]", flush=True)
    _run_both(cfg, [300, 64, 5, 130], 901)
    print("noalloc call 2 (smaller): lengths [70, 3]", flush=True)
    _run_both(cfg, [70, 3], 902)


def test_noalloc_prefill_at_config2_shape():
    """BASELINE config 2's batch (4 x 4096 tokens, 16 / 32 heads, d = 128) fits
    the array: bit for bit against the allocating entry point."""
    from logssms_amd import _lib
    cfg = _cfg(16, 32, 128, 128, layer=0)
    lengths = [4096] * 4
    need = 2 * sum(lengths) * 16 * 128 * 2 + 2 * sum(lengths) * 32 * 4
    assert need <= _lib.lib().gdn_prefill_noalloc_scratch_bytes()
    print("noalloc config 2: 4 x 4096 tokens, 16 / 32 heads", flush=True)
    _run_both(cfg, lengths, 904, slots=160, layers=1)


def test_noalloc_prefill_rejects_inputs_beyond_its_scratch():
    from logssms_amd import _lib
    from logssms_amd.kernel.linear_attention.fused_backend import prefill_fused_noalloc
    cfg = _cfg(2, 4, 128, 128)
    per_token = 2 * 2 * 128 * 2 + 2 * 4 * 4
    T = _lib.lib().gdn_prefill_noalloc_scratch_bytes() // per_token + 64
    pool, w, meta = _setup(cfg, [64], gen(903))
    mixed = torch.zeros(T, cfg.conv_dim, device=DEV, dtype=torch.bfloat16)
    gate = torch.zeros(T, cfg.num_v_heads, device=DEV, dtype=torch.bfloat16)
    cu = torch.tensor([0, T], device=DEV, dtype=torch.int32)
    chunks = torch.full(((T + 63) // 64,), -1, device=DEV, dtype=torch.int64)
    out = torch.empty(T, cfg.num_v_heads, cfg.head_v_dim, device=DEV, dtype=torch.bfloat16)
    before = pool.recurrent_state.clone()
    with pytest.raises(RuntimeError, match="scratch"):
        prefill_fused_noalloc(mixed, gate, gate, w["weight"].contiguous(), w["A_log"], w["dt_bias"], cfg,
                              pool.conv_state, pool.recurrent_state, cu, meta["baseline"][:1], chunks,
                              meta["rows"][:0], meta["snap_slots"][:0], out)
    torch.cuda.synchronize()
    assert torch.equal(pool.recurrent_state, before)
