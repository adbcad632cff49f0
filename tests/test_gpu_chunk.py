"""GPU parity of the chunked gated-delta-rule prefill (MFMA kernel) against the
CPU oracle, including pool slot semantics, varlen packing, GQA and HIP-graph
replay (tests/kernel/test_gdn_prefill_dispatch.py:143-197 is the model)."""

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn as ref
from tests.gpu_util import DEV, assert_bf16_close, assert_state_close, gen

pytestmark = pytest.mark.gpu


def _inputs(g, T, H, HV, dk, dv, dtype, g_scale=0.1):
    q = F.normalize(torch.randn(T, H, dk, generator=g), dim=-1).to(dtype)
    k = F.normalize(torch.randn(T, H, dk, generator=g), dim=-1).to(dtype)
    v = torch.randn(T, HV, dv, generator=g).to(dtype)
    gg = -torch.rand(T, HV, generator=g) * g_scale
    beta = torch.sigmoid(torch.randn(T, HV, generator=g))
    return q, k, v, gg, beta


def _run(q, k, v, gg, beta, storage, reads, writes, cu, finals=None, layer=0):
    from logssms_amd.kernel.linear_attention import ChunkStateIO, chunk_gated_delta_rule_to_cache
    io = ChunkStateIO(storage, reads, writes, final_write_slots=finals, layer=layer)
    return chunk_gated_delta_rule_to_cache(q[None], k[None], v[None], gg[None], beta[None], io, cu)


def _report(name, a, b):
    err = (a.float().cpu() - b.float().cpu()).abs()
    print(f"{name}: max-abs {float(err.max()):.3e} mean-abs {float(err.mean()):.3e}")


def test_config1_against_token_recurrence():
    """BASELINE config 1 (T=512, 4 heads, d=64, chunk 64, zero state) with
    bf16-rounded q/k/v: kernel vs the naive recurrence of the same inputs."""
    g = gen(1)
    T, H, d = 512, 4, 64
    q, k, v, gg, beta = _inputs(g, T, H, H, d, d, torch.bfloat16)
    s0 = torch.zeros(H, d, d)
    o_ref, s_ref, _ = ref.naive_recurrence(q.float(), k.float(), v.float(), gg, beta, d ** -0.5, s0)
    storage = torch.zeros(2, 1, H, d, d, device=DEV)
    o, v_new = _run(q.to(DEV), k.to(DEV), v.to(DEV), gg.to(DEV), beta.to(DEV), storage,
                    torch.tensor([-1], device=DEV), torch.full((8,), -1, device=DEV), torch.tensor([0, T], device=DEV),
                    finals=torch.tensor([1], device=DEV))
    _report("cfg1 out", o[0], o_ref)
    _report("cfg1 state", storage[1, 0], s_ref)
    assert_bf16_close(o[0], o_ref)
    assert_state_close(storage[1, 0], s_ref)
    assert v_new.shape == o.shape


@pytest.mark.parametrize("dims", [(128, 128), (64, 64), (32, 32), (128, 64)])
def test_varlen_gqa_pool_semantics(dims):
    g = gen(2)
    dk, dv = dims
    H, HV = 2, 4
    lengths = [1, 17, 64, 65, 130, 300]
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    T = cu[-1]
    q, k, v, gg, beta = _inputs(g, T, H, HV, dk, dv, torch.bfloat16, g_scale=0.3)
    N = len(lengths)
    nchunks = [(n + 63) // 64 for n in lengths]
    NT = sum(nchunks)
    slots = 2 * N + NT + 2
    storage = torch.zeros(slots, 2, HV, dk, dv)
    storage[:N, 1] = torch.randn(N, HV, dk, dv, generator=g) * 0.1
    reads = torch.tensor([0, -1, 2, 3, -1, 5])
    writes = torch.arange(2 * N, 2 * N + NT)
    writes[1] = -1  # skip one checkpoint
    finals = torch.arange(N, 2 * N)
    expected = storage.clone()
    o_ref, vn_ref = ref.chunk_gated_delta_rule_to_cache(q[None].float(), k[None].float(), v[None].float(),
                                                        gg[None], beta[None], expected, reads, writes, cu, layer=1,
                                                        final_write_slots=finals)
    dstore = storage.to(DEV)
    o, vn = _run(q.to(DEV), k.to(DEV), v.to(DEV), gg.to(DEV), beta.to(DEV), dstore, reads.to(DEV), writes.to(DEV),
                 torch.tensor(cu, device=DEV), finals=finals.to(DEV), layer=1)
    _report("varlen out", o[0], o_ref[0])
    _report("varlen states", dstore, expected)
    assert_bf16_close(o[0], o_ref[0])
    assert_bf16_close(vn[0], vn_ref[0], rel=2e-2, atol=2e-2)
    assert_state_close(dstore, expected)
    # untouched: layer 0 everywhere, the skipped checkpoint slot, and the spare slots
    torch.testing.assert_close(dstore[:, 0].cpu(), storage[:, 0], rtol=0, atol=0)
    torch.testing.assert_close(dstore[2 * N + 1].cpu(), storage[2 * N + 1], rtol=0, atol=0)
    torch.testing.assert_close(dstore[-2:].cpu(), storage[-2:], rtol=0, atol=0)


@pytest.mark.parametrize("lengths", [[31], [17, 31, 33, 65], [1] * 16])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_dispatch_style_recurrence_checkpoints_and_graph(lengths, dtype):
    """tests/kernel/test_gdn_prefill_dispatch.py:143-197 at chunk 64: outputs
    and every chunk-end checkpoint vs the token recurrence, final states to
    their own slots, then a captured graph replays bit-identically."""
    from logssms_amd.kernel.linear_attention import ChunkStateIO, chunk_gated_delta_rule_to_cache
    from oracle import metadata as md
    g = gen(41)
    n, heads = len(lengths), 6
    idx = md.from_lengths(lengths, 64)
    tokens = sum(lengths)
    q = F.normalize(torch.randn(1, tokens, 2, 128, generator=g), dim=-1).to(dtype)
    k = F.normalize(torch.randn(1, tokens, 2, 128, generator=g), dim=-1).to(dtype)
    v = (torch.randn(1, tokens, heads, 128, generator=g) * 0.1).to(dtype)
    gg = -torch.rand(1, tokens, heads, generator=g) * 0.1
    beta = torch.rand(1, tokens, heads, generator=g)
    nt = len(idx["chunk_indices"])
    storage = torch.zeros(2 * n + nt, 1, heads, 128, 128).to(dtype)
    storage[:n].normal_(std=0.01, generator=g)
    expected, checkpoints = [], []
    start = 0
    for req, length in enumerate(lengths):
        state = storage[req, 0].float()
        o, _, cks = ref.naive_recurrence(q[0, start:start + length].float(), k[0, start:start + length].float(),
                                         v[0, start:start + length].float(), gg[0, start:start + length],
                                         beta[0, start:start + length], 128 ** -0.5, state, checkpoint_every=64)
        expected.append(o)
        checkpoints.extend(cks)
        start += length
    expected = torch.cat(expected)[None]
    checkpoints = torch.stack(checkpoints)
    dstore = storage.to(DEV)
    reads = torch.arange(n, dtype=torch.int32, device=DEV)
    writes = torch.arange(2 * n, 2 * n + nt, dtype=torch.int32, device=DEV)
    io = ChunkStateIO(dstore, reads, writes, final_write_slots=reads + n)
    cu = torch.tensor(idx["cu_seqlens"], device=DEV)
    args = (q.to(DEV), k.to(DEV), v.to(DEV), gg.to(DEV), beta.to(DEV), io, cu)
    out = chunk_gated_delta_rule_to_cache(*args)[0]
    assert_bf16_close(out, expected, rel=3e-2, atol=2e-3)
    assert_bf16_close(dstore[2 * n:, 0], checkpoints, rel=3e-2, atol=3e-3)
    assert_bf16_close(dstore[n:2 * n, 0], checkpoints[idx["endings"]], rel=3e-2, atol=3e-3)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = chunk_gated_delta_rule_to_cache(*args)[0]
    dstore[n:].fill_(float("nan"))
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(captured, out, rtol=0, atol=0)
        assert_bf16_close(dstore[2 * n:, 0], checkpoints, rel=3e-2, atol=3e-3)


def test_bf16_pool_and_chunk_aligned_resume():
    """Split-at-64 resume == full run (tests/layers/test_linear_attention_backend.py:334-428)."""
    g = gen(17)
    T, H, HV, d = 200, 2, 4, 128
    q, k, v, gg, beta = _inputs(g, T, H, HV, d, d, torch.bfloat16)
    full = torch.zeros(4, 1, HV, d, d, device=DEV)
    o_full, _ = _run(q.to(DEV), k.to(DEV), v.to(DEV), gg.to(DEV), beta.to(DEV), full, torch.tensor([-1], device=DEV),
                     torch.tensor([-1, -1, -1, 1], device=DEV), torch.tensor([0, T], device=DEV))
    part = torch.zeros(4, 1, HV, d, d, device=DEV)
    o1, _ = _run(q[:128].to(DEV), k[:128].to(DEV), v[:128].to(DEV), gg[:128].to(DEV), beta[:128].to(DEV), part,
                 torch.tensor([-1], device=DEV), torch.tensor([-1, 2], device=DEV), torch.tensor([0, 128], device=DEV))
    o2, _ = _run(q[128:].to(DEV), k[128:].to(DEV), v[128:].to(DEV), gg[128:].to(DEV), beta[128:].to(DEV), part,
                 torch.tensor([2], device=DEV), torch.tensor([-1, 1], device=DEV), torch.tensor([0, T - 128], device=DEV))
    assert_bf16_close(torch.cat([o1[0], o2[0]]), o_full[0], rel=1e-2, atol=1e-2)
    assert_state_close(part[1], full[1])
    # bf16 pool: same run, state stored in bf16
    bpool = torch.zeros(4, 1, HV, d, d, device=DEV, dtype=torch.bfloat16)
    _run(q.to(DEV), k.to(DEV), v.to(DEV), gg.to(DEV), beta.to(DEV), bpool, torch.tensor([-1], device=DEV),
         torch.tensor([-1, -1, -1, 1], device=DEV), torch.tensor([0, T], device=DEV))
    assert_bf16_close(bpool[1], full[1], rel=2e-2, atol=2e-3)


def test_config1_against_committed_fixture():
    """The kernel against ``tests/golden/cfg1_bf16.npz`` (float64 recurrence of
    the same bf16 inputs), without running the oracle."""
    from tests.golden.make_golden import D, EVERY, H, T, cfg1_inputs
    from tests.test_golden import load_fixture
    o_rows, state = load_fixture()
    q, k, v, gg, beta = cfg1_inputs()
    storage = torch.zeros(2, 1, H, D, D, device=DEV)
    o, _ = _run(q.to(DEV), k.to(DEV), v.to(DEV), gg.to(DEV), beta.to(DEV), storage, torch.tensor([-1], device=DEV),
                torch.tensor([-1] * 7 + [1], device=DEV), torch.tensor([0, T], device=DEV))
    assert_bf16_close(o[0, ::EVERY], o_rows)
    assert_state_close(storage[1, 0], state)


@pytest.mark.parametrize("scale", [1e3, 1e5])
def test_large_magnitude_values(scale):
    """Where the f16 MFMA operands stop representing the values: v scaled so
    that v, v' and the state stay below f16's 65504 (scale 1e3: the kernel
    matches the recurrence to the bf16 output bar, relative to the values'
    size), and scaled past it (1e5: the operands become +-inf and the
    overflow shows in the outputs and the final state instead of being
    saturated silently)."""
    g = gen(31)
    T, H, d = 128, 2, 128
    q, k, v, gg, beta = _inputs(g, T, H, H, d, d, torch.bfloat16)
    v = (v.float() * scale).to(torch.bfloat16)
    s0 = torch.zeros(H, d, d)
    storage = torch.zeros(2, 1, H, d, d, device=DEV)
    o, _ = _run(q.to(DEV), k.to(DEV), v.to(DEV), gg.to(DEV), beta.to(DEV), storage, torch.tensor([-1], device=DEV),
                torch.full((2,), -1, device=DEV), torch.tensor([0, T], device=DEV), finals=torch.tensor([1], device=DEV))
    torch.cuda.synchronize()
    print(f"scale {scale:g}: |v| max {float(v.float().abs().max()):.3e}", flush=True)
    if scale < 65504 / 8:
        o_ref, s_ref, _ = ref.naive_recurrence(q.float(), k.float(), v.float(), gg, beta, d ** -0.5, s0)
        _report("out / scale", o[0].float() / scale, o_ref / scale)
        _report("state / scale", storage[1, 0] / scale, s_ref / scale)
        assert float(v.float().abs().max()) > 1e3 and float(s_ref.abs().max()) < 65504
        assert_bf16_close(o[0].float() / scale, o_ref / scale)
        assert_state_close(storage[1, 0].cpu() / scale, s_ref / scale)
    else:
        assert float(v.float().abs().max()) > 65504
        assert not torch.isfinite(o).all(), "values beyond f16's range should overflow visibly"
        assert not torch.isfinite(storage[1, 0]).all()
