"""Pins the CPU oracle (``oracle/gdn.py``) before anything is checked against it.

Each check is chosen so that a plausible slip in the oracle (dropped decay
term, wrong sign, transposed operand, off-by-one window) fails at least one:
closed forms, an independent algorithm (token recurrence vs WY chunk form),
library routines (``F.conv1d``, ``math.log1p``) and the reference tests'
known answers.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn


def _normal(*shape, gen, dtype=torch.float64):
    return torch.randn(*shape, generator=gen, dtype=dtype)


def _inputs(T, H, HV, dk, dv, gen, dtype=torch.float64, g_scale=0.1):
    q = F.normalize(_normal(T, H, dk, gen=gen, dtype=dtype), dim=-1)
    k = F.normalize(_normal(T, H, dk, gen=gen, dtype=dtype), dim=-1)
    v = _normal(T, HV, dv, gen=gen, dtype=dtype)
    g = -torch.rand(T, HV, generator=gen, dtype=dtype) * g_scale
    beta = torch.sigmoid(_normal(T, HV, gen=gen, dtype=dtype))
    return q, k, v, g, beta


# ---------------------------------------------------------------- recurrence

def test_single_token_closed_form():
    gen = torch.Generator().manual_seed(1)
    q, k, v, g, beta = _inputs(1, 2, 2, 8, 5, gen)
    scale = 8 ** -0.5
    o, s, _ = gdn.naive_recurrence(q, k, v, g, beta, scale, torch.zeros(2, 8, 5, dtype=torch.float64))
    for h in range(2):
        want_s = beta[0, h] * k[0, h][:, None] * v[0, h][None, :]
        torch.testing.assert_close(s[h], want_s, rtol=0, atol=1e-14)
        want_o = scale * beta[0, h] * (k[0, h] @ q[0, h]) * v[0, h]
        torch.testing.assert_close(o[0, h], want_o, rtol=0, atol=1e-14)


def test_zero_beta_is_pure_decay():
    gen = torch.Generator().manual_seed(2)
    q, k, v, g, beta = _inputs(13, 2, 4, 8, 6, gen)
    s0 = _normal(4, 8, 6, gen=gen)
    o, s, _ = gdn.naive_recurrence(q, k, v, g, torch.zeros_like(beta), 0.5, s0)
    torch.testing.assert_close(s, s0 * torch.exp(g.sum(0))[:, None, None], rtol=1e-12, atol=1e-14)
    qe = q.repeat_interleave(2, 1)
    cum = torch.cumsum(g, 0)
    want = 0.5 * torch.exp(cum)[:, :, None] * torch.einsum("hkv,thk->thv", s0, qe)
    torch.testing.assert_close(o, want, rtol=1e-12, atol=1e-14)


def test_orthonormal_keys_delta_overwrite():
    gen = torch.Generator().manual_seed(3)
    d = 8
    basis, _ = torch.linalg.qr(_normal(d, d, gen=gen))
    k = basis.T[:, None, :]  # 8 orthonormal keys, one head
    v = _normal(d, 1, 5, gen=gen)
    s0 = _normal(1, d, 5, gen=gen)
    _, s, _ = gdn.naive_recurrence(k, k, v, torch.zeros(d, 1, dtype=torch.float64),
                                   torch.ones(d, 1, dtype=torch.float64), 1.0, s0)
    # beta = 1, g = 0: every key's row is overwritten with its value.
    torch.testing.assert_close(s[0].T @ basis, v[:, 0].T, rtol=0, atol=1e-12)


def test_single_pass_decode_identity():
    gen = torch.Generator().manual_seed(4)
    q, k, v, g, beta = _inputs(1, 1, 1, 16, 9, gen)
    s0 = _normal(1, 16, 9, gen=gen)
    scale = 0.25
    o, _, _ = gdn.naive_recurrence(q, k, v, g, beta, scale, s0)
    want = gdn.single_pass_decode_output(s0[0], q[0, 0], k[0, 0], v[0, 0], float(g[0, 0]),
                                         float(beta[0, 0]), scale)
    torch.testing.assert_close(o[0, 0], want, rtol=1e-12, atol=1e-14)


# ---------------------------------------------------------------- chunk form

@pytest.mark.parametrize("T", [1, 17, 64, 65, 150])
@pytest.mark.parametrize("chunk", [1, 16, 32, 64])
def test_chunk_matches_recurrence(T, chunk):
    gen = torch.Generator().manual_seed(10 + T + chunk)
    q, k, v, g, beta = _inputs(T, 2, 4, 16, 12, gen, g_scale=0.5)
    s0 = _normal(4, 16, 12, gen=gen) * 0.3
    scale = 16 ** -0.5
    o_ref, s_ref, cks = gdn.naive_recurrence(q, k, v, g, beta, scale, s0, checkpoint_every=chunk)
    exact = 1.0 / math.log(2.0)
    o, v_new, ends, s = gdn.chunk_gdn(q, k, v, g, beta, scale, s0, chunk, rcp_ln2=exact)
    torch.testing.assert_close(o, o_ref, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(s, s_ref, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(ends, torch.stack(cks), rtol=1e-10, atol=1e-10)
    assert v_new.shape == v.shape
    # The reference's truncated 1/ln2 (gated_delta.py:12) moves results by
    # at most |G| * 1.3e-8 relative.
    o2, _, _, s2 = gdn.chunk_gdn(q, k, v, g, beta, scale, s0, chunk)
    torch.testing.assert_close(o2, o_ref, rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(s2, s_ref, rtol=1e-6, atol=1e-7)


def test_config1_chunk_vs_recurrence_fp32():
    """B=1, T=512, 4 heads, d=64, fp32, chunk 64."""
    gen = torch.Generator().manual_seed(1)
    T, H, d = 512, 4, 64
    q = F.normalize(torch.randn(T, H, d, generator=gen), dim=-1)
    k = F.normalize(torch.randn(T, H, d, generator=gen), dim=-1)
    v = torch.randn(T, H, d, generator=gen)
    g = -torch.rand(T, H, generator=gen) * 0.1
    beta = torch.sigmoid(torch.randn(T, H, generator=gen))
    s0 = torch.zeros(H, d, d)
    o_ref, s_ref, _ = gdn.naive_recurrence(q, k, v, g, beta, d ** -0.5, s0)
    o, _, _, s = gdn.chunk_gdn(q, k, v, g, beta, d ** -0.5, s0, 64)
    assert (s - s_ref).abs().max() <= 1e-3
    assert (o - o_ref).abs().max() <= 1e-3


def test_chunk_to_cache_slot_semantics():
    gen = torch.Generator().manual_seed(5)
    lengths = [70, 5, 128]
    T = sum(lengths)
    q, k, v, g, beta = _inputs(T, 1, 2, 8, 8, gen)
    storage = torch.zeros(12, 2, 2, 8, 8, dtype=torch.float64)
    storage[3, 1] = _normal(2, 8, 8, gen=gen)
    cu = [0, 70, 75, 203]
    read = [3, -1, 3]
    nt = 2 + 1 + 2
    writes = [-1, 6, 7, 8, -1]
    sentinel = storage.clone()
    o, _ = gdn.chunk_gated_delta_rule_to_cache(q[None], k[None], v[None], g[None], beta[None],
                                               storage, read, writes, cu, layer=1,
                                               final_write_slots=[9, -1, 10],
                                               dtype=torch.float64)
    s0 = sentinel[3, 1]
    _, s_a, ck_a = gdn.naive_recurrence(q[:70], k[:70], v[:70], g[:70], beta[:70], 8 ** -0.5, s0,
                                        checkpoint_every=64)
    _, s_b, _ = gdn.naive_recurrence(q[70:75], k[70:75], v[70:75], g[70:75], beta[70:75],
                                     8 ** -0.5, torch.zeros_like(s0))
    _, s_c, ck_c = gdn.naive_recurrence(q[75:], k[75:], v[75:], g[75:], beta[75:], 8 ** -0.5, s0,
                                        checkpoint_every=64)
    torch.testing.assert_close(storage[6, 1], ck_a[1], rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(storage[7, 1], s_b, rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(storage[8, 1], ck_c[0], rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(storage[9, 1], s_a, rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(storage[10, 1], s_c, rtol=1e-6, atol=1e-7)
    untouched = [i for i in range(12) if i not in (6, 7, 8, 9, 10)]
    torch.testing.assert_close(storage[untouched], sentinel[untouched], rtol=0, atol=0)
    assert nt == len(writes)


# ---------------------------------------------------------------- fused recurrent

def test_fused_recurrent_equals_prepare_plus_recurrence():
    gen = torch.Generator().manual_seed(6)
    B, T, H, HV, dk, dv = 2, 5, 2, 4, 16, 8
    q = _normal(B, T, H, dk, gen=gen)
    k = _normal(B, T, H, dk, gen=gen)
    v = _normal(B, T, HV, dv, gen=gen)
    gate = _normal(B, T, HV, gen=gen)
    beta = _normal(B, T, HV, gen=gen)
    A_log = _normal(HV, gen=gen) * 0.3
    dt_bias = _normal(HV, gen=gen) * 0.3
    init = _normal(B, HV, dk, dv, gen=gen)
    o, states = gdn.fused_recurrent(q, k, v, gate, beta, A_log, dt_bias, init, dtype=torch.float64)
    for b in range(B):
        g = -torch.exp(A_log) * F.softplus(gate[b] + dt_bias)
        o_ref, s_ref, cks = gdn.naive_recurrence(gdn.l2norm(q[b]), gdn.l2norm(k[b]), v[b], g,
                                                 torch.sigmoid(beta[b]), dk ** -0.5, init[b],
                                                 checkpoint_every=1)
        torch.testing.assert_close(o[b], o_ref, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(states[b], torch.stack(cks), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- prepare_gdn

def test_prepare_gdn_closed_form_and_softplus_edges():
    edges = [-80.0, -20.0, 0.0, 19.999, 20.0, 20.001, 80.0]
    gate = torch.tensor(edges, dtype=torch.float32)[None, :, None].expand(1, 7, 2).contiguous()
    q = torch.randn(1, 7, 1, 32)
    q[:, 0] = 0
    k = torch.randn(1, 7, 1, 32)
    v = torch.randn(1, 7, 2, 32)
    qh, kh, vv, g, b = gdn.prepare_gdn(q, k, v, gate, gate.clone(), torch.zeros(2), torch.zeros(2))
    for i, x in enumerate(edges):
        want = x if x > 20 else math.log1p(math.exp(min(x, 20.0)))
        assert abs(float(g[0, i, 0]) + want) <= 1e-6 * max(1.0, abs(want))
        assert abs(float(b[0, i, 0]) - 1.0 / (1.0 + math.exp(-x))) <= 1e-7
    torch.testing.assert_close(vv, v, rtol=0, atol=0)
    assert float(qh[0, 0].abs().max()) == 0.0
    norms = kh.float().norm(dim=-1)
    torch.testing.assert_close(norms, torch.ones_like(norms), rtol=0, atol=1e-4)


def test_softplus_variants_agree_off_the_threshold():
    x = torch.linspace(-30, 30, 601, dtype=torch.float64)
    ref = F.softplus(x, threshold=1000)
    torch.testing.assert_close(gdn.softplus_prefill(x), ref, rtol=1e-9, atol=1e-12)
    far = x[(x - 20).abs() > 1e-3]
    torch.testing.assert_close(gdn.softplus_decode(far), F.softplus(far, threshold=1000),
                               rtol=1e-8, atol=1e-12)


# ---------------------------------------------------------------- conv

def _conv_reference(x, weight, history, bias=None):
    """tests/layers/test_linear_attention_backend.py:191-197 closed form."""
    dt = torch.float64 if x.dtype == torch.float64 else torch.float32
    src = torch.cat([history.to(x.dtype), x.T[None]], -1).to(dt)
    out = F.conv1d(src, weight.to(dt), None if bias is None else bias.to(dt), groups=x.shape[1])
    return F.silu(out)[0].T


def test_packed_conv_matches_conv1d_and_windows():
    gen = torch.Generator().manual_seed(31)
    lengths = [1, 2, 17, 79]
    C, W = 65, 4
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    x = torch.randn(cu[-1], C, generator=gen, dtype=torch.float64)
    weight = torch.randn(C, 1, W, generator=gen, dtype=torch.float64) * 0.1
    history = torch.randn(len(lengths), C, W - 1, generator=gen, dtype=torch.float64)
    bias = torch.randn(C, generator=gen, dtype=torch.float64) * 0.1
    y, windows = gdn.packed_causal_conv1d(x, weight, history, cu, bias)
    for r in range(len(lengths)):
        b, e = cu[r], cu[r + 1]
        want = _conv_reference(x[b:e], weight, history[r:r + 1], bias)
        torch.testing.assert_close(y[b:e], want.to(y.dtype), rtol=1e-12, atol=1e-12)
        src = torch.cat([history[r], x[b:e].T], -1)
        for t in range(e - b):
            torch.testing.assert_close(windows[b + t], src[:, t + 1:t + W], rtol=0, atol=0)


def test_conv_decode_matches_conv1d_and_shift():
    gen = torch.Generator().manual_seed(93)
    C, W = 192, 4
    x = torch.randn(2, C, generator=gen).to(torch.bfloat16)
    weight = (torch.randn(C, 1, W, generator=gen) * 0.1).to(torch.bfloat16)
    state = torch.randn(3, 2, C, W - 1, generator=gen).to(torch.bfloat16)
    before = state.clone()
    y = gdn.conv_decode(x, weight, state, 1, [0, 2], [1, 2])
    for row, (r, w) in enumerate([(0, 1), (2, 2)]):
        want = _conv_reference(x[row:row + 1], weight, before[r:r + 1, 1])[0]
        torch.testing.assert_close(y[row].float(), want.float(), rtol=2e-2, atol=2e-2)
        torch.testing.assert_close(state[w, 1], torch.cat([before[r, 1, :, 1:], x[row, :, None]], -1),
                                   rtol=0, atol=0)
    torch.testing.assert_close(state[0], before[0], rtol=0, atol=0)
    torch.testing.assert_close(state[:, 0], before[:, 0], rtol=0, atol=0)


def test_verify_conv_matches_conv1d_and_unfold():
    gen = torch.Generator().manual_seed(7)
    B, T, C, W = 2, 5, 24, 4
    x = torch.randn(B, T, C, generator=gen, dtype=torch.float64)
    weight = torch.randn(C, 1, W, generator=gen, dtype=torch.float64) * 0.2
    hist = torch.randn(B, C, W - 1, generator=gen, dtype=torch.float64)
    y, windows = gdn.verify_conv(x, weight, hist)
    src = torch.cat([hist, x.transpose(1, 2)], -1)
    want = F.silu(F.conv1d(src, weight, groups=C)).transpose(1, 2)
    torch.testing.assert_close(y, want, rtol=1e-12, atol=1e-12)
    unf = src.unfold(-1, W - 1, 1)[:, :, 1:].permute(0, 2, 1, 3)
    torch.testing.assert_close(windows, unf, rtol=0, atol=0)


# ---------------------------------------------------------------- output norm

def test_rms_norm_gated_matches_library_routines():
    g = torch.Generator().manual_seed(40)
    x = _normal(5, 3, 64, gen=g)
    z = _normal(5, 3, 64 + 8, gen=g)[..., :64]  # strided gate view
    w = _normal(64, gen=g)
    got = gdn.rms_norm_gated(x, z, w, 1e-6)
    want = F.rms_norm(x, (64,), eps=1e-6) * w * F.silu(z)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-6)
    # the reference test's closed form (one group, norm before the gate; tests/kernel/test_grouped_norm_gated.py)
    variance = x.square().mean(-1, keepdim=True)
    torch.testing.assert_close(got, x * torch.rsqrt(variance + 1e-6) * w * F.silu(z), rtol=1e-5, atol=1e-6)


def test_rms_norm_gated_closed_forms():
    g = torch.Generator().manual_seed(41)
    w = _normal(16, gen=g)
    z = _normal(4, 16, gen=g)
    # a zero gate zeroes the row (silu(0) = 0, not sigmoid(0) = 1/2)
    x = _normal(4, 16, gen=g)
    assert torch.equal(gdn.rms_norm_gated(x, torch.zeros_like(z), w, 1e-5), torch.zeros_like(x))
    # a constant row c: c / sqrt(c^2 + eps) * w * silu(z) (eps inside the root)
    for c in (1e-3, -0.5, 2.0):
        xc = torch.full((4, 16), c, dtype=torch.float64)
        want = c / math.sqrt(c * c + 1e-5) * w * z * torch.sigmoid(z)
        torch.testing.assert_close(gdn.rms_norm_gated(xc, z, w, 1e-5), want, rtol=1e-5, atol=1e-7)
    # positive row scaling cancels (eps = 0); rows stay paired with their own gate rows
    scale = torch.tensor([0.5, 3.0, 7.0, 0.1], dtype=torch.float64)[:, None]
    torch.testing.assert_close(gdn.rms_norm_gated(x * scale, z, w, 0.0), gdn.rms_norm_gated(x, z, w, 0.0),
                               rtol=1e-5, atol=1e-6)
    swapped = gdn.rms_norm_gated(x, z.flip(0), w, 1e-5)
    assert not torch.allclose(swapped, gdn.rms_norm_gated(x, z, w, 1e-5))


def test_packed_conv_window_rows_select_the_same_windows():
    gen = torch.Generator().manual_seed(32)
    cu = [0, 3, 70, 72]
    C, W = 24, 4
    x = torch.randn(cu[-1], C, generator=gen).to(torch.bfloat16)
    weight = (torch.randn(C, 1, W, generator=gen) * 0.2).to(torch.bfloat16)
    history = torch.randn(3, C, W - 1, generator=gen).to(torch.bfloat16)
    y, windows = gdn.packed_causal_conv1d(x, weight, history, cu)
    rows = [71, 0, 2, 63, 3]
    y2, some = gdn.packed_causal_conv1d(x, weight, history, cu, window_rows=rows)
    assert torch.equal(y, y2)
    assert torch.equal(some, windows[rows])


# ---------------------------------------------------------------- slot I/O and compositions

def test_store_state_matches_index_copy():
    """kernel/store.py:69-83: ``pool[idx[i]] = states[i]`` for idx >= 0,
    pinned by ``Tensor.index_copy_`` (a library routine)."""
    gen = torch.Generator().manual_seed(50)
    pool = torch.randn(7, 2, 3, 5, generator=gen)
    states = torch.randn(4, 2, 3, 5, generator=gen)
    for dtype in (torch.int64, torch.int32):
        idx = torch.tensor([5, -1, 0, 3], dtype=dtype)
        got = pool.clone()
        gdn.store_state(got, idx, states)
        keep = idx >= 0
        want = pool.clone().view(7, -1).index_copy_(0, idx[keep].long(), states.view(4, -1)[keep]).view(pool.shape)
        assert torch.equal(got, want)


def test_fused_recurrent_to_slots_equals_gather_recurrence_scatter():
    """``fused_recurrent.py:396-458`` slotted mode: gather the read slots
    (``index_select``), one token recurrence per sequence (pinned by closed
    forms above), normalisation with ``sqrt`` and division, softplus from
    ``math.log1p``, then scatter to the write slots (``index_copy_``); an
    in-place slot, a shared read slot and untouched slots included."""
    gen = torch.Generator().manual_seed(51)
    B, H, HV, dk, dv, layer = 3, 2, 4, 8, 6, 1
    q = _normal(B, 1, H, dk, gen=gen)
    k = _normal(B, 1, H, dk, gen=gen)
    v = _normal(B, 1, HV, dv, gen=gen)
    gate = _normal(B, 1, HV, gen=gen)
    beta = _normal(B, 1, HV, gen=gen)
    A_log = _normal(HV, gen=gen) * 0.3
    dt_bias = _normal(HV, gen=gen) * 0.3
    pool = _normal(6, 2, HV, dk, dv, gen=gen)
    reads, writes = torch.tensor([1, 3, 3]), torch.tensor([1, 4, 0])
    before = pool.clone()
    o = gdn.fused_recurrent_to_slots(q, k, v, gate, beta, A_log, dt_bias, pool, reads, writes, layer,
                                     dtype=torch.float64)
    init = before.index_select(0, reads)[:, layer]
    expected = before.clone()
    for b in range(B):
        qn = q[b, 0] / torch.sqrt((q[b, 0] ** 2).sum(-1, keepdim=True) + 1e-6)
        kn = k[b, 0] / torch.sqrt((k[b, 0] ** 2).sum(-1, keepdim=True) + 1e-6)
        sp = torch.tensor([math.log1p(math.exp(float(x))) for x in gate[b, 0] + dt_bias], dtype=torch.float64)
        g = -torch.exp(A_log) * sp
        o_ref, s_ref, _ = gdn.naive_recurrence(qn[None], kn[None], v[b], g[None],
                                               (1.0 / (1.0 + torch.exp(-beta[b, 0])))[None], dk ** -0.5, init[b])
        torch.testing.assert_close(o[b, 0], o_ref[0], rtol=1e-12, atol=1e-12)
        expected[:, layer].index_copy_(0, writes[b:b + 1], s_ref[None])
    torch.testing.assert_close(pool, expected, rtol=1e-12, atol=1e-12)
    assert torch.equal(pool[2], before[2]) and torch.equal(pool[5], before[5])
    assert torch.equal(pool[:, 0], before[:, 0])


@pytest.mark.parametrize("decode", [False, True])
def test_partitioned_input_scales_closed_form(decode):
    """``_scale_inputs`` against the closed form of the reference's
    ``tests/layers/test_conv_decode.py:185-222``: each channel range scaled
    (and rounded to the input dtype) once, then ``silu(conv1d(...))`` with
    bias; snapshots are the scaled raw windows."""
    gen = torch.Generator().manual_seed(87)
    scales, widths = (0.7, 0.8, 0.9), (256, 128, 128)
    C = sum(widths)
    bounds = (256, 384)
    lengths = [1, 1] if decode else [7, 16]
    raw = (torch.randn(sum(lengths), C + 32, generator=gen).to(torch.bfloat16))[:, :C]
    scaled = torch.cat([part * s for part, s in zip(raw.split(widths, -1), scales)], -1)
    history = torch.randn(2, C, 3, generator=gen).to(torch.bfloat16)
    weight = (torch.randn(C, 1, 4, generator=gen) * 0.2).to(torch.bfloat16)
    bias = (torch.randn(C, generator=gen) * 0.1).to(torch.bfloat16)
    expected, snapshots, begin = [], [], 0
    for i, length in enumerate(lengths):
        source = torch.cat((history[i:i + 1], scaled[begin:begin + length].T[None]), -1)
        expected.append(F.silu(F.conv1d(source.float(), weight.float(), bias.float(), groups=C))[0].T)
        snapshots.append(source[0, :, -3:])
        begin += length
    if decode:
        storage = torch.zeros(4, 1, C, 3, dtype=torch.bfloat16)
        storage[:2, 0] = history
        got = gdn.conv_decode(raw, weight, storage, 0, [0, 1], [2, 3], bias=bias, round_conv=True,
                              input_boundaries=bounds, input_scales=scales)
        windows = storage[2:, 0]
    else:
        got, windows = gdn.packed_causal_conv1d(raw, weight, history, [0, 7, 23], bias, input_boundaries=bounds,
                                                input_scales=scales, window_rows=[6, 22])
    torch.testing.assert_close(got.float(), torch.cat(expected), rtol=2e-2, atol=2e-2)
    assert torch.equal(windows, torch.stack(snapshots))
    # unscaled inputs would miss the closed form: the scales are applied
    plain = gdn.packed_causal_conv1d(raw, weight, history, [0, 7, 23] if not decode else [0, 1, 2], bias)[0]
    assert not torch.allclose(plain.float(), torch.cat(expected), rtol=2e-2, atol=2e-2)


def test_conv_decode_round_conv_rounds_the_pre_activation():
    """``conv_decode(round_conv=True)`` rounds the conv sum to the io dtype
    before SiLU (``conv_decode.py:276-278``): its bf16 outputs equal
    ``silu(round_bf16(conv1d))`` from a float64 ``F.conv1d``, except where the
    fp32 sum and the float64 sum straddle a bf16 rounding boundary, and they
    differ from the unrounded chain in many elements."""
    gen = torch.Generator().manual_seed(94)
    B, C = 64, 512
    x = torch.randn(B, C, generator=gen).to(torch.bfloat16)
    weight = (torch.randn(C, 1, 4, generator=gen) * 0.5).to(torch.bfloat16)
    state = torch.randn(B, 1, C, 3, generator=gen).to(torch.bfloat16)
    src = torch.cat([state[:, 0], x[:, :, None]], -1).double()  # [B, C, 4]
    pre = F.conv1d(src.reshape(1, B * C, 4), weight.double().repeat(B, 1, 1), groups=B * C).reshape(B, C)
    rounded = F.silu(pre.to(torch.bfloat16).double()).to(torch.bfloat16)
    unrounded = F.silu(pre).to(torch.bfloat16)
    got = gdn.conv_decode(x, weight, state.clone(), 0, list(range(B)), list(range(B)), round_conv=True)
    assert (got != rounded).float().mean() < 1e-3
    assert (got != unrounded).float().mean() > 0.05
    plain = gdn.conv_decode(x, weight, state.clone(), 0, list(range(B)), list(range(B)))
    assert (plain != unrounded).float().mean() < 1e-3


def _composition_inputs(gen, T, H, HV, dk, dv, C):
    return dict(
        mixed=torch.randn(T, C, generator=gen),
        gate=torch.randn(T, HV, generator=gen),
        beta=torch.randn(T, HV, generator=gen),
        weight=torch.randn(C, 1, 4, generator=gen) * 0.3,
        A_log=-torch.rand(HV, generator=gen),
        dt_bias=torch.randn(HV, generator=gen) * 0.3,
    )


def test_forward_prefill_equals_successive_decode_steps():
    """In fp32 io the prefill composition (conv with history, windows,
    split, prepare, chunked rule with pool I/O, ``gdn.py:74-149``) and T
    decode steps (``gdn.py:222-265``, each reading the slot the previous step
    wrote) are two independent paths to the same outputs, checkpoint state,
    final state and conv window."""
    gen = torch.Generator().manual_seed(60)
    H, HV, dk, dv, T, layer = 2, 4, 16, 8, 70, 1
    C = 2 * H * dk + HV * dv
    w = _composition_inputs(gen, T, H, HV, dk, dv, C)
    slots = T + 4
    conv0 = torch.randn(slots, 2, C, 3, generator=gen)
    state0 = torch.randn(slots, 2, HV, dk, dv, generator=gen) * 0.1
    conv_p, state_p = conv0.clone(), state0.clone()
    chunk_writes = torch.tensor([slots - 2, slots - 1])  # checkpoint after token 64, final state
    token_slots = torch.full((T,), -1)
    token_slots[63], token_slots[T - 1] = slots - 2, slots - 1
    o_p = gdn.forward_prefill(w["mixed"], w["gate"], w["beta"], w["weight"], w["A_log"], w["dt_bias"], conv_p,
                              state_p, layer, [0, T], [0], chunk_writes, token_slots, H, dk, HV, dv)
    conv_d, state_d = conv0.clone(), state0.clone()
    outs = []
    for t in range(T):  # slot 0 -> 1 -> ... -> T
        outs.append(gdn.forward_decode(w["mixed"][t:t + 1], w["gate"][t:t + 1], w["beta"][t:t + 1], w["weight"],
                                       w["A_log"], w["dt_bias"], conv_d, state_d, layer, [t], [t + 1], H, dk, HV,
                                       dv))
    torch.testing.assert_close(o_p, torch.cat(outs), rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(state_p[slots - 2, layer], state_d[64, layer], rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(state_p[slots - 1, layer], state_d[T, layer], rtol=1e-4, atol=1e-5)
    assert torch.equal(conv_p[slots - 2, layer], conv_d[64, layer])
    assert torch.equal(conv_p[slots - 1, layer], conv_d[T, layer])
    assert torch.equal(state_p[:slots - 2], state0[:slots - 2]) and torch.equal(conv_p[:slots - 2], conv0[:slots - 2])


def test_forward_verify_equals_decode_steps_with_per_step_slots():
    """One verify length group (``gdn.py:151-220``): B sequences of T drafts
    from their baseline slots, step t's window and state to
    ``write_slots[b, t]``; equal to T decode steps per sequence whose step t
    reads step t-1's slot and writes ``write_slots[b, t]``."""
    gen = torch.Generator().manual_seed(61)
    H, HV, dk, dv, B, T, layer = 2, 4, 16, 8, 3, 5, 0
    C = 2 * H * dk + HV * dv
    w = _composition_inputs(gen, B * T, H, HV, dk, dv, C)
    slots = 4 + B * T
    conv0 = torch.randn(slots, 1, C, 3, generator=gen)
    state0 = torch.randn(slots, 1, HV, dk, dv, generator=gen) * 0.1
    base = torch.tensor([2, 0, 3])
    writes = torch.arange(4, 4 + B * T).view(B, T)
    conv_v, state_v = conv0.clone(), state0.clone()
    o_v = gdn.forward_verify(w["mixed"], w["gate"], w["beta"], w["weight"], w["A_log"], w["dt_bias"], conv_v,
                             state_v, layer, base, writes, H, dk, HV, dv)
    conv_d, state_d = conv0.clone(), state0.clone()
    for b in range(B):
        read = int(base[b])
        for t in range(T):
            r = b * T + t
            o = gdn.forward_decode(w["mixed"][r:r + 1], w["gate"][r:r + 1], w["beta"][r:r + 1], w["weight"],
                                   w["A_log"], w["dt_bias"], conv_d, state_d, layer, [read], [int(writes[b, t])], H,
                                   dk, HV, dv)
            torch.testing.assert_close(o_v[r:r + 1], o, rtol=1e-5, atol=1e-6)
            read = int(writes[b, t])
    torch.testing.assert_close(state_v, state_d, rtol=1e-5, atol=1e-6)
    assert torch.equal(conv_v, conv_d)


def test_batched_decode_and_verify_equal_the_per_sequence_forms():
    """The vectorised CPU-baseline forms (index_select / index_copy_ pool I/O)
    against ``forward_decode`` / ``forward_verify``."""
    gen = torch.Generator().manual_seed(62)
    H, HV, dk, dv, B, T = 2, 4, 16, 8, 4, 3
    C = 2 * H * dk + HV * dv
    w = _composition_inputs(gen, B * T, H, HV, dk, dv, C)
    w["mixed"] = w["mixed"].to(torch.bfloat16)
    conv0 = torch.randn(20, 2, C, 3, generator=gen).to(torch.bfloat16)
    state0 = torch.randn(20, 2, HV, dk, dv, generator=gen) * 0.1
    reads, writes = torch.tensor([3, 7, 1, 0]), torch.tensor([3, 9, 11, 12])
    a = (conv0.clone(), state0.clone())
    b = (conv0.clone(), state0.clone())
    args = (w["gate"][:B], w["beta"][:B], w["weight"].to(torch.bfloat16), w["A_log"], w["dt_bias"])
    o1 = gdn.forward_decode(w["mixed"][:B], *args, *a, 1, reads, writes, H, dk, HV, dv)
    o2 = gdn.forward_decode_batched(w["mixed"][:B], *args, *b, 1, reads, writes, H, dk, HV, dv)
    torch.testing.assert_close(o2.float(), o1.float(), rtol=1e-2, atol=1e-2)
    assert torch.equal(a[0], b[0])
    torch.testing.assert_close(a[1], b[1], rtol=1e-5, atol=1e-6)
    base, wt = torch.tensor([3, 7, 1, 0]), torch.arange(8, 8 + B * T).view(B, T)
    a = (conv0.clone(), state0.clone())
    b = (conv0.clone(), state0.clone())
    args = (w["gate"], w["beta"], w["weight"].to(torch.bfloat16), w["A_log"], w["dt_bias"])
    o1 = gdn.forward_verify(w["mixed"], *args, *a, 0, base, wt, H, dk, HV, dv)
    o2 = gdn.forward_verify_batched(w["mixed"], *args, *b, 0, base, wt, H, dk, HV, dv)
    torch.testing.assert_close(o2.float(), o1.float(), rtol=1e-2, atol=1e-2)
    assert torch.equal(a[0], b[0])
    torch.testing.assert_close(a[1], b[1], rtol=1e-5, atol=1e-6)
