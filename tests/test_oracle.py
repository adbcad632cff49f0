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
