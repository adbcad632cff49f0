"""CPU torch restatement of the reference's Gated DeltaNet arithmetic.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Paths cited below are
relative to the reference repository root (``python/logssms/...``).

Pinning (what makes these functions trustworthy, see ``tests/test_oracle.py``):

* ``naive_recurrence`` -- closed forms: one token from a zero state
  (``S = beta k v^T``, ``o = scale beta (k.q) v``), ``beta = 0`` (pure decay,
  ``S_T = exp(sum g) S_0``), ``g = 0, beta = 1`` with orthonormal keys (exact
  delta-rule overwrite: ``S^T k_i = v_i``), and the single-pass decode identity
  ``o = e^g S^T q + delta (k.q)`` (``fused_recurrent.py:219-222``).
* ``chunk_gdn`` -- an independent algorithm (WY/UT chunk form) checked
  against ``naive_recurrence`` in float64 to 1e-10 for chunk sizes 1..64,
  ragged lengths, partial chunks and initial states; chunk size 1 reduces the
  chunk form to the recurrence itself.
* ``fused_recurrent`` -- equals normalise + gate + ``naive_recurrence`` and
  the single-pass identity above.
* ``prepare_gdn`` -- closed form of ``tests/kernel/test_prepare_gdn.py:11-19``
  and the softplus edge table of ``:88-96`` computed with ``math.log1p``.
* ``packed_causal_conv1d`` / ``conv_decode`` / ``verify_conv`` -- checked
  against ``torch.nn.functional.conv1d`` (a library routine) on the
  reference tests' closed form ``silu(conv1d(cat(history, x)))``
  (``tests/layers/test_linear_attention_backend.py:191-197``,
  ``tests/layers/test_conv_decode.py:58-62``); window snapshots are compared
  bit-exactly with ``cat(history, x)[..., -3:]``.

* ``rms_norm_gated`` -- ``torch.nn.functional.rms_norm`` and
  ``torch.nn.functional.silu`` (library routines) in float64, the closed form
  of ``tests/kernel/test_grouped_norm_gated.py:21-30`` (one group, norm before
  the gate), and closed forms: a zero gate gives zero, a constant row ``c``
  gives ``c / sqrt(c^2 + eps) * w * silu(z)``, positive row scaling leaves the
  result unchanged (up to eps).

Parity unpinned (documented, within tolerance only): the reference GPU path's
intermediate bf16 roundings inside the chunk pipeline (A, W, U, h, v'
stored in bf16 by ``chunk_fwd.py:319``, ``wy_fast.py:125-126``,
``chunk_delta_h.py:164,307``), the decode conv's bf16 product rounding in
Triton (``conv_decode.py:262``), and libdevice transcendental rounding.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

# gated_delta.py:12 -- the cumulative gate is kept in log2 units.
RCP_LN2 = 1.4426950216


def _acc_dtype(dtype):
    """The reference kernels accumulate in fp32; float64 inputs (used only to
    pin the oracle itself) accumulate in float64."""
    return torch.float64 if dtype == torch.float64 else torch.float32


# --------------------------------------------------------------------------
# activations / gates
# --------------------------------------------------------------------------

def softplus_prefill(x: torch.Tensor) -> torch.Tensor:
    """kernel/fused.py:115 -- x if x > 20 else log1p(exp(min(x, 20)))."""
    return torch.where(x > 20.0, x, torch.log1p(torch.exp(torch.clamp(x, max=20.0))))


def softplus_decode(x: torch.Tensor) -> torch.Tensor:
    """vendor/fla/fused_recurrent.py:20-22 -- log(1 + exp(x)) if x < 20 else x."""
    return torch.where(x < 20.0, torch.log(1.0 + torch.exp(torch.clamp(x, max=20.0))), x)


def silu(x: torch.Tensor) -> torch.Tensor:
    """packed_conv.py:139 -- x / (1 + exp(-x))."""
    return x / (1.0 + torch.exp(-x))


def l2norm(x: torch.Tensor) -> torch.Tensor:
    """kernel/fused.py:95-96 -- x * rsqrt(sum(x^2) + 1e-6) over the last dim."""
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + 1e-6)


def prepare_gdn(query, key, value, gate, beta, A_log, dt_bias):
    """kernel/fused.py:120-158 (kernel :53-117).

    Returns (q_hat, k_hat, v, g_fp32, beta_fp32) with q/k/v in the input dtype.
    """
    dtype = query.dtype
    q = l2norm(query.float()).to(dtype)
    k = l2norm(key.float()).to(dtype)
    g = -torch.exp(A_log.float()) * softplus_prefill(gate.float() + dt_bias.float())
    b = torch.sigmoid(beta.float())
    return q, k, value.contiguous().clone(), g.float(), b.float()


# --------------------------------------------------------------------------
# causal conv1d
# --------------------------------------------------------------------------

def _scale_inputs(values: torch.Tensor, channels: torch.Tensor, boundaries, scales):
    """packed_conv.py:24-30 -- per-channel-range input scale, rounded back."""
    if tuple(scales) == (1.0, 1.0, 1.0):
        return values
    end0, end1 = boundaries
    s = torch.where(channels < end0, scales[0], torch.where(channels < end1, scales[1], scales[2]))
    return (values.float() * s.float()).to(values.dtype)


def packed_causal_conv1d(x, weight, history, cu_seqlens, bias=None, *,
                         input_boundaries=None, input_scales=(1.0, 1.0, 1.0), window_rows=None):
    """kernel/linear_attention/packed_conv.py:53-140 (wrapper :143-192).

    x [T, C] (any dtype), weight [C, 1, W], history [N, C, W-1].
    Returns (y [T, C] in x.dtype, windows [T, C, W-1]) where ``windows[t]`` is
    the raw (scaled) input window ``[x_{t-W+2}, ..., x_t]`` that the kernel
    scatters to ``slots[t] >= 0`` (``:112-123``).  With ``window_rows`` (a
    list of packed rows) only those windows are kept: ``windows[i]`` is the
    window of row ``window_rows[i]`` (large inputs need not hold all T).
    """
    T, C = x.shape
    K = weight.shape[-1]
    S = K - 1
    channels = torch.arange(C)
    if input_boundaries is None:
        input_boundaries = (C, C)
    xs = _scale_inputs(x, channels[None, :], input_boundaries, input_scales)
    y = torch.empty(T, C, dtype=x.dtype)
    rows = list(range(T)) if window_rows is None else [int(t) for t in window_rows]
    windows = torch.empty(len(rows), C, S, dtype=x.dtype)
    acc_t = _acc_dtype(x.dtype)
    w = weight.reshape(C, K).to(acc_t)
    cu = [int(v) for v in cu_seqlens]
    for r in range(len(cu) - 1):
        b, e = cu[r], cu[r + 1]
        src = torch.cat([history[r].T.to(x.dtype), xs[b:e]], 0)  # [S + L, C]
        L = e - b
        src_acc = src.to(acc_t)
        acc = torch.zeros(L, C, dtype=acc_t)
        for tap in range(K):
            acc = acc + src_acc[tap:tap + L] * w[None, :, tap]
        if bias is not None:
            acc = acc + bias.to(acc_t)[None, :]
        acc = acc.to(x.dtype).to(acc_t)
        y[b:e] = silu(acc).to(x.dtype)
        if window_rows is None:
            for tap in range(1, K):
                windows[b:e, :, tap - 1] = src[tap:tap + L]
            continue
        for i, t in enumerate(rows):
            if b <= t < e:  # src row (t - b) + tap holds x_{t - S + tap}
                windows[i] = src[t - b + 1:t - b + K].T
    return y, windows


def conv_decode(x, weight, conv_state, layer, read_slots, write_slots, *, bias=None,
                round_conv=False, input_boundaries=None, input_scales=(1.0, 1.0, 1.0)):
    """kernel/linear_attention/conv_decode.py:25-289 (wrapper :293-352).

    x [B, C]; conv_state [slots, L, C, W-1] is updated in place:
    ``conv_state[write, layer] = [window[1:], x]`` read from ``read`` (``:114-159``).
    Returns y [B, C] in x.dtype (``SiLU(sum w * [window, x] + bias)``, rounded
    to x.dtype before SiLU only when ``round_conv``).
    """
    B, C = x.shape
    K = weight.shape[-1]
    channels = torch.arange(C)
    if input_boundaries is None:
        input_boundaries = (C, C)
    xs = _scale_inputs(x, channels[None, :], input_boundaries, input_scales)
    reads = [int(v) for v in read_slots]
    writes = [int(v) for v in write_slots]
    windows = torch.stack([conv_state[s, layer] for s in reads])  # [B, C, S]
    acc_t = _acc_dtype(x.dtype)
    full = torch.cat([windows, xs[:, :, None]], -1).to(acc_t)  # [B, C, K]
    acc = (full * weight.reshape(C, K).to(acc_t)[None]).sum(-1)
    if bias is not None:
        acc = acc + bias.to(acc_t)[None]
    if round_conv:
        acc = acc.to(x.dtype).to(acc_t)
    y = silu(acc).to(x.dtype)
    new = torch.cat([windows[:, :, 1:], xs[:, :, None]], -1)
    for b in range(B):
        conv_state[writes[b], layer] = new[b]
    return y


def verify_conv(x, weight, history):
    """layers/linear_attention_backend/gdn.py:176-196 -- the verify path's
    torch conv: ``silu(conv1d(cat(state, x^T), w, groups=C))`` evaluated in the
    input dtype (rounded before and after SiLU), plus the per-step windows
    ``unfold(-1, W-1, 1)[:, :, 1:]``.

    x [B, T, C], history [B, C, W-1].  Returns (y [B, T, C], windows [B, T, C, W-1]).
    """
    B, T, C = x.shape
    K = weight.shape[-1]
    S = K - 1
    src = torch.cat([history.to(x.dtype), x.transpose(1, 2)], -1)  # [B, C, S+T]
    acc_t = _acc_dtype(x.dtype)
    acc = torch.zeros(B, C, T, dtype=acc_t)
    w = weight.reshape(C, K).to(acc_t)
    for tap in range(K):
        acc = acc + src[:, :, tap:tap + T].to(acc_t) * w[None, :, tap, None]
    y = silu(acc.to(x.dtype).to(acc_t)).to(x.dtype).transpose(1, 2)
    windows = torch.stack([src[:, :, t + 1:t + 1 + S] for t in range(T)], 1)
    return y.contiguous(), windows


# --------------------------------------------------------------------------
# recurrences
# --------------------------------------------------------------------------

def _expand_heads(x: torch.Tensor, hv: int) -> torch.Tensor:
    """GQA: key head of v-head h is h // (HV // H)."""
    h = x.shape[-2]
    return x.repeat_interleave(hv // h, dim=-2)


def naive_recurrence(q, k, v, g, beta, scale, state0, *, checkpoint_every=None):
    """Token-by-token gated delta rule, the semantics of
    ``tests/kernel/test_gdn_prefill_dispatch.py:165-180`` and
    ``vendor/fla/fused_recurrent.py:223-227``.

    q, k [T, H, dk] (already normalised), v [T, HV, dv], g (natural-log decay)
    and beta [T, HV], state0 [HV, dk, dv].  Computes in the dtype of ``state0``.
    Returns (o [T, HV, dv], final state, list of checkpoint states taken after
    every ``checkpoint_every`` tokens and at the end).
    """
    dt = state0.dtype
    T = q.shape[0]
    HV = v.shape[1]
    qe = _expand_heads(q.to(dt), HV) * scale
    ke = _expand_heads(k.to(dt), HV)
    v = v.to(dt)
    g = g.to(dt)
    beta = beta.to(dt)
    state = state0.clone()
    out = torch.empty(T, HV, v.shape[-1], dtype=dt)
    checkpoints = []
    for t in range(T):
        state = state * torch.exp(g[t])[:, None, None]
        residual = (v[t] - (state * ke[t][:, :, None]).sum(1)) * beta[t][:, None]
        state = state + ke[t][:, :, None] * residual[:, None, :]
        out[t] = (state * qe[t][:, :, None]).sum(1)
        if checkpoint_every is not None and ((t + 1) % checkpoint_every == 0 or t == T - 1):
            checkpoints.append(state.clone())
    return out, state, checkpoints


def chunk_gdn(q, k, v, g, beta, scale, state0, chunk_size=64, rcp_ln2=RCP_LN2, on_chunk_end=None):
    """The chunked (WY/UT) gated delta rule of one sequence, restating the
    reference pipeline ``vendor/fla/gated_delta.py:15-82``:

    * ``G`` = chunk-local cumsum of g times 1/ln2 (``cumsum.py:19-75``)
    * ``A = (I + strict_tril(beta_i k_i.k_j 2^(G_i - G_j)))^-1`` (``chunk_fwd.py:26-294``)
    * ``W = A (beta 2^G k)``, ``U = A (beta v)`` (``wy_fast.py:19-86``)
    * per chunk ``v' = U - W h``, ``h <- 2^G_last h + k^T (2^(G_last - G) v')``
      (``chunk_delta_h.py:142-254``)
    * ``o = scale (2^G (q h) + tril_incl(q k^T 2^(G_i - G_j)) v')`` (``chunk_o.py:85-130``)

    Shapes as in ``naive_recurrence``.  Returns (o, v_new, chunk_end_states
    [NT, HV, dk, dv], final state).  ``rcp_ln2`` defaults to the reference's
    truncated constant (relative exponent error 1.3e-8 against ``1/ln 2``).
    With ``on_chunk_end(i, h)`` each chunk-end state is handed to the callback
    instead and ``chunk_end_states`` comes back empty.
    """
    dt = state0.dtype
    T = q.shape[0]
    HV = v.shape[1]
    # head-major copies, so every chunk below is a contiguous slab
    qe = _expand_heads(q.to(dt), HV).transpose(0, 1).contiguous()  # [HV, T, dk]
    ke = _expand_heads(k.to(dt), HV).transpose(0, 1).contiguous()
    ve = v.to(dt).transpose(0, 1).contiguous()  # [HV, T, dv]
    ge = g.to(dt).transpose(0, 1).contiguous()  # [HV, T]
    be = beta.to(dt).transpose(0, 1).contiguous()
    h = state0.clone()
    o = torch.empty(HV, T, v.shape[-1], dtype=dt)
    v_new = torch.empty_like(o)
    ends = []
    for c0 in range(0, T, chunk_size):
        c1 = min(c0 + chunk_size, T)
        n = c1 - c0
        kc, qc, vc = ke[:, c0:c1], qe[:, c0:c1], ve[:, c0:c1]
        bc = be[:, c0:c1]
        G = torch.cumsum(ge[:, c0:c1], -1) * rcp_ln2  # [HV, n]
        diff = G[:, :, None] - G[:, None, :]
        strict = torch.tril(torch.ones(n, n, dtype=torch.bool), -1)
        incl = torch.tril(torch.ones(n, n, dtype=torch.bool))
        decay = torch.exp2(torch.where(incl, diff, torch.zeros_like(diff)))
        L = torch.where(strict, bc[:, :, None] * (kc @ kc.transpose(1, 2)) * decay, 0.0)
        eye = torch.eye(n, dtype=dt).expand(HV, n, n)
        A = torch.linalg.solve_triangular(eye + L, eye, upper=False, unitriangular=True)
        W = A @ (bc[:, :, None] * torch.exp2(G)[:, :, None] * kc)
        U = A @ (bc[:, :, None] * vc)
        vn = U - W @ h
        v_new[:, c0:c1] = vn
        M = torch.where(incl, (qc @ kc.transpose(1, 2)) * decay, 0.0)
        o[:, c0:c1] = scale * (torch.exp2(G)[:, :, None] * (qc @ h) + M @ vn)
        g_last = G[:, -1]
        h = torch.exp2(g_last)[:, None, None] * h + kc.transpose(1, 2) @ (
            torch.exp2(g_last[:, None] - G)[:, :, None] * vn)
        if on_chunk_end is not None:
            on_chunk_end(c0 // chunk_size, h)
        else:
            ends.append(h.clone())
    end_states = torch.stack(ends) if ends else torch.empty(0, *h.shape, dtype=dt)
    return o.transpose(0, 1), v_new.transpose(0, 1), end_states, h


def chunk_gated_delta_rule_to_cache(query, key, value, gate, beta, storage, read_slots,
                                    chunk_write_slots, cu_seqlens, *, layer=0,
                                    final_write_slots=None, chunk_size=64,
                                    dtype=torch.float32):
    """Pool-level semantics of ``vendor/fla/gated_delta.py:15-82`` +
    ``chunk_delta_h.py:89-139,226-284`` + ``state_io.py:79``:

    * initial state of sequence n = ``storage[read_slots[n], layer]`` or zero
      when the slot is negative;
    * after global chunk ``c`` the chunk-end state goes to
      ``storage[chunk_write_slots[c], layer]`` when that slot is >= 0;
    * optional ``final_write_slots[n]`` receives the final state.

    query/key [1, T, H, dk], value [1, T, HV, dv], gate/beta [1, T, HV]
    (already prepared: g natural-log decay, beta in [0, 1]).  ``storage`` is
    mutated in place (written in its own dtype).  Returns (o [1, T, HV, dv]
    in value.dtype, v_new in value.dtype).
    """
    cu = [int(x) for x in cu_seqlens]
    HV, dk, dv = storage.shape[2:]
    scale = query.shape[-1] ** -0.5
    T = query.shape[1]
    o = torch.empty(1, T, HV, dv, dtype=value.dtype)
    v_new = torch.empty_like(o)
    chunk = 0
    for n in range(len(cu) - 1):
        b, e = cu[n], cu[n + 1]
        slot = int(read_slots[n])
        if slot >= 0:
            s0 = storage[slot, layer].to(dtype)
        else:
            s0 = torch.zeros(HV, dk, dv, dtype=dtype)
        def write_end(i, h, first=chunk):
            ws = int(chunk_write_slots[first + i])
            if ws >= 0:
                storage[ws, layer] = h.to(storage.dtype)

        on, vn, _, final = chunk_gdn(query[0, b:e], key[0, b:e], value[0, b:e],
                                     gate[0, b:e], beta[0, b:e], scale, s0, chunk_size,
                                     on_chunk_end=write_end)
        o[0, b:e] = on.to(value.dtype)
        v_new[0, b:e] = vn.to(value.dtype)
        chunk += (e - b + chunk_size - 1) // chunk_size
        if final_write_slots is not None and int(final_write_slots[n]) >= 0:
            storage[int(final_write_slots[n]), layer] = final.to(storage.dtype)
    return o, v_new


def fused_recurrent(query, key, value, gate, beta, A_log, dt_bias, initial_state,
                    dtype=torch.float32):
    """vendor/fla/fused_recurrent.py:461-550 (kernel :31-288, plain mode).

    Raw inputs: q/k [B, T, H, dk] are L2-normalised inside (``:206-207``),
    ``g = -exp(A_log) softplus(gate + dt_bias)`` (decode softplus ``:20-22``),
    ``beta = sigmoid(beta)``.  initial_state [B, HV, dk, dv].
    Returns (o [B, T, HV, dv] in value.dtype, states [B, T, HV, dk, dv] in
    initial_state.dtype) -- every per-step state is kept (``:266-275``).
    """
    B, T, H, dk = query.shape
    HV, dv = value.shape[2:]
    scale = dk ** -0.5
    q = l2norm(query.to(dtype))
    k = l2norm(key.to(dtype))
    g = -torch.exp(A_log.to(dtype))[None, None] * softplus_decode(gate.to(dtype) + dt_bias.to(dtype))
    b = torch.sigmoid(beta.to(dtype))
    o = torch.empty(B, T, HV, dv, dtype=value.dtype)
    states = torch.empty(B, T, HV, dk, dv, dtype=initial_state.dtype)
    for i in range(B):
        state = initial_state[i].to(dtype)
        qe = _expand_heads(q[i], HV) * scale
        ke = _expand_heads(k[i], HV)
        for t in range(T):
            state = state * torch.exp(g[i, t])[:, None, None]
            delta = (value[i, t].to(dtype) - (state * ke[t][:, :, None]).sum(1)) * b[i, t][:, None]
            state = state + ke[t][:, :, None] * delta[:, None, :]
            o[i, t] = (state * qe[t][:, :, None]).sum(1).to(value.dtype)
            states[i, t] = state.to(initial_state.dtype)
    return o, states


def fused_recurrent_to_slots(query, key, value, gate, beta, A_log, dt_bias, state_pool,
                             read_slots, write_slots, layer, dtype=torch.float32):
    """vendor/fla/fused_recurrent.py:396-458 (SLOTTED_STORE mode, ``:98-114,262-281``).

    Decode (T = 1): ``state_pool[write, layer] <- step(state_pool[read, layer])``.
    The pool is mutated in place.  Returns o [B, 1, HV, dv].
    """
    reads = [int(x) for x in read_slots]
    writes = [int(x) for x in write_slots]
    init = torch.stack([state_pool[s, layer] for s in reads])
    o, states = fused_recurrent(query, key, value, gate, beta, A_log, dt_bias, init, dtype)
    for i, s in enumerate(writes):
        state_pool[s, layer] = states[i, -1].to(state_pool.dtype)
    return o


def store_state(pool, indices, states):
    """kernel/store.py:69-83 + csrc/jit/store.cu:152-182:
    ``pool[indices[i]] = states[i]`` for every ``indices[i] >= 0`` (byte copy)."""
    flat_pool = pool.view(pool.shape[0], -1)
    flat = states.reshape(states.shape[0], -1)
    for i, idx in enumerate(int(x) for x in indices):
        if idx >= 0:
            flat_pool[idx] = flat[i]


# --------------------------------------------------------------------------
# backend-level compositions (layers/linear_attention_backend/gdn.py)
# --------------------------------------------------------------------------

def split_qkv(mixed, num_k_heads, head_k_dim, num_v_heads, head_v_dim):
    """gdn.py:51-72 -- channel split ``[key_dim, key_dim, value_dim]``."""
    key_dim = num_k_heads * head_k_dim
    lead = mixed.shape[:-1]
    q = mixed[..., :key_dim].reshape(*lead, num_k_heads, head_k_dim)
    k = mixed[..., key_dim:2 * key_dim].reshape(*lead, num_k_heads, head_k_dim)
    v = mixed[..., 2 * key_dim:].reshape(*lead, num_v_heads, head_v_dim)
    return q, k, v


def forward_prefill(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, conv_state,
                    recurrent_state, layer, cu_seqlens, baseline_slots, chunk_write_slots,
                    conv_token_slots, num_k_heads, head_k_dim, num_v_heads, head_v_dim,
                    dtype=torch.float32):
    """gdn.py:74-149 -- conv history gather, packed conv with window snapshots
    at ``conv_token_slots``, split, prepare_gdn, chunked rule to cache.
    Mutates both pools; returns o [T, HV, dv]."""
    N = len(cu_seqlens) - 1
    C = mixed_qkv.shape[1]
    S = conv_weight.shape[-1] - 1
    history = torch.zeros(N, C, S, dtype=mixed_qkv.dtype)
    for n in range(N):
        s = int(baseline_slots[n])
        if s >= 0:
            history[n] = conv_state[s, layer]
    token_slots = [int(x) for x in conv_token_slots]
    rows = [t for t, s in enumerate(token_slots) if s >= 0]
    y, windows = packed_causal_conv1d(mixed_qkv, conv_weight, history, cu_seqlens, window_rows=rows)
    for i, t in enumerate(rows):
        conv_state[token_slots[t], layer] = windows[i]
    q, k, v = split_qkv(y[None], num_k_heads, head_k_dim, num_v_heads, head_v_dim)
    q, k, v, g, b = prepare_gdn(q, k, v, gate[None], beta[None], A_log, dt_bias)
    o, _ = chunk_gated_delta_rule_to_cache(q, k, v, g, b, recurrent_state, baseline_slots,
                                           chunk_write_slots, cu_seqlens, layer=layer,
                                           dtype=dtype)
    return o[0]


def forward_decode(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, conv_state,
                   recurrent_state, layer, read_slots, write_slots, num_k_heads, head_k_dim,
                   num_v_heads, head_v_dim, dtype=torch.float32):
    """gdn.py:222-265 -- conv_decode (split q/k/v, no pre-SiLU rounding) then
    the slotted recurrent update.  Mutates both pools; returns o [B, HV, dv]."""
    y = conv_decode(mixed_qkv, conv_weight, conv_state, layer, read_slots, write_slots)
    q, k, v = split_qkv(y[:, None], num_k_heads, head_k_dim, num_v_heads, head_v_dim)
    o = fused_recurrent_to_slots(q, k, v, gate[:, None], beta[:, None], A_log, dt_bias,
                                 recurrent_state, read_slots, write_slots, layer, dtype)
    return o[:, 0]


def forward_verify(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, conv_state,
                   recurrent_state, layer, baseline_slots, write_slots, num_k_heads,
                   head_k_dim, num_v_heads, head_v_dim, dtype=torch.float32):
    """gdn.py:151-220 for one length group: rows are ``B*T`` consecutive
    tokens (``B`` sequences of ``T`` drafts).  Conv windows and per-step states
    go to ``write_slots[B, T]``.  Returns o [B*T, HV, dv]."""
    B, T = write_slots.shape
    C = mixed_qkv.shape[1]
    x = mixed_qkv.view(B, T, C)
    hist = torch.stack([conv_state[int(s), layer] for s in baseline_slots])
    y, windows = verify_conv(x, conv_weight, hist)
    flat_slots = [int(s) for s in write_slots.flatten()]
    for i, s in enumerate(flat_slots):
        conv_state[s, layer] = windows.flatten(0, 1)[i]
    q, k, v = split_qkv(y, num_k_heads, head_k_dim, num_v_heads, head_v_dim)
    init = torch.stack([recurrent_state[int(s), layer] for s in baseline_slots])
    o, states = fused_recurrent(q, k, v, gate.view(B, T, -1), beta.view(B, T, -1), A_log,
                                dt_bias, init, dtype)
    pool_layer = recurrent_state[:, layer]
    for i, s in enumerate(flat_slots):
        if s >= 0:
            pool_layer[s] = states.flatten(0, 1)[i].to(recurrent_state.dtype)
    return o.flatten(0, 1)


def _batched_step(conv_state, recurrent_state, layer, x, gate, beta, conv_weight, A_log, dt_bias, reads,
                  writes, round_conv, H, dk, HV, dv, dtype):
    """One token for every sequence at once: conv window of ``reads`` ->
    ``writes``, split, normalise, gate, recurrence of ``reads`` -> ``writes``
    (pool I/O through ``index_select`` / ``index_copy_``).  Returns o [B, HV, dv]."""
    B, C = x.shape
    K = conv_weight.shape[-1]
    conv_layer = conv_state[:, layer]
    windows = conv_layer.index_select(0, reads)  # [B, C, K-1]
    acc = (torch.cat([windows, x[:, :, None]], -1).to(dtype) * conv_weight.reshape(C, K).to(dtype)[None]).sum(-1)
    if round_conv:
        acc = acc.to(x.dtype).to(dtype)
    y = silu(acc).to(x.dtype)
    conv_layer.index_copy_(0, writes, torch.cat([windows[:, :, 1:], x[:, :, None]], -1))
    q, k, v = split_qkv(y, H, dk, HV, dv)
    q = _expand_heads(l2norm(q.to(dtype)), HV) * dk ** -0.5  # [B, HV, dk]
    k = _expand_heads(l2norm(k.to(dtype)), HV)
    g = -torch.exp(A_log.to(dtype))[None] * softplus_decode(gate.to(dtype) + dt_bias.to(dtype))
    b = torch.sigmoid(beta.to(dtype))
    pool_layer = recurrent_state[:, layer]
    S = pool_layer.index_select(0, reads).to(dtype) * torch.exp(g)[:, :, None, None]
    delta = (v.to(dtype) - (S * k[..., None]).sum(2)) * b[..., None]
    S = S + k[..., None] * delta[:, :, None, :]
    o = (S * q[..., None]).sum(2)
    pool_layer.index_copy_(0, writes, S.to(recurrent_state.dtype))
    return o.to(x.dtype)


def forward_decode_batched(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, conv_state,
                           recurrent_state, layer, read_slots, write_slots, num_k_heads, head_k_dim,
                           num_v_heads, head_v_dim, dtype=torch.float32):
    """``forward_decode`` vectorised over sequences, with the pool I/O as
    ``index_select`` / ``index_copy_`` (the CPU baseline form for decode).
    Read and write slot sets must each be free of repeats."""
    reads = torch.as_tensor(read_slots, dtype=torch.long)
    writes = torch.as_tensor(write_slots, dtype=torch.long)
    return _batched_step(conv_state, recurrent_state, layer, mixed_qkv, gate, beta, conv_weight, A_log, dt_bias,
                         reads, writes, False, num_k_heads, head_k_dim, num_v_heads, head_v_dim, dtype)


def forward_verify_batched(mixed_qkv, gate, beta, conv_weight, A_log, dt_bias, conv_state,
                           recurrent_state, layer, baseline_slots, write_slots, num_k_heads,
                           head_k_dim, num_v_heads, head_v_dim, dtype=torch.float32):
    """``forward_verify`` as T batched steps (the CPU baseline form for
    verify): step t reads the window and state step t-1 wrote to
    ``write_slots[:, t-1]`` (the baseline slots for t = 0), with the conv
    pre-activation rounded to the io dtype as the verify torch conv does."""
    B, T = write_slots.shape
    writes = torch.as_tensor(write_slots, dtype=torch.long)
    x = mixed_qkv.view(B, T, -1)
    gv, bv = gate.view(B, T, -1), beta.view(B, T, -1)
    out = torch.empty(B, T, num_v_heads, head_v_dim, dtype=mixed_qkv.dtype)
    read = torch.as_tensor(baseline_slots, dtype=torch.long)
    for t in range(T):
        out[:, t] = _batched_step(conv_state, recurrent_state, layer, x[:, t], gv[:, t], bv[:, t], conv_weight,
                                  A_log, dt_bias, read, writes[:, t], True, num_k_heads, head_k_dim, num_v_heads,
                                  head_v_dim, dtype)
        read = writes[:, t]
    return out.flatten(0, 1)


def single_pass_decode_output(state, q_hat, k_hat, v, g, beta, scale):
    """The one-read decode identity of ``fused_recurrent.py:219-222`` /
    ``gdn_replay.py``: with ``S' = e^g S + k delta^T``,
    ``o = scale (e^g S^T q + delta (k.q))``.  Used to pin the recurrences."""
    decayed_k = math.exp(g) * (state * k_hat[:, None]).sum(0)
    decayed_q = math.exp(g) * (state * q_hat[:, None]).sum(0)
    delta = (v - decayed_k) * beta
    return scale * (decayed_q + delta * float((k_hat * q_hat).sum()))


def rms_norm_gated(hidden_states, gate, weight, eps):
    """``rms_norm_gated`` (``kernel/norm.py:151-187``; Triton kernel ``:113-148``):
    per row of ``hidden_states.shape[-1]`` channels,
    ``(x * rsqrt(sum(x^2) / n + eps)) * w * (z * sigmoid(z))`` in float32,
    returned in the dtype of ``hidden_states``.  Row ``r`` of the flattened
    hidden rows pairs with row ``r`` of ``gate.reshape(-1, n)``, as the
    reference's ``gate.reshape(-1, gate.shape[-2], n)`` indexing does
    (``:134-137``)."""
    n = hidden_states.shape[-1]
    assert hidden_states.shape == gate.shape and weight.numel() == n
    x = hidden_states.reshape(-1, n).float()
    z = gate.reshape(-1, n).float()
    variance = (x * x).sum(-1, keepdim=True) / n
    y = (x * torch.rsqrt(variance + eps)) * weight.float() * (z * torch.sigmoid(z))
    return y.to(hidden_states.dtype).view(hidden_states.shape)
