"""Pins the LogState frame-table addressing of the oracle (``oracle/frames.py``).

With the identity table (slot s owns frames s fps .. s fps + fps - 1) the frame
storage is one contiguous pool, so every read must equal a plain reshape of
the storage; relabelling frames must not change what a slot reads; the chunk
pipeline on frames must equal the plain-pool pipeline bit for bit.  An index
slip (frame vs element units, a head offset off by one, the wrong table
column) fails one of these.
"""

import pytest
import torch
import torch.nn.functional as F

from oracle import frames as fr
from oracle import gdn

# (dk, dv, frame_bytes, head_bytes): heads inside a frame, heads spanning two
# frames, a padded head (48 state bytes in a 64-byte payload)
LAYOUTS = [(8, 4, 128, 64), (8, 4, 32, 64), (6, 4, 128, 64), (4, 4, 64, 32)]


def _identity(slots, fps):
    return (torch.arange(slots)[:, None] * fps + torch.arange(fps)[None, :]).to(torch.int32)


def _setup(dk, dv, frame_bytes, head_bytes, layers=2, HV=3, slots=4, dtype=torch.bfloat16, seed=0):
    itemsize = torch.tensor([], dtype=dtype).element_size()
    fps = -(-layers * HV * head_bytes // frame_bytes)
    g = torch.Generator().manual_seed(seed)
    storage = torch.randn(slots * fps, frame_bytes // itemsize, generator=g).to(dtype)
    return storage, _identity(slots, fps), fps, itemsize


def _as_pool(storage, slots, layers, HV, dk, dv, head_bytes, itemsize):
    """The identity-table storage read as a plain [slots, layers, HV, dk, dv] pool."""
    head = head_bytes // itemsize
    per_slot = storage.reshape(slots, -1)[:, :layers * HV * head]
    return per_slot.reshape(slots, layers, HV, head)[..., :dk * dv].reshape(slots, layers, HV, dk, dv)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_identity_table_reads_a_contiguous_pool(layout):
    dk, dv, frame_bytes, head_bytes = layout
    storage, frames, _, itemsize = _setup(dk, dv, frame_bytes, head_bytes)
    pool = _as_pool(storage, 4, 2, 3, dk, dv, head_bytes, itemsize)
    for layer in range(2):
        got = fr.read_frame_states(storage, frames, [3, 0, 2], layer, 3, dk, dv, frame_bytes, head_bytes)
        torch.testing.assert_close(got, pool[[3, 0, 2], layer], rtol=0, atol=0)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_relabelled_frames_read_and_write_the_same(layout):
    dk, dv, frame_bytes, head_bytes = layout
    storage, frames, _, _ = _setup(dk, dv, frame_bytes, head_bytes, seed=1)
    perm = torch.randperm(storage.shape[0], generator=torch.Generator().manual_seed(2))
    moved = torch.empty_like(storage)
    moved[perm] = storage
    table = perm[frames.long()].to(torch.int32)
    for layer in range(2):
        a = fr.read_frame_states(storage, frames, [0, 1, 2, 3], layer, 3, dk, dv, frame_bytes, head_bytes)
        b = fr.read_frame_states(moved, table, [0, 1, 2, 3], layer, 3, dk, dv, frame_bytes, head_bytes)
        torch.testing.assert_close(a, b, rtol=0, atol=0)
    values = torch.randn(2, 3, dk, dv, generator=torch.Generator().manual_seed(3)).to(storage.dtype)
    fr.write_frame_states(storage, frames, [2, 1], 1, values, frame_bytes, head_bytes)
    fr.write_frame_states(moved, table, [2, 1], 1, values, frame_bytes, head_bytes)
    torch.testing.assert_close(moved[perm], storage, rtol=0, atol=0)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_write_touches_only_the_named_states(layout):
    dk, dv, frame_bytes, head_bytes = layout
    storage, frames, _, itemsize = _setup(dk, dv, frame_bytes, head_bytes, seed=4)
    before = storage.clone()
    values = torch.randn(3, 3, dk, dv, generator=torch.Generator().manual_seed(5)).to(storage.dtype)
    fr.write_frame_states(storage, frames, [2, -1, 0], 1, values, frame_bytes, head_bytes)
    got = fr.read_frame_states(storage, frames, [2, 0], 1, 3, dk, dv, frame_bytes, head_bytes)
    torch.testing.assert_close(got, values[[0, 2]], rtol=0, atol=0)
    expected = _as_pool(before.clone(), 4, 2, 3, dk, dv, head_bytes, itemsize)
    expected[[2, 0], 1] = values[[0, 2]]
    torch.testing.assert_close(_as_pool(storage, 4, 2, 3, dk, dv, head_bytes, itemsize), expected, rtol=0, atol=0)
    # padding bytes of the payload and the unused tail of the last frame stay as they were
    mask = torch.ones(storage.numel(), dtype=torch.bool)
    mask[fr.frame_state_index(frames, [2, 0], 1, 3, dk, dv, itemsize, frame_bytes, head_bytes).reshape(-1)] = False
    assert torch.equal(storage.reshape(-1)[mask], before.reshape(-1)[mask])


@pytest.mark.parametrize("chunk_size", [16, 32])
def test_chunk_on_frames_equals_the_plain_pool(chunk_size):
    dk = dv = 8
    H, HV, layers, slots = 1, 2, 2, 6
    head_bytes = dk * dv * 2
    frame_bytes = 2 * head_bytes
    storage, frames, _, itemsize = _setup(dk, dv, frame_bytes, head_bytes, layers=layers, HV=HV, slots=slots, seed=6)
    storage.mul_(0.1)
    g = torch.Generator().manual_seed(7)
    lengths = [40, 17]
    cu = [0, 40, 57]
    T = cu[-1]
    q = F.normalize(torch.randn(1, T, H, dk, generator=g), dim=-1)
    k = F.normalize(torch.randn(1, T, H, dk, generator=g), dim=-1)
    v = torch.randn(1, T, HV, dv, generator=g)
    gate = -torch.rand(1, T, HV, generator=g) * 0.2
    beta = torch.sigmoid(torch.randn(1, T, HV, generator=g))
    n_int = sum(-(-n // chunk_size) for n in lengths)
    reads = torch.tensor([0, -1])
    writes = torch.full((n_int,), -1)
    writes[0], writes[-1] = 2, 3
    finals = torch.tensor([4, 5])
    pool = _as_pool(storage.clone(), slots, layers, HV, dk, dv, head_bytes, itemsize).contiguous()
    o_a, vn_a = gdn.chunk_gated_delta_rule_to_cache(q, k, v, gate, beta, pool, reads, writes, cu, layer=1,
                                                    final_write_slots=finals, chunk_size=chunk_size)
    o_b, vn_b = fr.chunk_gated_delta_rule_to_frames(q, k, v, gate, beta, storage, frames, frame_bytes, head_bytes,
                                                    reads, writes, cu, layer=1, final_write_slots=finals,
                                                    chunk_size=chunk_size)
    torch.testing.assert_close(o_b, o_a, rtol=0, atol=0)
    torch.testing.assert_close(vn_b, vn_a, rtol=0, atol=0)
    torch.testing.assert_close(_as_pool(storage, slots, layers, HV, dk, dv, head_bytes, itemsize), pool,
                               rtol=0, atol=0)


def _log_case(frame_bytes, seed, key_heads=2):
    """A small token log: 2 layers, granularity 4, page 8, H = 2, HV = 4."""
    H, HV, dk, dv, layers, gran, page = 2, 4, 6, 8, 2, 4, 8
    log_elems = page * layers * (key_heads * dk + HV * dv)
    fps = -(-2 * log_elems // frame_bytes)
    slots = 3
    record = 4 * layers * page * HV
    g = torch.Generator().manual_seed(seed)
    T = 10
    frames = _identity(slots, fps)
    decay = torch.tensor([[slots * fps + s, 0] for s in range(slots)], dtype=torch.int32)
    storage = torch.randn(slots * fps + slots, frame_bytes // 2, generator=g).to(torch.bfloat16)
    log_slots = torch.tensor([0, 2, -1, 0, 2, 2, 0, -1, 2, 0])
    offsets = torch.tensor([0, 1, 3, 5, 7, 2, 3, 4, 6, 7])
    v_new = torch.randn(T, HV, dv, generator=g).to(torch.bfloat16)
    key = torch.randn(T, H, dk, generator=g).to(torch.bfloat16)
    gate = -torch.rand(T, HV, generator=g)
    kw = dict(layer=1, layers=layers, granularity=gran, page_size=page, key_heads=key_heads)
    return storage, frames, decay, record, log_slots, offsets, v_new, key, gate, kw, fps


@pytest.mark.parametrize("frame_bytes", [512, 264, 260])
@pytest.mark.parametrize("key_heads", [2, 1])
def test_identity_table_log_lands_in_the_reshaped_payload(frame_bytes, key_heads):
    """Rows within one frame (512 bytes), value rows straddling frames (264),
    key and value rows straddling frames (260); a decay record (256 bytes)
    always fits one frame."""
    storage, frames, decay, record, slots, offsets, v_new, key, gate, kw, fps = _log_case(frame_bytes, 8, key_heads)
    before = storage.clone()
    fr.store_chunk_log(storage, frames, frame_bytes, slots, offsets, v_new, key, gate, decay, record, **kw)
    H, HV, dk, dv = 2, 4, 6, 8
    gran, page, layers, layer = kw["granularity"], kw["page_size"], kw["layers"], kw["layer"]
    KH = key_heads
    n_slots = 3
    per_layer = gran * (KH * dk + HV * dv)
    payload = storage[:n_slots * fps].reshape(n_slots, -1)[:, :page * layers * (KH * dk + HV * dv)]
    payload = payload.reshape(n_slots, page // gran, layers, per_layer)
    keys = payload[..., :gran * KH * dk].reshape(n_slots, page // gran, layers, KH, gran, dk)
    values = payload[..., gran * KH * dk:].reshape(n_slots, page // gran, layers, HV, gran, dv)
    decay_view = storage[n_slots * fps:].view(torch.uint8)[:, :record].contiguous().view(torch.float32)
    decay_view = decay_view.reshape(n_slots, layers, page, HV)
    last = {}
    for t in range(len(slots)):
        if int(slots[t]) >= 0:
            last[(int(slots[t]), int(offsets[t]))] = t
    for (s, pos), t in last.items():
        assert torch.equal(values[s, pos // gran, layer, :, pos % gran], v_new[t])
        for kh in range(KH):
            h = kh * (HV // KH)
            assert torch.equal(keys[s, pos // gran, layer, kh, pos % gran], key[t, h // (HV // H)])
        assert torch.equal(decay_view[s, layer, pos], gate[t])
    # nothing else moved: restore the logged rows from `before` and compare
    restored = storage.clone()
    rv = restored[:n_slots * fps].reshape(n_slots, -1)[:, :page * layers * (KH * dk + HV * dv)]
    rv = rv.reshape(n_slots, page // gran, layers, per_layer)
    bv = before[:n_slots * fps].reshape(n_slots, -1)[:, :page * layers * (KH * dk + HV * dv)]
    bv = bv.reshape(n_slots, page // gran, layers, per_layer)
    rd = restored[n_slots * fps:].view(torch.uint8)
    bd = before[n_slots * fps:].view(torch.uint8)
    for (s, pos), _ in last.items():
        for kh in range(KH):
            o = (kh * gran + pos % gran) * dk
            rv[s, pos // gran, layer, o:o + dk] = bv[s, pos // gran, layer, o:o + dk]
        for h in range(HV):
            o = gran * KH * dk + (h * gran + pos % gran) * dv
            rv[s, pos // gran, layer, o:o + dv] = bv[s, pos // gran, layer, o:o + dv]
        b = 4 * ((layer * page + pos) * HV)
        rd[s, b:b + 4 * HV] = bd[s, b:b + 4 * HV]
    assert torch.equal(restored.view(torch.int16), before.view(torch.int16))


def test_relabelled_frames_log_the_same():
    storage, frames, decay, record, slots, offsets, v_new, key, gate, kw, _ = _log_case(260, 9)
    perm = torch.randperm(storage.shape[0], generator=torch.Generator().manual_seed(10))
    moved = torch.empty_like(storage)
    moved[perm] = storage
    table = perm[frames.long()].to(torch.int32)
    dtable = decay.clone()
    dtable[:, 0] = perm[decay[:, 0].long()].to(torch.int32)
    fr.store_chunk_log(storage, frames, 260, slots, offsets, v_new, key, gate, decay, record, **kw)
    fr.store_chunk_log(moved, table, 260, slots, offsets, v_new, key, gate, dtable, record, **kw)
    # bit patterns (decay floats written into 16-bit storage may read as NaN)
    assert torch.equal(moved[perm].view(torch.int16), storage.view(torch.int16))


# ---------------------------------------------------------------- LogState decode

def _decode_pool(seed, dtype=torch.float32, dk=8, dv=8, H=2, HV=4, layers=2, page=32, slots=4, conv_dim=12, W=4,
                 granules=2):
    """Frame storage with identity payload tables (state head in one frame of
    two heads), log payloads, decay records and identity conv tables."""
    g = torch.Generator().manual_seed(seed)
    item = torch.tensor([], dtype=dtype).element_size()
    head_bytes = dk * dv * item
    record = 4 * layers * page * HV
    frame_bytes = max(4 * head_bytes, record)
    log_bytes = item * page * layers * (H * dk + HV * dv)
    fps = max(-(-layers * HV * head_bytes // frame_bytes), -(-log_bytes // frame_bytes))
    conv_elems = layers * conv_dim * (W - 1)
    cf = -(-conv_elems * item // frame_bytes)
    n_payload = slots * fps
    n_decay = slots
    n_conv = slots * granules * cf
    storage = (torch.randn(n_payload + n_decay + n_conv, frame_bytes // item, generator=g) * 0.1).to(dtype)
    payload = _identity(slots, fps)
    decay = torch.tensor([[n_payload + s, 0] for s in range(slots)], dtype=torch.int32)
    conv = (n_payload + n_decay + torch.arange(slots * granules * cf).reshape(slots, granules, cf)).to(torch.int32)
    return dict(storage=storage, payload=payload, decay=decay, conv=conv, frame_bytes=frame_bytes,
                head_bytes=head_bytes, record=record, fps=fps, cf=cf, gen=g, dk=dk, dv=dv, H=H, HV=HV,
                layers=layers, page=page, slots=slots, conv_dim=conv_dim, W=W, granules=granules)


def test_logstate_conv_decode_equals_plain_conv_decode():
    P = _decode_pool(11)
    C, W, S, G = P["conv_dim"], P["W"], P["W"] - 1, P["granules"]
    fe = P["frame_bytes"] // P["storage"].element_size()
    g = P["gen"]
    B = 3
    x = torch.randn(B, C, generator=g)
    weight = torch.randn(C, 1, W, generator=g) * 0.3
    reads, rgran = torch.tensor([0, 3, 1]), torch.tensor([1, 0, 1])
    writes, wgran = torch.tensor([2, 1, 3]), torch.tensor([1, 1, 0])
    works = torch.tensor([0, 2, 1])
    # the plain pool of (slot, granule) windows that the identity conv table lays out
    base = P["slots"] * P["fps"] + P["slots"]
    before = P["storage"].clone()
    block = before[base:].reshape(P["slots"] * G, -1)[:, :P["layers"] * C * S].reshape(P["slots"] * G, P["layers"], C, S)
    plain = block.clone()
    y_ref = gdn.conv_decode(x, weight, plain, 1, reads * G + rgran, writes * G + wgran)
    y = fr.conv_decode_logstate(x, weight, P["storage"], P["conv"], P["frame_bytes"], 1, reads, rgran, writes, wgran,
                                works)
    torch.testing.assert_close(y, y_ref, rtol=0, atol=0)
    after = P["storage"][base:].reshape(P["slots"] * G, -1)[:, :P["layers"] * C * S].reshape(P["slots"] * G,
                                                                                             P["layers"], C, S)
    for b in range(B):
        torch.testing.assert_close(after[int(writes[b]) * G + int(wgran[b]), 1], plain[int(writes[b]) * G + int(wgran[b]), 1],
                                   rtol=0, atol=0)
        torch.testing.assert_close(after[int(works[b]) * G, 1], plain[int(writes[b]) * G + int(wgran[b]), 1],
                                   rtol=0, atol=0)
    assert torch.equal(P["storage"][:base], before[:base])


def _raw_step(g, B, H, HV, dk, dv):
    q = torch.randn(B, 1, H, dk, generator=g)
    k = torch.randn(B, 1, H, dk, generator=g)
    v = torch.randn(B, 1, HV, dv, generator=g) * 0.5
    a = torch.randn(B, 1, HV, generator=g)
    bt = torch.randn(B, 1, HV, generator=g)
    return q, k, v, a, bt


def test_eager_logstate_step_equals_slotted_decode():
    P = _decode_pool(12)
    g = P["gen"]
    B, H, HV, dk, dv = 2, P["H"], P["HV"], P["dk"], P["dv"]
    A_log, dt_bias = torch.randn(HV, generator=g) * 0.3, torch.randn(HV, generator=g) * 0.3
    q, k, v, a, bt = _raw_step(g, B, H, HV, dk, dv)
    works, logs = torch.tensor([1, 3]), torch.tensor([0, 2])
    payload = P["storage"][:P["slots"] * P["fps"]].clone()
    pool = _as_pool(payload, P["slots"], P["layers"], HV, dk, dv, P["head_bytes"], 4).contiguous()
    o_ref = gdn.fused_recurrent_to_slots(q, k, v, a, bt, A_log, dt_bias, pool, works, works, 1)
    o = fr.fused_recurrent_to_logstate(q, k, v, a, bt, A_log, dt_bias, P["storage"], P["payload"], P["decay"],
                                       P["frame_bytes"], P["head_bytes"], P["record"], works, logs,
                                       torch.tensor([5, 9]), torch.tensor([0, 0]), layer=1, layers=P["layers"],
                                       granularity=8, page_size=P["page"], eager=True)
    torch.testing.assert_close(o, o_ref, rtol=0, atol=0)
    got = fr.read_frame_states(P["storage"], P["payload"], works, 1, HV, dk, dv, P["frame_bytes"], P["head_bytes"])
    torch.testing.assert_close(got, pool[works, 1], rtol=0, atol=0)


def test_replayed_logstate_decode_equals_eager_decode():
    """The replay form (state written every 16 tokens, the tokens since
    rebuilt from the log) equals the eager recurrence over 40 steps: outputs,
    and the work states once both have written them (after step 31)."""
    T = 40
    runs = {}
    for eager in (True, False):
        P = _decode_pool(13, page=64)
        g = torch.Generator().manual_seed(14)
        B, H, HV, dk, dv = 2, P["H"], P["HV"], P["dk"], P["dv"]
        A_log, dt_bias = torch.randn(HV, generator=g) * 0.3, torch.randn(HV, generator=g) * 0.3
        works, logs = torch.tensor([1, 3]), torch.tensor([0, 2])
        outs, mid = [], None
        for t in range(T):
            q, k, v, a, bt = _raw_step(g, B, H, HV, dk, dv)
            counts = torch.tensor([0, 0]) if eager else torch.tensor([t % 16] * B)
            outs.append(fr.fused_recurrent_to_logstate(q, k, v, a, bt, A_log, dt_bias, P["storage"], P["payload"],
                                                       P["decay"], P["frame_bytes"], P["head_bytes"], P["record"],
                                                       works, logs, torch.tensor([t, t]), counts, layer=1,
                                                       layers=P["layers"], granularity=8, page_size=P["page"],
                                                       eager=eager))
            if t == 31:
                mid = fr.read_frame_states(P["storage"], P["payload"], works, 1, HV, dk, dv, P["frame_bytes"],
                                           P["head_bytes"])
        runs[eager] = (torch.cat(outs, 1), mid)
    torch.testing.assert_close(runs[False][0], runs[True][0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(runs[False][1], runs[True][1], rtol=1e-5, atol=1e-5)


def test_logstate_prefill_equals_the_plain_pipeline():
    """Identity tables: the LogState prefill's output, work-slot states and
    conv windows equal the plain pipeline (packed conv from the same history,
    prepare, the chunked rule at the same granularity into a plain pool)."""
    H, HV, dk, dv, W = 2, 4, 8, 8, 4
    C = 2 * H * dk + HV * dv
    P = _decode_pool(15, dtype=torch.float32, page=32, conv_dim=C, H=H, HV=HV, dk=dk, dv=dv, W=W)
    g = P["gen"]
    layers, G, S, gran = P["layers"], P["granules"], W - 1, 16
    lengths, cu = [21, 9], [0, 21, 30]
    T = cu[-1]
    mixed = torch.randn(T, C, generator=g)
    weight = torch.randn(C, 1, W, generator=g) * 0.3
    gate, beta = torch.randn(T, HV, generator=g), torch.randn(T, HV, generator=g)
    A_log, dt_bias = torch.randn(HV, generator=g) * 0.3, torch.randn(HV, generator=g) * 0.3
    works = torch.tensor([1, 3])
    conv_token = torch.full((T,), -1)
    conv_token[15], conv_token[26] = 0, 2
    conv_gran = torch.zeros(T, dtype=torch.int64)
    conv_gran[15] = 1
    chunk_writes = torch.full((sum(-(-n // gran) for n in lengths),), -1)
    logs = torch.tensor([0] * 21 + [2] * 9)
    offsets = torch.tensor(list(range(21)) + list(range(9)))
    storage = P["storage"]
    history = fr.read_conv_windows(storage, P["conv"], P["frame_bytes"], works, [0, 0], 1, C, S)
    y, win = gdn.packed_causal_conv1d(mixed, weight, history, cu, window_rows=[15, 26, 20, 29])
    q, k, v = gdn.split_qkv(y[None], H, dk, HV, dv)
    q, k, v, gg, bb = gdn.prepare_gdn(q, k, v, gate[None], beta[None], A_log, dt_bias)
    pool = _as_pool(storage[:P["slots"] * P["fps"]].clone(), P["slots"], layers, HV, dk, dv, P["head_bytes"],
                    4).contiguous()
    o_ref, _ = gdn.chunk_gated_delta_rule_to_cache(q, k, v, gg, bb, pool, works, chunk_writes, cu, layer=1,
                                                   final_write_slots=works, chunk_size=gran)
    o = fr.forward_prefill_logstate(mixed, gate, beta, weight, A_log, dt_bias, storage, P["payload"], P["decay"],
                                    P["conv"], P["frame_bytes"], P["head_bytes"], P["record"], layer=1,
                                    layers=layers, granularity=gran, page_size=P["page"], cu_seqlens=cu,
                                    work_slots=works, conv_read_slots=works, conv_read_granules=[0, 0],
                                    conv_token_slots=conv_token, conv_token_granules=conv_gran,
                                    chunk_write_slots=chunk_writes, log_write_slots=logs, token_offsets=offsets,
                                    num_k_heads=H, head_k_dim=dk, num_v_heads=HV, head_v_dim=dv)
    torch.testing.assert_close(o, o_ref[0], rtol=0, atol=0)
    got = fr.read_frame_states(storage, P["payload"], works, 1, HV, dk, dv, P["frame_bytes"], P["head_bytes"])
    torch.testing.assert_close(got, pool[works, 1], rtol=0, atol=0)
    # windows: token 15 -> (slot 0, granule 1), token 26 -> (2, 0), each last token -> its work slot's granule 0
    base = P["slots"] * P["fps"] + P["slots"]
    after = storage[base:].reshape(P["slots"] * G, -1)[:, :layers * C * S].reshape(P["slots"] * G, layers, C, S)
    for (slot, gr), w in zip([(0, 1), (2, 0), (1, 0), (3, 0)], win):
        torch.testing.assert_close(after[slot * G + gr, 1], w, rtol=0, atol=0)


# ---------------------------------------------------------------- LogState construction

def _decoded_log(seed, T=21, eager=True):
    """T eager LogState decode steps of one sequence (work slot 1, log slot
    0, layer 1) on an fp32 pool; the work state before them is copied to
    slot 2 first.  Returns the pool and the work state after the steps."""
    P = _decode_pool(seed, page=32)
    g = P["gen"]
    H, HV, dk, dv = P["H"], P["HV"], P["dk"], P["dv"]
    A_log, dt_bias = torch.randn(HV, generator=g) * 0.3, torch.randn(HV, generator=g) * 0.3
    fr.copy_states(P["storage"], P["payload"], P["frame_bytes"], P["head_bytes"], [1], [2], layers=P["layers"],
                   HV=HV, dk=dk, dv=dv)
    for t in range(T):
        q, k, v, a, bt = _raw_step(g, 1, H, HV, dk, dv)
        fr.fused_recurrent_to_logstate(q, k, v, a, bt, A_log, dt_bias, P["storage"], P["payload"], P["decay"],
                                       P["frame_bytes"], P["head_bytes"], P["record"], torch.tensor([1]),
                                       torch.tensor([0]), torch.tensor([t]), torch.tensor([0]), layer=1,
                                       layers=P["layers"], granularity=8, page_size=P["page"], eager=eager)
    final = fr.read_frame_states(P["storage"], P["payload"], [1], 1, HV, dk, dv, P["frame_bytes"], P["head_bytes"])
    return P, final


def _restore(P, chains):
    fr.restore_log_state_chains(P["storage"], P["payload"], P["decay"], P["frame_bytes"], P["head_bytes"], P["record"],
                                chains, layers=P["layers"], HV=P["HV"], key_heads=P["H"], dk=P["dk"], dv=P["dv"],
                                granularity=8, page_size=P["page"])
    return fr.read_frame_states(P["storage"], P["payload"], [3], 1, P["HV"], P["dk"], P["dv"], P["frame_bytes"],
                                P["head_bytes"])


@pytest.mark.parametrize("segments", [[(0, 0, 21)], [(0, 0, 7), (0, 7, 21)], [(0, 0, 8), (0, 8, 9), (0, 9, 21)]])
def test_restore_replays_the_decode(segments):
    """The state rebuilt from the copied base and the logged tokens (v' rows,
    keys, gates written by 21 eager decode steps) equals the state the decode
    left in the work slot, however the tokens split into segments."""
    P, final = _decoded_log(16)
    got = _restore(P, [(2, segments, 3)])
    torch.testing.assert_close(got, final, rtol=1e-5, atol=1e-5)


def test_restore_chains_compose_and_zero_base():
    """Restoring the first 10 tokens into slot 3 and then the rest from slot
    3 equals one restore; a None base equals a zeroed base slot."""
    P, final = _decoded_log(17)
    _restore(P, [(2, [(0, 0, 10)], 3)])
    got = _restore(P, [(3, [(0, 10, 21)], 3)])
    torch.testing.assert_close(got, final, rtol=1e-5, atol=1e-5)
    zero = torch.zeros(1, P["HV"], P["dk"], P["dv"])
    for layer in range(P["layers"]):
        fr.write_frame_states(P["storage"], P["payload"], [2], layer, zero, P["frame_bytes"], P["head_bytes"])
    a = _restore(P, [(2, [(0, 3, 21)], 3)])
    b = _restore(P, [(None, [(0, 3, 21)], 3)])
    assert torch.equal(a, b) and a.abs().sum() > 0


def test_restore_rounds_scaled_values_to_the_storage_dtype():
    """A bf16 pool: the one-token restore is e^g S + k round(v') exactly (the
    suffix of the last token is e^0), and a two-token restore rounds
    e^{g_2} v'_1 to bf16 before the product."""
    P = _decode_pool(18, dtype=torch.bfloat16, page=32)
    HV, dk, dv, H = P["HV"], P["dk"], P["dv"], P["H"]
    g_bytes = P["storage"].view(torch.uint8).view(-1)
    fr_, ri = int(P["decay"][0, 0]), int(P["decay"][0, 1])
    base = fr_ * P["frame_bytes"] + ri * P["record"]
    gates = -torch.rand(P["layers"] * P["page"] * HV, generator=P["gen"]) * 0.5
    g_bytes[base:base + 4 * gates.numel()] = gates.view(torch.uint8)
    s0 = fr.read_frame_states(P["storage"], P["payload"], [2], 1, HV, dk, dv, P["frame_bytes"], P["head_bytes"])[0]
    gl, keys, vals = fr.read_log_segment(P["storage"], P["payload"], P["decay"], P["frame_bytes"], P["record"], 0, 4, 6,
                                         layer=1, layers=P["layers"], granularity=8, page_size=P["page"], key_heads=H,
                                         HV=HV, dk=dk, dv=dv)
    got = _restore(P, [(2, [(0, 4, 6)], 3)])[0].float()
    total = gl[0] + gl[1]
    scaled1 = (vals[0].float() * torch.exp(total - gl[0])[:, None]).to(torch.bfloat16).float()
    want = (s0.float() * torch.exp(total)[:, None, None] + keys[0].float()[:, :, None] * scaled1[:, None, :]
            + keys[1].float()[:, :, None] * vals[1].float()[:, None, :])
    torch.testing.assert_close(got, want.to(torch.bfloat16).float(), rtol=0, atol=0)


def test_copy_states_moves_every_layer_and_nothing_else():
    P = _decode_pool(19)
    before = P["storage"].clone()
    fr.copy_states(P["storage"], P["payload"], P["frame_bytes"], P["head_bytes"], [3, 0], [1, 2], layers=P["layers"],
                   HV=P["HV"], dk=P["dk"], dv=P["dv"])
    args = (P["HV"], P["dk"], P["dv"], P["frame_bytes"], P["head_bytes"])
    for layer in range(P["layers"]):
        for src, dst in [(3, 1), (0, 2)]:
            assert torch.equal(fr.read_frame_states(P["storage"], P["payload"], [dst], layer, *args),
                               fr.read_frame_states(before, P["payload"], [src], layer, *args))
    mask = torch.ones(P["storage"].numel(), dtype=torch.bool)
    for layer in range(P["layers"]):
        mask[fr.frame_state_index(P["payload"], [1, 2], layer, P["HV"], P["dk"], P["dv"], 4, P["frame_bytes"],
                                  P["head_bytes"]).reshape(-1)] = False
    assert torch.equal(P["storage"].reshape(-1)[mask], before.reshape(-1)[mask])


def test_conv_store_and_copy_on_the_identity_table():
    """Identity conv tables: store_conv writes layer l of the reshaped
    [slot, granule, layer, C, S] block, copy_conv_snapshots copies whole
    blocks, and nothing else changes."""
    P = _decode_pool(20)
    C, S, G, L = P["conv_dim"], P["W"] - 1, P["granules"], P["layers"]
    base = P["slots"] * P["fps"] + P["slots"]
    g = P["gen"]

    def block(storage):
        return storage[base:].reshape(P["slots"] * G, -1)[:, :L * C * S].reshape(P["slots"], G, L, C, S)

    before = P["storage"].clone()
    values = torch.randn(3, C, S, generator=g)
    fr.store_conv(P["storage"], P["conv"], P["frame_bytes"], [2, -1, 0], [1, 0, 0], 1, values)
    want = block(before).clone()
    want[2, 1, 1], want[0, 0, 1] = values[0], values[2]
    assert torch.equal(block(P["storage"]), want)
    fr.copy_conv_snapshots(P["storage"], P["conv"], P["frame_bytes"], [2, 1], [1, 0], [3, -1], [0, 1], layers=L, C=C,
                           S=S)
    want[3, 0] = want[2, 1]
    assert torch.equal(block(P["storage"]), want)
    assert torch.equal(P["storage"][:base], before[:base])
