"""GPU parity of the LogState pieces of the chunked prefill: checkpoint
granularities 16 and 32 (``chunk_size`` of ``chunk_gated_delta_rule_to_cache``,
``vendor/fla/chunk_delta_h.py:89-139,226-284`` with BT = granularity) and the
frame-table state addressing (``kernel/linear_attention/layout.py:11-26``)
and the token log (``state_io.py:83-126``, ``layout.py:29-80``), against the
CPU oracle (``oracle/gdn.py``, ``oracle/frames.py``).
``tests/kernel/test_logstate.py:86-160`` (fragmented frame addresses,
granularities 16/32/64) is the model."""

import pytest
import torch
import torch.nn.functional as F

from oracle import frames as ofr
from oracle import gdn as ref
from tests.gpu_util import DEV, assert_bf16_close, assert_state_close, gen

pytestmark = pytest.mark.gpu

LENGTHS = [1, 17, 64, 65, 130, 300, 31, 32, 33]


def _inputs(g, T, H, HV, dk, dv):
    q = F.normalize(torch.randn(T, H, dk, generator=g), dim=-1).to(torch.bfloat16)
    k = F.normalize(torch.randn(T, H, dk, generator=g), dim=-1).to(torch.bfloat16)
    v = torch.randn(T, HV, dv, generator=g).to(torch.bfloat16)
    gg = -torch.rand(T, HV, generator=g) * 0.3
    beta = torch.sigmoid(torch.randn(T, HV, generator=g))
    return q, k, v, gg, beta


def _cu(lengths):
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return cu


def assert_state16_close(actual, expected, atol=1e-3):
    """16-bit stored states: the fp32 bar plus one rounding step of the
    stored value (2^-7 relative for bf16), since kernel and oracle each round
    their fp32 state independently."""
    a, e = actual.float().cpu(), expected.float().cpu()
    err = (a - e).abs()
    bad = err > atol + e.abs() * 2.0 ** -7
    assert not bad.any(), f"{int(bad.sum())} states out of tolerance; max err {float(err.max()):.3e}"


def _report(name, a, b):
    err = (a.float().cpu() - b.float().cpu()).abs()
    print(f"{name}: max-abs {float(err.max()):.3e}", flush=True)


@pytest.mark.parametrize("chunk_size", [32, 16])
def test_granularity_checkpoints_plain_pool(chunk_size):
    from logssms_amd.kernel.linear_attention import ChunkStateIO, chunk_gated_delta_rule_to_cache
    g = gen(31 + chunk_size)
    H, HV, dk, dv = 2, 4, 128, 128
    cu = _cu(LENGTHS)
    T, N = cu[-1], len(LENGTHS)
    q, k, v, gg, beta = _inputs(g, T, H, HV, dk, dv)
    n_int = sum(-(-n // chunk_size) for n in LENGTHS)
    slots = 2 * N + n_int + 1
    storage = torch.zeros(slots, 2, HV, dk, dv)
    storage[:N, 1] = torch.randn(N, HV, dk, dv, generator=g) * 0.1
    reads = torch.tensor([0, -1, 2, 3, -1, 5, 6, -1, 8])
    writes = torch.arange(2 * N, 2 * N + n_int)
    writes[3] = -1
    finals = torch.arange(N, 2 * N)
    expected = storage.clone()
    o_ref, vn_ref = ref.chunk_gated_delta_rule_to_cache(q[None].float(), k[None].float(), v[None].float(), gg[None],
                                                        beta[None], expected, reads, writes, cu, layer=1,
                                                        final_write_slots=finals, chunk_size=chunk_size)
    dstore = storage.to(DEV)
    io = ChunkStateIO(dstore, reads.to(DEV), writes.to(DEV), final_write_slots=finals.to(DEV), layer=1,
                      granularity=chunk_size)
    print(f"granularity {chunk_size}: {N} sequences, {n_int} intervals", flush=True)
    o, vn = chunk_gated_delta_rule_to_cache(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), gg[None].to(DEV),
                                            beta[None].to(DEV), io, torch.tensor(cu, device=DEV),
                                            chunk_size=chunk_size)
    torch.cuda.synchronize()
    _report("out", o[0], o_ref[0])
    _report("checkpoints", dstore[2 * N:, 1], expected[2 * N:, 1])
    assert_bf16_close(o[0], o_ref[0])
    assert_bf16_close(vn[0], vn_ref[0], rel=2e-2, atol=2e-2)
    assert_state_close(dstore[N:, 1], expected[N:, 1])
    host = dstore.cpu()
    assert torch.equal(host[:, 0], storage[:, 0])
    assert torch.equal(host[:N], expected[:N])
    assert torch.equal(host[2 * N + 3], storage[2 * N + 3])


def _frame_setup(g, slots, layers, HV, dk, dv, frame_bytes, head_bytes, spare=7, min_fps=1):
    """A fragmented frame storage: every slot's frames (at least min_fps)
    drawn at random from a shuffled pool with spare frames."""
    fps = max(min_fps, -(-layers * HV * head_bytes // frame_bytes))
    num_frames = slots * fps + spare
    order = torch.randperm(num_frames, generator=g)[:slots * fps]
    frames = order.reshape(slots, fps).to(torch.int32)
    storage = (torch.randn(num_frames, frame_bytes // 2, generator=g) * 0.1).to(torch.bfloat16)
    return storage, frames


# (dk, dv, frame_bytes, head_bytes): two heads per frame; a head over two
# frames; a padded head (128 x 192 bf16 = 48 KiB in a 64 KiB payload);
# d_v = 32 (a 32-column workgroup slice): 32 x 32 heads inside a frame, and
# 128 x 32 heads over two frames
FRAME_CASES = [(128, 128, 65536, 32768), (128, 128, 16384, 32768), (128, 192, 131072, 65536), (32, 32, 16384, 2048),
               (128, 32, 4096, 8192)]


@pytest.mark.parametrize("chunk_size", [32, 16, 64])
@pytest.mark.parametrize("case", FRAME_CASES)
def test_frame_table_states(case, chunk_size):
    from logssms_amd.kernel.linear_attention import ChunkStateIO, chunk_gated_delta_rule_to_cache
    dk, dv, frame_bytes, head_bytes = case
    g = gen(47 + chunk_size + dv)
    H, HV, layers, layer = 2, 4, 2, 1
    lengths = [100, 37, 64, 1, 130]
    cu = _cu(lengths)
    T, N = cu[-1], len(lengths)
    q, k, v, gg, beta = _inputs(g, T, H, HV, dk, dv)
    n_int = sum(-(-n // chunk_size) for n in lengths)
    slots = 2 * N + n_int
    storage, frames = _frame_setup(g, slots, layers, HV, dk, dv, frame_bytes, head_bytes)
    reads = torch.tensor([0, -1, 2, 3, 4])
    writes = torch.arange(2 * N, 2 * N + n_int)
    writes[1] = -1
    finals = torch.arange(N, 2 * N)
    expected = storage.clone()
    o_ref, _ = ofr.chunk_gated_delta_rule_to_frames(q[None].float(), k[None].float(), v[None].float(), gg[None],
                                                    beta[None], expected, frames, frame_bytes, head_bytes, reads,
                                                    writes, cu, layer=layer, final_write_slots=finals,
                                                    chunk_size=chunk_size)
    dstore = storage.to(DEV)
    io = ChunkStateIO(dstore, reads.to(DEV), writes.to(DEV), final_write_slots=finals.to(DEV),
                      payload_frames=frames.to(DEV), frame_bytes=frame_bytes, head_payload_bytes=head_bytes,
                      layer=layer, num_layers=layers, granularity=chunk_size)
    print(f"frames dk {dk} dv {dv} frame {frame_bytes} head {head_bytes} granularity {chunk_size}", flush=True)
    o, _ = chunk_gated_delta_rule_to_cache(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), gg[None].to(DEV),
                                           beta[None].to(DEV), io, torch.tensor(cu, device=DEV),
                                           chunk_size=chunk_size)
    torch.cuda.synchronize()
    host = dstore.cpu()
    written = [s for s in range(N, slots) if s != 2 * N + 1]
    got = ofr.read_frame_states(host, frames, written, layer, HV, dk, dv, frame_bytes, head_bytes)
    want = ofr.read_frame_states(expected, frames, written, layer, HV, dk, dv, frame_bytes, head_bytes)
    _report("out", o[0], o_ref[0])
    _report("states", got, want)
    assert_bf16_close(o[0], o_ref[0])
    assert_state16_close(got, want)
    # every byte outside the written states is as the oracle left it (= as before)
    mask = torch.ones(host.numel(), dtype=torch.bool)
    idx = ofr.frame_state_index(frames, written, layer, HV, dk, dv, 2, frame_bytes, head_bytes)
    mask[idx.reshape(-1)] = False
    assert torch.equal(host.reshape(-1)[mask], storage.reshape(-1)[mask])


# (dk, dv, frame_bytes, head_bytes)
LOG_SHAPES = [(128, 128, 65536, 32768), (32, 32, 16384, 2048)]


@pytest.mark.parametrize("shape", LOG_SHAPES)
@pytest.mark.parametrize("direct", [False, True])
def test_chunk_token_log(direct, shape):
    """ChunkLogIO: each logged token's v' rows, key rows and gate land in its
    log slot (state_io.py:83-126); keys and gates bit-exact, v' rows to the
    output tolerance, every other byte untouched.  direct: no v_new asked
    for, so the chunk kernel writes the v' rows into the log itself."""
    from logssms_amd.kernel.linear_attention import ChunkLogIO, ChunkStateIO, chunk_gated_delta_rule_to_cache
    g = gen(71)
    dk, dv, frame_bytes, head_bytes = shape
    H, HV, layers, layer, gran, page = 2, 4, 2, 1, 32, 64
    lengths = [100, 37]
    cu = _cu(lengths)
    T, N = cu[-1], len(lengths)
    q, k, v, gg, beta = _inputs(g, T, H, HV, dk, dv)
    n_int = sum(-(-n // gran) for n in lengths)
    state_slots = 2 * N + n_int
    # log slots: one per (sequence, page), after the state slots
    log_slot, pos = [], []
    next_slot = state_slots
    for n, length in enumerate(lengths):
        for t in range(length):
            if t % page == 0:
                cur = next_slot
                next_slot += 1
            log_slot.append(cur)
            pos.append(t % page)
    log_slot[5] = -1  # one token without a log
    slots = next_slot
    log_bytes = 2 * page * layers * (H * dk + HV * dv)  # a slot's frames also hold its log
    storage, frames = _frame_setup(g, slots, layers, HV, dk, dv, frame_bytes, head_bytes, spare=2,
                                   min_fps=-(-log_bytes // frame_bytes))
    record = 4 * layers * page * HV
    # decay records: 32 to a frame, in extra frames appended to the storage
    n_dec = -(-slots // (frame_bytes // record))
    storage = torch.cat([storage, (torch.randn(n_dec, frame_bytes // 2, generator=g) * 0.1).to(torch.bfloat16)])
    decay = torch.tensor([[storage.shape[0] - n_dec + s // (frame_bytes // record), s % (frame_bytes // record)]
                          for s in range(slots)], dtype=torch.int32)
    reads = torch.tensor([0, 1])
    writes = torch.arange(2 * N, 2 * N + n_int)
    finals = torch.arange(N, 2 * N)
    log_slots = torch.tensor(log_slot)
    offsets = torch.tensor(pos)

    expected = storage.clone()
    o_ref, vn_ref = ofr.chunk_gated_delta_rule_to_frames(q[None].float(), k[None].float(), v[None].float(), gg[None],
                                                         beta[None], expected, frames, frame_bytes, head_bytes, reads,
                                                         writes, cu, layer=layer, final_write_slots=finals,
                                                         chunk_size=gran)
    ofr.store_chunk_log(expected, frames, frame_bytes, log_slots, offsets, vn_ref[0].to(torch.bfloat16), k, gg,
                        decay, record, layer=layer, layers=layers, granularity=gran, page_size=page, key_heads=H)

    dstore = storage.to(DEV)
    io = ChunkStateIO(dstore, reads.to(DEV), writes.to(DEV), final_write_slots=finals.to(DEV),
                      payload_frames=frames.to(DEV), frame_bytes=frame_bytes, head_payload_bytes=head_bytes,
                      layer=layer, num_layers=layers, granularity=gran)
    log = ChunkLogIO(log_slots.to(DEV), offsets.to(DEV), decay.to(DEV), gg[None].to(DEV), page, record, H)
    print(f"token log: {T} tokens, {slots - state_slots} log slots", flush=True)
    o, _ = chunk_gated_delta_rule_to_cache(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), gg[None].to(DEV),
                                           beta[None].to(DEV), io, torch.tensor(cu, device=DEV), chunk_size=gran,
                                           log_io=log, return_v_new=not direct)
    torch.cuda.synchronize()
    host = dstore.cpu()
    assert_bf16_close(o[0], o_ref[0])
    # value rows of the log: output tolerance
    logged = [t for t in range(T) if log_slot[t] >= 0]
    vidx = torch.cat([ofr.log_element_index(frames, [log_slot[t]] * HV, [pos[t]] * HV, range(HV), range(dv), layer,
                                            layers, gran, H, HV, dk, dv, frame_bytes, True) for t in logged])
    assert_bf16_close(host.reshape(-1)[vidx], expected.reshape(-1)[vidx])
    # states
    written = list(range(N, state_slots))
    sidx = ofr.frame_state_index(frames, written, layer, HV, dk, dv, 2, frame_bytes, head_bytes)
    assert_state16_close(host.reshape(-1)[sidx], expected.reshape(-1)[sidx])
    # keys, gates and every untouched byte: bit-exact
    mask = torch.ones(host.numel(), dtype=torch.bool)
    mask[vidx.reshape(-1)] = False
    mask[sidx.reshape(-1)] = False
    a, e = host.view(torch.int16).reshape(-1), expected.view(torch.int16).reshape(-1)
    bad = (a != e) & mask
    assert not bad.any(), f"{int(bad.sum())} bytes differ outside the v' rows and states"


def _decode_pool(g, slots, H, HV, dk, dv, layers, page, gran, conv_dim, W, frame_bytes, head_bytes):
    """A fragmented LogState frame storage: payload frames (states and logs),
    one decay record per slot, conv snapshots per (slot, granule)."""
    from types import SimpleNamespace
    fps = max(-(-layers * HV * head_bytes // frame_bytes), -(-2 * page * layers * (H * dk + HV * dv) // frame_bytes))
    record = 4 * layers * page * HV
    per_frame = frame_bytes // record
    n_dec = -(-slots // per_frame)
    granules = page // gran
    conv_bytes = 2 * layers * conv_dim * (W - 1)
    cf = -(-conv_bytes // frame_bytes)
    total = slots * fps + n_dec + slots * granules * cf + 3
    order = torch.randperm(total, generator=g)
    payload = order[:slots * fps].reshape(slots, fps).to(torch.int32)
    dec = order[slots * fps:slots * fps + n_dec]
    decay = torch.tensor([[int(dec[s // per_frame]), s % per_frame] for s in range(slots)], dtype=torch.int32)
    conv = order[slots * fps + n_dec:slots * fps + n_dec + slots * granules * cf].reshape(slots, granules, cf)
    storage = (torch.randn(total, frame_bytes // 2, generator=g) * 0.05).to(torch.bfloat16)
    layout = SimpleNamespace(head_k_dim=dk, head_v_dim=dv, num_value_heads=HV, num_key_heads=H,
                             num_linear_layers=layers, granularity=gran, log_decay_bytes=record, num_granules=granules)
    pool = SimpleNamespace(storage=None, payload_frame_table=None, decay_frame_table=None,
                           conv_frame_table=None, frame_bytes=frame_bytes, head_payload_bytes=head_bytes,
                           page_size=page, layout=layout, dtype=torch.bfloat16)
    return storage, payload, decay, conv.to(torch.int32), record, pool


# (eager, dk, dv): both modes at Qwen3-Next shape, the replay form at the other head shapes
DECODE_CASES = [(False, 128, 128), (True, 128, 128), (False, 64, 64), (False, 32, 32), (False, 128, 64),
                (True, 64, 128)]


@pytest.mark.parametrize("case", DECODE_CASES)
def test_logstate_decode_steps(case):
    """34 LogState decode steps (conv through the conv frame table, the
    recurrence from the work state plus the replayed log) against the oracle:
    outputs every step, then the work states, the log rows, the gates and the
    conv windows (fused_recurrent.py:292-394, gdn_replay.py:17-148,
    conv_decode.py:293-352)."""
    eager, dk, dv = case
    _decode_steps(eager, dk, dv, seed=91 + int(eager) + dk + 3 * dv)


@pytest.mark.parametrize("B", [64, 128, 256])
def test_logstate_decode_wide_batches(B):
    """64, 128 and 256 sequences at 16 key / 32 value heads, where a decode
    block takes 2, 4 and 8 value heads of its sequence in turn (its loading
    wave fetching the next head while the current one computes): 18 steps
    against the oracle, with a write-back at position 15 and replays of up to
    15 logged tokens."""
    _decode_steps(False, 64, 64, seed=7 + B, B=B, H=16, HV=32, layers=1, layer=0, page=32, gran=16, T=18)


@pytest.mark.parametrize("eager,dk,frame_bytes", [(False, 64, 49152), (False, 128, 16384), (True, 128, 16384)])
def test_logstate_decode_frame_shapes(eager, dk, frame_bytes):
    """Frames of a size that is not a power of two (49152 bytes: frame
    arithmetic by division) and frames smaller than a head (a 128 x 128 bf16
    head over two 16 KiB frames: a frame lookup per state row, for the loads
    and for the write-backs): LogState decode steps against the oracle."""
    _decode_steps(eager, dk, dk, seed=301 + dk + frame_bytes // 4096 + int(eager), frame_bytes=frame_bytes, T=20)


def _decode_steps(eager, dk, dv, seed, B=3, H=2, HV=4, layers=2, layer=1, page=64, gran=16, T=34, frame_bytes=65536):
    from types import SimpleNamespace
    from logssms_amd.kernel.linear_attention import conv_decode, fused_recurrent_gated_delta_rule_to_logstate
    g = gen(seed)
    W = 4
    conv_dim = 2 * H * dk + HV * dv
    head_bytes = dk * dv * 2
    slots = 2 * B
    storage, payload, decay, conv, record, pool = _decode_pool(g, slots, H, HV, dk, dv, layers, page, gran, conv_dim,
                                                               W, frame_bytes, head_bytes)
    works, logs = torch.arange(0, 2 * B, 2), torch.arange(1, 2 * B, 2)
    weight = (torch.randn(conv_dim, 1, W, generator=g) * 0.3).to(torch.bfloat16)
    A_log, dt_bias = torch.randn(HV, generator=g) * 0.3, torch.randn(HV, generator=g) * 0.3
    cfg = SimpleNamespace(state_len=W - 1, conv_dim=conv_dim, num_k_heads=H, head_k_dim=dk, num_v_heads=HV,
                          head_v_dim=dv, key_dim=H * dk, layer_idx=layer)
    expected = storage.clone()
    dev_u8 = storage.view(torch.uint8).to(DEV)
    pool.storage = dev_u8
    pool.payload_frame_table, pool.decay_frame_table, pool.conv_frame_table = payload.to(DEV), decay.to(DEV), conv.to(DEV)
    print(f"LogState decode, eager={eager} dk={dk} dv={dv} HV={HV}: {T} steps x {B} sequences", flush=True)
    for t in range(T):
        mixed = (torch.randn(B, conv_dim, generator=g)).to(torch.bfloat16)
        a, bt = torch.randn(B, HV, generator=g), torch.randn(B, HV, generator=g)
        pos = torch.full((B,), t)
        counts = torch.zeros(B, dtype=torch.int64) if eager else pos % 16
        zeros = torch.zeros(B, dtype=torch.int64)
        # oracle
        y = ofr.conv_decode_logstate(mixed, weight, expected, conv, frame_bytes, layer, works, zeros, logs,
                                     pos // gran, works)
        q, k, v = (y[:, :H * dk].reshape(B, 1, H, dk), y[:, H * dk:2 * H * dk].reshape(B, 1, H, dk),
                   y[:, 2 * H * dk:].reshape(B, 1, HV, dv))
        o_ref = ofr.fused_recurrent_to_logstate(q, k, v, a[:, None], bt[:, None], A_log, dt_bias, expected, payload,
                                                decay, frame_bytes, head_bytes, record, works, logs, pos, counts,
                                                layer=layer, layers=layers, granularity=gran, page_size=page,
                                                eager=eager)
        # device
        dq, dk_, dvv = conv_decode(mixed.to(DEV), weight.to(DEV), cfg, split_qkv=True, read_slots=works.to(DEV),
                                   write_slots=logs.to(DEV), pool=pool, read_granules=zeros.to(DEV),
                                   write_granules=(pos // gran).to(DEV), work_slots=works.to(DEV))
        o = fused_recurrent_gated_delta_rule_to_logstate(dq, dk_, dvv, a[:, None].to(DEV), bt[:, None].to(DEV),
                                                         A_log.to(DEV), dt_bias.to(DEV), pool, works.to(DEV),
                                                         logs.to(DEV), pos.to(DEV), layer, counts.to(DEV),
                                                         enable_eager_state=eager)
        assert_bf16_close(dq.reshape(B, -1), q.reshape(B, -1))
        assert_bf16_close(o, o_ref)
    torch.cuda.synchronize()
    host = dev_u8.cpu().view(torch.bfloat16).reshape(storage.shape)
    _report("out (last step)", o, o_ref)
    got = ofr.read_frame_states(host, payload, works, layer, HV, dk, dv, frame_bytes, head_bytes)
    want = ofr.read_frame_states(expected, payload, works, layer, HV, dk, dv, frame_bytes, head_bytes)
    _report("work states", got, want)
    assert_state16_close(got, want)
    # log rows (v' to the output bar; keys within two bf16 rounding steps: the
    # conv output the key is normalised from may differ from the oracle's by
    # one step, and the logged key is rounded again), gates, conv windows
    for b in range(B):
        vidx = torch.cat([ofr.log_element_index(payload, [int(logs[b])] * HV, [t] * HV, range(HV), range(dv), layer,
                                                layers, gran, H, HV, dk, dv, frame_bytes, True) for t in range(T)])
        assert_bf16_close(host.reshape(-1)[vidx], expected.reshape(-1)[vidx])
        kidx = torch.cat([ofr.log_element_index(payload, [int(logs[b])] * H, [t] * H, range(H), range(dk), layer,
                                                layers, gran, H, HV, dk, dv, frame_bytes, False) for t in range(T)])
        ka, ke = host.reshape(-1)[kidx].float(), expected.reshape(-1)[kidx].float()
        bad = ~((ka - ke).abs() <= ke.abs() * 2.0 ** -6 + 1e-6)
        if bad.any():
            row, col = bad.nonzero()[0].tolist()
            raise AssertionError(f"sequence {b}: {int(bad.sum())} logged key elements differ, first at token "
                                 f"{row // H}, key head {row % H}, column {col}: {float(ka[row, col])} vs "
                                 f"{float(ke[row, col])}")
    hb, eb = host.view(torch.uint8).reshape(-1), expected.view(torch.uint8).reshape(-1)
    for b in range(B):
        fr_, ri = int(decay[int(logs[b]), 0]), int(decay[int(logs[b]), 1])
        base = fr_ * frame_bytes + ri * record + 4 * (layer * page) * HV
        ga = hb[base:base + 4 * T * HV].view(torch.float32)
        ge = eb[base:base + 4 * T * HV].view(torch.float32)
        torch.testing.assert_close(ga, ge, rtol=1e-5, atol=1e-6)
    fe = frame_bytes // 2
    for slot, gr in [(int(works[b]), 0) for b in range(B)] + [(int(logs[b]), t // gran) for b in range(B)
                                                                for t in (0, T - 1)]:
        idx = ofr.conv_element_index(conv, [slot], [gr], layer, conv_dim, W - 1, fe)
        assert torch.equal(host.reshape(-1)[idx].view(torch.int16), expected.reshape(-1)[idx].view(torch.int16))


@pytest.mark.parametrize("eager", [False, True])
def test_logstate_backend_prefill_then_decode(eager):
    """GatedDeltaLogStateBackend (gdn_logstate.py:18-224): a packed prefill of
    two sequences from their work slots (conv history, initial state), with
    conv snapshots at granule ends, two mid-sequence checkpoints and the token
    log, then 18 decode steps each, replaying the log between write-backs;
    against the oracle's LogState prefill and decode."""
    from types import SimpleNamespace
    from logssms_amd.core import Batch
    from logssms_amd.layers import GatedDeltaLogStateBackend, LogStateLinearAttnMetadata
    from logssms_amd.layers.linear_attention_backend import PackedLinearIndices
    g = gen(101 + int(eager))
    H, HV, dk, dv, layers, layer, page, gran, W = 2, 4, 128, 128, 2, 1, 64, 16, 4
    C = 2 * H * dk + HV * dv
    frame_bytes, head_bytes = 65536, 32768
    slots = 8  # 0, 1 work slots; 2, 3, 4 log pages; 5, 6 checkpoints; 7 spare
    storage, payload, decay, conv, record, pool = _decode_pool(g, slots, H, HV, dk, dv, layers, page, gran, C, W,
                                                               frame_bytes, head_bytes)
    pool.layout.num_key_heads = H
    fe = frame_bytes // 2

    def read_conv(s, gr, lay):
        idx = ofr.conv_element_index(conv, s.cpu(), gr.cpu(), lay, C, W - 1, fe).to(DEV)
        return pool.storage.view(torch.bfloat16).reshape(-1)[idx].view(len(s), C, W - 1)

    pool.read_conv = read_conv
    dev_u8 = storage.view(torch.uint8).to(DEV)
    pool.storage = dev_u8
    pool.payload_frame_table, pool.decay_frame_table, pool.conv_frame_table = payload.to(DEV), decay.to(DEV), conv.to(DEV)
    backend = GatedDeltaLogStateBackend(ctx=SimpleNamespace(linear_state=pool), enable_eager_state=eager)
    cfg = SimpleNamespace(key_dim=H * dk, value_dim=HV * dv, head_k_dim=dk, head_v_dim=dv, layer_idx=layer,
                          state_len=W - 1, conv_dim=C, num_k_heads=H, num_v_heads=HV)
    weight = (torch.randn(C, 1, W, generator=g) * 0.3).to(torch.bfloat16)
    A_log, dt_bias = torch.randn(HV, generator=g) * 0.3, torch.randn(HV, generator=g) * 0.3
    expected = storage.clone()

    # ---- prefill
    lengths = [100, 37]
    cu = [0, 100, 137]
    T = cu[-1]
    works = torch.tensor([0, 1])
    pages = {0: [2, 3], 1: [4]}  # log slot of each page
    log_slots, offsets, tok_slots, tok_gran = [], [], [], []
    for n, length in enumerate(lengths):
        for pos in range(length):
            ls = pages[n][pos // page]
            log_slots.append(ls)
            offsets.append(pos % page)
            end_of_granule = (pos % page) % gran == gran - 1
            tok_slots.append(ls if end_of_granule else -1)
            tok_gran.append((pos % page) // gran)
    n_int = sum(-(-n // gran) for n in lengths)
    chunk_writes = torch.full((n_int,), -1)
    chunk_writes[2], chunk_writes[7 + 1] = 5, 6
    mixed = torch.randn(T, C, generator=g).to(torch.bfloat16)
    gate, beta = torch.randn(T, HV, generator=g).to(torch.bfloat16), torch.randn(T, HV, generator=g).to(torch.bfloat16)
    o_ref = ofr.forward_prefill_logstate(mixed, gate, beta, weight, A_log, dt_bias, expected, payload, decay, conv,
                                         frame_bytes, head_bytes, record, layer=layer, layers=layers,
                                         granularity=gran, page_size=page, cu_seqlens=cu, work_slots=works,
                                         conv_read_slots=works, conv_read_granules=[0, 0],
                                         conv_token_slots=torch.tensor(tok_slots),
                                         conv_token_granules=torch.tensor(tok_gran), chunk_write_slots=chunk_writes,
                                         log_write_slots=torch.tensor(log_slots), token_offsets=torch.tensor(offsets),
                                         num_k_heads=H, head_k_dim=dk, num_v_heads=HV, head_v_dim=dv)
    meta = LogStateLinearAttnMetadata(
        phase="prefill", work_slots=works.to(DEV), log_slots=torch.tensor(log_slots, device=DEV),
        token_offsets=torch.tensor(offsets, device=DEV), conv_read_slots=works.to(DEV),
        conv_read_granules=torch.zeros(2, dtype=torch.int64, device=DEV),
        replay_counts=torch.zeros(2, dtype=torch.int64, device=DEV), cu_seqlens=torch.tensor(cu, device=DEV),
        prefill_indices=PackedLinearIndices.from_lengths(lengths, DEV, gran), chunk_write_slots=chunk_writes.to(DEV),
        log_write_slots=torch.tensor(log_slots, device=DEV), conv_token_slots=torch.tensor(tok_slots, device=DEV),
        conv_token_granules=torch.tensor(tok_gran, device=DEV))
    print(f"LogState backend, eager={eager}: prefill {lengths}", flush=True)
    o = backend.forward(mixed.to(DEV), gate.to(DEV), beta.to(DEV), weight.to(DEV), A_log.to(DEV), dt_bias.to(DEV),
                        cfg, Batch(reqs=[None, None], phase="prefill", linear_attn_metadata=meta))
    torch.cuda.synchronize()
    _report("prefill out", o, o_ref)
    assert_bf16_close(o, o_ref)

    # ---- decode: 18 steps; the replay count is the tokens logged since the last write-back
    pos = torch.tensor(lengths)
    since = [0, 0]
    for step in range(18):
        off = pos % page
        ls = torch.tensor([pages[n][int(pos[n]) // page] for n in range(2)])
        counts = torch.tensor([0, 0]) if eager else torch.tensor(since)
        x = torch.randn(2, C, generator=g).to(torch.bfloat16)
        a, bt = torch.randn(2, HV, generator=g).to(torch.bfloat16), torch.randn(2, HV, generator=g).to(torch.bfloat16)
        y = ofr.conv_decode_logstate(x, weight, expected, conv, frame_bytes, layer, works, torch.zeros(2, dtype=torch.int64),
                                     ls, off // gran, works)
        q, k, v = (y[:, :H * dk].reshape(2, 1, H, dk), y[:, H * dk:2 * H * dk].reshape(2, 1, H, dk),
                   y[:, 2 * H * dk:].reshape(2, 1, HV, dv))
        o_ref = ofr.fused_recurrent_to_logstate(q, k, v, a[:, None], bt[:, None], A_log, dt_bias, expected, payload,
                                                decay, frame_bytes, head_bytes, record, works, ls, off, counts,
                                                layer=layer, layers=layers, granularity=gran, page_size=page,
                                                eager=eager)
        meta = LogStateLinearAttnMetadata(
            phase="decode", work_slots=works.to(DEV), log_slots=ls.to(DEV), token_offsets=off.to(DEV),
            conv_read_slots=works.to(DEV), conv_read_granules=torch.zeros(2, dtype=torch.int64, device=DEV),
            replay_counts=counts.to(DEV))
        o = backend.forward(x.to(DEV), a.to(DEV), bt.to(DEV), weight.to(DEV), A_log.to(DEV), dt_bias.to(DEV), cfg,
                            Batch(reqs=[None, None], phase="decode", linear_attn_metadata=meta))
        assert_bf16_close(o, o_ref[:, 0])
        since = [0 if (int(off[n]) + 1) % 16 == 0 else since[n] + 1 for n in range(2)]
        pos = pos + 1
    torch.cuda.synchronize()
    _report("decode out (last step)", o, o_ref[:, 0])
    host = dev_u8.cpu().view(torch.bfloat16).reshape(storage.shape)
    for name, s in (("work", works.tolist()), ("checkpoints", [5, 6])):
        got = ofr.read_frame_states(host, payload, s, layer, HV, dk, dv, frame_bytes, head_bytes)
        want = ofr.read_frame_states(expected, payload, s, layer, HV, dk, dv, frame_bytes, head_bytes)
        _report(f"{name} states", got, want)
        assert_state16_close(got, want)
    for slot, gr in [(0, 0), (1, 0), (2, 3), (3, 1), (4, 1)]:
        idx = ofr.conv_element_index(conv, [slot], [gr], layer, C, W - 1, fe)
        assert torch.equal(host.reshape(-1)[idx].view(torch.int16), expected.reshape(-1)[idx].view(torch.int16))


# (H, frame_bytes, head_bytes, granularity): state heads inside a frame and
# spanning two frames, one and two key heads
# (H, frame_bytes, head_bytes, granularity, dk, dv[, page]); page 576: chains
# over three 256-token suffix spans, the last one partial
RESTORE_CASES = [(1, 65536, 32768, 16, 128, 128), (2, 16384, 32768, 32, 128, 128), (2, 65536, 32768, 64, 128, 128),
                 (2, 65536, 8192, 32, 64, 64), (1, 65536, 2048, 16, 32, 32), (2, 65536, 16384, 32, 128, 64),
                 (2, 16384, 16384, 32, 64, 128), (2, 65536, 32768, 32, 128, 128, 576)]


@pytest.mark.parametrize("case", RESTORE_CASES)
def test_logstate_store_copy_restore(case):
    """store_log_states, copy_states and restore_log_state_chains
    (kernel/linear_attention/logstate.py:59-128, logstate.cu:11-228,
    logstate_construction.cuh:265-416) on a fragmented frame storage against
    the oracle: the log bytes bit-exact after the stores, the copied states
    bit-exact, the restored states to the state bar (fp32 1e-3 plus one bf16
    rounding); no other byte changes.  Chains: a full page from a base, a None
    base over two segments of two log slots, and a copied base over three
    segments one of which is empty (tests/kernel/test_logstate_granules.py:24-49
    is the model)."""
    from logssms_amd.kernel.linear_attention.logstate import copy_states, restore_log_state_chains, store_log_states
    H, frame_bytes, head_bytes, gran, dk, dv, page = case if len(case) == 7 else case + (64,)
    g = gen(101 + gran + H + dk + dv)
    HV, layers, slots = 4, 2, 7
    storage, payload, decay, conv, record, pool = _decode_pool(g, slots, H, HV, dk, dv, layers, page, gran, 16, 4,
                                                               frame_bytes, head_bytes)
    expected = storage.clone()
    dev_u8 = storage.view(torch.uint8).to(DEV)
    pool.storage = dev_u8
    pool.payload_frame_table, pool.decay_frame_table = payload.to(DEV), decay.to(DEV)
    print(f"store/copy/restore H={H} frame_bytes={frame_bytes} granularity={gran} dk={dk} dv={dv} page={page}",
          flush=True)
    for slot in (1, 3):
        for layer in range(layers):
            heads = H if layer == 0 else HV  # keys per key head, then one row per value head
            keys = F.normalize(torch.randn(page, heads, dk, generator=g), dim=-1).to(torch.bfloat16)
            if heads == HV:
                keys = keys[:, ::HV // H].repeat_interleave(HV // H, 1)
            values = (torch.randn(page, HV, dv, generator=g) * 0.1).to(torch.bfloat16)
            decays = -torch.rand(page, HV, generator=g) * 0.3
            offsets = torch.randperm(page, generator=g)
            token_slots = torch.full((page,), slot)
            token_slots[5] = -1
            ofr.store_chunk_log(expected, payload, frame_bytes, token_slots, offsets, values, keys, decays, decay,
                                record, layer=layer, layers=layers, granularity=gran, page_size=page, key_heads=H)
            store_log_states(pool, token_slots.to(torch.int32).to(DEV), offsets.to(torch.int32).to(DEV),
                             keys.to(DEV), values.to(DEV), decays.to(DEV), layer)
    torch.cuda.synchronize()
    host = dev_u8.cpu().view(torch.bfloat16).reshape(storage.shape)
    assert torch.equal(host.view(torch.int16), expected.view(torch.int16)), "log stores differ"
    copy_states(pool, [0], [5])
    ofr.copy_states(expected, payload, frame_bytes, head_bytes, [0], [5], layers=layers, HV=HV, dk=dk, dv=dv)
    torch.cuda.synchronize()
    host = dev_u8.cpu().view(torch.bfloat16).reshape(storage.shape)
    assert torch.equal(host.view(torch.int16), expected.view(torch.int16)), "copied states differ"
    chains = [(0, [(1, 0, page)], 2), (None, [(1, 5, 40), (3, 0, 17)], 4),
              (5, [(3, 16, page), (1, 63, page), (1, 10, 10)], 6)]
    restore_log_state_chains(pool, chains)
    ofr.restore_log_state_chains(expected, payload, decay, frame_bytes, head_bytes, record, chains, layers=layers,
                                 HV=HV, key_heads=H, dk=dk, dv=dv, granularity=gran, page_size=page)
    torch.cuda.synchronize()
    host = dev_u8.cpu().view(torch.bfloat16).reshape(storage.shape)
    mask = torch.ones(host.numel(), dtype=torch.bool)
    for layer in range(layers):
        got = ofr.read_frame_states(host, payload, [2, 4, 6], layer, HV, dk, dv, frame_bytes, head_bytes)
        want = ofr.read_frame_states(expected, payload, [2, 4, 6], layer, HV, dk, dv, frame_bytes, head_bytes)
        _report(f"restored states, layer {layer}", got, want)
        assert_state16_close(got, want)
        mask[ofr.frame_state_index(payload, [2, 4, 6], layer, HV, dk, dv, 2, frame_bytes, head_bytes).reshape(-1)] = False
    a, e = host.view(torch.int16).reshape(-1), expected.view(torch.int16).reshape(-1)
    assert not ((a != e) & mask).any(), "restore wrote outside its output states"


@pytest.mark.parametrize("frame_bytes", [65536, 4096])
def test_logstate_masked_stores_and_conv_copy(frame_bytes):
    """store_states, store_conv (masked_store.py:11-72) and
    copy_conv_snapshots (conv_copy.py:7-52) on a fragmented frame storage
    against the oracle, bit-exact over the whole storage; negative slots are
    skipped.  frame_bytes 4096: state heads and conv snapshots span frames."""
    from logssms_amd.kernel.linear_attention.conv_copy import copy_conv_snapshots
    from logssms_amd.kernel.linear_attention.masked_store import store_conv, store_states
    g = gen(111 + frame_bytes % 1000)
    H, HV, dk, dv, layers, page, gran, W, slots = 2, 4, 128, 128, 2, 64, 16, 4, 5
    conv_dim = 2 * H * dk + HV * dv
    storage, payload, decay, conv, record, pool = _decode_pool(g, slots, H, HV, dk, dv, layers, page, gran, conv_dim,
                                                               W, max(frame_bytes, 4 * layers * page * HV), 32768)
    frame_bytes = pool.frame_bytes
    pool.layout.conv_dim, pool.layout.state_len = conv_dim, W - 1
    expected = storage.clone()
    dev_u8 = storage.view(torch.uint8).to(DEV)
    pool.storage = dev_u8
    pool.payload_frame_table, pool.conv_frame_table = payload.to(DEV), conv.to(DEV)
    print(f"masked stores / conv copy frame_bytes={frame_bytes}", flush=True)
    state_slots = torch.tensor([3, -1, 0], dtype=torch.int32)
    states = torch.randn(3, HV, dk, dv, generator=g)
    ofr.store_states(expected, payload, frame_bytes, 32768, state_slots.long(), 1, states)
    store_states(pool, state_slots.to(DEV), 1, states.to(DEV))
    conv_slots, conv_gran = torch.tensor([1, 4, -1, 2]), torch.tensor([3, 0, 1, 2])
    windows = torch.randn(4, conv_dim, W - 1, generator=g).to(torch.bfloat16)
    ofr.store_conv(expected, conv, frame_bytes, conv_slots, conv_gran, 0, windows)
    store_conv(pool, conv_slots.to(DEV), conv_gran.to(DEV), 0, windows.to(DEV))
    src, sg = torch.tensor([1, 2, -1], dtype=torch.int32), torch.tensor([3, 2, 0], dtype=torch.int32)
    dst, dg = torch.tensor([0, 3, 4], dtype=torch.int32), torch.tensor([1, 0, 1], dtype=torch.int32)
    ofr.copy_conv_snapshots(expected, conv, frame_bytes, src, sg, dst, dg, layers=layers, C=conv_dim, S=W - 1)
    copy_conv_snapshots(pool, src.to(DEV), sg.to(DEV), dst.to(DEV), dg.to(DEV))
    torch.cuda.synchronize()
    host = dev_u8.cpu().view(torch.bfloat16).reshape(storage.shape)
    diff = host.view(torch.int16) != expected.view(torch.int16)
    assert not diff.any(), f"{int(diff.sum())} elements differ"
    assert not torch.equal(expected, storage), "the stores changed nothing"


def test_logstate_metadata_then_prefill_and_captured_decode():
    """GatedDeltaLogStateBackend.prepare_metadata (logstate.py:92-272) from
    the state / work / page tables and a LogStateCacheMetadata: request A
    (no cached prefix, 100 tokens) and request B (32 cached tokens in log slot
    7, 37 new ones).  Checkpoint writes at granule ends (a work-kind slot takes
    granule 0, others the last granule), one that is not at a granule end
    (ignored), and an unlogged range.  The built fields are checked against a
    per-token statement of the same plan, then the prefill runs on them
    against the oracle, then one decode step through prepare_for_capture's
    capture buffers."""
    from types import SimpleNamespace
    from logssms_amd.core import Batch, Context, LogStateCacheMetadata, Request
    from logssms_amd.layers import GatedDeltaLogStateBackend
    g = gen(121)
    H, HV, dk, dv, layers, layer, page, gran, W = 2, 4, 128, 128, 2, 1, 64, 16, 4
    C = 2 * H * dk + HV * dv
    frame_bytes, head_bytes = 65536, 32768
    slots = 10  # 0, 1 work; 2, 3, 4, 7 log pages; 5, 6, 9 checkpoints; 8 a work-kind checkpoint
    storage, payload, decay, conv, record, pool = _decode_pool(g, slots, H, HV, dk, dv, layers, page, gran, C, W,
                                                               frame_bytes, head_bytes)
    fe = frame_bytes // 2

    def read_conv(s, gr, lay):
        idx = ofr.conv_element_index(conv, s.cpu(), gr.cpu(), lay, C, W - 1, fe).to(DEV)
        return pool.storage.view(torch.bfloat16).reshape(-1)[idx].view(len(s), C, W - 1)

    pool.read_conv = read_conv
    pool.allocator = SimpleNamespace(slot=lambda s: SimpleNamespace(kind="work" if s in (0, 1, 8) else "log"))
    dev_u8 = storage.view(torch.uint8).to(DEV)
    pool.storage = dev_u8
    pool.payload_frame_table, pool.decay_frame_table, pool.conv_frame_table = payload.to(DEV), decay.to(DEV), conv.to(DEV)
    # tables: row 0 = request A (log pages 2, 3), row 1 = request B (log pages 7, 4)
    width = 4 * page
    state_table = torch.full((2, width), -1, dtype=torch.int32)
    page_table = torch.zeros(2, width, dtype=torch.int64)
    log_pages = {0: [2, 3], 1: [7, 4]}
    kv_pages = {0: [5, 1], 1: [2, 7]}
    for row in (0, 1):
        for p in range(2):
            state_table[row, p * page:(p + 1) * page] = log_pages[row][p]
            page_table[row, p * page:(p + 1) * page] = kv_pages[row][p] * page + torch.arange(page)
    ctx = Context(page_size=page, linear_state=pool, state_table=state_table.to(DEV),
                  work_state_table=torch.tensor([[0], [1]], dtype=torch.int32, device=DEV), page_table=page_table.to(DEV))
    backend = GatedDeltaLogStateBackend(ctx=ctx)
    reqs = [Request(table_idx=0, cached_len=0, device_len=100), Request(table_idx=1, cached_len=32, device_len=69)]
    lengths, cu = [100, 37], [0, 100, 137]
    T = cu[-1]
    rows = [0] * 100 + [1] * 37
    positions = torch.tensor(list(range(100)) + list(range(32, 69)), dtype=torch.int32)
    out_loc = page_table[torch.tensor(rows), positions.long()]
    cache = LogStateCacheMetadata(checkpoint_writes=[(136, 6), (47, 5), (63, 8), (50, 9)],
                                  checkpoint_ranges=[(0, 80, 90)])
    batch = Batch(reqs=reqs, phase="prefill", cache_metadata=cache, positions=positions.to(DEV),
                  out_loc=out_loc.to(DEV))
    backend.prepare_metadata(batch)
    meta = batch.linear_attn_metadata
    # ---- the plan, token by token
    offsets = (out_loc % page).tolist()
    log_slots = [int(state_table[rows[t], int(positions[t])]) for t in range(T)]
    want_log = [-1 if 80 <= t < 90 else log_slots[t] for t in range(T)]
    want_conv, want_gran = [-1] * T, [0] * T
    for n in range(2):
        for r in range(lengths[n]):
            t = cu[n] + r
            if (offsets[t] + 1) % gran == 0 or r + 1 == lengths[n]:
                want_conv[t], want_gran[t] = log_slots[t], offsets[t] // gran
    for t in range(80, 90):
        want_conv[t] = -1
    for t, s, gr in [(136, 6, 3), (47, 5, 3), (63, 8, 0)]:
        want_conv[t], want_gran[t] = s, gr
    want_chunks = [-1] * (7 + 3)
    want_chunks[2], want_chunks[3], want_chunks[7 + 2] = 5, 8, 6
    assert meta.work_slots.tolist() == [0, 1]
    assert meta.log_slots.tolist() == log_slots and meta.token_offsets.tolist() == offsets
    assert meta.conv_read_slots.tolist() == [0, 7] and meta.conv_read_granules.tolist() == [0, 1]
    assert meta.log_write_slots.tolist() == want_log
    assert meta.conv_token_slots.tolist() == want_conv and meta.conv_token_granules.tolist() == want_gran
    assert meta.chunk_write_slots.tolist() == want_chunks
    assert meta.cu_seqlens.tolist() == cu
    # ---- the prefill on that metadata
    cfg = SimpleNamespace(key_dim=H * dk, value_dim=HV * dv, head_k_dim=dk, head_v_dim=dv, layer_idx=layer,
                          state_len=W - 1, conv_dim=C, num_k_heads=H, num_v_heads=HV)
    weight = (torch.randn(C, 1, W, generator=g) * 0.3).to(torch.bfloat16)
    A_log, dt_bias = torch.randn(HV, generator=g) * 0.3, torch.randn(HV, generator=g) * 0.3
    expected = storage.clone()
    mixed = torch.randn(T, C, generator=g).to(torch.bfloat16)
    gate, beta = torch.randn(T, HV, generator=g).to(torch.bfloat16), torch.randn(T, HV, generator=g).to(torch.bfloat16)
    o_ref = ofr.forward_prefill_logstate(mixed, gate, beta, weight, A_log, dt_bias, expected, payload, decay, conv,
                                         frame_bytes, head_bytes, record, layer=layer, layers=layers,
                                         granularity=gran, page_size=page, cu_seqlens=cu,
                                         work_slots=torch.tensor([0, 1]), conv_read_slots=torch.tensor([0, 7]),
                                         conv_read_granules=[0, 1], conv_token_slots=torch.tensor(want_conv),
                                         conv_token_granules=torch.tensor(want_gran),
                                         chunk_write_slots=torch.tensor(want_chunks),
                                         log_write_slots=torch.tensor(want_log), token_offsets=torch.tensor(offsets),
                                         num_k_heads=H, head_k_dim=dk, num_v_heads=HV, head_v_dim=dv)
    print("LogState metadata: prefill [100, 37 after 32 cached]", flush=True)
    o = backend.forward(mixed.to(DEV), gate.to(DEV), beta.to(DEV), weight.to(DEV), A_log.to(DEV), dt_bias.to(DEV),
                        cfg, batch)
    torch.cuda.synchronize()
    _report("prefill out", o, o_ref)
    assert_bf16_close(o, o_ref)
    # ---- one decode step through the capture buffers
    backend.init_capture_graph(256, [2, 4])
    dpos = torch.tensor([100, 69], dtype=torch.int32)
    dloc = page_table[torch.tensor([0, 1]), dpos.long()]
    dreqs = [Request(table_idx=0, cached_len=100, device_len=101), Request(table_idx=1, cached_len=69, device_len=70)]
    dbatch = Batch(reqs=dreqs, phase="decode", cache_metadata=LogStateCacheMetadata(replay_counts=[0, 0]),
                   positions=dpos.to(DEV), out_loc=dloc.to(DEV))
    backend.prepare_for_capture(dbatch)
    dmeta = dbatch.linear_attn_metadata
    assert dmeta.work_slots.data_ptr() == backend.capture.work_slots.data_ptr()
    dlogs = [int(state_table[0, 100]), int(state_table[1, 69])]
    assert dmeta.log_slots.tolist() == dlogs and dmeta.token_offsets.tolist() == (dloc % page).tolist()
    assert dmeta.conv_read_slots.tolist() == [0, 1] and dmeta.conv_read_granules.tolist() == [0, 0]
    assert dmeta.replay_counts.tolist() == [0, 0]
    x = torch.randn(2, C, generator=g).to(torch.bfloat16)
    a, bt = torch.randn(2, HV, generator=g).to(torch.bfloat16), torch.randn(2, HV, generator=g).to(torch.bfloat16)
    off = dloc % page
    y = ofr.conv_decode_logstate(x, weight, expected, conv, frame_bytes, layer, torch.tensor([0, 1]),
                                 torch.zeros(2, dtype=torch.int64), torch.tensor(dlogs), off // gran,
                                 torch.tensor([0, 1]))
    q, k, v = (y[:, :H * dk].reshape(2, 1, H, dk), y[:, H * dk:2 * H * dk].reshape(2, 1, H, dk),
               y[:, 2 * H * dk:].reshape(2, 1, HV, dv))
    o_ref = ofr.fused_recurrent_to_logstate(q, k, v, a[:, None], bt[:, None], A_log, dt_bias, expected, payload, decay,
                                            frame_bytes, head_bytes, record, torch.tensor([0, 1]), torch.tensor(dlogs),
                                            off, torch.tensor([0, 0]), layer=layer, layers=layers, granularity=gran,
                                            page_size=page)
    o = backend.forward(x.to(DEV), a.to(DEV), bt.to(DEV), weight.to(DEV), A_log.to(DEV), dt_bias.to(DEV), cfg, dbatch)
    torch.cuda.synchronize()
    _report("decode out", o, o_ref[:, 0])
    assert_bf16_close(o, o_ref[:, 0])
    host = dev_u8.cpu().view(torch.bfloat16).reshape(storage.shape)
    for name, s in (("work", [0, 1]), ("checkpoints", [5, 6, 8])):
        got = ofr.read_frame_states(host, payload, s, layer, HV, dk, dv, frame_bytes, head_bytes)
        want = ofr.read_frame_states(expected, payload, s, layer, HV, dk, dv, frame_bytes, head_bytes)
        _report(f"{name} states", got, want)
        assert_state16_close(got, want)
