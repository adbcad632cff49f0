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


def _frame_setup(g, slots, layers, HV, dk, dv, frame_bytes, head_bytes, spare=7):
    """A fragmented frame storage: every slot's frames drawn at random from a
    shuffled pool with spare frames, unused table columns -1."""
    fps = -(-layers * HV * head_bytes // frame_bytes)
    num_frames = slots * fps + spare
    order = torch.randperm(num_frames, generator=g)[:slots * fps]
    frames = order.reshape(slots, fps).to(torch.int32)
    storage = (torch.randn(num_frames, frame_bytes // 2, generator=g) * 0.1).to(torch.bfloat16)
    return storage, frames


# (dk, dv, frame_bytes, head_bytes): two heads per frame; a head over two
# frames; a padded head (128 x 192 bf16 = 48 KiB in a 64 KiB payload)
FRAME_CASES = [(128, 128, 65536, 32768), (128, 128, 16384, 32768), (128, 192, 131072, 65536)]


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


def test_chunk_token_log():
    """ChunkLogIO: each logged token's v' rows, key rows and gate land in its
    log slot (state_io.py:83-126); keys and gates bit-exact, v' rows to the
    output tolerance, every other byte untouched."""
    from logssms_amd.kernel.linear_attention import ChunkLogIO, ChunkStateIO, chunk_gated_delta_rule_to_cache
    g = gen(71)
    H, HV, dk, dv, layers, layer, gran, page = 2, 4, 128, 128, 2, 1, 32, 64
    frame_bytes, head_bytes = 65536, 32768
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
    storage, frames = _frame_setup(g, slots, layers, HV, dk, dv, frame_bytes, head_bytes, spare=2)
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
                                           log_io=log)
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
