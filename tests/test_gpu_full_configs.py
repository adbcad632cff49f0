"""Parity at the full BASELINE prefill shapes, built exactly as ``bench.py``
builds its workloads, on both prefill paths (the fused three-launch path and
the two-step front end + chunk kernel), against the fp32 CPU oracle:

* config 2 -- 4 x 4096 packed tokens, 16 qk / 32 v heads, d = 128, zero
  initial state, the final state of each sequence written to its slot (64
  chained chunks per sequence);
* config 4 -- 64 lognormal-length sequences (up to 14,270 tokens, 223
  chained chunks), half resuming from a cached N(0, 0.1) state and N(0, 1)
  conv history in a random pool slot, a checkpoint (state + conv window)
  every 1024 tokens and at the end, 178 checkpoints in fresh slots.

The checks follow the reference's dispatch and Marconi tests
(``tests/kernel/test_gdn_prefill_dispatch.py:143-197``: output and every
chunk-end checkpoint against the recurrence; ``tests/hybrid/test_marconi.py:
499-573``: the pool compared slot by slot): bf16 outputs within
``1e-2 + 2e-2 |e|``, every written state within max-abs 1e-3, the conv pool
bit-exact, and every slot that was not written (including the baseline slots
the hits read) bit-identical to its initial contents."""

import pytest
import torch

import bench
from oracle import gdn as ref
from tests.gpu_util import DEV, assert_bf16_close

pytestmark = pytest.mark.gpu

_CACHE = {}


def _workload(name):
    """(inputs, initial conv pool, initial state pool, oracle output, oracle
    conv pool, oracle state pool), computed once per config."""
    if name not in _CACHE:
        _CACHE.clear()  # one config's tensors at a time
        inp = bench.make_prefill(draw_device=DEV) if name == "cfg2" else bench.make_prefill_cfg4(draw_device=DEV)
        conv0, state0 = (t.cpu() for t in bench.make_prefill_pools(inp, DEV))
        conv, state = conv0.clone(), state0.clone()
        print(f"{name}: oracle over {inp['T']} tokens, {inp['N']} sequences", flush=True)
        out = ref.forward_prefill(inp["mixed"], inp["gate"], inp["beta"], inp["weight"], inp["A_log"],
                                  inp["dt_bias"], conv, state, 0, inp["cu"], inp["baseline"], inp["chunk_write"],
                                  inp["conv_tokens"], bench.H, bench.D, bench.HV, bench.D)
        _CACHE[name] = (inp, conv0, state0, out, conv, state)
    return _CACHE[name]


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "two_step"])
@pytest.mark.parametrize("name", ["cfg2", "cfg4"])
def test_full_config_prefill_matches_oracle(name, fused):
    inp, conv0, state0, want_o, want_conv, want_state = _workload(name)
    print(f"{name} {'fused' if fused else 'two-step'}: {inp['T']} tokens on the GPU", flush=True)
    pools = (conv0.to(DEV), state0.to(DEV))
    step, _, out = bench.prefill_gpu(inp, DEV, fused=fused, pools=pools)
    step()
    torch.cuda.synchronize()
    got_conv, got_state = pools[0].cpu(), pools[1].cpu()
    assert_bf16_close(out[0], want_o)
    out_err = float((out[0].float().cpu() - want_o.float()).abs().max())

    written = sorted({int(s) for s in inp["chunk_write"].tolist() if s >= 0})
    assert len(written) == (inp["N"] if name == "cfg2" else inp["checkpoints"])
    state_err = float((got_state[written] - want_state[written]).abs().max())
    assert state_err <= 1e-3, f"written state max-abs error {state_err:.3e}"
    untouched = torch.ones(got_state.shape[0], dtype=torch.bool)
    untouched[written] = False
    assert torch.equal(got_state[untouched], state0[untouched]), "a slot that was not written changed"
    assert torch.equal(got_conv, want_conv), "conv pool differs from the oracle"
    print(f"{name} {'fused' if fused else 'two-step'}: output max-abs {out_err:.3e}, "
          f"{len(written)} written states max-abs {state_err:.3e}", flush=True)


def test_full_config3_decode_matches_oracle():
    """Config 3 as ``bench.py`` builds it: 256 sequences, in-place
    read-modify-write of random-permutation slots of a 1024-slot fp32 pool
    (2 GiB) and its bf16 conv pool, against the oracle's batched decode on
    host copies: outputs within 1e-2 + 2e-2 |e|, the 256 written states within
    1e-3, conv windows bit-exact, the other 768 slots untouched."""
    step, t = bench.decode_gpu(DEV)
    conv0, state0 = t["conv"].cpu(), t["state"].cpu()
    h = {k: v.cpu() for k, v in t.items() if k not in ("conv", "state", "out")}
    print("config 3 decode: 256 sequences on the GPU", flush=True)
    step()
    torch.cuda.synchronize()
    got_o, got_conv, got_state = t["out"].cpu(), t["conv"].cpu(), t["state"].cpu()
    conv, state = conv0.clone(), state0.clone()
    want_o = ref.forward_decode_batched(h["mixed"], h["gate"], h["beta"], h["weight"], h["A_log"], h["dt_bias"],
                                        conv, state, 0, h["reads"], h["writes"], bench.H, bench.D, bench.HV, bench.D)
    assert_bf16_close(got_o, want_o.view(got_o.shape))
    slots = h["writes"].long()
    err = float((got_state[slots] - state[slots]).abs().max())
    assert err <= 1e-3, f"written state max-abs error {err:.3e}"
    assert torch.equal(got_conv, conv), "conv pool differs from the oracle"
    untouched = torch.ones(state.shape[0], dtype=torch.bool)
    untouched[slots] = False
    assert torch.equal(got_state[untouched], state0[untouched])
    print(f"config 3 decode: output max-abs {float((got_o.float() - want_o.float().view(got_o.shape)).abs().max()):.3e}, "
          f"states {err:.3e}", flush=True)


def test_full_config5_verify_and_commit_match_oracle():
    """Config 5 as ``bench.py`` builds it: 64 sequences x 8 drafts from random
    live slots, every per-step state and conv window written to 512 fresh
    slots, against the oracle's batched verify on host copies (outputs within
    1e-2 + 2e-2 |e|, the 512 step states within 1e-3, windows bit-exact, other
    slots untouched); then the commit copies each sequence's accepted step
    (accepted ~ U{1..8}) into its live slot, bit for bit."""
    step, commit, t = bench.verify_gpu(DEV)
    conv0, state0 = t["conv"].cpu(), t["state"].cpu()
    h = {k: v.cpu() for k, v in t.items() if k not in ("conv", "state", "out")}
    print("config 5 verify: 64 x 8 drafts on the GPU", flush=True)
    step()
    torch.cuda.synchronize()
    got_o, got_conv, got_state = t["out"].cpu(), t["conv"].cpu(), t["state"].cpu()
    conv, state = conv0.clone(), state0.clone()
    want_o = ref.forward_verify_batched(h["mixed"], h["gate"], h["beta"], h["weight"], h["A_log"], h["dt_bias"],
                                        conv, state, 0, h["live"], h["writes"], bench.H, bench.D, bench.HV, bench.D)
    assert_bf16_close(got_o, want_o.view(got_o.shape))
    written = h["writes"].reshape(-1).long()
    err = float((got_state[written] - state[written]).abs().max())
    assert err <= 1e-3, f"step state max-abs error {err:.3e}"
    assert torch.equal(got_conv, conv), "conv pool differs from the oracle"
    untouched = torch.ones(state.shape[0], dtype=torch.bool)
    untouched[written] = False
    assert torch.equal(got_state[untouched], state0[untouched])
    # commit: live[b] <- step accepted[b] - 1 of sequence b, state and conv window
    commit()
    torch.cuda.synchronize()
    live, acc = h["live"].long(), h["accepted"].long()
    src = h["writes"].long()[torch.arange(len(live)), acc - 1]
    assert torch.equal(t["state"].cpu()[live], got_state[src])
    assert torch.equal(t["conv"].cpu()[live], got_conv[src])
    print(f"config 5 verify: output max-abs {float((got_o.float() - want_o.float().view(got_o.shape)).abs().max()):.3e}, "
          f"states {err:.3e}; commit bit-exact", flush=True)
