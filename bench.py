"""Benchmark of the MI355X Gated DeltaNet hot path.

Headline (``value``): Qwen3-Next linear-attention layer prefill (BASELINE
config 2) -- 4 x 4096 packed tokens, 16 qk / 32 v heads, d = 128, bf16
projections, fp32 state pool, conv width 4.  One step = the backend prefill
``prefill_fused``: the q/k pass (conv + SiLU + L2 norm of the q/k channels),
then the chunk-kernel launch whose staging waves compute the v conv + SiLU and
the gates of each chunk from mixed_qkv, writing the output, the final
per-sequence states into pool slots and the conv windows into the conv pool.
``value`` is prefill tokens/s; ``roofline`` reports the chunk kernel (timed
alone with events around its launch) against the dense 16-bit MFMA peak from
the algorithmic flop count (10 C d + 6 d^2 + 2/3 C^2 per token per v-head).
``extra.prefill_two_step_ms`` times the unfused path (``prefill_frontend``
then the chunk kernel) on the same inputs.

``extra`` reports the varlen prefill with prefix-cache hits and checkpoints
(config 4), and the HBM-bound paths: decode (config 3), spec-decode verify
(config 5) and the gated RMS norm of the config 2 output, in GB/s against
8 TB/s, from the canonical byte formulas.

Every time is the median over the K timed steps, each bracketed by its own
pair of HIP events inside one synchronized region, after W warm-up steps
(defaults K = 50, W = 10).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_MFMA_16BIT = 2.5e15  # MI355X dense bf16/fp16 FLOP/s (published)
PEAK_HBM = 8.0e12  # MI355X HBM3E bytes/s (published)
MFMA_16BIT_FLOP_PER_CLK_PER_CU = 4096  # dense 16-bit MFMA issue of one CDNA4 CU

# hipDeviceAttribute_t values of this ROCm's hip_runtime_api.h: peak engine
# clock (kHz), peak memory clock (kHz), memory bus width (bits), compute units
_HIP_ATTRS = {"engine_clock_khz": 5, "memory_clock_khz": 60, "memory_bus_bits": 59, "compute_units": 63}

H, HV, D, W = 16, 32, 128, 4
CONV_DIM = 2 * H * D + HV * D  # 8192
C = 64
FLOP_PER_TOKEN_HEAD = 10 * C * D + 6 * D * D + (2 / 3) * C * C  # 182,954.67
S_BYTES = HV * D * D * 4  # fp32 state per sequence
SC_BYTES = CONV_DIM * (W - 1) * 2  # bf16 conv window per sequence


def _traffic(name):
    """HBM bytes per launch measured with the FETCH_SIZE / WRITE_SIZE counter
    passes (calibrated on a plain copy), from the committed profile summary;
    None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "gdn_kernels_hbm_traffic_pmc.md")
    try:
        with open(path) as fh:
            for line in fh:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic" and parts[1] == name:
                    return int(parts[2])
    except OSError:
        pass
    return None


def device_peaks(index=0):
    """The clocks the HIP runtime reports for the device and the peaks they
    imply: 16-bit MFMA = CUs x engine clock x 4096 FLOP/clk/CU, HBM = bus
    width x 4 transfers per reported memory clock (the HBM3/HBM3E pin rate
    is 4x the clock the runtime reports: 2 GHz x 4 x 8192 bits = 8.2 TB/s
    here).  The roofline fractions use the published peaks; these are
    printed beside them."""
    import ctypes
    out = {}
    try:
        hip = ctypes.CDLL("libamdhip64.so")
        for name, attr in _HIP_ATTRS.items():
            value = ctypes.c_int(0)
            out[name] = value.value if hip.hipDeviceGetAttribute(ctypes.byref(value), attr, index) == 0 else None
    except OSError:
        return out
    if out.get("compute_units") and out.get("engine_clock_khz"):
        out["mfma_16bit_peak_tflops"] = (out["compute_units"] * out["engine_clock_khz"] * 1e3
                                         * MFMA_16BIT_FLOP_PER_CLK_PER_CU / 1e12)
    if out.get("memory_clock_khz") and out.get("memory_bus_bits"):
        out["hbm_peak_gbps"] = 4 * out["memory_clock_khz"] * 1e3 * out["memory_bus_bits"] / 8 / 1e9
    out["published"] = {"mfma_16bit_tflops": PEAK_MFMA_16BIT / 1e12, "hbm_gbps": PEAK_HBM / 1e9}
    return out


def cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _median_time(fn, budget_s, max_runs=50):
    """Median wall time of fn over as many runs as fit in ``budget_s`` (at
    least one, after one untimed warm-up run)."""
    fn()
    times = []
    t_start = time.perf_counter()
    while not times or (time.perf_counter() - t_start < budget_s and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def _config(layer=0):
    from logssms_amd.layers import GatedDeltaConfig
    return GatedDeltaConfig(H, HV, D, D, CONV_DIM, W - 1, layer)


def _median(values):
    v = sorted(values)
    n = len(v)
    return v[n // 2] if n % 2 else 0.5 * (v[n // 2 - 1] + v[n // 2])


def _time(fn, steps, warmup, events=None, stats=None):
    """`warmup` untimed calls of fn, then `steps` timed calls between
    synchronize barriers, each call bracketed by its own pair of events on the
    current stream (one event between consecutive calls).  Returns the median
    ms per call; `stats` (dict) receives the mean, min and max.  `events`
    (list) collects per-kernel (start, end) pairs recorded inside fn."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    if events is not None:
        events.clear()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    marks[0].record()
    for i in range(steps):
        fn()
        marks[i + 1].record()
    torch.cuda.synchronize()
    per_step = [marks[i].elapsed_time(marks[i + 1]) for i in range(steps)]
    if stats is not None:
        stats.update(mean_ms=marks[0].elapsed_time(marks[-1]) / steps, min_ms=min(per_step), max_ms=max(per_step))
    return _median(per_step)


def _kernel_ms(events):
    """Median duration of the kernel launches bracketed by `events`."""
    if not events:
        return None
    return _median([a.elapsed_time(b) for a, b in events])


# ---------------------------------------------------------------- prefill (config 2)

def make_prefill(seed=2, lengths=(4096, 4096, 4096, 4096), draw_device="cpu"):
    """Config 2's inputs (host tensors).  The projections (``mixed``, the
    largest tensor) are drawn on ``draw_device`` with a generator of that
    device seeded with ``seed`` and copied to the host, so a GPU box draws
    config 4's 1.2 G values in milliseconds; the rest come from a CPU
    generator.  Every consumer (bench, parity tests, CPU baseline) reads the
    same host copy."""
    g = torch.Generator().manual_seed(seed)
    T = sum(lengths)
    N = len(lengths)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    gm = torch.Generator(device=draw_device).manual_seed(seed)
    mixed = torch.randn(T, CONV_DIM, generator=gm, device=draw_device).to(torch.bfloat16).cpu()
    weight = (torch.randn(CONV_DIM, 1, W, generator=g) * 0.02).to(torch.bfloat16)
    gate = torch.randn(T, HV, generator=g).to(torch.bfloat16)
    beta = torch.randn(T, HV, generator=g).to(torch.bfloat16)
    A_log = -torch.rand(HV, generator=g)  # g = -softplus(a) * exp(U(-1, 0))
    dt_bias = torch.zeros(HV)
    nchunks = [(n + C - 1) // C for n in lengths]
    chunk_write = torch.full((sum(nchunks),), -1, dtype=torch.int64)
    conv_tokens = torch.full((T,), -1, dtype=torch.int64)
    off = 0
    for i, nc in enumerate(nchunks):
        off += nc
        chunk_write[off - 1] = i  # final state of sequence i -> pool slot i
        conv_tokens[cu[i + 1] - 1] = i  # final conv window of sequence i -> pool slot i
    snap_rows = torch.tensor(cu[1:], dtype=torch.int64) - 1
    return dict(mixed=mixed, weight=weight, gate=gate, beta=beta, A_log=A_log, dt_bias=dt_bias,
                cu=torch.tensor(cu), baseline=torch.full((N,), -1, dtype=torch.int64), chunk_write=chunk_write,
                conv_tokens=conv_tokens, snap_rows=snap_rows, snap_slots=torch.arange(N, dtype=torch.int64), N=N, T=T)


def make_prefill_cfg4(seed=4, n=64, median=1500, sigma=1.0, every=1024, hit_rate=0.5, draw_device="cpu"):
    """64 packed sequences with lognormal lengths (median
    1500, sigma 1.0, clipped to 16..16384); half of them (seeded choice)
    start from a cached state and conv history in a random pool slot
    (state ~N(0, 0.1), conv ~N(0, 1)); a checkpoint (state + conv window) is
    written to a fresh slot at every multiple of 1024 tokens below the length
    and at the length."""
    import numpy as np
    rng = np.random.default_rng(seed)
    lengths = np.clip(np.rint(rng.lognormal(np.log(median), sigma, n)), 16, 16384).astype(int).tolist()
    inp = make_prefill(seed, lengths, draw_device)
    N, T = inp["N"], inp["T"]
    hits = rng.permutation(N)[: int(round(hit_rate * N))]
    nck = sum(len(range(every, m, every)) + 1 for m in lengths)
    slots = rng.permutation(len(hits) + nck + 8)
    baseline = torch.full((N,), -1, dtype=torch.int64)
    baseline[torch.as_tensor(hits)] = torch.as_tensor(slots[: len(hits)], dtype=torch.int64)
    fresh = iter(slots[len(hits):].tolist())
    nchunks = [(m + C - 1) // C for m in lengths]
    chunk_write = torch.full((sum(nchunks),), -1, dtype=torch.int64)
    rows, snap_slots = [], []
    c0 = t0 = 0
    for m, nc in zip(lengths, nchunks):
        for end in list(range(every, m, every)) + [m]:
            slot = next(fresh)
            chunk_write[c0 + (end - 1) // C] = slot
            rows.append(t0 + end - 1)
            snap_slots.append(slot)
        c0 += nc
        t0 += m
    conv_tokens = torch.full((T,), -1, dtype=torch.int64)
    conv_tokens[torch.tensor(rows)] = torch.tensor(snap_slots)
    inp.update(baseline=baseline, chunk_write=chunk_write, snap_rows=torch.tensor(rows),
               snap_slots=torch.tensor(snap_slots), conv_tokens=conv_tokens, slots=len(slots), random_pools=seed,
               lengths=lengths, checkpoints=len(rows))
    return inp


def make_prefill_pools(inp, dev):
    """The conv-window and fp32 state pools of a prefill workload: zeros, or
    for config 4 (``random_pools`` = seed) N(0, 1) windows and N(0, 0.1)
    states, the cached prefixes the hits resume from."""
    slots = inp.get("slots", max(8, inp["N"]))
    conv_pool = torch.zeros(slots, 1, CONV_DIM, W - 1, device=dev, dtype=torch.bfloat16)
    state_pool = torch.zeros(slots, 1, HV, D, D, device=dev, dtype=torch.float32)
    if inp.get("random_pools") is not None:
        gd = torch.Generator(device=dev).manual_seed(int(inp["random_pools"]))
        state_pool.normal_(0.0, 0.1, generator=gd)
        conv_pool.copy_(torch.randn(conv_pool.shape, device=dev, generator=gd).to(torch.bfloat16))
    return conv_pool, state_pool


def prefill_gpu(inp, dev, events=None, fused=True, pools=None):
    """One backend prefill step.  fused: ``prefill_fused`` (q/k pass, then the
    chunk kernel computing the v conv + SiLU and the gates itself and writing
    the conv windows); otherwise the two-step path (``prefill_frontend``
    writing q, k, v, g, beta and then the windows, then the chunk kernel).
    `events` collects a (start, end) event pair around each chunk-kernel
    launch; `pools` = (conv_pool, state_pool) to run on, else fresh ones."""
    from logssms_amd.kernel.linear_attention import ChunkStateIO, chunk_gated_delta_rule_to_cache
    from logssms_amd.kernel.linear_attention.fused_backend import prefill_frontend, prefill_fused
    cfg = _config()
    d = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    conv_pool, state_pool = pools if pools is not None else make_prefill_pools(inp, dev)
    out = torch.empty(1, d["T"], HV, D, device=dev, dtype=torch.bfloat16)
    io = ChunkStateIO(state_pool, d["baseline"], d["chunk_write"], layer=0)

    def mark():
        if events is None:
            return None
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        return ev

    def step():
        if fused:
            ev = None
            if events is not None:
                ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                events.append(ev)
            o = prefill_fused(d["mixed"], d["gate"], d["beta"], d["weight"], d["A_log"], d["dt_bias"], cfg,
                              conv_pool, state_pool, d["cu"], d["baseline"], d["chunk_write"], d["snap_rows"],
                              d["snap_slots"], out=out[0], chunk_events=ev)
            assert o is not None
            return out
        else:
            q, k, v, g, b = prefill_frontend(d["mixed"], d["gate"], d["beta"], d["weight"], d["A_log"],
                                             d["dt_bias"], cfg, conv_pool, d["cu"], d["baseline"], d["snap_rows"],
                                             d["snap_slots"])
            s = mark()
            chunk_gated_delta_rule_to_cache(q, k, v, g, b, io, d["cu"], out=out, return_v_new=False)
            if events is not None:
                events.append((s, mark()))
        return out

    return step, state_pool, out


def prefill_cpu_legs(inp, chunk_tokens, naive_tokens, budget_s):
    """The prefill CPU baseline on config 2's inputs, all host threads:
    (ii) the oracle's chunked restatement (conv + prepare + chunk rule,
    ``forward_prefill``) on the first ``chunk_tokens`` tokens of sequence 0 at
    full head count; (i) the naive token recurrence (the reference test's
    semantics) on the first ``naive_tokens`` of them, from the same prepared
    q, k, v, g, beta.  Returns the two cpu_baseline-style dicts."""
    from oracle import gdn as ref
    mixed, gate, beta = inp["mixed"][:chunk_tokens], inp["gate"][:chunk_tokens], inp["beta"][:chunk_tokens]
    nc = (chunk_tokens + C - 1) // C

    def chunked():
        conv = torch.zeros(1, 1, CONV_DIM, W - 1, dtype=torch.bfloat16)
        state = torch.zeros(1, 1, HV, D, D)
        ref.forward_prefill(mixed, gate, beta, inp["weight"], inp["A_log"], inp["dt_bias"], conv, state, 0,
                            [0, chunk_tokens], [-1], [-1] * nc, [-1] * chunk_tokens, H, D, HV, D)

    t_chunk, runs = _median_time(chunked, budget_s)
    n = naive_tokens
    y, _ = ref.packed_causal_conv1d(inp["mixed"][:n], inp["weight"], torch.zeros(1, CONV_DIM, W - 1,
                                                                                  dtype=torch.bfloat16), [0, n],
                                    window_rows=[])
    q, k, v = ref.split_qkv(y[None], H, D, HV, D)
    q, k, v, g, b = ref.prepare_gdn(q, k, v, inp["gate"][None, :n], inp["beta"][None, :n], inp["A_log"],
                                    inp["dt_bias"])
    t_naive, runs_naive = _median_time(
        lambda: ref.naive_recurrence(q[0], k[0], v[0], g[0], b[0], D ** -0.5, torch.zeros(HV, D, D)), budget_s / 3)
    return ({"value": chunk_tokens / t_chunk, "unit": "tokens/s",
             "sample": f"(ii) oracle forward_prefill (conv + prepare + chunked rule, fp32 torch) on the first "
                       f"{chunk_tokens} tokens of sequence 0 at full head count; median of {runs} runs"},
            {"value": n / t_naive, "unit": "tokens/s",
             "sample": f"(i) naive token recurrence (oracle naive_recurrence, the reference test's semantics, "
                       f"fp32 torch, 32 v-heads) on the first {n} tokens of sequence 0, truncated from 4096 to "
                       f"keep the run short; median of {runs_naive} runs"})


# ---------------------------------------------------------------- decode (config 3) / verify (config 5)

def decode_bytes(B):
    return B * (2 * S_BYTES + 2 * SC_BYTES + 2 * CONV_DIM + 2 * HV * D + 4 * HV) + CONV_DIM * W * 2 + 8 * HV


def verify_bytes(B, T):
    return (B * ((1 + T) * S_BYTES + (1 + T) * SC_BYTES + T * (2 * CONV_DIM + 2 * HV * D + 4 * HV))
            + CONV_DIM * W * 2 + 8 * HV)


def make_pools(g, slots, dev):
    state = torch.empty(slots, 1, HV, D, D, device=dev)
    state.normal_(0.0, 0.1, generator=torch.Generator(device=dev).manual_seed(int(torch.randint(1 << 30, (1,),
                                                                                                generator=g))))
    conv = torch.randn(slots, 1, CONV_DIM, W - 1, device=dev).to(torch.bfloat16)
    return state, conv


def decode_gpu(dev, B=256, slots=1024, seed=3, events=None):
    from logssms_amd.kernel.linear_attention.fused_backend import decode_step
    g = torch.Generator().manual_seed(seed)
    cfg = _config()
    state, conv = make_pools(g, slots, dev)
    slot_idx = torch.randperm(slots, generator=g)[:B].to(dev)
    mixed = torch.randn(B, CONV_DIM, generator=g).to(torch.bfloat16).to(dev)
    gate = torch.randn(B, HV, generator=g).to(torch.bfloat16).to(dev)
    beta = torch.randn(B, HV, generator=g).to(torch.bfloat16).to(dev)
    weight = (torch.randn(CONV_DIM, 1, W, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    A_log = (-torch.rand(HV, generator=g)).to(dev)
    dt_bias = torch.zeros(HV, device=dev)
    out = torch.empty(B, HV, D, device=dev, dtype=torch.bfloat16)

    def step():
        decode_step(mixed, gate, beta, weight, A_log, dt_bias, cfg, conv, state, slot_idx, slot_idx, out=out)

    tensors = dict(mixed=mixed, gate=gate, beta=beta, weight=weight, A_log=A_log, dt_bias=dt_bias, conv=conv,
                   state=state, reads=slot_idx, writes=slot_idx, out=out)
    return step, tensors


def decode_cpu_leg(t, budget_s):
    """Config 3 on the host: the oracle's vectorised decode step
    (``forward_decode_batched``: index_select / index_copy_ pool I/O, the
    recurrence batched over the 256 sequences) on a host copy of the GPU
    run's pools and inputs, all host threads."""
    from oracle import gdn as ref
    h = {k: v.cpu() for k, v in t.items() if k != "out"}

    def run():
        ref.forward_decode_batched(h["mixed"], h["gate"], h["beta"], h["weight"], h["A_log"], h["dt_bias"],
                                   h["conv"], h["state"], 0, h["reads"], h["writes"], H, D, HV, D)

    sec, runs = _median_time(run, budget_s, max_runs=10)
    nb = decode_bytes(h["mixed"].shape[0])
    return {"value": nb / sec / 1e9, "unit": "GB/s", "ms": sec * 1e3,
            "sample": f"oracle forward_decode_batched on config 3 in full (256 sequences, host copy of the GPU "
                      f"pools), fp32 torch; median of {runs} runs"}


def verify_gpu(dev, B=64, T=8, slots=1024, seed=5):
    from logssms_amd.kernel.linear_attention.fused_backend import verify_group
    from logssms_amd import _lib
    g = torch.Generator().manual_seed(seed)
    cfg = _config()
    state, conv = make_pools(g, slots, dev)
    perm = torch.randperm(slots, generator=g)
    live = perm[:B].to(dev)
    writes = perm[B:B + B * T].view(B, T).to(dev)
    accepted = torch.randint(1, T + 1, (B,), generator=g).to(dev)
    rows = B * T
    mixed = torch.randn(rows, CONV_DIM, generator=g).to(torch.bfloat16).to(dev)
    gate = torch.randn(rows, HV, generator=g).to(torch.bfloat16).to(dev)
    beta = torch.randn(rows, HV, generator=g).to(torch.bfloat16).to(dev)
    weight = (torch.randn(CONV_DIM, 1, W, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    A_log = (-torch.rand(HV, generator=g)).to(dev)
    dt_bias = torch.zeros(HV, device=dev)
    out = torch.empty(rows, HV, D, device=dev, dtype=torch.bfloat16)

    def step():
        verify_group(mixed, gate, beta, weight, A_log, dt_bias, cfg, conv, state, None, live, writes, out)

    def commit():
        _lib.call("gdn_commit_accepted", state.data_ptr(), state.stride(0) * 4, 0, S_BYTES, conv.data_ptr(),
                  conv.stride(0) * 2, 0, SC_BYTES, live.data_ptr(), 1, writes.data_ptr(), T, 1, 1,
                  accepted.data_ptr(), 1, B, T, _lib.stream_of(state))

    tensors = dict(mixed=mixed, gate=gate, beta=beta, weight=weight, A_log=A_log, dt_bias=dt_bias, conv=conv,
                   state=state, live=live, writes=writes, out=out, accepted=accepted)
    return step, commit, tensors


def verify_cpu_leg(t, budget_s):
    """Config 5 on the host: the oracle's batched verify
    (``forward_verify_batched``: 8 steps, each vectorised over the 64
    sequences, every per-step state and window written with index_copy_) on a
    host copy of the GPU run's pools and inputs, all host threads."""
    from oracle import gdn as ref
    h = {k: v.cpu() for k, v in t.items() if k not in ("out", "accepted")}

    def run():
        ref.forward_verify_batched(h["mixed"], h["gate"], h["beta"], h["weight"], h["A_log"], h["dt_bias"],
                                   h["conv"], h["state"], 0, h["live"], h["writes"], H, D, HV, D)

    sec, runs = _median_time(run, budget_s, max_runs=10)
    B, T = h["writes"].shape
    nb = verify_bytes(B, T)
    return {"value": nb / sec / 1e9, "unit": "GB/s", "ms": sec * 1e3,
            "sample": f"oracle forward_verify_batched on config 5 in full ({B} sequences x {T} drafts, host copy "
                      f"of the GPU pools), fp32 torch; median of {runs} runs"}


def norm_gpu(dev, T=16384, seed=6):
    """rms_norm_gated over the config 2 core output (T x HV rows of D channels)."""
    from logssms_amd.kernel.norm import rms_norm_gated
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, HV, D, generator=g).to(torch.bfloat16).to(dev)
    proj = torch.randn(T, 2 * HV * D, generator=g).to(torch.bfloat16).to(dev)
    z = proj[:, HV * D:].view(T, HV, D)
    w = torch.ones(D, device=dev)

    def step():
        rms_norm_gated(x, z, w, 1e-6)

    return step, 3 * T * HV * D * 2


def layer_gpu(dev, hidden=2048, seed=7):
    """The whole GatedDeltaNet layer (Qwen3-Next shape, hidden 2048) on the
    config 2 batch: merged projections (hipBLASLt GEMMs) whose column slices
    feed the backend prefill as strided views, the gated RMS norm and the
    output projection.  Returns (step, parts): parts times the three stages."""
    from logssms_amd.cache import LinearStatePool
    from logssms_amd.core import Batch, Context, Request, set_global_ctx
    from logssms_amd.layers import GatedDeltaNet
    g = torch.Generator(device=dev).manual_seed(seed)
    net = GatedDeltaNet(hidden, H, HV, D, D, W, 1e-6, 0, device=dev, dtype=torch.bfloat16)
    for t in (net.in_proj_qkvz_weight, net.in_proj_ba_weight, net.out_proj_weight):
        t.normal_(0.0, 0.02, generator=g)
    net.conv1d_weight.normal_(0.0, 0.02, generator=g)
    net.A_log.uniform_(-1.0, 0.0, generator=g)
    net.dt_bias.zero_()
    lengths = [4096] * 4
    pool = LinearStatePool(8, 1, CONV_DIM, W, HV, D, D, dev, torch.bfloat16)
    table = torch.arange(8, device=dev, dtype=torch.int32)[:4, None].expand(4, 4096).contiguous()
    ctx = Context(page_size=4096, linear_state=pool, state_table=table)
    set_global_ctx(ctx)
    batch = Batch(reqs=[Request(i, 0, n) for i, n in enumerate(lengths)], phase="prefill")
    ctx.batch = batch
    ctx.linear_attn_backend.prepare_metadata(batch)
    x = torch.randn(sum(lengths), hidden, device=dev, generator=g).to(torch.bfloat16)

    def step():
        return net.forward(x)

    def parts():
        mixed, z, beta, gate = net.proj(x)
        core = net.attend(mixed, beta, gate)
        return {"proj": lambda: net.proj(x), "core": lambda: net.attend(mixed, beta, gate),
                "output": lambda: net.output(core, z)}

    return step, parts


def _probe_lib():
    """The bench-only probe library (``logssms_amd/libgdn_probe.so``, built
    beside the product library from ``csrc/probe/rmw_probe.hip``)."""
    import ctypes
    path = os.path.join(ROOT, "logssms_amd", "libgdn_probe.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build with `make -C logssms_amd/csrc`")
    lib = ctypes.CDLL(path)
    lib.gdn_probe_rmw.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_void_p]
    lib.gdn_probe_rmw.restype = ctypes.c_int
    lib.gdn_probe_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.gdn_probe_mfma.restype = ctypes.c_int
    lib.gdn_probe_last_error.restype = ctypes.c_char_p
    return lib


def mfma_ceiling(dev, steps=10, warmup=3, iters=4096):
    """The box's sustained dense-f16 matrix-core rate: ``gdn_probe_mfma``
    (independent 16x16x32 f16 MFMA chains in every wave, 4 and 8 waves per
    CU, 4 workgroups per CU), timed like the kernels.  Under this load the
    engine clock falls below its 2.4 GHz maximum, so the rate lies below the
    published 2.5 PFLOP/s; the chunk kernel's fraction of it is reported beside
    the fraction of the published peak."""
    from logssms_amd import _lib
    probe = _probe_lib()
    props = torch.cuda.get_device_properties(dev)
    blocks = 4 * props.multi_processor_count
    runs = []
    for threads in (256, 512):
        out = torch.empty(blocks * threads, device=dev)
        stream = _lib.stream_of(out)

        def run():
            rc = probe.gdn_probe_mfma(out.data_ptr(), blocks, threads, iters, stream)
            if rc:
                raise RuntimeError(f"gdn_probe_mfma failed ({rc}): {probe.gdn_probe_last_error().decode()}")
        ms = _time(run, steps, warmup)
        flop = blocks * (threads // 64) * iters * 8 * 16384
        runs.append({"waves_per_cu": 4 * threads // 64, "ms": ms, "TFLOP/s": flop / (ms * 1e-3) / 1e12})
        del out
    best = max(runs, key=lambda r: r["TFLOP/s"])
    return {"config": f"gdn_probe_mfma: {blocks} workgroups, 8 independent v_mfma_f32_16x16x32_f16 chains per wave, "
                      f"{iters} rounds", "best_TFLOP/s": best["TFLOP/s"],
            "frac_of_published": best["TFLOP/s"] * 1e12 / PEAK_MFMA_16BIT, "runs": runs}


def rmw_sweep(dev, steps, warmup, nbytes=2 << 30):
    """The box's 1-read:1-write HBM ceiling over a 2 GiB buffer (the size of
    config 3's state pool), by three access patterns: ``gdn_probe_rmw`` (an
    in-place x <- 1.0 x stream over 16-byte vectors, for block sizes and loads
    in flight per lane), torch's in-place ``mul_`` and torch's device
    ``copy_`` (2 GiB read into another 2 GiB).  GB/s counts the bytes read plus
    the bytes written."""
    from logssms_amd import _lib
    probe = _probe_lib()

    def run(*args):
        rc = probe.gdn_probe_rmw(*args)
        if rc:
            raise RuntimeError(f"gdn_probe_rmw failed ({rc}): {probe.gdn_probe_last_error().decode()}")

    buf = torch.ones(nbytes // 4, device=dev)
    stream = _lib.stream_of(buf)
    runs = []
    for block_kib in (64, 1024):
        for loads in (1, 4, 16):
            for nt in (0, 1):
                ms = _time(lambda: run(buf.data_ptr(), nbytes, block_kib << 10, loads, nt, stream), steps, warmup)
                runs.append({"block_kib": block_kib, "loads_in_flight": loads, "nontemporal": nt, "ms": ms,
                             "GB/s": 2 * nbytes / (ms * 1e-3) / 1e9})
    best = max(runs, key=lambda r: r["GB/s"])
    # store-only stream (loads_in_flight 0): the write ceiling verify's per-step stores are read against
    writes = []
    for block_kib in (64, 1024):
        for nt in (0, 1):
            ms = _time(lambda: run(buf.data_ptr(), nbytes, block_kib << 10, 0, nt, stream), steps, warmup)
            writes.append({"block_kib": block_kib, "nontemporal": nt, "ms": ms, "GB/s": nbytes / (ms * 1e-3) / 1e9})
    best_w = max(writes, key=lambda r: r["GB/s"])
    # two library access patterns beside the probe
    ms_mul = _time(lambda: buf.mul_(1.0), steps, warmup)
    other = torch.empty_like(buf)
    ms_copy = _time(lambda: other.copy_(buf), steps, warmup)
    del buf, other
    torch.cuda.empty_cache()
    torch_legs = {"mul_": {"ms": ms_mul, "GB/s": 2 * nbytes / (ms_mul * 1e-3) / 1e9},
                  "copy_": {"ms": ms_copy, "GB/s": 2 * nbytes / (ms_copy * 1e-3) / 1e9}}
    ceiling = max([best["GB/s"]] + [leg["GB/s"] for leg in torch_legs.values()])
    return {"config": "gdn_probe_rmw over 2 GiB in place (1 read : 1 write, 16-byte vectors)", "best": best,
            "frac_hbm": best["GB/s"] * 1e9 / PEAK_HBM, "runs": runs,
            "torch": torch_legs, "best_GB/s": ceiling,
            "store_only": {"config": "gdn_probe_rmw loads_in_flight 0: 2 GiB of 16-byte stores", "best": best_w,
                           "frac_hbm": best_w["GB/s"] * 1e9 / PEAK_HBM, "runs": writes}}


# ---------------------------------------------------------------- LogState

LS_PAGE, LS_GRAN, LS_FRAME = 256, 32, 65536
LS_HEAD = D * D * 2  # bf16 state head


def make_frame_pool(dev, slots, seed=8):
    """A LogState frame storage at Qwen3-Next shape (one linear layer, bf16):
    64 KiB frames drawn at random for every slot's payload (states and the
    page's token log), one decay record per slot, one conv snapshot frame per
    (slot, granule); page 256, granularity 32."""
    from types import SimpleNamespace
    g = torch.Generator().manual_seed(seed)
    layers = 1
    fps = max(-(-layers * HV * LS_HEAD // LS_FRAME), -(-2 * LS_PAGE * layers * (H * D + HV * D) // LS_FRAME))
    record = 4 * layers * LS_PAGE * HV
    per = LS_FRAME // record
    n_dec = -(-slots // per)
    granules = LS_PAGE // LS_GRAN
    cf = -(-2 * layers * CONV_DIM * (W - 1) // LS_FRAME)
    total = slots * fps + n_dec + slots * granules * cf
    order = torch.randperm(total, generator=g)
    payload = order[:slots * fps].reshape(slots, fps).to(torch.int32)
    dec = order[slots * fps:slots * fps + n_dec]
    decay = torch.tensor([[int(dec[s // per]), s % per] for s in range(slots)], dtype=torch.int32)
    conv = order[slots * fps + n_dec:].reshape(slots, granules, cf).to(torch.int32)
    storage = torch.empty(total, LS_FRAME, dtype=torch.uint8, device=dev)
    storage.view(torch.bfloat16).normal_(0.0, 0.05, generator=torch.Generator(device=dev).manual_seed(seed))
    # decay records hold gates (natural-log decays <= 0)
    rec = storage[dec.to(dev)].view(torch.float32)
    rec.copy_(-torch.rand(rec.shape, device=dev) * 0.1)
    storage[dec.to(dev)] = rec.view(torch.uint8)
    layout = SimpleNamespace(head_k_dim=D, head_v_dim=D, num_value_heads=HV, num_key_heads=H, num_linear_layers=layers,
                             granularity=LS_GRAN, log_decay_bytes=record, num_granules=granules,
                             conv_dim=CONV_DIM, state_len=W - 1)
    return SimpleNamespace(storage=storage, dtype=torch.bfloat16, frame_bytes=LS_FRAME, head_payload_bytes=LS_HEAD,
                           page_size=LS_PAGE, payload_frame_table=payload.to(dev), decay_frame_table=decay.to(dev),
                           conv_frame_table=conv.to(dev), layout=layout)


def logstate_decode_bytes(counts, flush):
    """Algorithmic HBM bytes of one LogState recurrence launch: per sequence
    the bf16 work state, the replayed log rows (v' and gate per v-head, key
    per key head), the step's log row, the state write-back on flush steps,
    the q/k/v/gate/beta inputs and the output."""
    row = HV * (2 * D + 4) + H * 2 * D
    total = 0
    for n, f in zip(counts, flush):
        total += HV * LS_HEAD + n * row + row + (HV * LS_HEAD if f else 0)
        total += 2 * (2 * H * D + HV * D) + 2 * 2 * HV + 2 * HV * D
    return total


def logstate_gpu(dev, steps, warmup, B=256):
    """LogState decode (config 3 batch, replay counts pos % 16), the LogState
    chunked prefill (config 2 lengths at granularity 32 with frame-table
    states and the token log) and state reconstruction from logged pages."""
    from types import SimpleNamespace
    from logssms_amd.kernel.linear_attention import (
        ChunkLogIO, ChunkStateIO, chunk_gated_delta_rule_to_cache, conv_decode,
        fused_recurrent_gated_delta_rule_to_logstate, restore_log_state_chains)
    out = {}
    g = torch.Generator().manual_seed(9)
    pool = make_frame_pool(dev, 2 * B)
    cfg = SimpleNamespace(state_len=W - 1, conv_dim=CONV_DIM, num_k_heads=H, head_k_dim=D, num_v_heads=HV,
                          head_v_dim=D, key_dim=H * D, layer_idx=0)
    works = torch.arange(B, dtype=torch.int32, device=dev)
    logs = torch.arange(B, 2 * B, dtype=torch.int32, device=dev)
    pos = torch.randint(0, LS_PAGE, (B,), generator=g, dtype=torch.int32)
    counts = pos % 16
    flush = ((pos + 1) % 16 == 0).tolist()
    pos_d, counts_d = pos.to(dev), counts.to(dev)
    zeros = torch.zeros(B, dtype=torch.int32, device=dev)
    gran = (pos // LS_GRAN).to(dev)
    mixed = torch.randn(B, CONV_DIM, generator=g).to(torch.bfloat16).to(dev)
    gate = torch.randn(B, 1, HV, generator=g).to(torch.bfloat16).to(dev)
    beta = torch.randn(B, 1, HV, generator=g).to(torch.bfloat16).to(dev)
    weight = (torch.randn(CONV_DIM, 1, W, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    A_log = (-torch.rand(HV, generator=g)).to(dev)
    dt_bias = torch.zeros(HV, device=dev)
    o = torch.empty(B, 1, HV, D, dtype=torch.bfloat16, device=dev)
    qkv = conv_decode(mixed, weight, cfg, split_qkv=True, read_slots=works, write_slots=logs, pool=pool,
                      read_granules=zeros, write_granules=gran, work_slots=works)

    def conv_step():
        conv_decode(mixed, weight, cfg, split_qkv=True, read_slots=works, write_slots=logs, pool=pool,
                    read_granules=zeros, write_granules=gran, work_slots=works)

    def rec_step():
        fused_recurrent_gated_delta_rule_to_logstate(*qkv, gate, beta, A_log, dt_bias, pool, works, logs, pos_d, 0,
                                                      counts_d, out=o)

    # The conv is a 15 us kernel behind a host-side wrapper that takes longer
    # to run than the kernel: its steps are timed as replays of a HIP graph
    # of the call (eager steps would time the host).
    conv_timing = "HIP graph replay of the call"
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            conv_step()
        torch.cuda.current_stream().wait_stream(side)
        conv_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(conv_graph):
            conv_step()
        conv_ms = _time(conv_graph.replay, max(steps, 20), warmup)
    except RuntimeError as err:  # capture refused: time the eager call instead
        conv_timing = f"eager calls (graph capture failed: {err})"
        conv_ms = _time(conv_step, max(steps, 20), warmup)
    rec_ms = _time(rec_step, max(steps, 20), warmup)
    rb = logstate_decode_bytes(counts.tolist(), flush)
    cb = B * (CONV_DIM * 2 + 3 * (W - 1) * CONV_DIM * 2 + CONV_DIM * 2) + CONV_DIM * W * 2
    out["decode"] = {
        "config": f"{B} seqs at random page positions (replay counts pos % 16, mean {float(counts.float().mean()):.1f}), "
                  "bf16 frame storage, 64 KiB frames drawn at random, page 256, granularity 32",
        "ms": conv_ms + rec_ms, "recurrence_ms": rec_ms, "recurrence_bytes": rb,
        "recurrence_GB/s": rb / (rec_ms * 1e-3) / 1e9, "recurrence_frac_hbm": rb / (rec_ms * 1e-3) / PEAK_HBM,
        "conv_ms": conv_ms, "conv_timing": conv_timing, "conv_bytes": cb, "conv_GB/s": cb / (conv_ms * 1e-3) / 1e9}
    del qkv, o
    # state reconstruction: one task per sequence, base = its work slot, one full logged page
    tasks = [(int(works[i]), [(int(logs[i]), 0, LS_PAGE)], int(works[(i + 1) % B])) for i in range(0, B, 2)]
    rs_ms = _time(lambda: restore_log_state_chains(pool, tasks), max(steps // 2, 5), warmup)
    heads = len(tasks) * HV
    rs_bytes = heads * (2 * LS_HEAD + LS_PAGE * (2 * D + 4)) + len(tasks) * H * LS_PAGE * 2 * D
    rs_flop = heads * LS_PAGE * 2 * D * D
    out["restore"] = {"config": f"{len(tasks)} chains, base state + one logged page of {LS_PAGE} tokens, 32 v-heads",
                      "ms": rs_ms, "bytes": rs_bytes, "GB/s": rs_bytes / (rs_ms * 1e-3) / 1e9,
                      "flop": rs_flop, "TFLOP/s": rs_flop / (rs_ms * 1e-3) / 1e12}
    del pool
    torch.cuda.empty_cache()
    # prefill: config 2 lengths, frame-table states read from and written to work slots,
    # checkpoints every 1024 tokens, every token logged into its page's log slot
    lengths = [4096] * 4
    T = sum(lengths)
    pages = T // LS_PAGE
    n_int = T // LS_GRAN
    ppool = make_frame_pool(dev, 4 + pages + 16, seed=10)
    q = torch.nn.functional.normalize(torch.randn(1, T, H, D, generator=g), dim=-1).to(torch.bfloat16).to(dev)
    k = torch.nn.functional.normalize(torch.randn(1, T, H, D, generator=g), dim=-1).to(torch.bfloat16).to(dev)
    v = torch.randn(1, T, HV, D, generator=g).to(torch.bfloat16).to(dev)
    gg = (-torch.rand(1, T, HV, generator=g) * 0.1).to(dev)
    bb = torch.rand(1, T, HV, generator=g).to(dev)
    cu = torch.tensor([0, 4096, 8192, 12288, 16384], dtype=torch.int32, device=dev)
    work = torch.arange(4, dtype=torch.int32, device=dev)
    chunk_writes = torch.full((n_int,), -1, dtype=torch.int32)
    per_seq = 4096 // LS_GRAN
    for n in range(4):
        for j in range(1, 4):
            chunk_writes[n * per_seq + j * (1024 // LS_GRAN) - 1] = 4 + pages + 4 * n + j - 1
    tok = torch.arange(T)
    log_slots = (4 + tok // LS_PAGE).to(torch.int32).to(dev)
    offsets = (tok % LS_PAGE).to(torch.int32).to(dev)
    io = ChunkStateIO(storage=ppool.storage.view(torch.bfloat16), read_slots=work,
                      chunk_write_slots=chunk_writes.to(dev), final_write_slots=work,
                      payload_frames=ppool.payload_frame_table, frame_bytes=LS_FRAME, head_payload_bytes=LS_HEAD,
                      layer=0, num_layers=1, granularity=LS_GRAN, page_size=LS_PAGE)
    log = ChunkLogIO(slots=log_slots, token_offsets=offsets, decay_frames=ppool.decay_frame_table, gate=gg,
                     page_size=LS_PAGE, decay_record_bytes=ppool.layout.log_decay_bytes, num_key_heads=H)
    def prefill_step():  # as the LogState backend calls it: v' into the log only
        chunk_gated_delta_rule_to_cache(q, k, v, gg, bb, io, cu, chunk_size=LS_GRAN, log_io=log, return_v_new=False)

    pf_ms = _time(prefill_step, max(steps // 2, 5), warmup)
    flops = FLOP_PER_TOKEN_HEAD * T * HV
    out["prefill"] = {
        "config": "BASELINE config 2 lengths (4 x 4096), bf16 frame-table states in and out of work slots, "
                  "checkpoints every 1024 tokens, granularity 32, every token logged (v', key, gate); one step "
                  "= the chunk kernel (v' rows written into the log) + the key / gate log store",
        "ms": pf_ms, "tokens/s": T / (pf_ms * 1e-3), "step_tflops": flops / (pf_ms * 1e-3) / 1e12,
        "frac_mfma": flops / (pf_ms * 1e-3) / PEAK_MFMA_16BIT}
    del ppool, io, log
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="time budget of each CPU baseline leg (chunked prefill; naive prefill, decode and "
                         "verify get a share of it)")
    ap.add_argument("--only", choices=["all", "prefill", "decode", "verify", "norm", "layer", "logstate", "copy",
                                       "rmw", "mfma"],
                    default="all",
                    help="'copy' times a plain 512 MiB device copy (the calibration kernel for the "
                         "FETCH_SIZE / WRITE_SIZE counter passes); 'rmw' the in-place read-modify-write "
                         "ceiling sweep")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the GDN path would shard by sequences and v-heads, one process per GPU, with no "
              "collective on the path)", file=sys.stderr)
        sys.exit(2)
    dev = "cuda:0"
    torch.cuda.set_device(0)
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    result = {}
    extra = {"peaks": device_peaks(0)}
    cpu_info = {"cores": threads, "cpu_model": cpu_model()}
    if args.only == "copy":
        nbytes = 512 << 20
        src = torch.ones(nbytes // 4, device=dev)
        dst = torch.empty_like(src)
        ms = _time(lambda: dst.copy_(src), args.steps, args.warmup)
        print(json.dumps({"metric": "plain device copy GB/s", "value": 2 * nbytes / (ms * 1e-3) / 1e9,
                          "unit": "GB/s", "read_bytes": nbytes, "write_bytes": nbytes, "ms_per_step": ms}))
        return

    if args.only in ("all", "prefill"):
        inp = make_prefill(draw_device=dev)
        events = []
        step, state_pool, out = prefill_gpu(inp, dev, events)
        step_stats = {}
        ms = _time(step, args.steps, args.warmup, events, step_stats)
        chunk_ms = _kernel_ms(events)
        step2, _, _ = prefill_gpu(inp, dev, None, fused=False)
        extra["prefill_two_step_ms"] = _time(step2, args.steps, args.warmup)
        del step2
        T = inp["T"]
        flops = FLOP_PER_TOKEN_HEAD * T * HV
        achieved = flops / (chunk_ms * 1e-3)
        # HBM traffic of the fused chunk kernel (algorithmic): f16 q, k and the v columns of
        # mixed_qkv in, prepared fp32 g/beta in, o out, final states out, and each sequence's
        # conv window (its last W - 1 q/k input columns in, the whole window out)
        chunk_bytes = (T * (2 * H * D + HV * D) * 2 + 2 * T * HV * 4 + T * HV * D * 2 + inp["N"] * S_BYTES
                       + inp["N"] * (SC_BYTES + (W - 1) * 2 * H * D * 2))
        result.update(
            metric="GDN prefill tokens/s (% MFMA peak); decode state-update GB/s (% HBM peak)",
            value=T / (ms * 1e-3),
            unit="tokens/s",
            n_gpus=1, steps=args.steps, warmup=args.warmup, ms_per_step=ms,
            ms_per_step_stats={"median": ms, **step_stats,
                               "timing": "one event pair per step inside the synchronized region; median"},
            higher_is_better=True, scaling="weak", vs_baseline=None,
            dtype="bf16 in / fp16 MFMA operands / fp32 state",
            data="synthetic (seeded N(0,1) mixed_qkv, conv w N(0,0.02), zero initial state)",
            config={"workload": "BASELINE config 2: Qwen3-Next GDN layer prefill", "global_batch": inp["N"],
                    "seq_len": 4096, "heads_qk": H, "heads_v": HV, "head_dim": D, "chunk": C,
                    "parallelism": "single GPU"},
            roofline={"bound": "mfma", "achieved": achieved / 1e12, "peak": PEAK_MFMA_16BIT / 1e12,
                      "unit": "TFLOP/s", "frac": achieved / PEAK_MFMA_16BIT,
                      "traffic": _traffic("chunk_chain_kernel_fused_cfg2"),
                      "kernel": "chunk_chain_kernel<128, bf16, float, fused>", "kernel_ms": chunk_ms,
                      "algorithmic_flop_per_launch": flops, "algorithmic_bytes_per_launch": chunk_bytes},
        )
        extra["prefill_outside_chunk_kernel_ms"] = ms - chunk_ms  # the q/k pass and the launch gaps
        if args.only == "all":
            ceil = mfma_ceiling(dev)
            ceil["chunk_kernel_frac_of_ceiling"] = achieved / (ceil["best_TFLOP/s"] * 1e12)
            extra["mfma_ceiling"] = ceil
        if not args.no_cpu_baseline:
            chunked, naive = prefill_cpu_legs(inp, 4096, 256, args.cpu_seconds)
            result["cpu_baseline"] = {**chunked, **cpu_info, "kind": "port", "naive_recurrence": naive}
        del step, inp
        torch.cuda.empty_cache()
        inp4 = make_prefill_cfg4(draw_device=dev)
        ev4 = []
        step4, _, _ = prefill_gpu(inp4, dev, ev4)
        ms4 = _time(step4, max(args.steps // 2, 5), args.warmup, ev4)
        chunk4 = _kernel_ms(ev4)
        flops4 = FLOP_PER_TOKEN_HEAD * inp4["T"] * HV
        extra["prefill_cfg4"] = {
            "config": "BASELINE config 4: 64 seqs, lognormal lengths (median 1500, sigma 1.0, seed 4), "
                      "half from cached pool states + conv histories, checkpoints every 1024 tokens and at the end",
            "tokens": inp4["T"], "max_len": max(inp4["lengths"]), "checkpoints": inp4["checkpoints"],
            "ms": ms4, "tokens/s": inp4["T"] / (ms4 * 1e-3), "chunk_kernel_ms": chunk4,
            "chunk_tflops": flops4 / (chunk4 * 1e-3) / 1e12, "frac_mfma": flops4 / (chunk4 * 1e-3) / PEAK_MFMA_16BIT,
            "checkpoint_bytes": inp4["checkpoints"] * (S_BYTES + SC_BYTES),
            "chunk_traffic": _traffic("chunk_chain_kernel_fused_cfg4")}
        del step4, inp4
        torch.cuda.empty_cache()

    if args.only == "rmw":
        print(json.dumps({"rmw": rmw_sweep(dev, max(args.steps, 10), args.warmup)}))
        return
    if args.only == "mfma":
        print(json.dumps({"mfma_ceiling": mfma_ceiling(dev, max(args.steps, 10), args.warmup)}))
        return
    if args.only in ("all", "decode"):
        step, tensors = decode_gpu(dev)
        ms = _time(step, max(args.steps, 20), args.warmup)
        nb = decode_bytes(256)
        extra["decode"] = {"config": "BASELINE config 3 (256 seqs, in-place RMW of randperm pool slots)",
                           "ms": ms, "bytes": nb, "GB/s": nb / (ms * 1e-3) / 1e9,
                           "frac_hbm": nb / (ms * 1e-3) / PEAK_HBM, "traffic": _traffic("wave_kernel_decode_cfg3")}
        if not args.no_cpu_baseline:
            extra["decode"]["cpu_baseline"] = {**decode_cpu_leg(tensors, args.cpu_seconds / 2), **cpu_info,
                                               "kind": "port"}
        del step, tensors
        torch.cuda.empty_cache()
    if args.only == "all":
        extra["rmw_ceiling"] = rmw_sweep(dev, 10, 2)
    if args.only in ("all", "verify"):
        step, commit, tensors = verify_gpu(dev)
        ms = _time(step, max(args.steps, 20), args.warmup)
        nb = verify_bytes(64, 8)
        cms = _time(commit, max(args.steps, 20), args.warmup)
        cb = 64 * 2 * (S_BYTES + SC_BYTES)
        extra["verify"] = {"config": "BASELINE config 5 (64 seqs x 8 drafts, per-step states to slots)",
                           "ms": ms, "bytes": nb, "GB/s": nb / (ms * 1e-3) / 1e9,
                           "frac_hbm": nb / (ms * 1e-3) / PEAK_HBM, "traffic": _traffic("wave_kernel_verify_cfg5"),
                           "commit_ms": cms, "commit_GB/s": cb / (cms * 1e-3) / 1e9,
                           "commit_traffic": _traffic("commit_kernel_cfg5")}
        if not args.no_cpu_baseline:
            extra["verify"]["cpu_baseline"] = {**verify_cpu_leg(tensors, args.cpu_seconds / 2), **cpu_info,
                                               "kind": "port"}
        del step, commit, tensors
        torch.cuda.empty_cache()
    if args.only in ("all", "norm"):
        step, nb = norm_gpu(dev)
        ms = _time(step, max(args.steps, 20), args.warmup)
        extra["rms_norm_gated"] = {"config": "config 2 core output: 16384 tokens x 32 v-heads x 128, bf16, "
                                             "gate a column slice of a 2x wider projection output",
                                   "ms": ms, "bytes": nb, "GB/s": nb / (ms * 1e-3) / 1e9,
                                   "frac_hbm": nb / (ms * 1e-3) / PEAK_HBM, "traffic": _traffic("norm_vec_kernel_cfg2")}
    if args.only in ("all", "layer"):
        step, parts = layer_gpu(dev)
        ms = _time(step, max(args.steps // 2, 5), args.warmup)
        stages = {k: _time(fn, max(args.steps // 2, 5), args.warmup) for k, fn in parts().items()}
        T = 4 * 4096
        extra["gated_delta_layer"] = {
            "config": "GatedDeltaNet layer, hidden 2048, config 2 batch (4 x 4096): in_proj_qkvz/in_proj_ba GEMMs, "
                      "GDN prefill on their strided column slices, gated RMS norm, out_proj GEMM",
            "ms": ms, "tokens/s": T / (ms * 1e-3), "stage_ms": stages}
        del step, parts
        torch.cuda.empty_cache()
    if args.only in ("all", "logstate"):
        extra["logstate"] = logstate_gpu(dev, args.steps, args.warmup)
    if not result:
        keys = [k for k in ("decode", "verify", "rms_norm_gated") if k in extra]
        if not keys:  # --only layer / logstate
            print(json.dumps({"extra": extra}))
            return
        key = keys[0]
        e = extra[key]
        result.update(metric=f"GDN {key} GB/s", value=e["GB/s"], unit="GB/s", n_gpus=1,
                      steps=args.steps, warmup=args.warmup, ms_per_step=e["ms"], higher_is_better=True,
                      scaling="weak", vs_baseline=None, dtype="bf16 io / fp32 state", data="synthetic",
                      config={"workload": e["config"]},
                      roofline={"bound": "hbm", "achieved": e["GB/s"], "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                                "frac": e["frac_hbm"], "traffic": e.get("traffic")})
    result["extra"] = extra
    print(json.dumps(result))


if __name__ == "__main__":
    main()
