"""Per-head timestamps of the LogState decode recurrence (measurement only).

    python3 logssms_amd/csrc/probe/logstate_stamps.py build   # CPU: hipcc, after the product build
    python3 logssms_amd/csrc/probe/logstate_stamps.py run     # one MI355X

``build`` copies ``logstate.hip`` with ``s_memtime`` stamps in the head loops
of ``logstate_decode_kernel`` (first 4 blocks, first 8 heads of each): at the
head's start, after the compute waves have read and decayed the work state,
after the replay products, on both sides of the MID barrier (the replayed
rows consumed) and of the END barrier (the next head resident), and links it
with the other product objects (``_build/gdn``) into
``logssms_amd/libgdn_lsstamps.so``, a library of its own that the product
never loads.  ``run`` drives the LogState decode leg of ``bench.py``
(``bench.logstate_gpu``: 256 sequences, replay counts pos mod 16) through it
and prints, per wave role, the mean cycles from the head's start to each
stamp over heads 1-3 of the 4 blocks.
"""

import ctypes
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.dirname(HERE)
PKG = os.path.dirname(CSRC)
REPO = os.path.dirname(PKG)
BUILD = os.path.join(REPO, "_build", "lsstamps")
LIB = os.path.join(PKG, "libgdn_lsstamps.so")
BLOCKS, WAVES, HEADS, SLOTS = 4, 3, 8, 8

MACRO = r"""
__device__ uint64_t g_lsstamps[%d * %d * %d * %d];
#define LSTAMP(k)                                                                   \
  do {                                                                              \
    if (blockIdx.x < %d && hi < %d) {                                                \
      const uint64_t t_ = __builtin_amdgcn_s_memtime();                             \
      if ((threadIdx.x & 63) == 0)                                                  \
        g_lsstamps[((blockIdx.x * %d + (threadIdx.x >> 6)) * %d + hi) * %d + (k)] = t_; \
    }                                                                               \
  } while (0)
""" % (BLOCKS, WAVES, HEADS, SLOTS, BLOCKS, HEADS, WAVES, HEADS, SLOTS)

EXPORT = r"""
extern "C" int gdn_lsstamps_read(void* host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(gdn::g_lsstamps), sizeof(gdn::g_lsstamps)) == hipSuccess ? 0 : 1;
}
"""

# (text, replacement) pairs, each text exactly once in logstate.hip
EDITS = [
    # loading wave: head start, MID and END
    ("    for (uint32_t hi = 0; hi < hpb; ++hi) {\n      const bool more = hi + 1 < hpb;",
     "    for (uint32_t hi = 0; hi < hpb; ++hi) {\n      LSTAMP(0);\n      const bool more = hi + 1 < hpb;"),
    ("      lds_barrier();  // MID: the compute waves have read the replayed rows\n",
     "      LSTAMP(3); lds_barrier();  // MID: the compute waves have read the replayed rows\n      LSTAMP(4);\n"),
    ("      wait_all();\n      lds_barrier();  // END: the next head is resident\n",
     "      wait_all();\n      LSTAMP(5); lds_barrier();  // END: the next head is resident\n      LSTAMP(6);\n"),
    # compute waves
    ("  for (uint32_t hi = 0; hi < hpb; ++hi) {\n    const uint32_t h = h0 + hi;",
     "  for (uint32_t hi = 0; hi < hpb; ++hi) {\n    LSTAMP(0);\n    const uint32_t h = h0 + hi;"),
    ("    if (n > 0) {\n      // T += V'^T K:",
     "    LSTAMP(1);\n    if (n > 0) {\n      // T += V'^T K:"),
    ("    lds_barrier();  // MID: the replayed rows are consumed\n",
     "    LSTAMP(2); LSTAMP(3); lds_barrier();  // MID: the replayed rows are consumed\n    LSTAMP(4);\n"),
    ("    lds_barrier();  // END: the next head is resident\n",
     "    LSTAMP(5); lds_barrier();  // END: the next head is resident\n    LSTAMP(6);\n"),
]


def instrument(src):
    anchor = "constexpr int kReplayWindow = 16;"
    if src.count(anchor) != 1:
        raise SystemExit("logstate_stamps: logstate.hip has no unique '%s'" % anchor)
    out = src.replace(anchor, MACRO + anchor, 1)
    for old, new in EDITS:
        if out.count(old) != 1:
            raise SystemExit("logstate_stamps: expected one %r in logstate.hip" % old[:60])
        out = out.replace(old, new)
    return out + EXPORT


def build():
    src = open(os.path.join(CSRC, "logstate.hip")).read()
    os.makedirs(BUILD, exist_ok=True)
    stamped = os.path.join(BUILD, "logstate_stamped.hip")
    open(stamped, "w").write(instrument(src))
    objs = os.path.join(REPO, "_build", "gdn")
    others = sorted(os.path.join(objs, f) for f in os.listdir(objs) if f.endswith(".o") and f != "logstate.o")
    if not others:
        raise SystemExit("logstate_stamps: build the product first (make -C logssms_amd/csrc)")
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    flags = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-munsafe-fp-atomics", "-ffp-contract=fast", "-I", CSRC]
    obj = os.path.join(BUILD, "logstate_stamped.o")
    subprocess.run([hipcc] + flags + ["-c", stamped, "-o", obj], check=True)
    subprocess.run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", LIB] + others + [obj], check=True)
    # the stamps must leave the measured kernel (d_k = d_v = 128, bf16) without spills
    asm = os.path.join(BUILD, "logstate_stamped.s")
    subprocess.run([hipcc] + flags + ["--cuda-device-only", "-S", stamped, "-o", asm], check=True)
    meta = open(asm).read()
    at = meta.find(".name:           _ZN3gdn12_GLOBAL__N_122logstate_decode_kernelILi128ELi128ENS_4bf16E")
    spill = re.search(r"\.vgpr_spill_count:\s+(\d+)", meta[at:]) if at >= 0 else None
    if spill is None or int(spill.group(1)) != 0:
        raise SystemExit("logstate_stamps: the stamped decode kernel spills vector registers (or was not found)")
    print("built", LIB)


def run():
    import numpy as np
    import torch
    sys.path.insert(0, REPO)
    import bench
    from logssms_amd import _lib
    _lib._lib = None
    _lib.LIB_PATH = LIB
    bench.logstate_gpu("cuda:0", 5, 2)
    torch.cuda.synchronize()
    buf = np.zeros(BLOCKS * WAVES * HEADS * SLOTS, dtype=np.uint64)
    if ctypes.CDLL(LIB).gdn_lsstamps_read(buf.ctypes.data_as(ctypes.c_void_p)) != 0:
        raise SystemExit("logstate_stamps: reading the stamps failed")
    a = buf.reshape(BLOCKS, WAVES, HEADS, SLOTS).astype(np.int64)
    names = {0: "compute wave 0", 1: "compute wave 1", 2: "loading wave"}
    labels = {1: "state read + decayed", 2: "replay done", 3: "at MID", 4: "MID released", 5: "at END",
              6: "END released"}
    print("cycles (s_memtime) from a head's start, mean over heads 1-3 of blocks 0-3:")
    for w in range(WAVES):
        keys = (3, 4, 5, 6) if w == 2 else (1, 2, 3, 4, 5, 6)
        vals = {k: float(np.mean([a[b, w, h, k] - a[b, w, h, 0] for b in range(BLOCKS) for h in range(1, 4)]))
                for k in keys}
        print("  %s: " % names[w] + ", ".join("%s %.0f" % (labels[k], vals[k]) for k in keys))


if __name__ == "__main__":
    if len(sys.argv) != 2 or sys.argv[1] not in ("build", "run"):
        raise SystemExit(__doc__)
    {"build": build, "run": run}[sys.argv[1]]()
