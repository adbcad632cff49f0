"""Per-wave barrier timestamps of the fused chunk kernel (measurement only).

    python3 logssms_amd/csrc/probe/chunk_stamps.py build   # CPU: hipcc, after the product build
    python3 logssms_amd/csrc/probe/chunk_stamps.py run     # one MI355X

``build`` copies ``chunk_chain.hip`` with an ``s_memtime`` stamp on each side
of every loop barrier (M: the end of a chunk's first phase, B: the end of its
second) for the first 4 workgroups and 64 chunks, plus each wave's HW_ID
register, and links it with the other product objects (``_build/gdn``) into
``logssms_amd/libgdn_stamps.so``, a library of its own that the product never
loads.  ``run`` drives config 2's fused prefill (``bench.prefill_gpu``) through
that library and prints, per role, the cycles from one barrier's release to
the wave's arrival at the next (work) and from its arrival to the release
(slack), and which wave arrives last.  Lane 0 of each wave writes its stamps
with a vector store; the stamps add a few instructions per barrier.
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
BUILD = os.path.join(REPO, "_build", "stamps")
LIB = os.path.join(PKG, "libgdn_stamps.so")
BLOCKS, WAVES, CHUNKS, SLOTS = 4, 12, 64, 8
ROLES = ["chain 0", "chain 1", "chain 2", "chain 3", "inverse 4", "inverse 5", "tiles 6", "tiles 7",
         "tiles 8", "tiles 9", "conv 10", "conv 11"]

MACRO = r"""
__device__ uint64_t g_stamps[%d * %d * %d * %d];
// slot k of (block, wave, chunk c): 1 / 2 before / after M, 3 / 4 before / after B
#define STAMP(k)                                                                  \
  do {                                                                            \
    if (blockIdx.x < %d && c < %d) {                                               \
      const uint64_t t_ = __builtin_amdgcn_s_memtime();                           \
      if (lane == 0) g_stamps[((blockIdx.x * %d + wave) * %d + c) * %d + (k)] = t_; \
    }                                                                             \
  } while (0)
""" % (BLOCKS, WAVES, CHUNKS, SLOTS, BLOCKS, CHUNKS, WAVES, CHUNKS, SLOTS)

EXPORT = r"""
extern "C" int gdn_stamps_read(void* host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(gdn::g_stamps), sizeof(gdn::g_stamps)) == hipSuccess ? 0 : 1;
}
// The SIMD of each wave of a 768-thread workgroup that fills a CU's LDS, as
// the chunk kernel's does: HW_ID bits 5:4 of every wave's lane 0.
__global__ __launch_bounds__(768) void stamps_hwid_kernel(uint32_t* out) {
  extern __shared__ uint32_t fill[];
  if (threadIdx.x == 0) fill[0] = 0;
  if ((threadIdx.x & 63) == 0)
    out[blockIdx.x * 12 + (threadIdx.x >> 6)] = static_cast<uint32_t>(__builtin_amdgcn_s_getreg(63492)) >> 4 & 3;
}
extern "C" int gdn_stamps_simds(void* out_dev, int blocks, void* stream) {
  hipLaunchKernelGGL(stamps_hwid_kernel, dim3(blocks), dim3(768), 143456, static_cast<hipStream_t>(stream),
                     static_cast<uint32_t*>(out_dev));
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
"""


def instrument(src):
    """The stamped source: STAMP around each loop barrier (the kernel's own
    `wave` and `lane`: wave w runs on the SIMD HW_ID reports)."""
    anchor = "constexpr int kC = 64;"
    if src.count(anchor) != 1:
        raise SystemExit("chunk_stamps: chunk_chain.hip has no unique '%s'" % anchor)
    out = src.replace(anchor, MACRO + anchor, 1)
    m, b = "lds_barrier();  // M(c)", "lds_barrier();  // B(c+1)"
    nm, nb = out.count(m), out.count(b)
    if nm != 4 or nb != 4:
        raise SystemExit("chunk_stamps: expected 4 loop barriers of each kind, found %d M and %d B" % (nm, nb))
    out = out.replace(m, "STAMP(1); " + m + "\n      STAMP(2);")
    out = out.replace(b, "STAMP(3); " + b + "\n      STAMP(4);")
    # the fused conv waves' peeled last chunk
    tail = re.compile(r"(\n(\s*)snapshot_windows\(\);\n\s*lds_barrier\(\);  // M\(nchunks - 1\)\n"
                      r"\s*lds_barrier\(\);  // B\(nchunks\))")
    found = tail.search(out)
    if not found:
        raise SystemExit("chunk_stamps: the conv waves' peeled last chunk was not found")
    ind = found.group(2)
    out = out[:found.start()] + (
        "\n%s{\n%sconst int64_t c = nchunks - 1;\n%ssnapshot_windows();\n%sSTAMP(1); "
        "lds_barrier();  // M(nchunks - 1)\n%sSTAMP(2); STAMP(3); lds_barrier();  // B(nchunks)\n%sSTAMP(4);\n%s}"
        % (ind, ind, ind, ind, ind, ind, ind)) + out[found.end():]
    return out + EXPORT


def build():
    src = open(os.path.join(CSRC, "chunk_chain.hip")).read()
    os.makedirs(BUILD, exist_ok=True)
    stamped = os.path.join(BUILD, "chunk_chain_stamped.hip")
    open(stamped, "w").write(instrument(src))
    objs = os.path.join(REPO, "_build", "gdn")
    others = sorted(os.path.join(objs, f) for f in os.listdir(objs)
                    if f.endswith(".o") and f != "chunk_chain.o")
    if not others:
        raise SystemExit("chunk_stamps: build the product first (make -C logssms_amd/csrc)")
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    flags = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-munsafe-fp-atomics", "-ffp-contract=fast", "-I", CSRC]
    obj = os.path.join(BUILD, "chunk_chain_stamped.o")
    subprocess.run([hipcc] + flags + ["-c", stamped, "-o", obj], check=True)
    subprocess.run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", LIB] + others + [obj], check=True)
    # the stamps must leave the measured instantiation (d_k 128, bf16, fp32
    # state, fused) without spills
    asm = os.path.join(BUILD, "chunk_chain_stamped.s")
    subprocess.run([hipcc] + flags + ["--cuda-device-only", "-S", stamped, "-o", asm], check=True)
    meta = open(asm).read()
    at = meta.find(".name:           _ZN3gdn12_GLOBAL__N_118chunk_chain_kernelILi128ENS_4bf16EfLb1ELb0E")
    spill = re.search(r"\.vgpr_spill_count:\s+(\d+)", meta[at:]) if at >= 0 else None
    if spill is None or int(spill.group(1)) != 0:
        raise SystemExit("chunk_stamps: the stamped fused kernel spills vector registers (or was not found)")
    print("built", LIB)


def run():
    import numpy as np
    import torch
    sys.path.insert(0, REPO)
    import bench
    from logssms_amd import _lib
    _lib._lib = None
    _lib.LIB_PATH = LIB
    dev = "cuda:0"
    inp = bench.make_prefill(draw_device=dev)
    step, _, _ = bench.prefill_gpu(inp, dev, [])
    for _ in range(5):
        step()
    torch.cuda.synchronize()
    buf = np.zeros(BLOCKS * WAVES * CHUNKS * SLOTS, dtype=np.uint64)
    if ctypes.CDLL(LIB).gdn_stamps_read(buf.ctypes.data_as(ctypes.c_void_p)) != 0:
        raise SystemExit("chunk_stamps: reading the stamps failed")
    a = buf.reshape(BLOCKS, WAVES, CHUNKS, SLOTS).astype(np.int64)
    simds = torch.zeros(BLOCKS * WAVES, dtype=torch.int32, device=dev)
    if ctypes.CDLL(LIB).gdn_stamps_simds(ctypes.c_void_p(simds.data_ptr()), BLOCKS,
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) != 0:
        raise SystemExit("chunk_stamps: the HW_ID probe failed")
    simd = simds.view(BLOCKS, WAVES).cpu().tolist()
    groups = sorted({tuple(tuple(w for w in range(WAVES) if s[w] == s[v]) for v in range(4)) for s in simd})
    print("waves sharing a SIMD (HW_ID of a 768-thread workgroup filling the LDS):", groups)
    phase_a, phase_b, rows = [], [], {w: [[], [], [], []] for w in range(WAVES)}
    last_m, last_b = [0] * WAVES, [0] * WAVES
    for blk in range(BLOCKS):
        for c in range(2, 62):
            rel_b0 = a[blk, :, c - 1, 4].min()
            rel_m = a[blk, :, c, 2].min()
            rel_b1 = a[blk, :, c, 4].min()
            phase_a.append(rel_m - rel_b0)
            phase_b.append(rel_b1 - rel_m)
            last_m[int(a[blk, :, c, 1].argmax())] += 1
            last_b[int(a[blk, :, c, 3].argmax())] += 1
            for w in range(WAVES):
                rows[w][0].append(a[blk, w, c, 1] - a[blk, w, c - 1, 4])
                rows[w][1].append(rel_m - a[blk, w, c, 1])
                rows[w][2].append(a[blk, w, c, 3] - a[blk, w, c, 2])
                rows[w][3].append(rel_b1 - a[blk, w, c, 3])
    mean = lambda v: float(np.mean(v))
    print("cycles per chunk (s_memtime): phase A %.0f, phase B %.0f, chunk %.0f  (%d workgroups x 60 chunks)"
          % (mean(phase_a), mean(phase_b), mean(phase_a) + mean(phase_b), BLOCKS))
    print("| wave | work A | slack at M | work B | slack at B | last at M | last at B |")
    print("|---|---|---|---|---|---|---|")
    for w in range(WAVES):
        r = rows[w]
        print("| %s | %.0f | %.0f | %.0f | %.0f | %d | %d |"
              % (ROLES[w], mean(r[0]), mean(r[1]), mean(r[2]), mean(r[3]), last_m[w], last_b[w]))


if __name__ == "__main__":
    if len(sys.argv) != 2 or sys.argv[1] not in ("build", "run"):
        raise SystemExit(__doc__)
    {"build": build, "run": run}[sys.argv[1]]()
