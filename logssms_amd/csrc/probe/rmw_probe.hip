// Bandwidth probe for the HBM-bound kernels: an in-place read-modify-write
// stream (x <- a x over 16-byte vectors), the access mix of the decode state
// update (each 64 KiB of state read once and written back once).  Not part of
// the GDN path and not in libgdn_mi355x.so: it builds into the bench-only
// libgdn_probe.so, which bench.py --only rmw uses to measure the
// 1-read:1-write ceiling of the box that the decode / verify fractions are
// read against, and a store-only stream (the write ceiling for verify's
// per-step state stores).
//
// It also holds the matrix-core ceiling probe: gdn_probe_mfma runs independent
// 16x16x32 f16 MFMA chains on every CU, the dense-f16 rate the chunk kernel's
// MFMA fraction can be read against besides the published peak (under a
// sustained MFMA load the engine clock drops below its 2.4 GHz maximum).
//
// int gdn_probe_rmw(void* buf, int64_t bytes, int64_t block_bytes,
//                   int loads_in_flight, int nontemporal, void* stream):
// buf[i] <- buf[i] * 1.0 in place over `bytes` (16-byte vectors), each block
// owning `block_bytes` consecutive bytes and each lane keeping
// `loads_in_flight` (1, 2, 4, 8, 16) 16-byte loads in flight before its
// stores, optionally non-temporal; loads_in_flight 0: a store-only stream
// (buf[i] <- 1.0).  Returns 0, or an error code with gdn_probe_last_error().
#include <cstdarg>

#include "../common.hpp"

namespace gdn {

// This library's own error store (hidden: the product library has its own).
static thread_local char g_probe_error[512] = "";

__attribute__((visibility("hidden"))) void set_error(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_probe_error, sizeof(g_probe_error), fmt, args);
  va_end(args);
}

__attribute__((visibility("hidden"))) int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return GDN_OK;
  set_error("%s: %s", what, hipGetErrorString(err));
  return GDN_ERR_HIP;
}

namespace {

typedef float f4v __attribute__((ext_vector_type(4)));

// Each block owns `per_block` consecutive vectors; each lane keeps U loads in
// flight before its stores.
template <int U, bool NT>
__global__ __launch_bounds__(256) void rmw_kernel(f4v* buf, int64_t n_vec, int64_t per_block, float a) {
  const int64_t begin = static_cast<int64_t>(blockIdx.x) * per_block;
  const int64_t end = begin + per_block < n_vec ? begin + per_block : n_vec;
  for (int64_t i0 = begin + threadIdx.x; i0 < end; i0 += 256 * U) {
    f4v v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + 256 * u;
      if (i < end) v[u] = NT ? __builtin_nontemporal_load(buf + i) : buf[i];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + 256 * u;
      if (i < end) {
        if (NT) __builtin_nontemporal_store(v[u] * a, buf + i);
        else buf[i] = v[u] * a;
      }
    }
  }
}

// Store-only stream: buf[i] <- (a, a, a, a), 4 stores per lane per pass.
template <bool NT>
__global__ __launch_bounds__(256) void store_kernel(f4v* buf, int64_t n_vec, int64_t per_block, float a) {
  const int64_t begin = static_cast<int64_t>(blockIdx.x) * per_block;
  const int64_t end = begin + per_block < n_vec ? begin + per_block : n_vec;
  const f4v v = {a, a, a, a};
  for (int64_t i0 = begin + threadIdx.x; i0 < end; i0 += 256 * 4) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t i = i0 + 256 * u;
      if (i < end) {
        if (NT) __builtin_nontemporal_store(v, buf + i);
        else buf[i] = v;
      }
    }
  }
}

typedef _Float16 h8v __attribute__((ext_vector_type(8)));

// Each wave runs `iters` rounds of 8 independent 16x16x32 f16 MFMAs (fp32
// accumulators) and writes one value per lane so nothing is dead code.
__global__ __launch_bounds__(512) void mfma_kernel(float* out, int iters) {
  const int lane = threadIdx.x & 63;
  h8v a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = static_cast<_Float16>(0.001f * (lane + i));
    b[i] = static_cast<_Float16>(0.002f * (lane - i));
  }
  f4v acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f4v{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[i], 0, 0, 0);
  }
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) sum += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
  out[static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = sum;
}

template <int U>
int launch_rmw(f4v* buf, int64_t n_vec, int64_t per_block, int nontemporal, hipStream_t s) {
  const int64_t blocks = (n_vec + per_block - 1) / per_block;
  if (blocks > 0x7fffffff) {
    set_error("gdn_probe_rmw: grid too large");
    return GDN_ERR_INVALID;
  }
  if (nontemporal)
    hipLaunchKernelGGL((rmw_kernel<U, true>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, buf, n_vec,
                       per_block, 1.0f);
  else
    hipLaunchKernelGGL((rmw_kernel<U, false>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, buf, n_vec,
                       per_block, 1.0f);
  return GDN_LAUNCH_CHECK("gdn_probe_rmw launch");
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_probe_rmw(void* buf, int64_t bytes, int64_t block_bytes, int loads_in_flight, int nontemporal,
                             void* stream) {
  using namespace gdn;
  GDN_REQUIRE(buf && bytes > 0 && bytes % 16 == 0 && block_bytes >= 16 && block_bytes % 16 == 0,
              "gdn_probe_rmw: bad sizes");
  GDN_REQUIRE((reinterpret_cast<uintptr_t>(buf) & 15) == 0, "gdn_probe_rmw: buffer not 16-byte aligned");
  auto* v = static_cast<f4v*>(buf);
  const int64_t n = bytes / 16, per = block_bytes / 16;
  auto s = static_cast<hipStream_t>(stream);
  switch (loads_in_flight) {
    case 0: {
      const int64_t blocks = (n + per - 1) / per;
      GDN_REQUIRE(blocks <= 0x7fffffff, "gdn_probe_rmw: grid too large");
      if (nontemporal)
        hipLaunchKernelGGL((store_kernel<true>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, v, n, per, 1.0f);
      else
        hipLaunchKernelGGL((store_kernel<false>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, v, n, per, 1.0f);
      return GDN_LAUNCH_CHECK("gdn_probe_rmw launch");
    }
    case 1: return launch_rmw<1>(v, n, per, nontemporal, s);
    case 2: return launch_rmw<2>(v, n, per, nontemporal, s);
    case 4: return launch_rmw<4>(v, n, per, nontemporal, s);
    case 8: return launch_rmw<8>(v, n, per, nontemporal, s);
    case 16: return launch_rmw<16>(v, n, per, nontemporal, s);
    default:
      set_error("gdn_probe_rmw: loads_in_flight %d not in {0, 1, 2, 4, 8, 16}", loads_in_flight);
      return GDN_ERR_UNSUPPORTED;
  }
}

// Dense f16 matrix-core probe: `blocks` workgroups of `threads` (64..512,
// a multiple of 64) threads, each wave 8 x iters MFMAs of 16 x 16 x 32
// (16384 flop each); out holds blocks * threads floats.
extern "C" int gdn_probe_mfma(float* out, int64_t blocks, int threads, int iters, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(out && blocks > 0 && blocks <= 0x7fffffff && threads >= 64 && threads <= 512 && threads % 64 == 0 &&
                  iters > 0,
              "gdn_probe_mfma: bad sizes");
  hipLaunchKernelGGL(mfma_kernel, dim3(static_cast<unsigned>(blocks)), dim3(threads), 0,
                     static_cast<hipStream_t>(stream), out, iters);
  return GDN_LAUNCH_CHECK("gdn_probe_mfma launch");
}

extern "C" const char* gdn_probe_last_error(void) { return gdn::g_probe_error; }
