// gdn_prefill_fused_noalloc: the two-launch fused prefill (gdn_prefill_qk,
// then gdn_prefill_fused, which also writes the conv windows) with its
// staging -- the f16 q/k
// MFMA operands and the head-major prepared gates that pass from the first
// launch to the second -- in a file-scope device array instead of buffers
// the caller allocates.  For callers that cannot allocate device memory
// (code under HIP graph capture, serving loops that forbid allocation).
//
// The array lives in this code object, one copy per GPU the library runs
// on, held until the process ends.  Its device address comes from
// hipGetSymbolAddress, resolved once per device with that device current;
// the host-side name `scratch` is not a device address and is never passed
// to a kernel.  Every call on a device shares that device's array: calls
// that overlap on one GPU (different streams, no ordering) race.  Nothing in
// it needs clearing -- the q/k launch writes every row and gate the chunk
// kernel later reads (packed rows below cu[N]).
#include <mutex>

#include "common.hpp"

namespace gdn {
namespace {

constexpr size_t kScratchBytes = size_t(256) << 20;  // 256 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's `scratch`, resolved on first use.
int scratch_address(void** out) {
  int dev = -1;
  int rc = hip_status(hipGetDevice(&dev), "gdn_prefill_fused_noalloc: hipGetDevice");
  if (rc != GDN_OK) return rc;
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("gdn_prefill_fused_noalloc: device %d outside the %d supported", dev, kMaxDevices);
    return GDN_ERR_INVALID;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    rc = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "gdn_prefill_fused_noalloc: hipGetSymbolAddress");
    if (rc != GDN_OK) return rc;
    if (!p) {
      set_error("gdn_prefill_fused_noalloc: null scratch address");
      return GDN_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return GDN_OK;
}

constexpr int64_t align256(int64_t bytes) { return (bytes + 255) / 256 * 256; }

}  // namespace
}  // namespace gdn

extern "C" int64_t gdn_prefill_noalloc_scratch_bytes(void) { return static_cast<int64_t>(gdn::kScratchBytes); }

extern "C" int gdn_prefill_fused_noalloc(
    const void* mixed, int64_t row_stride, int io_dtype, const void* weight, int kernel_width, const void* cu_seqlens,
    int cu_dtype, int64_t num_seqs, int64_t total_tokens, int64_t H, int64_t HV, int64_t dk, int64_t dv,
    void* conv_state, int64_t conv_slot_stride, int64_t conv_layer_stride, const void* gate, int64_t gate_row_stride,
    int64_t gate_head_stride, int gate_dtype, const void* beta, int64_t beta_row_stride, int64_t beta_head_stride,
    int beta_dtype, const void* A_log, int a_dtype, const void* dt_bias, int dt_dtype, void* state, int state_dtype,
    int64_t slot_stride, int64_t layer_stride, int64_t head_stride, int64_t layer, const void* baseline_slots,
    int baseline_dtype, const void* chunk_write_slots, int chunk_write_dtype, const void* snapshot_rows,
    int snapshot_rows_dtype, const void* snapshot_slots, int snapshot_slots_dtype, int64_t snapshot_count, void* out,
    float scale, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(num_seqs >= 1 && total_tokens >= 0 && H > 0 && HV > 0 && HV % H == 0 && dk > 0 && dv > 0 &&
                  snapshot_count >= 0,
              "gdn_prefill_fused_noalloc: bad sizes");
  // staging: q, k [T, H, dk] f16, then g, beta [HV, T] fp32, each 256-byte aligned
  const int64_t qk_bytes = align256(total_tokens * H * dk * 2);
  const int64_t gate_bytes = align256(total_tokens * HV * 4);
  const int64_t need = 2 * qk_bytes + 2 * gate_bytes;
  if (need > static_cast<int64_t>(kScratchBytes)) {
    set_error("gdn_prefill_fused_noalloc: %lld tokens need %lld scratch bytes, more than the %lld this entry point "
              "holds; use gdn_prefill_qk + gdn_prefill_fused with caller-allocated staging",
              (long long)total_tokens, (long long)need, (long long)kScratchBytes);
    return GDN_ERR_INVALID;
  }
  if (total_tokens == 0) return GDN_OK;
  void* base = nullptr;
  int rc = scratch_address(&base);
  if (rc != GDN_OK) return rc;
  unsigned char* bytes = static_cast<unsigned char*>(base);
  void* q = bytes;
  void* k = bytes + qk_bytes;
  float* g = reinterpret_cast<float*>(bytes + 2 * qk_bytes);
  float* b = reinterpret_cast<float*>(bytes + 2 * qk_bytes + gate_bytes);
  rc = gdn_prefill_qk(mixed, row_stride, io_dtype, weight, kernel_width, cu_seqlens, cu_dtype, num_seqs,
                      total_tokens, H, dk, conv_state, conv_slot_stride, conv_layer_stride, layer, baseline_slots,
                      baseline_dtype, q, k, GDN_F16, HV, gate, gate_row_stride, gate_head_stride, gate_dtype, beta,
                      beta_row_stride, beta_head_stride, beta_dtype, A_log, a_dtype, dt_bias, dt_dtype, g, b, stream);
  if (rc != GDN_OK) return rc;
  rc = gdn_prefill_fused(q, k, mixed, row_stride, io_dtype, weight, kernel_width, cu_seqlens, cu_dtype, num_seqs,
                         total_tokens, H, HV, dk, dv, conv_state, conv_slot_stride, conv_layer_stride, g, b, state,
                         state_dtype, slot_stride, layer_stride, head_stride, layer, baseline_slots, baseline_dtype,
                         chunk_write_slots, chunk_write_dtype, nullptr, 0, snapshot_rows, snapshot_rows_dtype,
                         snapshot_slots, snapshot_slots_dtype, snapshot_count, out, scale, stream);
  return rc;
}
