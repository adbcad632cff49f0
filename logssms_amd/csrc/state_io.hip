// State-pool row movement: store_state, Marconi copy/zero, verify commit.
//
// All of these are pure HBM streaming (no arithmetic).  A row (one slot of
// one layer: 2 MiB of fp32 state at Qwen3-Next shape, or a 48 KiB conv
// window) is split into 64 KiB pieces so that a 512-row store keeps the whole
// chip busy, instead of one 32-lane warp per 2 MiB row as in
// csrc/jit/store.cu:152-182.  Each lane moves 16 bytes per access (global
// dwordx4), the widest coalesced access a CDNA4 lane issues.
#include <algorithm>
#include <initializer_list>

#include "common.hpp"

namespace gdn {
namespace {

constexpr int kThreads = 256;
constexpr int64_t kPieceBytes = 64 * 1024;

template <class V>
__device__ __forceinline__ void copy_span(char* dst, const char* src, int64_t bytes) {
  const int64_t n = bytes / static_cast<int64_t>(sizeof(V));
  V* d = reinterpret_cast<V*>(dst);
  const V* s = reinterpret_cast<const V*>(src);
  for (int64_t i = threadIdx.x; i < n; i += kThreads) d[i] = s[i];
}

template <class V>
__device__ __forceinline__ void zero_span(char* dst, int64_t bytes) {
  const int64_t n = bytes / static_cast<int64_t>(sizeof(V));
  V* d = reinterpret_cast<V*>(dst);
  V z{};
  for (int64_t i = threadIdx.x; i < n; i += kThreads) d[i] = z;
}

// grid: (pieces per segment, segments, pairs)
template <class V>
__global__ __launch_bounds__(kThreads) void copy_rows_kernel(char* dst_base, int64_t dst_row_stride,
                                                             const void* dst_idx, int dst_is64,
                                                             const char* src_base, int64_t src_row_stride,
                                                             const void* src_idx, int src_is64,
                                                             int64_t segment_bytes, int64_t segment_stride) {
  const int64_t pair = blockIdx.z;
  const int64_t d = dst_idx ? load_index(dst_idx, pair, dst_is64) : pair;
  const int64_t s = src_idx ? load_index(src_idx, pair, src_is64) : pair;
  if (d < 0 || s < 0) return;
  const int64_t begin = static_cast<int64_t>(blockIdx.x) * kPieceBytes;
  if (begin >= segment_bytes) return;
  const int64_t bytes = segment_bytes - begin < kPieceBytes ? segment_bytes - begin : kPieceBytes;
  const int64_t seg = static_cast<int64_t>(blockIdx.y) * segment_stride + begin;
  copy_span<V>(dst_base + d * dst_row_stride + seg, src_base + s * src_row_stride + seg, bytes);
}

template <class V>
__global__ __launch_bounds__(kThreads) void zero_rows_kernel(char* base, int64_t row_stride, const void* idx,
                                                             int is64, int64_t segment_bytes,
                                                             int64_t segment_stride) {
  const int64_t row = blockIdx.z;
  const int64_t r = idx ? load_index(idx, row, is64) : row;
  if (r < 0) return;
  const int64_t begin = static_cast<int64_t>(blockIdx.x) * kPieceBytes;
  if (begin >= segment_bytes) return;
  const int64_t bytes = segment_bytes - begin < kPieceBytes ? segment_bytes - begin : kPieceBytes;
  zero_span<V>(base + r * row_stride + static_cast<int64_t>(blockIdx.y) * segment_stride + begin, bytes);
}

// grid: (pieces of the larger row, 2 = {state, conv}, batch)
__global__ __launch_bounds__(kThreads) void commit_kernel(char* state, int64_t state_slot_stride,
                                                          int64_t state_layer_offset, int64_t state_row,
                                                          char* conv, int64_t conv_slot_stride,
                                                          int64_t conv_layer_offset, int64_t conv_row,
                                                          const void* live, int live_is64,
                                                          const void* writes, int64_t wb, int64_t wt,
                                                          int writes_is64, const void* accepted,
                                                          int accepted_is64, int64_t steps) {
  const int64_t b = blockIdx.z;
  const int64_t a = load_index(accepted, b, accepted_is64);
  if (a < 1 || a > steps) return;
  const int64_t src = load_index(writes, b * wb + (a - 1) * wt, writes_is64);
  const int64_t dst = load_index(live, b, live_is64);
  if (src < 0 || dst < 0 || src == dst) return;
  const bool is_state = blockIdx.y == 0;
  char* base = is_state ? state : conv;
  const int64_t stride = is_state ? state_slot_stride : conv_slot_stride;
  const int64_t offset = is_state ? state_layer_offset : conv_layer_offset;
  const int64_t row = is_state ? state_row : conv_row;
  const int64_t begin = static_cast<int64_t>(blockIdx.x) * kPieceBytes;
  if (begin >= row) return;
  const int64_t bytes = row - begin < kPieceBytes ? row - begin : kPieceBytes;
  copy_span<uint4>(base + dst * stride + offset + begin, base + src * stride + offset + begin, bytes);
}

int alignment_of(int64_t v) {
  if (v % 16 == 0) return 16;
  if (v % 4 == 0) return 4;
  return 1;
}

int common_alignment(std::initializer_list<int64_t> values) {
  int a = 16;
  for (int64_t v : values) a = std::min(a, alignment_of(v));
  return a;
}

}  // namespace
}  // namespace gdn

using namespace gdn;

extern "C" int gdn_copy_rows(void* dst_base, int64_t dst_row_stride_bytes, const void* dst_idx,
                             int dst_idx_dtype, const void* src_base, int64_t src_row_stride_bytes,
                             const void* src_idx, int src_idx_dtype, int64_t pairs, int64_t segments,
                             int64_t segment_bytes, int64_t segment_stride_bytes, void* stream) {
  GDN_REQUIRE(pairs >= 0 && segments >= 0 && segment_bytes >= 0, "gdn_copy_rows: negative size");
  if (pairs == 0 || segments == 0 || segment_bytes == 0) return GDN_OK;
  GDN_REQUIRE(dst_base && src_base, "gdn_copy_rows: null base pointer");
  GDN_REQUIRE(pairs <= 65535 && segments <= 65535, "gdn_copy_rows: too many rows/segments (%lld, %lld)",
              (long long)pairs, (long long)segments);
  const int64_t pieces = (segment_bytes + kPieceBytes - 1) / kPieceBytes;
  dim3 grid(static_cast<unsigned>(pieces), static_cast<unsigned>(segments), static_cast<unsigned>(pairs));
  const int align = common_alignment({reinterpret_cast<int64_t>(dst_base), reinterpret_cast<int64_t>(src_base),
                                      dst_row_stride_bytes, src_row_stride_bytes, segment_bytes,
                                      segment_stride_bytes});
  auto s = static_cast<hipStream_t>(stream);
  const int d64 = dst_idx_dtype == GDN_I64, s64 = src_idx_dtype == GDN_I64;
  char* d = static_cast<char*>(dst_base);
  const char* sb = static_cast<const char*>(src_base);
  if (align == 16)
    hipLaunchKernelGGL(copy_rows_kernel<uint4>, grid, dim3(kThreads), 0, s, d, dst_row_stride_bytes, dst_idx,
                       d64, sb, src_row_stride_bytes, src_idx, s64, segment_bytes, segment_stride_bytes);
  else if (align == 4)
    hipLaunchKernelGGL(copy_rows_kernel<uint32_t>, grid, dim3(kThreads), 0, s, d, dst_row_stride_bytes,
                       dst_idx, d64, sb, src_row_stride_bytes, src_idx, s64, segment_bytes,
                       segment_stride_bytes);
  else
    hipLaunchKernelGGL(copy_rows_kernel<uint8_t>, grid, dim3(kThreads), 0, s, d, dst_row_stride_bytes,
                       dst_idx, d64, sb, src_row_stride_bytes, src_idx, s64, segment_bytes,
                       segment_stride_bytes);
  return GDN_LAUNCH_CHECK("gdn_copy_rows launch");
}

extern "C" int gdn_store_state(void* pool, int64_t pool_row_stride_bytes, const void* indices, int index_dtype,
                               const void* states, int64_t state_row_stride_bytes, int64_t rows,
                               int64_t row_bytes, void* stream) {
  GDN_REQUIRE(rows >= 0, "gdn_store_state: negative row count");
  if (rows == 0) return GDN_OK;
  GDN_REQUIRE(indices != nullptr, "gdn_store_state: null indices");
  GDN_REQUIRE(index_dtype == GDN_I32 || index_dtype == GDN_I64, "gdn_store_state: indices must be int32/int64");
  return gdn_copy_rows(pool, pool_row_stride_bytes, indices, index_dtype, states, state_row_stride_bytes,
                       nullptr, GDN_I64, rows, 1, row_bytes, 0, stream);
}

extern "C" int gdn_zero_rows(void* base, int64_t row_stride_bytes, const void* idx, int idx_dtype, int64_t rows,
                             int64_t segments, int64_t segment_bytes, int64_t segment_stride_bytes,
                             void* stream) {
  GDN_REQUIRE(rows >= 0 && segments >= 0 && segment_bytes >= 0, "gdn_zero_rows: negative size");
  if (rows == 0 || segments == 0 || segment_bytes == 0) return GDN_OK;
  GDN_REQUIRE(base != nullptr, "gdn_zero_rows: null base");
  GDN_REQUIRE(rows <= 65535 && segments <= 65535, "gdn_zero_rows: too many rows/segments");
  const int64_t pieces = (segment_bytes + kPieceBytes - 1) / kPieceBytes;
  dim3 grid(static_cast<unsigned>(pieces), static_cast<unsigned>(segments), static_cast<unsigned>(rows));
  const int align = common_alignment({reinterpret_cast<int64_t>(base), row_stride_bytes, segment_bytes,
                                      segment_stride_bytes});
  auto s = static_cast<hipStream_t>(stream);
  char* b = static_cast<char*>(base);
  const int i64 = idx_dtype == GDN_I64;
  if (align == 16)
    hipLaunchKernelGGL(zero_rows_kernel<uint4>, grid, dim3(kThreads), 0, s, b, row_stride_bytes, idx, i64,
                       segment_bytes, segment_stride_bytes);
  else if (align == 4)
    hipLaunchKernelGGL(zero_rows_kernel<uint32_t>, grid, dim3(kThreads), 0, s, b, row_stride_bytes, idx, i64,
                       segment_bytes, segment_stride_bytes);
  else
    hipLaunchKernelGGL(zero_rows_kernel<uint8_t>, grid, dim3(kThreads), 0, s, b, row_stride_bytes, idx, i64,
                       segment_bytes, segment_stride_bytes);
  return GDN_LAUNCH_CHECK("gdn_zero_rows launch");
}

extern "C" int gdn_commit_accepted(void* state, int64_t state_slot_stride_bytes, int64_t state_layer_offset_bytes,
                                   int64_t state_row_bytes, void* conv_state, int64_t conv_slot_stride_bytes,
                                   int64_t conv_layer_offset_bytes, int64_t conv_row_bytes,
                                   const void* live_slots, int live_dtype, const void* write_slots,
                                   int64_t write_b_stride, int64_t write_t_stride, int write_dtype,
                                   const void* accepted, int accepted_dtype, int64_t batch, int64_t steps,
                                   void* stream) {
  GDN_REQUIRE(batch >= 0 && steps >= 1, "gdn_commit_accepted: bad batch/steps");
  if (batch == 0) return GDN_OK;
  GDN_REQUIRE(state && conv_state && live_slots && write_slots && accepted, "gdn_commit_accepted: null pointer");
  GDN_REQUIRE(batch <= 65535, "gdn_commit_accepted: batch too large");
  const int align = common_alignment({reinterpret_cast<int64_t>(state), reinterpret_cast<int64_t>(conv_state),
                                      state_slot_stride_bytes, state_layer_offset_bytes, state_row_bytes,
                                      conv_slot_stride_bytes, conv_layer_offset_bytes, conv_row_bytes});
  GDN_REQUIRE(align == 16, "gdn_commit_accepted: pools, strides and row sizes must be 16-byte aligned");
  const int64_t row = std::max(state_row_bytes, conv_row_bytes);
  const int64_t pieces = (row + kPieceBytes - 1) / kPieceBytes;
  dim3 grid(static_cast<unsigned>(pieces), 2, static_cast<unsigned>(batch));
  hipLaunchKernelGGL(commit_kernel, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<char*>(state), state_slot_stride_bytes, state_layer_offset_bytes,
                     state_row_bytes, static_cast<char*>(conv_state), conv_slot_stride_bytes,
                     conv_layer_offset_bytes, conv_row_bytes, live_slots, live_dtype == GDN_I64, write_slots,
                     write_b_stride, write_t_stride, write_dtype == GDN_I64, accepted,
                     accepted_dtype == GDN_I64, steps);
  return GDN_LAUNCH_CHECK("gdn_commit_accepted launch");
}
