// LogState frame stores and copies (pure data movement, HBM-bound):
//   * conv snapshot copy (kernel/linear_attention/conv_copy.py:7-52): every
//     layer's conv window of (source slot, source granule) to (output slot,
//     output granule);
//   * masked conv store (masked_store.py:37-72, store_conv): rows of
//     conv_dim x state_len elements to layer `layer` of (slot, granule)
//     snapshots, rows with a negative slot skipped;
//   * masked state store (masked_store.py:11-55, store_states): rows of HV
//     states of dk x dv elements to layer `layer` of the slots' state heads,
//     rows with a negative slot skipped.
//
// Every frame side is addressed the same way: a run of logical bytes x of
// one table row lies in frame table[row + x / frame_bytes] at offset
// x % frame_bytes.  Conv snapshots use row (slot G + granule) CF of the conv
// frame table [slots, G, CF] (kernel/linear_attention/layout.py:104-112), state
// heads row slot fps of the payload frame table with head h of layer l at
// logical byte (l HV + h) head_bytes (layout.py:11-26).
//
// One block per (task, 4 KiB span of its bytes); 16-byte vectors when every
// frame, run and source row is 16-byte aligned, 2-byte units otherwise.
#include "common.hpp"

namespace gdn {
namespace {

constexpr int kCopyThreads = 256;
constexpr int64_t kSpanBytes = 4096;

enum FrameCopyMode { kCopyConv = 0, kStoreConv = 1, kStoreStates = 2 };

struct FrameCopyParams {
  char* storage;
  int64_t frame_bytes, num_frames;
  const void* table; int table_is64;
  int64_t table_rows;              // slots in the table
  int64_t G, CF, fps;              // conv granules / frames per snapshot; payload frames per slot
  const void* src_slots; int src_is64;
  const void* src_gran; int src_gran_is64;
  const void* dst_slots; int dst_is64;
  const void* dst_gran; int dst_gran_is64;
  const char* values;              // linear source rows (stores)
  int64_t length;                  // bytes per task
  int64_t layer, HV, head_bytes;
  int64_t tasks, spans;            // spans of kSpanBytes per task
  Div32 fdiv;                      // frame_bytes
};

// Frame byte address of logical byte x of table row `row`, or null.
__device__ __forceinline__ char* frame_byte(const FrameCopyParams& p, int64_t row, int64_t per_row, int64_t x) {
  const uint32_t x32 = static_cast<uint32_t>(x);  // < per_row frame_bytes < 2^32 (checked by the host)
  const int64_t fr = load_index(p.table, row * per_row + p.fdiv.div(x32), p.table_is64);
  if (fr < 0 || fr >= p.num_frames) return nullptr;
  return p.storage + fr * p.frame_bytes + p.fdiv.mod(x32);
}

template <class U>
__global__ __launch_bounds__(kCopyThreads) void frame_copy_kernel(FrameCopyParams p, int mode) {
  const uint32_t bid = blockIdx.x, nspans = static_cast<uint32_t>(p.spans);
  const int64_t task = bid / nspans;
  const int64_t span = bid % nspans;
  // destination row / start, and source (frames or linear rows)
  int64_t dst_row, dst_start, per_row;
  int64_t src_row = -1;
  const char* src_linear = nullptr;
  if (mode == kStoreStates) {
    const int64_t r = task / p.HV, h = task % p.HV;
    const int64_t slot = load_index(p.dst_slots, r, p.dst_is64);
    if (slot < 0 || slot >= p.table_rows) return;
    dst_row = slot;
    per_row = p.fps;
    dst_start = (p.layer * p.HV + h) * p.head_bytes;
    src_linear = p.values + task * p.length;
  } else {
    const int64_t slot = load_index(p.dst_slots, task, p.dst_is64);
    const int64_t gran = load_index(p.dst_gran, task, p.dst_gran_is64);
    if (slot < 0 || slot >= p.table_rows || gran < 0 || gran >= p.G) return;
    dst_row = slot * p.G + gran;
    per_row = p.CF;
    if (mode == kCopyConv) {
      const int64_t s = load_index(p.src_slots, task, p.src_is64);
      const int64_t sg = load_index(p.src_gran, task, p.src_gran_is64);
      if (s < 0 || s >= p.table_rows || sg < 0 || sg >= p.G) return;
      src_row = s * p.G + sg;
      dst_start = 0;
    } else {
      dst_start = p.layer * p.length;
      src_linear = p.values + task * p.length;
    }
  }
  const int64_t begin = span * kSpanBytes;
  const int64_t end = begin + kSpanBytes < p.length ? begin + kSpanBytes : p.length;
  for (int64_t b = begin + threadIdx.x * static_cast<int64_t>(sizeof(U)); b < end;
       b += kCopyThreads * static_cast<int64_t>(sizeof(U))) {
    const char* src = src_linear ? src_linear + b : frame_byte(p, src_row, per_row, b);
    char* dst = frame_byte(p, dst_row, per_row, dst_start + b);
    if (src && dst) *reinterpret_cast<U*>(dst) = *reinterpret_cast<const U*>(src);
  }
}

int launch_frame_copy(FrameCopyParams& p, int mode, bool aligned16, hipStream_t stream, const char* who) {
  GDN_REQUIRE((mode == kStoreStates ? p.fps : p.CF) * p.frame_bytes < kMaxOffset32, "%s: a row's frames exceed 4 GiB",
              who);
  p.fdiv = make_div32(p.frame_bytes);
  p.spans = (p.length + kSpanBytes - 1) / kSpanBytes;
  const int64_t blocks = p.tasks * p.spans;
  if (blocks == 0) return GDN_OK;
  if (blocks > 0x7fffffff) {
    set_error("%s: grid too large", who);
    return GDN_ERR_INVALID;
  }
  if (aligned16)
    hipLaunchKernelGGL(frame_copy_kernel<uint4>, dim3(static_cast<unsigned>(blocks)), dim3(kCopyThreads), 0, stream,
                       p, mode);
  else
    hipLaunchKernelGGL(frame_copy_kernel<uint16_t>, dim3(static_cast<unsigned>(blocks)), dim3(kCopyThreads), 0,
                       stream, p, mode);
  return GDN_LAUNCH_CHECK(who);
}

bool aligned(int64_t v, int64_t a) { return v % a == 0; }

}  // namespace
}  // namespace gdn

extern "C" int gdn_logstate_copy_conv(void* storage, const void* conv_frames, int frames_dtype, int64_t table_rows,
                                      int64_t granules, int64_t frames_per_snapshot, int64_t frame_bytes,
                                      int64_t num_frames, int64_t snapshot_bytes, const void* source_slots,
                                      int source_slots_dtype, const void* source_granules, int source_granules_dtype,
                                      const void* output_slots, int output_slots_dtype, const void* output_granules,
                                      int output_granules_dtype, int64_t count, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(count >= 0 && snapshot_bytes >= 0, "gdn_logstate_copy_conv: bad sizes");
  if (count == 0 || snapshot_bytes == 0) return GDN_OK;
  GDN_REQUIRE(storage && conv_frames && source_slots && source_granules && output_slots && output_granules,
              "gdn_logstate_copy_conv: null input");
  GDN_REQUIRE(table_rows > 0 && granules > 0 && frames_per_snapshot > 0 && frame_bytes > 0 && num_frames > 0 &&
                  snapshot_bytes % 2 == 0 && frame_bytes % 2 == 0 &&
                  snapshot_bytes <= frames_per_snapshot * frame_bytes,
              "gdn_logstate_copy_conv: the snapshot (%lld bytes) must be whole 16-bit elements within %lld frames "
              "of %lld bytes",
              (long long)snapshot_bytes, (long long)frames_per_snapshot, (long long)frame_bytes);
  FrameCopyParams p{};
  p.storage = static_cast<char*>(storage);
  p.frame_bytes = frame_bytes; p.num_frames = num_frames;
  p.table = conv_frames; p.table_is64 = frames_dtype == GDN_I64; p.table_rows = table_rows;
  p.G = granules; p.CF = frames_per_snapshot;
  p.src_slots = source_slots; p.src_is64 = source_slots_dtype == GDN_I64;
  p.src_gran = source_granules; p.src_gran_is64 = source_granules_dtype == GDN_I64;
  p.dst_slots = output_slots; p.dst_is64 = output_slots_dtype == GDN_I64;
  p.dst_gran = output_granules; p.dst_gran_is64 = output_granules_dtype == GDN_I64;
  p.length = snapshot_bytes; p.tasks = count;
  const bool a16 = aligned(frame_bytes, 16) && aligned(snapshot_bytes, 16) &&
                   aligned(reinterpret_cast<uintptr_t>(storage), 16);
  return launch_frame_copy(p, kCopyConv, a16, static_cast<hipStream_t>(stream), "gdn_logstate_copy_conv");
}

extern "C" int gdn_logstate_store_conv(void* storage, const void* conv_frames, int frames_dtype, int64_t table_rows,
                                       int64_t granules, int64_t frames_per_snapshot, int64_t frame_bytes,
                                       int64_t num_frames, const void* slots, int slots_dtype, const void* slot_granules,
                                       int granules_dtype, int64_t count, int64_t layer, int64_t row_bytes,
                                       const void* values, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(count >= 0 && row_bytes >= 0 && layer >= 0, "gdn_logstate_store_conv: bad sizes");
  if (count == 0 || row_bytes == 0) return GDN_OK;
  GDN_REQUIRE(storage && conv_frames && slots && slot_granules && values, "gdn_logstate_store_conv: null input");
  GDN_REQUIRE(table_rows > 0 && granules > 0 && frames_per_snapshot > 0 && frame_bytes > 0 && num_frames > 0 &&
                  row_bytes % 2 == 0 && frame_bytes % 2 == 0 &&
                  (layer + 1) * row_bytes <= frames_per_snapshot * frame_bytes,
              "gdn_logstate_store_conv: layer %lld of %lld-byte rows exceeds the %lld frames of a snapshot",
              (long long)layer, (long long)row_bytes, (long long)frames_per_snapshot);
  FrameCopyParams p{};
  p.storage = static_cast<char*>(storage);
  p.frame_bytes = frame_bytes; p.num_frames = num_frames;
  p.table = conv_frames; p.table_is64 = frames_dtype == GDN_I64; p.table_rows = table_rows;
  p.G = granules; p.CF = frames_per_snapshot;
  p.dst_slots = slots; p.dst_is64 = slots_dtype == GDN_I64;
  p.dst_gran = slot_granules; p.dst_gran_is64 = granules_dtype == GDN_I64;
  p.values = static_cast<const char*>(values);
  p.length = row_bytes; p.layer = layer; p.tasks = count;
  const bool a16 = aligned(frame_bytes, 16) && aligned(row_bytes, 16) &&
                   aligned(reinterpret_cast<uintptr_t>(storage), 16) &&
                   aligned(reinterpret_cast<uintptr_t>(values), 16);
  return launch_frame_copy(p, kStoreConv, a16, static_cast<hipStream_t>(stream), "gdn_logstate_store_conv");
}

extern "C" int gdn_logstate_store_states(void* storage, const void* payload_frames, int frames_dtype,
                                         int64_t table_rows, int64_t frames_per_slot, int64_t frame_bytes,
                                         int64_t head_bytes, int64_t num_frames, const void* slots, int slots_dtype,
                                         int64_t count, int64_t layer, int64_t HV, int64_t state_bytes,
                                         const void* values, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(count >= 0 && state_bytes >= 0 && layer >= 0 && HV > 0, "gdn_logstate_store_states: bad sizes");
  if (count == 0 || state_bytes == 0) return GDN_OK;
  GDN_REQUIRE(storage && payload_frames && slots && values, "gdn_logstate_store_states: null input");
  GDN_REQUIRE(table_rows > 0 && frames_per_slot > 0 && frame_bytes > 0 && num_frames > 0 && state_bytes % 2 == 0 &&
                  frame_bytes % 2 == 0 && head_bytes >= state_bytes &&
                  (head_bytes <= frame_bytes ? frame_bytes % head_bytes == 0 : head_bytes % frame_bytes == 0) &&
                  (layer + 1) * HV * head_bytes <= frames_per_slot * frame_bytes,
              "gdn_logstate_store_states: bad frame layout (head_bytes %lld, frame_bytes %lld, layer %lld)",
              (long long)head_bytes, (long long)frame_bytes, (long long)layer);
  FrameCopyParams p{};
  p.storage = static_cast<char*>(storage);
  p.frame_bytes = frame_bytes; p.num_frames = num_frames;
  p.table = payload_frames; p.table_is64 = frames_dtype == GDN_I64; p.table_rows = table_rows;
  p.fps = frames_per_slot;
  p.dst_slots = slots; p.dst_is64 = slots_dtype == GDN_I64;
  p.values = static_cast<const char*>(values);
  p.length = state_bytes; p.layer = layer; p.HV = HV; p.head_bytes = head_bytes; p.tasks = count * HV;
  const bool a16 = aligned(frame_bytes, 16) && aligned(state_bytes, 16) && aligned(head_bytes, 16) &&
                   aligned(reinterpret_cast<uintptr_t>(storage), 16) &&
                   aligned(reinterpret_cast<uintptr_t>(values), 16);
  return launch_frame_copy(p, kStoreStates, a16, static_cast<hipStream_t>(stream), "gdn_logstate_store_states");
}
