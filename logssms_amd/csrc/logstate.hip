// LogState token log of the chunked prefill (ChunkLogIO,
// kernel/linear_attention/state_io.py:83-126 with the log layout of
// kernel/linear_attention/layout.py:29-80): for every packed token with a log
// slot, its v' residual row (u - w h) per value head, its key row per logged
// key head and its prepared gate per value head go into the slot's frames.
//
// Log payload of a slot, in 16-bit elements from logical byte 0 of the slot:
// granule (position / granularity), then layer, then the keys [key_heads,
// granularity, dk] followed by the values [HV, granularity, dv]; logical byte
// x lies in frame frames[slot fps + x / frame_bytes] at offset x %
// frame_bytes.  The gate of (layer, position, head) is the float at index
// (layer page + position) HV + head of the slot's decay record
// (decay_frames[slot] = {frame, record}, record_bytes apart in that frame).
//
// Pure data movement (about 2 (dv + dk / group) + 4 bytes per token-head), one
// 64-lane block per (token, value head); the lanes walk the row.
#include "common.hpp"

namespace gdn {
namespace {

constexpr int kThreads = 64;

struct LogParams {
  char* storage;
  const void* frames;
  int frames_is64;
  int64_t fps, frame_bytes, num_frames;
  const void* slots;
  int slots_is64;
  const void* offsets;
  int offsets_is64;
  const uint16_t* v_new;
  const uint16_t* key;
  int64_t H, HV, K, V, KH;
  const float* gate;
  const void* decay;
  int decay_is64;
  int64_t record_bytes;
  int64_t layer, layers, gran, page;
};

// Address of element `col` of log row `index` (a value head, or a logged key
// head) at `pos`, or null when its frame is unmapped.
__device__ __forceinline__ uint16_t* log_element(const LogParams& p, int64_t slot, int64_t pos, int64_t index,
                                                 int64_t col, bool value) {
  const int64_t key_size = p.gran * p.KH * p.K;
  const int64_t layer_size = key_size + p.gran * p.HV * p.V;
  const int64_t dim = value ? p.V : p.K;
  const int64_t elem = (pos / p.gran * p.layers + p.layer) * layer_size + (value ? key_size : 0) +
                       (index * p.gran + pos % p.gran) * dim + col;
  const int64_t byte = 2 * elem;
  const int64_t fr = load_index(p.frames, slot * p.fps + byte / p.frame_bytes, p.frames_is64);
  if (fr < 0 || fr >= p.num_frames) return nullptr;
  return reinterpret_cast<uint16_t*>(p.storage + fr * p.frame_bytes + byte % p.frame_bytes);
}

// grid (T, HV)
__global__ __launch_bounds__(kThreads) void chunk_log_kernel(LogParams p) {
  const int64_t t = blockIdx.x, h = blockIdx.y;
  const int64_t slot = load_index(p.slots, t, p.slots_is64);
  const int64_t pos = load_index(p.offsets, t, p.offsets_is64);
  if (slot < 0 || pos < 0 || pos >= p.page) return;
  const uint16_t* vrow = p.v_new + (t * p.HV + h) * p.V;
  for (int64_t col = threadIdx.x; col < p.V; col += kThreads) {
    uint16_t* d = log_element(p, slot, pos, h, col, true);
    if (d) *d = vrow[col];
  }
  const int64_t group = p.HV / p.KH;  // value heads per logged key head
  if (h % group == 0) {
    const uint16_t* krow = p.key + (t * p.H + h / (p.HV / p.H)) * p.K;
    for (int64_t col = threadIdx.x; col < p.K; col += kThreads) {
      uint16_t* d = log_element(p, slot, pos, h / group, col, false);
      if (d) *d = krow[col];
    }
  }
  if (threadIdx.x == 0) {
    const int64_t fr = load_index(p.decay, 2 * slot, p.decay_is64);
    const int64_t rec = load_index(p.decay, 2 * slot + 1, p.decay_is64);
    if (fr >= 0 && fr < p.num_frames && rec >= 0 && (rec + 1) * p.record_bytes <= p.frame_bytes) {
      float* d = reinterpret_cast<float*>(p.storage + fr * p.frame_bytes + rec * p.record_bytes);
      d[(p.layer * p.page + pos) * p.HV + h] = p.gate[t * p.HV + h];
    }
  }
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_store_chunk_log(void* storage, const void* frames, int frames_dtype, int64_t frames_per_slot,
                                   int64_t frame_bytes, int64_t num_frames, const void* log_slots, int slots_dtype,
                                   const void* token_offsets, int offsets_dtype, int64_t T, const void* v_new,
                                   const void* key, int64_t H, int64_t HV, int64_t dk, int64_t dv, int64_t key_heads,
                                   const float* gate, const void* decay_frames, int decay_dtype,
                                   int64_t decay_record_bytes, int64_t layer, int64_t num_layers, int64_t granularity,
                                   int64_t page_size, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(T >= 0 && H > 0 && HV > 0 && HV % H == 0 && dk > 0 && dv > 0 && key_heads > 0 &&
                  H % key_heads == 0 && HV % key_heads == 0,
              "gdn_store_chunk_log: bad head counts (H %lld, HV %lld, key_heads %lld)", (long long)H, (long long)HV,
              (long long)key_heads);
  GDN_REQUIRE(num_layers > 0 && layer >= 0 && layer < num_layers && granularity > 0 && page_size > 0 &&
                  page_size % granularity == 0,
              "gdn_store_chunk_log: bad layout (layer %lld of %lld, granularity %lld, page %lld)", (long long)layer,
              (long long)num_layers, (long long)granularity, (long long)page_size);
  GDN_REQUIRE(frames_per_slot > 0 && frame_bytes > 0 && frame_bytes % 4 == 0 && num_frames > 0,
              "gdn_store_chunk_log: bad frame table");
  const int64_t log_bytes = 2 * page_size * num_layers * (key_heads * dk + HV * dv);
  GDN_REQUIRE(log_bytes <= frames_per_slot * frame_bytes,
              "gdn_store_chunk_log: a slot's log (%lld bytes) exceeds its %lld frames", (long long)log_bytes,
              (long long)frames_per_slot);
  GDN_REQUIRE(decay_record_bytes % 4 == 0 && decay_record_bytes >= 4 * num_layers * page_size * HV &&
                  decay_record_bytes <= frame_bytes,
              "gdn_store_chunk_log: decay records of %lld bytes do not hold %lld layers x %lld positions x %lld heads",
              (long long)decay_record_bytes, (long long)num_layers, (long long)page_size, (long long)HV);
  if (T == 0) return GDN_OK;
  GDN_REQUIRE(storage && frames && log_slots && token_offsets && v_new && key && gate && decay_frames,
              "gdn_store_chunk_log: null input");
  GDN_REQUIRE(T <= 0x7fffffff && HV <= 65535, "gdn_store_chunk_log: grid too large");
  LogParams p{};
  p.storage = static_cast<char*>(storage);
  p.frames = frames; p.frames_is64 = frames_dtype == GDN_I64;
  p.fps = frames_per_slot; p.frame_bytes = frame_bytes; p.num_frames = num_frames;
  p.slots = log_slots; p.slots_is64 = slots_dtype == GDN_I64;
  p.offsets = token_offsets; p.offsets_is64 = offsets_dtype == GDN_I64;
  p.v_new = static_cast<const uint16_t*>(v_new);
  p.key = static_cast<const uint16_t*>(key);
  p.H = H; p.HV = HV; p.K = dk; p.V = dv; p.KH = key_heads;
  p.gate = gate;
  p.decay = decay_frames; p.decay_is64 = decay_dtype == GDN_I64;
  p.record_bytes = decay_record_bytes;
  p.layer = layer; p.layers = num_layers; p.gran = granularity; p.page = page_size;
  hipLaunchKernelGGL(chunk_log_kernel, dim3(static_cast<unsigned>(T), static_cast<unsigned>(HV)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), p);
  return GDN_LAUNCH_CHECK("gdn_store_chunk_log launch");
}
