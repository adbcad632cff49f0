// C-ABI entry points of the chunked gated delta rule
// (vendor/fla/gated_delta.py:15-82 with ChunkStateIO / ChunkLogIO,
// kernel/linear_attention/state_io.py:15-126): argument checks, frame-table
// layout validation and the launch of the register-chain kernel
// (chunk_chain.hip), which covers d_k in {32, 64, 128} and d_v = 32 or a
// multiple of 64.
#include "chunk_common.hpp"

namespace gdn {

int set_frame_layout(ChunkParams& p, int64_t dk, int state_dtype, const void* frames, int frames_dtype,
                     int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes, int64_t num_frames,
                     int64_t table_rows) {
  const int64_t elt = state_dtype == GDN_F32 ? 4 : 2;
  const int64_t state_bytes = dk * p.DV * elt;
  GDN_REQUIRE(frames_per_slot > 0 && frame_bytes > 0 && num_frames > 0 && table_rows >= 0 &&
                  head_bytes >= state_bytes && frame_bytes % elt == 0 && head_bytes % elt == 0,
              "gdn_chunk_gated_delta_rule: bad frame layout (frames_per_slot %lld, frame_bytes %lld, head_bytes "
              "%lld, num_frames %lld, table rows %lld, state %lld bytes per head)",
              (long long)frames_per_slot, (long long)frame_bytes, (long long)head_bytes, (long long)num_frames,
              (long long)table_rows, (long long)state_bytes);
  const bool inside = head_bytes <= frame_bytes;
  GDN_REQUIRE(inside ? frame_bytes % head_bytes == 0
                     : head_bytes % frame_bytes == 0 && frame_bytes % (16 * p.DV * elt) == 0,
              "gdn_chunk_gated_delta_rule: head_bytes %lld must divide frame_bytes %lld, or be a multiple of it "
              "with frames holding whole 16-row state tiles",
              (long long)head_bytes, (long long)frame_bytes);
  GDN_REQUIRE((p.layer + 1) * p.HV * head_bytes <= frames_per_slot * frame_bytes,
              "gdn_chunk_gated_delta_rule: layer %lld of %lld heads x %lld bytes lies past the %lld frames of a slot",
              (long long)p.layer, (long long)p.HV, (long long)head_bytes, (long long)frames_per_slot);
  p.frames = frames;
  p.frames_is64 = frames_dtype == GDN_I64;
  p.frame_rows = inside ? 0 : 1;
  p.frame_slots = table_rows;
  p.fps = frames_per_slot;
  p.frame_bytes = frame_bytes;
  p.head_bytes = head_bytes;
  p.num_frames = num_frames;
  p.fdiv = make_div32(frame_bytes);
  return GDN_OK;
}

namespace {
// The token log arguments of gdn_chunk_gated_delta_rule_logged.
struct LogArgs {
  const void* slots;
  int slots_dtype;
  const void* offsets;
  int offsets_dtype;
  int64_t key_heads, layers, page;
};

int chunk_entry(const void* q, const void* k, const void* v, int io_dtype, const float* g, const float* beta,
                const void* cu_seqlens, int cu_dtype, int64_t num_seqs, int64_t total_tokens, int64_t H, int64_t HV,
                int64_t dk, int64_t dv, void* state, int state_dtype, int64_t slot_stride, int64_t layer_stride,
                int64_t head_stride, int64_t layer, const void* read_slots, int read_dtype,
                const void* chunk_write_slots, int chunk_write_dtype, const void* final_write_slots,
                int final_write_dtype, int64_t chunk_size, const void* frames, int frames_dtype, int64_t table_rows,
                int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes, int64_t num_frames, void* out,
                void* v_new, float scale, const LogArgs* log, void* stream) {
  GDN_REQUIRE(num_seqs >= 0 && total_tokens >= 0 && H > 0 && HV > 0 && HV % H == 0 && layer >= 0,
              "gdn_chunk_gated_delta_rule: bad sizes");
  GDN_REQUIRE(chunk_size == 16 || chunk_size == 32 || chunk_size == 64,
              "gdn_chunk_gated_delta_rule: chunk_size %lld not in {16, 32, 64}", (long long)chunk_size);
  if (num_seqs == 0) return GDN_OK;
  GDN_REQUIRE(q && k && v && g && beta && cu_seqlens && state && read_slots && chunk_write_slots && out,
              "gdn_chunk_gated_delta_rule: null input");
  if (!((dk == 32 || dk == 64 || dk == 128) && (dv == 32 || (dv > 0 && dv % 64 == 0)))) {
    set_error("gdn_chunk_gated_delta_rule: unsupported head dims dk=%lld dv=%lld (dk in {32,64,128}, dv 32 or "
              "a multiple of 64)", (long long)dk, (long long)dv);
    return GDN_ERR_UNSUPPORTED;
  }
  ChunkParams p{};
  p.q = q; p.k = k; p.v = v; p.g = g; p.beta = beta;
  p.cu = cu_seqlens; p.cu_is64 = cu_dtype == GDN_I64;
  p.N = num_seqs; p.T = total_tokens; p.H = H; p.HV = HV; p.DV = dv;
  p.state = state; p.slot_stride = slot_stride; p.layer_stride = layer_stride; p.head_stride = head_stride;
  p.layer = layer;
  p.read_slots = read_slots; p.read_is64 = read_dtype == GDN_I64;
  p.cw_slots = chunk_write_slots; p.cw_is64 = chunk_write_dtype == GDN_I64;
  p.fw_slots = final_write_slots; p.fw_is64 = final_write_dtype == GDN_I64;
  p.out = out; p.v_new = v_new; p.scale = scale;
  p.gran = static_cast<int>(chunk_size);
  if (frames) {
    const int rc = set_frame_layout(p, dk, state_dtype, frames, frames_dtype, frames_per_slot, frame_bytes, head_bytes,
                                    num_frames, table_rows);
    if (rc != GDN_OK) return rc;
  }
  // the log-slot loads of the kernel read T words in any case: without a log, the gates
  p.logging = log != nullptr;
  p.log_slots = log ? log->slots : static_cast<const void*>(g);
  p.log_is64 = log ? log->slots_dtype == GDN_I64 : 0;
  p.log_pos = log ? log->offsets : static_cast<const void*>(g);
  p.log_pos_is64 = log ? log->offsets_dtype == GDN_I64 : 0;
  p.log_table = log ? frames : static_cast<const void*>(g);
  p.log_table_is64 = log ? frames_dtype == GDN_I64 : 0;
  p.log_rows = log ? table_rows : 0;
  if (log) {
    GDN_REQUIRE(frames && log->slots && log->offsets && log->key_heads > 0 && H % log->key_heads == 0 &&
                    HV % log->key_heads == 0 && log->layers > layer && log->page > 0 && log->page % chunk_size == 0,
                "gdn_chunk_gated_delta_rule_logged: bad token log layout");
    GDN_REQUIRE(io_dtype == state_dtype, "gdn_chunk_gated_delta_rule_logged: log rows are stored in the io dtype");
    GDN_REQUIRE(2 * log->page * log->layers * (log->key_heads * dk + HV * dv) <= frames_per_slot * frame_bytes &&
                    frames_per_slot * frame_bytes < kMaxOffset32,
                "gdn_chunk_gated_delta_rule_logged: the log exceeds a slot's frames or 4 GiB");
    p.log_key_heads = log->key_heads;
    p.log_layers = log->layers;
    p.log_page = log->page;
    // a workgroup's slice of a value row (64 columns, or all 32) starts at a
    // multiple of its own size and must not straddle two frames
    const int64_t slice_bytes = 2 * (dv < 64 ? dv : 64);
    if (frame_bytes % slice_bytes != 0) {
      set_error("gdn_chunk_gated_delta_rule_logged: frames must be a multiple of %lld bytes", (long long)slice_bytes);
      return GDN_ERR_UNSUPPORTED;
    }
  }
  p.nvs = static_cast<int>((dv + 63) / 64);
  p.members = static_cast<int>((HV / H) * p.nvs);
  const int rc = launch_chunk_chain(p, dk, io_dtype, state_dtype, num_seqs * H, static_cast<hipStream_t>(stream));
  if (rc == GDN_ERR_UNSUPPORTED)
    set_error("gdn_chunk_gated_delta_rule: unsupported io/state dtypes %d/%d (16-bit io, fp32 or io-typed state)",
              io_dtype, state_dtype);
  return rc;
}
}  // namespace
}  // namespace gdn

extern "C" int gdn_chunk_gated_delta_rule(const void* q, const void* k, const void* v, int io_dtype, const float* g,
                                          const float* beta, const void* cu_seqlens, int cu_dtype, int64_t num_seqs,
                                          int64_t total_tokens, int64_t H, int64_t HV, int64_t dk, int64_t dv,
                                          void* state, int state_dtype, int64_t slot_stride, int64_t layer_stride,
                                          int64_t head_stride, int64_t layer, const void* read_slots, int read_dtype,
                                          const void* chunk_write_slots, int chunk_write_dtype,
                                          const void* final_write_slots, int final_write_dtype, int64_t chunk_size,
                                          const void* frames, int frames_dtype, int64_t table_rows,
                                          int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes,
                                          int64_t num_frames, void* out, void* v_new, float scale, void* stream) {
  return gdn::chunk_entry(q, k, v, io_dtype, g, beta, cu_seqlens, cu_dtype, num_seqs, total_tokens, H, HV, dk, dv,
                          state, state_dtype, slot_stride, layer_stride, head_stride, layer, read_slots, read_dtype,
                          chunk_write_slots, chunk_write_dtype, final_write_slots, final_write_dtype, chunk_size, frames,
                          frames_dtype, table_rows, frames_per_slot, frame_bytes, head_bytes, num_frames, out, v_new,
                          scale, nullptr, stream);
}

extern "C" int gdn_chunk_gated_delta_rule_logged(
    const void* q, const void* k, const void* v, int io_dtype, const float* g, const float* beta,
    const void* cu_seqlens, int cu_dtype, int64_t num_seqs, int64_t total_tokens, int64_t H, int64_t HV, int64_t dk,
    int64_t dv, void* state, int state_dtype, int64_t layer, const void* read_slots, int read_dtype,
    const void* chunk_write_slots, int chunk_write_dtype, const void* final_write_slots, int final_write_dtype,
    int64_t chunk_size, const void* frames, int frames_dtype, int64_t table_rows, int64_t frames_per_slot,
    int64_t frame_bytes, int64_t head_bytes, int64_t num_frames, const void* log_slots, int log_dtype,
    const void* token_offsets, int offsets_dtype, int64_t key_heads, int64_t num_layers, int64_t page_size, void* out,
    float scale, void* stream) {
  GDN_REQUIRE(frames, "gdn_chunk_gated_delta_rule_logged: the token log lives in frame storage");
  const gdn::LogArgs log{log_slots, log_dtype, token_offsets, offsets_dtype, key_heads, num_layers, page_size};
  return gdn::chunk_entry(q, k, v, io_dtype, g, beta, cu_seqlens, cu_dtype, num_seqs, total_tokens, H, HV, dk, dv,
                          state, state_dtype, 0, 0, 0, layer, read_slots, read_dtype, chunk_write_slots,
                          chunk_write_dtype, final_write_slots, final_write_dtype, chunk_size, frames, frames_dtype,
                          table_rows, frames_per_slot, frame_bytes, head_bytes, num_frames, out, nullptr, scale, &log,
                          stream);
}
