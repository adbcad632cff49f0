// Parameters of the chunked gated-delta-rule kernel (chunk_chain.hip) and its
// entry points (chunk_entry.hip).
#pragma once

#include "common.hpp"

namespace gdn {

// Raw inputs of the v conv (packed_conv.py:49-133) for the chunk kernel
// variant that computes its V tiles itself instead of reading v.
struct FrontIn {
  const void* mixed;  // [T, conv_dim] projections, unit column stride
  int64_t row_stride;
  const void* weight;      // [conv_dim, 4]
  void* conv_state;  // [slots, layers, conv_dim, 3] conv history pool (windows written back)
  int64_t conv_slot_stride, conv_layer_stride;
  int64_t key_dim;  // H * d_k: q channels [0, key_dim), k, then v
  // conv windows: for i < snap_count with snap_slots[i] >= 0, the 3 raw inputs
  // ending at packed row snap_rows[i] go to conv_state[snap_slots[i], layer]
  const void* snap_rows;
  const void* snap_slots;
  int snap_rows_is64, snap_slots_is64;
  int64_t snap_count;
};

struct ChunkParams {
  const void* q;
  const void* k;
  const void* v;
  const float* g;
  const float* beta;
  const void* cu;
  int cu_is64;
  int64_t N, T, H, HV, DV;
  void* state;
  int64_t slot_stride, layer_stride, head_stride, layer;
  const void* read_slots;
  int read_is64;
  const void* cw_slots;
  int cw_is64;
  const void* fw_slots;
  int fw_is64;
  void* out;
  void* v_new;
  float scale;
  int nvs;      // 64-column v slices per head
  int members;  // workgroups per (sequence, key head)
  FrontIn front;
  // Checkpoint granularity: cw_slots holds one slot per `gran` tokens of each
  // sequence (16, 32 or 64; the kernels work in 64-token chunks throughout).
  int gran;
  // Frame-table state addressing (LogState payload frames,
  // kernel/linear_attention/layout.py:11-26) when `frames` is set: `state` is
  // the frame storage, head (layer, h) of slot s starts at logical byte
  // (layer HV + h) head_bytes of the slot, and logical byte x of slot s lies in
  // frame frames[s fps + x / frame_bytes] at offset x % frame_bytes.  With
  // head_bytes <= frame_bytes a head sits inside one frame; otherwise each
  // 16-row tile of it is looked up on its own (frame_rows).
  const void* frames;
  int frames_is64;
  int frame_rows;
  int64_t frame_slots;  // rows (slots) of the frame table; slots past it read as unmapped
  int64_t fps, frame_bytes, head_bytes, num_frames;
  // Token log of v' (frame storage, EXT instantiation): with `logging` set,
  // the v' row of token t and value head h goes to the value row (h,
  // position) of the log of slot log_slots[t] at position log_pos[t], when
  // that slot is >= 0 and 0 <= position < log_page (the log layout of
  // gdn_store_chunk_log), instead of v_new.  Without it both pointers still
  // name T readable words (the kernel loads them unconditionally).
  int logging;
  const void* log_slots;
  int log_is64;
  const void* log_pos;
  int log_pos_is64;
  const void* log_table;  // the frame table when logging, else the same T words (plain pools have none)
  int log_table_is64;
  int64_t log_rows;  // rows of the log's frame table; log slots past it take no write
  int64_t log_key_heads, log_layers, log_page;
  Div32 fdiv;  // frame_bytes
};

// Host-side validation of a frame-table state layout; returns GDN_OK or sets
// the error and returns GDN_ERR_INVALID.  Fills the frame fields of p.
int set_frame_layout(ChunkParams& p, int64_t dk, int state_dtype, const void* frames, int frames_dtype,
                     int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes, int64_t num_frames,
                     int64_t table_rows);

// Register-chain kernel (chunk_chain.hip) for d_k in {32, 64, 128} and d_v 32
// or a multiple of 64 (the fused variant: a multiple of 64).  Returns GDN_ERR_UNSUPPORTED (without setting an error) for
// shapes or dtypes it does not cover, so the caller can use another kernel.
int launch_chunk_chain(const ChunkParams& p, int64_t dk, int io_dtype, int state_dtype, int64_t groups,
                       hipStream_t stream);
// The same kernel with the V tiles computed from p.front (conv width 4,
// 16-byte aligned rows) and q, k read as f16 operands; p.v is not read.
int launch_chunk_chain_fused(const ChunkParams& p, int64_t dk, int io_dtype, int state_dtype, int64_t groups,
                             hipStream_t stream);


}  // namespace gdn
