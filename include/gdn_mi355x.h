/*
 * gdn_mi355x.h -- C ABI of libgdn_mi355x.so, the gfx950 (MI355X) kernels of
 * the Gated DeltaNet linear-attention hot path.
 *
 * Every entry point:
 *   - takes plain device pointers, element strides (in elements, not bytes,
 *     unless a name says _bytes), sizes and a hipStream_t passed as void*;
 *   - launches asynchronously on that stream, performs no host<->device
 *     synchronisation and never allocates, so it is HIP-graph capturable;
 *   - returns GDN_OK or an error code and records a message readable through
 *     gdn_last_error() (thread-local).  Nothing throws across the ABI.
 *
 * Index arrays (slots, cu_seqlens, ...) may be int32 or int64 (GDN_I32 /
 * GDN_I64); int64 entries must lie in the int32 range (the kernels read
 * their low word).  Negative slots are sentinels: a negative read slot means "zero
 * state" where the reference does so, a negative write slot means "skip".
 * Element types are GDN_F32, GDN_BF16 or GDN_F16.
 *
 * Citations are to the reference repository (dakingffo/LogSSMs), paths below
 * python/logssms/ unless rooted at csrc/.
 */
#ifndef GDN_MI355X_H
#define GDN_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { GDN_F32 = 0, GDN_BF16 = 1, GDN_F16 = 2 };
enum { GDN_I32 = 0, GDN_I64 = 1 };
enum { GDN_OK = 0, GDN_ERR_INVALID = 1, GDN_ERR_UNSUPPORTED = 2, GDN_ERR_HIP = 3 };

/* Message of the last failing call on this thread ("" if none). */
const char* gdn_last_error(void);
/* ABI version of this library (bumped on any signature change). */
int gdn_abi_version(void);

/*
 * Packed varlen causal depthwise conv1d + SiLU with conv-window snapshots.
 * Replaces kernel/linear_attention/packed_conv.py:143-192 (packed_causal_conv1d,
 * Triton kernel _packed_conv_kernel :53-140).
 *   x        [T, C] element (x_row_stride, x_col_stride), dtype
 *   weight   [C, W] contiguous (the reference's [C, 1, W]), dtype
 *   bias     [C] or NULL, dtype
 *   history  [N, C, W-1] contiguous, dtype: inputs before each sequence
 *   cu_seqlens [N+1]
 *   out      [T, C] contiguous, dtype: SiLU(round_dtype(sum_tap w x + b))
 *   conv_state [slots, L, C, W-1] (slot/layer strides, inner contiguous) or NULL;
 *     token_slots[T] (>=0: write the window ending at t), final_slots[N] or NULL
 *     (>=0: write the window of the last token of sequence n).
 *   boundary0/1 + scale0/1/2: per-channel-range input scale (packed_conv.py:24-30);
 *     pass C, C, 1, 1, 1 for none.
 */
int gdn_packed_causal_conv1d(const void* x, int64_t x_row_stride, int64_t x_col_stride, int dtype,
                             const void* weight, const void* bias, const void* history,
                             const void* cu_seqlens, int cu_dtype, int64_t num_seqs,
                             int64_t total_tokens, int64_t channels, int kernel_width, void* out,
                             void* conv_state, int64_t state_slot_stride, int64_t state_layer_stride,
                             int64_t layer, const void* token_slots, int token_slots_dtype,
                             const void* final_slots, int final_slots_dtype, int64_t boundary0,
                             int64_t boundary1, float scale0, float scale1, float scale2, void* stream);

/*
 * prepare_gdn: q,k <- x * rsqrt(sum x^2 + 1e-6); v copied; g = -exp(A_log) *
 * softplus(gate + dt_bias) (threshold 20); beta <- sigmoid(beta).
 * Replaces kernel/fused.py:120-158 (Triton _prepare_gdn_kernel :53-117).
 *   query/key [B, T, H, dk] with 4 element strides each (qs[4], ks[4]), value
 *   [B, T, HV, dv] with vs[4]; io dtype.  gate/beta [B, T, HV] with 3 strides,
 *   own dtypes.  A_log/dt_bias [HV] with 1 stride, own dtypes.
 *   Outputs contiguous: q_out/k_out [B,T,H,dk], v_out [B,T,HV,dv] (io dtype),
 *   g_out/beta_out [B,T,HV] fp32.
 */
int gdn_prepare(const void* query, const int64_t* qs, const void* key, const int64_t* ks,
                const void* value, const int64_t* vs, int io_dtype, const void* gate,
                const int64_t* gs, int gate_dtype, const void* beta, const int64_t* bs, int beta_dtype,
                const void* A_log, int64_t a_stride, int a_dtype, const void* dt_bias, int64_t dt_stride,
                int dt_dtype, int64_t batch, int64_t tokens, int64_t H, int64_t HV, int64_t dk, int64_t dv,
                void* q_out, void* k_out, void* v_out, float* g_out, float* beta_out, void* stream);

/*
 * Fused prefill front end (one pass over mixed_qkv): conv-history gather from
 * the conv pool (layers/linear_attention_backend/gdn.py:107-113), packed conv +
 * SiLU (packed_conv.py), q/k/v split (gdn.py:51-72) and prepare_gdn
 * (fused.py).  Bitwise the same rounding chain as running the two reference
 * ops back to back.  The conv windows are not written here: a window slot may
 * be the baseline slot another workgroup of this launch still reads its
 * history from (a prefill resuming mid-page), so the caller writes them with
 * gdn_conv_snapshots after this launch, as the reference gathers the history
 * before its conv writes any window (gdn.py:107-112).
 *   mixed [T, C] strided, C = 2*H*dk + HV*dv; gate/beta [T, HV] strided (2 strides).
 *   conv_state [slots, L, C, W-1] (read only); baseline_slots[N] (<0: zero history).
 *   Outputs: q_out/k_out [T, H, dk], v_out [T, HV, dv] (dtype), g_out/beta_out [T, HV] fp32.
 */
int gdn_prefill_frontend(const void* mixed, int64_t row_stride, int64_t col_stride, int dtype,
                         const void* weight, const void* bias, int kernel_width, const void* cu_seqlens,
                         int cu_dtype, int64_t num_seqs, int64_t total_tokens, int64_t H, int64_t HV,
                         int64_t dk, int64_t dv, const void* conv_state, int64_t state_slot_stride,
                         int64_t state_layer_stride, int64_t layer, const void* baseline_slots,
                         int baseline_dtype, const void* gate, int64_t gate_row_stride, int64_t gate_head_stride,
                         int gate_dtype, const void* beta, int64_t beta_row_stride,
                         int64_t beta_head_stride, int beta_dtype, const void* A_log, int a_dtype,
                         const void* dt_bias, int dt_dtype, void* q_out, void* k_out, void* v_out,
                         float* g_out, float* beta_out, void* stream);

/*
 * Chunked gated delta rule over packed varlen sequences with state-pool I/O.
 * Replaces vendor/fla/gated_delta.py:15-82
 * (chunk_gated_delta_rule_to_cache -> cumsum, kkt/solve, wy, fwd_h, fwd_o
 * kernels) and kernel/linear_attention/state_io.py:15-80 (ChunkStateIO,
 * _chunk_state_pointer, _store_chunk_state_tile).
 *   q, k [T, H, dk], v [T, HV, dv] contiguous, io dtype (bf16 or f16);
 *   g, beta [T, HV] fp32 contiguous (prepared: natural-log decay, beta in [0,1]).
 *   state pool [slots, L, HV, dk, dv] (slot/layer/head strides, inner
 *   contiguous), state_dtype; read_slots[N] (<0: zero initial state);
 *   chunk_write_slots[NT] indexed by global checkpoint interval: one per
 *   chunk_size (16, 32 or 64) tokens of each sequence, the last one of a
 *   sequence possibly shorter (<0: skip);
 *   final_write_slots[N] or NULL.
 *   out [T, HV, dv] io dtype; v_new [T, HV, dv] or NULL (u - w h of the reference).
 * Frame-table state (LogState payload frames, kernel/linear_attention/
 * layout.py:11-26) when frames != NULL: state is the frame storage
 * (num_frames frames of frame_bytes), the strides are ignored, and head h of
 * layer `layer` in slot s starts at logical byte (layer HV + h) head_bytes of
 * the slot; logical byte x lies in frame frames[s frames_per_slot + x /
 * frame_bytes] at offset x % frame_bytes.  head_bytes >= dk dv elt, and either
 * divides frame_bytes or is a multiple of it (then frame_bytes must be a
 * multiple of 16 state rows, 16 dv elt).  frames has table_rows rows
 * (slots); a slot >= table_rows, like a frame entry < 0 or >= num_frames,
 * reads as zero state and takes no write (table_rows is ignored without
 * frames).  dk in {32, 64, 128}; dv 32 or a multiple of 64.
 */
int gdn_chunk_gated_delta_rule(const void* q, const void* k, const void* v, int io_dtype, const float* g,
                               const float* beta, const void* cu_seqlens, int cu_dtype, int64_t num_seqs,
                               int64_t total_tokens, int64_t H, int64_t HV, int64_t dk, int64_t dv,
                               void* state, int state_dtype, int64_t slot_stride, int64_t layer_stride,
                               int64_t head_stride, int64_t layer, const void* read_slots, int read_dtype,
                               const void* chunk_write_slots, int chunk_write_dtype,
                               const void* final_write_slots, int final_write_dtype, int64_t chunk_size,
                               const void* frames, int frames_dtype, int64_t table_rows, int64_t frames_per_slot,
                               int64_t frame_bytes, int64_t head_bytes, int64_t num_frames, void* out, void* v_new,
                               float scale, void* stream);

/*
 * gdn_chunk_gated_delta_rule on frame storage with the token log's value rows
 * written by the chunk kernel itself: replaces the v_new output of the chunked
 * rule (vendor/fla/chunk_delta_h.py:183-192) followed by the value-row stores
 * of the log (kernel/linear_attention/state_io.py:83-126), so v' never makes
 * an HBM round trip.  Arguments as gdn_chunk_gated_delta_rule (the state is
 * the frame storage, frames required; no strides, no v_new) plus the log
 * arguments of gdn_store_chunk_log: for every token t with log_slots[t] >= 0
 * and 0 <= token_offsets[t] < page_size, v'[t, h, :] goes to the value row
 * (h, position) of that slot's log.  Keys and gates are then stored by
 * gdn_store_chunk_log with v_new = NULL.  Log slots >= table_rows take no
 * write.  Needs frames of a multiple of 2 min(dv, 64) bytes and io dtype ==
 * state dtype; returns status 2 (unsupported, nothing launched) otherwise.
 */
int gdn_chunk_gated_delta_rule_logged(const void* q, const void* k, const void* v, int io_dtype, const float* g,
                                      const float* beta, const void* cu_seqlens, int cu_dtype, int64_t num_seqs,
                                      int64_t total_tokens, int64_t H, int64_t HV, int64_t dk, int64_t dv,
                                      void* state, int state_dtype, int64_t layer, const void* read_slots,
                                      int read_dtype, const void* chunk_write_slots, int chunk_write_dtype,
                                      const void* final_write_slots, int final_write_dtype, int64_t chunk_size,
                                      const void* frames, int frames_dtype, int64_t table_rows,
                                      int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes,
                                      int64_t num_frames, const void* log_slots, int log_dtype, const void* token_offsets,
                                      int offsets_dtype, int64_t key_heads, int64_t num_layers, int64_t page_size,
                                      void* out, float scale, void* stream);

/*
 * LogState token log of the chunked prefill: replaces the log stores of
 * kernel/linear_attention/state_io.py:83-126 (_store_chunk_log, called from
 * vendor/fla/chunk_delta_h.py:183-192 when a ChunkLogIO is given), with the
 * log layout of kernel/linear_attention/layout.py:29-80 (log_pointer).
 * For every token t with log_slots[t] >= 0 and 0 <= token_offsets[t] <
 * page_size, and every value head h:
 *   v_new[t, h, :] -> the value row (h, position) of the slot's log (skipped
 *     when v_new is NULL: gdn_chunk_gated_delta_rule_logged wrote them);
 *   key[t, h / (HV / H), :] -> key row (h / (HV / key_heads), position) when
 *     h % (HV / key_heads) == 0;
 *   gate[t, h] (fp32) -> float (layer page_size + position) HV + h of the
 *     decay record decay_frames[slot] = {frame, record}.
 * The log of a slot holds, in 16-bit elements from logical byte 0, granule
 * (position / granularity), layer, then keys [key_heads, granularity, dk]
 * and values [HV, granularity, dv]; logical byte x lies in frame
 * frames[slot frames_per_slot + x / frame_bytes] at offset x % frame_bytes
 * (storage = num_frames frames).  frames and decay_frames have table_rows
 * rows (slots): a slot >= table_rows, like a frame entry < 0 or >=
 * num_frames, takes no write.  v_new and key [T, ., d] contiguous in the
 * storage's 16-bit dtype.
 */
int gdn_store_chunk_log(void* storage, const void* frames, int frames_dtype, int64_t table_rows,
                        int64_t frames_per_slot, int64_t frame_bytes, int64_t num_frames, const void* log_slots, int slots_dtype,
                        const void* token_offsets, int offsets_dtype, int64_t T, const void* v_new, const void* key,
                        int64_t H, int64_t HV, int64_t dk, int64_t dv, int64_t key_heads, const float* gate,
                        const void* decay_frames, int decay_dtype, int64_t decay_record_bytes, int64_t layer,
                        int64_t num_layers, int64_t granularity, int64_t page_size, void* stream);

/*
 * LogState conv windows of a packed prefill: replaces the state stores of
 * packed_causal_conv1d (kernel/linear_attention/packed_conv.py:53-133) with a
 * PackedConvStateIO that carries granules and a conv frame table.  For each
 * packed row t < cu[N] of sequence n, the raw window of the kernel_width - 1
 * inputs ending at t (rows before the sequence start from history[n], [N, C,
 * W-1]) goes to the snapshot (token_slots[t], token_granules[t]) when that
 * slot is >= 0, and the last row's window also to granule 0 of
 * final_slots[n] (when final_slots is non-NULL and the slot >= 0).
 * Snapshot addressing, table rows and input scales as in
 * gdn_conv_decode_logstate (inputs are scaled as the conv reads them, the
 * history is not).  The conv output itself comes from
 * gdn_packed_causal_conv1d (without state I/O).
 */
int gdn_conv_windows_logstate(const void* x, int64_t x_row_stride, int64_t x_col_stride, int dtype,
                              const void* history, const void* cu_seqlens, int cu_dtype, int64_t num_seqs,
                              int64_t total_tokens, int64_t channels, int kernel_width, void* storage,
                              const void* conv_frames, int frames_dtype, int64_t table_rows, int64_t num_granules,
                              int64_t frames_per_granule, int64_t frame_bytes, int64_t num_frames, int64_t layer,
                              const void* token_slots, int slots_dtype, const void* token_granules,
                              int granules_dtype, const void* final_slots, int finals_dtype, int64_t boundary0,
                              int64_t boundary1, float scale0, float scale1, float scale2, void* stream);

/*
 * LogState conv decode: replaces conv_decode (kernel/linear_attention/
 * conv_decode.py:293-352) with pool= (the conv snapshots of
 * cache/logstate/frame_pool.py in frames).  For sequence b the window of
 * channel ch is elements layer C (W-1) + ch (W-1) + s of the snapshot of
 * (read_slots[b], read_granules[b]); element e of snapshot (slot, granule) is
 * conv_frames[(slot G + granule) F + e / frame_elems] * frame_elems + e %
 * frame_elems of the storage (F = frames_per_granule; with F == 1,
 * conv_frames[slot G + granule] * frame_elems + e; layout.py:104-112).  The
 * shifted window goes to (write_slots[b], write_granules[b]) and to granule 0
 * of work_slots[b].  conv_frames has table_rows rows (slots): a negative
 * slot, a slot >= table_rows or an unmapped frame reads zeros and takes no
 * write.  Input scales as gdn_conv_decode (the scaled, rounded input also
 * enters the window).  Outputs as gdn_conv_decode; bf16 or f16 storage.
 */
int gdn_conv_decode_logstate(const void* x, int64_t x_row_stride, int64_t x_col_stride, int dtype,
                             const void* weight, const void* bias, int kernel_width, int64_t batch, int64_t channels,
                             void* storage, const void* conv_frames, int frames_dtype, int64_t table_rows,
                             int64_t num_granules, int64_t frames_per_granule, int64_t frame_bytes,
                             int64_t num_frames, int64_t layer,
                             const void* read_slots, int read_dtype, const void* read_granules,
                             int read_granules_dtype, const void* write_slots, int write_dtype,
                             const void* write_granules, int write_granules_dtype, const void* work_slots,
                             int work_dtype, void* q_out, void* k_out, void* v_out, int64_t key_dim, int split_qkv,
                             int round_conv, int64_t boundary0, int64_t boundary1, float scale0, float scale1,
                             float scale2, void* stream);

/*
 * LogState decode step: replaces fused_recurrent_gated_delta_rule_to_logstate
 * (vendor/fla/fused_recurrent.py:292-394 -> _fused_recurrent_gated_delta_kernel
 * with DIRECT_STORE, :31-288, and _gdn_replay_kernel, gdn_replay.py:17-148).
 * Per sequence b (work slot w, log slot l, page position p, replay count n <= 16):
 *   state = the work slot's state (frame-table addressed as in
 *   gdn_chunk_gated_delta_rule), plus, unless eager, the n tokens logged at
 *   positions p-n..p-1 of l replayed onto it (S = e^{sum g} S_w + sum_i k_i
 *   (e^{sum_{j>i} g_j} v'_i)^T, the scaled v' rounded to the io dtype);
 *   raw q, k [B, H, dk], v [B, HV, dv] (io dtype), gate/beta [B, HV] strided,
 *   A_log/dt_bias [HV]: q, k L2-normalised, g = -exp(A_log) softplus(gate +
 *   dt_bias), beta = sigmoid(beta); eager: the fused_recurrent step; else
 *   delta = (v - e^g S^T k) beta, o = e^g S^T q + delta (k.q);
 *   log rows at p of l: v' = delta, key (v-heads h with h % (HV/H) == 0) =
 *   normalised k, decay record float (layer page + p) HV + h = g;
 *   the new state goes to w every step (eager) or when (p + 1) % 16 == 0.
 * The log layout and decay records are those of gdn_store_chunk_log with
 * key_heads = H.  Work and log slots >= table_rows (the rows of both frame
 * tables) are unmapped, as negative ones.  out [B, HV, dv] io dtype.
 */
int gdn_recurrent_logstate(const void* q, const void* k, const void* v, int io_dtype, const void* gate,
                           int64_t gate_b_stride, int64_t gate_h_stride, int gate_dtype, const void* beta,
                           int64_t beta_b_stride, int64_t beta_h_stride, int beta_dtype, const void* A_log,
                           int a_dtype, const void* dt_bias, int dt_dtype, int64_t batch, int64_t H, int64_t HV,
                           int64_t dk, int64_t dv, void* storage, const void* payload_frames, int frames_dtype,
                           int64_t table_rows, int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes,
                           int64_t num_frames, const void* decay_frames, int decay_dtype, int64_t decay_record_bytes,
                           const void* work_slots, int work_dtype, const void* log_slots, int log_dtype,
                           const void* token_offsets, int offsets_dtype, const void* replay_counts, int counts_dtype,
                           int64_t layer, int64_t num_layers, int64_t granularity, int64_t page_size, int eager,
                           void* out, float scale, void* stream);

/*
 * LogState state reconstruction: replaces restore_log_state_chains
 * (kernel/linear_attention/logstate.py:59-88 -> csrc/jit/logstate_construction.cu
 * restore).  Task i: the state of base_slots[i] (< 0: zero) for every layer
 * and value head, then for each segment j in [segment_offsets[i],
 * segment_offsets[i+1]) the tokens at positions log_begins[j] ..
 * log_ends[j] - 1 of log slot log_slots[j] in order, S <- e^g S + k v'^T
 * (the log layout and decay records of gdn_store_chunk_log, key_heads log
 * key heads); the result goes to output_slots[i].  Slot states use the frame
 * layout of gdn_chunk_gated_delta_rule; dtype bf16 or f16.  Outputs must not
 * be read by another task of the same call.  frame_bytes must hold one logged
 * row (2 max(dk, dv) bytes), so that a row spans at most two frames
 * (GDN_ERR_INVALID otherwise).  Slots >= table_rows (the rows of both frame
 * tables) read as zero states, contribute no segment and take no write.
 */
int gdn_logstate_restore(void* storage, const void* payload_frames, int frames_dtype, int64_t table_rows,
                         int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes, int64_t num_frames, const void* decay_frames,
                         int decay_dtype, int64_t decay_record_bytes, int64_t num_layers, int64_t HV,
                         int64_t key_heads, int64_t dk, int64_t dv, int64_t granularity, int64_t page_size, int dtype,
                         const int32_t* base_slots, const int32_t* segment_offsets, const int32_t* log_slots,
                         const int32_t* log_begins, const int32_t* log_ends, const int32_t* output_slots,
                         int64_t num_tasks, void* stream);

/*
 * LogState state copy: replaces copy_states (kernel/linear_attention/logstate.py:118-128
 * -> logstate_construction.cu copy): the states of every layer and value
 * head of sources[i] to destinations[i]; pairs with a slot < 0 or >=
 * table_rows are skipped.
 */
int gdn_logstate_copy_states(void* storage, const void* payload_frames, int frames_dtype, int64_t table_rows,
                             int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes, int64_t num_frames, int64_t num_layers,
                             int64_t HV, int64_t dk, int64_t dv, int dtype, const int32_t* sources,
                             const int32_t* destinations, int64_t count, void* stream);

/*
 * LogState conv snapshot copy: replaces copy_conv_snapshots
 * (kernel/linear_attention/conv_copy.py:31-52).  The snapshot_bytes of
 * (source_slots[i], source_granules[i]) to (output_slots[i],
 * output_granules[i]); conv_frames is the [table_rows, granules,
 * frames_per_snapshot] frame table, snapshot byte x in frame
 * conv_frames[slot, granule, x / frame_bytes] at x % frame_bytes.  Pairs with
 * a negative or out-of-range slot or granule are skipped.
 */
int gdn_logstate_copy_conv(void* storage, const void* conv_frames, int frames_dtype, int64_t table_rows,
                           int64_t granules, int64_t frames_per_snapshot, int64_t frame_bytes, int64_t num_frames,
                           int64_t snapshot_bytes, const void* source_slots, int source_slots_dtype,
                           const void* source_granules, int source_granules_dtype, const void* output_slots,
                           int output_slots_dtype, const void* output_granules, int output_granules_dtype,
                           int64_t count, void* stream);

/*
 * LogState masked conv store: replaces store_conv
 * (kernel/linear_attention/masked_store.py:58-72).  Row i of values (row_bytes,
 * one layer's conv window) to bytes [layer row_bytes, (layer + 1) row_bytes)
 * of the (slots[i], slot_granules[i]) snapshot; rows with a negative slot are
 * skipped.
 */
int gdn_logstate_store_conv(void* storage, const void* conv_frames, int frames_dtype, int64_t table_rows,
                            int64_t granules, int64_t frames_per_snapshot, int64_t frame_bytes, int64_t num_frames,
                            const void* slots, int slots_dtype, const void* slot_granules, int granules_dtype,
                            int64_t count, int64_t layer, int64_t row_bytes, const void* values, void* stream);

/*
 * LogState masked state store: replaces store_states
 * (kernel/linear_attention/masked_store.py:45-55).  values [count, HV,
 * state_bytes] to head h of layer `layer` of slots[i] (logical byte
 * (layer HV + h) head_bytes of the slot's payload frames); rows with a
 * negative slot are skipped.
 */
int gdn_logstate_store_states(void* storage, const void* payload_frames, int frames_dtype, int64_t table_rows,
                              int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes, int64_t num_frames,
                              const void* slots, int slots_dtype, int64_t count, int64_t layer, int64_t HV,
                              int64_t state_bytes, const void* values, void* stream);

/*
 * The GDN prefill of one layer (layers/linear_attention_backend/gdn.py:100-150:
 * history gather, packed_causal_conv1d, split, prepare_gdn,
 * chunk_gated_delta_rule_to_cache) as two launches whose results equal
 * gdn_prefill_frontend followed by gdn_chunk_gated_delta_rule and
 * gdn_conv_snapshots bit for bit:
 *   1. gdn_prefill_qk: the q/k channels only -> normalised q, k, plus the
 *      prepared gates g, beta.
 *   2. gdn_prefill_fused: the chunk kernel, with the v conv + SiLU done by its
 *      staging waves from the projections (v never reaches HBM), and the conv
 *      windows of the snapshot rows written into the pool once the histories
 *      are read (a snapshot may overwrite a baseline slot).
 * Each returns GDN_ERR_UNSUPPORTED, launching nothing, for shapes outside it:
 * kernel_width 4, bf16/f16 io, dk in {32, 64, 128}, dv % 64 == 0, 16-byte
 * aligned rows and conv pool, fp32 or io-typed state.
 *
 * gdn_prefill_qk: mixed [T, 2 H dk + ...] (row_stride, unit column stride);
 *   weight [conv_dim, 4]; conv_state [slots, L, conv_dim, 3] (slot/layer
 *   strides); baseline_slots[N] (<0: zero history); q_out, k_out [T, H, dk]
 *   in out_dtype: the io dtype, or GDN_F16 for the f16 MFMA operands that
 *   gdn_prefill_fused reads (the io-rounded values, converted toward zero);
 *   gate, beta [T, HV] (row/head strides, any float dtype), A_log, dt_bias
 *   [HV] -> g_out, beta_out [HV, T] fp32, head-major so that the chunk
 *   kernel's per-head gate loads are contiguous (prepare_gdn,
 *   kernel/fused.py:105-117).
 */
int gdn_prefill_qk(const void* mixed, int64_t row_stride, int io_dtype, const void* weight, int kernel_width,
                   const void* cu_seqlens, int cu_dtype, int64_t num_seqs, int64_t total_tokens, int64_t H,
                   int64_t dk, const void* conv_state, int64_t conv_slot_stride, int64_t conv_layer_stride,
                   int64_t layer, const void* baseline_slots, int baseline_dtype, void* q_out, void* k_out,
                   int out_dtype, int64_t HV, const void* gate, int64_t gate_row_stride, int64_t gate_head_stride,
                   int gate_dtype, const void* beta, int64_t beta_row_stride, int64_t beta_head_stride,
                   int beta_dtype, const void* A_log, int a_dtype, const void* dt_bias, int dt_dtype, float* g_out,
                   float* beta_out, void* stream);

/*
 * gdn_prefill_fused: q, k (f16), g, beta ([HV, T]) from gdn_prefill_qk; mixed, weight,
 * conv_state and baseline_slots as there (the v channels' history, and the
 * initial recurrent state, come from baseline_slots); state pool,
 * chunk/final write slots and out as in gdn_chunk_gated_delta_rule;
 * snapshot_rows/slots[snapshot_count] as gdn_conv_snapshots' rows/slots
 * (the windows it would write, written by this launch; count 0: none).
 */
int gdn_prefill_fused(const void* q, const void* k, const void* mixed, int64_t row_stride, int io_dtype,
                      const void* weight, int kernel_width, const void* cu_seqlens, int cu_dtype, int64_t num_seqs,
                      int64_t total_tokens, int64_t H, int64_t HV, int64_t dk, int64_t dv, void* conv_state,
                      int64_t conv_slot_stride, int64_t conv_layer_stride, const float* g, const float* beta,
                      void* state, int state_dtype, int64_t slot_stride, int64_t layer_stride, int64_t head_stride,
                      int64_t layer, const void* baseline_slots, int baseline_dtype, const void* chunk_write_slots,
                      int chunk_write_dtype, const void* final_write_slots, int final_write_dtype,
                      const void* snapshot_rows, int rows_dtype, const void* snapshot_slots, int slots_dtype,
                      int64_t snapshot_count, void* out, float scale, void* stream);

/*
 * gdn_conv_snapshots: for each i < count with slots[i] >= 0, conv_state[slots[i],
 * layer] = the kernel_width - 1 raw inputs ending at packed row rows[i] (oldest
 * first), positions before the sequence start taken from
 * conv_state[baseline_slots[seq]] (zeros for a negative baseline).  Replaces
 * the token_slots writes of packed_conv.py:111-133.  16-bit dtype.
 */
int gdn_conv_snapshots(const void* mixed, int64_t row_stride, int dtype, const void* cu_seqlens, int cu_dtype,
                       int64_t num_seqs, int64_t total_tokens, int64_t channels, int kernel_width, void* conv_state,
                       int64_t state_slot_stride, int64_t state_layer_stride, int64_t layer,
                       const void* baseline_slots, int baseline_dtype, const void* rows, int rows_dtype,
                       const void* slots, int slots_dtype, int64_t count, void* stream);

/*
 * Single-token conv update from slot windows.  Replaces
 * kernel/linear_attention/conv_decode.py:293-352 (Triton _conv_decode_kernel
 * :25-289), standard-state mode.
 *   x [B, C] strided; conv_state [slots, L, C, W-1]; read/write slots [B] with strides.
 *   Writes conv_state[write] = [window[1:], x] and the SiLU output either split
 *   (q_out [B, key_dim], k_out [B, key_dim], v_out [B, C - 2 key_dim]) or
 *   whole (q_out [B, C]; split_qkv = 0).
 */
int gdn_conv_decode(const void* x, int64_t x_row_stride, int64_t x_col_stride, int dtype,
                    const void* weight, const void* bias, int kernel_width, int64_t batch,
                    int64_t channels, void* conv_state, int64_t state_slot_stride,
                    int64_t state_layer_stride, int64_t layer, const void* read_slots,
                    int64_t read_stride, int read_dtype, const void* write_slots, int64_t write_stride,
                    int write_dtype, void* q_out, void* k_out, void* v_out, int64_t key_dim,
                    int split_qkv, int round_conv, int64_t boundary0, int64_t boundary1, float scale0,
                    float scale1, float scale2, void* stream);

/*
 * Recurrent gated delta rule over T steps per sequence, raw inputs (q/k are
 * L2-normalised, g = -exp(A_log) softplus(gate + dt_bias) and beta = sigmoid(beta)
 * inside).  Replaces vendor/fla/fused_recurrent.py:396-458
 * (fused_recurrent_gated_delta_rule_to_slots) and :461-550
 * (fused_recurrent_gated_delta_rule).
 *   q, k [B, T, H, dk], v [B, T, HV, dv] contiguous, io dtype; gate/beta
 *   [B, T, HV] with strides (b, t, h), own dtypes; A_log/dt_bias [HV] contiguous.
 *   Slot mode (init_state == NULL): state pool [slots, L, HV, dk, dv];
 *     initial state from pool[read_slots[b]]; write_t_stride == 0 writes the
 *     final state to pool[write_slots[b]] (decode), otherwise every step t to
 *     pool[write_slots[b*write_b_stride + t*write_t_stride]] (skip <0).
 *   Plain mode (init_state != NULL): init_state [B, HV, dk, dv] contiguous,
 *     every step to states_out [B, T, HV, dk, dv] (state_dtype).
 *   out [B, T, HV, dv] io dtype.
 */
int gdn_fused_recurrent(const void* q, const void* k, const void* v, int io_dtype, const void* gate,
                        int64_t gate_b_stride, int64_t gate_t_stride, int64_t gate_h_stride,
                        int gate_dtype, const void* beta, int64_t beta_b_stride, int64_t beta_t_stride,
                        int64_t beta_h_stride, int beta_dtype, const void* A_log, int a_dtype,
                        const void* dt_bias, int dt_dtype, int64_t batch, int64_t steps, int64_t H,
                        int64_t HV, int64_t dk, int64_t dv, void* state, int state_dtype,
                        int64_t slot_stride, int64_t layer_stride, int64_t head_stride, int64_t layer,
                        const void* read_slots, int64_t read_stride, int read_dtype,
                        const void* write_slots, int64_t write_b_stride, int64_t write_t_stride,
                        int write_dtype, const void* init_state, void* states_out, void* out,
                        float scale, void* stream);

/*
 * Fused decode / spec-decode verify step of the backend: conv over the
 * token(s) from the conv pool window + recurrent update from the state pool,
 * one pass.  Replaces layers/linear_attention_backend/gdn.py:222-265
 * (_forward_decode: conv_decode + fused_recurrent_..._to_slots) when steps == 1
 * and write_t_stride == 0, and gdn.py:151-220 (_forward_verify: torch conv,
 * conv snapshots via index_copy_, fused_recurrent_gated_delta_rule, store_state)
 * for one length group when write_t_stride != 0.
 *   mixed [rows, C] strided; row of (b, t) = row_index[b*steps + t] if
 *   row_index != NULL else b*steps + t (the verify group's row_indices).
 *   gate/beta [rows, HV] strided (row, head).
 *   Decode rounds nothing before SiLU (conv_decode GDN mode); verify rounds the
 *   conv output to dtype before SiLU like the reference's torch conv1d.
 *   out [B*steps, HV, dv] dtype, written in (b, t) order at out_row = row index.
 *   steps <= 16.
 */
int gdn_fused_conv_recurrent(const void* mixed, int64_t row_stride, int64_t col_stride, int dtype,
                             const void* row_index, int row_index_dtype, const void* weight,
                             const void* bias, int kernel_width, const void* gate,
                             int64_t gate_row_stride, int64_t gate_head_stride, int gate_dtype,
                             const void* beta, int64_t beta_row_stride, int64_t beta_head_stride,
                             int beta_dtype, const void* A_log, int a_dtype, const void* dt_bias,
                             int dt_dtype, int64_t batch, int64_t steps, int64_t H, int64_t HV, int64_t dk,
                             int64_t dv, void* conv_state, int64_t conv_slot_stride,
                             int64_t conv_layer_stride, void* state, int state_dtype, int64_t slot_stride,
                             int64_t layer_stride, int64_t head_stride, int64_t layer,
                             const void* read_slots, int64_t read_stride, int read_dtype,
                             const void* write_slots, int64_t write_b_stride, int64_t write_t_stride,
                             int write_dtype, void* out, float scale, void* stream);

/*
 * pool[indices[i]] = states[i] for indices[i] >= 0 (row copy).  Replaces
 * kernel/store.py:69-83 -> csrc/jit/store.cu:143-252 (StateStoreKernel).
 *   pool_row_stride_bytes / state_row_stride_bytes: distance between rows;
 *   row_bytes: bytes per row (multiple of 16, rows 16-byte aligned).
 */
int gdn_store_state(void* pool, int64_t pool_row_stride_bytes, const void* indices, int index_dtype,
                    const void* states, int64_t state_row_stride_bytes, int64_t rows, int64_t row_bytes,
                    void* stream);

/*
 * Batched strided row copy dst_base[dst_idx[i]] <- src_base[src_idx[i]]
 * (pairs with a negative index are skipped).  A row is `segments` runs of
 * `segment_bytes` each, `segment_stride_bytes` apart (Marconi's lane stride).
 * Replaces cache/marconi/block_pool.py:90-94 (HybridBlockPool.copy_state: a
 * Python loop of .copy_() per block) and serves cache/marconi/manager.py:272-278
 * (after_forward checkpoint_copies).  src and dst may alias the same pool.
 */
int gdn_copy_rows(void* dst_base, int64_t dst_row_stride_bytes, const void* dst_idx, int dst_idx_dtype,
                  const void* src_base, int64_t src_row_stride_bytes, const void* src_idx,
                  int src_idx_dtype, int64_t pairs, int64_t segments, int64_t segment_bytes,
                  int64_t segment_stride_bytes, void* stream);

/*
 * Zero `rows` rows of the same segmented shape.  Replaces
 * cache/marconi/block_pool.py:96-99 (HybridBlockPool.zero_state).
 */
int gdn_zero_rows(void* base, int64_t row_stride_bytes, const void* idx, int idx_dtype, int64_t rows,
                  int64_t segments, int64_t segment_bytes, int64_t segment_stride_bytes, void* stream);

/*
 * Spec-decode commit by copy: for each sequence b with accepted[b] in [1, T],
 * pool[live_slots[b]] <- pool[write_slots[b, accepted[b]-1]] for one layer of
 * both the recurrent-state pool and the conv pool.  The device-side
 * alternative to the host slot remap of cache/radix/manager.py:248-268
 * (commit_speculative), for callers that keep a fixed live slot per sequence.
 *   rows are `state_row_bytes` at (slot_stride_bytes, layer offset) for the
 *   state pool and `conv_row_bytes` for the conv pool.
 */
int gdn_commit_accepted(void* state, int64_t state_slot_stride_bytes, int64_t state_layer_offset_bytes,
                        int64_t state_row_bytes, void* conv_state, int64_t conv_slot_stride_bytes,
                        int64_t conv_layer_offset_bytes, int64_t conv_row_bytes, const void* live_slots,
                        int live_dtype, const void* write_slots, int64_t write_b_stride,
                        int64_t write_t_stride, int write_dtype, const void* accepted, int accepted_dtype,
                        int64_t batch, int64_t steps, void* stream);

/* ------------------------------------------------------------------ graph metadata */

/*
 * Batched copy of `fields` small integer tensors in one launch:
 * dsts[i][j * dst_strides[i]] = srcs[i][j * src_strides[i]] for j < lengths[i]
 * (elem_sizes[i] bytes per element: 1, 2, 4 or 8; strides in elements).
 * The pointer and size tables are host arrays read at the call.  Replaces
 * copy_metadata (python/logssms/kernel/metadata.py:108-134), which
 * MixedLinearCopyPlan uses to refresh captured metadata before a replay
 * (layers/linear_attention_backend/mixed.py:127-197).
 */
int gdn_metadata_copy(const void* const* srcs, void* const* dsts, const int64_t* lengths, const int64_t* src_strides,
                      const int64_t* dst_strides, const int* elem_sizes, int fields, void* stream);

/*
 * Batched padding of contiguous integer tensors to fixed capacities in one
 * launch: dsts[i][j] = srcs[i][j] for j < lengths[i]; for lengths[i] <= j <
 * capacities[i] the value fills[i], or, when tails[i] >= 0 (a flattened pair
 * table), 0 at even and tails[i] at odd positions.  Replaces pad_metadata
 * (python/logssms/kernel/metadata.py:137-150), used by
 * prepare_mixed_linear_metadata (layers/linear_attention_backend/mixed.py:23-120).
 */
int gdn_metadata_pad(const void* const* srcs, void* const* dsts, const int64_t* lengths, const int64_t* capacities,
                     const int64_t* fills, const int64_t* tails, const int* elem_sizes, int fields, void* stream);

/*
 * LogState prefill write plan: replaces make_logstate_prefill_writes
 * (python/logssms/kernel/metadata.py:150-178), called by the LogState
 * backend's prefill metadata (layers/linear_attention_backend/logstate.py:214-272).
 * plan = int32 [conv slot | conv granule | log enabled] of `count` tokens;
 * out ([3, count], the dtype of log_slots) = [log_slots where enabled else -1 |
 * log_slots where conv slot == -2 else conv slot | token_offsets /
 * granularity where conv slot == -2 else conv granule].
 */
int gdn_logstate_prefill_writes(const void* log_slots, int slots_dtype, const void* token_offsets, int offsets_dtype,
                                const int32_t* plan, void* out, int64_t count, int64_t granularity, void* stream);

/*
 * Decode slots from the engine's prepared batch packet: replaces
 * gather_linear_slots (kernel/metadata.py:266-320), which the standard
 * (layers/linear_attention_backend/standard.py:114-117) and LogState
 * (logstate.py:113-126) backends call when batch.prepared_indices is set.
 * Request i has row = table_ids[i] and position = cached_lens[i] of the
 * [state_rows, state_width] state table (row stride state_row_stride).
 *   work_table == NULL (standard): out int64 [count, 2] = (state_table[row,
 *     position - 1], or [row, state_width - 1] when position is 0;
 *     state_table[row, position]).
 *   work_table != NULL (LogState): out int32 [4, count] = (work_table[row *
 *     work_row_stride]; state_table[row, position]; out_loc[i] mod page_size,
 *     floored; 0).
 * A row outside [0, state_rows) (or [0, work_rows) for the work slot) or a
 * position outside [0, state_width) gives -1 slots.
 */
int gdn_gather_linear_slots(const void* table_ids, int table_ids_dtype, const void* cached_lens, int cached_dtype,
                            const void* state_table, int state_dtype, int64_t state_rows, int64_t state_width,
                            int64_t state_row_stride, const void* work_table, int work_dtype, int64_t work_rows,
                            int64_t work_row_stride, const void* out_loc, int out_loc_dtype, int64_t page_size,
                            void* out, int64_t count, void* stream);

/* ------------------------------------------------------------------ output norm */

/*
 * Gated RMS normalisation of the core output, one row of `cols` channels at a
 * time: out[r, c] = (x[r, c] * rsqrt(sum_c x[r, c]^2 / cols + eps)) * weight[c]
 * * silu(gate(r, c)), computed in fp32 and stored in `dtype`.
 * Replaces rms_norm_gated (python/logssms/kernel/norm.py:151-187) and its
 * Triton kernel (:113-148), called by RMSNormGated.forward
 * (python/logssms/layers/norm.py:42-53).
 *   x, out: contiguous [rows, cols] of `dtype`.
 *   gate(r, c) = gate[(r / gate_rows) * gate_group_stride
 *                     + (r % gate_rows) * gate_row_stride + c * gate_col_stride]
 *     (element strides of the reference's gate.reshape(-1, gate_rows, cols)).
 *   weight: [cols] of `weight_dtype`.
 */
int gdn_rms_norm_gated(const void* x, int dtype, int64_t rows, int64_t cols, const void* gate, int gate_dtype,
                       int64_t gate_rows, int64_t gate_group_stride, int64_t gate_row_stride,
                       int64_t gate_col_stride, const void* weight, int weight_dtype, float eps, void* out,
                       void* stream);

/*
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops or harnesses that
 * forbid hipMalloc): the fused prefill of gdn_prefill_qk + gdn_prefill_fused
 * (with its conv windows) in one call, with the staging the first launch hands
 * to the second (f16 q/k operands, head-major g/beta) kept in a 256 MiB
 * file-scope device array of the library, one per GPU, instead of
 * caller-allocated buffers.  It allocates nothing.  Inputs, pools, slots and
 * `out` [T, HV, dv] as in those two entry points (snapshot_rows/slots[count]
 * as gdn_conv_snapshots' rows/slots; no final write slots).
 * Returns GDN_ERR_INVALID when the staging, 2 * align256(T * H * dk * 2) +
 * 2 * align256(T * HV * 4) bytes, exceeds gdn_prefill_noalloc_scratch_bytes()
 * (31,775 tokens at Qwen3-Next shape, H = 16, HV = 32, dk = 128), and
 * GDN_ERR_UNSUPPORTED for shapes outside the fused kernel.  Calls on one GPU
 * share the array: calls that overlap on one GPU (unordered streams) race.
 * The device must be current on the calling thread.
 */
int gdn_prefill_fused_noalloc(const void* mixed, int64_t row_stride, int io_dtype, const void* weight,
                              int kernel_width, const void* cu_seqlens, int cu_dtype, int64_t num_seqs,
                              int64_t total_tokens, int64_t H, int64_t HV, int64_t dk, int64_t dv, void* conv_state,
                              int64_t conv_slot_stride, int64_t conv_layer_stride, const void* gate,
                              int64_t gate_row_stride, int64_t gate_head_stride, int gate_dtype, const void* beta,
                              int64_t beta_row_stride, int64_t beta_head_stride, int beta_dtype, const void* A_log,
                              int a_dtype, const void* dt_bias, int dt_dtype, void* state, int state_dtype,
                              int64_t slot_stride, int64_t layer_stride, int64_t head_stride, int64_t layer,
                              const void* baseline_slots, int baseline_dtype, const void* chunk_write_slots,
                              int chunk_write_dtype, const void* snapshot_rows, int snapshot_rows_dtype,
                              const void* snapshot_slots, int snapshot_slots_dtype, int64_t snapshot_count, void* out,
                              float scale, void* stream);
/* Bytes of gdn_prefill_fused_noalloc's per-GPU staging array. */
int64_t gdn_prefill_noalloc_scratch_bytes(void);

#ifdef __cplusplus
}
#endif

#endif /* GDN_MI355X_H */
