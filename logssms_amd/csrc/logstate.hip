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
//
// LogState decode (vendor/fla/fused_recurrent.py:292-394, gdn_replay.py:17-148,
// conv_decode.py:293-352 with a pool):
//   * conv: the window comes from (read slot, read granule) of the conv frame
//     table, the shifted window goes to (write slot, write granule) and to
//     granule 0 of the work slot;
//   * recurrence: the work slot's state plus the n <= 16 tokens logged since
//     it (replayed from the log: S = e^{sum g} S_w + sum_i k_i (e^{sum_{j>i}
//     g_j} v'_i)^T), one step, the step's log rows, and the state written back
//     to the work slot every 16th position (every step in eager mode).
// Decode is HBM-bound: per (sequence, v-head) the work state (dk dv elements)
// and n logged (k, v') rows are read; one log row, and every 16th token the
// state, are written.
#include <type_traits>

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
  Div32 fdiv, gdiv;  // frame_bytes, gran
};

// Address of element `col` of log row `index` (a value head, or a logged key
// head) at `pos`, or null when its frame is unmapped.
__device__ __forceinline__ uint16_t* log_element(const LogParams& p, int64_t slot, int64_t pos, int64_t index,
                                                 int64_t col, bool value) {
  const int64_t key_size = p.gran * p.KH * p.K;
  const int64_t layer_size = key_size + p.gran * p.HV * p.V;
  const int64_t dim = value ? p.V : p.K;
  const uint32_t ps = static_cast<uint32_t>(pos);
  const int64_t elem = (p.gdiv.div(ps) * p.layers + p.layer) * layer_size + (value ? key_size : 0) +
                       (index * p.gran + p.gdiv.mod(ps)) * dim + col;
  const uint32_t byte = static_cast<uint32_t>(2 * elem);
  const int64_t fr = load_index(p.frames, slot * p.fps + p.fdiv.div(byte), p.frames_is64);
  if (fr < 0 || fr >= p.num_frames) return nullptr;
  return reinterpret_cast<uint16_t*>(p.storage + fr * p.frame_bytes + p.fdiv.mod(byte));
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

// grid (T): one 256-thread block per token moves all its log rows in 16-byte
// pieces (v' rows of every value head, the logged key rows) and its gates.
// Needs dk, dv multiples of 8, frames a multiple of 16 bytes and 16-byte
// aligned sources (checked by the host); a piece never straddles two frames.
constexpr int kLogThreads = 256;
__global__ __launch_bounds__(kLogThreads) void chunk_log_vec_kernel(LogParams p) {
  const int64_t t = blockIdx.x;
  const int64_t slot = load_index(p.slots, t, p.slots_is64);
  const int64_t pos = load_index(p.offsets, t, p.offsets_is64);
  if (slot < 0 || pos < 0 || pos >= p.page) return;
  const int64_t vv = p.V / 8, kv = p.K / 8;
  const int64_t group = p.HV / p.KH;  // value heads per logged key head
  const int64_t nval = p.HV * vv, total = nval + p.KH * kv;
  for (int64_t i = threadIdx.x; i < total; i += kLogThreads) {
    const bool value = i < nval;
    const int64_t j = value ? i : i - nval;
    const int64_t row = j / (value ? vv : kv), col = 8 * (j % (value ? vv : kv));
    const uint16_t* src = value ? p.v_new + (t * p.HV + row) * p.V + col
                                : p.key + (t * p.H + row * group / (p.HV / p.H)) * p.K + col;
    uint16_t* d = log_element(p, slot, pos, row, col, value);
    if (d) *reinterpret_cast<uint4*>(d) = *reinterpret_cast<const uint4*>(src);
  }
  const int64_t fr = load_index(p.decay, 2 * slot, p.decay_is64);
  const int64_t rec = load_index(p.decay, 2 * slot + 1, p.decay_is64);
  if (fr >= 0 && fr < p.num_frames && rec >= 0 && (rec + 1) * p.record_bytes <= p.frame_bytes) {
    float* d = reinterpret_cast<float*>(p.storage + fr * p.frame_bytes + rec * p.record_bytes);
    for (int64_t h = threadIdx.x; h < p.HV; h += kLogThreads) d[(p.layer * p.page + pos) * p.HV + h] = p.gate[t * p.HV + h];
  }
}

// ---------------------------------------------------------------- LogState decode

constexpr int kReplayWindow = 16;  // cache/logstate/layout.py:8
constexpr int kDecodeThreads = 256;

// Element e of the conv snapshot of (slot, granule), or null when unmapped
// (layout.py:104-112).
template <class T>
__device__ __forceinline__ T* conv_element(T* storage, const void* table, int is64, int64_t slot, int64_t granule,
                                           int64_t e, int64_t granules, int64_t cf, int64_t fe, int64_t num_frames) {
  if (slot < 0) return nullptr;
  const int64_t row = slot * granules + granule;
  if (cf == 1) {
    const int64_t fr = load_index(table, row, is64);
    if (fr < 0 || fr >= num_frames) return nullptr;
    return storage + fr * fe + e;
  }
  // e < layers C S and fe fit 32 bits (checked by the host)
  const uint32_t e32 = static_cast<uint32_t>(e), fe32 = static_cast<uint32_t>(fe);
  const int64_t fr = load_index(table, row * cf + e32 / fe32, is64);
  if (fr < 0 || fr >= num_frames) return nullptr;
  return storage + fr * fe + e32 % fe32;
}

struct ConvFrameParams {
  const void* x;
  int64_t xr, xc;
  const void* weight;
  const void* bias;
  int W;
  int64_t C;
  void* storage;
  const void* table;
  int table_is64;
  int64_t granules, cf, fe, num_frames, layer;
  const void* reads; int reads_is64;
  const void* rgran; int rgran_is64;
  const void* writes; int writes_is64;
  const void* wgran; int wgran_is64;
  const void* works; int works_is64;
  void* q; void* k; void* v;
  int64_t key_dim;
  int split, round_conv;
};

// grid (channel blocks, batch); one thread per channel.
template <class T>
__global__ __launch_bounds__(kDecodeThreads) void conv_decode_frames_kernel(ConvFrameParams p) {
  const int64_t b = blockIdx.y;
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * kDecodeThreads + threadIdx.x;
  if (ch >= p.C) return;
  const int S = p.W - 1;
  T* st = static_cast<T*>(p.storage);
  const int64_t e0 = p.layer * p.C * S + ch * S;
  const int64_t rs = load_index(p.reads, b, p.reads_is64), rg = load_index(p.rgran, b, p.rgran_is64);
  float win[8];
  for (int i = 0; i < S; ++i) {
    const T* src = conv_element(st, p.table, p.table_is64, rs, rg, e0 + i, p.granules, p.cf, p.fe, p.num_frames);
    win[i] = src ? to_f32(*src) : 0.f;
  }
  const T* x = static_cast<const T*>(p.x);
  const T* w = static_cast<const T*>(p.weight);
  const float xv = to_f32(x[b * p.xr + ch * p.xc]);
  float acc = 0.f;
  for (int i = 0; i < S; ++i) acc = fmaf(to_f32(w[ch * p.W + i]), win[i], acc);
  acc = fmaf(to_f32(w[ch * p.W + S]), xv, acc);
  if (p.bias) acc += to_f32(static_cast<const T*>(p.bias)[ch]);
  if (p.round_conv) acc = round_to<T>(acc);
  const T y = from_f32<T>(silu(acc));
  const int64_t ws = load_index(p.writes, b, p.writes_is64), wg = load_index(p.wgran, b, p.wgran_is64);
  const int64_t wk = load_index(p.works, b, p.works_is64);
  for (int i = 0; i < S; ++i) {
    const T val = from_f32<T>(i + 1 < S ? win[i + 1] : xv);
    T* d0 = conv_element(st, p.table, p.table_is64, ws, wg, e0 + i, p.granules, p.cf, p.fe, p.num_frames);
    T* d1 = conv_element(st, p.table, p.table_is64, wk, 0, e0 + i, p.granules, p.cf, p.fe, p.num_frames);
    if (d0) *d0 = val;
    if (d1) *d1 = val;
  }
  T* q = static_cast<T*>(p.q);
  if (!p.split) {
    q[b * p.C + ch] = y;
  } else if (ch < p.key_dim) {
    q[b * p.key_dim + ch] = y;
  } else if (ch < 2 * p.key_dim) {
    static_cast<T*>(p.k)[b * p.key_dim + ch - p.key_dim] = y;
  } else {
    static_cast<T*>(p.v)[b * (p.C - 2 * p.key_dim) + ch - 2 * p.key_dim] = y;
  }
}

// ---- LogState prefill conv windows (packed_conv.py:53-133 with LOGSTATE):
// the raw window ending at packed row t goes to (token_slots[t],
// token_granules[t]) when that slot is >= 0, and a sequence's last window to
// granule 0 of final_slots[seq]; window rows before the sequence start come
// from history [N, C, W-1].
struct ConvWindowParams {
  const void* x;
  int64_t xr, xc;
  const void* history;
  const void* cu; int cu_is64;
  int64_t N, T, C;
  int S;
  void* storage;
  const void* table; int table_is64;
  int64_t granules, cf, fe, num_frames, layer;
  const void* slots; int slots_is64;
  const void* gran; int gran_is64;
  const void* finals; int finals_is64;
};

// grid (T, channel blocks)
template <class T>
__global__ __launch_bounds__(kDecodeThreads) void conv_windows_frames_kernel(ConvWindowParams p) {
  const int64_t t = blockIdx.x;
  const int64_t ch = static_cast<int64_t>(blockIdx.y) * kDecodeThreads + threadIdx.x;
  if (ch >= p.C || t >= load_index(p.cu, p.N, p.cu_is64)) return;
  const int64_t slot = load_index(p.slots, t, p.slots_is64);
  const int64_t n = find_sequence(p.cu, p.cu_is64, p.N, t);
  const int64_t begin = load_index(p.cu, n, p.cu_is64), end = load_index(p.cu, n + 1, p.cu_is64);
  const int64_t fin = p.finals && t == end - 1 ? load_index(p.finals, n, p.finals_is64) : -1;
  if (slot < 0 && fin < 0) return;
  const int64_t granule = slot >= 0 ? load_index(p.gran, t, p.gran_is64) : 0;
  const T* x = static_cast<const T*>(p.x);
  const T* hist = static_cast<const T*>(p.history) + (n * p.C + ch) * p.S;
  T* st = static_cast<T*>(p.storage);
  const int64_t e0 = p.layer * p.C * p.S + ch * p.S;
  for (int j = 0; j < p.S; ++j) {
    const int64_t pos = t - (p.S - 1) + j;
    const T v = pos >= begin ? x[pos * p.xr + ch * p.xc] : hist[pos - begin + p.S];
    T* d0 = conv_element(st, p.table, p.table_is64, slot, granule, e0 + j, p.granules, p.cf, p.fe, p.num_frames);
    T* d1 = conv_element(st, p.table, p.table_is64, fin, 0, e0 + j, p.granules, p.cf, p.fe, p.num_frames);
    if (d0) *d0 = v;
    if (d1) *d1 = v;
  }
}

struct LogDecodeParams {
  const void* q; const void* k; const void* v;
  const void* gate; int64_t gate_b, gate_h; int gate_dtype;
  const void* beta; int64_t beta_b, beta_h; int beta_dtype;
  const void* A_log; int a_dtype;
  const void* dt_bias; int dt_dtype;
  int64_t H, HV;
  char* storage;
  const void* frames; int frames_is64;
  int64_t fps, frame_bytes, head_bytes, num_frames;
  const void* decay; int decay_is64;
  int64_t record_bytes;
  const void* work; int work_is64;
  const void* logs; int logs_is64;
  const void* offsets; int offsets_is64;
  const void* counts; int counts_is64;
  int64_t layer, layers, gran, page;
  int eager;
  void* out;
  float scale;
  Div32 fdiv, gdiv;  // frame_bytes, gran
};

// Element (row, col) of the state of value head h in slot s: logical byte
// (layer HV + h) head_bytes + (row dv + col) elt of the slot, one frame lookup
// per row (the host checks that no row straddles two frames).
template <class T>
__device__ __forceinline__ T* state_row(const LogDecodeParams& p, int64_t s, int64_t h, int64_t row, int DV) {
  if (s < 0) return nullptr;
  const uint32_t x = static_cast<uint32_t>((p.layer * p.HV + h) * p.head_bytes + row * DV * static_cast<int64_t>(sizeof(T)));
  const int64_t fr = load_index(p.frames, s * p.fps + p.fdiv.div(x), p.frames_is64);
  if (fr < 0 || fr >= p.num_frames) return nullptr;
  return reinterpret_cast<T*>(p.storage + fr * p.frame_bytes + p.fdiv.mod(x));
}

// 16-bit log element (the log layout of chunk_log_kernel, key heads = H).
template <class T>
__device__ __forceinline__ T* decode_log(const LogDecodeParams& p, int64_t slot, int64_t pos, int64_t index,
                                         int64_t col, bool value, int DK, int DV) {
  const int64_t key_size = p.gran * p.H * DK;
  const int64_t layer_size = key_size + p.gran * p.HV * DV;
  const uint32_t ps = static_cast<uint32_t>(pos);
  const int64_t elem = (p.gdiv.div(ps) * p.layers + p.layer) * layer_size + (value ? key_size : 0) +
                       (index * p.gran + p.gdiv.mod(ps)) * (value ? DV : DK) + col;
  const uint32_t byte = static_cast<uint32_t>(2 * elem);
  const int64_t fr = load_index(p.frames, slot * p.fps + p.fdiv.div(byte), p.frames_is64);
  if (fr < 0 || fr >= p.num_frames) return nullptr;
  return reinterpret_cast<T*>(p.storage + fr * p.frame_bytes + p.fdiv.mod(byte));
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// Barrier for LDS traffic only: global loads in flight stay in flight.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Two 16-bit values of a dword as floats, and back (round to nearest even).
template <class T> __device__ __forceinline__ void split2(uint32_t w, float& a, float& b);
template <> __device__ __forceinline__ void split2<bf16>(uint32_t w, float& a, float& b) {
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
}
template <> __device__ __forceinline__ void split2<f16>(uint32_t w, float& a, float& b) {
  const f16* h = reinterpret_cast<const f16*>(&w);
  a = static_cast<float>(h[0]);
  b = static_cast<float>(h[1]);
}

// N = 4 or 8 consecutive 16-bit values as N / 2 dwords.
template <int N> __device__ __forceinline__ void load_words(const void* src, uint32_t (&w)[N / 2]) {
  if constexpr (N == 8) {
    const uint4 v = *reinterpret_cast<const uint4*>(src);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(src);
    w[0] = v.x; w[1] = v.y;
  }
}
template <int N> __device__ __forceinline__ void store_words(void* dst, const uint32_t (&w)[N / 2]) {
  if constexpr (N == 8)
    *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
  else
    *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
}

typedef short s4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));

// 16 x 16 x 16 products on 16-bit operands, fp32 accumulation: lane l holds
// row (A) / column (B) l % 16 and k = 4 (l / 16) .. + 3; the result gives lane
// l column l % 16, rows 4 (l / 16) .. + 3.
template <class T> __device__ __forceinline__ f4_t mma16(uint2 a, uint2 b, f4_t c);
template <> __device__ __forceinline__ f4_t mma16<bf16>(uint2 a, uint2 b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4_t, a), __builtin_bit_cast(s4_t, b), c, 0, 0, 0);
}
template <> __device__ __forceinline__ f4_t mma16<f16>(uint2 a, uint2 b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4_t, a), __builtin_bit_cast(h4_t, b), c, 0, 0, 0);
}

// Sum over the 16 lanes of a row (every lane of the row receives it).
__device__ __forceinline__ float row16_sum(float v) { return head_sum<16>(v); }

constexpr int kReplayLd = kReplayWindow + 4;  // LDS row of one feature over the replay window

// grid (batch x HV), DV / (16 TPW) waves.  The state is held transposed,
// T = S^T (dv x dk), in 16 x 16 MFMA result tiles: wave w owns the TPW dv row
// tiles TPW w .. and every dk column, lane l the dk column 16 it + l % 16 of
// tile it and the dv rows 16 jt + 4 (l / 16) .. + 3 of row tile jt -- four
// consecutive elements of one state row in memory, moved as 8 bytes.  Two
// row tiles per wave (d_v = 128) keep 4 waves per block and 32 KiB of state
// in flight per 4 waves, which sets the block's share of HBM bandwidth.  The replayed tokens' rank-n update
// T += V'^T K runs as one 16-deep MFMA per tile from keys and scaled v' rows
// staged feature-major in LDS; S^T k and S^T q are per-lane FMAs and a
// 16-lane DPP sum, complete inside each wave.  Every global load is issued
// before the first wait; the only barrier guards the staged replay rows.
template <int DK, int DV, class T>
__global__ __launch_bounds__(DV * 4 / (DV >= 128 ? 2 : 1)) __attribute__((amdgpu_waves_per_eu(3))) void logstate_decode_kernel(LogDecodeParams p) {
  constexpr int TPW = DV >= 128 ? 2 : 1;         // dv row tiles per wave
  constexpr int NT = DV * 4 / TPW, RT = DK / 16;  // threads; dk tiles per wave
  constexpr int KV = DK / 8, VV = DV / 8;        // 16-byte pieces per row
  constexpr int PIECES = (kReplayWindow * (KV + VV) + NT - 1) / NT;
  static_assert(DK % 16 == 0 && DV % 16 == 0, "tile split");
  const uint32_t bid = blockIdx.x, nhv = static_cast<uint32_t>(p.HV);
  const int64_t b = bid / nhv, h = bid % nhv;
  const int64_t group = p.HV / p.H, kh = h / group;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  int j0[TPW];  // this lane's dv rows j0[u] .. j0[u] + 3 of row tile TPW wave + u
#pragma unroll
  for (int u = 0; u < TPW; ++u) j0[u] = 16 * (TPW * wave + u) + 4 * lg;
  __shared__ uint16_t s_kt[DK * kReplayLd];
  __shared__ uint16_t s_vt[DV * kReplayLd];

  const int64_t w = load_index(p.work, b, p.work_is64);
  const int64_t ls = load_index(p.logs, b, p.logs_is64);
  const int64_t pos = load_index(p.offsets, b, p.offsets_is64);
  const bool in_page = ls >= 0 && pos >= 0 && pos < p.page;
  int64_t n = p.eager || !in_page ? 0 : load_index(p.counts, b, p.counts_is64);
  n = n < 0 ? 0 : (n > kReplayWindow ? kReplayWindow : n);
  n = n > pos ? pos : n;  // the logged tokens precede the position within the page
  float* rec = nullptr;  // decay record of the log slot
  if (in_page) {
    const int64_t fr = load_index(p.decay, 2 * ls, p.decay_is64);
    const int64_t ri = load_index(p.decay, 2 * ls + 1, p.decay_is64);
    if (fr >= 0 && fr < p.num_frames && ri >= 0 && (ri + 1) * p.record_bytes <= p.frame_bytes)
      rec = reinterpret_cast<float*>(p.storage + fr * p.frame_bytes + ri * p.record_bytes);
  }
  if (!rec) n = 0;
  // Loads go to a valid address whatever the slot (an unmapped row reads the
  // storage's first bytes and is discarded), so no branch separates them.
  const T* const safe = reinterpret_cast<const T*>(p.storage);

  // ---- every global load
  uint2 raw[TPW][RT];  // S[16 it + lr][j0[u] .. j0[u] + 3]
  bool row_ok[RT];
  // a head inside one frame: one (uniform) frame lookup for all its rows
  const T* head = p.head_bytes <= p.frame_bytes ? state_row<T>(p, w, h, 0, DV) : nullptr;
#pragma unroll
  for (int it = 0; it < RT; ++it) {
    const T* row = p.head_bytes <= p.frame_bytes ? (head ? head + (16 * it + lr) * DV : nullptr)
                                                 : state_row<T>(p, w, h, 16 * it + lr, DV);
    row_ok[it] = row != nullptr;
#pragma unroll
    for (int u = 0; u < TPW; ++u) raw[u][it] = *reinterpret_cast<const uint2*>(row ? row + j0[u] : safe);
  }
  const T* qrow = static_cast<const T*>(p.q) + (b * p.H + kh) * DK;
  const T* krow = static_cast<const T*>(p.k) + (b * p.H + kh) * DK;
  float qv[RT], kv[RT];  // q, k at this lane's dk columns
#pragma unroll
  for (int it = 0; it < RT; ++it) {
    qv[it] = to_f32(qrow[16 * it + lr]);
    kv[it] = to_f32(krow[16 * it + lr]);
  }
  uint2 vraw[TPW];
#pragma unroll
  for (int u = 0; u < TPW; ++u)
    vraw[u] = *reinterpret_cast<const uint2*>(static_cast<const T*>(p.v) + (b * p.HV + h) * DV + j0[u]);
  const float a_log = load_any(p.A_log, h, p.a_dtype);
  const float dt = load_any(p.dt_bias, h, p.dt_dtype);
  const float graw = load_any(p.gate, b * p.gate_b + h * p.gate_h, p.gate_dtype);
  const float braw = load_any(p.beta, b * p.beta_b + h * p.beta_h, p.beta_dtype);
  const int64_t gbase = (p.layer * p.page + pos - n) * p.HV + h;
  const float glane = lane < n ? rec[gbase + (lane < n ? lane : 0) * p.HV] : 0.f;  // replayed gate of token `lane`
  uint4 pw[PIECES];  // replayed rows: piece j of token i (j < KV a key piece, else a value piece)
  bool live[PIECES];
#pragma unroll
  for (int k = 0; k < PIECES; ++k) {
    const int idx = tid + k * NT, i = idx / (KV + VV), j = idx % (KV + VV);
    const bool value = j >= KV;
    const int col = 8 * (value ? j - KV : j);
    const T* e = i < n ? decode_log<T>(p, ls, pos - n + i, value ? h : kh, col, value, DK, DV) : nullptr;
    live[k] = e != nullptr;
    pw[k] = *reinterpret_cast<const uint4*>(e ? e : safe);
  }

  // ---- norms, gates and the replay decays (every wave computes them)
  float qq = 0.f, kk = 0.f, qk = 0.f;
#pragma unroll
  for (int it = 0; it < RT; ++it) {
    qq = fmaf(qv[it], qv[it], qq);
    kk = fmaf(kv[it], kv[it], kk);
    qk = fmaf(qv[it], kv[it], qk);
  }
  qq = row16_sum(qq);
  kk = row16_sum(kk);
  qk = row16_sum(qk);
  const float rq = rsqrtf(qq + 1e-6f) * p.scale, rk = rsqrtf(kk + 1e-6f);
  const float kq = qk * rq * rk;
#pragma unroll
  for (int it = 0; it < RT; ++it) {
    qv[it] *= rq;
    kv[it] *= rk;
  }
  const float g = -expf(a_log) * softplus_decode(graw + dt);
  const float decay = expf(g), beta = sigmoid(braw);
  // inclusive scan of the replayed gates over lanes 0 .. n-1; suffix_i = e^{total - prefix_i}
  float scan = glane;
#pragma unroll
  for (int off = 1; off < kReplayWindow; off <<= 1) {
    const float y = __shfl_up(scan, off, 64);
    if (lane >= off) scan += y;
  }
  const float total = __shfl(scan, kReplayWindow - 1, 64);
  const float suffix = expf(total - scan);  // lanes < n
  const float total_decay = expf(total);

  // ---- the state, decayed over the replayed tokens
  f4_t Tt[TPW][RT];
#pragma unroll
  for (int u = 0; u < TPW; ++u)
#pragma unroll
    for (int it = 0; it < RT; ++it) {
      float a, c2, d, e;
      split2<T>(row_ok[it] ? raw[u][it].x : 0u, a, c2);
      split2<T>(row_ok[it] ? raw[u][it].y : 0u, d, e);
      Tt[u][it] = f4_t{a, c2, d, e} * total_decay;
    }
  if (n > 0) {
    // stage the replayed rows feature-major (token index contiguous): keys,
    // and values scaled by their suffix decay and rounded to the state dtype
#pragma unroll
    for (int k = 0; k < PIECES; ++k) {
      const int idx = tid + k * NT, i = idx / (KV + VV), j = idx % (KV + VV);
      const float sfx = __shfl(suffix, i < kReplayWindow ? i : 0, 64);
      if (i >= kReplayWindow) continue;
      const bool value = j >= KV;
      const int col = 8 * (value ? j - KV : j);
      const bool keep = live[k] && i < n;  // tokens i >= n stage zeros
      const uint32_t wv[4] = {keep ? pw[k].x : 0u, keep ? pw[k].y : 0u, keep ? pw[k].z : 0u, keep ? pw[k].w : 0u};
      uint16_t* dst = (value ? s_vt : s_kt) + col * kReplayLd + i;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t word = wv[q];
        if (value) {
          float a, c2;
          split2<T>(word, a, c2);
          word = out_pack2<T>(a * sfx, c2 * sfx);
        }
        dst[(2 * q) * kReplayLd] = static_cast<uint16_t>(word & 0xffffu);
        dst[(2 * q + 1) * kReplayLd] = static_cast<uint16_t>(word >> 16);
      }
    }
    lds_barrier();
    // T += V'^T K over the replayed tokens (zero rows past n)
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      const uint2 af = *reinterpret_cast<const uint2*>(s_vt + (16 * (TPW * wave + u) + lr) * kReplayLd + 4 * lg);
#pragma unroll
      for (int it = 0; it < RT; ++it) {
        const uint2 bf = *reinterpret_cast<const uint2*>(s_kt + (16 * it + lr) * kReplayLd + 4 * lg);
        Tt[u][it] = mma16<T>(af, bf, Tt[u][it]);
      }
    }
  }

  // ---- one step: row sums of T against k and q (S^T k, S^T q) for rows j0 + e
  float delta[TPW][4], out[TPW][4];
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    float vin[4];
    split2<T>(vraw[u].x, vin[0], vin[1]);
    split2<T>(vraw[u].y, vin[2], vin[3]);
    if (p.eager) {
      // S <- e^g S; delta = (v - S^T k) beta; S <- S + k delta^T; o = S^T q
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float acc = 0.f;
#pragma unroll
        for (int it = 0; it < RT; ++it) {
          Tt[u][it][e] *= decay;
          acc = fmaf(Tt[u][it][e], kv[it], acc);
        }
        delta[u][e] = (vin[e] - row16_sum(acc)) * beta;
        float accq = 0.f;
#pragma unroll
        for (int it = 0; it < RT; ++it) {
          Tt[u][it][e] = fmaf(delta[u][e], kv[it], Tt[u][it][e]);
          accq = fmaf(Tt[u][it][e], qv[it], accq);
        }
        out[u][e] = row16_sum(accq);
      }
    } else {
      // delta = (v - e^g S^T k) beta; o = e^g S^T q + delta (k . q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float ak = 0.f, aq = 0.f;
#pragma unroll
        for (int it = 0; it < RT; ++it) {
          ak = fmaf(Tt[u][it][e], kv[it], ak);
          aq = fmaf(Tt[u][it][e], qv[it], aq);
        }
        delta[u][e] = (vin[e] - row16_sum(ak) * decay) * beta;
        out[u][e] = row16_sum(aq) * decay + delta[u][e] * kq;
      }
    }
  }

  // ---- output and the step's log rows
  if (lr == 0) {
#pragma unroll
    for (int u = 0; u < TPW; ++u)
      *reinterpret_cast<uint2*>(static_cast<T*>(p.out) + (b * p.HV + h) * DV + j0[u]) =
          make_uint2(out_pack2<T>(out[u][0], out[u][1]), out_pack2<T>(out[u][2], out[u][3]));
  }
  if (in_page) {
    if (lr == 0) {
#pragma unroll
      for (int u = 0; u < TPW; ++u) {
        T* e = decode_log<T>(p, ls, pos, h, j0[u], true, DK, DV);
        if (e) *reinterpret_cast<uint2*>(e) =
            make_uint2(out_pack2<T>(delta[u][0], delta[u][1]), out_pack2<T>(delta[u][2], delta[u][3]));
      }
    }
    if (h % group == 0 && tid < KV) {
      const int col = 8 * tid;
      T* e = decode_log<T>(p, ls, pos, kh, col, false, DK, DV);
      if (e) {
        uint32_t pk[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          pk[q] = out_pack2<T>(to_f32(krow[col + 2 * q]) * rk, to_f32(krow[col + 2 * q + 1]) * rk);
        store_words<8>(e, pk);
      }
    }
    if (rec && tid == 0) rec[(p.layer * p.page + pos) * p.HV + h] = g;
  }

  // ---- the work state: every step (eager), else at the end of a replay window
  if (p.eager || (pos + 1) % kReplayWindow == 0) {
#pragma unroll
    for (int it = 0; it < RT; ++it) {
      T* row = p.head_bytes <= p.frame_bytes ? (head ? const_cast<T*>(head) + (16 * it + lr) * DV : nullptr)
                                             : state_row<T>(p, w, h, 16 * it + lr, DV);
      if (!row) continue;
#pragma unroll
      for (int u = 0; u < TPW; ++u) {
        float v4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v4[e] = p.eager ? Tt[u][it][e] : fmaf(delta[u][e], kv[it], Tt[u][it][e] * decay);
        *reinterpret_cast<uint2*>(row + j0[u]) =
            make_uint2(out_pack2<T>(v4[0], v4[1]), out_pack2<T>(v4[2], v4[3]));
      }
    }
  }
}

// ---- restore / copy of LogState slot states (kernel/linear_attention/logstate.py:59-128)
struct RestoreParams {
  char* storage;
  const void* frames; int frames_is64;
  int64_t fps, frame_bytes, head_bytes, num_frames;
  const void* decay; int decay_is64;
  int64_t record_bytes;
  int64_t layers, HV, KH, gran, page;
  const int32_t* base;      // [tasks], -1: zero state
  const int32_t* offsets;   // [tasks + 1] into the segments
  const int32_t* seg_slots; // [segments] log slot
  const int32_t* seg_begin; // [segments] first position
  const int32_t* seg_end;   // [segments] end position
  const int32_t* output;    // [tasks]
  Div32 fdiv, gdiv;         // frame_bytes, gran
};

// State row of (slot, layer, head) in a frame storage (the layout of
// gdn_chunk_gated_delta_rule's frame tables), or null.
template <class T>
__device__ __forceinline__ T* slot_row(const RestoreParams& p, int64_t s, int64_t layer, int64_t h, int64_t row,
                                       int DV) {
  if (s < 0) return nullptr;
  const uint32_t x = static_cast<uint32_t>((layer * p.HV + h) * p.head_bytes + row * DV * static_cast<int64_t>(sizeof(T)));
  const int64_t fr = load_index(p.frames, s * p.fps + p.fdiv.div(x), p.frames_is64);
  if (fr < 0 || fr >= p.num_frames) return nullptr;
  return reinterpret_cast<T*>(p.storage + fr * p.frame_bytes + p.fdiv.mod(x));
}

template <class T>
__device__ __forceinline__ const T* restore_log(const RestoreParams& p, int64_t slot, int64_t layer, int64_t pos,
                                                int64_t index, int64_t col, bool value, int DK, int DV) {
  const int64_t key_size = p.gran * p.KH * DK;
  const int64_t layer_size = key_size + p.gran * p.HV * DV;
  const uint32_t ps = static_cast<uint32_t>(pos);
  const int64_t elem = (p.gdiv.div(ps) * p.layers + layer) * layer_size + (value ? key_size : 0) +
                       (index * p.gran + p.gdiv.mod(ps)) * (value ? DV : DK) + col;
  const uint32_t byte = static_cast<uint32_t>(2 * elem);
  const int64_t fr = load_index(p.frames, slot * p.fps + p.fdiv.div(byte), p.frames_is64);
  if (fr < 0 || fr >= p.num_frames) return nullptr;
  return reinterpret_cast<const T*>(p.storage + fr * p.frame_bytes + p.fdiv.mod(byte));
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16 x 16 x 32 products with fp32 accumulation on 16-bit operands of the state
// dtype.  Operand fragments: lane l holds row (A) or column (B) l % 16 and the
// 8 consecutive k elements 8 (l / 16) .. + 7; the result tile gives lane l
// column l % 16, rows 4 (l / 16) .. + 3.
template <class T> struct RestoreMma;
template <> struct RestoreMma<bf16> {
  static __device__ __forceinline__ f32x4 run(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
};
template <> struct RestoreMma<f16> {
  static __device__ __forceinline__ f32x4 run(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                  c, 0, 0, 0);
  }
};

constexpr int kRestoreGroup = 64;               // tokens staged per step (two 32-deep products)
constexpr int kRestoreLd = kRestoreGroup + 8;   // LDS row of one feature over a group, padded
constexpr int kRestoreSpan = kDecodeThreads;    // tokens whose suffix decays one block scan yields

// grid (tasks x layers x HV), 4 waves: the state of the task's base slot (or
// zero), then each segment of logged tokens t = b .. e-1 in one step,
// S <- e^{sum_t g_t} S + sum_t k_t (e^{sum_{j>t} g_j} v'_t)^T with the scaled
// v' rounded to the state dtype (logstate_construction.cuh:329-393); written
// to the output slot.  The sum runs on MFMA, 64 tokens per step: the step's
// keys and scaled v' rows are staged feature-major in LDS (token index
// contiguous: the k dimension of both operands), and each wave owns the
// state's columns of DV / 64 (at least one) 16-wide tiles over all DK rows in
// fp32 accumulators.  The suffix decays of 256 tokens come from one block
// scan of their gates.
template <int DK, int DV, class T>
__global__ __launch_bounds__(kDecodeThreads) __attribute__((amdgpu_waves_per_eu(2))) void restore_kernel(RestoreParams p) {
  constexpr int RT = DK / 16, CTT = DV / 16, CT = CTT >= 4 ? CTT / 4 : 1;
  constexpr int KV = DK / 8, VV = DV / 8;  // 16-byte pieces per row
  constexpr int PIECES = kRestoreGroup * (KV + VV) / kDecodeThreads;
  static_assert(DK % 16 == 0 && DV % 16 == 0, "tile split");
  static_assert(kRestoreGroup * (KV + VV) % kDecodeThreads == 0, "piece split");
  const uint32_t bid = blockIdx.x, nhv = static_cast<uint32_t>(p.HV), nl = static_cast<uint32_t>(p.layers);
  const int64_t task = bid / (nl * nhv);
  const int64_t layer = (bid / nhv) % nl;
  const int64_t h = bid % nhv;
  const int64_t kh = h / (p.HV / p.KH);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, lq = lane >> 4;
  const bool owner = wave * CT < CTT;  // this wave holds column tiles
  __shared__ uint16_t s_kt[DK * kRestoreLd];
  __shared__ uint16_t s_vt[DV * kRestoreLd];
  __shared__ float s_suffix[kRestoreSpan];
  __shared__ float s_part[kDecodeThreads / 64];
  // acc[i][c] is the transposed tile T = S^T: lane l holds dk column
  // i 16 + l % 16 and dv rows (wave CT + c) 16 + 4 (l / 16) .. + 3, i.e. four
  // consecutive elements of one state row, moved as 8 bytes.
  f32x4 acc[RT][CT];
  const int64_t base = p.base[task];
  // Loads go to a valid address whatever the slot (an unmapped row reads the
  // storage's first elements and is then discarded), so every load is issued
  // before the first wait.
  const T* const safe = reinterpret_cast<const T*>(p.storage);
  // state row r of slot s (a head inside one frame: one uniform lookup)
  auto row_of = [&](int64_t s, const T* head, int r) __attribute__((always_inline)) -> const T* {
    if (p.head_bytes <= p.frame_bytes) return head ? head + r * DV : nullptr;
    return slot_row<T>(p, s, layer, h, r, DV);
  };
  const T* base_head = p.head_bytes <= p.frame_bytes ? slot_row<T>(p, base, layer, h, 0, DV) : nullptr;
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const T* row = owner ? row_of(base, base_head, 16 * i + lr) : nullptr;
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      const int col = (wave * CT + c) * 16 + 4 * lq;
      const uint2 w2 = *reinterpret_cast<const uint2*>(row ? row + col : safe);
      float a, b2, c2, d;
      split2<T>(row ? w2.x : 0u, a, b2);
      split2<T>(row ? w2.y : 0u, c2, d);
      acc[i][c] = f32x4{a, b2, c2, d};
    }
  }
  for (int64_t seg = p.offsets[task]; seg < p.offsets[task + 1]; ++seg) {
    const int64_t ls = p.seg_slots[seg];
    int64_t fr = -1, ri = -1;
    if (ls >= 0) {
      fr = load_index(p.decay, 2 * ls, p.decay_is64);
      ri = load_index(p.decay, 2 * ls + 1, p.decay_is64);
    }
    const bool ok = fr >= 0 && fr < p.num_frames && ri >= 0 && (ri + 1) * p.record_bytes <= p.frame_bytes;
    const int64_t begin = p.seg_begin[seg] < 0 ? 0 : p.seg_begin[seg];
    const int64_t end = p.seg_end[seg] < p.page ? p.seg_end[seg] : p.page;
    if (!ok || begin >= end) continue;
    const float* rec =
        reinterpret_cast<const float*>(p.storage + fr * p.frame_bytes + ri * p.record_bytes) + layer * p.page * p.HV + h;
    // gate sum over the segment
    float part = 0.f;
    for (int64_t t = begin + tid; t < end; t += kDecodeThreads) part += rec[t * p.HV];
    part = wave_sum(part);
    lds_barrier();  // the previous segment's last step is consumed
    if (lane == 0) s_part[wave] = part;
    lds_barrier();
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kDecodeThreads / 64; ++w) total += s_part[w];
    const float decay = expf(total);
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int c = 0; c < CT; ++c) acc[i][c] *= decay;
    float rest = 0.f;  // the gates of the segment's tokens before the span
    for (int64_t sb = begin; sb < end; sb += kRestoreSpan) {
      // suffix decays of the span: one block inclusive scan of its gates
      float x = sb + tid < end ? rec[(sb + tid) * p.HV] : 0.f;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
      }
      lds_barrier();  // s_part and the previous span's suffixes are consumed
      if (lane == 63) s_part[wave] = x;
      lds_barrier();
      float before = rest, span = 0.f;
#pragma unroll
      for (int w = 0; w < kDecodeThreads / 64; ++w) {
        before += w < wave ? s_part[w] : 0.f;
        span += s_part[w];
      }
      s_suffix[tid] = expf(total - (before + x));
      rest += span;
      const int64_t span_end = sb + kRestoreSpan < end ? sb + kRestoreSpan : end;
      for (int64_t g0 = sb; g0 < span_end; g0 += kRestoreGroup) {
        const int n = static_cast<int>(span_end - g0 < kRestoreGroup ? span_end - g0 : kRestoreGroup);
        // the step's pieces: piece j of token t (consecutive threads take consecutive tokens)
        uint4 raw[PIECES];
        bool live[PIECES];
#pragma unroll
        for (int k = 0; k < PIECES; ++k) {
          const int idx = tid + k * kDecodeThreads, t = idx % kRestoreGroup, piece = idx / kRestoreGroup;
          const bool value = piece >= KV;
          const int col = 8 * (value ? piece - KV : piece);
          const T* e = restore_log<T>(p, ls, layer, g0 + (t < n ? t : 0), value ? h : kh, col, value, DK, DV);
          live[k] = t < n && e;
          raw[k] = *reinterpret_cast<const uint4*>(e ? e : safe);
        }
        lds_barrier();  // suffixes written; the previous step's operands are consumed
#pragma unroll
        for (int k = 0; k < PIECES; ++k) {
          const int idx = tid + k * kDecodeThreads, t = idx % kRestoreGroup, piece = idx / kRestoreGroup;
          const bool value = piece >= KV;
          const int col = 8 * (value ? piece - KV : piece);
          const uint32_t wv[4] = {live[k] ? raw[k].x : 0u, live[k] ? raw[k].y : 0u, live[k] ? raw[k].z : 0u,
                                  live[k] ? raw[k].w : 0u};
          uint16_t* dst = (value ? s_vt : s_kt) + col * kRestoreLd + t;
          if (value) {
            const float sfx = s_suffix[g0 - sb + t];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              float a, b;
              split2<T>(wv[q], a, b);
              const uint32_t packed = out_pack2<T>(a * sfx, b * sfx);
              dst[(2 * q) * kRestoreLd] = static_cast<uint16_t>(packed & 0xffffu);
              dst[(2 * q + 1) * kRestoreLd] = static_cast<uint16_t>(packed >> 16);
            }
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              dst[(2 * q) * kRestoreLd] = static_cast<uint16_t>(wv[q] & 0xffffu);
              dst[(2 * q + 1) * kRestoreLd] = static_cast<uint16_t>(wv[q] >> 16);
            }
          }
        }
        lds_barrier();
        if (owner) {
#pragma unroll
          for (int ks = 0; ks < kRestoreGroup / 32; ++ks)
#pragma unroll
            for (int c = 0; c < CT; ++c) {
              const uint4 bfrag = *reinterpret_cast<const uint4*>(
                  s_vt + ((wave * CT + c) * 16 + lr) * kRestoreLd + 32 * ks + 8 * lq);
#pragma unroll
              for (int i = 0; i < RT; ++i) {
                const uint4 kfrag =
                    *reinterpret_cast<const uint4*>(s_kt + (i * 16 + lr) * kRestoreLd + 32 * ks + 8 * lq);
                acc[i][c] = RestoreMma<T>::run(bfrag, kfrag, acc[i][c]);  // T += V'^T K
              }
            }
        }
      }
    }
  }
  const int64_t out = p.output[task];
  if (!owner) return;
  const T* out_head = p.head_bytes <= p.frame_bytes ? slot_row<T>(p, out, layer, h, 0, DV) : nullptr;
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    T* row = const_cast<T*>(row_of(out, out_head, 16 * i + lr));
    if (!row) continue;
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      const int col = (wave * CT + c) * 16 + 4 * lq;
      *reinterpret_cast<uint2*>(row + col) =
          make_uint2(out_pack2<T>(acc[i][c][0], acc[i][c][1]), out_pack2<T>(acc[i][c][2], acc[i][c][3]));
    }
  }
}

// grid (pairs x layers x HV): the state of (source, layer, head) to destination.
template <int DK, int DV, class T>
__global__ __launch_bounds__(kDecodeThreads) void copy_states_kernel(RestoreParams p) {
  const int64_t pair = blockIdx.x / (p.layers * p.HV);
  const int64_t layer = (blockIdx.x / p.HV) % p.layers;
  const int64_t h = blockIdx.x % p.HV;
  const int64_t src = p.base[pair], dst = p.output[pair];
  for (int idx = threadIdx.x; idx < DK * (DV / 4); idx += kDecodeThreads) {
    const int row = idx / (DV / 4), c0 = 4 * (idx % (DV / 4));
    const T* a = slot_row<T>(p, src, layer, h, row, DV);
    T* b = slot_row<T>(p, dst, layer, h, row, DV);
    if (!a || !b) continue;
#pragma unroll
    for (int c = 0; c < 4; ++c) b[c0 + c] = a[c0 + c];
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
  GDN_REQUIRE(frames_per_slot * frame_bytes < kMaxOffset32, "gdn_store_chunk_log: a slot's frames exceed 4 GiB");
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
  p.fdiv = make_div32(frame_bytes); p.gdiv = make_div32(granularity);
  const bool vec = dk % 8 == 0 && dv % 8 == 0 && frame_bytes % 16 == 0 && aligned16(storage) && aligned16(v_new) &&
                   aligned16(key);
  if (vec)
    hipLaunchKernelGGL(chunk_log_vec_kernel, dim3(static_cast<unsigned>(T)), dim3(kLogThreads), 0,
                       static_cast<hipStream_t>(stream), p);
  else
    hipLaunchKernelGGL(chunk_log_kernel, dim3(static_cast<unsigned>(T), static_cast<unsigned>(HV)), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), p);
  return GDN_LAUNCH_CHECK("gdn_store_chunk_log launch");
}

extern "C" int gdn_conv_decode_logstate(const void* x, int64_t x_row_stride, int64_t x_col_stride, int dtype,
                                        const void* weight, const void* bias, int kernel_width, int64_t batch,
                                        int64_t channels, void* storage, const void* conv_frames, int frames_dtype,
                                        int64_t num_granules, int64_t frames_per_granule, int64_t frame_bytes,
                                        int64_t num_frames, int64_t layer, const void* read_slots, int read_dtype,
                                        const void* read_granules, int read_granules_dtype,
                                        const void* write_slots, int write_dtype, const void* write_granules,
                                        int write_granules_dtype, const void* work_slots, int work_dtype,
                                        void* q_out, void* k_out, void* v_out, int64_t key_dim, int split_qkv,
                                        int round_conv, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(batch >= 0 && channels > 0 && layer >= 0, "gdn_conv_decode_logstate: bad sizes");
  if (batch == 0) return GDN_OK;
  GDN_REQUIRE(kernel_width >= 2 && kernel_width <= 8, "gdn_conv_decode_logstate: kernel width %d not in [2, 8]",
              kernel_width);
  GDN_REQUIRE(x && weight && storage && conv_frames && read_slots && read_granules && write_slots && write_granules &&
                  work_slots && q_out,
              "gdn_conv_decode_logstate: null input");
  GDN_REQUIRE(!split_qkv || (k_out && v_out && 2 * key_dim < channels), "gdn_conv_decode_logstate: bad split");
  GDN_REQUIRE(num_granules > 0 && frames_per_granule > 0 && num_frames > 0 && frame_bytes > 0,
              "gdn_conv_decode_logstate: bad conv frame table");
  const int64_t elt = dtype == GDN_F32 ? 4 : 2;
  GDN_REQUIRE(frame_bytes % elt == 0, "gdn_conv_decode_logstate: frame_bytes %lld not a multiple of the element",
              (long long)frame_bytes);
  const int64_t fe = frame_bytes / elt;
  const int64_t span = (layer + 1) * channels * (kernel_width - 1);
  GDN_REQUIRE(frames_per_granule == 1 ? span <= fe : span <= frames_per_granule * fe,
              "gdn_conv_decode_logstate: layer %lld's conv windows exceed the snapshot's frames", (long long)layer);
  GDN_REQUIRE(span < kMaxOffset32 && fe < kMaxOffset32, "gdn_conv_decode_logstate: snapshot offsets exceed 32 bits");
  GDN_REQUIRE(batch <= 65535, "gdn_conv_decode_logstate: batch too large");
  ConvFrameParams p{};
  p.x = x; p.xr = x_row_stride; p.xc = x_col_stride; p.weight = weight; p.bias = bias; p.W = kernel_width;
  p.C = channels; p.storage = storage; p.table = conv_frames; p.table_is64 = frames_dtype == GDN_I64;
  p.granules = num_granules; p.cf = frames_per_granule; p.fe = fe; p.num_frames = num_frames; p.layer = layer;
  p.reads = read_slots; p.reads_is64 = read_dtype == GDN_I64;
  p.rgran = read_granules; p.rgran_is64 = read_granules_dtype == GDN_I64;
  p.writes = write_slots; p.writes_is64 = write_dtype == GDN_I64;
  p.wgran = write_granules; p.wgran_is64 = write_granules_dtype == GDN_I64;
  p.works = work_slots; p.works_is64 = work_dtype == GDN_I64;
  p.q = q_out; p.k = k_out; p.v = v_out; p.key_dim = key_dim; p.split = split_qkv; p.round_conv = round_conv;
  dim3 grid(static_cast<unsigned>((channels + kDecodeThreads - 1) / kDecodeThreads), static_cast<unsigned>(batch));
  auto s = static_cast<hipStream_t>(stream);
  if (dtype == GDN_BF16) {
    hipLaunchKernelGGL(conv_decode_frames_kernel<bf16>, grid, dim3(kDecodeThreads), 0, s, p);
  } else if (dtype == GDN_F16) {
    hipLaunchKernelGGL(conv_decode_frames_kernel<f16>, grid, dim3(kDecodeThreads), 0, s, p);
  } else {
    set_error("gdn_conv_decode_logstate: unsupported dtype %d (bf16 or f16)", dtype);
    return GDN_ERR_UNSUPPORTED;
  }
  return GDN_LAUNCH_CHECK("gdn_conv_decode_logstate launch");
}

extern "C" int gdn_recurrent_logstate(
    const void* q, const void* k, const void* v, int io_dtype, const void* gate, int64_t gate_b_stride,
    int64_t gate_h_stride, int gate_dtype, const void* beta, int64_t beta_b_stride, int64_t beta_h_stride,
    int beta_dtype, const void* A_log, int a_dtype, const void* dt_bias, int dt_dtype, int64_t batch, int64_t H,
    int64_t HV, int64_t dk, int64_t dv, void* storage, const void* payload_frames, int frames_dtype,
    int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes, int64_t num_frames, const void* decay_frames,
    int decay_dtype, int64_t decay_record_bytes, const void* work_slots, int work_dtype, const void* log_slots,
    int log_dtype, const void* token_offsets, int offsets_dtype, const void* replay_counts, int counts_dtype,
    int64_t layer, int64_t num_layers, int64_t granularity, int64_t page_size, int eager, void* out, float scale,
    void* stream) {
  using namespace gdn;
  GDN_REQUIRE(batch >= 0 && H > 0 && HV > 0 && HV % H == 0, "gdn_recurrent_logstate: bad sizes");
  if (batch == 0) return GDN_OK;
  GDN_REQUIRE(q && k && v && gate && beta && A_log && dt_bias && storage && payload_frames && decay_frames &&
                  work_slots && log_slots && token_offsets && replay_counts && out,
              "gdn_recurrent_logstate: null input");
  GDN_REQUIRE(io_dtype == GDN_BF16 || io_dtype == GDN_F16, "gdn_recurrent_logstate: io dtype must be bf16 or f16");
  GDN_REQUIRE(num_layers > 0 && layer >= 0 && layer < num_layers && granularity > 0 && page_size > 0 &&
                  page_size % granularity == 0,
              "gdn_recurrent_logstate: bad layout");
  const int64_t row = dv * 2;
  GDN_REQUIRE(frames_per_slot > 0 && frame_bytes > 0 && num_frames > 0 && frame_bytes % 16 == 0 &&
                  head_bytes >= dk * row && head_bytes % 16 == 0 && aligned16(storage),
              "gdn_recurrent_logstate: bad frame layout (frame and head bytes must be multiples of 16, the "
              "storage 16-byte aligned)");
  GDN_REQUIRE(head_bytes <= frame_bytes ? frame_bytes % head_bytes == 0
                                        : head_bytes % frame_bytes == 0 && frame_bytes % row == 0,
              "gdn_recurrent_logstate: head_bytes %lld must divide frame_bytes %lld, or be a multiple of it with "
              "frames holding whole state rows",
              (long long)head_bytes, (long long)frame_bytes);
  GDN_REQUIRE(frames_per_slot * frame_bytes < kMaxOffset32, "gdn_recurrent_logstate: a slot's frames exceed 4 GiB");
  GDN_REQUIRE((layer + 1) * HV * head_bytes <= frames_per_slot * frame_bytes &&
                  2 * page_size * num_layers * (H * dk + HV * dv) <= frames_per_slot * frame_bytes,
              "gdn_recurrent_logstate: the states or the log exceed a slot's frames");
  GDN_REQUIRE(decay_record_bytes % 4 == 0 && decay_record_bytes >= 4 * num_layers * page_size * HV &&
                  decay_record_bytes <= frame_bytes,
              "gdn_recurrent_logstate: bad decay record size");
  GDN_REQUIRE(batch * HV <= 0x7fffffff, "gdn_recurrent_logstate: grid too large");
  LogDecodeParams p{};
  p.q = q; p.k = k; p.v = v;
  p.gate = gate; p.gate_b = gate_b_stride; p.gate_h = gate_h_stride; p.gate_dtype = gate_dtype;
  p.beta = beta; p.beta_b = beta_b_stride; p.beta_h = beta_h_stride; p.beta_dtype = beta_dtype;
  p.A_log = A_log; p.a_dtype = a_dtype; p.dt_bias = dt_bias; p.dt_dtype = dt_dtype;
  p.H = H; p.HV = HV;
  p.storage = static_cast<char*>(storage);
  p.frames = payload_frames; p.frames_is64 = frames_dtype == GDN_I64;
  p.fps = frames_per_slot; p.frame_bytes = frame_bytes; p.head_bytes = head_bytes; p.num_frames = num_frames;
  p.decay = decay_frames; p.decay_is64 = decay_dtype == GDN_I64; p.record_bytes = decay_record_bytes;
  p.work = work_slots; p.work_is64 = work_dtype == GDN_I64;
  p.logs = log_slots; p.logs_is64 = log_dtype == GDN_I64;
  p.offsets = token_offsets; p.offsets_is64 = offsets_dtype == GDN_I64;
  p.counts = replay_counts; p.counts_is64 = counts_dtype == GDN_I64;
  p.layer = layer; p.layers = num_layers; p.gran = granularity; p.page = page_size;
  p.fdiv = make_div32(frame_bytes); p.gdiv = make_div32(granularity);
  p.eager = eager; p.out = out; p.scale = scale;
  const dim3 grid(static_cast<unsigned>(batch * HV));
  auto s = static_cast<hipStream_t>(stream);
  auto launch = [&](auto dkc, auto dvc) {
    constexpr int DK = decltype(dkc)::value, DV = decltype(dvc)::value;
    if (io_dtype == GDN_BF16)
      hipLaunchKernelGGL((logstate_decode_kernel<DK, DV, bf16>), grid, dim3(DV * 4 / (DV >= 128 ? 2 : 1)), 0, s, p);
    else
      hipLaunchKernelGGL((logstate_decode_kernel<DK, DV, f16>), grid, dim3(DV * 4 / (DV >= 128 ? 2 : 1)), 0, s, p);
    return GDN_LAUNCH_CHECK("gdn_recurrent_logstate launch");
  };
  using I128 = std::integral_constant<int, 128>;
  using I64 = std::integral_constant<int, 64>;
  using I32 = std::integral_constant<int, 32>;
  if (dk == 128 && dv == 128) return launch(I128{}, I128{});
  if (dk == 64 && dv == 64) return launch(I64{}, I64{});
  if (dk == 32 && dv == 32) return launch(I32{}, I32{});
  if (dk == 128 && dv == 64) return launch(I128{}, I64{});
  if (dk == 64 && dv == 128) return launch(I64{}, I128{});
  set_error("gdn_recurrent_logstate: unsupported head dims dk=%lld dv=%lld", (long long)dk, (long long)dv);
  return GDN_ERR_UNSUPPORTED;
}

extern "C" int gdn_conv_windows_logstate(const void* x, int64_t x_row_stride, int64_t x_col_stride, int dtype,
                                         const void* history, const void* cu_seqlens, int cu_dtype, int64_t num_seqs,
                                         int64_t total_tokens, int64_t channels, int kernel_width, void* storage,
                                         const void* conv_frames, int frames_dtype, int64_t num_granules,
                                         int64_t frames_per_granule, int64_t frame_bytes, int64_t num_frames,
                                         int64_t layer, const void* token_slots, int slots_dtype,
                                         const void* token_granules, int granules_dtype, const void* final_slots,
                                         int finals_dtype, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(num_seqs >= 1 && total_tokens >= 0 && channels > 0 && layer >= 0,
              "gdn_conv_windows_logstate: bad sizes");
  if (total_tokens == 0) return GDN_OK;
  GDN_REQUIRE(kernel_width >= 2 && kernel_width <= 8, "gdn_conv_windows_logstate: kernel width %d not in [2, 8]",
              kernel_width);
  GDN_REQUIRE(x && history && cu_seqlens && storage && conv_frames && token_slots && token_granules,
              "gdn_conv_windows_logstate: null input");
  GDN_REQUIRE(num_granules > 0 && frames_per_granule > 0 && num_frames > 0 && frame_bytes > 0 && frame_bytes % 2 == 0,
              "gdn_conv_windows_logstate: bad conv frame table");
  const int64_t fe = frame_bytes / 2;
  const int64_t span = (layer + 1) * channels * (kernel_width - 1);
  GDN_REQUIRE(frames_per_granule == 1 ? span <= fe : span <= frames_per_granule * fe,
              "gdn_conv_windows_logstate: layer %lld's conv windows exceed the snapshot's frames", (long long)layer);
  GDN_REQUIRE(span < kMaxOffset32 && fe < kMaxOffset32, "gdn_conv_windows_logstate: snapshot offsets exceed 32 bits");
  GDN_REQUIRE(total_tokens <= 0x7fffffff && (channels + kDecodeThreads - 1) / kDecodeThreads <= 65535,
              "gdn_conv_windows_logstate: grid too large");
  ConvWindowParams p{};
  p.x = x; p.xr = x_row_stride; p.xc = x_col_stride; p.history = history;
  p.cu = cu_seqlens; p.cu_is64 = cu_dtype == GDN_I64;
  p.N = num_seqs; p.T = total_tokens; p.C = channels; p.S = kernel_width - 1;
  p.storage = storage; p.table = conv_frames; p.table_is64 = frames_dtype == GDN_I64;
  p.granules = num_granules; p.cf = frames_per_granule; p.fe = fe; p.num_frames = num_frames; p.layer = layer;
  p.slots = token_slots; p.slots_is64 = slots_dtype == GDN_I64;
  p.gran = token_granules; p.gran_is64 = granules_dtype == GDN_I64;
  p.finals = final_slots; p.finals_is64 = finals_dtype == GDN_I64;
  const dim3 grid(static_cast<unsigned>(total_tokens), static_cast<unsigned>((channels + kDecodeThreads - 1) /
                                                                            kDecodeThreads));
  auto s = static_cast<hipStream_t>(stream);
  if (dtype == GDN_BF16) {
    hipLaunchKernelGGL(conv_windows_frames_kernel<bf16>, grid, dim3(kDecodeThreads), 0, s, p);
  } else if (dtype == GDN_F16) {
    hipLaunchKernelGGL(conv_windows_frames_kernel<f16>, grid, dim3(kDecodeThreads), 0, s, p);
  } else {
    set_error("gdn_conv_windows_logstate: unsupported dtype %d (bf16 or f16)", dtype);
    return GDN_ERR_UNSUPPORTED;
  }
  return GDN_LAUNCH_CHECK("gdn_conv_windows_logstate launch");
}

namespace gdn {
namespace {

int restore_setup(RestoreParams& p, void* storage, const void* payload_frames, int frames_dtype,
                  int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes, int64_t num_frames,
                  const void* decay_frames, int decay_dtype, int64_t record_bytes, int64_t layers, int64_t HV,
                  int64_t KH, int64_t dk, int64_t dv, int64_t granularity, int64_t page_size, const char* who) {
  GDN_REQUIRE(layers > 0 && HV > 0 && KH > 0 && HV % KH == 0 && granularity > 0 && page_size > 0 &&
                  page_size % granularity == 0,
              "%s: bad layout", who);
  const int64_t row = dv * 2;
  GDN_REQUIRE(frames_per_slot > 0 && frame_bytes > 0 && num_frames > 0 && frame_bytes % 16 == 0 &&
                  head_bytes >= dk * row && head_bytes % 16 == 0 && aligned16(storage),
              "%s: bad frame layout (frame and head bytes must be multiples of 16, the storage 16-byte aligned)",
              who);
  GDN_REQUIRE(head_bytes <= frame_bytes ? frame_bytes % head_bytes == 0
                                        : head_bytes % frame_bytes == 0 && frame_bytes % row == 0,
              "%s: head_bytes %lld must divide frame_bytes %lld, or be a multiple of it with frames holding whole "
              "state rows",
              who, (long long)head_bytes, (long long)frame_bytes);
  GDN_REQUIRE(frames_per_slot * frame_bytes < kMaxOffset32, "%s: a slot's frames exceed 4 GiB", who);
  GDN_REQUIRE(layers * HV * head_bytes <= frames_per_slot * frame_bytes &&
                  2 * page_size * layers * (KH * dk + HV * dv) <= frames_per_slot * frame_bytes,
              "%s: the states or the log exceed a slot's frames", who);
  GDN_REQUIRE(record_bytes % 4 == 0 && record_bytes >= 4 * layers * page_size * HV && record_bytes <= frame_bytes,
              "%s: bad decay record size", who);
  p.storage = static_cast<char*>(storage);
  p.frames = payload_frames; p.frames_is64 = frames_dtype == GDN_I64;
  p.fps = frames_per_slot; p.frame_bytes = frame_bytes; p.head_bytes = head_bytes; p.num_frames = num_frames;
  p.decay = decay_frames; p.decay_is64 = decay_dtype == GDN_I64; p.record_bytes = record_bytes;
  p.layers = layers; p.HV = HV; p.KH = KH; p.gran = granularity; p.page = page_size;
  p.fdiv = make_div32(frame_bytes); p.gdiv = make_div32(granularity);
  return GDN_OK;
}

// RESTORE: restore_kernel, else copy_states_kernel.
template <bool RESTORE>
int launch_state_kernel(const RestoreParams& p, int64_t blocks, int64_t dk, int64_t dv, int dtype, hipStream_t s,
                        const char* who) {
  if (blocks > 0x7fffffff) {
    set_error("%s: grid too large", who);
    return GDN_ERR_INVALID;
  }
  auto launch = [&](auto dkc, auto dvc) {
    constexpr int DK = decltype(dkc)::value, DV = decltype(dvc)::value;
    const dim3 grid(static_cast<unsigned>(blocks));
    if constexpr (RESTORE) {
      if (dtype == GDN_BF16)
        hipLaunchKernelGGL((restore_kernel<DK, DV, bf16>), grid, dim3(kDecodeThreads), 0, s, p);
      else
        hipLaunchKernelGGL((restore_kernel<DK, DV, f16>), grid, dim3(kDecodeThreads), 0, s, p);
    } else {
      if (dtype == GDN_BF16)
        hipLaunchKernelGGL((copy_states_kernel<DK, DV, bf16>), grid, dim3(kDecodeThreads), 0, s, p);
      else
        hipLaunchKernelGGL((copy_states_kernel<DK, DV, f16>), grid, dim3(kDecodeThreads), 0, s, p);
    }
    return GDN_LAUNCH_CHECK(who);
  };
  if (dtype != GDN_BF16 && dtype != GDN_F16) {
    set_error("%s: state dtype must be bf16 or f16", who);
    return GDN_ERR_UNSUPPORTED;
  }
  using I128 = std::integral_constant<int, 128>;
  using I64 = std::integral_constant<int, 64>;
  using I32 = std::integral_constant<int, 32>;
  if (dk == 128 && dv == 128) return launch(I128{}, I128{});
  if (dk == 64 && dv == 64) return launch(I64{}, I64{});
  if (dk == 32 && dv == 32) return launch(I32{}, I32{});
  if (dk == 128 && dv == 64) return launch(I128{}, I64{});
  if (dk == 64 && dv == 128) return launch(I64{}, I128{});
  set_error("%s: unsupported head dims dk=%lld dv=%lld", who, (long long)dk, (long long)dv);
  return GDN_ERR_UNSUPPORTED;
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_logstate_restore(void* storage, const void* payload_frames, int frames_dtype,
                                    int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes,
                                    int64_t num_frames, const void* decay_frames, int decay_dtype,
                                    int64_t decay_record_bytes, int64_t num_layers, int64_t HV, int64_t key_heads,
                                    int64_t dk, int64_t dv, int64_t granularity, int64_t page_size, int dtype,
                                    const int32_t* base_slots, const int32_t* segment_offsets,
                                    const int32_t* log_slots, const int32_t* log_begins, const int32_t* log_ends,
                                    const int32_t* output_slots, int64_t num_tasks, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(num_tasks >= 0, "gdn_logstate_restore: bad sizes");
  if (num_tasks == 0) return GDN_OK;
  GDN_REQUIRE(storage && payload_frames && decay_frames && base_slots && segment_offsets && log_slots &&
                  log_begins && log_ends && output_slots,
              "gdn_logstate_restore: null input");
  RestoreParams p{};
  int rc = restore_setup(p, storage, payload_frames, frames_dtype, frames_per_slot, frame_bytes, head_bytes,
                         num_frames, decay_frames, decay_dtype, decay_record_bytes, num_layers, HV, key_heads, dk, dv,
                         granularity, page_size, "gdn_logstate_restore");
  if (rc != GDN_OK) return rc;
  p.base = base_slots; p.offsets = segment_offsets; p.seg_slots = log_slots; p.seg_begin = log_begins;
  p.seg_end = log_ends; p.output = output_slots;
  return launch_state_kernel<true>(p, num_tasks * num_layers * HV, dk, dv, dtype,
                                             static_cast<hipStream_t>(stream), "gdn_logstate_restore");
}

extern "C" int gdn_logstate_copy_states(void* storage, const void* payload_frames, int frames_dtype,
                                        int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes,
                                        int64_t num_frames, int64_t num_layers, int64_t HV, int64_t dk, int64_t dv,
                                        int dtype, const int32_t* sources, const int32_t* destinations,
                                        int64_t count, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(count >= 0, "gdn_logstate_copy_states: bad sizes");
  if (count == 0) return GDN_OK;
  GDN_REQUIRE(storage && payload_frames && sources && destinations, "gdn_logstate_copy_states: null input");
  GDN_REQUIRE(num_layers > 0 && HV > 0 && frames_per_slot > 0 && frame_bytes > 0 && num_frames > 0 &&
                  head_bytes >= dk * dv * 2 &&
                  (head_bytes <= frame_bytes ? frame_bytes % head_bytes == 0
                                             : head_bytes % frame_bytes == 0 && frame_bytes % (dv * 2) == 0) &&
                  num_layers * HV * head_bytes <= frames_per_slot * frame_bytes &&
                  frames_per_slot * frame_bytes < kMaxOffset32,
              "gdn_logstate_copy_states: bad frame layout");
  RestoreParams p{};
  p.storage = static_cast<char*>(storage);
  p.frames = payload_frames; p.frames_is64 = frames_dtype == GDN_I64;
  p.fps = frames_per_slot; p.frame_bytes = frame_bytes; p.head_bytes = head_bytes; p.num_frames = num_frames;
  p.layers = num_layers; p.HV = HV; p.KH = 1;
  p.fdiv = make_div32(frame_bytes); p.gdiv = make_div32(1);
  p.base = sources; p.output = destinations;
  return launch_state_kernel<false>(p, count * num_layers * HV, dk, dv, dtype,
                                                 static_cast<hipStream_t>(stream), "gdn_logstate_copy_states");
}
