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
  int64_t rows;  // slots in the payload and decay frame tables
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
  if (slot < 0 || slot >= p.rows || pos < 0 || pos >= p.page) return;
  if (p.v_new) {  // null: the value rows were written by the chunk kernel
    const uint16_t* vrow = p.v_new + (t * p.HV + h) * p.V;
    for (int64_t col = threadIdx.x; col < p.V; col += kThreads) {
      uint16_t* d = log_element(p, slot, pos, h, col, true);
      if (d) *d = vrow[col];
    }
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
// Index arithmetic is 32-bit (a row has at most 64 pieces; 64-bit divisions
// per piece had cost a fifth of the kernel).  Needs dk, dv multiples of 8,
// frames a multiple of 16 bytes and 16-byte aligned sources (checked by the
// host); a piece never straddles two frames.
constexpr int kLogThreads = 256;
__global__ __launch_bounds__(kLogThreads) void chunk_log_vec_kernel(LogParams p) {
  const int64_t t = blockIdx.x;
  const int64_t slot = load_index(p.slots, t, p.slots_is64);
  const int64_t pos = load_index(p.offsets, t, p.offsets_is64);
  if (slot < 0 || slot >= p.rows || pos < 0 || pos >= p.page) return;
  const int vv = static_cast<int>(p.V / 8), kv = static_cast<int>(p.K / 8);
  const int group = static_cast<int>(p.HV / p.KH);   // value heads per logged key head
  const int kstride = static_cast<int>(p.HV / p.H);  // value heads per key head of the input
  const int nval = p.v_new ? static_cast<int>(p.HV) * vv : 0;  // no value rows: written by the chunk kernel
  const int total = nval + static_cast<int>(p.KH) * kv;
  for (int i = threadIdx.x; i < total; i += kLogThreads) {
    const bool value = i < nval;
    const int j = value ? i : i - nval;
    const int per = value ? vv : kv;
    const int row = j / per, col = 8 * (j - row * per);
    const uint16_t* src = value ? p.v_new + (t * p.HV + row) * p.V + col
                                : p.key + (t * p.H + row * group / kstride) * p.K + col;
    uint16_t* d = log_element(p, slot, pos, row, col, value);
    if (d) *reinterpret_cast<uint4*>(d) = *reinterpret_cast<const uint4*>(src);
  }
  const int64_t fr = load_index(p.decay, 2 * slot, p.decay_is64);
  const int64_t rec = load_index(p.decay, 2 * slot + 1, p.decay_is64);
  if (fr >= 0 && fr < p.num_frames && rec >= 0 && (rec + 1) * p.record_bytes <= p.frame_bytes) {
    float* d = reinterpret_cast<float*>(p.storage + fr * p.frame_bytes + rec * p.record_bytes);
    for (int h = threadIdx.x; h < p.HV; h += kLogThreads) d[(p.layer * p.page + pos) * p.HV + h] = p.gate[t * p.HV + h];
  }
}

// ---------------------------------------------------------------- LogState decode

constexpr int kReplayWindow = 16;  // cache/logstate/layout.py:8
constexpr int kDecodeThreads = 256;

// Element e of the conv snapshot of (slot, granule), or null when unmapped
// (layout.py:104-112).
template <class T>
__device__ __forceinline__ T* conv_element(T* storage, const void* table, int is64, int64_t rows, int64_t slot,
                                           int64_t granule, int64_t e, int64_t granules, int64_t cf, int64_t fe,
                                           int64_t num_frames) {
  if (slot < 0 || slot >= rows) return nullptr;
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
  int64_t rows;  // slots of the conv frame table
  int64_t granules, cf, fe, num_frames, layer;
  const void* reads; int reads_is64;
  const void* rgran; int rgran_is64;
  const void* writes; int writes_is64;
  const void* wgran; int wgran_is64;
  const void* works; int works_is64;
  void* q; void* k; void* v;
  int64_t key_dim;
  int split, round_conv;
  int64_t end0, end1;  // input scales: s0 below channel end0, s1 below end1, s2 after
  float s0, s1, s2;
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
    const T* src =
        conv_element(st, p.table, p.table_is64, p.rows, rs, rg, e0 + i, p.granules, p.cf, p.fe, p.num_frames);
    win[i] = src ? to_f32(*src) : 0.f;
  }
  const T* x = static_cast<const T*>(p.x);
  const T* w = static_cast<const T*>(p.weight);
  const float sc = ch < p.end0 ? p.s0 : (ch < p.end1 ? p.s1 : p.s2);
  const float x0 = to_f32(x[b * p.xr + ch * p.xc]);
  // a scaled input is rounded to the io type, and the window keeps it scaled
  const float xv = sc != 1.f ? round_to<T>(x0 * sc) : x0;
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
    T* d0 = conv_element(st, p.table, p.table_is64, p.rows, ws, wg, e0 + i, p.granules, p.cf, p.fe, p.num_frames);
    T* d1 = conv_element(st, p.table, p.table_is64, p.rows, wk, 0, e0 + i, p.granules, p.cf, p.fe, p.num_frames);
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

// The same for 8 consecutive channels per thread with 16-byte accesses
// (the scalar form moves 2-byte elements and looks its frames up per
// element): width 4, one frame per snapshot granule, unit input column
// stride and 16-byte aligned rows (checked by the host).  The 8 channels'
// windows ([channel][tap], 24 elements) are 48 contiguous bytes of one frame.
// Same arithmetic, order and rounding per channel as the scalar form.
template <class T>
__device__ __forceinline__ uint32_t bits16(T v) {
  if constexpr (std::is_same<T, bf16>::value) return v.bits;
  else return __builtin_bit_cast(uint16_t, v);
}
template <class T>
__global__ __launch_bounds__(kDecodeThreads) void conv_decode_frames_vec_kernel(ConvFrameParams p) {
  const int64_t b = blockIdx.y;
  const int64_t ch0 = (static_cast<int64_t>(blockIdx.x) * kDecodeThreads + threadIdx.x) * 8;
  if (ch0 >= p.C) return;
  T* st = static_cast<T*>(p.storage);
  const int64_t e0 = p.layer * p.C * 3 + ch0 * 3;
  const int64_t rs = load_index(p.reads, b, p.reads_is64), rg = load_index(p.rgran, b, p.rgran_is64);
  const T* src = conv_element(st, p.table, p.table_is64, p.rows, rs, rg, e0, p.granules, 1, p.fe, p.num_frames);
  float flat[24];  // window of channel c at flat[3 c ..]
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    float f[8];
    unpack8<T>(src ? reinterpret_cast<const uint4*>(src)[j] : make_uint4(0, 0, 0, 0), f);
#pragma unroll
    for (int e = 0; e < 8; ++e) flat[8 * j + e] = f[e];
  }
  float xv[8], wf[32], bias[8];
  unpack8<T>(*reinterpret_cast<const uint4*>(static_cast<const T*>(p.x) + b * p.xr + ch0), xv);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float f[8];
    unpack8<T>(reinterpret_cast<const uint4*>(static_cast<const T*>(p.weight) + ch0 * 4)[j], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) wf[8 * j + e] = f[e];
  }
  if (p.bias) {
    unpack8<T>(*reinterpret_cast<const uint4*>(static_cast<const T*>(p.bias) + ch0), bias);
  }
  uint32_t yb[8], nb[24];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int64_t ch = ch0 + c;
    const float sc = ch < p.end0 ? p.s0 : (ch < p.end1 ? p.s1 : p.s2);
    // a scaled input is rounded to the io type, and the window keeps it scaled
    const float x = sc != 1.f ? round_to<T>(xv[c] * sc) : xv[c];
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 3; ++i) acc = fmaf(wf[4 * c + i], flat[3 * c + i], acc);
    acc = fmaf(wf[4 * c + 3], x, acc);
    if (p.bias) acc += bias[c];
    if (p.round_conv) acc = round_to<T>(acc);
    yb[c] = bits16<T>(from_f32<T>(silu(acc)));
    nb[3 * c] = bits16<T>(from_f32<T>(flat[3 * c + 1]));
    nb[3 * c + 1] = bits16<T>(from_f32<T>(flat[3 * c + 2]));
    nb[3 * c + 2] = bits16<T>(from_f32<T>(x));
  }
  uint4 nw[3];
#pragma unroll
  for (int j = 0; j < 3; ++j)
    nw[j] = make_uint4(nb[8 * j] | nb[8 * j + 1] << 16, nb[8 * j + 2] | nb[8 * j + 3] << 16,
                       nb[8 * j + 4] | nb[8 * j + 5] << 16, nb[8 * j + 6] | nb[8 * j + 7] << 16);
  const int64_t ws = load_index(p.writes, b, p.writes_is64), wg = load_index(p.wgran, b, p.wgran_is64);
  const int64_t wk = load_index(p.works, b, p.works_is64);
  T* d0 = conv_element(st, p.table, p.table_is64, p.rows, ws, wg, e0, p.granules, 1, p.fe, p.num_frames);
  T* d1 = conv_element(st, p.table, p.table_is64, p.rows, wk, 0, e0, p.granules, 1, p.fe, p.num_frames);
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    if (d0) reinterpret_cast<uint4*>(d0)[j] = nw[j];
    if (d1) reinterpret_cast<uint4*>(d1)[j] = nw[j];
  }
  const uint4 y = make_uint4(yb[0] | yb[1] << 16, yb[2] | yb[3] << 16, yb[4] | yb[5] << 16, yb[6] | yb[7] << 16);
  T* dst;
  if (!p.split) dst = static_cast<T*>(p.q) + b * p.C + ch0;
  else if (ch0 < p.key_dim) dst = static_cast<T*>(p.q) + b * p.key_dim + ch0;
  else if (ch0 < 2 * p.key_dim) dst = static_cast<T*>(p.k) + b * p.key_dim + ch0 - p.key_dim;
  else dst = static_cast<T*>(p.v) + b * (p.C - 2 * p.key_dim) + ch0 - 2 * p.key_dim;
  *reinterpret_cast<uint4*>(dst) = y;
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
  int64_t rows;  // slots of the conv frame table
  int64_t granules, cf, fe, num_frames, layer;
  const void* slots; int slots_is64;
  const void* gran; int gran_is64;
  const void* finals; int finals_is64;
  int64_t end0, end1;  // input scales, as ConvFrameParams
  float s0, s1, s2;
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
  const float sc = ch < p.end0 ? p.s0 : (ch < p.end1 ? p.s1 : p.s2);
  for (int j = 0; j < p.S; ++j) {
    const int64_t pos = t - (p.S - 1) + j;
    // inputs are scaled (and rounded) as the conv reads them; the history is not
    const T v = pos >= begin ? (sc != 1.f ? from_f32<T>(to_f32(x[pos * p.xr + ch * p.xc]) * sc)
                                          : x[pos * p.xr + ch * p.xc])
                             : hist[pos - begin + p.S];
    T* d0 = conv_element(st, p.table, p.table_is64, p.rows, slot, granule, e0 + j, p.granules, p.cf, p.fe,
                         p.num_frames);
    T* d1 = conv_element(st, p.table, p.table_is64, p.rows, fin, 0, e0 + j, p.granules, p.cf, p.fe, p.num_frames);
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
  int64_t rows;  // slots of the payload and decay frame tables
  int64_t fps, frame_bytes, head_bytes, num_frames;
  const void* decay; int decay_is64;
  int64_t record_bytes;
  const void* work; int work_is64;
  const void* logs; int logs_is64;
  const void* offsets; int offsets_is64;
  const void* counts; int counts_is64;
  int64_t layer, layers, gran, page;
  int eager;
  int hpb;    // value heads per block (divides HV)
  int group;  // value heads per key head
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

// grid (batch x HV / hpb); a block takes hpb value heads of one sequence in
// turn with NCW compute waves and one loading wave.
//
// The loading wave issues every global load of the block.  One head ahead of
// the compute waves it resolves the head's frame-table entries and moves the
// state (row-major, 16-byte chunks XOR-swizzled by row), the replayed log rows
// (token-major, zero past the replay count), the q / k / v rows and the
// step's store addresses into LDS -- the state and rows by direct-to-LDS
// loads into a double buffer -- and waits for its own loads only.  The
// compute waves read LDS, compute and store; they issue no global load, so no
// wait of theirs covers a store, and a head's loads are in flight while the
// previous head computes.  Two barriers per head: MID (the replayed rows are
// consumed, the single row buffer may be refilled) and END (the next head is
// resident).
//
// Compute wave w owns the TPW d_v row tiles TPW w .. of T = S^T (dv x dk),
// held as 16 x 16 MFMA result tiles: lane l has the dk column 16 it + l % 16
// of tile it and the dv rows 16 jt + 4 (l / 16) .. + 3 of row tile jt, four
// consecutive elements of a state row.  The replay T += V'^T K is one 16-deep
// MFMA per tile, its operands read from the token-major rows by LDS transpose
// reads; S^T k and S^T q are per-lane FMAs and a 16-lane DPP sum.
template <int DK, int DV>
struct DecodeShape {
  static constexpr int TPW = DV >= 128 ? 4 : 1;           // dv row tiles per compute wave
  static constexpr int NCW = DV / (16 * TPW);             // compute waves
  static constexpr int NT = 64 * (NCW + 1);               // threads (the last wave loads)
  static constexpr int RT = DK / 16;                      // dk tiles
  static constexpr int KV = DK / 8, VV = DV / 8;          // 16-byte chunks of a key / value row
  static constexpr int SCH = DK * VV;                     // 16-byte chunks of a state
  static constexpr int PCH = kReplayWindow * (KV + VV);   // 16-byte chunks of the replayed rows
  static constexpr int QCH = 2 * KV + VV;                 // 16-byte chunks of q, k and v
  static_assert(QCH <= 64 && SCH % 64 == 0 && PCH % 64 == 0, "chunk split");
};

constexpr int kMaxHeadsPerBlock = 8;
// A head's scalars, computed by the loading wave when the block starts.
struct HeadScalars {
  float g, decay, beta;
  int state;  // frame-table entry of the work state (a head inside one frame)
};
template <int DK, int DV>
struct HeadSlot {
  int ok;                             // the work state is mapped
  // byte offsets into the frame storage (-1: none); offsets rather than
  // pointers, so that stores through them are known to be global stores
  int64_t head;                       // work state (a head inside one frame)
  int64_t vlog[DV / 8];               // the step's value row, per 16-byte chunk
  int64_t klog[DK / 8];               // the step's key row
  int64_t grec;                       // the step's gate record
};

typedef __attribute__((address_space(3))) void lds_void;
typedef short s4v_t __attribute__((ext_vector_type(4)));
// LDS transpose read: the 16 lanes of a group read a 4-row x 16-column block of
// 16-bit values (lane r: row r / 4, columns 4 (r % 4)..+3) and lane r receives
// column r of the 4 rows.
__device__ __forceinline__ uint2 tr_read16(const uint16_t* p) {
  typedef __attribute__((address_space(3))) s4v_t lds_s4;
  return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p)));
}
// Direct-to-LDS load of 16 bytes per active lane: lane l lands at lds + 16 l.
__device__ __forceinline__ void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_void*)(lds), 16, 0, 0);
}
// x of the lane CTRL names inside the lane's 16-lane row (row_shr:k), 0 past the row start.
template <int CTRL> __device__ __forceinline__ float dpp_shr(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, true));
}
// s_waitcnt vmcnt(0) lgkmcnt(0) as the builtin, so that the compiler knows
// that every earlier load has landed and adds no wait of its own for them.
__device__ __forceinline__ void wait_all() {
  __builtin_amdgcn_s_waitcnt(0x0070);  // gfx9 encoding: vmcnt 0, expcnt 7 (no wait), lgkmcnt 0
  asm volatile("" ::: "memory");
}
// s_waitcnt vmcnt(N) as the builtin (expcnt and lgkmcnt not waited for).
template <int N> __device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0070 | 0x0f00);
  asm volatile("" ::: "memory");
}
// LDS reads issued as one statement with their own lgkmcnt wait.  A wave
// that also has direct-to-LDS loads in flight uses these: the compiler orders
// every LDS read it knows of behind all such loads (s_waitcnt vmcnt(0)),
// whatever buffer they fill; the caller's own counted wait and barrier make
// the data it reads resident instead.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)(p)));
}
// Four transpose reads (two 16-column operand tiles of 8 tokens).
__device__ __forceinline__ void tr_read16x4(const uint16_t* a0, const uint16_t* a1, const uint16_t* a2,
                                            const uint16_t* a3, uint4& x, uint4& y) {
  uint2 r0, r1, r2, r3;
  asm volatile(
      "ds_read_b64_tr_b16 %0, %4\n\t"
      "ds_read_b64_tr_b16 %1, %5\n\t"
      "ds_read_b64_tr_b16 %2, %6\n\t"
      "ds_read_b64_tr_b16 %3, %7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
      : "v"(lds_addr(a0)), "v"(lds_addr(a1)), "v"(lds_addr(a2)), "v"(lds_addr(a3))
      : "memory");
  x = make_uint4(r0.x, r0.y, r1.x, r1.y);
  y = make_uint4(r2.x, r2.y, r3.x, r3.y);
}
__device__ __forceinline__ uint4 tr_read16x2(const uint16_t* a0, const uint16_t* a1) {
  uint2 r0, r1;
  asm volatile(
      "ds_read_b64_tr_b16 %0, %2\n\t"
      "ds_read_b64_tr_b16 %1, %3\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1)
      : "v"(lds_addr(a0)), "v"(lds_addr(a1))
      : "memory");
  return make_uint4(r0.x, r0.y, r1.x, r1.y);
}
// Direct-to-LDS load of 4 bytes per active lane: lane l lands at lds + 4 l.
__device__ __forceinline__ void dma4(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)(lds), 4, 0, 0);
}
// N (1..4) 4-byte reads.
template <int N> __device__ __forceinline__ void lds_read32(const int32_t* const (&a)[N], int32_t (&v)[N]) {
  static_assert(N >= 1 && N <= 4, "1..4 reads");
  if constexpr (N == 1) {
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v[0]) : "v"(lds_addr(a[0])) : "memory");
  } else if constexpr (N == 2) {
    asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]) : "v"(lds_addr(a[0])), "v"(lds_addr(a[1])) : "memory");
  } else if constexpr (N == 3) {
    asm volatile("ds_read_b32 %0, %3\n\tds_read_b32 %1, %4\n\tds_read_b32 %2, %5\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2])
                 : "v"(lds_addr(a[0])), "v"(lds_addr(a[1])), "v"(lds_addr(a[2])) : "memory");
  } else {
    asm volatile(
        "ds_read_b32 %0, %4\n\tds_read_b32 %1, %5\n\tds_read_b32 %2, %6\n\tds_read_b32 %3, %7\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
        : "v"(lds_addr(a[0])), "v"(lds_addr(a[1])), "v"(lds_addr(a[2])), "v"(lds_addr(a[3])) : "memory");
  }
}
// Two 16-byte reads.
__device__ __forceinline__ void lds_read128x2(const float* a0, const float* a1, float4& x, float4& y) {
  asm volatile(
      "ds_read_b128 %0, %2\n\t"
      "ds_read_b128 %1, %3\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x), "=&v"(y)
      : "v"(lds_addr(a0)), "v"(lds_addr(a1))
      : "memory");
}
// Chunk position of logical chunk c in row r of a swizzled row-major array
// with `chunks` 16-byte chunks per row (a power of two).
__device__ __forceinline__ int swz_state(int r, int c, int chunks) { return c ^ (r & (chunks - 1)); }
__device__ __forceinline__ int swz_rows(int t, int c, int chunks) { return c ^ ((2 * (t & 3)) & (chunks - 1)); }

template <int DK, int DV, class T>
__global__ __launch_bounds__((DecodeShape<DK, DV>::NT)) __attribute__((amdgpu_waves_per_eu(2))) void logstate_decode_kernel(LogDecodeParams p) {
  using S = DecodeShape<DK, DV>;
  constexpr int TPW = S::TPW, NCW = S::NCW, RT = S::RT, KV = S::KV, VV = S::VV;
  constexpr uint32_t kRow = DV * 2;  // bytes of a state row
  static_assert(sizeof(T) == 2, "16-bit frames");
  __shared__ __align__(16) uint16_t sS[2][DK * DV];                      // states
  __shared__ __align__(16) uint16_t sP[kReplayWindow * (DK + DV)];       // replayed key rows, then value rows
  __shared__ __align__(16) uint16_t sQ[2][2 * DK + DV];                  // q, k, v rows
  __shared__ HeadSlot<DK, DV> sH[2];
  __shared__ HeadScalars sHS[kMaxHeadsPerBlock];
  __shared__ float sGt[kMaxHeadsPerBlock][kReplayWindow];  // replayed tokens' gates per head
  __shared__ float sSfx[NCW][kReplayWindow];
  uint16_t* const sPk = sP;
  uint16_t* const sPv = sP + kReplayWindow * DK;

  const uint32_t nhv = static_cast<uint32_t>(p.HV), hpb = static_cast<uint32_t>(p.hpb);
  const uint32_t group = static_cast<uint32_t>(p.group);
  const uint32_t ngroups = nhv / hpb, bid = blockIdx.x;
  const uint32_t b = bid / ngroups, h0 = (bid % ngroups) * hpb;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, lg = lane >> 4;

  // ---- the sequence's slots, read by every wave (uniform)
  // slots past the frame tables are unmapped, as negative ones
  const int64_t w_raw = load_index(p.work, b, p.work_is64), ls_raw = load_index(p.logs, b, p.logs_is64);
  const int w = w_raw < p.rows ? static_cast<int>(w_raw) : -1;
  const int ls = ls_raw < p.rows ? static_cast<int>(ls_raw) : -1;
  const int pos = static_cast<int>(load_index(p.offsets, b, p.offsets_is64));
  const bool in_page = ls >= 0 && pos >= 0 && pos < p.page;
  int n = p.eager || !in_page ? 0 : static_cast<int>(load_index(p.counts, b, p.counts_is64));
  n = n < 0 ? 0 : (n > kReplayWindow ? kReplayWindow : n);
  n = n > pos ? pos : n;  // the logged tokens precede the position within the page
  float* rec = nullptr;   // decay record of the log slot
  if (in_page) {
    const int64_t fr = load_index(p.decay, 2 * static_cast<int64_t>(ls), p.decay_is64);
    const int64_t ri = load_index(p.decay, 2 * static_cast<int64_t>(ls) + 1, p.decay_is64);
    if (fr >= 0 && fr < p.num_frames && ri >= 0 && (ri + 1) * p.record_bytes <= p.frame_bytes)
      rec = reinterpret_cast<float*>(p.storage + fr * p.frame_bytes + ri * p.record_bytes);
  }
  if (!rec) n = 0;
  const bool one_frame = p.head_bytes <= p.frame_bytes;  // a head inside one frame
  const uint32_t layer = static_cast<uint32_t>(p.layer), gran = static_cast<uint32_t>(p.gran);

  if (wave == NCW) {
    // ==================================================================== loading wave
    // The loading wave issues before the compute waves of its SIMD, and its
    // frame arithmetic is shifts and masks for power-of-two frames.
    __builtin_amdgcn_s_setprio(3);
    auto loader = [&](auto pow2) __attribute__((always_inline)) {
    constexpr bool POW2 = decltype(pow2)::value;
    auto fdivv = [&](uint32_t x) -> uint32_t {
      if constexpr (POW2) return x >> p.fdiv.shift;
      else return x / p.fdiv.d;
    };
    auto fmodv = [&](uint32_t x) -> uint32_t {
      if constexpr (POW2) return x & (p.fdiv.d - 1);
      else return x % p.fdiv.d;
    };
    auto fbase = [&](int64_t fr) -> int64_t {
      if constexpr (POW2) return fr << p.fdiv.shift;
      else return fr * p.frame_bytes;
    };
    const int64_t wrow = static_cast<int64_t>(w >= 0 ? w : 0) * p.fps;   // frame-table rows of the slots
    const int64_t lrow = static_cast<int64_t>(ls >= 0 ? ls : 0) * p.fps;
    auto frame_at = [&](int64_t fr, uint32_t byte) -> char* {  // null for an unmapped entry
      return fr >= 0 && fr < p.num_frames ? p.storage + fbase(fr) + fmodv(byte) : nullptr;
    };
    const uint32_t key_size = gran * static_cast<uint32_t>(p.H) * DK;
    const uint32_t layer_size = key_size + gran * nhv * DV;
    auto log_byte = [&](uint32_t t, uint32_t index, uint32_t col, bool value) -> uint32_t {
      const uint32_t elem = (p.gdiv.div(t) * static_cast<uint32_t>(p.layers) + layer) * layer_size +
                            (value ? key_size : 0u) + (index * gran + p.gdiv.mod(t)) * (value ? DV : DK) + col;
      return 2u * elem;
    };
    auto state_byte = [&](uint32_t h) { return static_cast<uint32_t>((layer * nhv + h) * p.head_bytes); };
    // log positions outside the page are never read or written; they look up position 0
    const uint32_t tp = in_page ? static_cast<uint32_t>(pos) : 0u;
    // replayed chunk k * 64 + lane: token t, chunk position c of its key or value
    // row; its byte offset in the slot's log without the head term (per block)
    constexpr int PK = S::PCH / 64;
    bool pval[PK], plive[PK];
    uint32_t pbase[PK];
#pragma unroll
    for (int k = 0; k < PK; ++k) {
      const int P = k * 64 + lane;
      const bool value = P >= kReplayWindow * KV;
      const int Q = value ? P - kReplayWindow * KV : P;
      const int per = value ? VV : KV;
      const int t = Q / per, c = swz_rows(t, Q % per, per);  // logical chunk stored at this position
      const uint32_t tok = in_page ? static_cast<uint32_t>(pos - n + (t < n ? t : 0)) : 0u;
      pval[k] = value;
      plive[k] = t < n;
      pbase[k] = log_byte(tok, 0, 8u * c, value);
    }
    const uint32_t vhead = 2u * gran * DV, khead = 2u * gran * DK;  // log bytes per value / key head
    const uint32_t vbase = log_byte(tp, 0, 8u * (lane < VV ? lane : 0), true);
    const uint32_t kbase = log_byte(tp, 0, 8u * (lane < KV ? lane : 0), false);
    // head h's frame-table entries and scalars, loaded one head ahead
    struct Entries {
      int piece[PK], vrow, krow;
    };
    auto entries = [&](uint32_t h) {
      Entries e;
      const uint32_t kh = h / group;
#pragma unroll
      for (int k = 0; k < PK; ++k)
        e.piece[k] = static_cast<int>(load_index(
            p.frames, lrow + fdivv(pbase[k] + (pval[k] ? h * vhead : kh * khead)), p.frames_is64));
      e.vrow = static_cast<int>(load_index(p.frames, lrow + fdivv(vbase + h * vhead), p.frames_is64));
      e.krow = static_cast<int>(load_index(p.frames, lrow + fdivv(kbase + kh * khead), p.frames_is64));
      return e;
    };
    // state rows: instruction k = 4 kk + j moves rows RPI k .. of the state; the
    // lane part of its source offset depends on j only
    constexpr int NI = S::SCH / 64, RPI = 64 / VV;
    uint32_t soff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = RPI * j + lane / VV;
      soff[j] = r * kRow + 16 * swz_state(r, lane % VV, VV);
    }
    // state, q / k / v rows and the head's scalars and store addresses into slot s
    auto fill_main = [&](uint32_t h, int s, const Entries& e) {
      const uint32_t kh = h / group;
      char* head = one_frame && w >= 0 ? frame_at(sHS[h - h0].state, state_byte(h)) : nullptr;
      const bool ok = one_frame ? head != nullptr : w >= 0;
      if (one_frame) {
        if (head) {  // else the compute waves take a zero state
#pragma unroll 1
          for (int kk = 0; kk < (NI + 3) / 4; ++kk) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int k = 4 * kk + j;
              if (k < NI) dma16(head + kk * 4 * RPI * kRow + soff[j], &sS[s][k * 64 * 8]);
            }
          }
        }
      } else if (w >= 0) {  // a head over several frames: a lookup per row, unmapped rows zero
#pragma unroll 1
        for (int k = 0; k < NI; ++k) {
          const int P = k * 64 + lane, r = P / VV, c = swz_state(r, P % VV, VV);
          const T* row = state_row<T>(p, w, h, r, DV);
          if (row) dma16(reinterpret_cast<const char*>(row) + 16 * c, &sS[s][k * 64 * 8]);
          else *reinterpret_cast<uint4*>(&sS[s][P * 8]) = make_uint4(0, 0, 0, 0);
        }
      }
      // q, k, v rows
      {
        const T* q = static_cast<const T*>(p.q) + (static_cast<int64_t>(b) * p.H + kh) * DK;
        const T* k = static_cast<const T*>(p.k) + (static_cast<int64_t>(b) * p.H + kh) * DK;
        const T* v = static_cast<const T*>(p.v) + (static_cast<int64_t>(b) * nhv + h) * DV;
        const int c = lane < KV ? lane : (lane < 2 * KV ? lane - KV : lane - 2 * KV);
        const T* src = lane < KV ? q : (lane < 2 * KV ? k : v);
        if (lane < S::QCH) dma16(src + 8 * c, &sQ[s][0]);
      }
      // scalars and addresses
      HeadSlot<DK, DV>& hs = sH[s];
      auto off = [&](const char* q) -> int64_t { return q ? q - p.storage : -1; };
      if (lane < VV) hs.vlog[lane] = in_page ? off(frame_at(e.vrow, vbase + h * vhead)) : -1;
      if (lane < KV) hs.klog[lane] = in_page && h % group == 0 ? off(frame_at(e.krow, kbase + kh * khead)) : -1;
      if (lane == 0) {
        hs.ok = ok ? 1 : 0;
        hs.head = off(head);
        hs.grec = in_page && rec ? off(reinterpret_cast<const char*>(
                                       rec + (layer * static_cast<uint32_t>(p.page) + static_cast<uint32_t>(pos)) * nhv + h))
                                 : -1;
      }
    };
    // the replayed rows of head h into registers (issued early), then into LDS
    // (zeros past n and for unmapped chunks)
    struct Rows {
      uint4 v[PK];
      bool live[PK];
    };
    auto load_rows = [&](uint32_t h, const Entries& e) {
      Rows r;
      const uint32_t kh = h / group;
#pragma unroll
      for (int k = 0; k < PK; ++k) {
        const char* src = plive[k] ? frame_at(e.piece[k], pbase[k] + (pval[k] ? h * vhead : kh * khead)) : nullptr;
        r.live[k] = src != nullptr;
        r.v[k] = *reinterpret_cast<const uint4*>(src ? src : p.storage);
      }
      return r;
    };
    auto store_rows = [&](const Rows& r) {
#pragma unroll
      for (int k = 0; k < PK; ++k)
        *reinterpret_cast<uint4*>(&sP[(k * 64 + lane) * 8]) = r.live[k] ? r.v[k] : make_uint4(0, 0, 0, 0);
    };
    // every head's scalars and work-state entry, and the replayed gates
    if (lane < static_cast<int>(hpb)) {
      const uint32_t h = h0 + lane;
      const float a_log = load_any(p.A_log, h, p.a_dtype);
      const float dt = load_any(p.dt_bias, h, p.dt_dtype);
      const float graw = load_any(p.gate, b * p.gate_b + h * p.gate_h, p.gate_dtype);
      const float braw = load_any(p.beta, b * p.beta_b + h * p.beta_h, p.beta_dtype);
      const float g = -expf(a_log) * softplus_decode(graw + dt);
      sHS[lane] = HeadScalars{g, expf(g), sigmoid(braw),
                              static_cast<int>(load_index(p.frames, wrow + fdivv(state_byte(h)), p.frames_is64))};
    }
    for (int i = lane; i < static_cast<int>(hpb) * kReplayWindow; i += 64) {
      const int hh = i / kReplayWindow, t = i % kReplayWindow;
      const uint32_t gbase = (layer * static_cast<uint32_t>(p.page) + static_cast<uint32_t>(pos - n)) * nhv + h0 + hh;
      sGt[hh][t] = t < n ? rec[gbase + (t < n ? t : 0) * nhv] : 0.f;
    }
    wait_all();
    Entries cur = entries(h0);
    fill_main(h0, 0, cur);
    store_rows(load_rows(h0, cur));
    cur = entries(hpb > 1 ? h0 + 1 : h0);
    wait_all();
    lds_barrier();  // head 0 resident
    for (uint32_t hi = 0; hi < hpb; ++hi) {
      const bool more = hi + 1 < hpb;
      Rows rows;
      Entries nxt = cur;
      if (more) {
        fill_main(h0 + hi + 1, (hi + 1) & 1, cur);
        rows = load_rows(h0 + hi + 1, cur);
        nxt = entries(hi + 2 < hpb ? h0 + hi + 2 : h0 + hi + 1);
      }
      lds_barrier();  // MID: the compute waves have read the replayed rows
      if (more) store_rows(rows);
      cur = nxt;
      wait_all();
      lds_barrier();  // END: the next head is resident
    }
    };
    if (p.fdiv.shift >= 0) loader(std::true_type{});
    else loader(std::false_type{});
    return;
  }

  // ====================================================================== compute waves
  int j0[TPW];  // this lane's dv rows j0[u] .. j0[u] + 3 of row tile TPW wave + u
#pragma unroll
  for (int u = 0; u < TPW; ++u) j0[u] = 16 * (TPW * wave + u) + 4 * lg;
  lds_barrier();  // head 0 resident
  for (uint32_t hi = 0; hi < hpb; ++hi) {
    const uint32_t h = h0 + hi;
    const int s = hi & 1;
    const HeadSlot<DK, DV>& hs = sH[s];
    const uint16_t* q = &sQ[s][0];
    const uint16_t* k = q + DK;
    const uint16_t* v = k + DK;
    float qv[RT], kv[RT];  // q, k at this lane's dk columns
#pragma unroll
    for (int it = 0; it < RT; ++it) {
      qv[it] = to_f32(__builtin_bit_cast(T, q[16 * it + lr]));
      kv[it] = to_f32(__builtin_bit_cast(T, k[16 * it + lr]));
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
    const float decay = sHS[hi].decay, beta = sHS[hi].beta;
    // inclusive scan of the replayed gates over lanes 0 .. n-1 (DPP shifts
    // inside the first 16-lane row); suffix_i = e^{total - prefix_i}
    float scan = lane < n ? sGt[hi][lane & (kReplayWindow - 1)] : 0.f;
    scan += dpp_shr<0x111>(scan);
    scan += dpp_shr<0x112>(scan);
    scan += dpp_shr<0x114>(scan);
    scan += dpp_shr<0x118>(scan);
    const float total = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(scan), kReplayWindow - 1));
    const float total_decay = expf(total);
    if (lane < kReplayWindow) {
      int l = lane;  // opaque, so that no address is held in a register across heads
      asm volatile("" : "+v"(l));
      (&sSfx[0][0])[wave * kReplayWindow + l] = expf(total - scan);
    }

    // ---- the state, decayed over the replayed tokens
    f4_t Tt[TPW][RT];
#pragma unroll
    for (int u = 0; u < TPW; ++u)
#pragma unroll
      for (int it = 0; it < RT; ++it) {
        const int r = 16 * it + lr, c = j0[u] >> 3;
        const uint2 raw = *reinterpret_cast<const uint2*>(&sS[s][r * DV + 8 * swz_state(r, c, VV) + (j0[u] & 7)]);
        float a, c2, d, e;
        split2<T>(hs.ok ? raw.x : 0u, a, c2);
        split2<T>(hs.ok ? raw.y : 0u, d, e);
        Tt[u][it] = f4_t{a, c2, d, e} * total_decay;
      }
    if (n > 0) {
      // T += V'^T K: values scaled by their suffix decay and rounded to the
      // state dtype (tokens past n are zero rows)
      f4_t sfx;
#pragma unroll
      for (int e = 0; e < 4; ++e) sfx[e] = sSfx[wave][4 * lg + e];
      auto row_addr = [&](const uint16_t* base, int per, int col) {  // lane's transpose-read address
        const int t = 4 * lg + (lr >> 2), cc = (col >> 3), half = (col & 7);
        return base + t * per * 8 + 8 * swz_rows(t, cc, per) + half;
      };
#pragma unroll
      for (int u = 0; u < TPW; ++u) {
        const uint2 raw = tr_read16(row_addr(sPv, VV, 16 * (TPW * wave + u) + 4 * (lr & 3)));
        float a, c2, d, e;
        split2<T>(raw.x, a, c2);
        split2<T>(raw.y, d, e);
        const uint2 af = make_uint2(out_pack2<T>(a * sfx[0], c2 * sfx[1]), out_pack2<T>(d * sfx[2], e * sfx[3]));
#pragma unroll
        for (int it = 0; it < RT; ++it) {
          const uint2 bf = tr_read16(row_addr(sPk, KV, 16 * it + 4 * (lr & 3)));
          Tt[u][it] = mma16<T>(af, bf, Tt[u][it]);
        }
      }
    }
    float vin[TPW][4];
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      const uint2 raw = *reinterpret_cast<const uint2*>(v + j0[u]);
      split2<T>(raw.x, vin[u][0], vin[u][1]);
      split2<T>(raw.y, vin[u][2], vin[u][3]);
    }
    lds_barrier();  // MID: the replayed rows are consumed

    // ---- the step's scalars and store addresses (this slot's stay until END)
    const float g = sHS[hi].g;
    const bool ok = hs.ok != 0;
    const int64_t klog = hs.klog[tid % KV];
    const int64_t grec = hs.grec;
    const bool write_back = ok && (p.eager || (pos + 1) % kReplayWindow == 0);
    char* const orow = static_cast<char*>(p.out) + (static_cast<int64_t>(b) * nhv + h) * kRow;
    // a work state in one frame: a uniform base plus an opaque 32-bit lane offset
    const uint64_t ho = hs.head;
    char* const hb = p.storage + ((static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(ho >> 32)))
                                   << 32) |
                                  __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(ho)));

    // ---- one step per d_v tile: row sums of T against k and q (S^T k, S^T q)
    // for rows j0 + e, then the tile's output, log row and work-state rows
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      float delta[4], out[4];
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
          delta[e] = (vin[u][e] - row16_sum(acc)) * beta;
          float accq = 0.f;
#pragma unroll
          for (int it = 0; it < RT; ++it) {
            Tt[u][it][e] = fmaf(delta[e], kv[it], Tt[u][it][e]);
            accq = fmaf(Tt[u][it][e], qv[it], accq);
          }
          out[e] = row16_sum(accq);
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
          delta[e] = (vin[u][e] - row16_sum(ak) * decay) * beta;
          out[e] = row16_sum(aq) * decay + delta[e] * kq;
        }
      }
      if (lr == 0) {
        uint32_t o = 2 * j0[u];  // opaque 32-bit lane offset from a uniform base
        asm volatile("" : "+v"(o));
        *reinterpret_cast<uint2*>(orow + o) = make_uint2(out_pack2<T>(out[0], out[1]), out_pack2<T>(out[2], out[3]));
        const int64_t vlog = hs.vlog[j0[u] >> 3];
        if (vlog >= 0)
          *reinterpret_cast<uint2*>(p.storage + vlog + (o & 15)) =
              make_uint2(out_pack2<T>(delta[0], delta[1]), out_pack2<T>(delta[2], delta[3]));
      }
      // the work state: every step (eager), else at the end of a replay window
      if (write_back) {
#pragma unroll
        for (int it = 0; it < RT; ++it) {
          uint32_t lo = lr * kRow + 2 * j0[u];
          asm volatile("" : "+v"(lo));
          char* row = hb + it * 16 * kRow + lo;
          if (!one_frame) {  // a head over several frames: a lookup per row
            T* r = state_row<T>(p, w, h, 16 * it + lr, DV);
            if (!r) continue;
            row = reinterpret_cast<char*>(r) + 2 * j0[u];
          }
          float v4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v4[e] = p.eager ? Tt[u][it][e] : fmaf(delta[e], kv[it], Tt[u][it][e] * decay);
          *reinterpret_cast<uint2*>(row) = make_uint2(out_pack2<T>(v4[0], v4[1]), out_pack2<T>(v4[2], v4[3]));
        }
      }
    }
    if (tid < KV && klog >= 0) {
      int c = 8 * tid;  // opaque, as above
      asm volatile("" : "+v"(c));
      const uint4 raw = *reinterpret_cast<const uint4*>(k + c);
      const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
      uint32_t pk[4];
#pragma unroll
      for (int q2 = 0; q2 < 4; ++q2) {
        float a, b2;
        split2<T>(wv[q2], a, b2);
        pk[q2] = out_pack2<T>(a * rk, b2 * rk);
      }
      *reinterpret_cast<uint4*>(p.storage + klog) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
    if (grec >= 0 && tid == 0) *reinterpret_cast<float*>(p.storage + grec) = g;
    lds_barrier();  // END: the next head is resident
  }
}

// ---- restore / copy of LogState slot states (kernel/linear_attention/logstate.py:59-128)
struct RestoreParams {
  char* storage;
  const void* frames; int frames_is64;
  int64_t rows;  // slots of the payload and decay frame tables
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
  int64_t tasks;
  Div32 fdiv, gdiv;         // frame_bytes, gran
};

// State row of (slot, layer, head) in a frame storage (the layout of
// gdn_chunk_gated_delta_rule's frame tables), or null.
template <class T>
__device__ __forceinline__ T* slot_row(const RestoreParams& p, int64_t s, int64_t layer, int64_t h, int64_t row,
                                       int DV) {
  if (s < 0 || s >= p.rows) return nullptr;
  const uint32_t x = static_cast<uint32_t>((layer * p.HV + h) * p.head_bytes + row * DV * static_cast<int64_t>(sizeof(T)));
  const int64_t fr = load_index(p.frames, s * p.fps + p.fdiv.div(x), p.frames_is64);
  if (fr < 0 || fr >= p.num_frames) return nullptr;
  return reinterpret_cast<T*>(p.storage + fr * p.frame_bytes + p.fdiv.mod(x));
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

constexpr int kRestoreStep = 32;              // tokens staged per step (one 32-deep product per tile)
constexpr int kRestoreSpan = kDecodeThreads;  // tokens whose suffix decays one block scan yields

// 16 zero bytes: the source of the direct-to-LDS loads for rows past a
// segment's end or in an unmapped frame.
__device__ uint4 g_zero_piece;

// grid (tasks x layers x HV), 4 waves: the state of the task's base slot (or
// zero), then each segment of logged tokens t = b .. e-1 in one step,
// S <- e^{sum_t g_t} S + sum_t k_t (e^{sum_{j>t} g_j} v'_t)^T with the scaled
// v' rounded to the state dtype (logstate_construction.cuh:329-393); written
// to the output slot.  The sum runs on MFMA, 32 tokens per step: the step's
// key and value rows land token-major in one of two LDS buffers by
// direct-to-LDS loads (16-byte chunks XOR-swizzled by row), issued one step
// ahead of the products, with their frame-table entries loaded two steps
// ahead; both MFMA operands come out of the token-major rows by transpose
// reads (`ds_read_b64_tr_b16`), the values scaled by their suffix decay on
// the way.  Each wave owns the state's columns of DV / 64 (at least one)
// 16-wide tiles over all DK rows in fp32 accumulators.  The suffix decays of
// 256 tokens come from one block scan of their gates.  Every wait of the
// step loop covers loads only (the state is stored after the loop).
template <int DK, int DV, class T>
__global__ __launch_bounds__(kDecodeThreads) __attribute__((amdgpu_waves_per_eu(3))) void restore_kernel(RestoreParams p) {
  constexpr int RT = DK / 16, CTT = DV / 16, CT = CTT >= 4 ? CTT / 4 : 1;
  constexpr int CHK = DK / 8, CHV = DV / 8;             // 16-byte chunks per key / value row
  constexpr int KI = kRestoreStep * 2 * DK / 1024;      // 1 KiB wave loads of a step's key rows
  constexpr int NI = KI + kRestoreStep * 2 * DV / 1024;  // ... and of all its rows
  constexpr int NIW = (NI + 3) / 4;                     // per wave
  static_assert(DK % 16 == 0 && DV % 16 == 0 && DK <= 512 && DV <= 512, "tile split");
  static_assert((kRestoreStep * 2 * DK) % 1024 == 0 && (kRestoreStep * 2 * DV) % 1024 == 0, "whole wave loads");
  // block -> (task, layer, key head, member v-head): the v-heads of one key
  // head run on one XCD (block i goes to XCD i mod 8) one after another, so
  // the key rows the first one fetches are L2 hits for the others
  const uint32_t bid = blockIdx.x, nl = static_cast<uint32_t>(p.layers), nkh = static_cast<uint32_t>(p.KH);
  const uint32_t members = static_cast<uint32_t>(p.HV / p.KH);
  const uint32_t slot = bid / 8;
  const uint64_t group = static_cast<uint64_t>(slot / members) * 8 + bid % 8;
  if (group >= static_cast<uint64_t>(p.tasks) * nl * nkh) return;
  const int64_t task = static_cast<int64_t>(group / (nl * nkh));
  const int64_t layer = static_cast<int64_t>((group / nkh) % nl);
  const int64_t kh = static_cast<int64_t>(group % nkh);
  const int64_t h = kh * members + slot % members;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, lq = lane >> 4;
  const bool owner = wave * CT < CTT;  // this wave holds column tiles
  __shared__ __attribute__((aligned(16))) uint16_t s_k[3][kRestoreStep * DK];
  __shared__ __attribute__((aligned(16))) uint16_t s_v[3][kRestoreStep * DV];
  __shared__ __attribute__((aligned(16))) float s_suffix[kRestoreSpan];
  __shared__ int32_t s_ent[4][4 * kRestoreStep];  // frame entries of a step's 2 S rows (first / last byte), by step % 4
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
  // The piece of wave load k of this lane: token row t of the step, logical
  // 16-byte chunk c (the XOR swizzle of its LDS position), key or value row.
  struct Piece { int t, c; bool key; };
  auto piece_of = [&](int k) __attribute__((always_inline)) -> Piece {
    const int rg = wave + 4 * k;
    const bool key = rg < KI;
    const int r = key ? rg : rg - KI, ch = key ? CHK : CHV;
    const int t = r * (64 / ch) + lane / ch;  // 64 / ch rows of ch chunks per 1 KiB wave load
    return Piece{t, swz_rows(t, lane % ch, ch), key};
  };
  const void* const zero_piece = &g_zero_piece;
  const uint32_t key_size = static_cast<uint32_t>(p.gran * p.KH * DK);
  const uint32_t layer_size = key_size + static_cast<uint32_t>(p.gran * p.HV * DV);
  // Slot-relative byte of row r of the step at g0: rows 0 .. S-1 are the
  // tokens' key rows, S .. 2S-1 their value rows (a token past n reads the
  // first token's place).
  auto row_byte = [&](int64_t g0, int n, int r) __attribute__((always_inline)) -> uint32_t {
    const bool key = r < kRestoreStep;
    const int t = key ? r : r - kRestoreStep;
    const uint32_t ps = static_cast<uint32_t>(g0 + (t < n ? t : 0));
    const uint32_t elem = (p.gdiv.div(ps) * static_cast<uint32_t>(p.layers) + static_cast<uint32_t>(layer)) * layer_size +
                          (key ? 0u : key_size) +
                          (static_cast<uint32_t>(key ? kh : h) * static_cast<uint32_t>(p.gran) + p.gdiv.mod(ps)) *
                              static_cast<uint32_t>(key ? DK : DV);
    return 2u * elem;
  };
  // Frame-table entries of the step's rows into entry slot `slot`: waves 0
  // and 1, one 4-byte direct-to-LDS load per lane, entry 2 r + 0 / 1 for the
  // frames of row r's first / last byte (a row spans at most two frames).
  const int32_t* const ftab = static_cast<const int32_t*>(p.frames);
  auto lookup = [&](int64_t ls, int64_t g0, int n, int slot) __attribute__((always_inline)) {
    if (wave < 2) {
      const int q = wave * 64 + lane, r = q >> 1;
      const uint32_t last = 2u * static_cast<uint32_t>(r < kRestoreStep ? DK : DV) - 1u;
      const uint32_t b = row_byte(g0, n, r) + ((q & 1) ? last : 0u);
      dma4(ftab + (ls * p.fps + p.fdiv.div(b)) * (p.frames_is64 ? 2 : 1), &s_ent[slot][wave * 64]);
    }
  };
  // Direct-to-LDS loads of the step's rows into buffer b from the entries in
  // slot `slot` (zeros past n and for unmapped frames).
  auto stage = [&](int b, int64_t g0, int n, int slot) __attribute__((always_inline)) {
    const int32_t* ea[NIW];
    uint32_t pb[NIW];
#pragma unroll
    for (int k = 0; k < NIW; ++k) {
      const Piece pc = piece_of(k);
      const int r = wave + 4 * k < NI ? (pc.key ? pc.t : kRestoreStep + pc.t) : 0;  // pieces past NI: unused
      const uint32_t rb = row_byte(g0, n, r);
      pb[k] = rb + 16u * static_cast<uint32_t>(pc.c);
      ea[k] = &s_ent[slot][2 * r + (p.fdiv.div(pb[k]) != p.fdiv.div(rb) ? 1 : 0)];
    }
    int32_t entry[NIW];
    lds_read32<NIW>(ea, entry);
#pragma unroll
    for (int k = 0; k < NIW; ++k) {
      const int rg = wave + 4 * k;
      if (rg >= NI) break;
      // branch-free select
      const bool live = (piece_of(k).t < n) & (entry[k] >= 0) & (entry[k] < p.num_frames);
      const char* a = p.storage + static_cast<int64_t>(entry[k]) * p.frame_bytes + p.fdiv.mod(pb[k]);
      const void* src = live ? static_cast<const void*>(a) : zero_piece;
      uint16_t* dst = rg < KI ? &s_k[b][rg * 512] : &s_v[b][(rg - KI) * 512];
      dma16(src, dst);
    }
  };
  const int64_t out = p.output[task];
  const T* out_head = p.head_bytes <= p.frame_bytes ? slot_row<T>(p, out, layer, h, 0, DV) : nullptr;
  // Loads a wave has in flight after the last step's rows at the end of a
  // step: its rows of the next step and, in waves 0-1, one lookup.  The
  // count is exact when NI is a multiple of 4 (every wave the same pieces).
  auto wait_step = [&]() __attribute__((always_inline)) {
    if constexpr (NI % 4 == 0) {
      if (wave < 2) wait_vm<NIW + 1>(); else wait_vm<NIW>();
    } else {
      wait_all();
    }
  };
  for (int64_t seg = p.offsets[task]; seg < p.offsets[task + 1]; ++seg) {
    const int64_t ls = p.seg_slots[seg];
    const int64_t begin = p.seg_begin[seg] < 0 ? 0 : p.seg_begin[seg];
    const int64_t end = p.seg_end[seg] < p.page ? p.seg_end[seg] : p.page;
    int64_t fr = -1, ri = -1;
    if (ls >= 0 && ls < p.rows && begin < end) {
      fr = load_index(p.decay, 2 * ls, p.decay_is64);
      ri = load_index(p.decay, 2 * ls + 1, p.decay_is64);
    }
    const bool ok = fr >= 0 && fr < p.num_frames && ri >= 0 && (ri + 1) * p.record_bytes <= p.frame_bytes;
    if (!ok || begin >= end) continue;
    const float* rec =
        reinterpret_cast<const float*>(p.storage + fr * p.frame_bytes + ri * p.record_bytes) + layer * p.page * p.HV + h;
    // gate sum over the segment: a pass of its own when the segment spans
    // more than one scan, else the scan's total
    const bool one_span = end - begin <= kRestoreSpan;
    float total = 0.f;
    if (!one_span) {
      float part = 0.f;
      for (int64_t t = begin + tid; t < end; t += kDecodeThreads) part += rec[t * p.HV];
      part = wave_sum(part);
      lds_barrier();  // the previous segment's last step is consumed
      if (lane == 0) s_part[wave] = part;
      lds_barrier();
#pragma unroll
      for (int w = 0; w < kDecodeThreads / 64; ++w) total += s_part[w];
    }
    float rest = 0.f;  // the gates of the segment's tokens before the span
    for (int64_t sb = begin; sb < end; sb += kRestoreSpan) {
      const int64_t span_end = sb + kRestoreSpan < end ? sb + kRestoreSpan : end;
      const int steps = static_cast<int>((span_end - sb + kRestoreStep - 1) / kRestoreStep);
      // step j of the span: its first position and token count (a step past
      // the span is a dummy with no tokens at the span start)
      auto first = [&](int j) __attribute__((always_inline)) {
        return j < steps ? sb + static_cast<int64_t>(j) * kRestoreStep : sb;
      };
      auto count = [&](int j) __attribute__((always_inline)) {
        const int64_t left = span_end - sb - static_cast<int64_t>(j) * kRestoreStep;
        return j < steps ? static_cast<int>(left < kRestoreStep ? left : kRestoreStep) : 0;
      };
      lds_barrier();  // s_part, the entry slots and the previous span's suffixes and rows are consumed
#pragma unroll
      for (int j = 0; j < 4; ++j) lookup(ls, first(j), count(j), j);
      // suffix decays of the span: one block inclusive scan of its gates
      float x = sb + tid < end ? rec[(sb + tid) * p.HV] : 0.f;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
      }
      if (lane == 63) s_part[wave] = x;
      wait_all();     // the entries of steps 0-3 have landed
      lds_barrier();  // for every wave
      stage(0, first(0), count(0), 0);
      stage(1, first(1), count(1), 1);
      float before = rest, span = 0.f;
#pragma unroll
      for (int w = 0; w < kDecodeThreads / 64; ++w) {
        before += w < wave ? s_part[w] : 0.f;
        span += s_part[w];
      }
      if (one_span) total = span;
      if (sb == begin) {
        const float decay = expf(total);
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
          for (int c = 0; c < CT; ++c) acc[i][c] *= decay;
      }
      s_suffix[tid] = expf(total - (before + x));
      rest += span;
      if constexpr (NI % 4 == 0) wait_vm<NIW>(); else wait_all();  // step 0 resident
      lds_barrier();  // for every wave, with the suffixes
      // Step j: look up step j + 4 (entry slot j % 4), load step j + 2 into
      // buffer (j + 2) % 3 from entry slot (j + 2) % 4, multiply step j, then
      // wait for step j + 1's rows and step j + 3's entries.  Every step
      // issues the same loads, dummies included, so the counted wait is exact.
      for (int j = 0; j < steps; ++j) {
        lookup(ls, first(j + 4), count(j + 4), j & 3);
        stage((j + 2) % 3, first(j + 2), count(j + 2), (j + 2) & 3);
        if (owner) {
          const uint16_t* sk = s_k[j % 3];
          const uint16_t* sv = s_v[j % 3];
          float4 s0, s1;
          lds_read128x2(&s_suffix[j * kRestoreStep + 8 * lq], &s_suffix[j * kRestoreStep + 8 * lq + 4], s0, s1);
          // transpose-read address of the lane: token 8 (l / 16) + 4 hf + (l % 16) / 4,
          // columns col0 + 4 (l % 4) .. + 3
          auto tr_addr = [&](const uint16_t* buf, int ch, int hf, int col0) __attribute__((always_inline)) {
            const int t = 8 * lq + 4 * hf + (lr >> 2), col = col0 + 4 * (lr & 3);
            return buf + t * ch * 8 + 8 * swz_rows(t, col >> 3, ch) + (col & 7);
          };
          uint4 raw[CT];
          if constexpr (CT == 2) {
            tr_read16x4(tr_addr(sv, CHV, 0, wave * 32), tr_addr(sv, CHV, 1, wave * 32), tr_addr(sv, CHV, 0, wave * 32 + 16),
                        tr_addr(sv, CHV, 1, wave * 32 + 16), raw[0], raw[CT - 1]);
          } else {
#pragma unroll
            for (int c = 0; c < CT; ++c)
              raw[c] = tr_read16x2(tr_addr(sv, CHV, 0, (wave * CT + c) * 16), tr_addr(sv, CHV, 1, (wave * CT + c) * 16));
          }
          const float sf[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
          uint4 af[CT];
#pragma unroll
          for (int c = 0; c < CT; ++c) {
            float v[8];
            split2<T>(raw[c].x, v[0], v[1]);
            split2<T>(raw[c].y, v[2], v[3]);
            split2<T>(raw[c].z, v[4], v[5]);
            split2<T>(raw[c].w, v[6], v[7]);
            af[c] = make_uint4(out_pack2<T>(v[0] * sf[0], v[1] * sf[1]), out_pack2<T>(v[2] * sf[2], v[3] * sf[3]),
                               out_pack2<T>(v[4] * sf[4], v[5] * sf[5]), out_pack2<T>(v[6] * sf[6], v[7] * sf[7]));
          }
          static_assert(RT % 2 == 0, "key tiles in pairs");
#pragma unroll
          for (int i = 0; i < RT; i += 2) {
            uint4 kf0, kf1;
            tr_read16x4(tr_addr(sk, CHK, 0, 16 * i), tr_addr(sk, CHK, 1, 16 * i), tr_addr(sk, CHK, 0, 16 * i + 16),
                        tr_addr(sk, CHK, 1, 16 * i + 16), kf0, kf1);
#pragma unroll
            for (int c = 0; c < CT; ++c) acc[i][c] = RestoreMma<T>::run(af[c], kf0, acc[i][c]);  // T += V'^T K
#pragma unroll
            for (int c = 0; c < CT; ++c) acc[i + 1][c] = RestoreMma<T>::run(af[c], kf1, acc[i + 1][c]);
          }
        }
        wait_step();
        lds_barrier();  // step j + 1 and the entries of step j + 3 resident; step j's buffer consumed
      }
      wait_all();  // the dummies have landed before the buffers are reused
    }
  }
  if (!owner) return;
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

extern "C" int gdn_store_chunk_log(void* storage, const void* frames, int frames_dtype, int64_t table_rows,
                                   int64_t frames_per_slot,
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
  GDN_REQUIRE(frames_per_slot > 0 && frame_bytes > 0 && frame_bytes % 4 == 0 && num_frames > 0 && table_rows >= 0,
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
  GDN_REQUIRE(storage && frames && log_slots && token_offsets && key && gate && decay_frames,
              "gdn_store_chunk_log: null input");
  GDN_REQUIRE(T <= 0x7fffffff && HV <= 65535, "gdn_store_chunk_log: grid too large");
  LogParams p{};
  p.storage = static_cast<char*>(storage);
  p.frames = frames; p.frames_is64 = frames_dtype == GDN_I64; p.rows = table_rows;
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
                                        int64_t table_rows, int64_t num_granules, int64_t frames_per_granule,
                                        int64_t frame_bytes,
                                        int64_t num_frames, int64_t layer, const void* read_slots, int read_dtype,
                                        const void* read_granules, int read_granules_dtype,
                                        const void* write_slots, int write_dtype, const void* write_granules,
                                        int write_granules_dtype, const void* work_slots, int work_dtype,
                                        void* q_out, void* k_out, void* v_out, int64_t key_dim, int split_qkv,
                                        int round_conv, int64_t boundary0, int64_t boundary1, float scale0,
                                        float scale1, float scale2, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(batch >= 0 && channels > 0 && layer >= 0, "gdn_conv_decode_logstate: bad sizes");
  if (batch == 0) return GDN_OK;
  GDN_REQUIRE(kernel_width >= 2 && kernel_width <= 8, "gdn_conv_decode_logstate: kernel width %d not in [2, 8]",
              kernel_width);
  GDN_REQUIRE(x && weight && storage && conv_frames && read_slots && read_granules && write_slots && write_granules &&
                  work_slots && q_out,
              "gdn_conv_decode_logstate: null input");
  GDN_REQUIRE(!split_qkv || (k_out && v_out && 2 * key_dim < channels), "gdn_conv_decode_logstate: bad split");
  GDN_REQUIRE(num_granules > 0 && frames_per_granule > 0 && num_frames > 0 && frame_bytes > 0 && table_rows >= 0,
              "gdn_conv_decode_logstate: bad conv frame table");
  GDN_REQUIRE(0 <= boundary0 && boundary0 <= boundary1 && boundary1 <= channels,
              "gdn_conv_decode_logstate: bad input scale boundaries");
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
  p.rows = table_rows;
  p.granules = num_granules; p.cf = frames_per_granule; p.fe = fe; p.num_frames = num_frames; p.layer = layer;
  p.end0 = boundary0; p.end1 = boundary1; p.s0 = scale0; p.s1 = scale1; p.s2 = scale2;
  p.reads = read_slots; p.reads_is64 = read_dtype == GDN_I64;
  p.rgran = read_granules; p.rgran_is64 = read_granules_dtype == GDN_I64;
  p.writes = write_slots; p.writes_is64 = write_dtype == GDN_I64;
  p.wgran = write_granules; p.wgran_is64 = write_granules_dtype == GDN_I64;
  p.works = work_slots; p.works_is64 = work_dtype == GDN_I64;
  p.q = q_out; p.k = k_out; p.v = v_out; p.key_dim = key_dim; p.split = split_qkv; p.round_conv = round_conv;
  dim3 grid(static_cast<unsigned>((channels + kDecodeThreads - 1) / kDecodeThreads), static_cast<unsigned>(batch));
  auto s = static_cast<hipStream_t>(stream);
  // 8 channels per thread, 16-byte accesses (windows 48 contiguous bytes of one frame)
  const bool vec = kernel_width == 4 && frames_per_granule == 1 && x_col_stride == 1 && channels % 8 == 0 &&
                   x_row_stride % 8 == 0 && frame_bytes % 16 == 0 && aligned16(x) && aligned16(weight) &&
                   (bias == nullptr || aligned16(bias)) && aligned16(storage) && aligned16(q_out) &&
                   (!split_qkv || (key_dim % 8 == 0 && aligned16(k_out) && aligned16(v_out)));
  const dim3 vgrid(static_cast<unsigned>((channels / 8 + kDecodeThreads - 1) / kDecodeThreads),
                   static_cast<unsigned>(batch));
  if (dtype == GDN_BF16) {
    if (vec)
      hipLaunchKernelGGL(conv_decode_frames_vec_kernel<bf16>, vgrid, dim3(kDecodeThreads), 0, s, p);
    else
      hipLaunchKernelGGL(conv_decode_frames_kernel<bf16>, grid, dim3(kDecodeThreads), 0, s, p);
  } else if (dtype == GDN_F16) {
    if (vec)
      hipLaunchKernelGGL(conv_decode_frames_vec_kernel<f16>, vgrid, dim3(kDecodeThreads), 0, s, p);
    else
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
    int64_t table_rows, int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes, int64_t num_frames,
    const void* decay_frames,
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
                  head_bytes >= dk * row && head_bytes % 16 == 0 && aligned16(storage) && table_rows >= 0,
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
  p.frames = payload_frames; p.frames_is64 = frames_dtype == GDN_I64; p.rows = table_rows;
  p.fps = frames_per_slot; p.frame_bytes = frame_bytes; p.head_bytes = head_bytes; p.num_frames = num_frames;
  p.decay = decay_frames; p.decay_is64 = decay_dtype == GDN_I64; p.record_bytes = decay_record_bytes;
  p.work = work_slots; p.work_is64 = work_dtype == GDN_I64;
  p.logs = log_slots; p.logs_is64 = log_dtype == GDN_I64;
  p.offsets = token_offsets; p.offsets_is64 = offsets_dtype == GDN_I64;
  p.counts = replay_counts; p.counts_is64 = counts_dtype == GDN_I64;
  p.layer = layer; p.layers = num_layers; p.gran = granularity; p.page = page_size;
  p.fdiv = make_div32(frame_bytes); p.gdiv = make_div32(granularity);
  p.eager = eager; p.out = out; p.scale = scale;
  p.group = static_cast<int>(HV / H);
  // Heads per block: a block's first head waits for the whole lookup chain,
  // the later ones overlap the previous head's compute; up to 8 while the
  // grid keeps 1024 blocks (2 rounds of 2 blocks per CU), fewer for small batches.
  p.hpb = 1;
  while (p.hpb < kMaxHeadsPerBlock && HV % (2 * p.hpb) == 0 && batch * HV / (2 * p.hpb) >= 1024) p.hpb *= 2;
  const dim3 grid(static_cast<unsigned>(batch * HV / p.hpb));
  auto s = static_cast<hipStream_t>(stream);
  auto launch = [&](auto dkc, auto dvc) {
    constexpr int DK = decltype(dkc)::value, DV = decltype(dvc)::value;
    const dim3 block(DecodeShape<DK, DV>::NT);
    if (io_dtype == GDN_BF16)
      hipLaunchKernelGGL((logstate_decode_kernel<DK, DV, bf16>), grid, block, 0, s, p);
    else
      hipLaunchKernelGGL((logstate_decode_kernel<DK, DV, f16>), grid, block, 0, s, p);
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
                                         const void* conv_frames, int frames_dtype, int64_t table_rows,
                                         int64_t num_granules,
                                         int64_t frames_per_granule, int64_t frame_bytes, int64_t num_frames,
                                         int64_t layer, const void* token_slots, int slots_dtype,
                                         const void* token_granules, int granules_dtype, const void* final_slots,
                                         int finals_dtype, int64_t boundary0, int64_t boundary1, float scale0,
                                         float scale1, float scale2, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(num_seqs >= 1 && total_tokens >= 0 && channels > 0 && layer >= 0,
              "gdn_conv_windows_logstate: bad sizes");
  if (total_tokens == 0) return GDN_OK;
  GDN_REQUIRE(kernel_width >= 2 && kernel_width <= 8, "gdn_conv_windows_logstate: kernel width %d not in [2, 8]",
              kernel_width);
  GDN_REQUIRE(x && history && cu_seqlens && storage && conv_frames && token_slots && token_granules,
              "gdn_conv_windows_logstate: null input");
  GDN_REQUIRE(num_granules > 0 && frames_per_granule > 0 && num_frames > 0 && frame_bytes > 0 &&
                  frame_bytes % 2 == 0 && table_rows >= 0,
              "gdn_conv_windows_logstate: bad conv frame table");
  GDN_REQUIRE(0 <= boundary0 && boundary0 <= boundary1 && boundary1 <= channels,
              "gdn_conv_windows_logstate: bad input scale boundaries");
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
  p.storage = storage; p.table = conv_frames; p.table_is64 = frames_dtype == GDN_I64; p.rows = table_rows;
  p.granules = num_granules; p.cf = frames_per_granule; p.fe = fe; p.num_frames = num_frames; p.layer = layer;
  p.end0 = boundary0; p.end1 = boundary1; p.s0 = scale0; p.s1 = scale1; p.s2 = scale2;
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
                  int64_t table_rows, int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes, int64_t num_frames,
                  const void* decay_frames, int decay_dtype, int64_t record_bytes, int64_t layers, int64_t HV,
                  int64_t KH, int64_t dk, int64_t dv, int64_t granularity, int64_t page_size, const char* who) {
  GDN_REQUIRE(layers > 0 && HV > 0 && KH > 0 && HV % KH == 0 && granularity > 0 && page_size > 0 &&
                  page_size % granularity == 0 && table_rows >= 0,
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
  p.frames = payload_frames; p.frames_is64 = frames_dtype == GDN_I64; p.rows = table_rows;
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
                                    int64_t table_rows, int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes,
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
  int rc = restore_setup(p, storage, payload_frames, frames_dtype, table_rows, frames_per_slot, frame_bytes, head_bytes,
                         num_frames, decay_frames, decay_dtype, decay_record_bytes, num_layers, HV, key_heads, dk, dv,
                         granularity, page_size, "gdn_logstate_restore");
  if (rc != GDN_OK) return rc;
  // the kernel looks up a logged row's frames at its first and last byte
  GDN_REQUIRE(frame_bytes >= 2 * (dk > dv ? dk : dv),
              "gdn_logstate_restore: frame_bytes %lld smaller than a logged row (%lld bytes)", (long long)frame_bytes,
              (long long)(2 * (dk > dv ? dk : dv)));
  p.base = base_slots; p.offsets = segment_offsets; p.seg_slots = log_slots; p.seg_begin = log_begins;
  p.seg_end = log_ends; p.output = output_slots; p.tasks = num_tasks;
  // (task, layer, key head) groups in runs of 8, each run once per member v-head
  const int64_t groups = num_tasks * num_layers * key_heads;
  return launch_state_kernel<true>(p, (groups + 7) / 8 * 8 * (HV / key_heads), dk, dv, dtype,
                                             static_cast<hipStream_t>(stream), "gdn_logstate_restore");
}

extern "C" int gdn_logstate_copy_states(void* storage, const void* payload_frames, int frames_dtype,
                                        int64_t table_rows, int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes,
                                        int64_t num_frames, int64_t num_layers, int64_t HV, int64_t dk, int64_t dv,
                                        int dtype, const int32_t* sources, const int32_t* destinations,
                                        int64_t count, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(count >= 0, "gdn_logstate_copy_states: bad sizes");
  if (count == 0) return GDN_OK;
  GDN_REQUIRE(storage && payload_frames && sources && destinations, "gdn_logstate_copy_states: null input");
  GDN_REQUIRE(num_layers > 0 && HV > 0 && frames_per_slot > 0 && frame_bytes > 0 && num_frames > 0 &&
                  table_rows >= 0 && head_bytes >= dk * dv * 2 &&
                  (head_bytes <= frame_bytes ? frame_bytes % head_bytes == 0
                                             : head_bytes % frame_bytes == 0 && frame_bytes % (dv * 2) == 0) &&
                  num_layers * HV * head_bytes <= frames_per_slot * frame_bytes &&
                  frames_per_slot * frame_bytes < kMaxOffset32,
              "gdn_logstate_copy_states: bad frame layout");
  RestoreParams p{};
  p.storage = static_cast<char*>(storage);
  p.frames = payload_frames; p.frames_is64 = frames_dtype == GDN_I64; p.rows = table_rows;
  p.fps = frames_per_slot; p.frame_bytes = frame_bytes; p.head_bytes = head_bytes; p.num_frames = num_frames;
  p.layers = num_layers; p.HV = HV; p.KH = 1;
  p.fdiv = make_div32(frame_bytes); p.gdiv = make_div32(1);
  p.base = sources; p.output = destinations;
  return launch_state_kernel<false>(p, count * num_layers * HV, dk, dv, dtype,
                                                 static_cast<hipStream_t>(stream), "gdn_logstate_copy_states");
}
