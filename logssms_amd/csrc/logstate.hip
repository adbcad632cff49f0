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
  const int64_t fr = cf == 1 ? load_index(table, row, is64) : load_index(table, row * cf + e / fe, is64);
  if (fr < 0 || fr >= num_frames) return nullptr;
  return storage + fr * fe + (cf == 1 ? e : e % fe);
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
};

// Element (row, col) of the state of value head h in slot s: logical byte
// (layer HV + h) head_bytes + (row dv + col) elt of the slot, one frame lookup
// per row (the host checks that no row straddles two frames).
template <class T>
__device__ __forceinline__ T* state_row(const LogDecodeParams& p, int64_t s, int64_t h, int64_t row, int DV) {
  if (s < 0) return nullptr;
  const int64_t x = (p.layer * p.HV + h) * p.head_bytes + row * DV * static_cast<int64_t>(sizeof(T));
  const int64_t fr = load_index(p.frames, s * p.fps + x / p.frame_bytes, p.frames_is64);
  if (fr < 0 || fr >= p.num_frames) return nullptr;
  return reinterpret_cast<T*>(p.storage + fr * p.frame_bytes + x % p.frame_bytes);
}

// 16-bit log element (the log layout of chunk_log_kernel, key heads = H).
template <class T>
__device__ __forceinline__ T* decode_log(const LogDecodeParams& p, int64_t slot, int64_t pos, int64_t index,
                                         int64_t col, bool value, int DK, int DV) {
  const int64_t key_size = p.gran * p.H * DK;
  const int64_t layer_size = key_size + p.gran * p.HV * DV;
  const int64_t elem = (pos / p.gran * p.layers + p.layer) * layer_size + (value ? key_size : 0) +
                       (index * p.gran + pos % p.gran) * (value ? DV : DK) + col;
  const int64_t byte = 2 * elem;
  const int64_t fr = load_index(p.frames, slot * p.fps + byte / p.frame_bytes, p.frames_is64);
  if (fr < 0 || fr >= p.num_frames) return nullptr;
  return reinterpret_cast<T*>(p.storage + fr * p.frame_bytes + byte % p.frame_bytes);
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// grid (batch x HV); 256 threads hold the dk x dv state as RPT rows x 4
// columns each (columns 4 (tid % (dv / 4)) .. + 3).
template <int DK, int DV, class T>
__global__ __launch_bounds__(kDecodeThreads) void logstate_decode_kernel(LogDecodeParams p) {
  constexpr int CG = DV / 4, RG = kDecodeThreads / CG, RPT = DK / RG;
  static_assert(RPT >= 1 && DK % RG == 0, "state split");
  const int64_t b = blockIdx.x / p.HV, h = blockIdx.x % p.HV;
  const int64_t group = p.HV / p.H, kh = h / group;
  const int tid = threadIdx.x, cg = tid % CG, rg = tid / CG;
  const int c0 = 4 * cg, r0 = rg * RPT;
  __shared__ float s_q[DK], s_k[DK], s_delta[DV];
  __shared__ float s_keys[kReplayWindow][DK];
  __shared__ float s_vals[kReplayWindow][DV];
  __shared__ float s_red[2][RG][DV];
  __shared__ float s_part[4][3];
  __shared__ float s_suffix[kReplayWindow];
  __shared__ float s_scal[6];  // kq, g, decay, beta, e^{sum g}, replay count

  const int64_t w = load_index(p.work, b, p.work_is64);
  const int64_t ls = load_index(p.logs, b, p.logs_is64);
  const int64_t pos = load_index(p.offsets, b, p.offsets_is64);
  const bool in_page = ls >= 0 && pos >= 0 && pos < p.page;
  int64_t n = p.eager || !in_page ? 0 : load_index(p.counts, b, p.counts_is64);
  n = n < 0 ? 0 : (n > kReplayWindow ? kReplayWindow : n);
  n = n > pos ? pos : n;  // the logged tokens precede the position within the page
  // decay record of the log slot
  float* rec = nullptr;
  if (in_page) {
    const int64_t fr = load_index(p.decay, 2 * ls, p.decay_is64);
    const int64_t ri = load_index(p.decay, 2 * ls + 1, p.decay_is64);
    if (fr >= 0 && fr < p.num_frames && ri >= 0 && (ri + 1) * p.record_bytes <= p.frame_bytes)
      rec = reinterpret_cast<float*>(p.storage + fr * p.frame_bytes + ri * p.record_bytes);
  }
  if (!rec) n = 0;

  // ---- q, k (L2 norm), the gates
  {
    float qv = 0.f, kv = 0.f;
    if (tid < DK) {
      qv = to_f32(static_cast<const T*>(p.q)[(b * p.H + kh) * DK + tid]);
      kv = to_f32(static_cast<const T*>(p.k)[(b * p.H + kh) * DK + tid]);
    }
    const float qq = wave_sum(qv * qv), kk = wave_sum(kv * kv), qk = wave_sum(qv * kv);
    if ((tid & 63) == 0) {
      s_part[tid >> 6][0] = qq;
      s_part[tid >> 6][1] = kk;
      s_part[tid >> 6][2] = qk;
    }
    __syncthreads();
    const float sqq = s_part[0][0] + s_part[1][0] + s_part[2][0] + s_part[3][0];
    const float skk = s_part[0][1] + s_part[1][1] + s_part[2][1] + s_part[3][1];
    const float sqk = s_part[0][2] + s_part[1][2] + s_part[2][2] + s_part[3][2];
    const float rq = rsqrtf(sqq + 1e-6f) * p.scale, rk = rsqrtf(skk + 1e-6f);
    if (tid < DK) {
      s_q[tid] = qv * rq;
      s_k[tid] = kv * rk;
    }
    if (tid == 0) {
      const float a = load_any(p.A_log, h, p.a_dtype);
      const float bias = load_any(p.dt_bias, h, p.dt_dtype);
      const float gv = load_any(p.gate, b * p.gate_b + h * p.gate_h, p.gate_dtype);
      const float bv = load_any(p.beta, b * p.beta_b + h * p.beta_h, p.beta_dtype);
      const float g = -expf(a) * softplus_decode(gv + bias);
      s_scal[0] = sqk * rq * rk;
      s_scal[1] = g;
      s_scal[2] = expf(g);
      s_scal[3] = sigmoid(bv);
      // replay decays: e^{sum g} and the suffix factors e^{sum_{j > i} g_j}
      float total = 0.f;
      for (int i = 0; i < n; ++i) total += rec[(p.layer * p.page + pos - n + i) * p.HV + h];
      float prefix = 0.f;
      for (int i = 0; i < n; ++i) {
        prefix += rec[(p.layer * p.page + pos - n + i) * p.HV + h];
        s_suffix[i] = expf(total - prefix);
      }
      s_scal[4] = expf(total);
    }
    __syncthreads();
  }
  // ---- stage the replayed rows: keys, and values scaled by their suffix decay
  for (int64_t idx = tid; idx < n * DK; idx += kDecodeThreads) {
    const int64_t i = idx / DK, col = idx % DK;
    const T* e = decode_log<T>(p, ls, pos - n + i, kh, col, false, DK, DV);
    s_keys[i][col] = e ? to_f32(*e) : 0.f;
  }
  for (int64_t idx = tid; idx < n * DV; idx += kDecodeThreads) {
    const int64_t i = idx / DV, col = idx % DV;
    const T* e = decode_log<T>(p, ls, pos - n + i, h, col, true, DK, DV);
    s_vals[i][col] = e ? round_to<T>(to_f32(*e) * s_suffix[i]) : 0.f;
  }
  __syncthreads();

  // ---- the state: work slot, replayed
  float S[RPT][4];
  const float total_decay = s_scal[4];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const T* row = state_row<T>(p, w, h, r0 + r, DV);
#pragma unroll
    for (int c = 0; c < 4; ++c) S[r][c] = row ? to_f32(row[c0 + c]) * total_decay : 0.f;
  }
  for (int i = 0; i < n; ++i) {
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const float kr = s_keys[i][r0 + r];
#pragma unroll
      for (int c = 0; c < 4; ++c) S[r][c] = fmaf(kr, s_vals[i][c0 + c], S[r][c]);
    }
  }

  const float kq = s_scal[0], g = s_scal[1], decay = s_scal[2], beta = s_scal[3];
  const T* vin = static_cast<const T*>(p.v) + (b * p.HV + h) * DV;
  float out_c = 0.f;
  if (p.eager) {
    // S <- e^g S; delta = (v - S^T k) beta; S <- S + k delta^T; o = S^T q
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float acc = 0.f;
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        S[r][c] *= decay;
        acc = fmaf(S[r][c], s_k[r0 + r], acc);
      }
      s_red[0][rg][c0 + c] = acc;
    }
    __syncthreads();
    if (tid < DV) {
      float sk = 0.f;
      for (int i = 0; i < RG; ++i) sk += s_red[0][i][tid];
      s_delta[tid] = (to_f32(vin[tid]) - sk) * beta;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float acc = 0.f;
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        S[r][c] = fmaf(s_k[r0 + r], s_delta[c0 + c], S[r][c]);
        acc = fmaf(S[r][c], s_q[r0 + r], acc);
      }
      s_red[1][rg][c0 + c] = acc;
    }
    __syncthreads();
    if (tid < DV) {
      for (int i = 0; i < RG; ++i) out_c += s_red[1][i][tid];
    }
  } else {
    // delta = (v - e^g S^T k) beta; o = e^g S^T q + delta (k . q)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float ak = 0.f, aq = 0.f;
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        ak = fmaf(S[r][c], s_k[r0 + r], ak);
        aq = fmaf(S[r][c], s_q[r0 + r], aq);
      }
      s_red[0][rg][c0 + c] = ak;
      s_red[1][rg][c0 + c] = aq;
    }
    __syncthreads();
    if (tid < DV) {
      float sk = 0.f, sq = 0.f;
      for (int i = 0; i < RG; ++i) {
        sk += s_red[0][i][tid];
        sq += s_red[1][i][tid];
      }
      const float delta = (to_f32(vin[tid]) - sk * decay) * beta;
      s_delta[tid] = delta;
      out_c = sq * decay + delta * kq;
    }
    __syncthreads();
  }

  // ---- output and the step's log rows
  if (tid < DV) {
    static_cast<T*>(p.out)[(b * p.HV + h) * DV + tid] = from_f32<T>(out_c);
    if (in_page) {
      T* e = decode_log<T>(p, ls, pos, h, tid, true, DK, DV);
      if (e) *e = from_f32<T>(s_delta[tid]);
    }
  }
  if (in_page && h % group == 0 && tid < DK) {
    T* e = decode_log<T>(p, ls, pos, kh, tid, false, DK, DV);
    if (e) *e = from_f32<T>(s_k[tid]);
  }
  if (in_page && rec && tid == 0) rec[(p.layer * p.page + pos) * p.HV + h] = g;

  // ---- the work state: every step (eager), else at the end of a replay window
  if (p.eager || (pos + 1) % kReplayWindow == 0) {
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      T* row = state_row<T>(p, w, h, r0 + r, DV);
      if (!row) continue;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float val = p.eager ? S[r][c] : fmaf(s_k[r0 + r], s_delta[c0 + c], S[r][c] * decay);
        row[c0 + c] = from_f32<T>(val);
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
};

// State row of (slot, layer, head) in a frame storage (the layout of
// gdn_chunk_gated_delta_rule's frame tables), or null.
template <class T>
__device__ __forceinline__ T* slot_row(const RestoreParams& p, int64_t s, int64_t layer, int64_t h, int64_t row,
                                       int DV) {
  if (s < 0) return nullptr;
  const int64_t x = (layer * p.HV + h) * p.head_bytes + row * DV * static_cast<int64_t>(sizeof(T));
  const int64_t fr = load_index(p.frames, s * p.fps + x / p.frame_bytes, p.frames_is64);
  if (fr < 0 || fr >= p.num_frames) return nullptr;
  return reinterpret_cast<T*>(p.storage + fr * p.frame_bytes + x % p.frame_bytes);
}

template <class T>
__device__ __forceinline__ const T* restore_log(const RestoreParams& p, int64_t slot, int64_t layer, int64_t pos,
                                                int64_t index, int64_t col, bool value, int DK, int DV) {
  const int64_t key_size = p.gran * p.KH * DK;
  const int64_t layer_size = key_size + p.gran * p.HV * DV;
  const int64_t elem = (pos / p.gran * p.layers + layer) * layer_size + (value ? key_size : 0) +
                       (index * p.gran + pos % p.gran) * (value ? DV : DK) + col;
  const int64_t byte = 2 * elem;
  const int64_t fr = load_index(p.frames, slot * p.fps + byte / p.frame_bytes, p.frames_is64);
  if (fr < 0 || fr >= p.num_frames) return nullptr;
  return reinterpret_cast<const T*>(p.storage + fr * p.frame_bytes + byte % p.frame_bytes);
}

// grid (tasks x layers x HV): the state of the task's base slot (or zero),
// then each segment of logged tokens t = b .. e-1 in one step,
// S <- e^{sum_t g_t} S + sum_t k_t (e^{sum_{j>t} g_j} v'_t)^T with the scaled
// v' rounded to the state dtype (logstate_construction.cuh:329-393), taken
// 16 tokens at a time; written to the output slot.
template <int DK, int DV, class T>
__global__ __launch_bounds__(kDecodeThreads) void restore_kernel(RestoreParams p) {
  constexpr int CG = DV / 4, RG = kDecodeThreads / CG, RPT = DK / RG;
  static_assert(RPT >= 1 && DK % RG == 0, "state split");
  const int64_t task = blockIdx.x / (p.layers * p.HV);
  const int64_t layer = (blockIdx.x / p.HV) % p.layers;
  const int64_t h = blockIdx.x % p.HV;
  const int64_t kh = h / (p.HV / p.KH);
  const int tid = threadIdx.x, c0 = 4 * (tid % CG), r0 = (tid / CG) * RPT;
  __shared__ float s_keys[kReplayWindow][DK];
  __shared__ float s_vals[kReplayWindow][DV];
  __shared__ float s_suffix[kReplayWindow];
  __shared__ float s_part[kDecodeThreads / 64];
  __shared__ float s_rest;
  float S[RPT][4];
  const int64_t base = p.base[task];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const T* row = slot_row<T>(p, base, layer, h, r0 + r, DV);
#pragma unroll
    for (int c = 0; c < 4; ++c) S[r][c] = row ? to_f32(row[c0 + c]) : 0.f;
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
    __syncthreads();  // the previous segment's last group is consumed
    if ((tid & 63) == 0) s_part[tid >> 6] = part;
    if (tid == 0) s_rest = 0.f;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kDecodeThreads / 64; ++w) total += s_part[w];
    const float decay = expf(total);
#pragma unroll
    for (int r = 0; r < RPT; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) S[r][c] *= decay;
    for (int64_t t0 = begin; t0 < end; t0 += kReplayWindow) {
      const int n = static_cast<int>(end - t0 < kReplayWindow ? end - t0 : kReplayWindow);
      __syncthreads();  // the previous group's rows are consumed
      if (tid == 0) {
        // s_rest: the gates of the segment's tokens before this group
        float prefix = s_rest;
        for (int i = 0; i < n; ++i) {
          prefix += rec[(t0 + i) * p.HV];
          s_suffix[i] = expf(total - prefix);
        }
        s_rest = prefix;
      }
      for (int idx = tid; idx < n * DK; idx += kDecodeThreads) {
        const T* e = restore_log<T>(p, ls, layer, t0 + idx / DK, kh, idx % DK, false, DK, DV);
        s_keys[idx / DK][idx % DK] = e ? to_f32(*e) : 0.f;
      }
      __syncthreads();
      for (int idx = tid; idx < n * DV; idx += kDecodeThreads) {
        const T* e = restore_log<T>(p, ls, layer, t0 + idx / DV, h, idx % DV, true, DK, DV);
        s_vals[idx / DV][idx % DV] = e ? to_f32(from_f32<T>(to_f32(*e) * s_suffix[idx / DV])) : 0.f;
      }
      __syncthreads();
      for (int i = 0; i < n; ++i) {
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
          const float kr = s_keys[i][r0 + r];
#pragma unroll
          for (int c = 0; c < 4; ++c) S[r][c] = fmaf(kr, s_vals[i][c0 + c], S[r][c]);
        }
      }
    }
  }
  const int64_t out = p.output[task];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    T* row = slot_row<T>(p, out, layer, h, r0 + r, DV);
    if (!row) continue;
#pragma unroll
    for (int c = 0; c < 4; ++c) row[c0 + c] = from_f32<T>(S[r][c]);
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
  GDN_REQUIRE(frames_per_slot > 0 && frame_bytes > 0 && num_frames > 0 && frame_bytes % 8 == 0 &&
                  head_bytes >= dk * row && head_bytes % 8 == 0,
              "gdn_recurrent_logstate: bad frame layout");
  GDN_REQUIRE(head_bytes <= frame_bytes ? frame_bytes % head_bytes == 0
                                        : head_bytes % frame_bytes == 0 && frame_bytes % row == 0,
              "gdn_recurrent_logstate: head_bytes %lld must divide frame_bytes %lld, or be a multiple of it with "
              "frames holding whole state rows",
              (long long)head_bytes, (long long)frame_bytes);
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
  p.eager = eager; p.out = out; p.scale = scale;
  const dim3 grid(static_cast<unsigned>(batch * HV));
  auto s = static_cast<hipStream_t>(stream);
  auto launch = [&](auto dkc, auto dvc) {
    constexpr int DK = decltype(dkc)::value, DV = decltype(dvc)::value;
    if (io_dtype == GDN_BF16)
      hipLaunchKernelGGL((logstate_decode_kernel<DK, DV, bf16>), grid, dim3(kDecodeThreads), 0, s, p);
    else
      hipLaunchKernelGGL((logstate_decode_kernel<DK, DV, f16>), grid, dim3(kDecodeThreads), 0, s, p);
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
  GDN_REQUIRE(frames_per_slot > 0 && frame_bytes > 0 && num_frames > 0 && frame_bytes % 8 == 0 &&
                  head_bytes >= dk * row && head_bytes % 8 == 0,
              "%s: bad frame layout", who);
  GDN_REQUIRE(head_bytes <= frame_bytes ? frame_bytes % head_bytes == 0
                                        : head_bytes % frame_bytes == 0 && frame_bytes % row == 0,
              "%s: head_bytes %lld must divide frame_bytes %lld, or be a multiple of it with frames holding whole "
              "state rows",
              who, (long long)head_bytes, (long long)frame_bytes);
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
                  num_layers * HV * head_bytes <= frames_per_slot * frame_bytes,
              "gdn_logstate_copy_states: bad frame layout");
  RestoreParams p{};
  p.storage = static_cast<char*>(storage);
  p.frames = payload_frames; p.frames_is64 = frames_dtype == GDN_I64;
  p.fps = frames_per_slot; p.frame_bytes = frame_bytes; p.head_bytes = head_bytes; p.num_frames = num_frames;
  p.layers = num_layers; p.HV = HV; p.KH = 1;
  p.base = sources; p.output = destinations;
  return launch_state_kernel<false>(p, count * num_layers * HV, dk, dv, dtype,
                                                 static_cast<hipStream_t>(stream), "gdn_logstate_copy_states");
}
