// Recurrent gated delta rule: decode, spec-decode verify and the plain
// T-step recurrence, plus the single-token conv update.
//
// Roofline: HBM.  Per (sequence, v-head) the whole d_k x d_v state is read
// once and written once per launch (decode) or once per step (verify); the
// arithmetic (two column reductions and a rank-1 update) is ~6 flop/element,
// far below the CDNA4 balance point, so no MFMA is used.  The state lives in
// VGPRs for all steps of a launch, 4 consecutive columns (one 16-byte access)
// per row and lane.
//   * wave_kernel (decode and verify with the conv, gdn_fused_conv_recurrent):
//     one wave per 32 columns of a v-head, the column sums as in-wave
//     butterflies, every state load of a (sequence, key head) block issued up
//     front (see the kernel).
//   * recurrent_kernel (the standalone recurrence): thread (rg, cg) owns
//     columns 4 cg.. of rows rg, rg + RG, ..., so each load instruction of the
//     block covers RG full rows contiguously; column sums through LDS.
//
// Both column reductions (S^T k and S^T q) are taken from the decayed state
// in one pass, using o = e^g S^T q + delta (k.q) with S' = e^g S + k delta^T
// (vendor/fla/fused_recurrent.py:219-222), so the state is touched exactly
// once per step.
#include "common.hpp"

namespace gdn {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxFusedSteps = 16;
constexpr int kStepChunk = 16;

// -------------------------------------------------------------- vector I/O
template <class T> struct Vec4;
// fp32 states are stored non-temporally: a state row is not read again by
// the same launch, and streaming stores keep L2 and the MALL for the loads
// (measured: verify, which writes one state per step, runs 12 % faster).
// Decode also streams its loads (load_nt): its in-place read-modify-write
// then runs 9 % faster; verify's loads are faster cached.
template <> struct Vec4<float> {
  typedef float f4v __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ void load(const float* p, float (&v)[4]) {
    float4 x = *reinterpret_cast<const float4*>(p);
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
  }
  static __device__ __forceinline__ void load_nt(const float* p, float (&v)[4]) {
    const f4v x = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(p));
    v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[4]) {
    __builtin_nontemporal_store(f4v{v[0], v[1], v[2], v[3]}, reinterpret_cast<f4v*>(p));
  }
};
template <> struct Vec4<bf16> {
  static __device__ __forceinline__ void load_nt(const bf16* p, float (&v)[4]) { load(p, v); }
  static __device__ __forceinline__ void load(const bf16* p, float (&v)[4]) {
    uint2 x = *reinterpret_cast<const uint2*>(p);
    v[0] = __uint_as_float(x.x << 16);
    v[1] = __uint_as_float(x.x & 0xffff0000u);
    v[2] = __uint_as_float(x.y << 16);
    v[3] = __uint_as_float(x.y & 0xffff0000u);
  }
  static __device__ __forceinline__ void store(bf16* p, const float (&v)[4]) {
    uint2 x;
    x.x = static_cast<uint32_t>(f32_to_bf16_bits(v[0])) | (static_cast<uint32_t>(f32_to_bf16_bits(v[1])) << 16);
    x.y = static_cast<uint32_t>(f32_to_bf16_bits(v[2])) | (static_cast<uint32_t>(f32_to_bf16_bits(v[3])) << 16);
    *reinterpret_cast<uint2*>(p) = x;
  }
};
template <> struct Vec4<f16> {
  static __device__ __forceinline__ void load_nt(const f16* p, float (&v)[4]) { load(p, v); }
  static __device__ __forceinline__ void load(const f16* p, float (&v)[4]) {
    const f16* q = p;
    v[0] = (float)q[0]; v[1] = (float)q[1]; v[2] = (float)q[2]; v[3] = (float)q[3];
  }
  static __device__ __forceinline__ void store(f16* p, const float (&v)[4]) {
    p[0] = (f16)v[0]; p[1] = (f16)v[1]; p[2] = (f16)v[2]; p[3] = (f16)v[3];
  }
};

struct RecParams {
  // raw token inputs (unfused): q, k [B, T, H, DK], v [B, T, HV, DV]
  const void* q;
  const void* k;
  const void* v;
  // fused conv source: mixed [rows, C]
  const void* mixed;
  int64_t mixed_row_stride, mixed_col_stride;
  const void* row_index;
  int row_index_is64;
  const void* conv_w;
  const void* conv_b;
  int kernel_width;
  void* conv_state;
  int64_t conv_slot_stride, conv_layer_stride;
  int round_conv;
  // gates
  const void* gate;
  int64_t gate_b, gate_t, gate_h;
  int gate_dtype;
  const void* beta;
  int64_t beta_b, beta_t, beta_h;
  int beta_dtype;
  const void* A_log;
  int a_dtype;
  const void* dt_bias;
  int dt_dtype;
  // state
  void* state;
  int64_t slot_stride, layer_stride, head_stride, layer;
  const void* read_slots;
  int64_t read_stride;
  int read_is64;
  const void* write_slots;
  int64_t write_b, write_t;
  int write_is64;
  const void* init_state;
  void* states_out;
  // output
  void* out;
  int64_t B, T, H, HV;
  float scale;
};

// LDS carve-up for `steps` staged steps and `group` v-heads.
struct Smem {
  float* qn;     // [steps][DK]   normalised q * scale
  float* kn;     // [steps][DK]   normalised k
  float* vv;     // [steps][group][DV]
  float* kq;     // [steps]       k.q
  float* decay;  // [steps][group]
  float* beta;   // [steps][group]
  float2* red;   // [RG][DV]
  float* delta;  // [DV]
};

template <int DK, int DV>
__host__ __device__ constexpr int64_t smem_bytes(int steps, int group) {
  constexpr int CG = DV / 4;
  constexpr int RG = kThreads / CG;
  return (int64_t)4 * (steps * (2 * DK + group * DV + 1 + 2 * group) + DV) + (int64_t)8 * RG * DV;
}

template <int DK, int DV>
__device__ __forceinline__ Smem carve(char* base, int steps, int group) {
  constexpr int CG = DV / 4;
  constexpr int RG = kThreads / CG;
  Smem s;
  s.red = reinterpret_cast<float2*>(base);
  float* f = reinterpret_cast<float*>(base + 8 * RG * DV);
  s.qn = f; f += steps * DK;
  s.kn = f; f += steps * DK;
  s.vv = f; f += steps * group * DV;
  s.kq = f; f += steps;
  s.decay = f; f += steps * group;
  s.beta = f; f += steps * group;
  s.delta = f;
  return s;
}

// Normalise the staged raw q/k of `steps` steps in place and compute gates.
template <int DK>
__device__ __forceinline__ void normalise_and_gate(const RecParams& p, Smem& s, int64_t b, int t0, int steps,
                                                   int head0, int group) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int t = wave; t < steps; t += kThreads / 64) {
    float sq = 0.f, sk = 0.f;
    for (int i = lane; i < DK; i += 64) {
      const float qv = s.qn[t * DK + i], kv = s.kn[t * DK + i];
      sq += qv * qv;
      sk += kv * kv;
    }
    sq = wave_sum<64>(sq);
    sk = wave_sum<64>(sk);
    const float rq = rsqrtf(sq + 1e-6f) * p.scale;
    const float rk = rsqrtf(sk + 1e-6f);
    float kq = 0.f;
    for (int i = lane; i < DK; i += 64) {
      const float qv = s.qn[t * DK + i] * rq, kv = s.kn[t * DK + i] * rk;
      s.qn[t * DK + i] = qv;
      s.kn[t * DK + i] = kv;
      kq += qv * kv;
    }
    kq = wave_sum<64>(kq);
    if (lane == 0) s.kq[t] = kq;
  }
  for (int i = threadIdx.x; i < steps * group; i += kThreads) {
    const int t = i / group, j = i % group;
    const int64_t h = head0 + j;
    const int64_t tt = t0 + t;
    const float a = load_any(p.A_log, h, p.a_dtype);
    const float bias = load_any(p.dt_bias, h, p.dt_dtype);
    const float gv = load_any(p.gate, b * p.gate_b + tt * p.gate_t + h * p.gate_h, p.gate_dtype);
    const float bv = load_any(p.beta, b * p.beta_b + tt * p.beta_t + h * p.beta_h, p.beta_dtype);
    const float g = -expf(a) * softplus_decode(gv + bias);
    s.decay[i] = expf(g);
    s.beta[i] = sigmoid(bv);
  }
}

// Advance the register-resident state of v-head `j` over staged steps.
template <int DK, int DV, class IOT, class ST>
__device__ __forceinline__ void run_steps(const RecParams& p, Smem& s, float (&st)[DK / (kThreads / (DV / 4))][4],
                                          int64_t b, int64_t h, int j, int group, int t0, int steps, bool fused) {
  constexpr int CG = DV / 4;
  constexpr int RG = kThreads / CG;
  constexpr int RPT = DK / RG;
  const int cg = threadIdx.x % CG;
  const int rg = threadIdx.x / CG;
  for (int t = 0; t < steps; ++t) {
    const float* kn = s.kn + t * DK;
    const float* qn = s.qn + t * DK;
    float pk[4] = {0.f, 0.f, 0.f, 0.f}, pq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const float kr = kn[rg + RG * i], qr = qn[rg + RG * i];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        pk[c] = fmaf(st[i][c], kr, pk[c]);
        pq[c] = fmaf(st[i][c], qr, pq[c]);
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) s.red[rg * DV + cg * 4 + c] = make_float2(pk[c], pq[c]);
    __syncthreads();
    const float d = s.decay[t * group + j];
    if (threadIdx.x < DV) {
      const int col = threadIdx.x;
      float sk = 0.f, sq = 0.f;
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        const float2 v = s.red[r * DV + col];
        sk += v.x;
        sq += v.y;
      }
      const float delta = (s.vv[(t * group + j) * DV + col] - d * sk) * s.beta[t * group + j];
      const float o = d * sq + delta * s.kq[t];
      s.delta[col] = delta;
      int64_t orow;
      if (fused) {
        const int64_t flat = b * p.T + t0 + t;
        orow = p.row_index ? load_index(p.row_index, flat, p.row_index_is64) : flat;
      } else {
        orow = b * p.T + t0 + t;
      }
      static_cast<IOT*>(p.out)[(orow * p.HV + h) * DV + col] = from_f32<IOT>(o);
    }
    __syncthreads();
    float dl[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) dl[c] = s.delta[cg * 4 + c];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const float kr = kn[rg + RG * i];
#pragma unroll
      for (int c = 0; c < 4; ++c) st[i][c] = fmaf(kr, dl[c], d * st[i][c]);
    }
    // per-step state writes (verify / plain mode)
    ST* dst = nullptr;
    if (p.init_state) {
      dst = static_cast<ST*>(p.states_out) + (((b * p.T + t0 + t) * p.HV + h) * DK) * DV;
    } else if (p.write_t != 0) {
      const int64_t slot = load_index(p.write_slots, b * p.write_b + (t0 + t) * p.write_t, p.write_is64);
      if (slot >= 0) dst = static_cast<ST*>(p.state) + slot * p.slot_stride + p.layer * p.layer_stride + h * p.head_stride;
    }
    if (dst) {
#pragma unroll
      for (int i = 0; i < RPT; ++i) Vec4<ST>::store(dst + (rg + RG * i) * DV + cg * 4, st[i]);
    }
  }
}

template <int DK, int DV, class ST, bool kStreaming = false>
__device__ __forceinline__ void load_state(const RecParams& p, float (&st)[DK / (kThreads / (DV / 4))][4], int64_t b,
                                           int64_t h) {
  constexpr int CG = DV / 4;
  constexpr int RG = kThreads / CG;
  constexpr int RPT = DK / RG;
  const int cg = threadIdx.x % CG;
  const int rg = threadIdx.x / CG;
  const ST* src;
  if (p.init_state) {
    src = static_cast<const ST*>(p.init_state) + (b * p.HV + h) * DK * DV;
  } else {
    const int64_t slot = load_index(p.read_slots, b * p.read_stride, p.read_is64);
    src = static_cast<const ST*>(p.state) + slot * p.slot_stride + p.layer * p.layer_stride + h * p.head_stride;
  }
  if constexpr (kStreaming) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) Vec4<ST>::load_nt(src + (rg + RG * i) * DV + cg * 4, st[i]);
  } else {
#pragma unroll
    for (int i = 0; i < RPT; ++i) Vec4<ST>::load(src + (rg + RG * i) * DV + cg * 4, st[i]);
  }
}

template <int DK, int DV, class ST>
__device__ __forceinline__ void store_final(const RecParams& p, const float (&st)[DK / (kThreads / (DV / 4))][4],
                                            int64_t b, int64_t h) {
  constexpr int CG = DV / 4;
  constexpr int RG = kThreads / CG;
  constexpr int RPT = DK / RG;
  if (p.init_state || p.write_t != 0) return;  // per-step writes already done
  const int64_t slot = load_index(p.write_slots, b * p.write_b, p.write_is64);
  if (slot < 0) return;
  const int cg = threadIdx.x % CG;
  const int rg = threadIdx.x / CG;
  ST* dst = static_cast<ST*>(p.state) + slot * p.slot_stride + p.layer * p.layer_stride + h * p.head_stride;
#pragma unroll
  for (int i = 0; i < RPT; ++i) Vec4<ST>::store(dst + (rg + RG * i) * DV + cg * 4, st[i]);
}

// Unfused: one block per (sequence, v-head); q/k/v read from global memory.
template <int DK, int DV, class IOT, class ST>
__global__ __launch_bounds__(kThreads) void recurrent_kernel(RecParams p) {
  extern __shared__ __align__(16) char smem_raw[];
  constexpr int CG = DV / 4;
  constexpr int RG = kThreads / CG;
  constexpr int RPT = DK / RG;
  const int64_t b = blockIdx.x / p.HV;
  const int64_t h = blockIdx.x % p.HV;
  const int64_t kh = h / (p.HV / p.H);
  const int chunk = p.T < kStepChunk ? static_cast<int>(p.T) : kStepChunk;
  Smem s = carve<DK, DV>(smem_raw, chunk, 1);
  float st[RPT][4];
  load_state<DK, DV, ST>(p, st, b, h);
  for (int64_t t0 = 0; t0 < p.T; t0 += chunk) {
    const int steps = static_cast<int>(p.T - t0 < chunk ? p.T - t0 : chunk);
    for (int i = threadIdx.x; i < steps * DK; i += kThreads) {
      const int t = i / DK, c = i % DK;
      const int64_t base = ((b * p.T + t0 + t) * p.H + kh) * DK + c;
      s.qn[i] = to_f32(static_cast<const IOT*>(p.q)[base]);
      s.kn[i] = to_f32(static_cast<const IOT*>(p.k)[base]);
    }
    for (int i = threadIdx.x; i < steps * DV; i += kThreads) {
      const int t = i / DV, c = i % DV;
      s.vv[i] = to_f32(static_cast<const IOT*>(p.v)[((b * p.T + t0 + t) * p.HV + h) * DV + c]);
    }
    __syncthreads();
    normalise_and_gate<DK>(p, s, b, static_cast<int>(t0), steps, static_cast<int>(h), 1);
    __syncthreads();
    run_steps<DK, DV, IOT, ST>(p, s, st, b, h, 0, 1, static_cast<int>(t0), steps, false);
    __syncthreads();
  }
  store_final<DK, DV, ST>(p, st, b, h);
}

// Conv of one key head's group of channels (q and k of key head kh, v of its
// `group` v-heads) over `steps` tokens, one channel per thread tid, tid +
// nthreads, ... (conv_decode.py:25-289 per step): raw q, k into s.qn / s.kn,
// v into s.vv, and each step's shifted window to that step's write slot.  A
// negative read slot is a zero history.
template <int DK, int DV, class IOT>
__device__ __forceinline__ void conv_group(const RecParams& p, Smem& s, int64_t b, int64_t kh, int group, int steps,
                                           int tid, int nthreads) {
  const int64_t key_dim = p.H * DK;
  const int nch = 2 * DK + group * DV;
  const int W = p.kernel_width;
  const int64_t read_slot = load_index(p.read_slots, b * p.read_stride, p.read_is64);
  for (int c = tid; c < nch; c += nthreads) {
    int64_t ch;
    float* dst;
    int dst_stride;
    if (c < DK) {
      ch = kh * DK + c;
      dst = s.qn + c;
      dst_stride = DK;
    } else if (c < 2 * DK) {
      ch = key_dim + kh * DK + (c - DK);
      dst = s.kn + (c - DK);
      dst_stride = DK;
    } else {
      const int vc = c - 2 * DK;  // = j * DV + col
      ch = 2 * key_dim + kh * group * DV + vc;
      dst = s.vv + vc;
      dst_stride = group * DV;
    }
    float win[8];
    float w[9];
    const IOT* cs = static_cast<const IOT*>(p.conv_state) + (read_slot >= 0 ? read_slot : 0) * p.conv_slot_stride +
                    p.layer * p.conv_layer_stride + ch * (W - 1);
    for (int i = 0; i < W - 1; ++i) win[i] = read_slot >= 0 ? to_f32(cs[i]) : 0.f;
    for (int i = 0; i < W; ++i) w[i] = to_f32(static_cast<const IOT*>(p.conv_w)[ch * W + i]);
    const float bias = p.conv_b ? to_f32(static_cast<const IOT*>(p.conv_b)[ch]) : 0.f;
    for (int t = 0; t < steps; ++t) {
      const int64_t flat = b * p.T + t;
      const int64_t row = p.row_index ? load_index(p.row_index, flat, p.row_index_is64) : flat;
      const float x = to_f32(static_cast<const IOT*>(p.mixed)[row * p.mixed_row_stride + ch * p.mixed_col_stride]);
      float acc = 0.f;
      for (int i = 0; i < W - 1; ++i) acc = fmaf(w[i], win[i], acc);
      acc = fmaf(w[W - 1], x, acc);
      acc += bias;
      if (p.round_conv) acc = round_to<IOT>(acc);
      dst[t * dst_stride] = round_to<IOT>(silu(acc));
      for (int i = 0; i + 1 < W - 1; ++i) win[i] = win[i + 1];
      win[W - 2] = x;
      const int64_t ws = load_index(p.write_slots, b * p.write_b + t * p.write_t, p.write_is64);
      if (ws >= 0) {
        IOT* out = static_cast<IOT*>(p.conv_state) + ws * p.conv_slot_stride + p.layer * p.conv_layer_stride +
                   ch * (W - 1);
        for (int i = 0; i < W - 1; ++i) out[i] = from_f32<IOT>(win[i]);
      }
    }
  }
}

// The q / k L2 norms and k.q of each staged token, and the gates of each
// (token, v-head) (fused_recurrent.py:202-215; gate/beta rows follow the
// token rows: (row, head) strides).
// with_gates false: the caller has written s.decay / s.beta itself.
template <int DK>
__device__ __forceinline__ void norm_group(const RecParams& p, Smem& s, int64_t b, int64_t kh, int group, int steps,
                                           int tid, int nthreads, bool with_gates = true) {
  // gate/beta rows follow the token rows: (row, head) strides
  {
    const int lane = tid & 63;
    const int wave = tid >> 6;
    for (int t = wave; t < steps; t += nthreads / 64) {
      float sq = 0.f, sk = 0.f;
      for (int i = lane; i < DK; i += 64) {
        const float qv = s.qn[t * DK + i], kv = s.kn[t * DK + i];
        sq += qv * qv;
        sk += kv * kv;
      }
      sq = wave_sum<64>(sq);
      sk = wave_sum<64>(sk);
      const float rq = rsqrtf(sq + 1e-6f) * p.scale;
      const float rk = rsqrtf(sk + 1e-6f);
      float kq = 0.f;
      for (int i = lane; i < DK; i += 64) {
        const float qv = s.qn[t * DK + i] * rq, kv = s.kn[t * DK + i] * rk;
        s.qn[t * DK + i] = qv;
        s.kn[t * DK + i] = kv;
        kq += qv * kv;
      }
      kq = wave_sum<64>(kq);
      if (lane == 0) s.kq[t] = kq;
    }
    for (int i = tid; with_gates && i < steps * group; i += nthreads) {
      const int t = i / group, j = i % group;
      const int64_t h = kh * group + j;
      const int64_t flat = b * p.T + t;
      const int64_t row = p.row_index ? load_index(p.row_index, flat, p.row_index_is64) : flat;
      const float a = load_any(p.A_log, h, p.a_dtype);
      const float bias = load_any(p.dt_bias, h, p.dt_dtype);
      const float gv = load_any(p.gate, row * p.gate_t + h * p.gate_h, p.gate_dtype);
      const float bv = load_any(p.beta, row * p.beta_t + h * p.beta_h, p.beta_dtype);
      const float g = -expf(a) * softplus_decode(gv + bias);
      s.decay[i] = expf(g);
      s.beta[i] = sigmoid(bv);
    }
  }
}

// Three zero elements of any io type: the conv history of a negative read slot.
__device__ const uint32_t kZeroWindow[4] = {0u, 0u, 0u, 0u};

// Block-uniform index read through the scalar data cache (waited on with the
// LDS / scalar counter, never behind the block's vector loads).
__device__ __forceinline__ int64_t scalar_index(const void* p, int64_t i, int is64) {
  typedef __attribute__((address_space(4))) const int32_t ci32;
  return static_cast<int64_t>(reinterpret_cast<ci32*>(reinterpret_cast<uintptr_t>(p))[is64 ? 2 * i : i]);
}

// The bits of one io element (zero-extended 16-bit or 32-bit) and its value.
// (read through a global address-space pointer, so the load is a global load
// that the waits count exactly, whatever the pointer's origin)
template <class T> __device__ __forceinline__ uint32_t raw_bits(const T* p) {
  typedef __attribute__((address_space(1))) const uint16_t g16;
  typedef __attribute__((address_space(1))) const uint32_t g32;
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  if constexpr (sizeof(T) == 2) return *reinterpret_cast<g16*>(a);
  else return *reinterpret_cast<g32*>(a);
}
// Element i of a runtime-typed float array (bf16, f16, else fp32) as two
// 16-bit loads whose address is chosen by arithmetic, not by a branch (an fp32
// element as its two halves, a 16-bit one read twice), so that the loads issue
// back to back and their waits are counted; float_of_halves gives the value.
__device__ __forceinline__ void load_halves(const void* base, int64_t i, int dtype, uint32_t (&r)[2]) {
  const bool wide = dtype != GDN_BF16 && dtype != GDN_F16;
  const uint16_t* a = reinterpret_cast<const uint16_t*>(static_cast<const char*>(base) + i * (wide ? 4 : 2));
  r[0] = raw_bits(a);
  r[1] = raw_bits(a + (wide ? 1 : 0));
}
__device__ __forceinline__ float float_of_halves(const uint32_t (&r)[2], int dtype) {
  if (dtype == GDN_BF16) return __uint_as_float(r[0] << 16);
  if (dtype == GDN_F16) return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r[0])));
  return __uint_as_float(r[0] | (r[1] << 16));
}
template <class T> __device__ __forceinline__ float f32_from_bits(uint32_t r);
template <> __device__ __forceinline__ float f32_from_bits<bf16>(uint32_t r) { return __uint_as_float(r << 16); }
template <> __device__ __forceinline__ float f32_from_bits<f16>(uint32_t r) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r)));
}
template <> __device__ __forceinline__ float f32_from_bits<float>(uint32_t r) { return __uint_as_float(r); }

// Decode and verify with one wave per 32 state columns of a v-head (d_v a
// multiple of 32, d_k in {32, 64, 128}): one block per (sequence, key head)
// of group * d_v / 32 waves.  Lane (rg = lane / 8, cg = lane % 8) of a wave
// holds state columns 4 cg .. 4 cg + 3 of its 32 and rows rg RPT .. rg RPT +
// RPT - 1 (RPT = d_k / 8), moved as RPT 16-byte pieces (each load or store
// instruction of a wave covers 8 rows of 128 contiguous bytes).  Every wave
// issues its state loads before the conv phase, so all of the group's states
// are in flight while the conv runs; a step's column sums (S^T k, S^T q) are
// butterflies over the wave's 8 row groups (lanes xor 8, 16, 32), with no LDS
// round trip and no block barrier.  A negative read slot is a zero state, a
// negative write slot takes no write.
template <int DK, int DV, class IOT, class ST, bool kStream, bool kEarlyConv>
__global__ __launch_bounds__(1024) void wave_kernel(RecParams p) {
  extern __shared__ __align__(16) char smem_raw[];
  constexpr int WPH = DV / 32;  // waves per v-head
  constexpr int RPT = DK / 8;   // state rows per lane
  static_assert(DV % 32 == 0 && RPT % 4 == 0, "d_v % 32 == 0, d_k in {32, 64, 128}");
  const int group = static_cast<int>(p.HV / p.H);
  const int steps = static_cast<int>(p.T);
  const int64_t b = blockIdx.x / p.H;
  const int64_t kh = blockIdx.x % p.H;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, rg = lane >> 3, cg = lane & 7;
  const int j = wave / WPH;  // v-head of the group
  const int64_t h = kh * group + j;
  const int c0 = (wave % WPH) * 32 + 4 * cg;  // first state column of the lane
  const int r0 = rg * RPT;                    // first state row of the lane
  Smem s = carve<DK, DV>(smem_raw, steps, group);
  ST* const pool = static_cast<ST*>(p.state);
  const int64_t head_off = p.layer * p.layer_stride + h * p.head_stride + static_cast<int64_t>(r0) * DV + c0;
  const int64_t rs = scalar_index(p.read_slots, b * p.read_stride, p.read_is64);
  // kEarlyConv (decode with conv width 4 and at most one channel per thread,
  // chosen by the host): the conv inputs are requested (as raw bits,
  // branch-free, idle threads reading a clamped channel) before the state, and
  // unpacked after it, so the conv waits for them alone (a wave's loads return
  // in order) while the state arrives.
  const int nch = 2 * DK + group * DV;
  constexpr bool early_conv = kEarlyConv;
  const int c = threadIdx.x < nch ? static_cast<int>(threadIdx.x) : nch - 1;
  const int64_t key_dim = p.H * DK;
  const int64_t ch = c < DK ? kh * DK + c
                            : (c < 2 * DK ? key_dim + kh * DK + (c - DK) : 2 * key_dim + kh * group * DV + (c - 2 * DK));
  float* const cdst = c < DK ? s.qn + c : (c < 2 * DK ? s.kn + (c - DK) : s.vv + (c - 2 * DK));
  uint32_t rwin[3] = {0u, 0u, 0u}, rw[4] = {0u, 0u, 0u, 0u}, rx = 0u, rb = 0u;
  // (early path, one step) the gate inputs of v-head threadIdx.x of the group,
  // requested with the conv inputs: A_log, dt_bias, gate, beta
  uint32_t rg4[4][2] = {{0u, 0u}, {0u, 0u}, {0u, 0u}, {0u, 0u}};
  if (early_conv) {
    // a negative read slot reads its (zero) history from a zero array: no select on loaded data
    const IOT* ccs = rs >= 0 ? static_cast<const IOT*>(p.conv_state) + rs * p.conv_slot_stride +
                                   p.layer * p.conv_layer_stride + ch * 3
                             : reinterpret_cast<const IOT*>(kZeroWindow);
    const int64_t row = p.row_index ? scalar_index(p.row_index, b, p.row_index_is64) : b;
    const IOT* wts = static_cast<const IOT*>(p.conv_w) + ch * 4;
#pragma unroll
    for (int i = 0; i < 3; ++i) rwin[i] = raw_bits(ccs + i);
#pragma unroll
    for (int i = 0; i < 4; ++i) rw[i] = raw_bits(wts + i);
    rx = raw_bits(static_cast<const IOT*>(p.mixed) + row * p.mixed_row_stride + ch * p.mixed_col_stride);
    rb = raw_bits(p.conv_b ? static_cast<const IOT*>(p.conv_b) + ch : wts);  // no branch: a bias-less read is unused
    const int64_t hg = kh * group + (static_cast<int>(threadIdx.x) < group ? static_cast<int>(threadIdx.x) : 0);
    load_halves(p.A_log, hg, p.a_dtype, rg4[0]);
    load_halves(p.dt_bias, hg, p.dt_dtype, rg4[1]);
    load_halves(p.gate, row * p.gate_t + hg * p.gate_h, p.gate_dtype, rg4[2]);
    load_halves(p.beta, row * p.beta_t + hg * p.beta_h, p.beta_dtype, rg4[3]);
  }
  float st[RPT][4];
  {
    const ST* src = pool + (rs >= 0 ? rs : 0) * p.slot_stride + head_off;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      if constexpr (kStream) Vec4<ST>::load_nt(src + i * DV, st[i]);
      else Vec4<ST>::load(src + i * DV, st[i]);
    }
  }
  if (early_conv) {  // conv_decode.py:25-289 for one token, as conv_group computes it
    float win[3], acc = 0.f;
#pragma unroll
    for (int i = 0; i < 3; ++i) win[i] = f32_from_bits<IOT>(rwin[i]);
#pragma unroll
    for (int i = 0; i < 3; ++i) acc = fmaf(f32_from_bits<IOT>(rw[i]), win[i], acc);
    const float x = f32_from_bits<IOT>(rx);
    acc = fmaf(f32_from_bits<IOT>(rw[3]), x, acc);
    acc += p.conv_b ? f32_from_bits<IOT>(rb) : 0.f;
    if (p.round_conv) acc = round_to<IOT>(acc);
    if (static_cast<int>(threadIdx.x) < nch) {
      *cdst = round_to<IOT>(silu(acc));
      const int64_t ws = load_index(p.write_slots, b * p.write_b, p.write_is64);
      if (ws >= 0) {
        IOT* out = static_cast<IOT*>(p.conv_state) + ws * p.conv_slot_stride + p.layer * p.conv_layer_stride + ch * 3;
        out[0] = from_f32<IOT>(win[1]);
        out[1] = from_f32<IOT>(win[2]);
        out[2] = from_f32<IOT>(x);
      }
    }
    if (static_cast<int>(threadIdx.x) < group) {  // fused_recurrent.py:202-215, as norm_group computes it
      const float a = float_of_halves(rg4[0], p.a_dtype), bias = float_of_halves(rg4[1], p.dt_dtype);
      const float gv = float_of_halves(rg4[2], p.gate_dtype), bv = float_of_halves(rg4[3], p.beta_dtype);
      const float g = -expf(a) * softplus_decode(gv + bias);
      s.decay[threadIdx.x] = expf(g);
      s.beta[threadIdx.x] = sigmoid(bv);
    }
  } else {
    conv_group<DK, DV, IOT>(p, s, b, kh, group, steps, threadIdx.x, blockDim.x);
  }
  __syncthreads();
  norm_group<DK>(p, s, b, kh, group, steps, threadIdx.x, blockDim.x, !early_conv);
  __syncthreads();
  if (rs < 0) {
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
      for (int c = 0; c < 4; ++c) st[i][c] = 0.f;
  }
  auto store_state = [&](int64_t slot) __attribute__((always_inline)) {
    ST* dst = pool + slot * p.slot_stride + head_off;
#pragma unroll
    for (int i = 0; i < RPT; ++i) Vec4<ST>::store(dst + i * DV, st[i]);
  };
  for (int t = 0; t < steps; ++t) {
    const float* kn = s.kn + t * DK + r0;
    const float* qn = s.qn + t * DK + r0;
    float pk[4] = {0.f, 0.f, 0.f, 0.f}, pq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < RPT; i += 4) {
      const float4 k4 = *reinterpret_cast<const float4*>(kn + i);
      const float4 q4 = *reinterpret_cast<const float4*>(qn + i);
      const float kr[4] = {k4.x, k4.y, k4.z, k4.w}, qr[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          pk[c] = fmaf(st[i + u][c], kr[u], pk[c]);
          pq[c] = fmaf(st[i + u][c], qr[u], pq[c]);
        }
    }
#pragma unroll
    for (int m = 8; m < 64; m <<= 1)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        pk[c] += __shfl_xor(pk[c], m);
        pq[c] += __shfl_xor(pq[c], m);
      }
    const float d = s.decay[t * group + j], bt = s.beta[t * group + j], kq = s.kq[t];
    const float4 v4 = *reinterpret_cast<const float4*>(s.vv + (t * group + j) * DV + c0);
    const float vr[4] = {v4.x, v4.y, v4.z, v4.w};
    float dl[4], o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      dl[c] = (vr[c] - d * pk[c]) * bt;
      o[c] = d * pq[c] + dl[c] * kq;
    }
    if (rg == 0) {
      const int64_t flat = b * p.T + t;
      const int64_t orow = p.row_index ? load_index(p.row_index, flat, p.row_index_is64) : flat;
      Vec4<IOT>::store(static_cast<IOT*>(p.out) + (orow * p.HV + h) * DV + c0, o);
    }
#pragma unroll
    for (int i = 0; i < RPT; i += 4) {
      const float4 k4 = *reinterpret_cast<const float4*>(kn + i);
      const float kr[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int c = 0; c < 4; ++c) st[i + u][c] = fmaf(kr[u], dl[c], d * st[i + u][c]);
    }
    if (p.write_t != 0) {  // verify: every step's state to its slot
      const int64_t slot = load_index(p.write_slots, b * p.write_b + t * p.write_t, p.write_is64);
      if (slot >= 0) store_state(slot);
    }
  }
  if (p.write_t == 0) {  // decode: the final state
    const int64_t slot = load_index(p.write_slots, b * p.write_b, p.write_is64);
    if (slot >= 0) store_state(slot);
  }
}

// Single-token conv update (conv_decode.py:25-289, standard state).
template <class IOT>
__global__ __launch_bounds__(kThreads) void conv_decode_kernel(
    const IOT* x, int64_t xr, int64_t xc, const IOT* weight, const IOT* bias, int W, int64_t C, IOT* state,
    int64_t slot_stride, int64_t layer_stride, int64_t layer, const void* reads, int64_t read_stride,
    int read_is64, const void* writes, int64_t write_stride, int write_is64, IOT* q, IOT* k, IOT* v,
    int64_t key_dim, int split, int round_conv, int64_t end0, int64_t end1, float s0, float s1, float s2) {
  const int64_t b = blockIdx.y;
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (ch >= C) return;
  const int64_t rs = load_index(reads, b * read_stride, read_is64);
  const int64_t ws = load_index(writes, b * write_stride, write_is64);
  float win[8];
  if (rs >= 0) {  // a negative read slot is a zero history
    const IOT* src = state + rs * slot_stride + layer * layer_stride + ch * (W - 1);
    for (int i = 0; i < W - 1; ++i) win[i] = to_f32(src[i]);
  } else {
    for (int i = 0; i < W - 1; ++i) win[i] = 0.f;
  }
  float xv = to_f32(x[b * xr + ch * xc]);
  if (s0 != 1.f || s1 != 1.f || s2 != 1.f) {
    const float sc = ch < end0 ? s0 : (ch < end1 ? s1 : s2);
    xv = round_to<IOT>(xv * sc);
  }
  float acc = 0.f;
  for (int i = 0; i < W - 1; ++i) acc = fmaf(to_f32(weight[ch * W + i]), win[i], acc);
  acc = fmaf(to_f32(weight[ch * W + W - 1]), xv, acc);
  if (bias) acc += to_f32(bias[ch]);
  if (round_conv) acc = round_to<IOT>(acc);
  const IOT y = from_f32<IOT>(silu(acc));
  if (ws >= 0) {  // a negative write slot takes no write
    IOT* dst = state + ws * slot_stride + layer * layer_stride + ch * (W - 1);
    for (int i = 0; i + 1 < W - 1; ++i) dst[i] = from_f32<IOT>(win[i + 1]);
    dst[W - 2] = from_f32<IOT>(xv);
  }
  if (!split) {
    q[b * C + ch] = y;
  } else if (ch < key_dim) {
    q[b * key_dim + ch] = y;
  } else if (ch < 2 * key_dim) {
    k[b * key_dim + ch - key_dim] = y;
  } else {
    v[b * (C - 2 * key_dim) + ch - 2 * key_dim] = y;
  }
}

// ------------------------------------------------------------------ dispatch
template <class F>
int dispatch_dims(int64_t dk, int64_t dv, F&& f) {
  if (dk == 128 && dv == 128) return f(std::integral_constant<int, 128>{}, std::integral_constant<int, 128>{});
  if (dk == 64 && dv == 64) return f(std::integral_constant<int, 64>{}, std::integral_constant<int, 64>{});
  if (dk == 32 && dv == 32) return f(std::integral_constant<int, 32>{}, std::integral_constant<int, 32>{});
  if (dk == 128 && dv == 64) return f(std::integral_constant<int, 128>{}, std::integral_constant<int, 64>{});
  if (dk == 64 && dv == 128) return f(std::integral_constant<int, 64>{}, std::integral_constant<int, 128>{});
  set_error("unsupported head dims dk=%lld dv=%lld (supported: 32/32, 64/64, 128/128, 64/128, 128/64)",
            (long long)dk, (long long)dv);
  return GDN_ERR_UNSUPPORTED;
}

template <class F>
int dispatch_io_state(int io, int st, F&& f) {
  if (io == GDN_BF16 && st == GDN_F32) return f(bf16{}, float{});
  if (io == GDN_BF16 && st == GDN_BF16) return f(bf16{}, bf16{});
  if (io == GDN_F16 && st == GDN_F32) return f(f16{}, float{});
  if (io == GDN_F16 && st == GDN_F16) return f(f16{}, f16{});
  if (io == GDN_F32 && st == GDN_F32) return f(float{}, float{});
  set_error("unsupported (io dtype %d, state dtype %d)", io, st);
  return GDN_ERR_UNSUPPORTED;
}

}  // namespace
}  // namespace gdn

using namespace gdn;

extern "C" int gdn_fused_recurrent(const void* q, const void* k, const void* v, int io_dtype, const void* gate,
                                   int64_t gate_b_stride, int64_t gate_t_stride, int64_t gate_h_stride,
                                   int gate_dtype, const void* beta, int64_t beta_b_stride, int64_t beta_t_stride,
                                   int64_t beta_h_stride, int beta_dtype, const void* A_log, int a_dtype,
                                   const void* dt_bias, int dt_dtype, int64_t batch, int64_t steps, int64_t H,
                                   int64_t HV, int64_t dk, int64_t dv, void* state, int state_dtype,
                                   int64_t slot_stride, int64_t layer_stride, int64_t head_stride, int64_t layer,
                                   const void* read_slots, int64_t read_stride, int read_dtype,
                                   const void* write_slots, int64_t write_b_stride, int64_t write_t_stride,
                                   int write_dtype, const void* init_state, void* states_out, void* out,
                                   float scale, void* stream) {
  GDN_REQUIRE(batch >= 0 && steps >= 0 && H > 0 && HV > 0 && HV % H == 0, "gdn_fused_recurrent: bad sizes");
  if (batch == 0 || steps == 0) return GDN_OK;
  GDN_REQUIRE(q && k && v && gate && beta && A_log && dt_bias && out, "gdn_fused_recurrent: null input");
  if (init_state) {
    GDN_REQUIRE(states_out != nullptr, "gdn_fused_recurrent: plain mode needs states_out");
  } else {
    GDN_REQUIRE(state && read_slots && write_slots, "gdn_fused_recurrent: slot mode needs pool and slots");
  }
  GDN_REQUIRE(batch * HV <= 0x7fffffff, "gdn_fused_recurrent: grid too large");
  RecParams p{};
  p.q = q; p.k = k; p.v = v;
  p.gate = gate; p.gate_b = gate_b_stride; p.gate_t = gate_t_stride; p.gate_h = gate_h_stride; p.gate_dtype = gate_dtype;
  p.beta = beta; p.beta_b = beta_b_stride; p.beta_t = beta_t_stride; p.beta_h = beta_h_stride; p.beta_dtype = beta_dtype;
  p.A_log = A_log; p.a_dtype = a_dtype; p.dt_bias = dt_bias; p.dt_dtype = dt_dtype;
  p.state = state; p.slot_stride = slot_stride; p.layer_stride = layer_stride; p.head_stride = head_stride;
  p.layer = layer;
  p.read_slots = read_slots; p.read_stride = read_stride; p.read_is64 = read_dtype == GDN_I64;
  p.write_slots = write_slots; p.write_b = write_b_stride; p.write_t = write_t_stride;
  p.write_is64 = write_dtype == GDN_I64;
  p.init_state = init_state; p.states_out = states_out;
  p.out = out; p.B = batch; p.T = steps; p.H = H; p.HV = HV; p.scale = scale;
  return dispatch_dims(dk, dv, [&](auto DKc, auto DVc) {
    constexpr int DK = decltype(DKc)::value, DV = decltype(DVc)::value;
    return dispatch_io_state(io_dtype, state_dtype, [&](auto iot, auto stt) {
      using IOT = decltype(iot);
      using ST = decltype(stt);
      const int chunk = steps < kStepChunk ? static_cast<int>(steps) : kStepChunk;
      const size_t shm = smem_bytes<DK, DV>(chunk, 1);
      hipLaunchKernelGGL((recurrent_kernel<DK, DV, IOT, ST>), dim3(static_cast<unsigned>(batch * HV)),
                         dim3(kThreads), shm, static_cast<hipStream_t>(stream), p);
      return GDN_LAUNCH_CHECK("gdn_fused_recurrent launch");
    });
  });
}

extern "C" int gdn_fused_conv_recurrent(const void* mixed, int64_t row_stride, int64_t col_stride, int dtype,
                                        const void* row_index, int row_index_dtype, const void* weight,
                                        const void* bias, int kernel_width, const void* gate,
                                        int64_t gate_row_stride, int64_t gate_head_stride, int gate_dtype,
                                        const void* beta, int64_t beta_row_stride, int64_t beta_head_stride,
                                        int beta_dtype, const void* A_log, int a_dtype, const void* dt_bias,
                                        int dt_dtype, int64_t batch, int64_t steps, int64_t H, int64_t HV,
                                        int64_t dk, int64_t dv, void* conv_state, int64_t conv_slot_stride,
                                        int64_t conv_layer_stride, void* state, int state_dtype,
                                        int64_t slot_stride, int64_t layer_stride, int64_t head_stride,
                                        int64_t layer, const void* read_slots, int64_t read_stride,
                                        int read_dtype, const void* write_slots, int64_t write_b_stride,
                                        int64_t write_t_stride, int write_dtype, void* out, float scale,
                                        void* stream) {
  GDN_REQUIRE(batch >= 0 && steps >= 0 && H > 0 && HV > 0 && HV % H == 0, "gdn_fused_conv_recurrent: bad sizes");
  if (batch == 0 || steps == 0) return GDN_OK;
  GDN_REQUIRE(steps <= kMaxFusedSteps, "gdn_fused_conv_recurrent: steps %lld > %d", (long long)steps,
              kMaxFusedSteps);
  GDN_REQUIRE(kernel_width >= 2 && kernel_width <= 8, "gdn_fused_conv_recurrent: kernel width %d not in [2, 8]",
              kernel_width);
  GDN_REQUIRE(mixed && weight && gate && beta && A_log && dt_bias && conv_state && state && read_slots &&
                  write_slots && out,
              "gdn_fused_conv_recurrent: null input");
  GDN_REQUIRE(HV / H <= 4, "gdn_fused_conv_recurrent: at most 4 v-heads per key head");
  GDN_REQUIRE(steps == 1 || write_t_stride != 0, "gdn_fused_conv_recurrent: multi-step needs per-step slots");
  GDN_REQUIRE(batch * H <= 0x7fffffff, "gdn_fused_conv_recurrent: grid too large");
  RecParams p{};
  p.mixed = mixed; p.mixed_row_stride = row_stride; p.mixed_col_stride = col_stride;
  p.row_index = row_index; p.row_index_is64 = row_index_dtype == GDN_I64;
  p.conv_w = weight; p.conv_b = bias; p.kernel_width = kernel_width;
  p.conv_state = conv_state; p.conv_slot_stride = conv_slot_stride; p.conv_layer_stride = conv_layer_stride;
  p.round_conv = write_t_stride != 0 ? 1 : 0;
  p.gate = gate; p.gate_b = 0; p.gate_t = gate_row_stride; p.gate_h = gate_head_stride; p.gate_dtype = gate_dtype;
  p.beta = beta; p.beta_b = 0; p.beta_t = beta_row_stride; p.beta_h = beta_head_stride; p.beta_dtype = beta_dtype;
  p.A_log = A_log; p.a_dtype = a_dtype; p.dt_bias = dt_bias; p.dt_dtype = dt_dtype;
  p.state = state; p.slot_stride = slot_stride; p.layer_stride = layer_stride; p.head_stride = head_stride;
  p.layer = layer;
  p.read_slots = read_slots; p.read_stride = read_stride; p.read_is64 = read_dtype == GDN_I64;
  p.write_slots = write_slots; p.write_b = write_b_stride; p.write_t = write_t_stride;
  p.write_is64 = write_dtype == GDN_I64;
  p.out = out; p.B = batch; p.T = steps; p.H = H; p.HV = HV; p.scale = scale;
  return dispatch_dims(dk, dv, [&](auto DKc, auto DVc) {
    constexpr int DK = decltype(DKc)::value, DV = decltype(DVc)::value;
    return dispatch_io_state(dtype, state_dtype, [&](auto iot, auto stt) {
      using IOT = decltype(iot);
      using ST = decltype(stt);
      const size_t shm = smem_bytes<DK, DV>(static_cast<int>(steps), static_cast<int>(HV / H));
      const dim3 grid(static_cast<unsigned>(batch * H));
      auto s = static_cast<hipStream_t>(stream);
      const unsigned waves = static_cast<unsigned>((HV / H) * (DV / 32));
      // decode: streaming state loads, and the conv inputs fetched before the state
      // when the conv has width 4 and at most one channel per thread
      const bool early = kernel_width == 4 && 2 * DK + (HV / H) * DV <= 64 * static_cast<int64_t>(waves);
      if (steps == 1 && early)
        hipLaunchKernelGGL((wave_kernel<DK, DV, IOT, ST, true, true>), grid, dim3(64 * waves), shm, s, p);
      else if (steps == 1)
        hipLaunchKernelGGL((wave_kernel<DK, DV, IOT, ST, true, false>), grid, dim3(64 * waves), shm, s, p);
      else
        hipLaunchKernelGGL((wave_kernel<DK, DV, IOT, ST, false, false>), grid, dim3(64 * waves), shm, s, p);
      return GDN_LAUNCH_CHECK("gdn_fused_conv_recurrent launch");
    });
  });
}

extern "C" int gdn_conv_decode(const void* x, int64_t x_row_stride, int64_t x_col_stride, int dtype,
                               const void* weight, const void* bias, int kernel_width, int64_t batch,
                               int64_t channels, void* conv_state, int64_t state_slot_stride,
                               int64_t state_layer_stride, int64_t layer, const void* read_slots,
                               int64_t read_stride, int read_dtype, const void* write_slots, int64_t write_stride,
                               int write_dtype, void* q_out, void* k_out, void* v_out, int64_t key_dim,
                               int split_qkv, int round_conv, int64_t boundary0, int64_t boundary1, float scale0,
                               float scale1, float scale2, void* stream) {
  GDN_REQUIRE(batch >= 0 && channels > 0, "gdn_conv_decode: bad sizes");
  if (batch == 0) return GDN_OK;
  GDN_REQUIRE(kernel_width >= 2 && kernel_width <= 8, "gdn_conv_decode: kernel width %d not in [2, 8]",
              kernel_width);
  GDN_REQUIRE(x && weight && conv_state && read_slots && write_slots && q_out, "gdn_conv_decode: null input");
  GDN_REQUIRE(!split_qkv || (k_out && v_out && 2 * key_dim < channels), "gdn_conv_decode: bad split");
  GDN_REQUIRE(batch <= 65535, "gdn_conv_decode: batch too large");
  dim3 grid(static_cast<unsigned>((channels + kThreads - 1) / kThreads), static_cast<unsigned>(batch));
  auto s = static_cast<hipStream_t>(stream);
  auto launch = [&](auto tag) {
    using T = decltype(tag);
    hipLaunchKernelGGL((conv_decode_kernel<T>), grid, dim3(kThreads), 0, s, static_cast<const T*>(x), x_row_stride,
                       x_col_stride, static_cast<const T*>(weight), static_cast<const T*>(bias), kernel_width,
                       channels, static_cast<T*>(conv_state), state_slot_stride, state_layer_stride, layer,
                       read_slots, read_stride, read_dtype == GDN_I64, write_slots, write_stride,
                       write_dtype == GDN_I64, static_cast<T*>(q_out), static_cast<T*>(k_out),
                       static_cast<T*>(v_out), key_dim, split_qkv, round_conv, boundary0, boundary1, scale0, scale1,
                       scale2);
    return GDN_LAUNCH_CHECK("gdn_conv_decode launch");
  };
  if (dtype == GDN_BF16) return launch(bf16{});
  if (dtype == GDN_F16) return launch(f16{});
  if (dtype == GDN_F32) return launch(float{});
  set_error("gdn_conv_decode: unsupported dtype %d", dtype);
  return GDN_ERR_UNSUPPORTED;
}
