// Prefill front end: packed varlen causal conv1d (+ SiLU, window snapshots),
// prepare_gdn, and the fused conv -> split -> prepare pass used by the backend.
//
// Roofline: HBM.  Each thread owns one channel and walks a tile of
// consecutive packed tokens with the W-1 previous inputs in registers, so
// every input element is read once (the reference's Triton kernel reloads
// each element W times through 4 shifted masked loads, packed_conv.py:99-110)
// and consecutive threads touch consecutive channels (coalesced rows).
// Per token and channel: 2 bytes in, 2 bytes out (bf16).
#include <type_traits>

#include "common.hpp"

namespace gdn {
namespace {

constexpr int kThreads = 256;
constexpr int kTile = 32;  // tokens per thread

// End of the packed tokens, cu[N]: rows at or past it (the padding of a
// fixed-capacity input) belong to no sequence and are neither read nor written.
__device__ __forceinline__ int64_t tile_end(const void* cu, int cu_is64, int64_t n, int64_t rows, int64_t t0,
                                            int64_t tile) {
  const int64_t packed = load_index(cu, n, cu_is64);
  const int64_t lim = packed < rows ? packed : rows;
  return t0 + tile < lim ? t0 + tile : lim;
}

struct ConvParams {
  const void* x;
  int64_t xr, xc;
  const void* w;
  const void* bias;
  const void* history;  // [N, C, W-1] or nullptr (use pool + baseline slots)
  const void* cu;
  int cu_is64;
  int64_t N, T, C;
  int W;
  void* out;
  void* state;
  int64_t slot_stride, layer_stride, layer;
  const void* token_slots;
  int token_is64;
  const void* final_slots;
  int final_is64;
  const void* baseline;  // frontend: history from state[baseline[r]]
  int baseline_is64;
  int64_t end0, end1;
  float s0, s1, s2;
};

// Walks tokens [t0, t1) of one channel.  Emits, per token, the rounded SiLU
// output through `emit(t, y)` and writes window snapshots.
template <class T, class Emit>
__device__ __forceinline__ void conv_channel(const ConvParams& p, int64_t ch, int64_t t0, int64_t t1, Emit&& emit) {
  const int W = p.W;
  const int S = W - 1;
  float w[8];
  for (int i = 0; i < W; ++i) w[i] = to_f32(static_cast<const T*>(p.w)[ch * W + i]);
  const float bias = p.bias ? to_f32(static_cast<const T*>(p.bias)[ch]) : 0.f;
  const bool scaled = p.s0 != 1.f || p.s1 != 1.f || p.s2 != 1.f;
  const float sc = ch < p.end0 ? p.s0 : (ch < p.end1 ? p.s1 : p.s2);
  int64_t r = find_sequence(p.cu, p.cu_is64, p.N, t0);
  int64_t begin = load_index(p.cu, r, p.cu_is64);
  int64_t end = load_index(p.cu, r + 1, p.cu_is64);
  float win[8];
  auto history_at = [&](int64_t req, int i) -> float {  // i in [0, S): oldest first
    if (p.history) return to_f32(static_cast<const T*>(p.history)[(req * p.C + ch) * S + i]);
    const int64_t slot = load_index(p.baseline, req, p.baseline_is64);
    if (slot < 0) return 0.f;
    return to_f32(static_cast<const T*>(p.state)[slot * p.slot_stride + p.layer * p.layer_stride + ch * S + i]);
  };
  auto x_at = [&](int64_t t) -> float {
    float v = to_f32(static_cast<const T*>(p.x)[t * p.xr + ch * p.xc]);
    return scaled ? round_to<T>(v * sc) : v;
  };
  auto load_window = [&](int64_t t) {
    // window = inputs at positions t-S .. t-1 of the sequence containing t
    for (int i = 0; i < S; ++i) {
      const int64_t pos = t - S + i;
      win[i] = pos >= begin ? x_at(pos) : history_at(r, static_cast<int>(pos - begin + S));
    }
  };
  load_window(t0);
  for (int64_t t = t0; t < t1; ++t) {
    while (t >= end) {  // next sequence (skips empty ones)
      ++r;
      begin = end;
      end = load_index(p.cu, r + 1, p.cu_is64);
      if (t < end) load_window(t);
    }
    const float xv = x_at(t);
    float acc = 0.f;
    for (int i = 0; i < S; ++i) acc = fmaf(win[i], w[i], acc);
    acc = fmaf(xv, w[S], acc);
    acc += bias;
    const float y = round_to<T>(silu(round_to<T>(acc)));
    emit(t, y);
    for (int i = 0; i + 1 < S; ++i) win[i] = win[i + 1];
    win[S - 1] = xv;
    if (p.state) {
      int64_t slot = p.token_slots ? load_index(p.token_slots, t, p.token_is64) : -1;
      const bool last = t == end - 1;
      int64_t fslot = (last && p.final_slots) ? load_index(p.final_slots, r, p.final_is64) : -1;
      for (int k = 0; k < 2; ++k) {
        const int64_t s = k == 0 ? slot : fslot;
        if (s < 0) continue;
        T* dst = static_cast<T*>(p.state) + s * p.slot_stride + p.layer * p.layer_stride + ch * S;
        for (int i = 0; i < S; ++i) dst[i] = from_f32<T>(win[i]);
      }
    }
  }
}

template <class T>
__global__ __launch_bounds__(kThreads) void packed_conv_kernel(ConvParams p) {
  const int64_t ch = static_cast<int64_t>(blockIdx.y) * kThreads + threadIdx.x;
  if (ch >= p.C) return;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kTile;
  const int64_t t1 = tile_end(p.cu, p.cu_is64, p.N, p.T, t0, kTile);
  if (t0 >= t1) return;
  T* out = static_cast<T*>(p.out);
  conv_channel<T>(p, ch, t0, t1, [&](int64_t t, float y) { out[t * p.C + ch] = from_f32<T>(y); });
}

// ------------------------------------------------------------ fused frontend
struct FrontParams {
  ConvParams conv;
  int64_t H, HV, DK, DV;
  const void* gate;
  int64_t gate_r, gate_h;
  int gate_dtype;
  const void* beta;
  int64_t beta_r, beta_h;
  int beta_dtype;
  const void* A_log;
  int a_dtype;
  const void* dt_bias;
  int dt_dtype;
  void* q_out;
  void* k_out;
  void* v_out;
  float* g_out;
  float* b_out;
  int64_t g_ld;  // 0: g_out / b_out [T, HV]; else head-major [HV, g_ld]
  int qk_f16;  // q_out / k_out as f16 MFMA operands (the bf16-rounded values, converted)
};

// grid: (token tiles, C / 256).  A 256-channel slab holds whole q/k heads
// (DK divides 256 and the q/k sections start at multiples of DK).
template <class T, int DK>
__global__ __launch_bounds__(kThreads) void frontend_kernel(FrontParams fp) {
  __shared__ float part[kTile][kThreads / 64];
  const ConvParams& p = fp.conv;
  const int64_t ch = static_cast<int64_t>(blockIdx.y) * kThreads + threadIdx.x;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kTile;
  const int64_t t1 = tile_end(p.cu, p.cu_is64, p.N, p.T, t0, kTile);
  if (t0 >= t1) return;  // whole block: padding rows only
  const int n = static_cast<int>(t1 - t0);
  const int64_t key_dim = fp.H * DK;
  const bool active = ch < p.C;
  const bool is_qk = active && ch < 2 * key_dim;
  // Each thread parks its own column here (no cross-thread traffic), so the
  // per-token loop below can index registers statically.
  __shared__ float tile[kTile][kThreads];
  if (active) conv_channel<T>(p, ch, t0, t1, [&](int64_t t, float v) { tile[t - t0][threadIdx.x] = v; });
  float y[kTile];
#pragma unroll
  for (int i = 0; i < kTile; ++i) y[i] = (active && i < n) ? tile[i][threadIdx.x] : 0.f;
  // per-token sum of squares over each q/k head (DK consecutive channels)
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  constexpr int kWidth = DK < 64 ? DK : 64;
#pragma unroll
  for (int i = 0; i < kTile; ++i) {
    float s = is_qk ? y[i] * y[i] : 0.f;
    s = wave_sum<kWidth>(s);
    if (DK >= 64 && lane == 0) part[i][wave] = s;
    if (DK < 64) y[i] = is_qk ? y[i] * rsqrtf(s + 1e-6f) : y[i];
  }
  if (DK >= 64) {
    __syncthreads();
    constexpr int waves_per_head = DK / 64;
    const int first = (wave / waves_per_head) * waves_per_head;
#pragma unroll
    for (int i = 0; i < kTile; ++i) {
      float s = 0.f;
      for (int w = 0; w < waves_per_head; ++w) s += part[i][first + w];
      if (is_qk) y[i] *= rsqrtf(s + 1e-6f);
    }
  }
  if (active) {
    const int64_t value_dim = fp.HV * fp.DV;
    for (int i = 0; i < n; ++i) {
      const int64_t t = t0 + i;
      const T v = from_f32<T>(y[i]);
      if (ch < key_dim)
        static_cast<T*>(fp.q_out)[t * key_dim + ch] = v;
      else if (ch < 2 * key_dim)
        static_cast<T*>(fp.k_out)[t * key_dim + ch - key_dim] = v;
      else
        static_cast<T*>(fp.v_out)[t * value_dim + ch - 2 * key_dim] = v;
    }
  }
  if (blockIdx.y == 0) {
    for (int idx = threadIdx.x; idx < n * fp.HV; idx += kThreads) {
      const int64_t t = t0 + idx / fp.HV;
      const int64_t h = idx % fp.HV;
      const float a = load_any(fp.A_log, h, fp.a_dtype);
      const float bias = load_any(fp.dt_bias, h, fp.dt_dtype);
      const float gv = load_any(fp.gate, t * fp.gate_r + h * fp.gate_h, fp.gate_dtype) + bias;
      const float bv = load_any(fp.beta, t * fp.beta_r + h * fp.beta_h, fp.beta_dtype);
      fp.g_out[t * fp.HV + h] = -expf(a) * softplus_prefill(gv);
      fp.b_out[t * fp.HV + h] = sigmoid(bv);
    }
  }
}

// ---------------------------------------------- vectorised path (8 channels / thread)
// Used when the input rows are unit-stride, 16-byte aligned and C % 8 == 0.
// Each thread owns 8 consecutive channels for a tile of kVTok tokens: one
// 16-byte load and one 16-byte store per token, the W-1 previous inputs in
// registers, and the per-head q/k sum of squares reduced across the DK/8
// lanes of the head with cross-lane shuffles (no LDS).
constexpr int kVTok = 32;


// FRONT: fused front end (q/k normalised into q_out/k_out, v into v_out, history
// from the pool); otherwise the plain packed conv into conv.out.
template <class T, int W, int DK, bool FRONT>
__global__ __launch_bounds__(256) void conv_vec_kernel(FrontParams fp) {
  const ConvParams& p = fp.conv;
  constexpr int S = W - 1;
  const int64_t ch0 = (static_cast<int64_t>(blockIdx.y) * 256 + threadIdx.x) * 8;
  const bool active = ch0 < p.C;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kVTok;
  const int64_t t1 = tile_end(p.cu, p.cu_is64, p.N, p.T, t0, kVTok);
  if (t0 >= t1) return;  // whole block: padding rows only
  const int64_t key_dim = FRONT ? fp.H * DK : 0;
  float w[W][8], bias[8];
  // The last S inputs live in a ring of W rows: at phase PH (the token's
  // index mod W inside the tile, known at compile time through the unrolled
  // loop below) tap i is row (PH + i) % W and the token's own input goes to
  // row (PH + S) % W, so the window never moves between registers.
  float ring[W][8];
  const bool scaled = !FRONT && (p.s0 != 1.f || p.s1 != 1.f || p.s2 != 1.f);
  float sc[8];
  if (active) {
    // weights [C][W] contiguous: 8 channels x W taps = W 16-byte pieces
    const uint4* wp = reinterpret_cast<const uint4*>(static_cast<const T*>(p.w) + ch0 * W);
    float wv[8 * W];
#pragma unroll
    for (int i = 0; i < W; ++i) {
      float x[8];
      unpack8<T>(wp[i], x);
#pragma unroll
      for (int e = 0; e < 8; ++e) wv[8 * i + e] = x[e];
    }
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int tap = 0; tap < W; ++tap) w[tap][c] = wv[c * W + tap];
    if (p.bias) {
      unpack8<T>(*reinterpret_cast<const uint4*>(static_cast<const T*>(p.bias) + ch0), bias);
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) bias[c] = 0.f;
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int64_t ch = ch0 + c;
      sc[c] = ch < p.end0 ? p.s0 : (ch < p.end1 ? p.s1 : p.s2);
    }
  }
  const T* x = static_cast<const T*>(p.x);
  auto x_raw = [&](int64_t t) { return *reinterpret_cast<const uint4*>(x + t * p.xr + ch0); };
  auto x_unpack = [&](uint4 raw, float (&v)[8]) {
    unpack8<T>(raw, v);
    if (scaled) {
#pragma unroll
      for (int c = 0; c < 8; ++c) v[c] = round_to<T>(v[c] * sc[c]);
    }
  };
  auto x_at = [&](int64_t t, float (&v)[8]) { x_unpack(x_raw(t), v); };
  int64_t r = find_sequence(p.cu, p.cu_is64, p.N, t0);
  int64_t begin = load_index(p.cu, r, p.cu_is64);
  int64_t end = load_index(p.cu, r + 1, p.cu_is64);
  auto load_window = [&](int64_t t, auto ph) {
    constexpr int PH = decltype(ph)::value;
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int64_t pos = t - S + i;
      if (pos >= begin) {
        float v[8];
        x_at(pos, v);
#pragma unroll
        for (int c = 0; c < 8; ++c) ring[(PH + i) % W][c] = v[c];
      } else {
        const int j = static_cast<int>(pos - begin + S);
        const T* src;
        if (p.history) {
          src = static_cast<const T*>(p.history) + (r * p.C + ch0) * S + j;
        } else {
          const int64_t slot = load_index(p.baseline, r, p.baseline_is64);
          src = slot >= 0 ? static_cast<const T*>(p.state) + slot * p.slot_stride + p.layer * p.layer_stride +
                                ch0 * S + j
                          : nullptr;
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) ring[(PH + i) % W][c] = src ? to_f32(src[c * S]) : 0.f;
      }
    }
  };
  // y = round(silu(round(sum_tap w x + b))) of the token at phase PH, each
  // stage over all 8 channels (independent exp / reciprocal latencies overlap)
  auto conv_silu = [&](const float (&xv)[8], float (&y)[8], auto ph) __attribute__((always_inline)) {
    constexpr int PH = decltype(ph)::value;
    float d[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float acc = bias[c];
#pragma unroll
      for (int i = 0; i < S; ++i) acc = fmaf(ring[(PH + i) % W][c], w[i][c], acc);
      y[c] = fmaf(xv[c], w[S][c], acc);
    }
    round8<T>(y);
#pragma unroll
    for (int c = 0; c < 8; ++c) d[c] = fast_exp2(-1.4426950408889634f * y[c]);
#pragma unroll
    for (int c = 0; c < 8; ++c) d[c] = __builtin_amdgcn_rcpf(1.0f + d[c]);
#pragma unroll
    for (int c = 0; c < 8; ++c) y[c] *= d[c];  // fast_silu
    round8<T>(y);
  };
  // The outputs of token t (ALL: every lane of the block is active).
  auto emit = [&](int64_t t, float (&y)[8], auto all) __attribute__((always_inline)) {
    constexpr bool ALL = decltype(all)::value;
    const bool on = ALL || active;
    if (FRONT) {
      // per-head sum of squares over DK / 8 lanes (heads start at multiples of DK)
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < 8; ++c) ss = fmaf(y[c], y[c], ss);
      ss = head_sum<DK / 8>(ss);
      if (on) {
        if (ch0 < 2 * key_dim) {
          // ss + 1e-6 is a normal float, so the hardware rsq needs no range scaling
          const float rn = __builtin_amdgcn_rsqf(ss + 1e-6f);
#pragma unroll
          for (int c = 0; c < 8; ++c) y[c] *= rn;
          T* dst = ch0 < key_dim ? static_cast<T*>(fp.q_out) + t * key_dim + ch0
                                 : static_cast<T*>(fp.k_out) + t * key_dim + ch0 - key_dim;
          const uint4 packed = pack8_io<T>(y);
          *reinterpret_cast<uint4*>(dst) = fp.qk_f16 ? to_f16x8<T>(packed) : packed;
        } else {
          *reinterpret_cast<uint4*>(static_cast<T*>(fp.v_out) + t * (fp.HV * fp.DV) + ch0 - 2 * key_dim) =
              pack8_io<T>(y);
        }
      }
    } else if (on) {
      *reinterpret_cast<uint4*>(static_cast<T*>(p.out) + t * p.C + ch0) = pack8_io<T>(y);
    }
  };
  // One token in general: sequence starts, snapshots, outputs.
  auto token = [&](int64_t t, const float (&xv)[8], auto ph) __attribute__((always_inline)) {
    constexpr int PH = decltype(ph)::value;
    float y[8];
    conv_silu(xv, y, ph);
    if (active && p.state) {  // window snapshots (raw inputs, oldest first)
      const int64_t slot = p.token_slots ? load_index(p.token_slots, t, p.token_is64) : -1;
      const int64_t fslot = (!FRONT && p.final_slots && t == end - 1) ? load_index(p.final_slots, r, p.final_is64) : -1;
      for (int k = 0; k < 2; ++k) {
        const int64_t s_ = k == 0 ? slot : fslot;
        if (s_ < 0) continue;
        T* dst = static_cast<T*>(p.state) + s_ * p.slot_stride + p.layer * p.layer_stride + ch0 * S;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
#pragma unroll
          for (int i = 0; i + 1 < S; ++i) dst[c * S + i] = from_f32<T>(ring[(PH + i + 1) % W][c]);
          dst[c * S + S - 1] = from_f32<T>(xv[c]);
        }
      }
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) ring[(PH + S) % W][c] = xv[c];
    emit(t, y, std::false_type{});
  };
  if (active) load_window(t0, std::integral_constant<int, 0>{});
  // the input row of the next token is loaded one token ahead, so its HBM
  // latency overlaps this token's arithmetic (inactive lanes keep zeros)
  uint4 next = active ? x_raw(t0) : make_uint4(0, 0, 0, 0);
  int64_t t = t0;
  auto step = [&](auto ph) __attribute__((always_inline)) {
    while (t >= end) {  // next sequence (skips empty ones)
      ++r;
      begin = end;
      end = load_index(p.cu, r + 1, p.cu_is64);
      if (t < end && active) load_window(t, ph);
    }
    const uint4 cur = next;
    if (active && t + 1 < t1) next = x_raw(t + 1);
    float xv[8];
    x_unpack(cur, xv);
    token(t, xv, ph);
    ++t;
  };
  // tokens go in groups of W, one per phase of the window ring
  auto group = [&](auto... ph) __attribute__((always_inline)) { (step(ph), ...); };
  auto tail = [&](auto... ph) __attribute__((always_inline)) { ((t < t1 ? step(ph) : void()), ...); };
  auto phases = [&](auto f) __attribute__((always_inline)) {
    if constexpr (W == 2) f(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{});
    else if constexpr (W == 3)
      f(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{}, std::integral_constant<int, 2>{});
    else
      f(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{}, std::integral_constant<int, 2>{},
        std::integral_constant<int, 3>{});
  };
  while (t + W <= t1) phases(group);
  phases(tail);
  if (FRONT && fp.g_out) {
    // the tile's gates, split over the blocks of its channel groups
    const int n = static_cast<int>(t1 - t0);
    for (int idx = threadIdx.x + 256 * static_cast<int>(blockIdx.y); idx < n * fp.HV; idx += 256 * gridDim.y) {
      // head-major output: consecutive threads take consecutive tokens of a head
      const int64_t t = t0 + (fp.g_ld ? idx % n : idx / fp.HV);
      const int64_t h = fp.g_ld ? idx / n : idx % fp.HV;
      const int64_t o = fp.g_ld ? h * fp.g_ld + t : t * fp.HV + h;
      const float a = load_any(fp.A_log, h, fp.a_dtype);
      const float b = load_any(fp.dt_bias, h, fp.dt_dtype);
      const float gv = load_any(fp.gate, t * fp.gate_r + h * fp.gate_h, fp.gate_dtype) + b;
      const float bv = load_any(fp.beta, t * fp.beta_r + h * fp.beta_h, fp.beta_dtype);
      fp.g_out[o] = -expf(a) * softplus_prefill(gv);
      fp.b_out[o] = sigmoid(bv);
    }
  }
}

// Launch the vectorised kernel when the layout allows it; returns -1 if not.
template <class T, bool FRONT>
int launch_vec(const FrontParams& fp, int dk, hipStream_t s) {
  const ConvParams& p = fp.conv;
  const bool aligned = p.xc == 1 && p.xr % 8 == 0 && p.C % 8 == 0 &&
                       (reinterpret_cast<uintptr_t>(p.x) & 15) == 0 && (reinterpret_cast<uintptr_t>(p.w) & 15) == 0 &&
                       (!p.bias || (reinterpret_cast<uintptr_t>(p.bias) & 15) == 0) &&
                       (FRONT || (reinterpret_cast<uintptr_t>(p.out) & 15) == 0) && p.W >= 2 && p.W <= 4;
  if (!aligned) return -1;
  dim3 grid(static_cast<unsigned>((p.T + kVTok - 1) / kVTok), static_cast<unsigned>((p.C / 8 + 255) / 256));
  auto go = [&](auto Wc, auto DKc) {
    constexpr int Wv = decltype(Wc)::value, DKv = decltype(DKc)::value;
    hipLaunchKernelGGL((conv_vec_kernel<T, Wv, DKv, FRONT>), grid, dim3(256), 0, s, fp);
  };
  auto by_dk = [&](auto Wc) {
    switch (dk) {
      case 32: go(Wc, std::integral_constant<int, 32>{}); return 0;
      case 64: go(Wc, std::integral_constant<int, 64>{}); return 0;
      case 128: go(Wc, std::integral_constant<int, 128>{}); return 0;
      case 256: go(Wc, std::integral_constant<int, 256>{}); return 0;
      default: return -1;
    }
  };
  switch (p.W) {
    case 2: return by_dk(std::integral_constant<int, 2>{});
    case 3: return by_dk(std::integral_constant<int, 3>{});
    default: return by_dk(std::integral_constant<int, 4>{});
  }
}

// ------------------------------------------------------------- prepare_gdn
struct PrepParams {
  const void* q;
  const void* k;
  const void* v;
  int64_t qs[4], ks[4], vs[4];
  const void* gate;
  int64_t gs[3];
  int gate_dtype;
  const void* beta;
  int64_t bs[3];
  int beta_dtype;
  const void* A_log;
  int64_t a_stride;
  int a_dtype;
  const void* dt_bias;
  int64_t dt_stride;
  int dt_dtype;
  int64_t B, T, H, HV, DK, DV;
  void* q_out;
  void* k_out;
  void* v_out;
  float* g_out;
  float* b_out;
};

// One wave per (b, t, v-head) row, 4 rows per block (kernel/fused.py:53-117).
template <class T>
__global__ __launch_bounds__(kThreads) void prepare_kernel(PrepParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  const int64_t rows = p.B * p.T * p.HV;
  if (row >= rows) return;
  const int64_t h = row % p.HV;
  const int64_t t = (row / p.HV) % p.T;
  const int64_t b = row / (p.HV * p.T);
  const int64_t group = p.HV / p.H;
  const int64_t kh = h / group;
  if (h % group == 0) {
    for (int which = 0; which < 2; ++which) {
      const T* src = static_cast<const T*>(which == 0 ? p.q : p.k);
      const int64_t* st = which == 0 ? p.qs : p.ks;
      const int64_t base = b * st[0] + t * st[1] + kh * st[2];
      float ss = 0.f;
      for (int64_t d = lane; d < p.DK; d += 64) {
        const float v = to_f32(src[base + d * st[3]]);
        ss += v * v;
      }
      ss = wave_sum<64>(ss);
      const float r = rsqrtf(ss + 1e-6f);
      T* dst = static_cast<T*>(which == 0 ? p.q_out : p.k_out) + ((b * p.T + t) * p.H + kh) * p.DK;
      for (int64_t d = lane; d < p.DK; d += 64) dst[d] = from_f32<T>(to_f32(src[base + d * st[3]]) * r);
    }
  }
  const T* vsrc = static_cast<const T*>(p.v);
  const int64_t vbase = b * p.vs[0] + t * p.vs[1] + h * p.vs[2];
  T* vdst = static_cast<T*>(p.v_out) + row * p.DV;
  for (int64_t d = lane; d < p.DV; d += 64) vdst[d] = vsrc[vbase + d * p.vs[3]];
  if (lane == 0) {
    const float a = load_any(p.A_log, h * p.a_stride, p.a_dtype);
    const float bias = load_any(p.dt_bias, h * p.dt_stride, p.dt_dtype);
    const float g = load_any(p.gate, b * p.gs[0] + t * p.gs[1] + h * p.gs[2], p.gate_dtype) + bias;
    const float bt = load_any(p.beta, b * p.bs[0] + t * p.bs[1] + h * p.bs[2], p.beta_dtype);
    p.g_out[row] = -expf(a) * softplus_prefill(g);
    p.b_out[row] = sigmoid(bt);
  }
}

template <class F>
int dispatch_dtype(int dtype, F&& f) {
  if (dtype == GDN_BF16) return f(bf16{});
  if (dtype == GDN_F16) return f(f16{});
  if (dtype == GDN_F32) return f(float{});
  set_error("unsupported dtype %d", dtype);
  return GDN_ERR_UNSUPPORTED;
}

struct SnapshotParams {
  const void* mixed;
  int64_t row_stride;
  const void* cu;
  int cu_is64;
  int64_t N, T, C;
  int S;  // kernel width - 1
  void* conv_state;
  int64_t slot_stride, layer_stride, layer;
  const void* baseline;
  int baseline_is64;
  const void* rows;
  int rows_is64;
  const void* slots;
  int slots_is64;
};

// Grid (snapshot, 256-channel block), one channel per thread (16-bit values
// copied as bits, so the window is the raw input exactly).
__global__ __launch_bounds__(kThreads) void conv_snapshot_kernel(SnapshotParams sp) {
  const int64_t i = blockIdx.x;
  const int64_t ch = static_cast<int64_t>(blockIdx.y) * kThreads + threadIdx.x;
  if (ch >= sp.C) return;
  const int64_t slot = load_index(sp.slots, i, sp.slots_is64);
  if (slot < 0) return;
  const int64_t row = load_index(sp.rows, i, sp.rows_is64);
  if (row < 0 || row >= sp.T) return;
  const int64_t r = find_sequence(sp.cu, sp.cu_is64, sp.N, row);
  const int64_t begin = load_index(sp.cu, r, sp.cu_is64);
  const int64_t base = load_index(sp.baseline, r, sp.baseline_is64);
  const uint16_t* x = static_cast<const uint16_t*>(sp.mixed);
  uint16_t* pool = static_cast<uint16_t*>(sp.conv_state);
  const uint16_t* hist = base >= 0 ? pool + base * sp.slot_stride + sp.layer * sp.layer_stride : nullptr;
  uint16_t* dst = pool + slot * sp.slot_stride + sp.layer * sp.layer_stride;
  const int S = sp.S;
  for (int j = 0; j < S; ++j) {
    const int64_t pos = row - (S - 1) + j;
    uint16_t v;
    if (pos >= begin) v = x[pos * sp.row_stride + ch];
    else v = hist ? hist[ch * S + (pos - begin + S)] : 0;
    dst[ch * S + j] = v;
  }
}

}  // namespace

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_packed_causal_conv1d(const void* x, int64_t x_row_stride, int64_t x_col_stride, int dtype,
                                        const void* weight, const void* bias, const void* history,
                                        const void* cu_seqlens, int cu_dtype, int64_t num_seqs,
                                        int64_t total_tokens, int64_t channels, int kernel_width, void* out,
                                        void* conv_state, int64_t state_slot_stride, int64_t state_layer_stride,
                                        int64_t layer, const void* token_slots, int token_slots_dtype,
                                        const void* final_slots, int final_slots_dtype, int64_t boundary0,
                                        int64_t boundary1, float scale0, float scale1, float scale2,
                                        void* stream) {
  GDN_REQUIRE(num_seqs >= 1 && total_tokens >= 0 && channels > 0, "gdn_packed_causal_conv1d: bad sizes");
  if (total_tokens == 0) return GDN_OK;
  GDN_REQUIRE(kernel_width >= 2 && kernel_width <= 8, "gdn_packed_causal_conv1d: kernel width %d not in [2, 8]",
              kernel_width);
  GDN_REQUIRE(x && weight && history && cu_seqlens && out, "gdn_packed_causal_conv1d: null input");
  GDN_REQUIRE(channels <= 65535LL * kThreads, "gdn_packed_causal_conv1d: too many channels");
  ConvParams p{};
  p.x = x; p.xr = x_row_stride; p.xc = x_col_stride; p.w = weight; p.bias = bias; p.history = history;
  p.cu = cu_seqlens; p.cu_is64 = cu_dtype == GDN_I64; p.N = num_seqs; p.T = total_tokens; p.C = channels;
  p.W = kernel_width; p.out = out; p.state = conv_state; p.slot_stride = state_slot_stride;
  p.layer_stride = state_layer_stride; p.layer = layer; p.token_slots = token_slots;
  p.token_is64 = token_slots_dtype == GDN_I64; p.final_slots = final_slots;
  p.final_is64 = final_slots_dtype == GDN_I64; p.end0 = boundary0; p.end1 = boundary1;
  p.s0 = scale0; p.s1 = scale1; p.s2 = scale2;
  dim3 grid(static_cast<unsigned>((total_tokens + kTile - 1) / kTile),
            static_cast<unsigned>((channels + kThreads - 1) / kThreads));
  return dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    auto s = static_cast<hipStream_t>(stream);
    if constexpr (sizeof(T) == 2) {
      FrontParams fp{};
      fp.conv = p;
      if (launch_vec<T, false>(fp, 128, s) == 0) return GDN_LAUNCH_CHECK("gdn_packed_causal_conv1d launch");
    }
    hipLaunchKernelGGL((packed_conv_kernel<T>), grid, dim3(kThreads), 0, s, p);
    return GDN_LAUNCH_CHECK("gdn_packed_causal_conv1d launch");
  });
}

extern "C" int gdn_prefill_frontend(const void* mixed, int64_t row_stride, int64_t col_stride, int dtype,
                                    const void* weight, const void* bias, int kernel_width, const void* cu_seqlens,
                                    int cu_dtype, int64_t num_seqs, int64_t total_tokens, int64_t H, int64_t HV,
                                    int64_t dk, int64_t dv, const void* conv_state, int64_t state_slot_stride,
                                    int64_t state_layer_stride, int64_t layer, const void* baseline_slots,
                                    int baseline_dtype, const void* gate, int64_t gate_row_stride, int64_t gate_head_stride,
                                    int gate_dtype, const void* beta, int64_t beta_row_stride,
                                    int64_t beta_head_stride, int beta_dtype, const void* A_log, int a_dtype,
                                    const void* dt_bias, int dt_dtype, void* q_out, void* k_out, void* v_out,
                                    float* g_out, float* beta_out, void* stream) {
  GDN_REQUIRE(num_seqs >= 1 && total_tokens >= 0 && H > 0 && HV > 0 && HV % H == 0,
              "gdn_prefill_frontend: bad sizes");
  if (total_tokens == 0) return GDN_OK;
  GDN_REQUIRE(kernel_width >= 2 && kernel_width <= 8, "gdn_prefill_frontend: kernel width %d not in [2, 8]",
              kernel_width);
  GDN_REQUIRE(mixed && weight && cu_seqlens && conv_state && baseline_slots && gate && beta && A_log && dt_bias &&
                  q_out && k_out && v_out && g_out && beta_out,
              "gdn_prefill_frontend: null input");
  const int64_t channels = 2 * H * dk + HV * dv;
  ConvParams p{};
  p.x = mixed; p.xr = row_stride; p.xc = col_stride; p.w = weight; p.bias = bias; p.history = nullptr;
  p.cu = cu_seqlens; p.cu_is64 = cu_dtype == GDN_I64; p.N = num_seqs; p.T = total_tokens; p.C = channels;
  // conv_state is only read (history); token_slots / final_slots stay null so
  // no window is written in this launch
  p.W = kernel_width; p.out = nullptr; p.state = const_cast<void*>(conv_state); p.slot_stride = state_slot_stride;
  p.layer_stride = state_layer_stride; p.layer = layer; p.token_slots = nullptr;
  p.token_is64 = 0; p.final_slots = nullptr; p.final_is64 = 0;
  p.baseline = baseline_slots; p.baseline_is64 = baseline_dtype == GDN_I64;
  p.end0 = channels; p.end1 = channels; p.s0 = p.s1 = p.s2 = 1.f;
  FrontParams fp{};
  fp.conv = p; fp.H = H; fp.HV = HV; fp.DK = dk; fp.DV = dv;
  fp.gate = gate; fp.gate_r = gate_row_stride; fp.gate_h = gate_head_stride; fp.gate_dtype = gate_dtype;
  fp.beta = beta; fp.beta_r = beta_row_stride; fp.beta_h = beta_head_stride; fp.beta_dtype = beta_dtype;
  fp.A_log = A_log; fp.a_dtype = a_dtype; fp.dt_bias = dt_bias; fp.dt_dtype = dt_dtype;
  fp.q_out = q_out; fp.k_out = k_out; fp.v_out = v_out; fp.g_out = g_out; fp.b_out = beta_out;
  dim3 grid(static_cast<unsigned>((total_tokens + kTile - 1) / kTile),
            static_cast<unsigned>((channels + kThreads - 1) / kThreads));
  return dispatch_dtype(dtype, [&](auto tag) -> int {
    using T = decltype(tag);
    auto s = static_cast<hipStream_t>(stream);
    if constexpr (sizeof(T) == 2) {
      if (launch_vec<T, true>(fp, static_cast<int>(dk), s) == 0) return GDN_LAUNCH_CHECK("gdn_prefill_frontend launch");
    }
    switch (dk) {
      case 32: hipLaunchKernelGGL((frontend_kernel<T, 32>), grid, dim3(kThreads), 0, s, fp); break;
      case 64: hipLaunchKernelGGL((frontend_kernel<T, 64>), grid, dim3(kThreads), 0, s, fp); break;
      case 128: hipLaunchKernelGGL((frontend_kernel<T, 128>), grid, dim3(kThreads), 0, s, fp); break;
      case 256: hipLaunchKernelGGL((frontend_kernel<T, 256>), grid, dim3(kThreads), 0, s, fp); break;
      default:
        set_error("gdn_prefill_frontend: head_k_dim %lld not in {32, 64, 128, 256}", (long long)dk);
        return GDN_ERR_UNSUPPORTED;
    }
    return GDN_LAUNCH_CHECK("gdn_prefill_frontend launch");
  });
}

extern "C" int gdn_prepare(const void* query, const int64_t* qs, const void* key, const int64_t* ks,
                           const void* value, const int64_t* vs, int io_dtype, const void* gate, const int64_t* gs,
                           int gate_dtype, const void* beta, const int64_t* bs, int beta_dtype, const void* A_log,
                           int64_t a_stride, int a_dtype, const void* dt_bias, int64_t dt_stride, int dt_dtype,
                           int64_t batch, int64_t tokens, int64_t H, int64_t HV, int64_t dk, int64_t dv,
                           void* q_out, void* k_out, void* v_out, float* g_out, float* beta_out, void* stream) {
  GDN_REQUIRE(batch >= 0 && tokens >= 0 && H > 0 && HV > 0 && HV % H == 0 && dk > 0 && dv > 0,
              "gdn_prepare: bad sizes");
  const int64_t rows = batch * tokens * HV;
  if (rows == 0) return GDN_OK;
  GDN_REQUIRE(query && key && value && gate && beta && A_log && dt_bias && q_out && k_out && v_out && g_out &&
                  beta_out && qs && ks && vs && gs && bs,
              "gdn_prepare: null input");
  PrepParams p{};
  p.q = query; p.k = key; p.v = value;
  for (int i = 0; i < 4; ++i) { p.qs[i] = qs[i]; p.ks[i] = ks[i]; p.vs[i] = vs[i]; }
  for (int i = 0; i < 3; ++i) { p.gs[i] = gs[i]; p.bs[i] = bs[i]; }
  p.gate = gate; p.gate_dtype = gate_dtype; p.beta = beta; p.beta_dtype = beta_dtype;
  p.A_log = A_log; p.a_stride = a_stride; p.a_dtype = a_dtype;
  p.dt_bias = dt_bias; p.dt_stride = dt_stride; p.dt_dtype = dt_dtype;
  p.B = batch; p.T = tokens; p.H = H; p.HV = HV; p.DK = dk; p.DV = dv;
  p.q_out = q_out; p.k_out = k_out; p.v_out = v_out; p.g_out = g_out; p.b_out = beta_out;
  const int64_t blocks = (rows + (kThreads / 64) - 1) / (kThreads / 64);
  GDN_REQUIRE(blocks <= 0x7fffffff, "gdn_prepare: too many rows");
  return dispatch_dtype(io_dtype, [&](auto tag) {
    using T = decltype(tag);
    hipLaunchKernelGGL((prepare_kernel<T>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), p);
    return GDN_LAUNCH_CHECK("gdn_prepare launch");
  });
}

extern "C" int gdn_prefill_qk(const void* mixed, int64_t row_stride, int io_dtype, const void* weight, int kernel_width,
                              const void* cu_seqlens, int cu_dtype, int64_t num_seqs, int64_t total_tokens, int64_t H,
                              int64_t dk, const void* conv_state, int64_t conv_slot_stride, int64_t conv_layer_stride,
                              int64_t layer, const void* baseline_slots, int baseline_dtype, void* q_out, void* k_out,
                              int out_dtype, int64_t HV, const void* gate, int64_t gate_row_stride,
                              int64_t gate_head_stride, int gate_dtype, const void* beta, int64_t beta_row_stride,
                              int64_t beta_head_stride, int beta_dtype, const void* A_log, int a_dtype,
                              const void* dt_bias, int dt_dtype, float* g_out, float* beta_out, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(num_seqs >= 1 && total_tokens >= 0 && H > 0 && HV > 0, "gdn_prefill_qk: bad sizes");
  GDN_REQUIRE(mixed && weight && cu_seqlens && conv_state && baseline_slots && q_out && k_out && gate && beta &&
                  A_log && dt_bias && g_out && beta_out,
              "gdn_prefill_qk: null input");
  GDN_REQUIRE(out_dtype == io_dtype || out_dtype == GDN_F16, "gdn_prefill_qk: out_dtype must be the io dtype or f16");
  auto al = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  const bool covered = kernel_width == 4 && (io_dtype == GDN_BF16 || io_dtype == GDN_F16) &&
                       (dk == 32 || dk == 64 || dk == 128) && row_stride % 8 == 0 && al(mixed) && al(weight) &&
                       al(q_out) && al(k_out);
  if (!covered) {
    set_error("gdn_prefill_qk: not covered (needs conv width 4, 16-bit io, dk in {32, 64, 128}, 16-byte aligned "
              "rows)");
    return GDN_ERR_UNSUPPORTED;
  }
  if (total_tokens == 0) return GDN_OK;
  ConvParams p{};
  p.x = mixed; p.xr = row_stride; p.xc = 1; p.w = weight; p.bias = nullptr; p.history = nullptr;
  p.cu = cu_seqlens; p.cu_is64 = cu_dtype == GDN_I64; p.N = num_seqs; p.T = total_tokens; p.C = 2 * H * dk; p.W = 4;
  p.out = nullptr; p.state = const_cast<void*>(conv_state); p.slot_stride = conv_slot_stride;
  p.layer_stride = conv_layer_stride; p.layer = layer; p.token_slots = nullptr; p.final_slots = nullptr;
  p.baseline = baseline_slots; p.baseline_is64 = baseline_dtype == GDN_I64;
  p.end0 = p.C; p.end1 = p.C; p.s0 = p.s1 = p.s2 = 1.f;
  FrontParams fp{};
  fp.conv = p; fp.H = H; fp.HV = HV; fp.DK = dk; fp.DV = 0;
  fp.q_out = q_out; fp.k_out = k_out;  // no v_out: channels [0, 2 H dk) only
  fp.qk_f16 = out_dtype == GDN_F16;
  fp.gate = gate; fp.gate_r = gate_row_stride; fp.gate_h = gate_head_stride; fp.gate_dtype = gate_dtype;
  fp.beta = beta; fp.beta_r = beta_row_stride; fp.beta_h = beta_head_stride; fp.beta_dtype = beta_dtype;
  fp.A_log = A_log; fp.a_dtype = a_dtype; fp.dt_bias = dt_bias; fp.dt_dtype = dt_dtype;
  fp.g_out = g_out; fp.b_out = beta_out; fp.g_ld = total_tokens;  // [HV, T]
  auto s = static_cast<hipStream_t>(stream);
  const int rc = io_dtype == GDN_BF16 ? launch_vec<bf16, true>(fp, static_cast<int>(dk), s)
                                      : launch_vec<f16, true>(fp, static_cast<int>(dk), s);
  if (rc != 0) {
    set_error("gdn_prefill_qk: layout not covered");
    return GDN_ERR_UNSUPPORTED;
  }
  return GDN_LAUNCH_CHECK("gdn_prefill_qk launch");
}

extern "C" int gdn_conv_snapshots(const void* mixed, int64_t row_stride, int dtype, const void* cu_seqlens,
                                  int cu_dtype, int64_t num_seqs, int64_t total_tokens, int64_t channels,
                                  int kernel_width, void* conv_state, int64_t state_slot_stride,
                                  int64_t state_layer_stride, int64_t layer, const void* baseline_slots,
                                  int baseline_dtype, const void* rows, int rows_dtype, const void* slots,
                                  int slots_dtype, int64_t count, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(num_seqs >= 1 && total_tokens >= 0 && channels > 0 && count >= 0 && count <= 0x7fffffff &&
                  kernel_width >= 2 && kernel_width <= 8,
              "gdn_conv_snapshots: bad sizes");
  GDN_REQUIRE(dtype == GDN_BF16 || dtype == GDN_F16, "gdn_conv_snapshots: 16-bit dtype expected");
  if (count == 0) return GDN_OK;
  GDN_REQUIRE(mixed && cu_seqlens && conv_state && baseline_slots && rows && slots, "gdn_conv_snapshots: null input");
  SnapshotParams sp{};
  sp.mixed = mixed; sp.row_stride = row_stride; sp.cu = cu_seqlens; sp.cu_is64 = cu_dtype == GDN_I64;
  sp.N = num_seqs; sp.T = total_tokens; sp.C = channels; sp.S = kernel_width - 1;
  sp.conv_state = conv_state; sp.slot_stride = state_slot_stride; sp.layer_stride = state_layer_stride;
  sp.layer = layer; sp.baseline = baseline_slots; sp.baseline_is64 = baseline_dtype == GDN_I64;
  sp.rows = rows; sp.rows_is64 = rows_dtype == GDN_I64; sp.slots = slots; sp.slots_is64 = slots_dtype == GDN_I64;
  hipLaunchKernelGGL(conv_snapshot_kernel,
                     dim3(static_cast<unsigned>(count), static_cast<unsigned>((channels + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, static_cast<hipStream_t>(stream), sp);
  return GDN_LAUNCH_CHECK("gdn_conv_snapshots launch");
}
