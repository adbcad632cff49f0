// Gated RMS normalisation of the GDN core output, per row of head_v_dim:
//   y = (x * rsqrt(mean(x^2) + eps)) * w * (z * sigmoid(z)),
// computed in fp32 and stored once in the dtype of x
// (python/logssms/kernel/norm.py:113-148, called through RMSNormGated at
// python/logssms/layers/norm.py:42-53 from GatedDeltaNet.output,
// python/logssms/layers/gated_delta.py:133-139).
//
// Roofline: HBM.  Per row 2 * cols * sizeof(io) bytes are read (x and z) and
// cols * sizeof(io) written; the weight row stays in L2.  Fast path: a group
// of G = cols / 8 lanes owns one row (8 channels per lane, one 16-byte access
// per operand), the sum of squares is reduced across the group with DPP moves,
// and a 256-thread block covers 256 / G rows.  Other layouts (widths that are
// not a multiple of 8 or above 512, strided gate columns, fp32 x) take one
// wave per row with scalar loads.
#include "common.hpp"

namespace gdn {
namespace {

constexpr int kThreads = 256;

struct NormParams {
  const void* x;
  void* out;
  const void* gate;
  const void* weight;
  int64_t rows, cols;
  int64_t gate_rows, gate_group_stride, gate_row_stride, gate_col_stride;
  int x_dtype, gate_dtype, weight_dtype;
  float eps;
};

__device__ __forceinline__ int64_t gate_offset(const NormParams& p, int64_t r) {
  return (r / p.gate_rows) * p.gate_group_stride + (r % p.gate_rows) * p.gate_row_stride;
}

__device__ __forceinline__ float silu_ref(float z) { return z * (1.0f / (1.0f + __expf(-z))); }

// G lanes per row; gate in the io dtype with unit column stride; fp32 weight.
template <class IOT, int G>
__global__ __launch_bounds__(kThreads) void norm_vec_kernel(NormParams p) {
  constexpr int kRows = kThreads / G;
  const int lr = threadIdx.x % G;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kRows + threadIdx.x / G;
  const int64_t c = 8 * static_cast<int64_t>(lr);
  const bool live = r < p.rows && c < p.cols;
  float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float w[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (live) {
    unpack8<IOT>(*reinterpret_cast<const uint4*>(static_cast<const IOT*>(p.x) + r * p.cols + c), x);
    unpack8<IOT>(*reinterpret_cast<const uint4*>(static_cast<const IOT*>(p.gate) + gate_offset(p, r) + c), z);
    const float4 w0 = *reinterpret_cast<const float4*>(static_cast<const float*>(p.weight) + c);
    const float4 w1 = *reinterpret_cast<const float4*>(static_cast<const float*>(p.weight) + c + 4);
    w[0] = w0.x, w[1] = w0.y, w[2] = w0.z, w[3] = w0.w, w[4] = w1.x, w[5] = w1.y, w[6] = w1.z, w[7] = w1.w;
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
  ss = head_sum<G>(ss);
  const float rn = rsqrtf(ss / static_cast<float>(p.cols) + p.eps);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = (x[e] * rn) * w[e] * silu_ref(z[e]);
  if (live) *reinterpret_cast<uint4*>(static_cast<IOT*>(p.out) + r * p.cols + c) = pack8_io<IOT>(y);
}

// Any width, dtype and gate stride: one wave per row, two passes over x.
template <class IOT>
__global__ __launch_bounds__(kThreads) void norm_any_kernel(NormParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  if (r >= p.rows) return;  // whole wave
  const IOT* x = static_cast<const IOT*>(p.x) + r * p.cols;
  float ss = 0.f;
  for (int64_t c = lane; c < p.cols; c += 64) {
    const float v = to_f32(x[c]);
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum<64>(ss);
  const float rn = rsqrtf(ss / static_cast<float>(p.cols) + p.eps);
  const int64_t g0 = gate_offset(p, r);
  IOT* out = static_cast<IOT*>(p.out) + r * p.cols;
  for (int64_t c = lane; c < p.cols; c += 64) {
    const float z = load_any(p.gate, g0 + c * p.gate_col_stride, p.gate_dtype);
    const float w = load_any(p.weight, c, p.weight_dtype);
    out[c] = from_f32<IOT>((to_f32(x[c]) * rn) * w * silu_ref(z));
  }
}

template <class IOT>
void launch_vec(const NormParams& p, hipStream_t s) {
  const int64_t lanes = p.cols / 8;
  auto go = [&](auto Gc) {
    constexpr int G = decltype(Gc)::value;
    const int64_t blocks = (p.rows + kThreads / G - 1) / (kThreads / G);
    hipLaunchKernelGGL((norm_vec_kernel<IOT, G>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s, p);
  };
  if (lanes <= 1) go(std::integral_constant<int, 1>{});
  else if (lanes <= 2) go(std::integral_constant<int, 2>{});
  else if (lanes <= 4) go(std::integral_constant<int, 4>{});
  else if (lanes <= 8) go(std::integral_constant<int, 8>{});
  else if (lanes <= 16) go(std::integral_constant<int, 16>{});
  else if (lanes <= 32) go(std::integral_constant<int, 32>{});
  else go(std::integral_constant<int, 64>{});
}

template <class IOT>
int launch_norm(const NormParams& p, hipStream_t s) {
  const bool vec = !std::is_same_v<IOT, float> && p.gate_dtype == p.x_dtype && p.weight_dtype == GDN_F32 &&
                   p.cols % 8 == 0 && p.cols <= 512 && p.gate_col_stride == 1 && p.gate_group_stride % 8 == 0 &&
                   p.gate_row_stride % 8 == 0 && aligned16(p.x) && aligned16(p.out) && aligned16(p.gate) &&
                   aligned16(p.weight);
  if constexpr (!std::is_same_v<IOT, float>) {
    if (vec) {
      launch_vec<IOT>(p, s);
      return GDN_LAUNCH_CHECK("gdn_rms_norm_gated launch");
    }
  }
  const int64_t blocks = (p.rows + kThreads / 64 - 1) / (kThreads / 64);
  hipLaunchKernelGGL((norm_any_kernel<IOT>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s, p);
  return GDN_LAUNCH_CHECK("gdn_rms_norm_gated launch");
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_rms_norm_gated(const void* x, int dtype, int64_t rows, int64_t cols, const void* gate,
                                  int gate_dtype, int64_t gate_rows, int64_t gate_group_stride,
                                  int64_t gate_row_stride, int64_t gate_col_stride, const void* weight,
                                  int weight_dtype, float eps, void* out, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(rows >= 0 && cols > 0 && gate_rows > 0, "gdn_rms_norm_gated: bad shape (rows %lld, cols %lld)",
              static_cast<long long>(rows), static_cast<long long>(cols));
  GDN_REQUIRE((dtype == GDN_F32 || dtype == GDN_BF16 || dtype == GDN_F16) &&
                  (gate_dtype == GDN_F32 || gate_dtype == GDN_BF16 || gate_dtype == GDN_F16) &&
                  (weight_dtype == GDN_F32 || weight_dtype == GDN_BF16 || weight_dtype == GDN_F16),
              "gdn_rms_norm_gated: unknown dtype");
  GDN_REQUIRE((rows + 3) / 4 <= 0x7fffffff, "gdn_rms_norm_gated: too many rows");
  if (rows == 0) return GDN_OK;
  GDN_REQUIRE(x && gate && weight && out, "gdn_rms_norm_gated: null input");
  NormParams p{x, out, gate, weight, rows, cols, gate_rows, gate_group_stride, gate_row_stride, gate_col_stride,
               dtype, gate_dtype, weight_dtype, eps};
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case GDN_BF16: return launch_norm<bf16>(p, s);
    case GDN_F16: return launch_norm<f16>(p, s);
    default: return launch_norm<float>(p, s);
  }
}
