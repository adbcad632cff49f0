// Shared device/host helpers for the gfx950 GDN kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <type_traits>

#include "../../include/gdn_mi355x.h"

namespace gdn {

// ---------------------------------------------------------------- element types
// bf16 is carried as raw bits; conversions are written out so that rounding is
// explicit (round-to-nearest-even, NaN kept quiet), matching torch's
// ``.to(torch.bfloat16)``.
struct bf16 {
  uint16_t bits;
};
using f16 = _Float16;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(f16 x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f32(bf16 x) {
  return __uint_as_float(static_cast<uint32_t>(x.bits) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

template <class T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float x) { return static_cast<f16>(x); }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) {
  bf16 r;
  r.bits = f32_to_bf16_bits(x);
  return r;
}

// Round a float through element type T and back (models a store + load).
template <class T> __device__ __forceinline__ float round_to(float x) { return to_f32(from_f32<T>(x)); }

// Scalar load of a runtime-typed value.
__device__ __forceinline__ float load_any(const void* p, int64_t i, int dtype) {
  switch (dtype) {
    case GDN_BF16: return to_f32(static_cast<const bf16*>(p)[i]);
    case GDN_F16: return to_f32(static_cast<const f16*>(p)[i]);
    default: return static_cast<const float*>(p)[i];
  }
}

// Entry i of an int32 or int64 index array.  An int64 entry is read as its
// low (little-endian) word, sign-extended: one 4-byte load either way, with
// no branch on the width, so consecutive index loads issue back to back
// instead of each waiting behind a branch.  int64 entries must therefore lie
// in the int32 range (slots, frames, token offsets and sentinels do).
__device__ __forceinline__ int64_t load_index(const void* p, int64_t i, int is64) {
  return static_cast<int64_t>(static_cast<const int32_t*>(p)[is64 ? 2 * i : i]);
}

// x / d and x % d for 0 <= x < 2^32: a shift and a mask when d is a power of
// two (frame sizes, granularities), a 32-bit division otherwise -- never the
// long 64-bit division sequence.  The host checks that the offsets fit.
struct Div32 {
  uint32_t d;
  int32_t shift;  // >= 0: d == 1 << shift; -1: general divisor
  __device__ __forceinline__ uint32_t div(uint32_t x) const { return shift >= 0 ? x >> shift : x / d; }
  __device__ __forceinline__ uint32_t mod(uint32_t x) const { return shift >= 0 ? x & (d - 1) : x % d; }
};
inline Div32 make_div32(int64_t d) {
  Div32 v{static_cast<uint32_t>(d > 0 ? d : 1), -1};
  if (d > 0 && (d & (d - 1)) == 0) v.shift = __builtin_ctzll(static_cast<unsigned long long>(d));
  return v;
}
constexpr int64_t kMaxOffset32 = int64_t{1} << 32;

// Sequence of packed row t: the largest r < n with cu[r] <= t (cu is
// non-decreasing with cu[0] = 0, so empty sequences are skipped).
__device__ __forceinline__ int64_t find_sequence(const void* cu, int cu_is64, int64_t n, int64_t t) {
  int64_t lo = 0, hi = n - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (load_index(cu, mid, cu_is64) <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// ---------------------------------------------------------------- math
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float exp_f(float x) { return __expf(x); }
__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Decode/verify softplus (vendor/fla/fused_recurrent.py:20-22).
__device__ __forceinline__ float softplus_decode(float x) { return x < 20.0f ? logf(1.0f + expf(x)) : x; }
// Prefill softplus (kernel/fused.py:115).
__device__ __forceinline__ float softplus_prefill(float x) {
  return x > 20.0f ? x : log1pf(expf(fminf(x, 20.0f)));
}

// SiLU with the hardware exp2 and reciprocal (the prefill conv's activation).
__device__ __forceinline__ float fast_silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + fast_exp2(-1.4426950408889634f * x));
}

// 8 packed 16-bit values -> 8 floats (exact).
template <class T> __device__ __forceinline__ void unpack8(uint4 v, float (&x)[8]);
template <> __device__ __forceinline__ void unpack8<bf16>(uint4 v, float (&x)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(w[i] << 16);
    x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
template <> __device__ __forceinline__ void unpack8<f16>(uint4 v, float (&x)[8]) {
  const f16* h = reinterpret_cast<const f16*>(&v);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = static_cast<float>(h[i]);
}

// Two outputs rounded to the io type (round-to-nearest-even, one packed convert).
typedef float f2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
template <class IOT> __device__ __forceinline__ uint32_t out_pack2(float a, float b);
template <> __device__ __forceinline__ uint32_t out_pack2<bf16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{a, b}, bf2_t));
}
template <> __device__ __forceinline__ uint32_t out_pack2<f16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{a, b}, h2_t));
}
// Round 8 floats through the io type (round-to-nearest-even, packed converts).
template <class IOT> __device__ __forceinline__ void round8(float (&y)[8]);
template <> __device__ __forceinline__ void round8<bf16>(float (&y)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t u = out_pack2<bf16>(y[2 * i], y[2 * i + 1]);
    y[2 * i] = __uint_as_float(u << 16);
    y[2 * i + 1] = __uint_as_float(u & 0xffff0000u);
  }
}
template <> __device__ __forceinline__ void round8<f16>(float (&y)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = static_cast<float>(static_cast<_Float16>(y[i]));
}
template <class IOT> __device__ __forceinline__ uint4 pack8_io(const float (&y)[8]) {
  return make_uint4(out_pack2<IOT>(y[0], y[1]), out_pack2<IOT>(y[2], y[3]), out_pack2<IOT>(y[4], y[5]),
                    out_pack2<IOT>(y[6], y[7]));
}
// 8 input halfs -> 8 f16 operand halfs (bf16 -> f16 is exact in range;
// round-toward-zero saturates out-of-range values at +-65504).
template <class IOT> __device__ __forceinline__ uint4 to_f16x8(uint4 raw);
template <> __device__ __forceinline__ uint4 to_f16x8<f16>(uint4 raw) { return raw; }
template <> __device__ __forceinline__ uint4 to_f16x8<bf16>(uint4 raw) {
  auto cvt = [](uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(__uint_as_float(w << 16),
                                                                   __uint_as_float(w & 0xffff0000u)));
  };
  return make_uint4(cvt(raw.x), cvt(raw.y), cvt(raw.z), cvt(raw.w));
}
// Sum over aligned groups of L lanes (L a power of two up to 64), every lane
// of a group receiving the group's sum.  Inside a 16-lane row the moves are
// DPP (no LDS round trip): pair swap, quad swap, half-row mirror, half-row
// rotation; 32 and 64 lanes add cross-row shuffles.  The additions pair up
// exactly as in the xor butterfly, so every lane holds the same bits.
template <int L> __device__ __forceinline__ float head_sum(float v) {
  static_assert(L >= 1 && L <= 64 && (L & (L - 1)) == 0, "a power of two up to 64 lanes");
  auto dpp = [](float x, auto ctrl) __attribute__((always_inline)) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xf, 0xf, false));
  };
  if constexpr (L >= 2) v += dpp(v, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
  if constexpr (L >= 4) v += dpp(v, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
  if constexpr (L >= 8) v += dpp(v, std::integral_constant<int, 0x141>{});  // row_half_mirror
  if constexpr (L >= 16) v += dpp(v, std::integral_constant<int, 0x128>{}); // row_ror:8
  if constexpr (L >= 32) v += __shfl_xor(v, 16, 64);
  if constexpr (L >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}
template <int W> __device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = W / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---------------------------------------------------------------- host helpers
inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

// ---------------------------------------------------------------- host errors
void set_error(const char* fmt, ...);
int hip_status(hipError_t err, const char* what);

}  // namespace gdn

#define GDN_REQUIRE(cond, ...)            \
  do {                                    \
    if (!(cond)) {                        \
      ::gdn::set_error(__VA_ARGS__);      \
      return GDN_ERR_INVALID;             \
    }                                     \
  } while (0)

#define GDN_LAUNCH_CHECK(what) ::gdn::hip_status(hipGetLastError(), what)
