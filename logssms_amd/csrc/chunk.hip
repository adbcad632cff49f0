// Chunked gated delta rule over packed varlen sequences (chunk 64) with
// state-pool I/O -- the prefill core of Gated DeltaNet.
//
// Algorithm (vendor/fla/gated_delta.py:15-82 and the kernels it chains):
//   G   = chunk-local cumsum(g) / ln 2                      (cumsum.py:19-75)
//   L   = strict_tril(beta_i k_i.k_j 2^(G_i - G_j)),  A = (I + L)^-1
//                                                           (chunk_fwd.py:26-294)
//   v'  = A (beta (v - 2^G (k h)))      == U - W h with U = A beta v,
//                                          W = A beta 2^G k (wy_fast.py:19-86,
//                                          chunk_delta_h.py:162-181)
//   o   = scale (2^G (q h) + tril_incl(q k^T 2^(G_i - G_j)) v')   (chunk_o.py:85-130)
//   h  <- 2^G_last h + (2^(G_last - G) k)^T v'              (chunk_delta_h.py:194-224)
// Writing v' as A applied to the state-corrected values avoids materialising
// W and U: the state pass needs only k h (the same product the reference
// spends on w h) plus one 64x64 triangular product.
//
// Mapping: one workgroup per (sequence, v-head, 64-column slice of d_v),
// walking the sequence's chunks in order, 8 waves software-pipelined:
//   * state waves 0-3 run only the recurrence chain of chunk c in three
//     barrier-separated stages: (I) k h -> R, (II) A R -> v', (III)
//     h <- 2^G_last h + (2^(G_last-G) k)^T v'.  The fp32 state slice
//     (d_k x 64) lives in MFMA accumulators for the whole sequence; an f16
//     copy is staged in LDS as the B operand of the next chunk's products.
//   * side waves 4-7 do everything off that chain in the same stages: the
//     global prefetch of later chunks into registers, M = q k^T tiles and
//     o = 2^G q h + M v' of chunk c, and the triangular inverse
//     A = (I + L)^-1 of chunk c+1 (k k^T tiles; 16x16 diagonal blocks by fp32
//     forward substitution; off-diagonal blocks by block products on
//     split-f16 MFMA -- x = hi + lo -- which keeps them at ~fp32 accuracy).
// All dense products run on v_mfma_f32_16x16x32_f16 with fp32 accumulation:
// operands are held in fp16 whatever the input dtype (bf16 inputs convert
// exactly), because fp16's 10-bit mantissa keeps the carried fp32 state
// within 1e-3 of an fp32 recurrence where bf16 operands drift to ~4e-3, at
// the same MFMA rate.  Operand magnitudes must stay below 65504 (values are
// saturated there).
// Workgroups sharing a key head (HV/H v-heads x slices) get block ids that
// are equal modulo 8, so they land on the same XCD and share its L2 for q/k.
//
// Roofline: MFMA (16-bit).  Algorithmic flops per token per v-head:
// 10 C d + 6 d^2 + 2/3 C^2 (C = 64, d = 128).
#include "chunk_common.hpp"

namespace gdn {
namespace {

constexpr int kC = 64;
constexpr int kThreads = 512;
constexpr float kRcpLn2 = 1.4426950216f;  // gated_delta.py:12

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <class T> struct Mma;
template <> struct Mma<bf16> {
  using frag = bf16x8_t;
  static __device__ __forceinline__ f32x4 run(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma<f16> {
  using frag = f16x8_t;
  static __device__ __forceinline__ f32x4 run(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <class T> __device__ __forceinline__ uint16_t bits_of(float x);
template <> __device__ __forceinline__ uint16_t bits_of<bf16>(float x) { return f32_to_bf16_bits(x); }
template <> __device__ __forceinline__ uint16_t bits_of<f16>(float x) {
  f16 h = static_cast<f16>(fminf(fmaxf(x, -65504.f), 65504.f));
  return *reinterpret_cast<uint16_t*>(&h);
}
// MFMA operand encoding (see the header comment).
__device__ __forceinline__ uint16_t op_bits(float x) { return bits_of<f16>(x); }
__device__ __forceinline__ uint32_t op_pack(float a, float b) {
  return op_bits(a) | (static_cast<uint32_t>(op_bits(b)) << 16);
}
__device__ __forceinline__ float op_val(uint16_t b) { return static_cast<float>(*reinterpret_cast<f16*>(&b)); }

// 8 input halfs (bf16 or f16) -> 8 operand halfs (f16).
template <class IOT> __device__ __forceinline__ uint4 to_operands(uint4 raw);
template <> __device__ __forceinline__ uint4 to_operands<f16>(uint4 raw) { return raw; }
template <> __device__ __forceinline__ uint4 to_operands<bf16>(uint4 raw) {
  uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = op_pack(__uint_as_float(w[i] << 16), __uint_as_float(w[i] & 0xffff0000u));
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// fp32 16x16 blocks of the triangular solve live in LDS with a row stride of
// 20 floats: 16-byte row reads of 16 different rows hit distinct banks.
constexpr int LDB = 20;
constexpr int BLK = 16 * LDB;
__device__ __forceinline__ int blk(int ti, int tj) { return ti * (ti + 1) / 2 + tj; }

// LDS carve-up (bytes).  Row paddings of 8 halfs keep 16-byte fragment reads
// of consecutive rows on different banks.
template <int DK, int DVS>
struct Smem {
  static constexpr int LDK = DK + 8;   // Kb[2], Qb: [64][LDK] token-major f16
  static constexpr int LDT = kC + 8;   // A16[2], Mb: [64][LDT]; Rt/Vt: [DVS][LDT]
  static constexpr int LDV = DVS + 8;  // Vb: [64][LDV]
  static constexpr int LDH = DK + 8;   // Ht: [DVS][LDH] (h transposed)
  static constexpr int GT = 4 * kC + 4;  // G, 2^G, 2^(G_last-G), beta, 2^G_last
  static constexpr size_t kb = 0;
  static constexpr size_t qb = kb + 2 * 2ull * kC * LDK;
  static constexpr size_t vb = qb + 2ull * kC * LDK;
  static constexpr size_t gt = vb + 2ull * kC * LDV;
  static constexpr size_t lf = gt + 2 * 4ull * GT;
  static constexpr size_t af = lf + 10 * 4ull * BLK;
  static constexpr size_t a16 = af + 10 * 4ull * BLK;
  static constexpr size_t mb = a16 + 2 * 2ull * kC * LDT;
  static constexpr size_t rt = mb + 2ull * kC * LDT;
  static constexpr size_t vt = rt + 2ull * DVS * LDT;
  static constexpr size_t ht = vt + 2ull * DVS * LDT;
  static constexpr size_t tmp = ht + 2ull * DVS * LDH;
  static constexpr size_t total = tmp + 2 * 2 * 4ull * BLK;
  static_assert(total <= 160 * 1024, "LDS budget");
};

typedef f16x8_t frag_t;

// 16-byte f16 fragment: row (row0 + lane % 16), halfs k0 + 8 (lane / 16) .. + 7.
__device__ __forceinline__ frag_t frag_at(const uint16_t* base, int ld, int row0, int k0, int lane) {
  return *reinterpret_cast<const frag_t*>(base + (row0 + (lane & 15)) * ld + k0 + 8 * (lane >> 4));
}
__device__ __forceinline__ f32x4 mma(frag_t a, frag_t b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Synchronisation.  Every cross-wave hand-off in this kernel goes through
// LDS, and nothing the kernel writes to global memory is read back by it, so
// barriers wait only for LDS traffic (lgkmcnt) -- not for the global
// prefetch loads still in flight, which a full __syncthreads() fence would
// drain every stage.  The asm "memory" clobber keeps the compiler from moving
// memory accesses across either point.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// In-wave LDS hand-off (DS operations of one wave execute in order).
__device__ __forceinline__ void wave_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// ---- split-f16 products on fp32 LDS blocks: x = hi + lo, both f16, so a
// product of hi/lo pairs (dropping lo*lo) carries ~fp32 accuracy.
struct Split {
  frag_t hi, lo;
};
__device__ __forceinline__ Split split8(const float (&x)[8]) {
  Split s;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const f16 h = static_cast<f16>(x[e]);
    s.hi[e] = h;
    s.lo[e] = static_cast<f16>(x[e] - static_cast<float>(h));
  }
  return s;
}
// A operand of a 16 x 32 matrix [X0 | X1] (fp32 blocks; nullptr = zero block).
__device__ __forceinline__ Split a_operand(const float* X0, const float* X1, int lane) {
  const int row = lane & 15, kq = lane >> 4;
  const float* X = kq < 2 ? X0 : X1;
  float x[8];
  if (X) {
    const float4 a = *reinterpret_cast<const float4*>(X + row * LDB + 8 * (kq & 1));
    const float4 b = *reinterpret_cast<const float4*>(X + row * LDB + 8 * (kq & 1) + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = 0.f;
  }
  return split8(x);
}
// B operand of a 32 x 16 matrix [Y0; Y1].
__device__ __forceinline__ Split b_operand(const float* Y0, const float* Y1, int lane) {
  const int col = lane & 15, kq = lane >> 4;
  const float* Y = kq < 2 ? Y0 : Y1;
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = Y ? Y[(8 * (kq & 1) + e) * LDB + col] : 0.f;
  return split8(x);
}
__device__ __forceinline__ f32x4 mma_split(const Split& a, const Split& b, f32x4 c) {
  c = mma(a.hi, b.hi, c);
  c = mma(a.hi, b.lo, c);
  return mma(a.lo, b.hi, c);
}
// C-layout tile (rows 4 (lane/16) + e, col lane % 16) -> fp32 block.
__device__ __forceinline__ void store_block(float* B, f32x4 v, int lane, float sign) {
#pragma unroll
  for (int e = 0; e < 4; ++e) B[(4 * (lane >> 4) + e) * LDB + (lane & 15)] = sign * v[e];
}
__device__ __forceinline__ void store_a16(uint16_t* A16, int ld, int ti, int tj, f32x4 v, int lane, float sign) {
#pragma unroll
  for (int e = 0; e < 4; ++e)
    A16[(ti * 16 + 4 * (lane >> 4) + e) * ld + tj * 16 + (lane & 15)] = op_bits(sign * v[e]);
}

template <class ST> __device__ __forceinline__ float load_st(const ST* p) { return to_f32(*p); }
template <class ST> __device__ __forceinline__ void store_st(ST* p, float v) { *p = from_f32<ST>(v); }

template <int DK, int DVS, class IOT, class ST>
__global__ __launch_bounds__(kThreads, 1) void chunk_kernel(ChunkParams p) {
  using SM = Smem<DK, DVS>;
  constexpr int HT = DK / 16;            // h row tiles
  constexpr int CT = DVS / 16;           // column tiles of the slice
  constexpr int HRT = (HT + 3) / 4;      // h row tiles per state wave (ti = wave + 4 i)
  constexpr int KPT = (kC * DK / 8) / 256;   // 16-byte K (or Q) pieces per side thread
  constexpr int VPT = (kC * DVS / 8) / 256;  // 16-byte V pieces per side thread
  static_assert(KPT >= 1 && VPT >= 1, "tile split");

  // Separate LDS objects (not one carved buffer) so the compiler can tell the
  // buffers apart and overlap loads of one with stores to another.
  __shared__ __align__(16) uint16_t sK[2 * kC * SM::LDK];
  __shared__ __align__(16) uint16_t sQ[kC * SM::LDK];
  __shared__ __align__(16) uint16_t sV[kC * SM::LDV];
  __shared__ __align__(16) float sG[2 * SM::GT];
  __shared__ __align__(16) float sL[10 * BLK];
  __shared__ __align__(16) float sA[10 * BLK];
  __shared__ __align__(16) uint16_t sA16[2 * kC * SM::LDT];
  __shared__ __align__(16) uint16_t sM[kC * SM::LDT];
  __shared__ __align__(16) uint16_t sR[DVS * SM::LDT];
  __shared__ __align__(16) uint16_t sVt[DVS * SM::LDT];
  __shared__ __align__(16) uint16_t sH[DVS * SM::LDH];
  __shared__ __align__(16) float sT[4 * BLK];
  uint16_t* Kb0 = sK;
  uint16_t* Qb = sQ;
  uint16_t* Vb = sV;
  float* Gt0 = sG;
  float* Lf = sL;
  float* Af = sA;
  uint16_t* A160 = sA16;
  uint16_t* Mb = sM;
  uint16_t* Rt = sR;
  uint16_t* Vt = sVt;
  uint16_t* Ht = sH;
  float* Tmp = sT;
  auto Kb = [&](int64_t c) { return Kb0 + (c & 1) * kC * SM::LDK; };
  auto Gt = [&](int64_t c) { return Gt0 + (c & 1) * SM::GT; };
  auto A16 = [&](int64_t c) { return A160 + (c & 1) * kC * SM::LDT; };
  auto Lb = [&](int ti, int tj) { return Lf + blk(ti, tj) * BLK; };
  auto Ab = [&](int ti, int tj) { return Af + blk(ti, tj) * BLK; };

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lr = lane & 15, lq = lane >> 4;
  const bool side = wave >= 4;
  const int sw = wave - 4;      // side wave index
  const int st_ = tid - 256;    // side thread index

  // ---- block -> (sequence, key head, member) with XCD-aware grouping
  const int64_t L = blockIdx.x;
  const int64_t slot = L / 8;
  const int64_t group = (slot / p.members) * 8 + (L % 8);
  if (group >= p.N * p.H) return;
  const int member = static_cast<int>(slot % p.members);
  const int64_t n = group / p.H;
  const int64_t kh = group % p.H;
  const int64_t r = p.HV / p.H;
  const int64_t h = kh * r + member / p.nvs;
  const int64_t col_base = static_cast<int64_t>(member % p.nvs) * DVS;

  const int64_t bos = load_index(p.cu, n, p.cu_is64);
  const int64_t eos = load_index(p.cu, n + 1, p.cu_is64);
  const int64_t len = eos - bos;
  const int64_t nchunks = (len + kC - 1) / kC;
  int64_t chunk_base = 0;
  for (int64_t m = 0; m < n; ++m) {
    const int64_t lm = load_index(p.cu, m + 1, p.cu_is64) - load_index(p.cu, m, p.cu_is64);
    chunk_base += (lm + kC - 1) / kC;
  }
  auto valid_rows = [&](int64_t c) -> int {
    const int64_t rem = len - c * kC;
    return rem <= 0 ? 0 : (rem < kC ? static_cast<int>(rem) : kC);
  };

  const uint16_t* qg = static_cast<const uint16_t*>(p.q);
  const uint16_t* kg = static_cast<const uint16_t*>(p.k);
  const uint16_t* vg = static_cast<const uint16_t*>(p.v);
  uint16_t* og = static_cast<uint16_t*>(p.out);
  uint16_t* vng = static_cast<uint16_t*>(p.v_new);
  ST* pool = static_cast<ST*>(p.state);

  // ---------------------------------------------------------------- side-wave prefetch
  uint4 pk[KPT], pq[KPT], pv[VPT];
  float pg = 0.f, pb = 0.f;
  // Each side thread owns KPT (VPT) consecutive 16-byte pieces of one row, so
  // a single base address (plus immediate offsets) covers all of them.
  const int krow = (st_ * KPT) / (DK / 8), kch = (st_ * KPT) % (DK / 8);
  const int vrow = (st_ * VPT) / (DVS / 8), vch = (st_ * VPT) % (DVS / 8);
  const uint16_t* kbase = kg + ((bos + krow) * p.H + kh) * DK + kch * 8;
  const uint16_t* qbase = qg + ((bos + krow) * p.H + kh) * DK + kch * 8;
  const uint16_t* vbase = vg + ((bos + vrow) * p.HV + h) * p.DV + col_base + vch * 8;
  const int64_t kstride = kC * p.H * DK;     // one chunk of K/Q rows
  const int64_t vstride = kC * p.HV * p.DV;  // one chunk of V rows
  auto prefetch = [&](int64_t ck, int64_t cq) {  // K, g, beta of chunk ck; Q, V of chunk cq
    const int nk = valid_rows(ck), nq = valid_rows(cq);
#pragma unroll
    for (int i = 0; i < KPT; ++i) pk[i] = pq[i] = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < VPT; ++i) pv[i] = make_uint4(0, 0, 0, 0);
    if (krow < nk) {
      const uint4* src = reinterpret_cast<const uint4*>(kbase + ck * kstride);
#pragma unroll
      for (int i = 0; i < KPT; ++i) pk[i] = src[i];
    }
    if (krow < nq) {
      const uint4* src = reinterpret_cast<const uint4*>(qbase + cq * kstride);
#pragma unroll
      for (int i = 0; i < KPT; ++i) pq[i] = src[i];
    }
    if (vrow < nq) {
      const uint4* src = reinterpret_cast<const uint4*>(vbase + cq * vstride);
#pragma unroll
      for (int i = 0; i < VPT; ++i) pv[i] = src[i];
    }
    if (st_ < 64) {
      const bool ok = st_ < nk;
      const int64_t off = (bos + ck * kC + (ok ? st_ : 0)) * p.HV + h;
      pg = ok ? p.g[off] : 0.f;
      pb = ok ? p.beta[off] : 0.f;
    }
  };
  // Prefetched registers -> LDS (K and gates of chunk ck, Q and V of chunk cq).
  auto stage = [&](int64_t ck, bool with_k, int64_t cq, bool with_qv) {
    if (with_k) {
      uint4* dst = reinterpret_cast<uint4*>(Kb(ck) + krow * SM::LDK + kch * 8);
#pragma unroll
      for (int i = 0; i < KPT; ++i) dst[i] = to_operands<IOT>(pk[i]);
      if (st_ < 64) {  // chunk-local cumulative gate, log2 units (cumsum.py:19-75)
        const int nk = valid_rows(ck);
        float x = pg;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const float y = __shfl_up(x, off, 64);
          if (st_ >= off) x += y;
        }
        const float G = x * kRcpLn2;
        const float Glast = __shfl(G, nk > 0 ? nk - 1 : 0, 64);
        float* gt = Gt(ck);
        gt[st_] = G;
        gt[kC + st_] = fast_exp2(G);
        gt[2 * kC + st_] = st_ < nk ? fast_exp2(Glast - G) : 0.f;
        gt[3 * kC + st_] = pb;
        if (st_ == 0) gt[4 * kC] = fast_exp2(Glast);
      }
    }
    if (with_qv) {
      uint4* qdst = reinterpret_cast<uint4*>(Qb + krow * SM::LDK + kch * 8);
#pragma unroll
      for (int i = 0; i < KPT; ++i) qdst[i] = to_operands<IOT>(pq[i]);
      uint4* vdst = reinterpret_cast<uint4*>(Vb + vrow * SM::LDV + vch * 8);
#pragma unroll
      for (int i = 0; i < VPT; ++i) vdst[i] = to_operands<IOT>(pv[i]);
    }
  };

  // ---------------------------------------------------------------- side-wave solve pieces
  // S = K K^T tile (ti, tj) of chunk c -> L values (fp32), C layout.
  auto skk_tile = [&](int64_t c, int ti, int tj) {
    const uint16_t* K = Kb(c);
    f32x4 acc = zero4();
#pragma unroll
    for (int k0 = 0; k0 < DK; k0 += 32)
      acc = mma(frag_at(K, SM::LDK, ti * 16, k0, lane), frag_at(K, SM::LDK, tj * 16, k0, lane), acc);
    const float* gt = Gt(c);
    const int j = tj * 16 + lr;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = ti * 16 + 4 * lq + e;
      acc[e] = i > j ? gt[3 * kC + i] * acc[e] * fast_exp2(fminf(gt[i] - gt[j], 0.f)) : 0.f;
    }
    return acc;
  };
  // M = tril_incl(Q K^T 2^(G_i - G_j)) tile of the current chunk -> Mb.
  auto sqk_tile = [&](int64_t c, int ti, int tj) {
    const uint16_t* K = Kb(c);
    f32x4 acc = zero4();
#pragma unroll
    for (int k0 = 0; k0 < DK; k0 += 32)
      acc = mma(frag_at(Qb, SM::LDK, ti * 16, k0, lane), frag_at(K, SM::LDK, tj * 16, k0, lane), acc);
    const float* gt = Gt(c);
    const int j = tj * 16 + lr;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = ti * 16 + 4 * lq + e;
      Mb[i * SM::LDT + j] = op_bits(i >= j ? acc[e] * fast_exp2(fminf(gt[i] - gt[j], 0.f)) : 0.f);
    }
  };
  // (I + L_bb)^-1 for the 4 diagonal blocks by forward substitution (one wave:
  // lane = (block, column)), fp32.  Writes Af diagonal blocks and A16.
  auto diag_inverse = [&](int64_t c) {
    asm volatile("" ::: "memory");  // keep surrounding loads from being hoisted into this region
    const int b = lane >> 4, col = lane & 15;
    const float* Lbb = Lb(b, b);
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float v0 = (i == col) ? 1.f : 0.f, v1 = 0.f;
#pragma unroll
      for (int j = 0; j < i; j += 2) {
        v0 = fmaf(-Lbb[i * LDB + j], x[j], v0);
        if (j + 1 < i) v1 = fmaf(-Lbb[i * LDB + j + 1], x[j + 1], v1);
      }
      x[i] = v0 + v1;
      // keep the compiler from hoisting every row's loads (register pressure)
      asm volatile("" ::: "memory");
    }
    float* Abb = Ab(b, b);
    uint16_t* A = A16(c);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      Abb[i * LDB + col] = x[i];
      A[(16 * b + i) * SM::LDT + 16 * b + col] = op_bits(x[i]);
    }
    asm volatile("" ::: "memory");
  };
  // A_{j+1,j} = -A_{j+1,j+1} L_{j+1,j} A_jj for j = 0 (A10) or j = 2 (A32).
  auto first_offdiag = [&](int64_t c, int j, float* T) {
    f32x4 t = mma_split(a_operand(Lb(j + 1, j), nullptr, lane), b_operand(Ab(j, j), nullptr, lane), zero4());
    store_block(T, t, lane, 1.f);
    wave_sync();
    f32x4 a = mma_split(a_operand(Ab(j + 1, j + 1), nullptr, lane), b_operand(T, nullptr, lane), zero4());
    store_block(Ab(j + 1, j), a, lane, -1.f);
    store_a16(A16(c), SM::LDT, j + 1, j, a, lane, -1.f);
  };
  // Lower-left 32x32 block, column q: [A2q; A3q] = -A_(1,1) L_(1,0) [A0q; A1q].
  auto corner_column = [&](int64_t c, int q, float* T0, float* T1) {
    const float* A0q = q == 0 ? Ab(0, 0) : nullptr;
    const float* A1q = Ab(1, q);
    const Split b0 = b_operand(A0q, A1q, lane);
    f32x4 t0 = mma_split(a_operand(Lb(2, 0), Lb(2, 1), lane), b0, zero4());
    f32x4 t1 = mma_split(a_operand(Lb(3, 0), Lb(3, 1), lane), b0, zero4());
    store_block(T0, t0, lane, 1.f);
    store_block(T1, t1, lane, 1.f);
    wave_sync();
    f32x4 a2 = mma_split(a_operand(Ab(2, 2), nullptr, lane), b_operand(T0, nullptr, lane), zero4());
    f32x4 a3 = mma_split(a_operand(Ab(3, 2), Ab(3, 3), lane), b_operand(T0, T1, lane), zero4());
    store_a16(A16(c), SM::LDT, 2, q, a2, lane, -1.f);
    store_a16(A16(c), SM::LDT, 3, q, a3, lane, -1.f);
  };

  // ---------------------------------------------------------------- state-wave pieces
  f32x4 hacc[HRT][CT];
  auto load_initial = [&]() {
    const int64_t rs = load_index(p.read_slots, n, p.read_is64);
    const ST* src = rs >= 0 ? pool + rs * p.slot_stride + p.layer * p.layer_stride + h * p.head_stride : nullptr;
#pragma unroll
    for (int i = 0; i < HRT; ++i) {
      const int ti = wave + 4 * i;
#pragma unroll
      for (int tj = 0; tj < CT; ++tj) {
        hacc[i][tj] = zero4();
        if (ti < HT && src) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            hacc[i][tj][e] = load_st(src + (ti * 16 + 4 * lq + e) * p.DV + col_base + tj * 16 + lr);
        }
      }
    }
  };
  auto stage_h = [&]() {  // f16 copy of h, column-major (B operand)
#pragma unroll
    for (int i = 0; i < HRT; ++i) {
      const int ti = wave + 4 * i;
      if (ti < HT) {
#pragma unroll
        for (int tj = 0; tj < CT; ++tj) {
          uint2 w;
          w.x = op_pack(hacc[i][tj][0], hacc[i][tj][1]);
          w.y = op_pack(hacc[i][tj][2], hacc[i][tj][3]);
          *reinterpret_cast<uint2*>(Ht + (tj * 16 + lr) * SM::LDH + ti * 16 + 4 * lq) = w;
        }
      }
    }
  };
  auto store_h = [&](int64_t slot_idx) {
    ST* dst = pool + slot_idx * p.slot_stride + p.layer * p.layer_stride + h * p.head_stride;
#pragma unroll
    for (int i = 0; i < HRT; ++i) {
      const int ti = wave + 4 * i;
      if (ti < HT) {
#pragma unroll
        for (int tj = 0; tj < CT; ++tj)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            store_st(dst + (ti * 16 + 4 * lq + e) * p.DV + col_base + tj * 16 + lr, hacc[i][tj][e]);
      }
    }
  };

  // ---------------------------------------------------------------- prologue
  for (int e = tid; e < kC * kC; e += kThreads) {  // upper triangles of A and M stay zero
    const int i = e / kC, j = e % kC;
    if (j > i) {
      A160[i * SM::LDT + j] = 0;
      A160[kC * SM::LDT + i * SM::LDT + j] = 0;
      Mb[i * SM::LDT + j] = 0;
    }
  }
  // The two roles run separate code paths (wave-uniform branch) that execute
  // the same sequence of workgroup barriers: 1 + 3 (if any chunk) in the
  // prologue, then 3 per chunk.
  if (!side) {
    // ============================================================ state waves
    load_initial();
    stage_h();
    lds_barrier();
    if (nchunks > 0) {
      lds_barrier();
      lds_barrier();
      lds_barrier();
    }
    for (int64_t c = 0; c < nchunks; ++c) {
      const int nv = valid_rows(c);
      // ----- stage I: k h for token tile `wave` -> R = beta (v - 2^G k h) -> Rt
      {
        const uint16_t* K = Kb(c);
        const float* gt = Gt(c);
        f32x4 acc[CT];
#pragma unroll
        for (int tj = 0; tj < CT; ++tj) acc[tj] = zero4();
#pragma unroll
        for (int k0 = 0; k0 < DK; k0 += 32) {
          const frag_t a = frag_at(K, SM::LDK, wave * 16, k0, lane);
#pragma unroll
          for (int tj = 0; tj < CT; ++tj) acc[tj] = mma(a, frag_at(Ht, SM::LDH, tj * 16, k0, lane), acc[tj]);
        }
        const int row0 = wave * 16 + 4 * lq;
#pragma unroll
        for (int tj = 0; tj < CT; ++tj) {
          const int col = tj * 16 + lr;
          float rv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int row = row0 + e;
            rv[e] = gt[3 * kC + row] * (op_val(Vb[row * SM::LDV + col]) - gt[kC + row] * acc[tj][e]);
          }
          uint2 w;
          w.x = op_pack(rv[0], rv[1]);
          w.y = op_pack(rv[2], rv[3]);
          *reinterpret_cast<uint2*>(Rt + col * SM::LDT + row0) = w;
        }
      }
      lds_barrier();
      // ----- stage II: v' = A R for token tile `wave` -> Vt; gather decayed k^T
      frag_t kd[HRT][2];
      float gl;
      {
        const uint16_t* A = A16(c);
        f32x4 acc[CT];
#pragma unroll
        for (int tj = 0; tj < CT; ++tj) acc[tj] = zero4();
#pragma unroll
        for (int k0 = 0; k0 < kC; k0 += 32) {
          if (k0 <= wave * 16 + 15) {
            const frag_t a = frag_at(A, SM::LDT, wave * 16, k0, lane);
#pragma unroll
            for (int tj = 0; tj < CT; ++tj) acc[tj] = mma(a, frag_at(Rt, SM::LDT, tj * 16, k0, lane), acc[tj]);
          }
        }
        const int row0 = wave * 16 + 4 * lq;
#pragma unroll
        for (int tj = 0; tj < CT; ++tj) {
          const int col = tj * 16 + lr;
          uint2 w;
          w.x = op_pack(acc[tj][0], acc[tj][1]);
          w.y = op_pack(acc[tj][2], acc[tj][3]);
          *reinterpret_cast<uint2*>(Vt + col * SM::LDT + row0) = w;
          if (vng) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (row0 + e < nv)
                vng[((bos + c * kC + row0 + e) * p.HV + h) * p.DV + col_base + col] = bits_of<IOT>(acc[tj][e]);
          }
        }
        // K and the gates of this chunk are overwritten during stage III
        const uint16_t* K = Kb(c);
        const float* gt = Gt(c);
        gl = gt[4 * kC];
#pragma unroll
        for (int i = 0; i < HRT; ++i) {
          const int ti = wave + 4 * i;
          const int d = ti < HT ? ti * 16 + lr : 0;
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            frag_t f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int tok = ks * 32 + 8 * lq + e;
              f[e] = static_cast<f16>(op_val(K[tok * SM::LDK + d]) * gt[2 * kC + tok]);
            }
            kd[i][ks] = f;
          }
        }
      }
      lds_barrier();
      // ----- stage III: h <- 2^G_last h + (2^(G_last - G) k)^T v'
#pragma unroll
      for (int i = 0; i < HRT; ++i) {
        const int ti = wave + 4 * i;
        if (ti < HT) {
#pragma unroll
          for (int tj = 0; tj < CT; ++tj) {
            f32x4 acc = hacc[i][tj] * gl;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) acc = mma(kd[i][ks], frag_at(Vt, SM::LDT, tj * 16, ks * 32, lane), acc);
            hacc[i][tj] = acc;
          }
        }
      }
      const int64_t cw = load_index(p.cw_slots, chunk_base + c, p.cw_is64);
      if (cw >= 0) store_h(cw);
      stage_h();
      lds_barrier();
    }
    if (p.fw_slots) {
      const int64_t fw = load_index(p.fw_slots, n, p.fw_is64);
      if (fw >= 0) store_h(fw);
    }
  } else {
    // ============================================================ side waves
    prefetch(0, 0);
    stage(0, true, 0, true);
    prefetch(1, 1);
    stage(1, nchunks > 1, 1, false);
    prefetch(2, 1);  // K, g, beta of chunk 2; Q, V of chunk 1 (staged in iteration 0)
    lds_barrier();
    if (nchunks > 0) {  // full solve of chunk 0
      for (int s = sw; s < 10; s += 4) {
        int ti = 0, idx = s;
        while (idx > ti) { idx -= ti + 1; ++ti; }
        store_block(Lb(ti, idx), skk_tile(0, ti, idx), lane, 1.f);
      }
      lds_barrier();
      if (sw == 0) diag_inverse(0);
      lds_barrier();
      if (sw == 0) first_offdiag(0, 0, Tmp);
      if (sw == 1) first_offdiag(0, 2, Tmp + 2 * BLK);
      lds_barrier();
    }
    for (int64_t c = 0; c < nchunks; ++c) {
      const bool next = c + 1 < nchunks;
      const int nv = valid_rows(c);
      // ----- stage I: corner of A(c) (waves 4, 5); M tiles of chunk c; k k^T tiles of chunk c+1
      f32x4 late0 = zero4(), late1 = zero4();
      if (sw < 2) corner_column(c, sw, Tmp + (2 * sw) * BLK, Tmp + (2 * sw + 1) * BLK);
      if (sw == 0) { sqk_tile(c, 0, 0); sqk_tile(c, 1, 0); sqk_tile(c, 1, 1); }
      if (sw == 1) { sqk_tile(c, 2, 0); sqk_tile(c, 2, 1); sqk_tile(c, 2, 2); }
      if (sw == 2) {
        sqk_tile(c, 3, 0);
        sqk_tile(c, 3, 1);
        if (next) {
          store_block(Lb(0, 0), skk_tile(c + 1, 0, 0), lane, 1.f);
          store_block(Lb(1, 1), skk_tile(c + 1, 1, 1), lane, 1.f);
          store_block(Lb(2, 2), skk_tile(c + 1, 2, 2), lane, 1.f);
          store_block(Lb(3, 3), skk_tile(c + 1, 3, 3), lane, 1.f);
        }
      }
      if (sw == 3) {
        sqk_tile(c, 3, 2);
        sqk_tile(c, 3, 3);
        if (next) {
          store_block(Lb(1, 0), skk_tile(c + 1, 1, 0), lane, 1.f);
          store_block(Lb(3, 2), skk_tile(c + 1, 3, 2), lane, 1.f);
        }
      }
      if (next && sw < 2) {  // blocks (2,0),(2,1) / (3,0),(3,1): the corner above still reads them
        late0 = skk_tile(c + 1, 2 + sw, 0);
        late1 = skk_tile(c + 1, 2 + sw, 1);
      }
      lds_barrier();
      // ----- stage II: late L blocks; diagonal inverses of chunk c+1; q h of chunk c
      if (next && sw < 2) {
        store_block(Lb(2 + sw, 0), late0, lane, 1.f);
        store_block(Lb(2 + sw, 1), late1, lane, 1.f);
      }
      if (next && sw == 0) diag_inverse(c + 1);
      f32x4 oq[CT];
      {
        const float* gt = Gt(c);
#pragma unroll
        for (int tj = 0; tj < CT; ++tj) oq[tj] = zero4();
#pragma unroll
        for (int k0 = 0; k0 < DK; k0 += 32) {
          const frag_t a = frag_at(Qb, SM::LDK, sw * 16, k0, lane);
#pragma unroll
          for (int tj = 0; tj < CT; ++tj) oq[tj] = mma(a, frag_at(Ht, SM::LDH, tj * 16, k0, lane), oq[tj]);
        }
#pragma unroll
        for (int tj = 0; tj < CT; ++tj)
#pragma unroll
          for (int e = 0; e < 4; ++e) oq[tj][e] *= gt[kC + sw * 16 + 4 * lq + e];
      }
      lds_barrier();
      // ----- stage III: A10/A32 of chunk c+1; o of chunk c; stage / prefetch later chunks
      if (next && sw < 2) first_offdiag(c + 1, 2 * sw, Tmp + (2 * sw) * BLK);
#pragma unroll
      for (int k0 = 0; k0 < kC; k0 += 32) {
        if (k0 <= sw * 16 + 15) {
          const frag_t a = frag_at(Mb, SM::LDT, sw * 16, k0, lane);
#pragma unroll
          for (int tj = 0; tj < CT; ++tj) oq[tj] = mma(a, frag_at(Vt, SM::LDT, tj * 16, k0, lane), oq[tj]);
        }
      }
#pragma unroll
      for (int tj = 0; tj < CT; ++tj) {
        const int col = tj * 16 + lr;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = sw * 16 + 4 * lq + e;
          if (row < nv)
            og[((bos + c * kC + row) * p.HV + h) * p.DV + col_base + col] = bits_of<IOT>(p.scale * oq[tj][e]);
        }
      }
      stage(c + 2, c + 2 < nchunks, c + 1, next);
      prefetch(c + 3, c + 2);
      lds_barrier();
    }
  }
}

template <int DK, int DVS, class IOT, class ST>
int launch(const ChunkParams& p, int64_t groups, hipStream_t stream) {
  const int64_t blocks = ((groups + 7) / 8) * 8 * p.members;
  if (blocks > 0x7fffffff) {
    set_error("gdn_chunk_gated_delta_rule: grid too large");
    return GDN_ERR_INVALID;
  }
  hipLaunchKernelGGL((chunk_kernel<DK, DVS, IOT, ST>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                     stream, p);
  return GDN_LAUNCH_CHECK("gdn_chunk_gated_delta_rule launch");
}

template <int DK, int DVS>
int dispatch_types(const ChunkParams& p, int io, int st, int64_t groups, hipStream_t s) {
  if (io == GDN_BF16 && st == GDN_F32) return launch<DK, DVS, bf16, float>(p, groups, s);
  if (io == GDN_BF16 && st == GDN_BF16) return launch<DK, DVS, bf16, bf16>(p, groups, s);
  if (io == GDN_F16 && st == GDN_F32) return launch<DK, DVS, f16, float>(p, groups, s);
  if (io == GDN_F16 && st == GDN_F16) return launch<DK, DVS, f16, f16>(p, groups, s);
  set_error("gdn_chunk_gated_delta_rule: unsupported (io %d, state %d); io must be bf16/f16", io, st);
  return GDN_ERR_UNSUPPORTED;
}

}  // namespace
}  // namespace gdn

using namespace gdn;

namespace gdn {

int set_frame_layout(ChunkParams& p, int64_t dk, int state_dtype, const void* frames, int frames_dtype,
                     int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes, int64_t num_frames) {
  const int64_t elt = state_dtype == GDN_F32 ? 4 : 2;
  const int64_t state_bytes = dk * p.DV * elt;
  GDN_REQUIRE(frames_per_slot > 0 && frame_bytes > 0 && num_frames > 0 && head_bytes >= state_bytes &&
                  frame_bytes % elt == 0 && head_bytes % elt == 0,
              "gdn_chunk_gated_delta_rule: bad frame layout (frames_per_slot %lld, frame_bytes %lld, head_bytes "
              "%lld, num_frames %lld, state %lld bytes per head)",
              (long long)frames_per_slot, (long long)frame_bytes, (long long)head_bytes, (long long)num_frames,
              (long long)state_bytes);
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
  p.fps = frames_per_slot;
  p.frame_bytes = frame_bytes;
  p.head_bytes = head_bytes;
  p.num_frames = num_frames;
  p.fdiv = make_div32(frame_bytes);
  return GDN_OK;
}

}  // namespace gdn

namespace gdn {
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
                int final_write_dtype, int64_t chunk_size, const void* frames, int frames_dtype,
                int64_t frames_per_slot, int64_t frame_bytes, int64_t head_bytes, int64_t num_frames, void* out,
                void* v_new, float scale, const LogArgs* log, void* stream) {
  GDN_REQUIRE(num_seqs >= 0 && total_tokens >= 0 && H > 0 && HV > 0 && HV % H == 0 && layer >= 0,
              "gdn_chunk_gated_delta_rule: bad sizes");
  GDN_REQUIRE(chunk_size == 16 || chunk_size == 32 || chunk_size == 64,
              "gdn_chunk_gated_delta_rule: chunk_size %lld not in {16, 32, 64}", (long long)chunk_size);
  if (num_seqs == 0) return GDN_OK;
  GDN_REQUIRE(q && k && v && g && beta && cu_seqlens && state && read_slots && chunk_write_slots && out,
              "gdn_chunk_gated_delta_rule: null input");
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
                                    num_frames);
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
    // a 64-column slice of a value row (128-byte aligned) must not straddle two frames
    if (dv % 64 != 0 || frame_bytes % 128 != 0) {
      set_error("gdn_chunk_gated_delta_rule_logged: needs dv %% 64 == 0 and frames of a multiple of 128 bytes");
      return GDN_ERR_UNSUPPORTED;
    }
  }
  auto s = static_cast<hipStream_t>(stream);
  const int64_t groups = num_seqs * H;
  const int64_t r = HV / H;
  if (dv % 64 == 0) {
    p.nvs = static_cast<int>(dv / 64);
    p.members = static_cast<int>(r * p.nvs);
    // the 12-wave kernel covers every (d_k, io, state) combination this entry
    // accepts; anything it declines is unsupported here as well
    const int rc = launch_chunk_chain(p, dk, io_dtype, state_dtype, groups, s);
    if (rc != GDN_ERR_UNSUPPORTED) return rc;
  } else if (dv == 32) {
    if (chunk_size != 64 || frames) {
      set_error("gdn_chunk_gated_delta_rule: dv = 32 takes chunk_size 64 and a plain state pool only");
      return GDN_ERR_UNSUPPORTED;
    }
    p.nvs = 1;
    p.members = static_cast<int>(r);
    if (dk == 128) return dispatch_types<128, 32>(p, io_dtype, state_dtype, groups, s);
    if (dk == 64) return dispatch_types<64, 32>(p, io_dtype, state_dtype, groups, s);
    if (dk == 32) return dispatch_types<32, 32>(p, io_dtype, state_dtype, groups, s);
  }
  set_error("gdn_chunk_gated_delta_rule: unsupported head dims dk=%lld dv=%lld (dk in {32,64,128}, dv 32 or "
            "a multiple of 64)", (long long)dk, (long long)dv);
  return GDN_ERR_UNSUPPORTED;
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
                                          const void* frames, int frames_dtype, int64_t frames_per_slot,
                                          int64_t frame_bytes, int64_t head_bytes, int64_t num_frames, void* out,
                                          void* v_new, float scale, void* stream) {
  return gdn::chunk_entry(q, k, v, io_dtype, g, beta, cu_seqlens, cu_dtype, num_seqs, total_tokens, H, HV, dk, dv,
                          state, state_dtype, slot_stride, layer_stride, head_stride, layer, read_slots, read_dtype,
                          chunk_write_slots, chunk_write_dtype, final_write_slots, final_write_dtype, chunk_size, frames,
                          frames_dtype, frames_per_slot, frame_bytes, head_bytes, num_frames, out, v_new, scale,
                          nullptr, stream);
}

extern "C" int gdn_chunk_gated_delta_rule_logged(
    const void* q, const void* k, const void* v, int io_dtype, const float* g, const float* beta,
    const void* cu_seqlens, int cu_dtype, int64_t num_seqs, int64_t total_tokens, int64_t H, int64_t HV, int64_t dk,
    int64_t dv, void* state, int state_dtype, int64_t layer, const void* read_slots, int read_dtype,
    const void* chunk_write_slots, int chunk_write_dtype, const void* final_write_slots, int final_write_dtype,
    int64_t chunk_size, const void* frames, int frames_dtype, int64_t frames_per_slot, int64_t frame_bytes,
    int64_t head_bytes, int64_t num_frames, const void* log_slots, int log_dtype, const void* token_offsets,
    int offsets_dtype, int64_t key_heads, int64_t num_layers, int64_t page_size, void* out, float scale,
    void* stream) {
  GDN_REQUIRE(frames, "gdn_chunk_gated_delta_rule_logged: the token log lives in frame storage");
  const gdn::LogArgs log{log_slots, log_dtype, token_offsets, offsets_dtype, key_heads, num_layers, page_size};
  return gdn::chunk_entry(q, k, v, io_dtype, g, beta, cu_seqlens, cu_dtype, num_seqs, total_tokens, H, HV, dk, dv,
                          state, state_dtype, 0, 0, 0, layer, read_slots, read_dtype, chunk_write_slots,
                          chunk_write_dtype, final_write_slots, final_write_dtype, chunk_size, frames, frames_dtype,
                          frames_per_slot, frame_bytes, head_bytes, num_frames, out, nullptr, scale, &log, stream);
}
