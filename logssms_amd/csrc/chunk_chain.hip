// Chunked gated delta rule (chunk 64) over packed varlen sequences with
// state-pool I/O, with the recurrence chain held in registers.
//
// Algorithm (vendor/fla/gated_delta.py:15-82 and the kernels it chains):
//   G  = chunk-local cumsum(g) / ln 2                            (cumsum.py:19-75)
//   L  = strict_tril(beta_i k_i.k_j 2^(G_i - G_j))                (chunk_fwd.py:26-294)
//   R  = beta (v - 2^G (k h))                                     (wy_fast.py, chunk_delta_h.py:162-181)
//   v' = (I + L)^-1 R                                             (= U - W h)
//   o  = scale (2^G (q h) + tril_incl(q k^T 2^(G_i - G_j)) v')    (chunk_o.py:85-130)
//   h <- 2^G_last h + (2^(G_last - G) k)^T v'                     (chunk_delta_h.py:194-224)
// The solve uses the 2x2 split of the 64-token chunk into 32-token halves:
//   v'_top = A11 R_top,  v'_bot = A22 (R_bot - L21 v'_top),  A_ii = (I + L_ii)^-1,
// so only the two 32x32 diagonal inverses are formed off the chain.
//
// Mapping: one workgroup per (sequence, v-head, 64-column slice of d_v); 8 waves.
//   * Chain waves 0-3: wave j owns state columns 16j..16j+15 for the whole
//     sequence, as fp32 MFMA accumulator tiles.  Every product of the chain
//     takes its right operand straight from accumulator registers: the k index
//     of each 32-deep product is ordered so that lane group g holds rows
//     4g..4g+3 and 16+4g..16+4g+3 of the block -- exactly the rows a C-layout
//     tile pair holds -- and the left operand (K, Q, A, M or K^T rows in LDS)
//     is read in that same order.  Per chunk: P = K h and Q h, R, v', o (M v'
//     added), h update; nothing but the output goes through LDS.
//   * Side waves 4-7 prepare chunk c+1 while the chain runs chunk c: k k^T and
//     q k^T tiles with the decay masks (L, the masked M), the 16x16 diagonal
//     inverses (fp32 forward substitution), the two off-diagonal blocks of
//     A11/A22 (split-f16 products, ~fp32 accurate), the d-major copy of K the
//     state update reads, and the staging / global prefetch of later chunks.
// Two workgroup barriers per chunk (LDS-only waits, so global prefetches stay
// in flight).  MFMA operands are f16 (bf16 inputs convert exactly; values
// saturate at +-65504) with fp32 accumulation.
//
// Roofline: MFMA (16-bit).  Algorithmic flops per token per v-head:
// 10 C d + 6 d^2 + 2/3 C^2 (C = 64, d = 128).
#include "chunk_common.hpp"

namespace gdn {
namespace {

constexpr int kC = 64;
constexpr int kThreads = 512;
constexpr float kRcpLn2 = 1.4426950216f;  // gated_delta.py:12

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int LDA = kC + 8;  // row stride (halfs) of the A and M tiles
constexpr int LDT = kC + 4;  // row stride (halfs) of the d-major K and column-major V tiles
constexpr int LDB = 20;      // row stride (floats) of fp32 16x16 blocks
constexpr int BLK = 16 * LDB + 16;  // block stride: consecutive blocks start 16 banks apart
// Gate table per chunk (floats): G, 2^G, 2^(G_last - G) (0 past the end),
// beta, then 2^G_last.
constexpr int GTS = 264;
constexpr int G_EXP = 64, G_DEC = 128, G_BETA = 192, G_LAST = 256;

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void wave_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ f4_t mma(h8_t a, h8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4_t zero4() { return f4_t{0.f, 0.f, 0.f, 0.f}; }

__device__ __forceinline__ _Float16 to_op(float x) {
  return static_cast<_Float16>(__builtin_amdgcn_fmed3f(x, -65504.f, 65504.f));
}
// Left operand, row `row` of a row-major f16 matrix, k block at column k0.
__device__ __forceinline__ h8_t afrag(const _Float16* base, int ld, int row, int k0, int g) {
  const _Float16* p = base + row * ld + k0 + 4 * g;
  const h4_t lo = *reinterpret_cast<const h4_t*>(p);
  const h4_t hi = *reinterpret_cast<const h4_t*>(p + 16);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}
// Right operand from two C-layout accumulator tiles (rows 0-15, rows 16-31).
__device__ __forceinline__ h8_t bfrag(f4_t a, f4_t b) {
  h8_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    o[e] = to_op(a[e]);
    o[4 + e] = to_op(b[e]);
  }
  return o;
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
template <class IOT> __device__ __forceinline__ uint16_t out_bits(float x);
template <> __device__ __forceinline__ uint16_t out_bits<bf16>(float x) { return f32_to_bf16_bits(x); }
template <> __device__ __forceinline__ uint16_t out_bits<f16>(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

// ---- split-f16 products of fp32 16x16 blocks (x = hi + lo; the product
// drops lo*lo).  Standard operand layout, second half of k zero.
struct Split {
  h8_t hi, lo;
};
__device__ __forceinline__ Split split8(const float (&x)[8]) {
  Split s;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const _Float16 h = static_cast<_Float16>(x[e]);
    s.hi[e] = h;
    s.lo[e] = static_cast<_Float16>(x[e] - static_cast<float>(h));
  }
  return s;
}
__device__ __forceinline__ Split a_block(const float* X, int lane) {
  float x[8];
  const int row = lane & 15, kq = lane >> 4;
  if (kq < 2) {
    const float4 a = *reinterpret_cast<const float4*>(X + row * LDB + 8 * kq);
    const float4 b = *reinterpret_cast<const float4*>(X + row * LDB + 8 * kq + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = 0.f;
  }
  return split8(x);
}
__device__ __forceinline__ Split b_block(const float* Y, int lane) {
  float x[8];
  const int col = lane & 15, kq = lane >> 4;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = kq < 2 ? Y[(8 * kq + e) * LDB + col] : 0.f;
  return split8(x);
}
__device__ __forceinline__ f4_t mma_split(const Split& a, const Split& b) {
  f4_t c = mma(a.hi, b.hi, zero4());
  c = mma(a.hi, b.lo, c);
  return mma(a.lo, b.hi, c);
}

template <class ST> __device__ __forceinline__ float load_st(const ST* p) { return to_f32(*p); }
template <class ST> __device__ __forceinline__ void store_st(ST* p, float v) { *p = from_f32<ST>(v); }

// Side-thread staging blocks: a thread moves 4 tokens x 8 columns.  Within a
// wave, lane l takes token block (l & 3) + 4 ((l >> 4) & 1) and column block
// ((l >> 2) & 3) + 4 (l >> 5) of an 8 x 8 patch, which keeps both the 16-byte
// row accesses (4 passes of 16 lanes) and the 8-byte transposed accesses
// (2 passes of 32 lanes) free of LDS bank conflicts for the row strides used
// here (136 B token rows, 136 B transposed rows).
struct Blk {
  int tb, db;
};
__device__ __forceinline__ Blk staging_block(int idx, int ndb) {
  const int w = idx >> 6, l = idx & 63;
  if (ndb >= 8) return {8 * (w & 1) + (l & 3) + 4 * ((l >> 4) & 1), 8 * (w >> 1) + ((l >> 2) & 3) + 4 * (l >> 5)};
  return {(l & 3) + 4 * (l >> 4), (l >> 2) & 3};
}

template <int DK, class IOT, class ST>
__global__ __launch_bounds__(kThreads, 1) void chunk_chain_kernel(ChunkParams p) {
  constexpr int HT = DK / 16;   // 16-row state tiles
  constexpr int KS = DK / 32;   // 32-deep k steps over d_k
  constexpr int LDK = DK + 8;   // K / Q row stride (halfs)
  constexpr int DB = DK / 8;    // 8-column blocks of a K row
  constexpr int KBLK = 16 * DB; // K (Q) staging blocks per chunk
  static_assert(KS >= 1, "d_k >= 32");

  __shared__ __align__(16) _Float16 sKx[2 * kC * LDK];
  __shared__ __align__(16) _Float16 sQx[2 * kC * LDK];
  __shared__ __align__(16) _Float16 sKt[DK * LDT];     // K of the running chunk, d-major
  __shared__ __align__(16) _Float16 sVt[64 * LDT];     // V of the running chunk, column-major
  __shared__ __align__(16) _Float16 sA[2 * kC * LDA];  // [A11 | 0 ; -L21 | A22]
  __shared__ __align__(16) _Float16 sM[2 * kC * LDA];  // tril_incl(q k^T 2^(G_i - G_j))
  __shared__ __align__(16) float sG[3 * GTS];
  __shared__ __align__(16) float sL[6 * BLK];   // L diagonal blocks 0-3, L_10, L_32
  __shared__ __align__(16) float sAf[4 * BLK];  // fp32 inverses of the diagonal blocks
  __shared__ __align__(16) float sT[2 * BLK];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;

  // ---- block -> (sequence, key head, member); members of one key head share an XCD
  const int64_t Lb = blockIdx.x;
  const int64_t slot = Lb / 8;
  const int64_t group = (slot / p.members) * 8 + (Lb % 8);
  if (group >= p.N * p.H) return;
  const int member = static_cast<int>(slot % p.members);
  const int64_t n = group / p.H;
  const int64_t kh = group % p.H;
  const int64_t h = kh * (p.HV / p.H) + member / p.nvs;
  const int64_t col_base = static_cast<int64_t>(member % p.nvs) * 64;

  const int64_t bos = load_index(p.cu, n, p.cu_is64);
  const int64_t len = load_index(p.cu, n + 1, p.cu_is64) - bos;
  const int64_t nchunks = (len + kC - 1) / kC;
  auto valid_rows = [&](int64_t c) -> int {
    const int64_t rem = len - c * kC;
    return rem <= 0 ? 0 : (rem < kC ? static_cast<int>(rem) : kC);
  };

  ST* pool = static_cast<ST*>(p.state);
  const int64_t head_off = p.layer * p.layer_stride + h * p.head_stride + col_base;
  const int j = wave;  // chain wave: state columns 16j..16j+15
  f4_t hT[HT];
  auto load_state = [&]() {
    const int64_t rs = load_index(p.read_slots, n, p.read_is64);
    const ST* src = rs >= 0 ? pool + rs * p.slot_stride + head_off + 16 * j + lr : nullptr;
#pragma unroll
    for (int ti = 0; ti < HT; ++ti)
#pragma unroll
      for (int e = 0; e < 4; ++e) hT[ti][e] = src ? load_st(src + (16 * ti + 4 * lg + e) * p.DV) : 0.f;
  };
  auto store_state = [&](int64_t slot_idx) {
    ST* dst = pool + slot_idx * p.slot_stride + head_off + 16 * j + lr;
#pragma unroll
    for (int ti = 0; ti < HT; ++ti)
#pragma unroll
      for (int e = 0; e < 4; ++e) store_st(dst + (16 * ti + 4 * lg + e) * p.DV, hT[ti][e]);
  };

  if (nchunks == 0) {  // empty sequence: the final state is the initial state
    if (wave < 4 && p.fw_slots) {
      const int64_t fw = load_index(p.fw_slots, n, p.fw_is64);
      if (fw >= 0) {
        load_state();
        store_state(fw);
      }
    }
    return;
  }
  int64_t chunk_base = 0;
  for (int64_t m = 0; m < n; ++m) {
    const int64_t lm = load_index(p.cu, m + 1, p.cu_is64) - load_index(p.cu, m, p.cu_is64);
    chunk_base += (lm + kC - 1) / kC;
  }

  // A and M start zero: their upper blocks are never written.
  for (int e = tid; e < 2 * kC * LDA / 8; e += kThreads) {
    reinterpret_cast<uint4*>(sA)[e] = make_uint4(0, 0, 0, 0);
    reinterpret_cast<uint4*>(sM)[e] = make_uint4(0, 0, 0, 0);
  }

  if (wave < 4) {
    // ==================================================================== chain waves
    uint16_t* og = static_cast<uint16_t*>(p.out) + (bos * p.HV + h) * p.DV + col_base + 16 * j;
    uint16_t* vng = p.v_new ? static_cast<uint16_t*>(p.v_new) + (bos * p.HV + h) * p.DV + col_base + 16 * j : nullptr;
    const int64_t tok_stride = p.HV * p.DV;
    load_state();
    lds_barrier();  // P0
    lds_barrier();  // P1
    lds_barrier();  // B(0)
    for (int64_t c = 0; c < nchunks; ++c) {
      const int nv = valid_rows(c);
      const _Float16* K = sKx + (c & 1) * kC * LDK;
      const _Float16* Q = sQx + (c & 1) * kC * LDK;
      const float* gt = sG + (c % 3) * GTS;
      // ---- S1: P = K h;  O^T = h^T Q^T (token columns);  R = beta (v - 2^G P)
      f4_t P[4], Ot[4], R[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) P[i] = Ot[i] = zero4();
#pragma unroll
      for (int m = 0; m < KS; ++m) {
        const h8_t hb = bfrag(hT[2 * m], hT[2 * m + 1]);  // also the left operand of h^T
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          P[i] = mma(afrag(K, LDK, 16 * i + lr, 32 * m, lg), hb, P[i]);
          Ot[i] = mma(hb, afrag(Q, LDK, 16 * i + lr, 32 * m, lg), Ot[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t0 = 16 * i + 4 * lg;
        const f4_t e4 = *reinterpret_cast<const f4_t*>(gt + G_EXP + t0);
        const f4_t b4 = *reinterpret_cast<const f4_t*>(gt + G_BETA + t0);
        const h4_t v4 = *reinterpret_cast<const h4_t*>(sVt + (16 * j + lr) * LDT + t0);
#pragma unroll
        for (int e = 0; e < 4; ++e) R[i][e] = b4[e] * (static_cast<float>(v4[e]) - e4[e] * P[i][e]);
        Ot[i] *= gt[G_EXP + 16 * i + lr];
      }
      lds_barrier();  // M(c)
      // ---- S2: v'_top = A11 R_top; R_bot -= L21 v'_top; v'_bot = A22 R_bot
      const _Float16* A = sA + (c & 1) * kC * LDA;
      f4_t V[4];
      {
        const h8_t rb0 = bfrag(R[0], R[1]);
        V[0] = mma(afrag(A, LDA, lr, 0, lg), rb0, zero4());
        V[1] = mma(afrag(A, LDA, 16 + lr, 0, lg), rb0, zero4());
      }
      const h8_t vb0 = bfrag(V[0], V[1]);  // also the left operand of v'^T
      R[2] = mma(afrag(A, LDA, 32 + lr, 0, lg), vb0, R[2]);  // rows 32-63, cols 0-31 hold -L21
      R[3] = mma(afrag(A, LDA, 48 + lr, 0, lg), vb0, R[3]);
      {
        const h8_t rb1 = bfrag(R[2], R[3]);
        V[2] = mma(afrag(A, LDA, 32 + lr, 32, lg), rb1, zero4());
        V[3] = mma(afrag(A, LDA, 48 + lr, 32, lg), rb1, zero4());
      }
      const h8_t vb1 = bfrag(V[2], V[3]);
      // ---- S3a: o^T += v'^T M^T; lane holds 4 consecutive output columns of one token
      const _Float16* M = sM + (c & 1) * kC * LDA;
#pragma unroll
      for (int i = 0; i < 4; ++i) Ot[i] = mma(vb0, afrag(M, LDA, 16 * i + lr, 0, lg), Ot[i]);
      Ot[2] = mma(vb1, afrag(M, LDA, 32 + lr, 32, lg), Ot[2]);
      Ot[3] = mma(vb1, afrag(M, LDA, 48 + lr, 32, lg), Ot[3]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * i + lr;
        if (t < nv) {
          uint2 w;
          w.x = out_bits<IOT>(p.scale * Ot[i][0]) | (static_cast<uint32_t>(out_bits<IOT>(p.scale * Ot[i][1])) << 16);
          w.y = out_bits<IOT>(p.scale * Ot[i][2]) | (static_cast<uint32_t>(out_bits<IOT>(p.scale * Ot[i][3])) << 16);
          *reinterpret_cast<uint2*>(og + (c * kC + t) * tok_stride + 4 * lg) = w;
        }
      }
      if (vng) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int t = 16 * i + 4 * lg + e;
            if (t < nv) vng[(c * kC + t) * tok_stride + lr] = out_bits<IOT>(V[i][e]);
          }
      }
      // ---- S3b: h <- 2^G_last h + K^T (2^(G_last - G) v')
      {
        f4_t Vd[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) Vd[i] = V[i] * *reinterpret_cast<const f4_t*>(gt + G_DEC + 16 * i + 4 * lg);
        const h8_t db0 = bfrag(Vd[0], Vd[1]);
        const h8_t db1 = bfrag(Vd[2], Vd[3]);
        const float gl = gt[G_LAST];
#pragma unroll
        for (int ti = 0; ti < HT; ++ti) {
          f4_t acc = hT[ti] * gl;
          acc = mma(afrag(sKt, LDT, 16 * ti + lr, 0, lg), db0, acc);
          hT[ti] = mma(afrag(sKt, LDT, 16 * ti + lr, 32, lg), db1, acc);
        }
      }
      const int64_t cw = load_index(p.cw_slots, chunk_base + c, p.cw_is64);
      if (cw >= 0) store_state(cw);
      lds_barrier();  // B(c+1)
    }
    if (p.fw_slots) {
      const int64_t fw = load_index(p.fw_slots, n, p.fw_is64);
      if (fw >= 0) store_state(fw);
    }
  } else {
    // ==================================================================== side waves
    const int sw = wave - 4, st = tid - 256;
    const bool kq_thread = st < KBLK;
    const Blk kb = staging_block(st, DB);
    const bool v_thread = st >= 128;  // waves 6, 7: 4 tokens x 8 columns of the 64-column V slice
    const Blk vb = staging_block(st - 128, 8);
    const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + ((bos + 4 * kb.tb) * p.H + kh) * DK + 8 * kb.db;
    const uint16_t* qbase = static_cast<const uint16_t*>(p.q) + ((bos + 4 * kb.tb) * p.H + kh) * DK + 8 * kb.db;
    const uint16_t* vbase =
        static_cast<const uint16_t*>(p.v) + ((bos + 4 * vb.tb) * p.HV + h) * p.DV + col_base + 8 * vb.db;
    const int64_t krow = p.H * DK, kstride = kC * krow;
    const int64_t vrow = p.HV * p.DV, vstride = kC * vrow;
    const int gtid = st - 192;  // wave 7 carries the gates
    uint4 pk[4], pq[4], pv[4];
    float pgate = 0.f, pbeta = 0.f;

    auto prefetch_kq = [&](int64_t ck) {
      const int nk = valid_rows(ck);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        pk[u] = pq[u] = make_uint4(0, 0, 0, 0);
        if (kq_thread && 4 * kb.tb + u < nk) {
          pk[u] = *reinterpret_cast<const uint4*>(kbase + ck * kstride + u * krow);
          pq[u] = *reinterpret_cast<const uint4*>(qbase + ck * kstride + u * krow);
        }
      }
      if (sw == 3) {
        const bool ok = gtid < nk;
        const int64_t off = (bos + ck * kC + (ok ? gtid : 0)) * p.HV + h;
        pgate = ok ? p.g[off] : 0.f;
        pbeta = ok ? p.beta[off] : 0.f;
      }
    };
    auto prefetch_v = [&](int64_t cv) {
      const int nk = valid_rows(cv);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        pv[u] = make_uint4(0, 0, 0, 0);
        if (v_thread && 4 * vb.tb + u < nk) pv[u] = *reinterpret_cast<const uint4*>(vbase + cv * vstride + u * vrow);
      }
    };
    auto stage_kq = [&](int64_t ck) {
      if (kq_thread) {
        _Float16* kd = sKx + (ck & 1) * kC * LDK + (4 * kb.tb) * LDK + 8 * kb.db;
        _Float16* qd = sQx + (ck & 1) * kC * LDK + (4 * kb.tb) * LDK + 8 * kb.db;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          *reinterpret_cast<uint4*>(kd + u * LDK) = to_f16x8<IOT>(pk[u]);
          *reinterpret_cast<uint4*>(qd + u * LDK) = to_f16x8<IOT>(pq[u]);
        }
      }
      if (sw == 3) {  // chunk-local cumulative gate in log2 units (cumsum.py:19-75)
        const int nk = valid_rows(ck);
        float x = pgate;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const float y = __shfl_up(x, off, 64);
          if (gtid >= off) x += y;
        }
        const float G = x * kRcpLn2;
        const float Gl = __shfl(G, nk > 0 ? nk - 1 : 0, 64);
        float* gt = sG + (ck % 3) * GTS;
        gt[gtid] = G;
        gt[G_EXP + gtid] = fast_exp2(G);
        gt[G_DEC + gtid] = gtid < nk ? fast_exp2(Gl - G) : 0.f;
        gt[G_BETA + gtid] = pbeta;
        if (gtid == 0) gt[G_LAST] = fast_exp2(Gl);
      }
    };
    // 4 token rows x 8 columns (registers, raw) -> 8 column rows x 4 tokens (f16)
    auto write_transposed = [&](_Float16* dst, const uint4 (&rows)[4], int tb, int db) {
      h8_t r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) r[u] = __builtin_bit_cast(h8_t, to_f16x8<IOT>(rows[u]));
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const h4_t w = {r[0][d], r[1][d], r[2][d], r[3][d]};
        *reinterpret_cast<h4_t*>(dst + (8 * db + d) * LDT + 4 * tb) = w;
      }
    };
    auto stage_v = [&]() {
      if (v_thread) write_transposed(sVt, pv, vb.tb, vb.db);
    };
    // d-major copy of K(ck) for the state update, read back from the f16 K rows.
    auto stage_kt = [&](int64_t ck) {
      if (kq_thread) {
        const _Float16* src = sKx + (ck & 1) * kC * LDK + (4 * kb.tb) * LDK + 8 * kb.db;
        h8_t r[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) r[u] = *reinterpret_cast<const h8_t*>(src + u * LDK);
#pragma unroll
        for (int d = 0; d < 8; ++d) {
          const h4_t w = {r[0][d], r[1][d], r[2][d], r[3][d]};
          *reinterpret_cast<h4_t*>(sKt + (8 * kb.db + d) * LDT + 4 * kb.tb) = w;
        }
      }
    };

    // First half of the solve for chunk nc: tiles (transposed: lane = one row
    // t, 4 consecutive columns s), masks, diagonal inverses.
    auto solve_front = [&](int64_t nc) {
      const _Float16* K = sKx + (nc & 1) * kC * LDK;
      const _Float16* Q = sQx + (nc & 1) * kC * LDK;
      const float* gt = sG + (nc % 3) * GTS;
      _Float16* A = sA + (nc & 1) * kC * LDA;
      _Float16* M = sM + (nc & 1) * kC * LDA;
      // tile (ti, tj) entry for row t = 16 ti + lr, columns s = 16 tj + 4 lg + e
      auto decays = [&](int ti, int tj) {
        const f4_t gs = *reinterpret_cast<const f4_t*>(gt + 16 * tj + 4 * lg);
        const float gti = gt[16 * ti + lr];
        f4_t d;
#pragma unroll
        for (int e = 0; e < 4; ++e) d[e] = fast_exp2(fminf(gti - gs[e], 0.f));
        return d;
      };
      auto lmask = [&](f4_t s, int ti, int tj) {
        const f4_t d = decays(ti, tj);
        const float bt = gt[G_BETA + 16 * ti + lr];
#pragma unroll
        for (int e = 0; e < 4; ++e) s[e] = (16 * ti + lr > 16 * tj + 4 * lg + e) ? bt * s[e] * d[e] : 0.f;
        return s;
      };
      auto store_blockf = [&](float* B, f4_t v) { *reinterpret_cast<f4_t*>(B + lr * LDB + 4 * lg) = v; };
      auto store_h4 = [&](_Float16* X, int ti, int tj, f4_t v) {
        const h4_t w = {to_op(v[0]), to_op(v[1]), to_op(v[2]), to_op(v[3])};
        *reinterpret_cast<h4_t*>(X + (16 * ti + lr) * LDA + 16 * tj + 4 * lg) = w;
      };
      auto mstore = [&](f4_t s, int ti, int tj) {
        const f4_t d = decays(ti, tj);
#pragma unroll
        for (int e = 0; e < 4; ++e) s[e] = (16 * ti + lr >= 16 * tj + 4 * lg + e) ? s[e] * d[e] : 0.f;
        store_h4(M, ti, tj, s);
      };
      // transposed tile (ti, tj) of X K^T: left operand K rows of tj, right X rows of ti
      if (sw == 0) {
        f4_t dg[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) dg[b] = zero4();
#pragma unroll
        for (int m = 0; m < KS; ++m)
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const h8_t kf = afrag(K, LDK, 16 * b + lr, 32 * m, lg);
            dg[b] = mma(kf, kf, dg[b]);
          }
#pragma unroll
        for (int b = 0; b < 4; ++b) store_blockf(sL + b * BLK, lmask(dg[b], b, b));
        wave_sync();
        // (I + L_bb)^-1 by forward substitution; lane = (block, column)
        const int b = lane >> 4, col = lane & 15;
        const float* Lbb = sL + b * BLK;
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float a0 = (i == col) ? 1.f : 0.f, a1 = 0.f;
#pragma unroll
          for (int jj = 0; jj < i; jj += 2) {
            a0 = fmaf(-Lbb[i * LDB + jj], x[jj], a0);
            if (jj + 1 < i) a1 = fmaf(-Lbb[i * LDB + jj + 1], x[jj + 1], a1);
          }
          x[i] = a0 + a1;
        }
        float* Ab = sAf + b * BLK;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          Ab[i * LDB + col] = x[i];
          A[(16 * b + i) * LDA + 16 * b + col] = to_op(x[i]);
        }
      } else if (sw == 1) {
        f4_t s10 = zero4(), s32 = zero4(), s20 = zero4(), s21 = zero4(), s30 = zero4(), s31 = zero4();
#pragma unroll
        for (int m = 0; m < KS; ++m) {
          const h8_t k0 = afrag(K, LDK, lr, 32 * m, lg);
          const h8_t k1 = afrag(K, LDK, 16 + lr, 32 * m, lg);
          const h8_t k2 = afrag(K, LDK, 32 + lr, 32 * m, lg);
          const h8_t k3 = afrag(K, LDK, 48 + lr, 32 * m, lg);
          s10 = mma(k0, k1, s10);
          s32 = mma(k2, k3, s32);
          s20 = mma(k0, k2, s20);
          s21 = mma(k1, k2, s21);
          s30 = mma(k0, k3, s30);
          s31 = mma(k1, k3, s31);
        }
        store_blockf(sL + 4 * BLK, lmask(s10, 1, 0));
        store_blockf(sL + 5 * BLK, lmask(s32, 3, 2));
        store_h4(A, 2, 0, -lmask(s20, 2, 0));
        store_h4(A, 2, 1, -lmask(s21, 2, 1));
        store_h4(A, 3, 0, -lmask(s30, 3, 0));
        store_h4(A, 3, 1, -lmask(s31, 3, 1));
      } else if (sw == 2) {
        f4_t m00 = zero4(), m10 = zero4(), m11 = zero4(), m20 = zero4(), m21 = zero4();
#pragma unroll
        for (int m = 0; m < KS; ++m) {
          const h8_t q0 = afrag(Q, LDK, lr, 32 * m, lg);
          const h8_t q1 = afrag(Q, LDK, 16 + lr, 32 * m, lg);
          const h8_t q2 = afrag(Q, LDK, 32 + lr, 32 * m, lg);
          const h8_t k0 = afrag(K, LDK, lr, 32 * m, lg);
          const h8_t k1 = afrag(K, LDK, 16 + lr, 32 * m, lg);
          m00 = mma(k0, q0, m00);
          m10 = mma(k0, q1, m10);
          m11 = mma(k1, q1, m11);
          m20 = mma(k0, q2, m20);
          m21 = mma(k1, q2, m21);
        }
        mstore(m00, 0, 0);
        mstore(m10, 1, 0);
        mstore(m11, 1, 1);
        mstore(m20, 2, 0);
        mstore(m21, 2, 1);
      } else {
        f4_t m22 = zero4(), m30 = zero4(), m31 = zero4(), m32 = zero4(), m33 = zero4();
#pragma unroll
        for (int m = 0; m < KS; ++m) {
          const h8_t q2 = afrag(Q, LDK, 32 + lr, 32 * m, lg);
          const h8_t q3 = afrag(Q, LDK, 48 + lr, 32 * m, lg);
          const h8_t k0 = afrag(K, LDK, lr, 32 * m, lg);
          const h8_t k1 = afrag(K, LDK, 16 + lr, 32 * m, lg);
          const h8_t k2 = afrag(K, LDK, 32 + lr, 32 * m, lg);
          const h8_t k3 = afrag(K, LDK, 48 + lr, 32 * m, lg);
          m22 = mma(k2, q2, m22);
          m30 = mma(k0, q3, m30);
          m31 = mma(k1, q3, m31);
          m32 = mma(k2, q3, m32);
          m33 = mma(k3, q3, m33);
        }
        mstore(m22, 2, 2);
        mstore(m30, 3, 0);
        mstore(m31, 3, 1);
        mstore(m32, 3, 2);
        mstore(m33, 3, 3);
      }
    };
    // Second half: A_{j+1,j} = -A_{j+1,j+1} L_{j+1,j} A_jj for j = 0 (wave 4) and j = 2 (wave 5).
    auto solve_back = [&](int64_t nc) {
      if (sw < 2) {
        const int jb = 2 * sw;
        float* T = sT + sw * BLK;
        const f4_t t = mma_split(a_block(sL + (4 + sw) * BLK, lane), b_block(sAf + jb * BLK, lane));
#pragma unroll
        for (int e = 0; e < 4; ++e) T[(4 * lg + e) * LDB + lr] = t[e];
        wave_sync();
        const f4_t a = mma_split(a_block(sAf + (jb + 1) * BLK, lane), b_block(T, lane));
        _Float16* A = sA + (nc & 1) * kC * LDA;
#pragma unroll
        for (int e = 0; e < 4; ++e) A[(16 * (jb + 1) + 4 * lg + e) * LDA + 16 * jb + lr] = to_op(-a[e]);
      }
    };

    // ---- prologue: chunks 0 and 1 staged, chunk 0 solved
    prefetch_kq(0);
    prefetch_v(0);
    stage_kq(0);
    stage_v();
    if (nchunks > 1) {
      prefetch_kq(1);
      prefetch_v(1);
      stage_kq(1);
    }
    if (nchunks > 2) prefetch_kq(2);
    lds_barrier();  // P0
    solve_front(0);
    lds_barrier();  // P1
    solve_back(0);
    lds_barrier();  // B(0)
    for (int64_t c = 0; c < nchunks; ++c) {
      if (c + 1 < nchunks) solve_front(c + 1);
      stage_kt(c);
      lds_barrier();  // M(c)
      if (c + 1 < nchunks) {
        solve_back(c + 1);
        stage_v();
      }
      if (c + 2 < nchunks) stage_kq(c + 2);
      if (c + 3 < nchunks) prefetch_kq(c + 3);
      if (c + 2 < nchunks) prefetch_v(c + 2);
      lds_barrier();  // B(c+1)
    }
  }
}

template <int DK, class IOT, class ST>
int launch_typed(const ChunkParams& p, int64_t groups, hipStream_t stream) {
  const int64_t blocks = ((groups + 7) / 8) * 8 * p.members;
  if (blocks > 0x7fffffff) {
    set_error("gdn_chunk_gated_delta_rule: grid too large");
    return GDN_ERR_INVALID;
  }
  hipLaunchKernelGGL((chunk_chain_kernel<DK, IOT, ST>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                     stream, p);
  return GDN_LAUNCH_CHECK("gdn_chunk_gated_delta_rule launch");
}

template <int DK>
int launch_dk(const ChunkParams& p, int io, int st, int64_t groups, hipStream_t s) {
  if (io == GDN_BF16 && st == GDN_F32) return launch_typed<DK, bf16, float>(p, groups, s);
  if (io == GDN_BF16 && st == GDN_BF16) return launch_typed<DK, bf16, bf16>(p, groups, s);
  if (io == GDN_F16 && st == GDN_F32) return launch_typed<DK, f16, float>(p, groups, s);
  if (io == GDN_F16 && st == GDN_F16) return launch_typed<DK, f16, f16>(p, groups, s);
  return GDN_ERR_UNSUPPORTED;
}

}  // namespace

int launch_chunk_chain(const ChunkParams& p, int64_t dk, int io_dtype, int state_dtype, int64_t groups,
                       hipStream_t stream) {
  if (p.DV % 64 != 0) return GDN_ERR_UNSUPPORTED;
  if (dk == 128) return launch_dk<128>(p, io_dtype, state_dtype, groups, stream);
  if (dk == 64) return launch_dk<64>(p, io_dtype, state_dtype, groups, stream);
  if (dk == 32) return launch_dk<32>(p, io_dtype, state_dtype, groups, stream);
  return GDN_ERR_UNSUPPORTED;
}

}  // namespace gdn
