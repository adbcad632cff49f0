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
// Mapping: one workgroup (4 waves) per (sequence, v-head, 64-column slice of
// d_v), walking the sequence's chunks in order.  The fp32 state slice
// (d_k x 64) lives in MFMA accumulator registers for the whole sequence; a
// half-precision copy is staged in LDS as the B operand of the next chunk's
// products.  All dense products run on v_mfma_f32_16x16x32_f16 with fp32
// accumulation: operands are held in fp16 whatever the input dtype (bf16
// inputs convert exactly), because fp16's 10-bit mantissa keeps the carried
// fp32 state within 1e-3 of an fp32 recurrence where bf16 operands drift to
// ~4e-3, at the same MFMA rate.  Operand magnitudes must stay below 65504
// (values are saturated there).  The 16x16 diagonal blocks of the triangular
// inverse use fp32 forward substitution and the off-diagonal blocks fp32
// products (the reference solves in fp32 as well).
// Workgroups sharing a key head (HV/H v-heads x slices) get block ids that
// are equal modulo 8, so they land on the same XCD and share its L2 for q/k.
//
// Roofline: MFMA (16-bit).  Algorithmic flops per token per v-head:
// 10 C d + 6 d^2 + 2/3 C^2 (C = 64, d = 128).
#include "common.hpp"

namespace gdn {
namespace {

constexpr int kC = 64;
constexpr int kThreads = 256;
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
template <class T> __device__ __forceinline__ float from_bits(uint16_t b);
template <> __device__ __forceinline__ float from_bits<bf16>(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
template <> __device__ __forceinline__ float from_bits<f16>(uint16_t b) {
  return static_cast<float>(*reinterpret_cast<f16*>(&b));
}
__device__ __forceinline__ float op_val(uint16_t b) { return from_bits<f16>(b); }

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

// LDS carve-up (bytes).  Row paddings of 8 halfs keep 16-byte fragment reads
// of consecutive rows on different banks.
template <int DK, int DVS>
struct Smem {
  static constexpr int LDK = DK + 8;   // Kr, Qr: [64][LDK] token-major
  static constexpr int LDT = kC + 8;   // Ktd [DK][LDT], Ab/Mb [64][LDT], Rt/Vt [DVS][LDT]
  static constexpr int LDF = kC + 4;   // Lf/Af fp32 [64][LDF]
  static constexpr int LDV = DVS + 8;  // Vr [64][LDV]
  static constexpr int LDH = DK + 8;   // ht [DVS][LDH]
  static constexpr size_t kr = 0;
  static constexpr size_t qr = kr + 2ull * kC * LDK;
  static constexpr size_t ktd = qr + 2ull * kC * LDK;
  static constexpr size_t vr = ktd + 2ull * DK * LDT;
  static constexpr size_t ab = vr + 2ull * kC * LDV;
  static constexpr size_t mb = ab + 2ull * kC * LDT;
  static constexpr size_t rt = mb + 2ull * kC * LDT;
  static constexpr size_t vt = rt + 2ull * DVS * LDT;
  static constexpr size_t ht = vt + 2ull * DVS * LDT;
  static constexpr size_t lf = ht + 2ull * DVS * LDH;
  static constexpr size_t af = lf + 4ull * kC * LDF;
  static constexpr size_t tmp = af + 4ull * kC * LDF;  // 4 scratch 16x16 fp32 tiles
  static constexpr size_t gates = tmp + 4ull * 4 * 256;
  static constexpr size_t total = gates + 4ull * (4 * kC + 4);
};

struct ChunkParams {
  const void* q;
  const void* k;
  const void* v;
  const float* g;
  const float* beta;
  const void* cu;
  int cu_is64;
  int64_t N, T, H, HV, DV;
  void* state;
  int64_t slot_stride, layer_stride, head_stride, layer;
  const void* read_slots;
  int read_is64;
  const void* cw_slots;
  int cw_is64;
  const void* fw_slots;
  int fw_is64;
  void* out;
  void* v_new;
  float scale;
  int nvs;      // v slices per head
  int members;  // workgroups per (sequence, key head)
};

// 16-byte fragment: row (row0 + lane % 16), halfs k0 + 8 (lane / 16) .. + 7.
template <class IOT>
__device__ __forceinline__ typename Mma<IOT>::frag frag_at(const uint16_t* base, int ld, int row0, int k0, int lane) {
  return *reinterpret_cast<const typename Mma<IOT>::frag*>(base + (row0 + (lane & 15)) * ld + k0 + 8 * (lane >> 4));
}

// (X Y)[row][col0 .. col0+3] for 16x16 fp32 tiles, row = lane / 4, col0 = 4 (lane % 4).
__device__ __forceinline__ void mm16(const float* X, int ldx, const float* Y, int ldy, int lane, float (&acc)[4]) {
  const int row = lane >> 2, col0 = 4 * (lane & 3);
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) {
    const float x = X[row * ldx + kk];
    const float4 y = *reinterpret_cast<const float4*>(Y + kk * ldy + col0);
    acc[0] = fmaf(x, y.x, acc[0]);
    acc[1] = fmaf(x, y.y, acc[1]);
    acc[2] = fmaf(x, y.z, acc[2]);
    acc[3] = fmaf(x, y.w, acc[3]);
  }
}

template <class ST> __device__ __forceinline__ float load_st(const ST* p) { return to_f32(*p); }
template <class ST> __device__ __forceinline__ void store_st(ST* p, float v) { *p = from_f32<ST>(v); }

template <int DK, int DVS, class IOT, class ST>
__global__ __launch_bounds__(kThreads, 1) void chunk_kernel(ChunkParams p) {
  using SM = Smem<DK, DVS>;
  using M = Mma<f16>;
  constexpr int HT = DK / 16;         // h row tiles
  constexpr int CT = DVS / 16;        // column tiles of the slice
  constexpr int HTILES = HT * CT;     // h tiles, distributed t = wave + 4 i
  constexpr int HPW = (HTILES + 3) / 4;
  constexpr int PTILES = 8 * CT;      // [k; q] h tiles (128 rows)
  constexpr int PPW = PTILES / 4;
  constexpr int VTILES = 4 * CT;      // v' / o tiles (64 rows)
  constexpr int VPW = VTILES / 4;
  static_assert(PTILES % 4 == 0 && VTILES % 4 == 0, "tile split");

  __shared__ __align__(16) char smem[SM::total];
  uint16_t* Kr = reinterpret_cast<uint16_t*>(smem + SM::kr);
  uint16_t* Qr = reinterpret_cast<uint16_t*>(smem + SM::qr);
  uint16_t* Ktd = reinterpret_cast<uint16_t*>(smem + SM::ktd);
  uint16_t* Vr = reinterpret_cast<uint16_t*>(smem + SM::vr);
  uint16_t* Ab = reinterpret_cast<uint16_t*>(smem + SM::ab);
  uint16_t* Mb = reinterpret_cast<uint16_t*>(smem + SM::mb);
  uint16_t* Rt = reinterpret_cast<uint16_t*>(smem + SM::rt);
  uint16_t* Vt = reinterpret_cast<uint16_t*>(smem + SM::vt);
  uint16_t* Ht = reinterpret_cast<uint16_t*>(smem + SM::ht);
  float* Lf = reinterpret_cast<float*>(smem + SM::lf);
  float* Af = reinterpret_cast<float*>(smem + SM::af);
  float* Tmp = reinterpret_cast<float*>(smem + SM::tmp);
  float* gG = reinterpret_cast<float*>(smem + SM::gates);
  float* eG = gG + kC;
  float* eGl = eG + kC;
  float* bt = eGl + kC;
  float* misc = bt + kC;  // [0] = 2^G_last

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lr = lane & 15, lq = lane >> 4;

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

  const uint16_t* qg = static_cast<const uint16_t*>(p.q);
  const uint16_t* kg = static_cast<const uint16_t*>(p.k);
  const uint16_t* vg = static_cast<const uint16_t*>(p.v);
  uint16_t* og = static_cast<uint16_t*>(p.out);
  uint16_t* vng = static_cast<uint16_t*>(p.v_new);
  ST* pool = static_cast<ST*>(p.state);

  // upper off-diagonal tiles of A and M stay zero for the whole launch
  for (int e = tid; e < kC * kC; e += kThreads) {
    const int i = e / kC, j = e % kC;
    if (j > i) {
      Ab[i * SM::LDT + j] = 0;
      Mb[i * SM::LDT + j] = 0;
    }
  }

  // ---- initial state slice -> accumulators (tile t = wave + 4 i)
  f32x4 hacc[HPW];
  {
    const int64_t rs = load_index(p.read_slots, n, p.read_is64);
    const ST* src = rs >= 0 ? pool + rs * p.slot_stride + p.layer * p.layer_stride + h * p.head_stride : nullptr;
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
      const int t = wave + 4 * i;
#pragma unroll
      for (int e = 0; e < 4; ++e) hacc[i][e] = 0.f;
      if (t < HTILES && src) {
        const int row0 = (t / CT) * 16 + 4 * lq, col = (t % CT) * 16 + lr;
#pragma unroll
        for (int e = 0; e < 4; ++e) hacc[i][e] = load_st(src + (row0 + e) * p.DV + col_base + col);
      }
    }
  }
  auto stage_state = [&]() {  // bf16/f16 copy of h, column-major (B operand)
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
      const int t = wave + 4 * i;
      if (t < HTILES) {
        const int row0 = (t / CT) * 16 + 4 * lq, col = (t % CT) * 16 + lr;
        uint2 w;
        w.x = op_bits(hacc[i][0]) | (static_cast<uint32_t>(op_bits(hacc[i][1])) << 16);
        w.y = op_bits(hacc[i][2]) | (static_cast<uint32_t>(op_bits(hacc[i][3])) << 16);
        *reinterpret_cast<uint2*>(Ht + col * SM::LDH + row0) = w;
      }
    }
  };
  auto store_state_to = [&](int64_t slot_idx) {
    ST* dst = pool + slot_idx * p.slot_stride + p.layer * p.layer_stride + h * p.head_stride;
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
      const int t = wave + 4 * i;
      if (t < HTILES) {
        const int row0 = (t / CT) * 16 + 4 * lq, col = (t % CT) * 16 + lr;
#pragma unroll
        for (int e = 0; e < 4; ++e) store_st(dst + (row0 + e) * p.DV + col_base + col, hacc[i][e]);
      }
    }
  };
  stage_state();

  for (int64_t c = 0; c < nchunks; ++c) {
    const int64_t t0 = bos + c * kC;
    const int nv = static_cast<int>(len - c * kC < kC ? len - c * kC : kC);

    // ---- phase 0: chunk tiles -> LDS; gates (wave 0)
    {
      constexpr int KCH = DK / 8;  // 16-byte chunks per key row
      for (int e = tid; e < kC * KCH; e += kThreads) {
        const int row = e / KCH, ch = e % KCH;
        uint4 kv = make_uint4(0, 0, 0, 0), qv = kv;
        if (row < nv) {
          const int64_t off = ((t0 + row) * p.H + kh) * DK + ch * 8;
          kv = to_operands<IOT>(*reinterpret_cast<const uint4*>(kg + off));
          qv = to_operands<IOT>(*reinterpret_cast<const uint4*>(qg + off));
        }
        *reinterpret_cast<uint4*>(Kr + row * SM::LDK + ch * 8) = kv;
        *reinterpret_cast<uint4*>(Qr + row * SM::LDK + ch * 8) = qv;
      }
      constexpr int VCH = DVS / 8;
      for (int e = tid; e < kC * VCH; e += kThreads) {
        const int row = e / VCH, ch = e % VCH;
        uint4 vv = make_uint4(0, 0, 0, 0);
        if (row < nv)
          vv = to_operands<IOT>(
              *reinterpret_cast<const uint4*>(vg + ((t0 + row) * p.HV + h) * p.DV + col_base + ch * 8));
        *reinterpret_cast<uint4*>(Vr + row * SM::LDV + ch * 8) = vv;
      }
      if (wave == 0) {
        const bool ok = lane < nv;
        float x = ok ? p.g[(t0 + lane) * p.HV + h] : 0.f;
        const float b = ok ? p.beta[(t0 + lane) * p.HV + h] : 0.f;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const float y = __shfl_up(x, off, 64);
          if (lane >= off) x += y;
        }
        const float G = x * kRcpLn2;
        const float Glast = __shfl(G, nv - 1, 64);
        gG[lane] = G;
        eG[lane] = fast_exp2(G);
        eGl[lane] = ok ? fast_exp2(Glast - G) : 0.f;
        bt[lane] = b;
        if (lane == 0) misc[0] = fast_exp2(Glast);
      }
    }
    __syncthreads();

    // ---- phase 1: K Kt, Q Kt (lower tiles), [K; Q] h, decayed K^T
    for (int e = tid; e < DK * (kC / 2); e += kThreads) {
      const int d = e / (kC / 2), i = 2 * (e % (kC / 2));
      const float a = op_val(Kr[i * SM::LDK + d]) * eGl[i];
      const float b = op_val(Kr[(i + 1) * SM::LDK + d]) * eGl[i + 1];
      *reinterpret_cast<uint32_t*>(Ktd + d * SM::LDT + i) =
          op_bits(a) | (static_cast<uint32_t>(op_bits(b)) << 16);
    }
    for (int s = wave; s < 20; s += 4) {
      const bool is_q = s >= 10;
      int idx = is_q ? s - 10 : s;
      int ti = 0;
      while (idx > ti) { idx -= ti + 1; ++ti; }
      const int tj = idx;  // tj <= ti
      const uint16_t* X = is_q ? Qr : Kr;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k0 = 0; k0 < DK; k0 += 32)
        acc = M::run(frag_at<f16>(X, SM::LDK, ti * 16, k0, lane), frag_at<f16>(Kr, SM::LDK, tj * 16, k0, lane), acc);
      const int j = tj * 16 + lr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = ti * 16 + 4 * lq + e;
        const float decay = fast_exp2(fminf(gG[i] - gG[j], 0.f));
        if (is_q) {
          Mb[i * SM::LDT + j] = op_bits(i >= j ? acc[e] * decay : 0.f);
        } else {
          Lf[i * SM::LDF + j] = i > j ? bt[i] * acc[e] * decay : 0.f;
        }
      }
    }
    f32x4 pacc[PPW];
#pragma unroll
    for (int i = 0; i < PPW; ++i) {
      const int t = wave + 4 * i;
      const int ti = t / CT, tj = t % CT;
      const uint16_t* X = ti < 4 ? Kr : Qr;
      const int row0 = (ti & 3) * 16;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k0 = 0; k0 < DK; k0 += 32)
        acc = M::run(frag_at<f16>(X, SM::LDK, row0, k0, lane), frag_at<f16>(Ht, SM::LDH, tj * 16, k0, lane), acc);
      pacc[i] = acc;
      if (ti < 4) {  // R = beta (v - 2^G (k h)) -> Rt (column-major)
        const int col = tj * 16 + lr;
        float rv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = row0 + 4 * lq + e;
          rv[e] = bt[row] * (op_val(Vr[row * SM::LDV + col]) - eG[row] * acc[e]);
        }
        uint2 w;
        w.x = op_bits(rv[0]) | (static_cast<uint32_t>(op_bits(rv[1])) << 16);
        w.y = op_bits(rv[2]) | (static_cast<uint32_t>(op_bits(rv[3])) << 16);
        *reinterpret_cast<uint2*>(Rt + col * SM::LDT + row0 + 4 * lq) = w;
      }
    }
    __syncthreads();

    // ---- phase 2: A = (I + L)^-1 -- diagonal 16x16 blocks by forward substitution
    {
      const int blk = wave;
      if (lane < 16) {
        float x[16];
        const float* Lb = Lf + (blk * 16) * SM::LDF + blk * 16;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float v = (i == lane) ? 1.f : 0.f;
#pragma unroll
          for (int j = 0; j < i; ++j) v = fmaf(-Lb[i * SM::LDF + j], x[j], v);
          x[i] = v;
        }
        float* Ad = Af + (blk * 16) * SM::LDF + blk * 16;
        uint16_t* Bd = Ab + (blk * 16) * SM::LDT + blk * 16;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          Ad[i * SM::LDF + lane] = x[i];
          Bd[i * SM::LDT + lane] = op_bits(x[i]);
        }
      }
    }
    __syncthreads();
    // off-diagonal blocks: A_ij = -A_ii (sum_{k=j}^{i-1} L_ik A_kj), by block distance
    auto lblk = [&](int i, int j) { return Lf + (i * 16) * SM::LDF + j * 16; };
    auto ablk = [&](int i, int j) { return Af + (i * 16) * SM::LDF + j * 16; };
    auto finish = [&](int i, int j, const float* T) {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      mm16(ablk(i, i), SM::LDF, T, 16, lane, acc);
      const int row = lane >> 2, col0 = 4 * (lane & 3);
      float* Ad = ablk(i, j);
      uint16_t* Bd = Ab + (i * 16) * SM::LDT + j * 16;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        Ad[row * SM::LDF + col0 + e] = -acc[e];
        Bd[row * SM::LDT + col0 + e] = op_bits(-acc[e]);
      }
    };
    for (int dist = 1; dist < 4; ++dist) {
      const int count = 4 - dist;
      if (wave < count) {
        const int j = wave, i = wave + dist;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int k = j; k < i; ++k) mm16(lblk(i, k), SM::LDF, ablk(k, j), SM::LDF, lane, acc);
        float* T = Tmp + wave * 256;
        const int row = lane >> 2, col0 = 4 * (lane & 3);
#pragma unroll
        for (int e = 0; e < 4; ++e) T[row * 16 + col0 + e] = acc[e];
      }
      __syncthreads();
      if (wave < count) finish(wave + dist, wave, Tmp + wave * 256);
      __syncthreads();
    }

    // ---- phase 3: v' = A R  (tile t = wave + 4 i over 4 x CT)
#pragma unroll
    for (int i = 0; i < VPW; ++i) {
      const int t = wave + 4 * i;
      const int ti = t / CT, tj = t % CT;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k0 = 0; k0 < kC; k0 += 32)
        if (k0 <= ti * 16 + 15)
          acc = M::run(frag_at<f16>(Ab, SM::LDT, ti * 16, k0, lane), frag_at<f16>(Rt, SM::LDT, tj * 16, k0, lane), acc);
      const int col = tj * 16 + lr, row0 = ti * 16 + 4 * lq;
      uint2 w;
      w.x = op_bits(acc[0]) | (static_cast<uint32_t>(op_bits(acc[1])) << 16);
      w.y = op_bits(acc[2]) | (static_cast<uint32_t>(op_bits(acc[3])) << 16);
      *reinterpret_cast<uint2*>(Vt + col * SM::LDT + row0) = w;
      if (vng) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (row0 + e < nv) vng[((t0 + row0 + e) * p.HV + h) * p.DV + col_base + col] = bits_of<IOT>(acc[e]);
      }
    }
    __syncthreads();

    // ---- phase 4: o = scale (2^G q h + M v'); h <- 2^G_last h + Kd^T v'
#pragma unroll
    for (int i = 0; i < PPW; ++i) {
      const int t = wave + 4 * i;
      const int ti = t / CT, tj = t % CT;
      if (ti < 4) continue;
      const int qt = ti - 4;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k0 = 0; k0 < kC; k0 += 32)
        if (k0 <= qt * 16 + 15)
          acc = M::run(frag_at<f16>(Mb, SM::LDT, qt * 16, k0, lane), frag_at<f16>(Vt, SM::LDT, tj * 16, k0, lane), acc);
      const int col = tj * 16 + lr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = qt * 16 + 4 * lq + e;
        if (row < nv) {
          const float o = p.scale * (eG[row] * pacc[i][e] + acc[e]);
          og[((t0 + row) * p.HV + h) * p.DV + col_base + col] = bits_of<IOT>(o);
        }
      }
    }
    {
      const float gl = misc[0];
#pragma unroll
      for (int i = 0; i < HPW; ++i) {
        const int t = wave + 4 * i;
        if (t < HTILES) {
          const int ti = t / CT, tj = t % CT;
          f32x4 acc = hacc[i] * gl;
#pragma unroll
          for (int k0 = 0; k0 < kC; k0 += 32)
            acc = M::run(frag_at<f16>(Ktd, SM::LDT, ti * 16, k0, lane), frag_at<f16>(Vt, SM::LDT, tj * 16, k0, lane),
                         acc);
          hacc[i] = acc;
        }
      }
    }
    const int64_t cw = load_index(p.cw_slots, chunk_base + c, p.cw_is64);
    if (cw >= 0) store_state_to(cw);
    __syncthreads();  // all reads of Ht / chunk tiles done
    stage_state();
  }
  if (p.fw_slots) {
    const int64_t fw = load_index(p.fw_slots, n, p.fw_is64);
    if (fw >= 0) store_state_to(fw);
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

extern "C" int gdn_chunk_gated_delta_rule(const void* q, const void* k, const void* v, int io_dtype, const float* g,
                                          const float* beta, const void* cu_seqlens, int cu_dtype, int64_t num_seqs,
                                          int64_t total_tokens, int64_t H, int64_t HV, int64_t dk, int64_t dv,
                                          void* state, int state_dtype, int64_t slot_stride, int64_t layer_stride,
                                          int64_t head_stride, int64_t layer, const void* read_slots, int read_dtype,
                                          const void* chunk_write_slots, int chunk_write_dtype,
                                          const void* final_write_slots, int final_write_dtype, void* out,
                                          void* v_new, float scale, void* stream) {
  GDN_REQUIRE(num_seqs >= 0 && total_tokens >= 0 && H > 0 && HV > 0 && HV % H == 0,
              "gdn_chunk_gated_delta_rule: bad sizes");
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
  auto s = static_cast<hipStream_t>(stream);
  const int64_t groups = num_seqs * H;
  const int64_t r = HV / H;
  if (dv % 64 == 0) {
    p.nvs = static_cast<int>(dv / 64);
    p.members = static_cast<int>(r * p.nvs);
    if (dk == 128) return dispatch_types<128, 64>(p, io_dtype, state_dtype, groups, s);
    if (dk == 64) return dispatch_types<64, 64>(p, io_dtype, state_dtype, groups, s);
    if (dk == 32) return dispatch_types<32, 64>(p, io_dtype, state_dtype, groups, s);
  } else if (dv == 32) {
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
