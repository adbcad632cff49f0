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
// The solve splits the 64-token chunk into 32-token halves:
//   v'_top = A11 R_top,  v'_bot = A22 (R_bot - L21 v'_top),  A_ii = (I + L_ii)^-1,
// and each 32x32 inverse is formed from its 16x16 blocks, L = [D0 0; O D1]:
//   (I + L)^-1 = [A0 0; -A1 O A0  A1],  A_j = (I - D)(I + D^2)(I + D^4)(I + D^8)
// (D strictly lower triangular, so D^16 = 0), evaluated with 16x16x16 MFMA
// products in registers.
//
// Mapping: one workgroup per (sequence, v-head, 64-column slice of d_v); 12
// waves, waves i, i + 4 and i + 8 on SIMD i.
//   * Chain waves 0-3: wave j owns state columns 16j..16j+15 for the whole
//     sequence as fp32 MFMA accumulator tiles.  Every product of the chain
//     takes its right operand straight from accumulator registers: the k index
//     of each 32-deep product is ordered so that lane group g (= lane / 16)
//     holds rows 4g..4g+3 and 16+4g..16+4g+3 of the block -- exactly the rows
//     a C-layout tile pair holds -- and the left operand (K, Q, A or M rows in
//     LDS) is read in that same order; K^T rows come from the token-major K
//     tile through the LDS transpose read.  Per chunk: P = K h and o^T = h^T
//     q^T, R, v', o^T += v'^T M^T (stored directly: a lane holds 4 consecutive
//     output columns of one token), h update, checkpoint stores.
//   * Side waves prepare chunk c+1 while the chain runs chunk c: waves 4-5
//     form A11 and A22 (k k^T tiles, masks, blocked inverse, all in
//     registers) and two masked tiles; waves 6-9 the other masked q k^T tiles
//     (M) and -L21, and stage / prefetch later chunks (K, Q tiles); waves
//     10-11 the V tiles (staged, or on the fused path computed) and wave 10
//     the gate table.
//   * Fused variant (FUSED): the V tiles are the conv + SiLU of the raw
//     projections, computed by waves 10-11 (three of each lane's four rows
//     before the M barrier, the fourth after it), and the gate
//     table is prepared from the raw gate / beta projections; q and k come
//     normalised from a separate pass (their conv is shared by every
//     workgroup of a key head).
//   * EXT variant: checkpoints every 16 or 32 tokens (the states at interval
//     ends inside a chunk, formed from the chunk's K and v') and frame-table
//     state addressing (LogState payload frames).
// Two workgroup barriers per chunk (LDS-only waits, so global prefetches stay
// in flight).  MFMA operands are f16 with fp32 accumulation: bf16 values
// convert exactly within f16's normal range, magnitudes below 2^-14 keep
// fewer bits (f16 subnormals; at most 2^-25 absolute error) and magnitudes
// beyond 65504 become +-inf.  The operands are normalised q / k, decays and
// beta <= 1, the solve's A, the residuals R and v', and the state slices; v
// itself stays in the io type in LDS and enters R exactly.
//
// Roofline: MFMA (16-bit).  Algorithmic flops per token per v-head:
// 10 C d + 6 d^2 + 2/3 C^2 (C = 64, d = 128).
#include <type_traits>

#include "chunk_common.hpp"

namespace gdn {
namespace {

constexpr int kC = 64;
// Workgroup roles (waves i, i + 4 and i + 8 share a SIMD):
//   0-3 chain, 4-5 inverses, 6-9 tiles and K/Q (V) staging, 10-11 fused v conv and gates.
constexpr int kThreads = 768;
constexpr int kChainWaves = 4;
constexpr int kGateWave = 10;
constexpr float kRcpLn2 = 1.4426950216f;  // gated_delta.py:12

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef short s4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 to_uint4(u4_t v) { return make_uint4(v[0], v[1], v[2], v[3]); }

// LDS row strides (halfs).  The LDS serves a 64-bit access 16 lanes at a
// time over 32 four-byte banks (the layouts below measure zero bank-conflict
// cycles on the K/Q tiles, against 44 % of all LDS-busy cycles with padded
// rows alone).
//
// K and Q tiles: rows of d_k + 16 halfs (a stride of 8 mod 32 dwords), and
// 8-byte chunk q of row r stored at chunk q ^ ((r / 4) mod 4).  The 16 rows of
// a left-operand read (one chunk each) then fall on 4 row phases x 4 chunk
// swizzles = 16 distinct bank pairs, and so do the 4 rows x 4 chunks of a
// transpose read; the swizzle keeps chunks q and q + 4 16 halfs apart.
constexpr int LDV = 80;      // V rows (64 columns)
// A and M rows: 34 dwords.  The LDS serves a 64-bit access 16 lanes at a time
// over 32 four-byte banks; 16 rows at a stride of 2 mod 4 dwords hit all 32
// banks once (a stride of 0 mod 4 pairs rows r and r + 8 on one bank).
constexpr int LDA = kC + 4;
// Gate table per chunk (floats): G, 2^G, 2^(G_last - G) (0 past the end),
// beta, 2^G_last; then the factors of the off-diagonal 16 x 16 decay tiles:
// 2^(G_t - G_16b) for token t of 16-token block b (G_RF), and for b = 1..3
// 2^(G_16b - G_s) for s < 16 b (G_CF + 64 (b - 1) + s).  For t >= 16 b > s
// their product is 2^(G_t - G_s), so off-diagonal tiles need no exponential;
// with log-decay gates (<= 0, G non-increasing) both factors are <= 1.
constexpr int GTS = 520;
constexpr int G_EXP = 64, G_DEC = 128, G_BETA = 192, G_LAST = 256, G_RF = 264, G_CF = 328;

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ f4_t mma(h8_t a, h8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4_t zero4() { return f4_t{0.f, 0.f, 0.f, 0.f}; }

// f16 MFMA operand, round to nearest even (pairs become one v_cvt_pk_f16_f32).
// Magnitudes beyond the f16 range (65504) become +-inf, which then shows in
// the outputs and states rather than passing as a saturated value.
__device__ __forceinline__ _Float16 to_op(float x) { return static_cast<_Float16>(x); }
__device__ __forceinline__ h8_t cat(h4_t lo, h4_t hi) { return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7); }
// Left operand, row `row` of a row-major f16 matrix, k block at column k0.
__device__ __forceinline__ h8_t afrag(const _Float16* base, int ld, int row, int k0, int g) {
  const _Float16* p = base + row * ld + k0 + 4 * g;
  return cat(*reinterpret_cast<const h4_t*>(p), *reinterpret_cast<const h4_t*>(p + 16));
}
// afrag of a swizzled K / Q tile: k0 is a multiple of 32 and g < 4, so chunk
// k0 / 4 + g lands on k0 / 4 + (g ^ a), a = (row / 4) mod 4, and chunk + 4 16
// halfs after it.
__device__ __forceinline__ h8_t kqfrag(const _Float16* base, int ld, int row, int k0, int g) {
  const _Float16* p = base + row * ld + k0 + 4 * (g ^ ((row >> 2) & 3));
  return cat(*reinterpret_cast<const h4_t*>(p), *reinterpret_cast<const h4_t*>(p + 16));
}
// Four V values read from the V buffer, which holds them in the io type
// (exact: no operand conversion on the way in).
template <class IOT> __device__ __forceinline__ void v_rows(h4_t raw, float (&x)[4]);
template <> __device__ __forceinline__ void v_rows<f16>(h4_t raw, float (&x)[4]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) x[e] = static_cast<float>(raw[e]);
}
template <> __device__ __forceinline__ void v_rows<bf16>(h4_t raw, float (&x)[4]) {
  const uint2 w = __builtin_bit_cast(uint2, raw);
  x[0] = __uint_as_float(w.x << 16);
  x[1] = __uint_as_float(w.x & 0xffff0000u);
  x[2] = __uint_as_float(w.y << 16);
  x[3] = __uint_as_float(w.y & 0xffff0000u);
}
// LDS transpose read: the 16 lanes of a group read a 4-row x 16-column block
// (lane r: row r / 4, columns 4 (r % 4)..+3) and lane r receives column r.
__device__ __forceinline__ h4_t tr_read(const _Float16* p) {
  typedef __attribute__((address_space(3))) s4_t lds_s4;
  return __builtin_bit_cast(h4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p)));
}
// Left operand of K^T for a token-major, swizzled K tile: rows of K^T =
// columns c0 + lane % 16 of K (c0 a multiple of 16), k block = tokens
// t0..t0+31 (t0 a multiple of 32) in the k order above.  Lane (lr, lg) reads
// rows r = t0 + 4 lg + lr / 4 and r + 16, whose row phase (r / 4) mod 4 is lg
// for every t0 in {0, 32}: the lane part of the address is the byte offset
// lane_tr_offset(...) from the tile, computed once, and the rest a constant.
__device__ __forceinline__ uint32_t lane_tr_offset(int ld, int lr, int lg) {
  return static_cast<uint32_t>(((4 * lg + (lr >> 2)) * ld + 4 * ((lr & 3) ^ lg)) * 2);
}
template <int LD>
__device__ __forceinline__ h8_t kq_tfrag(const char* lane_tile, int t0, int c0) {
  const char* p = lane_tile + (t0 * LD + c0) * 2;
  return cat(tr_read(reinterpret_cast<const _Float16*>(p)), tr_read(reinterpret_cast<const _Float16*>(p + 16 * LD * 2)));
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

// Inclusive prefix sum over the 64 lanes of a wave with DPP moves (no LDS):
// a scan within each 16-lane row (row_shr 1, 2, 4, 8), then the row totals
// carried upwards (row_bcast 15 into rows 1 and 3, row_bcast 31 into rows 2
// and 3).  Masked-off rows and lanes shifted in from outside a row add 0.
template <int CTRL, int ROW_MASK> __device__ __forceinline__ float dpp_src(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, true));
}
__device__ __forceinline__ float wave_prefix_sum(float x) {
  x += dpp_src<0x111, 0xf>(x);
  x += dpp_src<0x112, 0xf>(x);
  x += dpp_src<0x114, 0xf>(x);
  x += dpp_src<0x118, 0xf>(x);
  x += dpp_src<0x142, 0xa>(x);
  x += dpp_src<0x143, 0xc>(x);
  return x;
}

// Block-uniform index read through the scalar data cache (a scalar load: it
// is waited on with the LDS counter, never behind outstanding vector stores).
__device__ __forceinline__ int64_t uniform_index(const void* p, int64_t i, int is64) {
  typedef __attribute__((address_space(4))) const int64_t ci64;
  typedef __attribute__((address_space(4))) const int32_t ci32;
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  return is64 ? reinterpret_cast<ci64*>(a)[i] : static_cast<int64_t>(reinterpret_cast<ci32*>(a)[i]);
}

template <class ST> __device__ __forceinline__ float load_st(const ST* p) { return to_f32(*p); }
template <class ST> __device__ __forceinline__ void store_st(ST* p, float v) { *p = from_f32<ST>(v); }

// ---- 32x32 lower-triangular matrices held as C-layout tiles of X and X^T.
// x[0] = X(0,0), x[1] = X(1,0), x[2] = X(1,1); t[0] = X^T(0,0), t[1] =
// X^T(0,1), t[2] = X^T(1,1) (tile (a, b): rows 16a.., columns 16b..).
struct Tri {
  f4_t x[3], t[3];
};
// A 16 x 16 block X as C-layout tiles of X (x) and of X^T (t).  Fed to a
// 16x16x16 MFMA, the 4 halfs a lane holds of a C-layout tile of Y are the
// A operand Y^T or the B operand Y, so X W comes from (X.t, W.x) and
// (X W)^T from (W.x, X.t) with no data movement between lanes.
struct Sq {
  f4_t x, t;
};
__device__ __forceinline__ h4_t hfrag(f4_t a) {
  h4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = to_op(a[e]);
  return o;
}
__device__ __forceinline__ f4_t mma16(h4_t a, h4_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
// X X for a block in both orientations.
__device__ __forceinline__ Sq sq_square(const Sq& X) {
  const h4_t xt = hfrag(X.t), xx = hfrag(X.x);
  return Sq{mma16(xt, xx, zero4()), mma16(xx, xt, zero4())};
}

// EXT: checkpoint granularities below 64 and frame-table states (a separate
// instantiation, so that the plain path carries none of their registers).
template <int DK, class IOT, class ST, bool FUSED, bool EXT>
__global__ __launch_bounds__(kThreads, 1) void chunk_chain_kernel(ChunkParams p) {
  constexpr int HT = DK / 16;    // 16-row state tiles
  constexpr int KS = DK / 32;    // 32-deep k steps over d_k
  constexpr int LDK = DK + 16;   // K / Q row strides (halfs; swizzled tiles)
  constexpr int LDQ = DK + 16;
  constexpr int DB = DK / 8;     // 8-column blocks of a K row
  constexpr int KBLK = 16 * DB;  // K (Q) staging blocks (4 tokens x 8 columns) per chunk
  static_assert(KS >= 1 && KBLK <= 256, "d_k in {32, 64, 128}");

  __shared__ __align__(16) _Float16 sK[3 * kC * LDK];
  __shared__ __align__(16) _Float16 sQ[2 * kC * LDQ];
  __shared__ __align__(16) _Float16 sV[kC * LDV];  // V rows, io-type bits (bf16 or f16)
  __shared__ __align__(16) _Float16 sA[2 * kC * LDA];  // [A11 | 0 ; -L21 | A22]
  __shared__ __align__(16) _Float16 sM[2 * kC * LDA];  // tril_incl(q k^T 2^(G_i - G_j))
  __shared__ __align__(16) float sG[3 * GTS];
  // EXT: byte offset in the frame storage of each token's logged v' slice (-1: none), 3 chunks
  __shared__ int64_t sLog[EXT ? 3 * kC : 1];

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
  // columns of this slice: 64, or 32 for d_v = 32, where chain waves 2-3 run on
  // zero columns (zero state, zero V) and store nothing
  const int vwidth = p.DV - col_base < 64 ? static_cast<int>(p.DV - col_base) : 64;
  const bool live = 16 * wave < vwidth;

  const int64_t bos = uniform_index(p.cu, n, p.cu_is64);
  const int64_t len = uniform_index(p.cu, n + 1, p.cu_is64) - bos;
  const int64_t nchunks = (len + kC - 1) / kC;
  auto valid_rows = [&](int64_t c) -> int {
    const int64_t rem = len - c * kC;
    return rem <= 0 ? 0 : (rem < kC ? static_cast<int>(rem) : kC);
  };

  ST* pool = static_cast<ST*>(p.state);
  const int64_t head_off = p.layer * p.layer_stride + h * p.head_stride + col_base;
  const int j = wave;  // chain wave: state columns 16j..16j+15
  constexpr int64_t kRowBytes = sizeof(ST);
  const int64_t row_bytes = p.DV * kRowBytes;
  f4_t hT[HT];
  // State slice rows 16 ti + 4 lg + e, column 16 j + lr: a wave-uniform base
  // plus a 32-bit lane offset (kept opaque so the per-element offsets are not
  // hoisted and held in registers across the chunk loop).
  auto state_lane_off = [&]() {
    uint32_t o = static_cast<uint32_t>((4 * lg * p.DV + 16 * j + lr) * sizeof(ST));
    asm volatile("" : "+v"(o));
    return o;
  };
  // Byte address of element (0, col_base) of the slice in slot s, or null for
  // a negative slot or an unmapped frame (entry < 0 or past the storage).
  // Rows follow every row_bytes (plain pools and heads inside one frame).
  auto slice_base = [&](int64_t s) __attribute__((always_inline)) -> char* {
    if (s < 0) return nullptr;
    if (!EXT || !p.frames) return reinterpret_cast<char*>(pool + s * p.slot_stride + head_off);
    if (s >= p.frame_slots) return nullptr;  // past the frame table: unmapped
    const int64_t logical = (p.layer * p.HV + h) * p.head_bytes;
    const int64_t fr = uniform_index(p.frames, s * p.fps + logical / p.frame_bytes, p.frames_is64);
    if (fr < 0 || fr >= p.num_frames) return nullptr;
    return static_cast<char*>(p.state) + fr * p.frame_bytes + logical % p.frame_bytes + col_base * kRowBytes;
  };
  // Heads spanning several frames (each frame holds whole 16-row tiles):
  // byte address of element (16 ti, col_base) of slot s, or null.
  auto frame_tile = [&](int64_t s, int ti) __attribute__((always_inline)) -> char* {
    if (s >= p.frame_slots) return nullptr;
    const int64_t logical = (p.layer * p.HV + h) * p.head_bytes + 16 * ti * row_bytes;
    const int64_t fr = uniform_index(p.frames, s * p.fps + logical / p.frame_bytes, p.frames_is64);
    if (fr < 0 || fr >= p.num_frames) return nullptr;
    return static_cast<char*>(p.state) + fr * p.frame_bytes + logical % p.frame_bytes + col_base * kRowBytes;
  };
  // Row 16 ti of the slice in slot s (slice = slice_base(s)), or null.
  auto tile_at = [&](char* slice, int64_t s, int ti) __attribute__((always_inline)) -> char* {
    if (EXT && p.frame_rows) return s >= 0 ? frame_tile(s, ti) : nullptr;
    return slice ? slice + 16 * ti * row_bytes : nullptr;
  };
  auto load_state = [&]() __attribute__((always_inline)) {
    const int64_t rs = live ? uniform_index(p.read_slots, n, p.read_is64) : -1;
    char* src = EXT && p.frame_rows ? nullptr : slice_base(rs);
    const uint32_t o = state_lane_off();
#pragma unroll
    for (int ti = 0; ti < HT; ++ti) {
      const char* tile = tile_at(src, rs, ti);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        hT[ti][e] = tile ? load_st(reinterpret_cast<const ST*>(tile + e * row_bytes + o)) : 0.f;
    }
  };
  // Stores tile(ti) (rows 16 ti.., this wave's columns) for every ti to slot s >= 0.
  auto store_tiles = [&](int64_t s, auto&& tile) __attribute__((always_inline)) {
    if (!live) return;
    char* dst = EXT && p.frame_rows ? nullptr : slice_base(s);
    if (!(EXT && p.frame_rows) && !dst) return;
    const uint32_t o = state_lane_off();
#pragma unroll
    for (int ti = 0; ti < HT; ++ti) {
      const f4_t v = tile(ti);
      char* t = tile_at(dst, s, ti);
      if (t) {
#pragma unroll
        for (int e = 0; e < 4; ++e) store_st(reinterpret_cast<ST*>(t + e * row_bytes + o), v[e]);
      }
    }
  };
  auto store_state = [&](int64_t s) __attribute__((always_inline)) {
    store_tiles(s, [&](int ti) __attribute__((always_inline)) { return hT[ti]; });
  };

  if (nchunks == 0) {  // empty sequence: the final state is the initial state
    if (wave < kChainWaves && p.fw_slots) {
      const int64_t fw = uniform_index(p.fw_slots, n, p.fw_is64);
      if (fw >= 0) {
        load_state();
        store_state(fw);
      }
    }
    return;
  }
  // checkpoint slots before this sequence: one per `gran` tokens of each earlier sequence
  const int gran = EXT ? p.gran : kC;
  int64_t chunk_base = 0;
  for (int64_t m = 0; m < n; ++m) {
    const int64_t lm = uniform_index(p.cu, m + 1, p.cu_is64) - uniform_index(p.cu, m, p.cu_is64);
    chunk_base += (lm + gran - 1) / gran;
  }

  // A and M start zero: their upper blocks are never written.
  for (int e = tid; e < 2 * kC * LDA / 8; e += kThreads) {
    reinterpret_cast<uint4*>(sA)[e] = make_uint4(0, 0, 0, 0);
    reinterpret_cast<uint4*>(sM)[e] = make_uint4(0, 0, 0, 0);
  }

  if (wave < kChainWaves) {
    // ==================================================================== chain waves
    uint16_t* og = static_cast<uint16_t*>(p.out) + (bos * p.HV + h) * p.DV + col_base + 16 * j;
    uint16_t* vng = p.v_new ? static_cast<uint16_t*>(p.v_new) + (bos * p.HV + h) * p.DV + col_base + 16 * j : nullptr;
    const int64_t tok_stride = p.HV * p.DV;
    uint32_t ktr = lane_tr_offset(LDK, lr, lg);
    asm volatile("" : "+v"(ktr));
    load_state();
    // No vector-memory load may be outstanding at the loop head (a wait there
    // would also wait for the previous chunk's output stores): consume the
    // loaded state before entering the loop.
#pragma unroll
    for (int ti = 0; ti < HT; ++ti) asm volatile("" ::"v"(hT[ti]));
    lds_barrier();  // P0
    lds_barrier();  // B(0)
    for (int64_t c = 0; c < nchunks; ++c) {
      const int nv = valid_rows(c);
      const int nsub = (nv + gran - 1) / gran;  // checkpoint intervals in this chunk
      const int64_t sub0 = chunk_base + c * (kC / gran);
      const int64_t cw = uniform_index(p.cw_slots, sub0 + nsub - 1, p.cw_is64);  // checkpoint slot
      const _Float16* K = sK + (c % 3) * kC * LDK;
      const _Float16* Q = sQ + (c & 1) * kC * LDQ;
      const float* gt = sG + (c % 3) * GTS;
      // ---- S1: P = K h -> R = beta (v - 2^G P);  O^T = h^T Q^T (token columns).
      // Per 32-deep k step the K and Q fragments are read together and the
      // converted state is both the right operand of K h and the left operand
      // of h^T Q^T: eight independent accumulations in flight.
      f4_t R[4], Ot[4];
      {
        f4_t P[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) P[i] = Ot[i] = zero4();
#pragma unroll
        for (int m = 0; m < KS; ++m) {
          h8_t kf[4], qf[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) kf[i] = kqfrag(K, LDK, 16 * i + lr, 32 * m, lg);
#pragma unroll
          for (int i = 0; i < 4; ++i) qf[i] = kqfrag(Q, LDQ, 16 * i + lr, 32 * m, lg);
          const h8_t hb = bfrag(hT[2 * m], hT[2 * m + 1]);
#pragma unroll
          for (int i = 0; i < 4; ++i) P[i] = mma(kf[i], hb, P[i]);
#pragma unroll
          for (int i = 0; i < 4; ++i) Ot[i] = mma(hb, qf[i], Ot[i]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t0 = 16 * i + 4 * lg;
          const f4_t e4 = *reinterpret_cast<const f4_t*>(gt + G_EXP + t0);
          const f4_t b4 = *reinterpret_cast<const f4_t*>(gt + G_BETA + t0);
          // V rows t0..t0+3 at column 16j + lr
          float v4[4];
          v_rows<IOT>(tr_read(sV + (16 * i + 4 * lg + (lr >> 2)) * LDV + 16 * j + 4 * (lr & 3)), v4);
#pragma unroll
          for (int e = 0; e < 4; ++e) R[i][e] = b4[e] * (v4[e] - e4[e] * P[i][e]);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) Ot[i] *= gt[G_EXP + 16 * i + lr];
      lds_barrier();  // M(c)
      // ---- S2: v'_top = A11 R_top; R_bot -= L21 v'_top; v'_bot = A22 R_bot
      const _Float16* A = sA + (c & 1) * kC * LDA;
      f4_t V[4];
      h8_t vb0, vb1;
      h8_t mf[6];  // M's fragments for S3a
      auto read_m = [&]() __attribute__((always_inline)) {
        const _Float16* M = sM + (c & 1) * kC * LDA;
#pragma unroll
        for (int i = 0; i < 4; ++i) mf[i] = afrag(M, LDA, 16 * i + lr, 0, lg);
        mf[4] = afrag(M, LDA, 32 + lr, 32, lg);
        mf[5] = afrag(M, LDA, 48 + lr, 32, lg);
      };
      {
        const h8_t a0 = afrag(A, LDA, lr, 0, lg), a1 = afrag(A, LDA, 16 + lr, 0, lg);
        const h8_t l2 = afrag(A, LDA, 32 + lr, 0, lg), l3 = afrag(A, LDA, 48 + lr, 0, lg);  // -L21
        const h8_t a2 = afrag(A, LDA, 32 + lr, 32, lg), a3 = afrag(A, LDA, 48 + lr, 32, lg);
        if constexpr (!EXT) {
          // M's fragments are read with A's, so their LDS latency passes under
          // the solve's dependent steps (the EXT kernel would spill for it)
          read_m();
          __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
        }
        const h8_t rb0 = bfrag(R[0], R[1]);
        V[0] = mma(a0, rb0, zero4());
        V[1] = mma(a1, rb0, zero4());
        vb0 = bfrag(V[0], V[1]);  // also the left operand of v'^T
        R[2] = mma(l2, vb0, R[2]);
        R[3] = mma(l3, vb0, R[3]);
        const h8_t rb1 = bfrag(R[2], R[3]);
        V[2] = mma(a2, rb1, zero4());
        V[3] = mma(a3, rb1, zero4());
        vb1 = bfrag(V[2], V[3]);
        if (live && (vng || (EXT && p.logging))) {
          // v'^T = R^T A^T: the same fragments with the operands swapped (a
          // B fragment of R is an A fragment of R^T), so lane (g, c) holds
          // columns 4g..4g+3 of token 16 i + c and writes them as 8 bytes,
          // to v_new or to the token's log row.
          const f4_t vt[4] = {mma(rb0, a0, zero4()), mma(rb0, a1, zero4()), mma(rb1, a2, zero4()),
                              mma(rb1, a3, zero4())};
          if (EXT && p.logging) {
            const int64_t* lrow = sLog + (c % 3) * kC;
            char* const st = static_cast<char*>(p.state);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int64_t off = lrow[16 * i + lr];
              if (off >= 0) {
                uint2 w;
                w.x = out_pack2<IOT>(vt[i][0], vt[i][1]);
                w.y = out_pack2<IOT>(vt[i][2], vt[i][3]);
                *reinterpret_cast<uint2*>(st + off + (16 * j + 4 * lg) * 2) = w;
              }
            }
          } else {
            char* vb = reinterpret_cast<char*>(vng + c * kC * tok_stride);
            uint32_t ov = static_cast<uint32_t>((lr * tok_stride + 4 * lg) * 2);
            asm volatile("" : "+v"(ov));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if (16 * i + lr < nv) {
                uint2 w;
                w.x = out_pack2<IOT>(vt[i][0], vt[i][1]);
                w.y = out_pack2<IOT>(vt[i][2], vt[i][3]);
                *reinterpret_cast<uint2*>(vb + 16 * i * tok_stride * 2 + ov) = w;
              }
            }
          }
        }
      }
      // ---- S3a: o^T += v'^T M^T; a lane holds 4 consecutive output columns of one token
      {
        if constexpr (EXT) read_m();
#pragma unroll
        for (int i = 0; i < 4; ++i) Ot[i] = mma(vb0, mf[i], Ot[i]);
        Ot[2] = mma(vb1, mf[4], Ot[2]);
        Ot[3] = mma(vb1, mf[5], Ot[3]);
      }
      {
        char* ob = reinterpret_cast<char*>(og + c * kC * tok_stride);
        uint32_t o = static_cast<uint32_t>((lr * tok_stride + 4 * lg) * 2);
        asm volatile("" : "+v"(o));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (live && 16 * i + lr < nv) {
            uint2 w;
            w.x = out_pack2<IOT>(p.scale * Ot[i][0], p.scale * Ot[i][1]);
            w.y = out_pack2<IOT>(p.scale * Ot[i][2], p.scale * Ot[i][3]);
            *reinterpret_cast<uint2*>(ob + 16 * i * tok_stride * 2 + o) = w;
          }
        }
      }
      // ---- checkpoints inside the chunk (granularity 16 or 32): the state after
      // token te = (s + 1) gran - 1 is 2^G_te h + K^T (2^(G_te - G) v'), the
      // decay taken over tokens t <= te only.
      for (int sc = 0; EXT && sc + 1 < nsub; ++sc) {
        const int64_t ws = uniform_index(p.cw_slots, sub0 + sc, p.cw_is64);
        if (ws < 0) continue;
        const int te = (sc + 1) * gran - 1;
        const float Ge = gt[te], ge = gt[G_EXP + te];
        f4_t dm[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f4_t g4 = *reinterpret_cast<const f4_t*>(gt + 16 * i + 4 * lg);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            dm[i][e] = 16 * i + 4 * lg + e <= te ? V[i][e] * fast_exp2(Ge - g4[e]) : 0.f;
        }
        const h8_t m0 = bfrag(dm[0], dm[1]), m1 = bfrag(dm[2], dm[3]);
        store_tiles(ws, [&](int ti) __attribute__((always_inline)) {
          const char* kl = reinterpret_cast<const char*>(K) + ktr;
          f4_t r = mma(kq_tfrag<LDK>(kl, 0, 16 * ti), m0, hT[ti] * ge);
          if (te >= 32) r = mma(kq_tfrag<LDK>(kl, 32, 16 * ti), m1, r);
          return r;
        });
      }
      // ---- S3b: h <- 2^G_last h + K^T (2^(G_last - G) v')
      {
        const f4_t d0 = *reinterpret_cast<const f4_t*>(gt + G_DEC + 4 * lg);
        const f4_t d1 = *reinterpret_cast<const f4_t*>(gt + G_DEC + 16 + 4 * lg);
        const f4_t d2 = *reinterpret_cast<const f4_t*>(gt + G_DEC + 32 + 4 * lg);
        const f4_t d3 = *reinterpret_cast<const f4_t*>(gt + G_DEC + 48 + 4 * lg);
        const h8_t db0 = bfrag(V[0] * d0, V[1] * d1);
        const h8_t db1 = bfrag(V[2] * d2, V[3] * d3);
        const float gl = gt[G_LAST];
#pragma unroll
        for (int ti = 0; ti < HT; ++ti) {
          const char* kl = reinterpret_cast<const char*>(K) + ktr;
          const h8_t k0 = kq_tfrag<LDK>(kl, 0, 16 * ti);
          const h8_t k1 = kq_tfrag<LDK>(kl, 32, 16 * ti);
          hT[ti] = mma(k1, db1, mma(k0, db0, hT[ti] * gl));
        }
      }
      if (cw >= 0) store_state(cw);
      lds_barrier();  // B(c+1)
    }
    if (p.fw_slots) {
      const int64_t fw = uniform_index(p.fw_slots, n, p.fw_is64);
      if (fw >= 0) store_state(fw);
    }
  } else {
    // ==================================================================== side waves
    const int sw = wave - kChainWaves;  // 0-1 inverses, 2-5 tiles and staging, 6-7 conv and gates
    // Entries (t, s..s+3) of a row-orientation tile -> masked values.
    auto masked = [&](const float* gt, f4_t s, int t, int s0, bool strict, bool with_beta)
        __attribute__((always_inline)) {
      const f4_t gs = *reinterpret_cast<const f4_t*>(gt + s0);
      const float gti = gt[t];
      const float bt = with_beta ? gt[G_BETA + t] : 1.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool keep = strict ? t > s0 + e : t >= s0 + e;
        // G is a running sum of log-decays, so kept entries (t >= s) have a
        // non-positive exponent; a dropped entry's exponent may overflow to
        // inf, which the select discards.
        s[e] = keep ? bt * s[e] * fast_exp2(gti - gs[e]) : 0.f;
      }
      return s;
    };
    // The same for a tile whose rows t lie in 16-token block t / 16 >= 1 and
    // whose columns lie in earlier blocks (every entry kept): the decay from
    // the gate table's row and boundary factors.
    auto masked_off = [&](const float* gt, f4_t s, int t, int s0, bool with_beta) __attribute__((always_inline)) {
      const f4_t cf = *reinterpret_cast<const f4_t*>(gt + G_CF + 64 * ((t >> 4) - 1) + s0);
      const float r = with_beta ? gt[G_RF + t] * gt[G_BETA + t] : gt[G_RF + t];
#pragma unroll
      for (int e = 0; e < 4; ++e) s[e] = r * s[e] * cf[e];
      return s;
    };
    auto store_row4 = [&](_Float16* X, int t, int s0, f4_t v) __attribute__((always_inline)) {
      const h4_t w = {to_op(v[0]), to_op(v[1]), to_op(v[2]), to_op(v[3])};
      *reinterpret_cast<h4_t*>(X + t * LDA + s0) = w;
    };

    // ---- inverses (waves 4-5): A_bb = (I + L_bb)^-1 for the 32-token half b,
    // blocked into 16 x 16 blocks: with L_bb = [D0 0; O D1], A_bb = [A0 0;
    // -A1 O A0  A1], and each (I + D)^-1 = (I - D)(I + D^2)(I + D^4)(I + D^8)
    // (D strictly lower triangular, so D^16 = 0).  In two parts, so that it
    // spans both phases of a chunk:
    //   first:  L, D^2, D^4, G = (I - D)(I + D^2) for both diagonal blocks
    //   second: D^8, A_i = G (I + D^4)(I + D^8), -A1 O A0, stored into A.
    // Block 1 is needed only as A1^T (the store and -A1 O A0 take that form);
    // block 0 also as A0 (the right factor of O A0).
    Sq invD4[2], invG[2];
    f4_t invOt;  // C-layout tile of O^T
    auto inv_first = [&](int64_t nc) __attribute__((always_inline)) {
      const _Float16* K = sK + (nc % 3) * kC * LDK;
      const float* gt = sG + (nc % 3) * GTS;
      const int r0 = 32 * sw;
      f4_t s00 = zero4(), s11 = zero4(), s01 = zero4();
      h8_t k0[KS], k1[KS];
#pragma unroll
      for (int m = 0; m < KS; ++m) {
        k0[m] = kqfrag(K, LDK, r0 + lr, 32 * m, lg);
        k1[m] = kqfrag(K, LDK, r0 + 16 + lr, 32 * m, lg);
      }
#pragma unroll
      for (int m = 0; m < KS; ++m) {
        s00 = mma(k0[m], k0[m], s00);
        s11 = mma(k1[m], k1[m], s11);
        s01 = mma(k0[m], k1[m], s01);  // C layout: entry (4g + e, 16 + c) of S^T
      }
      // C-layout tiles of L (row 4g + e, col c) and of L^T (row 4g + e, col c
      // of L^T = entry (c, 4g + e) of L); S is symmetric on the diagonal tiles.
      auto lmask_c = [&](f4_t s, int t0, int sc) {  // entries (t0 + 4g + e, sc + c)
        const f4_t gt4 = *reinterpret_cast<const f4_t*>(gt + t0 + 4 * lg);
        const f4_t bt4 = *reinterpret_cast<const f4_t*>(gt + G_BETA + t0 + 4 * lg);
        const float gsc = gt[sc + lr];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          s[e] = (t0 + 4 * lg + e > sc + lr) ? bt4[e] * s[e] * fast_exp2(gt4[e] - gsc) : 0.f;
        return s;
      };
      auto lmask_t = [&](f4_t s, int tc, int s0) {  // entries (tc + c, s0 + 4g + e)
        return masked(gt, s, tc + lr, s0 + 4 * lg, true, true);
      };
      // L.x[1], the off-diagonal block itself, is not needed: O enters only
      // as the left factor of O A0, that is through O^T (L.t[1], from the
      // table's row and boundary factors)
      Tri L;
      L.x[0] = lmask_c(s00, r0, r0);
      L.x[2] = lmask_c(s11, r0 + 16, r0 + 16);
      L.t[0] = lmask_t(s00, r0, r0);
      L.t[1] = masked_off(gt, s01, r0 + 16 + lr, r0 + 4 * lg, true);
      L.t[2] = lmask_t(s11, r0 + 16, r0 + 16);
      const f4_t id = f4_t{4 * lg == lr ? 1.f : 0.f, 4 * lg + 1 == lr ? 1.f : 0.f, 4 * lg + 2 == lr ? 1.f : 0.f,
                           4 * lg + 3 == lr ? 1.f : 0.f};
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const Sq D{L.x[2 * b], L.t[2 * b]};
        const Sq D2 = sq_square(D);
        invD4[b] = sq_square(D2);
        const Sq F{id - D.x, id - D.t};
        const h4_t d2x = hfrag(D2.x), ft = hfrag(F.t);
        invG[b].t = mma16(d2x, ft, F.t);
        invG[b].x = b == 0 ? mma16(ft, d2x, F.x) : zero4();
      }
      invOt = L.t[1];
    };
    auto inv_second = [&](int64_t nc) __attribute__((always_inline)) {
      _Float16* A = sA + (nc & 1) * kC * LDA;
      const int r0 = 32 * sw;
      Sq Ai[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const Sq& D4 = invD4[b];
        const Sq& G = invG[b];
        const h4_t d4x = hfrag(D4.x), d4t = hfrag(D4.t), gt4 = hfrag(G.t);
        const h4_t d8x = hfrag(mma16(d4t, d4x, zero4()));
        const Sq H{b == 0 ? mma16(gt4, d4x, G.x) : zero4(), mma16(d4x, gt4, G.t)};
        const h4_t ht = hfrag(H.t);
        Ai[b].t = mma16(d8x, ht, H.t);
        Ai[b].x = b == 0 ? mma16(ht, d8x, H.x) : zero4();
      }
      // T = O A0, then (-A1 T)^T = -T^T A1^T
      const f4_t Tx = mma16(hfrag(invOt), hfrag(Ai[0].x), zero4());
      const f4_t A10t = -mma16(hfrag(Tx), hfrag(Ai[1].t), zero4());
      // row-major A_bb: C-layout tile (a, b) of A^T holds row 16b + c, columns 16a + 4g..+3
      store_row4(A, r0 + lr, r0 + 4 * lg, Ai[0].t);
      store_row4(A, r0 + 16 + lr, r0 + 4 * lg, A10t);
      store_row4(A, r0 + 16 + lr, r0 + 16 + 4 * lg, Ai[1].t);
    };

    // ---- row-orientation tiles (waves 6-9): (ti, tj) of Q K^T -> M, and of
    // K K^T for -L21 (lane (g, c) holds entry (t = 16 ti + c, s = 16 tj + 4 g + e)).
    // Each wave forms some before the M barrier and the rest after it (the
    // chain reads them one chunk later).
    auto tiles = [&](int64_t nc, bool second) __attribute__((always_inline)) {
      const _Float16* K = sK + (nc % 3) * kC * LDK;
      const _Float16* Q = sQ + (nc & 1) * kC * LDQ;
      const float* gt = sG + (nc % 3) * GTS;
      _Float16* A = sA + (nc & 1) * kC * LDA;
      _Float16* M = sM + (nc & 1) * kC * LDA;
      auto tile = [&](const _Float16* X, int ldx, int ti, int tj) {
        h8_t a[KS], b[KS];
#pragma unroll
        for (int m = 0; m < KS; ++m) {
          a[m] = kqfrag(K, LDK, 16 * tj + lr, 32 * m, lg);
          b[m] = kqfrag(X, ldx, 16 * ti + lr, 32 * m, lg);
        }
        f4_t acc = zero4();
#pragma unroll
        for (int m = 0; m < KS; ++m) acc = mma(a[m], b[m], acc);
        return acc;
      };
      auto mtile = [&](int ti, int tj) {
        const int t = 16 * ti + lr, s0 = 16 * tj + 4 * lg;
        const f4_t x = tile(Q, LDQ, ti, tj);
        store_row4(M, t, s0, ti > tj ? masked_off(gt, x, t, s0, false) : masked(gt, x, t, s0, false, false));
      };
      const int w = sw - 2;  // 0..3 tile waves; -2, -1 the inverse waves (phase B only)
      // waves 6-7 share SIMDs with the v conv waves, 8-9 with the inverse waves;
      // the inverse waves, done early in the second phase, take its two tiles.
      // A wave's tiles are formed together: every fragment read first (each
      // 16-row block once), then the independent products, then the masks,
      // so the LDS and MFMA latencies of the tiles overlap.
      auto frags = [&](const _Float16* X, int ldx, int r, h8_t (&f)[KS]) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < KS; ++m) f[m] = kqfrag(X, ldx, 16 * r + lr, 32 * m, lg);
      };
      auto dot = [&](const h8_t (&a)[KS], const h8_t (&b)[KS]) __attribute__((always_inline)) {
        f4_t acc = zero4();
#pragma unroll
        for (int m = 0; m < KS; ++m) acc = mma(a[m], b[m], acc);
        return acc;
      };
      auto put_l = [&](int ti, int tj, f4_t x) __attribute__((always_inline)) {
        const int t = 16 * ti + lr, s0 = 16 * tj + 4 * lg;
        store_row4(A, t, s0, -masked_off(gt, x, t, s0, true));
      };
      auto put_m = [&](int ti, int tj, f4_t x) __attribute__((always_inline)) {
        const int t = 16 * ti + lr, s0 = 16 * tj + 4 * lg;
        store_row4(M, t, s0, ti > tj ? masked_off(gt, x, t, s0, false) : masked(gt, x, t, s0, false, false));
      };
      if (!second) {
        if (w == 0) {
          h8_t k0[KS], k1[KS], k2[KS], q0[KS], q1[KS];
          frags(K, LDK, 0, k0);
          frags(K, LDK, 2, k2);
          frags(K, LDK, 1, k1);
          frags(Q, LDQ, 0, q0);
          frags(Q, LDQ, 1, q1);
          const f4_t l20 = dot(k0, k2), l21 = dot(k1, k2), m00 = dot(k0, q0), m10 = dot(k0, q1);
          put_l(2, 0, l20);
          put_l(2, 1, l21);
          put_m(0, 0, m00);
          put_m(1, 0, m10);
        } else if (w == 1) {
          h8_t k0[KS], k1[KS], k3[KS], q1[KS], q2[KS];
          frags(K, LDK, 0, k0);
          frags(K, LDK, 3, k3);
          frags(K, LDK, 1, k1);
          frags(Q, LDQ, 1, q1);
          frags(Q, LDQ, 2, q2);
          const f4_t l30 = dot(k0, k3), l31 = dot(k1, k3), m11 = dot(k1, q1), m20 = dot(k0, q2);
          put_l(3, 0, l30);
          put_l(3, 1, l31);
          put_m(1, 1, m11);
          put_m(2, 0, m20);
        } else if (w == 2) {
          h8_t k1[KS], k2[KS], q2[KS];
          frags(Q, LDQ, 2, q2);
          frags(K, LDK, 1, k1);
          frags(K, LDK, 2, k2);
          const f4_t m21 = dot(k1, q2), m22 = dot(k2, q2);
          put_m(2, 1, m21);
          put_m(2, 2, m22);
        } else {
          h8_t k0[KS], k1[KS], q3[KS];
          frags(Q, LDQ, 3, q3);
          frags(K, LDK, 0, k0);
          frags(K, LDK, 1, k1);
          const f4_t m30 = dot(k0, q3), m31 = dot(k1, q3);
          put_m(3, 0, m30);
          put_m(3, 1, m31);
        }
      } else {
        if (w == -2) {
          mtile(3, 2);
        } else if (w == -1) {
          mtile(3, 3);
        }
      }
    };

    // Gate table of chunk ck from per-lane (token) g and beta: chunk-local
    // cumulative gate in log2 units (cumsum.py:19-75) and its exponentials.
    auto gate_table = [&](int64_t ck, float x, float bt) __attribute__((always_inline)) {
      const int nk = valid_rows(ck);
      const float G = wave_prefix_sum(x) * kRcpLn2;
      const float Gl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(G), nk > 0 ? nk - 1 : 0));
      float* gt = sG + (ck % 3) * GTS;
      gt[lane] = G;
      gt[G_EXP + lane] = fast_exp2(G);
      gt[G_DEC + lane] = lane < nk ? fast_exp2(Gl - G) : 0.f;
      gt[G_BETA + lane] = bt;
      if (lane == 0) gt[G_LAST] = fast_exp2(Gl);
    };
    // The off-diagonal decay factors of chunk ck (the other conv wave, from
    // its own scan of the same gates, so that it balances the gate wave).
    auto factor_table = [&](int64_t ck, float x) __attribute__((always_inline)) {
      const float G = wave_prefix_sum(x) * kRcpLn2;
      float* gt = sG + (ck % 3) * GTS;
      const float G16 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(G), 16));
      const float G32 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(G), 32));
      const float G48 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(G), 48));
      const float G0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(G), 0));
      gt[G_RF + lane] = fast_exp2(G - (lane < 16 ? G0 : lane < 32 ? G16 : lane < 48 ? G32 : G48));
      gt[G_CF + lane] = lane < 16 ? fast_exp2(G16 - G) : 0.f;
      gt[G_CF + 64 + lane] = lane < 32 ? fast_exp2(G32 - G) : 0.f;
      gt[G_CF + 128 + lane] = lane < 48 ? fast_exp2(G48 - G) : 0.f;
    };

    // ---- gates (the conv waves, after the M barrier), one token per lane; the
    // prepared g and beta (kernel/fused.py:105-117) feed the gate table.
    const FrontIn& f = p.front;
    float pgate = 0.f, pbeta = 0.f;
    auto prefetch_g = [&](int64_t ck) __attribute__((always_inline)) {
      const bool ok = lane < valid_rows(ck);
      const int64_t t = len > 0 ? bos + (ok ? ck * kC + lane : 0) : 0;  // a valid row for every chunk index
      // fused: head-major [HV, T] gates from the q/k pass (contiguous per head)
      const int64_t gi = FUSED ? h * p.T + t : t * p.HV + h;
      pgate = p.g[gi];
      pbeta = p.beta[gi];
    };
    auto stage_g = [&](int64_t ck) __attribute__((always_inline)) {
      const bool ok = lane < valid_rows(ck);
      if (wave == kGateWave) gate_table(ck, ok ? pgate : 0.f, ok ? pbeta : 0.f);
      else factor_table(ck, ok ? pgate : 0.f);
    };
    // EXT, token log: the log slice of the lane's token of chunk ck, in three
    // steps one chunk apart so that no wait of the conv waves covers them:
    // prefetch_log loads the token's log slot and position (stage A),
    // resolve_log turns stage A into its frame-table entry (stage B), and
    // stage_log (wave 10) writes stage B's byte offset to LDS.  Both waves 10
    // and 11 issue the loads, with clamped indices, every chunk.
    int aslot = 0, apos = 0, bentry = 0;
    bool aok = false, bvalid = false;
    uint32_t bbyte = 0;
    auto prefetch_log = [&](int64_t ck) __attribute__((always_inline)) {
      const bool ok = lane < valid_rows(ck);
      const int64_t t = len > 0 ? bos + (ok ? ck * kC + lane : 0) : 0;
      aslot = static_cast<int>(load_index(p.log_slots, t, p.log_is64));
      apos = static_cast<int>(load_index(p.log_pos, t, p.log_pos_is64));
      aok = p.logging && ok;
    };
    auto resolve_log = [&]() __attribute__((always_inline)) {
      const bool valid = aok && aslot >= 0 && aslot < p.log_rows && apos >= 0 && apos < p.log_page;
      const uint32_t ps = valid ? static_cast<uint32_t>(apos) : 0u;
      const uint32_t g = static_cast<uint32_t>(p.gran), sh = static_cast<uint32_t>(__builtin_ctz(g));
      const uint32_t key_size = g * static_cast<uint32_t>(p.log_key_heads) * DK;
      const uint32_t layer_size = key_size + g * static_cast<uint32_t>(p.HV) * static_cast<uint32_t>(p.DV);
      const uint32_t elem = ((ps >> sh) * static_cast<uint32_t>(p.log_layers) + static_cast<uint32_t>(p.layer)) *
                                layer_size +
                            key_size + (static_cast<uint32_t>(h) * g + (ps & (g - 1))) * static_cast<uint32_t>(p.DV) +
                            static_cast<uint32_t>(col_base);
      bbyte = 2u * elem;
      const int64_t idx = valid ? static_cast<int64_t>(aslot) * p.fps + p.fdiv.div(bbyte) : 0;
      bentry = static_cast<int>(load_index(p.log_table, idx, p.log_table_is64));
      bvalid = valid;
    };
    auto stage_log = [&](int64_t ck) __attribute__((always_inline)) {
      if (wave == kGateWave)
        sLog[(ck % 3) * kC + lane] = bvalid && bentry >= 0 && bentry < p.num_frames
                                         ? static_cast<int64_t>(bentry) * p.frame_bytes + p.fdiv.mod(bbyte)
                                         : -1;
    };

    // ---- fused path: V rows are the conv + SiLU of the projections
    // (packed_conv.py:49-133), computed by waves 10-11 before the M barrier and
    // staged after it.  A
    // lane convolves VT tokens x 8 channels with the 3 inputs before them (the
    // tokens before, or the conv history at the sequence start).
    constexpr int VT = 4, VNR = VT + 3;
    const int fst = tid - 640;
    // (waves 10-11 only; prefetch_fv, conv_v and stage_fv are called from that
    // role alone and run unconditionally, so no prefetch register is left
    // maybe-pending on a skipped path)
    const bool fv_thread = FUSED && fst >= 0 && fst < 128;
    const int fvtb = fst >> 3, fvdb = fst & 7;
    const uint16_t* mixed = static_cast<const uint16_t*>(f.mixed);
    const int64_t rs = f.row_stride;
    const int64_t vch = 2 * f.key_dim + h * p.DV + col_base;  // first channel of the slice
    const int64_t ch0 = vch + 8 * fvdb;
    u4_t vraw[VNR];
    float vw[4][8];
    const uint16_t* hist = nullptr;
    if constexpr (FUSED) {
      if (fv_thread) {
        const uint4* wp = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(f.weight) + ch0 * 4);
        float wv[32];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x[8];
          unpack8<IOT>(wp[i], x);
#pragma unroll
          for (int e = 0; e < 8; ++e) wv[8 * i + e] = x[e];
        }
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
          for (int tap = 0; tap < 4; ++tap) vw[tap][c] = wv[c * 4 + tap];
      }
      const int64_t bslot = uniform_index(p.read_slots, n, p.read_is64);
      if (bslot >= 0)
        hist = static_cast<const uint16_t*>(f.conv_state) + bslot * f.conv_slot_stride + p.layer * f.conv_layer_stride;
    }
    // The window rows of a chunk, [cv kC - 3, cv kC + 63], come through one
    // buffer resource per chunk whose range is the sequence's rows from
    // max(cv kC - 3, 0) to the end: rows before the sequence start (first
    // chunk: the conv history or zero, which conv_v substitutes) and past
    // its end read as zeros, with no select on the data, so nothing waits
    // for these loads before the next chunk's conv.  Rows past the end only
    // feed V rows that beta = 0 removes from the chain.  A lane's offset is
    // one add per row (row_stride < 2^24 elements keeps the range's 67 rows
    // in 32 bits; a negative row wraps far past the range).
    const uint32_t vrow_bytes = static_cast<uint32_t>(2 * rs);
    auto prefetch_fv = [&](int64_t cv) __attribute__((always_inline)) {
      const int64_t c0 = cv * kC;
      const int64_t b0 = c0 >= 3 ? c0 - 3 : 0;  // first row of the range
      const int64_t left = len - b0;
      const uint32_t nrec = static_cast<uint32_t>(left <= 0 ? 0 : (left < kC + 3 ? left : kC + 3)) * vrow_bytes;
      const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(mixed + (bos + b0) * rs + vch), 0, nrec, 0x00020000);
      // window row 0 of the lane (token VT fvtb - 3 of the chunk), from row b0
      const int first = VT * fvtb - 3 + static_cast<int>(c0 - b0);
      const uint32_t vbase = static_cast<uint32_t>(first) * vrow_bytes + static_cast<uint32_t>(16 * fvdb);
#pragma unroll
      for (int i = 0; i < VNR; ++i)
        vraw[i] = __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(vr, vbase + i * vrow_bytes, 0, 0));
    };
    // conv of chunk cv into registers, stage by stage over the rows' x 8
    // values so the exp / reciprocal latencies overlap.  In the loop the
    // first VT - 1 rows are convolved before M and the last after it (the
    // conv waves are the first phase's longest and have slack in the second);
    // all rows go into the single V buffer after M, when the chain has read
    // the previous chunk's.  Same operation order and rounding as the
    // standalone front end: y = round(silu(round(sum_tap w x))), the outer
    // rounding being the io pack.
    uint4 vo[VT];
    // rows I0 .. I0 + NR - 1 of the lane's VT (row i's window is vraw rows
    // i .. i + 3, unpacked again per call)
    auto conv_rows = [&](int64_t cv, auto i0c, auto nrc) __attribute__((always_inline)) {
      constexpr int I0 = decltype(i0c)::value, NR = decltype(nrc)::value;
      float win[3][8];
#pragma unroll
      for (int j = 0; j < 3; ++j) unpack8<IOT>(to_uint4(vraw[I0 + j]), win[j]);
      if (I0 == 0 && cv == 0 && fvtb == 0) {  // the 3 inputs before the sequence: history ([channel][tap]) or zero
        float e[3][8];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          uint4 hv = make_uint4(0, 0, 0, 0);
          if (hist != nullptr) hv = *reinterpret_cast<const uint4*>(hist + ch0 * 3 + 8 * j);
          unpack8<IOT>(hv, e[j]);
        }
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
          for (int j = 0; j < 3; ++j) win[j][c] = e[(3 * c + j) / 8][(3 * c + j) % 8];
      }
      float y[NR][8];
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        float x[8];
        unpack8<IOT>(to_uint4(vraw[3 + I0 + i]), x);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          float acc = 0.f;
          acc = fmaf(win[0][c], vw[0][c], acc);
          acc = fmaf(win[1][c], vw[1][c], acc);
          acc = fmaf(win[2][c], vw[2][c], acc);
          acc = fmaf(x[c], vw[3][c], acc);
          y[i][c] = acc;
          win[0][c] = win[1][c];
          win[1][c] = win[2][c];
          win[2][c] = x[c];
        }
        round8<IOT>(y[i]);
      }
      float d[NR][8];
#pragma unroll
      for (int i = 0; i < NR; ++i)
#pragma unroll
        for (int c = 0; c < 8; ++c) d[i][c] = fast_exp2(-1.4426950408889634f * y[i][c]);
#pragma unroll
      for (int i = 0; i < NR; ++i)
#pragma unroll
        for (int c = 0; c < 8; ++c) d[i][c] = __builtin_amdgcn_rcpf(1.0f + d[i][c]);
#pragma unroll
      for (int i = 0; i < NR; ++i) {
#pragma unroll
        for (int c = 0; c < 8; ++c) y[i][c] *= d[i][c];  // fast_silu
        // rows past the end hold the conv of clamped (real, finite) rows; the
        // chain scales them by beta = 0 there
        vo[I0 + i] = pack8_io<IOT>(y[i]);
      }
    };
    auto conv_v = [&](int64_t cv) __attribute__((always_inline)) {
      conv_rows(cv, std::integral_constant<int, 0>{}, std::integral_constant<int, VT>{});
    };
    auto stage_fv = [&]() __attribute__((always_inline)) {
      _Float16* vd = sV + (VT * fvtb) * LDV + 8 * fvdb;
#pragma unroll
      for (int i = 0; i < VT; ++i) *reinterpret_cast<uint4*>(vd + i * LDV) = vo[i];
    };

    // Two-step path: waves 10-11 stage the V rows (4 tokens x 8 columns per
    // lane, the fv lane mapping) as they are, in the io type.  Rows past the
    // end are clamped loads, zeroed when staged.
    uint4 pv[4];
    // columns past a 32-wide slice read the slice's last 8 columns (staged as zeros)
    const int vcol = 8 * fvdb < vwidth ? 8 * fvdb : vwidth - 8;
    auto prefetch_v = [&](int64_t cv) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t t = cv * kC + VT * fvtb + u;
        const int64_t row = len > 0 ? bos + (t < len ? t : len - 1) : 0;  // a row of the sequence
        pv[u] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.v) + (row * p.HV + h) * p.DV +
                                                col_base + vcol);
      }
    };
    auto stage_v = [&](int64_t cv) __attribute__((always_inline)) {
      const int nk = valid_rows(cv);
      _Float16* vd = sV + (VT * fvtb) * LDV + 8 * fvdb;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint4 o = pv[u];
        const bool ok = VT * fvtb + u < nk && 8 * fvdb < vwidth;
        *reinterpret_cast<uint4*>(vd + u * LDV) = make_uint4(ok ? o.x : 0u, ok ? o.y : 0u, ok ? o.z : 0u,
                                                             ok ? o.w : 0u);
      }
    };

    // Fused path: the conv windows of this sequence's snapshot rows (the raw
    // inputs ending at each row, oldest first; before the sequence start, the
    // history), written by the conv waves in the last chunk's first phase,
    // while the chain runs that chunk.  Each workgroup writes its own v slice
    // (whose history only its conv waves read, in the prologue) and a
    // 1/members share of its key head's q and k channels (whose history the
    // q/k pass read in the previous launch).  Writes into the baseline slot
    // come last, after every read of that slot's history.
    // Its parameters are read after the loop through an opaque kernarg-segment
    // pointer and an opaque block index: loaded at kernel entry, they would
    // hold scalar registers through every role's loop (the kernel is at its
    // scalar register limit).  mixed, rs, vch, bos, len and hist are live in
    // the conv loop anyway.  The first 256 entries of the snapshot list are
    // loaded before the loop (lane l: entries l, 64 + l, 128 + l, 192 + l),
    // so the end waits on no list load.
    typedef __attribute__((address_space(4))) const ChunkParams kernarg_params;
    constexpr int kSnapBlocks = 4;
    int snap_row[kSnapBlocks], snap_slot[kSnapBlocks];
    auto snapshot_prefetch = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int k = 0; k < kSnapBlocks; ++k) {
        const int64_t i = 64 * k + lane;
        snap_row[k] = snap_slot[k] = -1;
        if (i < f.snap_count) {
          snap_row[k] = static_cast<int>(load_index(f.snap_rows, i, f.snap_rows_is64));
          snap_slot[k] = static_cast<int>(load_index(f.snap_slots, i, f.snap_slots_is64));
        }
      }
    };
    auto snapshot_windows = [&]() __attribute__((always_inline)) {
      kernarg_params* ka = (kernarg_params*)__builtin_amdgcn_kernarg_segment_ptr();
      asm volatile("" : "+s"(ka));
      kernarg_params& q = *ka;
      const int64_t count = q.front.snap_count;
      if (count == 0 || !fv_thread) return;
      uint32_t bid = blockIdx.x;
      asm volatile("" : "+s"(bid));
      const int64_t sl8 = bid / 8;
      const int mem = static_cast<int>(sl8 % q.members);
      const int64_t grp = (sl8 / q.members) * 8 + (bid % 8);
      const int64_t khq = grp % q.H;
      const int64_t cb = static_cast<int64_t>(mem % q.nvs) * 64;
      const int64_t vw_ = q.DV - cb < 64 ? q.DV - cb : 64;
      const int64_t share = (DK + q.members - 1) / q.members;
      const int64_t q0 = mem * share;
      const int64_t nq = q0 >= DK ? 0 : (DK - q0 < share ? DK - q0 : share);
      const int64_t nch = 2 * nq + vw_;
      const int bslot = static_cast<int>(uniform_index(q.read_slots, grp / q.H, q.read_is64));
      uint16_t* const pool = static_cast<uint16_t*>(q.front.conv_state) + q.layer * q.front.conv_layer_stride;
      const int64_t sstride = q.front.conv_slot_stride;
      // Windows of up to 4 matching entries of a lane-indexed (row, slot)
      // block, taken lowest lane first: rows and slots are broadcast into
      // vector registers (ds_bpermute), and every load comes before any store
      // (the history of the baseline slot is read before a window may
      // overwrite it).  Non-baseline slots go first (pass 0).
      auto block = [&](int row, int sl, int pass) __attribute__((always_inline)) {
        const bool mine = sl >= 0 && row >= bos && row < bos + len && ((sl == bslot) == (pass == 1));
        uint64_t mask = __ballot(mine);
        while (mask) {
          int r[4], s[4], m = 0;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int b = mask ? __builtin_ctzll(mask) : 0;
            r[k] = __shfl(row, b);
            s[k] = __shfl(sl, b);
            if (mask) {
              mask &= mask - 1;
              m = k + 1;
            }
          }
          for (int64_t u = fst; u < nch; u += 128) {
            const int64_t ch = u < nq ? khq * DK + q0 + u
                                      : (u < 2 * nq ? q.front.key_dim + khq * DK + q0 + (u - nq) : vch + (u - 2 * nq));
            uint16_t w[4][3];
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
              for (int j = 0; j < 3; ++j) {
                const int64_t pos = static_cast<int64_t>(r[k]) - 2 + j;
                w[k][j] = k >= m ? 0
                                 : (pos >= bos ? mixed[pos * rs + ch] : (hist ? hist[ch * 3 + (pos - bos + 3)] : 0));
              }
#pragma unroll
            for (int k = 0; k < 4; ++k)
              if (k < m) {
#pragma unroll
                for (int j = 0; j < 3; ++j) pool[static_cast<int64_t>(s[k]) * sstride + ch * 3 + j] = w[k][j];
              }
          }
        }
      };
      for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
        for (int k = 0; k < kSnapBlocks; ++k) block(snap_row[k], snap_slot[k], pass);
        for (int64_t i0 = 64 * kSnapBlocks; i0 < count; i0 += 64) {  // entries past the prefetched ones
          const int64_t i = i0 + lane;
          int row = -1, sl = -1;
          if (i < count) {
            row = static_cast<int>(load_index(q.front.snap_rows, i, q.front.snap_rows_is64));
            sl = static_cast<int>(load_index(q.front.snap_slots, i, q.front.snap_slots_is64));
          }
          block(row, sl, pass);
        }
      }
    };

    // Waves 4-5 (inverses), 6-9 (tiles, K/Q staging) and 10-11 (v conv on the
    // fused path or V staging on the two-step path, gates) run separate loops
    // with the same barrier sequence.  Staging and
    // prefetches run unconditionally, also for chunks past the end (their
    // loads are masked off or clamped and their LDS targets are free): a
    // skipped consumer would leave the prefetch registers "maybe pending" at
    // the loop head, and the next prefetch would then wait for every load in
    // flight.
    if (sw < 2) {
      lds_barrier();  // P0
      inv_first(0);
      inv_second(0);
      tiles(0, true);
      lds_barrier();  // B(0)
      for (int64_t c = 0; c < nchunks; ++c) {
        if (c + 1 < nchunks) inv_first(c + 1);
        lds_barrier();  // M(c)
        if (c + 1 < nchunks) {
          inv_second(c + 1);
          tiles(c + 1, true);
        }
        lds_barrier();  // B(c+1)
      }
    } else if (sw >= 6) {
      prefetch_g(0);  // (both conv waves: the gate table on one, its decay factors on the other)
      stage_g(0);
      prefetch_g(1);
      stage_g(1);
      if constexpr (FUSED) {
        prefetch_fv(0);
        conv_v(0);
        stage_fv();
        prefetch_fv(1);
      } else {
        prefetch_v(0);
        stage_v(0);
        prefetch_v(1);
      }
      prefetch_g(2);
      if constexpr (EXT) {  // log rows of chunks 0 and 1 staged, 2 resolved, 3 loaded
        for (int64_t ck = 0; ck < 2; ++ck) {
          prefetch_log(ck);
          resolve_log();
          stage_log(ck);
        }
        prefetch_log(2);
        resolve_log();
        prefetch_log(3);
      }
      if constexpr (FUSED) snapshot_prefetch();
      lds_barrier();  // P0
      lds_barrier();  // B(0)
      // fused: the last chunk, with nothing left to convolve or stage, is
      // peeled off below and writes the conv windows while the chain runs it
      for (int64_t c = 0; c < (FUSED ? nchunks - 1 : nchunks); ++c) {
        if constexpr (FUSED) {
          conv_rows(c + 1, std::integral_constant<int, 0>{}, std::integral_constant<int, VT - 1>{});
          // keep the conv in this phase: the scheduler would otherwise sink
          // it past the barrier into the busier second phase
#pragma unroll
          for (int i = 0; i < VT - 1; ++i) asm volatile("" ::"v"(vo[i].x), "v"(vo[i].y), "v"(vo[i].z), "v"(vo[i].w));
        }
        lds_barrier();  // M(c)
        // the last conv row, before the row loads of chunk c + 2 replace vraw
        if constexpr (FUSED) conv_rows(c + 1, std::integral_constant<int, VT - 1>{}, std::integral_constant<int, 1>{});
        // The row loads for the conv of c + 2 go out first, so they have the
        // whole phase to arrive before that conv (right after the next
        // barrier).  Both waves issue the gate loads, after the row loads:
        // the loads in flight at the conv are then the same on either
        // wave, and the conv's waits never cover the younger gate loads.
        if constexpr (FUSED) {
          prefetch_fv(c + 2);
          stage_fv();
        } else {
          stage_v(c + 1);
          prefetch_v(c + 2);
        }
        stage_g(c + 2);
        prefetch_g(c + 3);
        if constexpr (EXT) {
          stage_log(c + 2);   // resolved one chunk ago
          resolve_log();      // chunk c + 3, loaded one chunk ago
          prefetch_log(c + 4);
        }
        lds_barrier();  // B(c+1)
      }
      if constexpr (FUSED) {
        snapshot_windows();
        lds_barrier();  // M(nchunks - 1)
        lds_barrier();  // B(nchunks)
      }
    } else {
      const int st = tid - 384;       // staging thread index (waves 6-9)
      const bool kq_thread = st >= 0 && st < KBLK;
      // K/Q block: 16-byte column block fastest (conflict-free 16-byte LDS writes)
      const int ktb = st / DB, kdb = st % DB;
      // row 0 of the sequence, this thread's column block (threads past KBLK
      // read block 0: their loads are never staged)
      const int kcol = kq_thread ? 8 * kdb : 0;
      // this key head's row 0 of the sequence (wave-uniform)
      const uint16_t* kseq = static_cast<const uint16_t*>(p.k) + (bos * p.H + kh) * DK;
      const uint16_t* qseq = static_cast<const uint16_t*>(p.q) + (bos * p.H + kh) * DK;
      const int64_t krow = p.H * DK;
      const uint32_t row_bytes = static_cast<uint32_t>(krow * 2);
      // the lane's byte offsets inside a chunk: rows 4 ktb + u, its column block
      uint32_t lane_off[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) lane_off[u] = static_cast<uint32_t>(4 * ktb + u) * row_bytes + 2 * kcol;
      uint4 pk[4], pq[4];

      // Every thread loads every chunk through a buffer resource per chunk
      // whose range ends at the sequence end: rows past it read as zeros (no
      // branch, so no prefetch register is left maybe-pending, and no address
      // arithmetic per load).  Those rows only meet beta = 0 (R and v' rows
      // zero), strictly earlier columns in L and M, and outputs that are not
      // stored.
      auto prefetch_kq = [&](int64_t ck) __attribute__((always_inline)) {
        const int64_t left = len - ck * kC;  // rows of the chunk inside the sequence
        const uint32_t nrec = static_cast<uint32_t>(left <= 0 ? 0 : (left < kC ? left : kC)) * row_bytes;
        const __amdgpu_buffer_rsrc_t kr =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kseq + ck * kC * krow), 0, nrec, 0x00020000);
        const __amdgpu_buffer_rsrc_t qr =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(qseq + ck * kC * krow), 0, nrec, 0x00020000);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          pk[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kr, lane_off[u], 0, 0));
          pq[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(qr, lane_off[u], 0, 0));
        }
      };
      auto stage_kq = [&](int64_t ck) __attribute__((always_inline)) {
        if (kq_thread) {
          // rows 4 ktb + u share the swizzle a = ktb mod 4: chunks 2 kdb and
          // 2 kdb + 1 go to (2 kdb) ^ a and (2 kdb + 1) ^ a, as two 8-byte writes
          const int a = ktb & 3;
          const int o0 = 4 * ((2 * kdb) ^ a), o1 = 4 * ((2 * kdb + 1) ^ a);
          _Float16* kd = sK + (ck % 3) * kC * LDK + (4 * ktb) * LDK;
          _Float16* qd = sQ + (ck & 1) * kC * LDQ + (4 * ktb) * LDQ;
#pragma unroll
          for (int u = 0; u < 4; ++u) {  // (fused: q and k arrive as f16 operands)
            const uint4 kv = FUSED ? pk[u] : to_f16x8<IOT>(pk[u]);
            const uint4 qv = FUSED ? pq[u] : to_f16x8<IOT>(pq[u]);
            *reinterpret_cast<uint2*>(kd + u * LDK + o0) = make_uint2(kv.x, kv.y);
            *reinterpret_cast<uint2*>(kd + u * LDK + o1) = make_uint2(kv.z, kv.w);
            *reinterpret_cast<uint2*>(qd + u * LDQ + o0) = make_uint2(qv.x, qv.y);
            *reinterpret_cast<uint2*>(qd + u * LDQ + o1) = make_uint2(qv.z, qv.w);
          }
        }
      };
      // ---- prologue: chunks 0 and 1 staged, chunk 0 solved
      prefetch_kq(0);
      stage_kq(0);
      prefetch_kq(1);
      stage_kq(1);
      lds_barrier();  // P0
      tiles(0, false);
      lds_barrier();  // B(0)
      // The loads of chunk c + 2 go out at the start of the first phase, which
      // has few other memory operations (the second carries the chain's
      // stores and the conv waves' row loads), and arrive while the tiles run.
      for (int64_t c = 0; c < nchunks; ++c) {
        prefetch_kq(c + 2);
        if (c + 1 < nchunks) tiles(c + 1, false);
        lds_barrier();  // M(c)
        stage_kq(c + 2);
        lds_barrier();  // B(c+1)
      }
    }
  }
}

template <int DK, class IOT, class ST, bool FUSED>
int launch_typed(const ChunkParams& p, int64_t groups, hipStream_t stream) {
  const int64_t blocks = ((groups + 7) / 8) * 8 * p.members;
  if (blocks > 0x7fffffff) {
    set_error("gdn_chunk_gated_delta_rule: grid too large");
    return GDN_ERR_INVALID;
  }
  const dim3 grid(static_cast<unsigned>(blocks));
  if constexpr (FUSED) {  // the fused prefill takes 64-token checkpoints into a plain pool
    hipLaunchKernelGGL((chunk_chain_kernel<DK, IOT, ST, true, false>), grid, dim3(kThreads), 0, stream, p);
  } else if (p.gran < kC || p.frames) {
    hipLaunchKernelGGL((chunk_chain_kernel<DK, IOT, ST, false, true>), grid, dim3(kThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((chunk_chain_kernel<DK, IOT, ST, false, false>), grid, dim3(kThreads), 0, stream, p);
  }
  return GDN_LAUNCH_CHECK("gdn_chunk_gated_delta_rule launch");
}

template <int DK, bool FUSED>
int launch_dk(const ChunkParams& p, int io, int st, int64_t groups, hipStream_t s) {
  if (io == GDN_BF16 && st == GDN_F32) return launch_typed<DK, bf16, float, FUSED>(p, groups, s);
  if (io == GDN_BF16 && st == GDN_BF16) return launch_typed<DK, bf16, bf16, FUSED>(p, groups, s);
  if (io == GDN_F16 && st == GDN_F32) return launch_typed<DK, f16, float, FUSED>(p, groups, s);
  if (io == GDN_F16 && st == GDN_F16) return launch_typed<DK, f16, f16, FUSED>(p, groups, s);
  return GDN_ERR_UNSUPPORTED;
}

template <bool FUSED>
int launch_any(const ChunkParams& p, int64_t dk, int io_dtype, int state_dtype, int64_t groups, hipStream_t stream) {
  if (p.DV % 64 != 0 && (FUSED || p.DV != 32)) return GDN_ERR_UNSUPPORTED;
  if (dk == 128) return launch_dk<128, FUSED>(p, io_dtype, state_dtype, groups, stream);
  if (dk == 64) return launch_dk<64, FUSED>(p, io_dtype, state_dtype, groups, stream);
  if (dk == 32) return launch_dk<32, FUSED>(p, io_dtype, state_dtype, groups, stream);
  return GDN_ERR_UNSUPPORTED;
}

}  // namespace

int launch_chunk_chain(const ChunkParams& p, int64_t dk, int io_dtype, int state_dtype, int64_t groups,
                       hipStream_t stream) {
  return launch_any<false>(p, dk, io_dtype, state_dtype, groups, stream);
}

int launch_chunk_chain_fused(const ChunkParams& p, int64_t dk, int io_dtype, int state_dtype, int64_t groups,
                             hipStream_t stream) {
  return launch_any<true>(p, dk, io_dtype, state_dtype, groups, stream);
}

}  // namespace gdn

extern "C" int gdn_prefill_fused(const void* q, const void* k, const void* mixed, int64_t row_stride, int io_dtype,
                                 const void* weight, int kernel_width, const void* cu_seqlens, int cu_dtype,
                                 int64_t num_seqs, int64_t total_tokens, int64_t H, int64_t HV, int64_t dk,
                                 int64_t dv, void* conv_state, int64_t conv_slot_stride,
                                 int64_t conv_layer_stride, const float* g, const float* beta, void* state,
                                 int state_dtype,
                                 int64_t slot_stride, int64_t layer_stride, int64_t head_stride, int64_t layer,
                                 const void* baseline_slots, int baseline_dtype, const void* chunk_write_slots,
                                 int chunk_write_dtype, const void* final_write_slots, int final_write_dtype,
                                 const void* snapshot_rows, int rows_dtype, const void* snapshot_slots,
                                 int slots_dtype, int64_t snapshot_count, void* out, float scale, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(num_seqs >= 1 && total_tokens >= 0 && H > 0 && HV > 0 && HV % H == 0, "gdn_prefill_fused: bad sizes");
  GDN_REQUIRE(q && k && mixed && weight && cu_seqlens && conv_state && baseline_slots && g && beta && state &&
                  chunk_write_slots && out,
              "gdn_prefill_fused: null input");
  GDN_REQUIRE(snapshot_count >= 0 && snapshot_count <= 0x7fffffff &&
                  (snapshot_count == 0 || (snapshot_rows && snapshot_slots)),
              "gdn_prefill_fused: bad snapshot list");
  const bool covered = kernel_width == 4 && (io_dtype == GDN_BF16 || io_dtype == GDN_F16) && dv % 64 == 0 &&
                       (dk == 32 || dk == 64 || dk == 128) && row_stride % 8 == 0 && row_stride > 0 &&
                       row_stride < (int64_t(1) << 24) && aligned16(mixed) &&
                       aligned16(weight) && aligned16(conv_state) && conv_slot_stride % 8 == 0 &&
                       conv_layer_stride % 8 == 0 && (state_dtype == GDN_F32 || state_dtype == io_dtype);
  if (!covered) {
    set_error("gdn_prefill_fused: not covered (needs conv width 4, 16-bit io, dk in {32, 64, 128}, dv %% 64 == 0, "
              "16-byte aligned rows shorter than 2^24 elements and conv pool, fp32 or io-typed state)");
    return GDN_ERR_UNSUPPORTED;
  }
  ChunkParams p{};
  p.q = q; p.k = k; p.g = g; p.beta = beta;
  p.cu = cu_seqlens; p.cu_is64 = cu_dtype == GDN_I64;
  p.N = num_seqs; p.T = total_tokens; p.H = H; p.HV = HV; p.DV = dv;
  p.state = state; p.slot_stride = slot_stride; p.layer_stride = layer_stride; p.head_stride = head_stride;
  p.layer = layer;
  p.read_slots = baseline_slots; p.read_is64 = baseline_dtype == GDN_I64;
  p.cw_slots = chunk_write_slots; p.cw_is64 = chunk_write_dtype == GDN_I64;
  p.fw_slots = final_write_slots; p.fw_is64 = final_write_dtype == GDN_I64;
  p.out = out; p.v_new = nullptr; p.scale = scale;
  p.gran = kC;
  p.nvs = static_cast<int>(dv / 64);
  p.members = static_cast<int>((HV / H) * p.nvs);
  FrontIn& f = p.front;
  f.mixed = mixed; f.row_stride = row_stride; f.weight = weight;
  f.conv_state = conv_state; f.conv_slot_stride = conv_slot_stride; f.conv_layer_stride = conv_layer_stride;
  f.key_dim = H * dk;
  f.snap_rows = snapshot_rows; f.snap_rows_is64 = rows_dtype == GDN_I64;
  f.snap_slots = snapshot_slots; f.snap_slots_is64 = slots_dtype == GDN_I64;
  f.snap_count = snapshot_count;
  return launch_chunk_chain_fused(p, dk, io_dtype, state_dtype, num_seqs * H, static_cast<hipStream_t>(stream));
}
