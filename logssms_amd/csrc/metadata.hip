// Batched metadata copies for fixed-capacity graph replay: one launch moves a
// group of small index tensors (python/logssms/kernel/metadata.py:77-150,
// copy_metadata / pad_metadata, used by the mixed prefill/decode graph
// buckets of layers/linear_attention_backend/mixed.py).
//
// Roofline: launch latency.  A group holds a few hundred to a few thousand
// indices; one launch per group replaces one copy_/fill_ launch per tensor.
// The field table travels in the kernel arguments, so a captured graph
// replays the same pointers.
#include "common.hpp"

namespace gdn {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxFields = 16;

struct Field {
  const char* src;
  char* dst;
  int64_t length;    // source elements
  int64_t capacity;  // destination elements (pad) or = length (copy)
  int64_t src_stride, dst_stride;  // in elements (copy)
  int64_t fill, tail;              // pad values
  int elem;                        // bytes per element: 1, 2, 4 or 8
};

struct FieldTable {
  Field f[kMaxFields];
};

__device__ __forceinline__ int64_t load_int(const char* p, int elem) {
  switch (elem) {
    case 8: return *reinterpret_cast<const int64_t*>(p);
    case 4: return *reinterpret_cast<const int32_t*>(p);
    case 2: return *reinterpret_cast<const int16_t*>(p);
    default: return *reinterpret_cast<const int8_t*>(p);
  }
}
__device__ __forceinline__ void store_int(char* p, int elem, int64_t v) {
  switch (elem) {
    case 8: *reinterpret_cast<int64_t*>(p) = v; break;
    case 4: *reinterpret_cast<int32_t*>(p) = static_cast<int32_t>(v); break;
    case 2: *reinterpret_cast<int16_t*>(p) = static_cast<int16_t>(v); break;
    default: *reinterpret_cast<int8_t*>(p) = static_cast<int8_t>(v); break;
  }
}

// grid (element blocks, fields): dst[i * dst_stride] = src[i * src_stride], i < length.
__global__ __launch_bounds__(kThreads) void metadata_copy_kernel(FieldTable t) {
  const Field& f = t.f[blockIdx.y];
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= f.length) return;
  store_int(f.dst + i * f.dst_stride * f.elem, f.elem, load_int(f.src + i * f.src_stride * f.elem, f.elem));
}

// grid (element blocks, fields): dst[i] = src[i] for i < length; beyond it the
// fill value, or for a pair table (tail >= 0) the pair (0, tail).
__global__ __launch_bounds__(kThreads) void metadata_pad_kernel(FieldTable t) {
  const Field& f = t.f[blockIdx.y];
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= f.capacity) return;
  int64_t v;
  if (i < f.length) v = load_int(f.src + i * f.elem, f.elem);
  else v = f.tail >= 0 ? (i % 2 == 1 ? f.tail : 0) : f.fill;
  store_int(f.dst + i * f.elem, f.elem, v);
}

int launch_fields(bool pad, const Field* fields, int n, hipStream_t s) {
  for (int base = 0; base < n; base += kMaxFields) {
    const int m = n - base < kMaxFields ? n - base : kMaxFields;
    FieldTable t{};
    int64_t most = 0;
    for (int j = 0; j < m; ++j) {
      t.f[j] = fields[base + j];
      const int64_t count = pad ? t.f[j].capacity : t.f[j].length;
      most = count > most ? count : most;
    }
    if (most == 0) continue;
    const int64_t blocks = (most + kThreads - 1) / kThreads;
    GDN_REQUIRE(blocks <= 0x7fffffff, "metadata: too many elements");
    if (pad)
      hipLaunchKernelGGL(metadata_pad_kernel, dim3(static_cast<unsigned>(blocks), m), dim3(kThreads), 0, s, t);
    else
      hipLaunchKernelGGL(metadata_copy_kernel, dim3(static_cast<unsigned>(blocks), m), dim3(kThreads), 0, s, t);
    const int rc = GDN_LAUNCH_CHECK(pad ? "gdn_metadata_pad launch" : "gdn_metadata_copy launch");
    if (rc != GDN_OK) return rc;
  }
  return GDN_OK;
}

bool elem_ok(int e) { return e == 1 || e == 2 || e == 4 || e == 8; }

}  // namespace
}  // namespace gdn

extern "C" int gdn_metadata_copy(const void* const* srcs, void* const* dsts, const int64_t* lengths,
                                 const int64_t* src_strides, const int64_t* dst_strides, const int* elem_sizes,
                                 int fields, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(fields >= 0, "gdn_metadata_copy: negative field count");
  if (fields == 0) return GDN_OK;
  GDN_REQUIRE(srcs && dsts && lengths && src_strides && dst_strides && elem_sizes, "gdn_metadata_copy: null table");
  Field table[64];
  for (int base = 0; base < fields; base += 64) {
    const int m = fields - base < 64 ? fields - base : 64;
    for (int j = 0; j < m; ++j) {
      const int i = base + j;
      GDN_REQUIRE(elem_ok(elem_sizes[i]) && lengths[i] >= 0, "gdn_metadata_copy: field %d: bad size", i);
      GDN_REQUIRE(lengths[i] == 0 || (srcs[i] && dsts[i]), "gdn_metadata_copy: field %d: null pointer", i);
      table[j] = Field{static_cast<const char*>(srcs[i]), static_cast<char*>(dsts[i]), lengths[i], lengths[i],
                       src_strides[i], dst_strides[i], 0, -1, elem_sizes[i]};
    }
    const int rc = launch_fields(false, table, m, static_cast<hipStream_t>(stream));
    if (rc != GDN_OK) return rc;
  }
  return GDN_OK;
}

extern "C" int gdn_metadata_pad(const void* const* srcs, void* const* dsts, const int64_t* lengths,
                                const int64_t* capacities, const int64_t* fills, const int64_t* tails,
                                const int* elem_sizes, int fields, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(fields >= 0, "gdn_metadata_pad: negative field count");
  if (fields == 0) return GDN_OK;
  GDN_REQUIRE(srcs && dsts && lengths && capacities && fills && tails && elem_sizes, "gdn_metadata_pad: null table");
  Field table[64];
  for (int base = 0; base < fields; base += 64) {
    const int m = fields - base < 64 ? fields - base : 64;
    for (int j = 0; j < m; ++j) {
      const int i = base + j;
      GDN_REQUIRE(elem_ok(elem_sizes[i]) && lengths[i] >= 0 && capacities[i] >= lengths[i],
                  "gdn_metadata_pad: field %d: source longer than its capacity", i);
      GDN_REQUIRE(capacities[i] == 0 || dsts[i], "gdn_metadata_pad: field %d: null destination", i);
      GDN_REQUIRE(lengths[i] == 0 || srcs[i], "gdn_metadata_pad: field %d: null source", i);
      table[j] = Field{static_cast<const char*>(srcs[i]), static_cast<char*>(dsts[i]), lengths[i], capacities[i],
                       1, 1, fills[i], tails[i], elem_sizes[i]};
    }
    const int rc = launch_fields(true, table, m, static_cast<hipStream_t>(stream));
    if (rc != GDN_OK) return rc;
  }
  return GDN_OK;
}

// LogState prefill write plan (python/logssms/kernel/metadata.py:150-178,
// make_logstate_prefill_writes): from the per-token log slots, page offsets
// and the host plan [conv slot | conv granule | log enabled] (conv slot -2:
// the token's own log slot at granule offset / granularity) build
// [log write slots | conv token slots | conv token granules].
namespace gdn {
namespace {

__global__ __launch_bounds__(kThreads) void logstate_prefill_writes_kernel(const void* logs, const void* offsets,
                                                                          int offsets_is64, const int32_t* plan,
                                                                          void* out, int out_is64, int64_t count,
                                                                          int64_t granularity) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (r >= count) return;
  const int64_t slot = load_index(logs, r, out_is64);
  const int64_t conv = plan[r];
  const int64_t values[3] = {plan[2 * count + r] != 0 ? slot : -1, conv == -2 ? slot : conv,
                             conv == -2 ? load_index(offsets, r, offsets_is64) / granularity : plan[count + r]};
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    if (out_is64)
      static_cast<int64_t*>(out)[j * count + r] = values[j];
    else
      static_cast<int32_t*>(out)[j * count + r] = static_cast<int32_t>(values[j]);
  }
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_logstate_prefill_writes(const void* log_slots, int slots_dtype, const void* token_offsets,
                                           int offsets_dtype, const int32_t* plan, void* out, int64_t count,
                                           int64_t granularity, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(count >= 0 && granularity > 0, "gdn_logstate_prefill_writes: bad sizes");
  if (count == 0) return GDN_OK;
  GDN_REQUIRE(log_slots && token_offsets && plan && out, "gdn_logstate_prefill_writes: null input");
  GDN_REQUIRE((slots_dtype == GDN_I32 || slots_dtype == GDN_I64) && (offsets_dtype == GDN_I32 || offsets_dtype == GDN_I64),
              "gdn_logstate_prefill_writes: index tensors must be int32 or int64");
  const int64_t blocks = (count + kThreads - 1) / kThreads;
  GDN_REQUIRE(blocks <= 0x7fffffff, "gdn_logstate_prefill_writes: too many tokens");
  hipLaunchKernelGGL(logstate_prefill_writes_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), log_slots, token_offsets, offsets_dtype == GDN_I64, plan, out,
                     slots_dtype == GDN_I64, count, granularity);
  return GDN_LAUNCH_CHECK("gdn_logstate_prefill_writes");
}

// Decode slots from the engine's prepared batch packet (kernel/metadata.py:
// 266-320, gather_linear_slots): per request i, row = table_ids[i] and
// position = cached_lens[i] of the state table (and, for LogState, the work
// table and the request's KV location).
//   standard: out int64 [count, 2] = (state_table[row, position - 1, or the
//     row's last column when position is 0], state_table[row, position]);
//   LogState: out int32 [4, count] = (work_table[row, 0],
//     state_table[row, position], out_loc[i] mod page_size (floored), 0).
// A row outside the tables or a position outside [0, width) gives -1 slots.
namespace gdn {
namespace {

__global__ __launch_bounds__(kThreads) void gather_linear_slots_kernel(
    const void* tables, int tables_is64, const void* cached, int cached_is64, const void* state, int state_is64,
    int64_t rows, int64_t state_stride, int64_t width, const void* work, int work_is64, int64_t work_rows,
    int64_t work_stride, const void* out_loc, int loc_is64, int64_t page_size, void* out, int64_t count) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= count) return;
  const int64_t row = load_index(tables, i, tables_is64);
  const int64_t pos = load_index(cached, i, cached_is64);
  const bool ok = row >= 0 && row < rows && pos >= 0 && pos < width;
  const int64_t now = ok ? load_index(state, row * state_stride + pos, state_is64) : -1;
  if (work) {
    int32_t* o = static_cast<int32_t*>(out);
    const int64_t loc = load_index(out_loc, i, loc_is64);
    const int64_t r = loc % page_size;
    const bool wok = row >= 0 && row < work_rows;
    o[i] = wok ? static_cast<int32_t>(load_index(work, row * work_stride, work_is64)) : -1;
    o[count + i] = static_cast<int32_t>(now);
    o[2 * count + i] = static_cast<int32_t>(r < 0 ? r + page_size : r);
    o[3 * count + i] = 0;
  } else {
    int64_t* o = static_cast<int64_t*>(out);
    o[2 * i] = ok ? load_index(state, row * state_stride + (pos > 0 ? pos - 1 : width - 1), state_is64) : -1;
    o[2 * i + 1] = now;
  }
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_gather_linear_slots(const void* table_ids, int table_ids_dtype, const void* cached_lens,
                                       int cached_dtype, const void* state_table, int state_dtype,
                                       int64_t state_rows, int64_t state_width, int64_t state_row_stride,
                                       const void* work_table, int work_dtype, int64_t work_rows,
                                       int64_t work_row_stride,
                                       const void* out_loc, int out_loc_dtype, int64_t page_size, void* out,
                                       int64_t count, void* stream) {
  using namespace gdn;
  GDN_REQUIRE(count >= 0 && state_rows > 0 && state_width > 0 && state_row_stride >= state_width,
              "gdn_gather_linear_slots: bad sizes");
  if (count == 0) return GDN_OK;
  GDN_REQUIRE(table_ids && cached_lens && state_table && out, "gdn_gather_linear_slots: null input");
  GDN_REQUIRE(!work_table || (out_loc && page_size > 0 && work_row_stride > 0),
              "gdn_gather_linear_slots: LogState slots need the work table, out_loc and the page size");
  const int64_t blocks = (count + kThreads - 1) / kThreads;
  GDN_REQUIRE(blocks <= 0x7fffffff, "gdn_gather_linear_slots: too many requests");
  hipLaunchKernelGGL(gather_linear_slots_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), table_ids, table_ids_dtype == GDN_I64, cached_lens,
                     cached_dtype == GDN_I64, state_table, state_dtype == GDN_I64, state_rows, state_row_stride,
                     state_width, work_table, work_dtype == GDN_I64, work_rows, work_row_stride, out_loc,
                     out_loc_dtype == GDN_I64, page_size, out, count);
  return GDN_LAUNCH_CHECK("gdn_gather_linear_slots");
}
