// Parameters shared by the chunked gated-delta-rule kernels (chunk.hip,
// chunk_chain.hip).
#pragma once

#include "common.hpp"

namespace gdn {

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
  int nvs;      // 64-column v slices per head
  int members;  // workgroups per (sequence, key head)
};

// Register-chain kernel (chunk_chain.hip) for d_k in {32, 64, 128} and d_v a
// multiple of 64.  Returns GDN_ERR_UNSUPPORTED (without setting an error) for
// shapes or dtypes it does not cover, so the caller can use another kernel.
int launch_chunk_chain(const ChunkParams& p, int64_t dk, int io_dtype, int state_dtype, int64_t groups,
                       hipStream_t stream);

}  // namespace gdn
