// Chunked gated delta rule (placeholder until the MFMA kernel lands).
#include "common.hpp"

extern "C" int gdn_chunk_gated_delta_rule(const void*, const void*, const void*, int, const float*, const float*,
                                          const void*, int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                                          void*, int, int64_t, int64_t, int64_t, int64_t, const void*, int,
                                          const void*, int, const void*, int, void*, void*, float, void*) {
  gdn::set_error("gdn_chunk_gated_delta_rule: not built yet");
  return GDN_ERR_UNSUPPORTED;
}
