// Causal chunked-prefill paged attention (placeholder until the MFMA kernel lands).
#include "ifn_common.hpp"

extern "C" size_t ifn_paged_prefill_workspace_bytes(int32_t, int32_t, int32_t, int32_t, int32_t,
                                                    int32_t) {
  return 256;
}

extern "C" int ifn_paged_prefill(void*, const void*, const void*, int64_t, const int32_t*, int32_t,
                                 int32_t, int32_t, int32_t, int32_t, int32_t, int32_t, float, void*,
                                 size_t, void*) {
  return IFN_ERR_UNSUPPORTED;
}
