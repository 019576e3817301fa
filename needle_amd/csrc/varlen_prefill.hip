// Varlen causal prefill over the paged cache (kernel lands in a later commit).
#include "ndl_common.hpp"

extern "C" int ndl_varlen_prefill(void*, const void*, int64_t, const void*, int64_t,
                                  const int32_t*, int64_t, int, const int32_t*, const int32_t*,
                                  int, int64_t, int, int, int, int, int, int, int, float,
                                  ndl_stream_t) {
  return NDL_ERR_UNSUPPORTED;
}
