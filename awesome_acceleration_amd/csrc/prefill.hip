// placeholder: replaced by the MFMA prefill kernel
#include "aac_common.h"
extern "C" int aac_prefill_varlen(const void*, const void*, const void*, int64_t, int64_t, int64_t,
                                  const int32_t*, const int32_t*, int32_t, int32_t, int32_t, int32_t,
                                  int32_t, int32_t, float, int32_t, void*, int64_t, int32_t, void*) {
  return AAC_ERR_UNSUPPORTED;
}
extern "C" int aac_prefill_varlen_store(const void*, const void*, const void*, int64_t, int64_t, int64_t,
                                        const int32_t*, const int32_t*, int32_t, int32_t, int32_t,
                                        int32_t, int32_t, int32_t, float, int32_t, void*, int64_t,
                                        void*, void*, int64_t, const int64_t*, int32_t, void*) {
  return AAC_ERR_UNSUPPORTED;
}
