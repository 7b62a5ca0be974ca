// Library-level entry points of libaac_attn.so: ABI version and messages.
#include "aac_common.h"

extern "C" int aac_abi_version(void) { return AAC_ABI_VERSION; }

extern "C" const char* aac_strerror(int code) {
  switch (code) {
    case AAC_OK: return "success";
    case AAC_ERR_INVALID_ARGUMENT: return "invalid argument (null pointer or bad size)";
    case AAC_ERR_UNSUPPORTED: return "unsupported dtype, head_dim or GQA group";
    case AAC_ERR_MISALIGNED: return "pointer or stride not aligned for vector access";
    case AAC_ERR_WORKSPACE: return "split-K workspace missing or too small";
    case AAC_ERR_SHAPE: return "inconsistent shape arguments";
    case AAC_ERR_SCRATCH:
      return "the split-K plan needs more than the library's static scratch "
             "(AAC_DECODE_SCRATCH_BYTES); use the entry point with a workspace";
    default: break;
  }
  if (code > 0) return hipGetErrorString((hipError_t)code);
  return "unknown aac error";
}
