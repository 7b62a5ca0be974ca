/* Plain C99 caller of libaac_attn.so through include/aac_attn.h: the header
 * compiles as C, every declared entry point links, and the host-side argument
 * checks answer without a GPU (no device memory is touched). */
#include <stdio.h>
#include <string.h>

#include "aac_attn.h"

int main(void) {
  int fails = 0;
  if (aac_abi_version() != AAC_ABI_VERSION) { puts("abi version"); ++fails; }
  if (!strstr(aac_strerror(AAC_ERR_SCRATCH), "scratch")) { puts("strerror"); ++fails; }
  /* null pointers with work to do: rejected before any launch */
  if (aac_kv_store(NULL, NULL, 1024, 1024, NULL, NULL, 16, NULL, 4, 8, 128, AAC_DTYPE_BF16, NULL) !=
      AAC_ERR_INVALID_ARGUMENT) { puts("kv_store"); ++fails; }
  /* fp32 prefill is not built for the MFMA path */
  if (aac_prefill_varlen(NULL, NULL, NULL, 0, 0, 0, NULL, NULL, 1, 1, 1, 16, 8, 128, 1.0f, 1, NULL, 0,
                         NULL, 0, AAC_DTYPE_FP32, NULL) != AAC_ERR_UNSUPPORTED) { puts("prefill"); ++fails; }
  /* a split-K plan larger than the no-allocation scratch: refused on the host */
  if (aac_decode_workspace_bytes(1024, 32, 8, 128, 256, 256, 0, 256) <= AAC_DECODE_SCRATCH_BYTES) {
    puts("workspace size"); ++fails;
  }
  if (aac_decode_paged_noalloc((void*)4096, 4096, (void*)4096, (void*)4096, 1 << 16, 256, (void*)4096,
                               256, (void*)4096, 1024, 0, 32, 8, 128, 0.088f, (void*)4096, 4096, 256,
                               AAC_DTYPE_BF16, NULL) != AAC_ERR_SCRATCH) { puts("noalloc"); ++fails; }
  /* every other entry point is referenced, so a missing export fails the link */
  void* volatile refs[] = {(void*)aac_kv_append_paged, (void*)aac_prefill_varlen_store,
                           (void*)aac_prefill_workspace_bytes, (void*)aac_decode_paged,
                           (void*)aac_decode_append_paged, (void*)aac_rmsnorm,
                           (void*)aac_qk_norm_rope_store, (void*)aac_silu_mul, (void*)aac_gemm_nt,
                           (void*)aac_qkv_norm_rope_store, (void*)aac_argmax_rows,
                           (void*)aac_kv_export_paged, (void*)aac_kv_import_paged};
  for (size_t i = 0; i < sizeof(refs) / sizeof(refs[0]); ++i)
    if (!refs[i]) { puts("missing export"); ++fails; }
  puts(fails ? "FAIL" : "OK");
  return fails != 0;
}
