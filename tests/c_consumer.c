/* A plain C99 consumer of the C ABI: includes both public headers, links
 * libmoe_dispatch.so (and libmoe_probes.so for the probes) and calls entry points whose argument checks fail before
 * any HIP call (no GPU needed). Prints one line per check; exit status 0 when
 * every call returned what the header documents. */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "moe_dispatch.h"
#include "moe_probes.h"

static int failures = 0;

static void expect(const char *what, int got, int want) {
  printf("%s: %d (%s)%s\n", what, got, moe_status_string(got), got == want ? "" : "  <-- unexpected");
  if (got != want) ++failures;
}

int main(void) {
  void *fake = (void *)(uintptr_t)0x1000; /* never dereferenced: validation fails first */
  if (moe_abi_version() != MOE_DISPATCH_ABI_VERSION) {
    printf("abi version %d != header %d\n", moe_abi_version(), MOE_DISPATCH_ABI_VERSION);
    return 1;
  }
  expect("moe_topk negative T", moe_topk((const float *)fake, -1, 8, 2, NULL, NULL, NULL, NULL, NULL), MOE_ERR_SHAPE);
  expect("moe_row_id_map null mask",
         moe_row_id_map(NULL, 16, 4, (int64_t *)fake, NULL, NULL, NULL, NULL, 0, fake, 4096, NULL), MOE_ERR_INVALID_ARG);
  expect("moe_permute bad layout",
         moe_permute((const moe_bf16_t *)fake, 4, 8, fake, MOE_IDX_I64, 7, 2, NULL, (moe_bf16_t *)fake, NULL, 8, 0, NULL, 0,
                     NULL),
         MOE_ERR_INVALID_ARG);
  expect("moe_grouped_gemm odd SwiGLU N",
         moe_grouped_gemm((const moe_bf16_t *)fake, 4, 16, (const moe_bf16_t *)fake, 1, 9, (const int32_t *)fake,
                          MOE_EPILOGUE_SWIGLU, (moe_bf16_t *)fake, NULL, 0, NULL),
         MOE_ERR_SHAPE);
  expect("moe_grouped_gemm_dgrad G=0",
         moe_grouped_gemm_dgrad((const moe_bf16_t *)fake, 4, 16, (const moe_bf16_t *)fake, 0, 16, (const int32_t *)fake,
                                (moe_bf16_t *)fake, NULL, 0, NULL),
         MOE_ERR_CAPACITY);
  expect("moe_map_extent small workspace",
         moe_map_extent(fake, MOE_IDX_I64, 16, (int64_t *)fake, fake, 8, NULL), MOE_ERR_WORKSPACE);
  expect("moe_probe_mfma waves not a multiple of 4", moe_probe_mfma(6, 1, (float *)fake, NULL), MOE_ERR_SHAPE);
  if (strlen(moe_last_error()) == 0) {
    printf("moe_last_error is empty after a failed call\n");
    ++failures;
  }
  printf("workspace sizes: row_id_map(16384, 64) = %zu, map_extent(5242880) = %zu\n",
         moe_row_id_map_workspace_size(16384, 64), moe_map_extent_workspace_size(5242880));
  return failures == 0 ? 0 : 1;
}
