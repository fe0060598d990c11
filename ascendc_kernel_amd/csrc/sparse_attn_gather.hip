// Task1 true-gather variant (n_kv > 32): placeholder until the kernel lands.
#include "dsa_common.h"

int dsa_sparse_attn_gather_launch(const void*, const void*, const int32_t*, const float*, void*,
                                  int64_t, int64_t, int64_t, int64_t, int64_t, float,
                                  hipStream_t) {
  return DSA_ERR_UNSUPPORTED;
}
