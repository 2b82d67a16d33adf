// Split-K partial attention kernels for head dim 256 (all bit widths, row-group sizes).
#include "tq_attn_impl.h"

namespace tq {
int launch_partial_d256(const AttnParams& p, int kv_kind, int kv_dtype, int kb, int vb,
                       hipStream_t st) {
  return launch_partial_dim<256>(p, kv_kind, kv_dtype, kb, vb, st);
}
}  // namespace tq
