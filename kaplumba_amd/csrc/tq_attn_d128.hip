// Split-K partial attention kernels for head dim 128 (all bit widths, row-group sizes).
#include "tq_attn_impl.h"

namespace tq {
int launch_partial_d128(const AttnParams& p, int kv_kind, int kv_dtype, int kb, int vb,
                       hipStream_t st) {
  return launch_partial_dim<128>(p, kv_kind, kv_dtype, kb, vb, st);
}
}  // namespace tq

#ifdef TQ_PHASE_STAMPS
// Phase stamps of the last attn_stage_kernel<128, *, *> launch (stamps build only).
extern "C" int tq_dbg_stage_stamps(void* dst, long long bytes) {
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(tq::g_stage_stamps), bytes) == hipSuccess ? 0 : 1;
}
#endif
