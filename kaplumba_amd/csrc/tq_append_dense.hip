// Dense-rotation append (matrix cores).  Placeholder until the MFMA kernel lands.
#include "tq_common.h"

namespace tq {
struct AppendArgs;
int launch_append_dense(const AppendArgs&, int dim, int bits, int, hipStream_t) {
  return fail(TQ_ERR_UNSUPPORTED, "append: dense rotation (dim %d, bits %d) not built yet", dim, bits);
}
}  // namespace tq
