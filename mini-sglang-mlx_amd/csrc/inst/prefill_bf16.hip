// Ragged prefill kernels for bf16 queries over a bf16 pool: every built
// head_dim and query-head group.
#include "prefill_launch.h"

int msgl::pf::prefill_launch_bf16(const PrefillParams& p, int max_e, int head_dim, int group, hipStream_t stream) {
  return prefill_dim<bf16_t>(p, max_e, head_dim, group, stream);
}
