// Ragged prefill kernels for fp32 queries over an fp32 pool: every built
// head_dim and query-head group.
#include "prefill_launch.h"

int msgl::pf::prefill_launch_f32(const PrefillParams& p, int max_e, int head_dim, int group, hipStream_t stream) {
  return prefill_dim<float>(p, max_e, head_dim, group, stream);
}
