// Ragged prefill kernels for fp16 queries over an fp8 e4m3 pool: every built
// head_dim and query-head group.
#include "prefill_launch.h"

int msgl::pf::prefill_launch_f16_fp8(const PrefillParams& p, int max_e, int head_dim, int group, hipStream_t stream) {
  return prefill_dim<f16_t, fp8e4m3>(p, max_e, head_dim, group, stream);
}
