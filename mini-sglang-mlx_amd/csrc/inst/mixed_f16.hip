// Single-launch mixed step kernels for fp16 queries over an fp16 pool:
// head_dim 64 and 128, query-head groups 1 to 8.
#include "mixed_launch.h"

int msgl::mixed_launch_f16(const pf::PrefillParams& pp, const dec::DecodeParams& dp, int batch, int max_e,
                       int head_dim, int group, hipStream_t stream) {
  return mixed_dim<f16_t>(pp, dp, batch, max_e, head_dim, group, stream);
}
