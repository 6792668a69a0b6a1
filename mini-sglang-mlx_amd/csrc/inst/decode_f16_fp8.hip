// Paged decode kernels for fp16 queries over an fp8 e4m3 pool: every built
// head_dim and query-head group.
#include "decode_launch.h"

int msgl::dec::decode_op_f16_fp8(const DecodeOp& op, int head_dim, int group) {
  return dispatch_dim<f16_t, fp8e4m3>(OpRun{op}, head_dim, group);
}
