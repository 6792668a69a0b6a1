// Paged decode kernels for fp32 queries over an fp32 pool: every built
// head_dim and query-head group.
#include "decode_launch.h"

int msgl::dec::decode_op_f32(const DecodeOp& op, int head_dim, int group) {
  return dispatch_dim<float>(OpRun{op}, head_dim, group);
}
