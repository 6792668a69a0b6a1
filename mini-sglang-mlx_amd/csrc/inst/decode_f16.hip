// Paged decode kernels for fp16 queries over an fp16 pool: every built
// head_dim and query-head group.
#include "decode_launch.h"

int msgl::dec::decode_op_f16(const DecodeOp& op, int head_dim, int group) {
  return dispatch_dim<f16_t>(OpRun{op}, head_dim, group);
}
