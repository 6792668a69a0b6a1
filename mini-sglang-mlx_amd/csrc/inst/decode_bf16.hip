// Paged decode kernels for bf16 queries over a bf16 pool: every built
// head_dim and query-head group.
#include "decode_launch.h"

int msgl::dec::decode_op_bf16(const DecodeOp& op, int head_dim, int group) {
  return dispatch_dim<bf16_t>(OpRun{op}, head_dim, group);
}
