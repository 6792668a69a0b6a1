// Opt-in validation of the index metadata a decode or prefill call reads.
//
// The reference asserts its preconditions on the host (attention/metal.py:122)
// and builds its indices from the page table it owns (attention/metal.py:145-152,
// attention/base.py:70-83). Here the indices live on the device, so a caller
// that wants the same guarantee runs this check over them before the attention
// launches: it walks exactly the entries those launches will read and records
// the first violation it finds in a status word. The attention kernels
// themselves are memory-safe for any metadata (index reads are clamped to
// kv_indptr[R], slots outside the pool read slot 0), but their results are then
// unspecified; this check turns such metadata into an error.
//
// Checks, per request r of R:
//   kv_indptr[0] >= 0, kv_indptr[r] <= kv_indptr[r+1], kv_indptr[R] <= num_indices
//   L_r = seq_lens[r] (or the CSR row length) >= 0 and its index entries
//   (L_r, or ceil(L_r / page_size) page ids) fit in its CSR row
//   every entry it reads names a slot (page) inside the pool
//   with q_indptr: q_indptr[0] == 0, non-decreasing, q_indptr[R] == num_tokens,
//   and E_r = q_indptr[r+1] - q_indptr[r] <= L_r
#include "msgl_common.h"

namespace msgl {
namespace {

constexpr int kValidateThreads = 256;

struct ValidateParams {
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* seq_lens;
  const int32_t* q_indptr;
  int64_t num_indices;
  int64_t num_slots;
  int32_t num_reqs;
  int32_t page_size;
  int32_t num_tokens;
  long long* status;  // [code, where, value]
};

__device__ __forceinline__ void report(long long* status, int code, long long where, long long value) {
  if (atomicCAS(reinterpret_cast<unsigned long long*>(status), 0ull, (unsigned long long)code) == 0ull) {
    status[1] = where;
    status[2] = value;
  }
}

__global__ void validate_clear_kernel(long long* status) {
  if (threadIdx.x < 3) status[threadIdx.x] = 0;
}

// One workgroup per request (grid-stride): thread 0 checks the request's
// offsets and length, all threads the index entries it reads.
__global__ __launch_bounds__(kValidateThreads) void validate_kernel(ValidateParams p) {
  for (int r = blockIdx.x; r < p.num_reqs; r += gridDim.x) {
    const int64_t ip0 = p.kv_indptr[r], ip1 = p.kv_indptr[r + 1];
    const int64_t L = p.seq_lens ? (int64_t)p.seq_lens[r] : ip1 - ip0;
    if (threadIdx.x == 0) {
      if (r == 0 && ip0 < 0) report(p.status, MSGL_META_KV_INDPTR, r, ip0);
      if (ip1 < ip0) report(p.status, MSGL_META_KV_INDPTR, r + 1, ip1);
      if (r == p.num_reqs - 1 && ip1 > p.num_indices) report(p.status, MSGL_META_KV_RANGE, r + 1, ip1);
      const int64_t need = L < 0 ? 0 : (p.page_size == 1 ? L : (L + p.page_size - 1) / p.page_size);
      if (L < 0 || need > ip1 - ip0) report(p.status, MSGL_META_SEQ_LEN, r, L);
      if (p.q_indptr) {
        const int64_t q0 = p.q_indptr[r], q1 = p.q_indptr[r + 1];
        if (r == 0 && q0 != 0) report(p.status, MSGL_META_Q_INDPTR, 0, q0);
        if (q1 < q0) report(p.status, MSGL_META_Q_INDPTR, r + 1, q1);
        if (r == p.num_reqs - 1 && q1 != p.num_tokens) report(p.status, MSGL_META_Q_INDPTR, r + 1, q1);
        if (q1 - q0 > L) report(p.status, MSGL_META_EXTEND, r, q1 - q0);
      }
    }
    // the entries the attention kernels read for this request, inside kv_indices
    const int64_t need = L <= 0 ? 0 : (p.page_size == 1 ? L : (L + p.page_size - 1) / p.page_size);
    const int64_t lo = ip0 < 0 ? 0 : ip0;
    int64_t hi = ip0 + need;
    if (hi > ip1) hi = ip1;
    if (hi > p.num_indices) hi = p.num_indices;
    for (int64_t i = lo + threadIdx.x; i < hi; i += kValidateThreads) {
      const int64_t s = p.kv_indices[i];
      const bool ok = p.page_size == 1 ? (s >= 0 && s < p.num_slots)
                                       : (s >= 0 && (s + 1) * (int64_t)p.page_size <= p.num_slots);
      if (!ok) report(p.status, MSGL_META_SLOT, i, s);
    }
  }
}

}  // namespace
}  // namespace msgl

extern "C" int msgl_validate_metadata(const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                                      const int32_t* q_indptr, int32_t num_reqs, int32_t page_size,
                                      int64_t num_indices, int64_t num_slots, int32_t num_tokens, int64_t* status,
                                      void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(status != nullptr && (uintptr_t)status % 8 == 0, "msgl_validate_metadata: status must be int64[3]");
  MSGL_CHECK_ARG(num_reqs >= 0 && page_size >= 1 && num_indices >= 0 && num_slots > 0 && num_tokens >= 0,
                 "msgl_validate_metadata: bad sizes");
  MSGL_CHECK_ARG(page_size == 1 || seq_lens != nullptr,
                 "msgl_validate_metadata: page_size > 1 needs seq_lens (as the attention calls do)");
  MSGL_CHECK_ARG(num_reqs == 0 || (kv_indptr != nullptr && (kv_indices != nullptr || num_indices == 0)),
                 "msgl_validate_metadata: null kv_indptr or kv_indices");
  hipStream_t s = (hipStream_t)stream;
  long long* st = reinterpret_cast<long long*>(status);
  hipLaunchKernelGGL(validate_clear_kernel, dim3(1), dim3(64), 0, s, st);
  MSGL_CHECK_LAUNCH("msgl_validate_metadata (clear)");
  if (num_reqs == 0) return MSGL_OK;
  ValidateParams p;
  p.kv_indptr = kv_indptr;
  p.kv_indices = kv_indices;
  p.seq_lens = seq_lens;
  p.q_indptr = q_indptr;
  p.num_indices = num_indices;
  p.num_slots = num_slots;
  p.num_reqs = num_reqs;
  p.page_size = page_size;
  p.num_tokens = num_tokens;
  p.status = st;
  const int grid = num_reqs < 4096 ? num_reqs : 4096;
  hipLaunchKernelGGL(validate_kernel, dim3(grid), dim3(kValidateThreads), 0, s, p);
  MSGL_CHECK_LAUNCH("msgl_validate_metadata");
  return MSGL_OK;
}
