// Per-step index construction on the GPU from a device copy of the page table
// (req_to_token), so a step's slot lists never cross PCIe.
//
// Restates, bit-exact:
//   scheduler/scheduler.py:154-157  positions = concat(arange(cached, device_len)),
//                                   out_loc = page_table[rows, positions]
//   attention/base.py:70-83         q_offsets = [0, cumsum(extend)], last_indices = q_offsets[1:] - 1
//   attention/metal.py:145-152      kv_indptr = [0, cumsum(lens)], kv_indices = page_table[rows, :len] (row-major)
// and, for page_size > 1, the page-level form the decode/prefill kernels take:
//   kv_indptr = [0, cumsum(ceil(len / page_size))], kv_indices = page_table[row, j * page_size] / page_size
// (pages are page-aligned runs of slots, scheduler/cache.py:138-143).
//
// Two launches on the caller's stream: a one-workgroup scan of the per-request
// counts (wavefront prefix sums, carried across 1024-request chunks), then a
// grid-stride fill in which every output element finds its request by binary
// search over the offsets (staged in LDS when they fit). Table reads outside
// [0, num_rows) x [0, row_stride) yield -1 instead of touching memory; writes
// stop at the caller's capacities. The totals are q_indptr[R] and kv_indptr[R].
#include "msgl_common.h"

namespace msgl {
namespace {

constexpr int kScanThreads = 1024;
constexpr int kFillThreads = 256;
constexpr int kLdsOffsets = 4096;  // offsets staged in LDS by the fill kernel (each array)

struct IndexParams {
  const int32_t* table;
  int64_t num_rows;
  int64_t row_stride;
  const int32_t* table_idx;
  const int32_t* cached_len;
  const int32_t* device_len;
  int num_reqs;
  int page_size;
  int32_t* q_indptr;
  int32_t* positions;
  int32_t* out_loc;
  int32_t* last_indices;
  int64_t token_capacity;
  int32_t* kv_indptr;
  int32_t* kv_indices;
  int64_t kv_capacity;
};

__device__ __forceinline__ int wave_inclusive_scan(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d);
    if (lane >= d) v += o;
  }
  return v;
}

// Block-wide inclusive scan of two counters; returns both, and leaves the
// block totals in tot[0..1] (all threads).
__device__ __forceinline__ void block_scan2(int& a, int& b, int* lds, int2& tot) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int NW = kScanThreads / 64;
  a = wave_inclusive_scan(a, lane);
  b = wave_inclusive_scan(b, lane);
  if (lane == 63) {
    lds[wave] = a;
    lds[NW + wave] = b;
  }
  __syncthreads();
  if (wave == 0) {
    int x = lane < NW ? lds[lane] : 0;
    int y = lane < NW ? lds[NW + lane] : 0;
    x = wave_inclusive_scan(x, lane);
    y = wave_inclusive_scan(y, lane);
    if (lane < NW) {
      lds[2 * NW + lane] = x;
      lds[3 * NW + lane] = y;
    }
  }
  __syncthreads();
  if (wave > 0) {
    a += lds[2 * NW + wave - 1];
    b += lds[3 * NW + wave - 1];
  }
  tot = make_int2(lds[3 * NW - 1], lds[4 * NW - 1]);
  __syncthreads();  // lds is reused by the next chunk
}

__global__ __launch_bounds__(kScanThreads) void scan_kernel(IndexParams p) {
  __shared__ int lds[4 * (kScanThreads / 64)];
  int carry_q = 0, carry_kv = 0;
  if (threadIdx.x == 0) {
    p.q_indptr[0] = 0;
    p.kv_indptr[0] = 0;
  }
  for (int base = 0; base < p.num_reqs; base += kScanThreads) {
    const int r = base + threadIdx.x;
    int e = 0, kv = 0;
    if (r < p.num_reqs) {
      const int c = p.cached_len[r], d = p.device_len[r];
      e = d > c ? d - c : 0;  // extend length (scheduler.py:154-157 ranges)
      const int L = d > 0 ? d : 0;
      kv = p.page_size == 1 ? L : (L + p.page_size - 1) / p.page_size;
    }
    int2 tot;
    block_scan2(e, kv, lds, tot);
    if (r < p.num_reqs) {
      // offsets past a capacity are clamped to it: the outputs stop there, and
      // no launch that reads these offsets next reads past them
      p.q_indptr[r + 1] = (int)min((int64_t)carry_q + e, p.token_capacity);
      p.kv_indptr[r + 1] = (int)min((int64_t)carry_kv + kv, p.kv_capacity);
      if (p.last_indices) p.last_indices[r] = (int)min((int64_t)carry_q + e, p.token_capacity) - 1;
    }
    carry_q += tot.x;
    carry_kv += tot.y;
  }
}

// Request owning element e: the last r with off[r] <= e (off has R+1 entries,
// non-decreasing, off[0] = 0 <= e < off[R]).
__device__ __forceinline__ int owner(const int32_t* off, int R, int e) {
  int lo = 0, hi = R - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (off[mid] <= e) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__device__ __forceinline__ int32_t table_at(const IndexParams& p, int r, int64_t col) {
  const int64_t row = p.table_idx[r];
  if (row < 0 || row >= p.num_rows || col < 0 || col >= p.row_stride) return -1;
  return p.table[row * p.row_stride + col];
}

__global__ __launch_bounds__(kFillThreads) void fill_kernel(IndexParams p) {
  __shared__ int32_t lq[kLdsOffsets + 1];
  __shared__ int32_t lk[kLdsOffsets + 1];
  const int R = p.num_reqs;
  const bool staged = R <= kLdsOffsets;
  if (staged) {
    for (int i = threadIdx.x; i <= R; i += kFillThreads) {
      lq[i] = p.q_indptr[i];
      lk[i] = p.kv_indptr[i];
    }
    __syncthreads();
  }
  const int32_t* qo = staged ? lq : p.q_indptr;
  const int32_t* ko = staged ? lk : p.kv_indptr;
  const int64_t T = min((int64_t)qo[R], p.token_capacity);
  const int64_t K = min((int64_t)ko[R], p.kv_capacity);
  const int64_t stride = (int64_t)gridDim.x * kFillThreads;
  for (int64_t e = (int64_t)blockIdx.x * kFillThreads + threadIdx.x; e < T; e += stride) {
    const int r = owner(qo, R, (int)e);
    const int pos = p.cached_len[r] + (int)(e - qo[r]);
    if (p.positions) p.positions[e] = pos;
    if (p.out_loc) p.out_loc[e] = table_at(p, r, pos);
  }
  for (int64_t e = (int64_t)blockIdx.x * kFillThreads + threadIdx.x; e < K; e += stride) {
    const int r = owner(ko, R, (int)e);
    const int j = (int)(e - ko[r]);
    if (p.page_size == 1) {
      p.kv_indices[e] = table_at(p, r, j);
    } else {
      const int32_t s = table_at(p, r, (int64_t)j * p.page_size);
      p.kv_indices[e] = s < 0 ? -1 : s / p.page_size;
    }
  }
}

}  // namespace
}  // namespace msgl

extern "C" int msgl_build_step_indices(const int32_t* req_to_token, int64_t num_rows, int64_t row_stride,
                                       const int32_t* table_idx, const int32_t* cached_len,
                                       const int32_t* device_len, int32_t num_reqs, int32_t page_size,
                                       int32_t* q_indptr, int32_t* positions, int32_t* out_loc,
                                       int32_t* last_indices, int64_t token_capacity, int32_t* kv_indptr,
                                       int32_t* kv_indices, int64_t kv_capacity, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(num_reqs >= 0, "msgl_build_step_indices: num_reqs must be >= 0");
  if (num_reqs == 0) return MSGL_OK;
  MSGL_CHECK_ARG(page_size >= 1, "msgl_build_step_indices: page_size must be >= 1");
  MSGL_CHECK_ARG(num_rows > 0 && row_stride > 0 && row_stride <= INT32_MAX,
                 "msgl_build_step_indices: table must be [num_rows > 0, 0 < row_stride < 2^31]");
  MSGL_CHECK_ARG(token_capacity >= 0 && kv_capacity >= 0, "msgl_build_step_indices: capacities must be >= 0");
  MSGL_CHECK_ARG(req_to_token && table_idx && cached_len && device_len && q_indptr && kv_indptr,
                 "msgl_build_step_indices: null pointer");
  MSGL_CHECK_ARG((token_capacity == 0 || positions || out_loc) && (kv_capacity == 0 || kv_indices),
                 "msgl_build_step_indices: an output with non-zero capacity is null");
  IndexParams p;
  p.table = req_to_token;
  p.num_rows = num_rows;
  p.row_stride = row_stride;
  p.table_idx = table_idx;
  p.cached_len = cached_len;
  p.device_len = device_len;
  p.num_reqs = num_reqs;
  p.page_size = page_size;
  p.q_indptr = q_indptr;
  p.positions = positions;
  p.out_loc = out_loc;
  p.last_indices = last_indices;
  p.token_capacity = token_capacity;
  p.kv_indptr = kv_indptr;
  p.kv_indices = kv_indices;
  p.kv_capacity = kv_capacity;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(kScanThreads), 0, s, p);
  MSGL_CHECK_LAUNCH("msgl_build_step_indices (scan)");
  const int64_t work = token_capacity > kv_capacity ? token_capacity : kv_capacity;
  int64_t blocks = (work + kFillThreads - 1) / kFillThreads;
  blocks = blocks < 1 ? 1 : (blocks > 2048 ? 2048 : blocks);
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)blocks), dim3(kFillThreads), 0, s, p);
  MSGL_CHECK_LAUNCH("msgl_build_step_indices (fill)");
  return MSGL_OK;
}

namespace msgl {
namespace {
__global__ __launch_bounds__(kFillThreads) void table_scatter_kernel(int32_t* table, int64_t num_rows,
                                                                     int64_t row_stride, const int32_t* rows,
                                                                     const int32_t* cols, const int32_t* values,
                                                                     int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kFillThreads;
  for (int64_t i = (int64_t)blockIdx.x * kFillThreads + threadIdx.x; i < n; i += stride) {
    const int64_t r = rows[i], c = cols[i];
    if (r >= 0 && r < num_rows && c >= 0 && c < row_stride) table[r * row_stride + c] = values[i];
  }
}
}  // namespace
}  // namespace msgl

extern "C" int msgl_table_scatter(int32_t* req_to_token, int64_t num_rows, int64_t row_stride, const int32_t* rows,
                                  const int32_t* cols, const int32_t* values, int64_t n, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(n >= 0, "msgl_table_scatter: n must be >= 0");
  if (n == 0) return MSGL_OK;
  MSGL_CHECK_ARG(num_rows > 0 && row_stride > 0, "msgl_table_scatter: table must be non-empty");
  MSGL_CHECK_ARG(req_to_token && rows && cols && values, "msgl_table_scatter: null pointer");
  int64_t blocks = (n + kFillThreads - 1) / kFillThreads;
  blocks = blocks > 2048 ? 2048 : blocks;
  hipLaunchKernelGGL(table_scatter_kernel, dim3((unsigned)blocks), dim3(kFillThreads), 0, (hipStream_t)stream,
                     req_to_token, num_rows, row_stride, rows, cols, values, n);
  MSGL_CHECK_LAUNCH("msgl_table_scatter");
  return MSGL_OK;
}
