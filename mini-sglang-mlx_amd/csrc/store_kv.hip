// KV-store scatter: k_pool[out_loc[t]] = k[t], v_pool[out_loc[t]] = v[t].
//
// Restates kvcache/pool.py:47-50 (MHAKVCache.store_kv) as one launch for both
// pools. A pool row (one token slot) is Hkv*D contiguous elements, so the copy
// is dtype-agnostic: each lane moves 16-byte chunks, a wavefront covers 1 KiB
// of a row per instruction, and K and V chunks are issued back to back so both
// streams are in flight together. HBM-bound: 2 * T * row_bytes read + written.
#include "msgl_common.h"

namespace msgl {

__global__ __launch_bounds__(256) void store_kv_kernel(const uint8_t* __restrict__ k,
                                                       const uint8_t* __restrict__ v,
                                                       const int32_t* __restrict__ out_loc,
                                                       uint8_t* __restrict__ k_pool,
                                                       uint8_t* __restrict__ v_pool, int64_t num_tokens,
                                                       int32_t chunks_per_row, int64_t num_slots) {
  const int64_t row_bytes = (int64_t)chunks_per_row * 16;
  const int64_t total = num_tokens * chunks_per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / chunks_per_row;
    const int64_t c = i - t * chunks_per_row;
    // the data loads do not wait for the slot: all three go out together
    const int64_t src = t * row_bytes + c * 16;
    const u32x4 kv = ld16(k + src);
    const u32x4 vv = ld16(v + src);
    const int64_t slot = out_loc[t];
    if (slot < 0 || slot >= num_slots) continue;  // never write outside the pool
    const int64_t dst = slot * row_bytes + c * 16;
    st16(k_pool + dst, kv);
    st16(v_pool + dst, vv);
  }
}

}  // namespace msgl

extern "C" int msgl_store_kv(const void* k, const void* v, const int32_t* out_loc, void* k_pool,
                             void* v_pool, int64_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                             int64_t num_slots, int32_t dtype, void* stream) {
  using namespace msgl;
  clear_error();
  const int es = dtype_size(dtype);
  if (es == 0) {
    set_error("msgl_store_kv: unknown dtype %d", dtype);
    return MSGL_ERR_UNSUPPORTED;
  }
  MSGL_CHECK_ARG(num_tokens >= 0, "msgl_store_kv: num_tokens must be >= 0 (got %lld)", (long long)num_tokens);
  MSGL_CHECK_ARG(num_kv_heads > 0 && head_dim > 0, "msgl_store_kv: num_kv_heads and head_dim must be > 0");
  MSGL_CHECK_ARG(num_slots > 0, "msgl_store_kv: num_slots must be > 0");
  if (num_tokens == 0) return MSGL_OK;
  MSGL_CHECK_ARG(k && v && out_loc && k_pool && v_pool, "msgl_store_kv: null pointer");
  const int64_t row_bytes = (int64_t)num_kv_heads * head_dim * es;
  if (row_bytes % 16 != 0) {
    set_error("msgl_store_kv: row of %lld bytes is not a multiple of 16", (long long)row_bytes);
    return MSGL_ERR_UNSUPPORTED;
  }
  MSGL_CHECK_ARG(((uintptr_t)k | (uintptr_t)v | (uintptr_t)k_pool | (uintptr_t)v_pool) % 16 == 0,
                 "msgl_store_kv: k, v and pools must be 16-byte aligned");
  const int32_t cpr = (int32_t)(row_bytes / 16);
  const int64_t total = num_tokens * cpr;
  const int threads = 256;
  int64_t blocks = (total + threads - 1) / threads;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(store_kv_kernel, dim3((unsigned)blocks), dim3(threads), 0, (hipStream_t)stream,
                     (const uint8_t*)k, (const uint8_t*)v, out_loc, (uint8_t*)k_pool, (uint8_t*)v_pool,
                     num_tokens, cpr, num_slots);
  MSGL_CHECK_LAUNCH("msgl_store_kv");
  return MSGL_OK;
}
