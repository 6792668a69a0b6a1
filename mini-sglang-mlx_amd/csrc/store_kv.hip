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

// ---------------------------------------------------------------------------
// fp8 KV store: the extension of kvcache/pool.py:47-50 that docs/09-exercises.md:81-82
// describes -- rows quantised to OCP fp8 e4m3 with one fp32 scale per (slot, kv
// head), kept as kv_scale[slot, head] = (K scale, V scale) so that a reader
// gets both with one 8-byte load. For each (token, kv head) row of D elements:
// amax = max |x|, the
// codes are e4m3(x * (448 / amax)) rounded to nearest even and the scale is
// amax / 448 (a row of zeros: codes 0, scale 0). A row is LPR = D / VEC
// consecutive lanes (VEC = elements per 16-byte input chunk); amax is reduced
// across them with lane exchanges, then each lane writes its VEC codes and the
// row's first lane the scale. K and V rows of a token are neighbouring rows.
// ---------------------------------------------------------------------------
namespace msgl {
namespace {

template <typename T>
__global__ __launch_bounds__(256) void store_kv_fp8_kernel(const uint8_t* __restrict__ k,
                                                           const uint8_t* __restrict__ v,
                                                           const int32_t* __restrict__ out_loc,
                                                           uint8_t* __restrict__ k_codes,
                                                           uint8_t* __restrict__ v_codes, float* __restrict__ kv_scale,
                                                           int64_t num_tokens, int hkv,
                                                           int head_dim, int lpr, int64_t num_slots) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int64_t rows = num_tokens * hkv * 2;
  const int64_t per_block_rows = 256 / lpr;
  const int sub = threadIdx.x % lpr;  // lane within the row
  for (int64_t row = (int64_t)blockIdx.x * per_block_rows + threadIdx.x / lpr; row < rows;
       row += (int64_t)gridDim.x * per_block_rows) {
    const int64_t th = row >> 1;  // (token, head)
    const bool is_v = row & 1;
    const int64_t t = th / hkv;
    const int h = (int)(th - t * hkv);
    const uint8_t* src = (is_v ? v : k) + (th * head_dim + (int64_t)sub * VEC) * sizeof(T);
    uint32_t w[VEC / 4];
    const float amax = fp8_quantize_chunk<T>(ld16(src), lpr, w);
    const int64_t slot = out_loc[t];
    if (slot < 0 || slot >= num_slots) continue;  // never write outside the pool (uniform per row)
    uint8_t* dst = (is_v ? v_codes : k_codes) + (slot * hkv + h) * head_dim + (int64_t)sub * VEC;
    if constexpr (VEC == 8) {
      *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
    } else {
      *reinterpret_cast<uint32_t*>(dst) = w[0];
    }
    if (sub == 0) kv_scale[(slot * hkv + h) * 2 + (is_v ? 1 : 0)] = amax / 448.f;
  }
}

}  // namespace
}  // namespace msgl

extern "C" int msgl_store_kv_fp8(const void* k, const void* v, const int32_t* out_loc, void* k_pool, void* v_pool,
                                 float* kv_scale, int64_t num_tokens, int32_t num_kv_heads,
                                 int32_t head_dim, int64_t num_slots, int32_t dtype, void* stream) {
  using namespace msgl;
  clear_error();
  const int es = dtype_size(dtype);
  if (es == 0) {
    set_error("msgl_store_kv_fp8: unknown dtype %d", dtype);
    return MSGL_ERR_UNSUPPORTED;
  }
  MSGL_CHECK_ARG(num_tokens >= 0, "msgl_store_kv_fp8: num_tokens must be >= 0");
  MSGL_CHECK_ARG(num_kv_heads > 0 && num_slots > 0, "msgl_store_kv_fp8: num_kv_heads and num_slots must be > 0");
  const int vec = 16 / es;
  const int lpr = head_dim / vec;
  if (head_dim <= 0 || head_dim % vec != 0 || lpr > 64 || (lpr & (lpr - 1)) != 0) {
    set_error("msgl_store_kv_fp8: head_dim %d unsupported (a power-of-two multiple of %d, at most %d)", head_dim, vec,
              64 * vec);
    return MSGL_ERR_UNSUPPORTED;
  }
  if (num_tokens == 0) return MSGL_OK;
  MSGL_CHECK_ARG(k && v && out_loc && k_pool && v_pool && kv_scale, "msgl_store_kv_fp8: null pointer");
  MSGL_CHECK_ARG(((uintptr_t)k | (uintptr_t)v) % 16 == 0 && ((uintptr_t)k_pool | (uintptr_t)v_pool) % 8 == 0 &&
                     (uintptr_t)kv_scale % 8 == 0,
                 "msgl_store_kv_fp8: k, v must be 16-byte aligned, pools and kv_scale 8-byte");
  const int64_t rows = num_tokens * num_kv_heads * 2;
  const int64_t per_block = 256 / lpr;
  int64_t blocks = (rows + per_block - 1) / per_block;
  if (blocks > 65536) blocks = 65536;
  hipStream_t s = (hipStream_t)stream;
  const uint8_t* kb = (const uint8_t*)k;
  const uint8_t* vb = (const uint8_t*)v;
  uint8_t* kp = (uint8_t*)k_pool;
  uint8_t* vp = (uint8_t*)v_pool;
  switch (dtype) {
    case MSGL_F32:
      hipLaunchKernelGGL(store_kv_fp8_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, s, kb, vb, out_loc, kp,
                         vp, kv_scale, num_tokens, num_kv_heads, head_dim, lpr, num_slots);
      break;
    case MSGL_BF16:
      hipLaunchKernelGGL(store_kv_fp8_kernel<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, s, kb, vb, out_loc, kp,
                         vp, kv_scale, num_tokens, num_kv_heads, head_dim, lpr, num_slots);
      break;
    default:
      hipLaunchKernelGGL(store_kv_fp8_kernel<f16_t>, dim3((unsigned)blocks), dim3(256), 0, s, kb, vb, out_loc, kp,
                         vp, kv_scale, num_tokens, num_kv_heads, head_dim, lpr, num_slots);
      break;
  }
  MSGL_CHECK_LAUNCH("msgl_store_kv_fp8");
  return MSGL_OK;
}
