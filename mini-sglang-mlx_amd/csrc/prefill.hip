// Ragged chunked-prefill attention for gfx950, one launch per packed batch.
//
// Semantics: attention/base.py:85-105 (_forward_prefill): request i's E_i
// extend queries q[q_indptr[i] : q_indptr[i+1]] attend to its first L_i =
// P_i + E_i tokens of KV (the cached prefix plus this step's rows, already
// stored in the pool) with MLX's bottom-right causal mask
// (docs/04-attention.md:35-36): query t sees key j iff j <= P_i + t. With
// E_i == 1 the mask keeps every key (attention/base.py:103, mask=None).
//
// Query rows are (token, grouped head) pairs, so the G query heads of one kv
// head share every K/V tile (GQA). A workgroup owns one block of query rows
// of one (request, kv head) and one contiguous range of that block's keys.
//
// bf16 / fp16 (prefill16_kernel), the serving path:
//  * 4 wavefronts x 32 query rows, all products on v_mfma_f32_32x32x16 (the
//    16x16x32 form runs at half its rate on gfx950).
//  * 32-key K and V tiles are gathered from the pool straight into LDS with
//    gfx950's global_load_lds_dwordx4 (16 bytes per lane, no register
//    staging) into a ring of NS stages, NS-1 tiles ahead of the compute. The
//    wait for a tile is an explicit vmcnt on the issuing wavefront plus one
//    barrier, so later tiles stay in flight. Slot indices for up to 1024 keys
//    are staged in LDS first, so no other global load sits in the loop.
//  * Rows are stored unpadded with an XOR swizzle of their 16-byte chunks
//    (chunk c of row r lives at c ^ swz(r)); the K operand reads (16 rows,
//    same chunk) and the transposing V reads (4 rows x 2 chunks per 16 lanes)
//    are bank-conflict free on the 64-bank LDS.
//  * S^T = K Q^T per 32-key tile: lane l holds 16 keys (8c + 4(l/32) + r) of
//    query row l%32, which are exactly the A operand slots P needs for the two
//    16-key steps of O += P V (converted in registers, no shuffle); a row's max
//    and sum take one exchange with lane l^32. The B operand of P V (keys
//    contiguous per lane) is read from the row-major V tile with
//    ds_read_b64_tr_b16.
//  * Online softmax per query row in the exp2 domain, scores scaled inside
//    the exponent's FMA.
//  * Split-K: a block's visible key range [0, kv_end) is cut into at most
//    `splits` chunks of one batch-wide length (ceil(max_seq_len / splits),
//    at least 256 keys), so only long blocks are split and every workgroup's
//    key loop is about equally short. A block with one chunk writes the output
//    directly; otherwise each chunk writes (m, l, unnormalised O) in fp32 to
//    the workspace and prefill_merge_kernel combines them.
//  * Online softmax with a lazily moved reference maximum (see the loop).
//  * A one-workgroup plan kernel lists the (request, query block, chunk)
//    items that have keys, longest first, each expanded to the kv heads; the
//    attention grid reads its item from the list, so no empty workgroup sits
//    between real ones and the dispatcher hands out long items first.
//
// fp32 (prefill_f32_kernel): one pass per block, 4 wavefronts x 16 rows,
// register-staged gather into padded LDS tiles, v_mfma_f32_16x16x4f32.
//
// Causal tiles past a block's last visible key are never loaded.
#include "prefill_device.h"

namespace msgl {

namespace {
using namespace pf;

// Work list for prefill16_kernel, one workgroup: every (request, query block,
// chunk) triple with keys to process, counting-sorted by its tile count
// (longest first, buckets of 1..255+ tiles) so the hardware dispatcher hands
// out the long items first, each expanded to the kv heads as consecutive
// items (consecutive workgroups go to consecutive XCDs, so with 8 kv heads a
// head's query blocks share one L2). A grid without empty workgroups in the
// middle keeps every CU slot busy; the list order does not change any result.
constexpr int kPlanThreads = 1024;

__device__ __forceinline__ int plan_tiles(const PrefillParams& p, int bq, int t, int& req, int& qblk, int& split) {
  split = t % p.splits;
  qblk = (t / p.splits) % p.nqb;
  req = t / (p.splits * p.nqb);
  const int q0 = p.q_indptr[req];
  const int E = p.q_indptr[req + 1] - q0;
  const int qb = qblk * bq;
  if (qb >= E) return 0;
  const int L = p.seq_lens ? p.seq_lens[req] : (p.kv_indptr[req + 1] - p.kv_indptr[req]);
  const int kv_end = block_kv_end(L, E, qb, bq);
  int n, clen;
  chunk_geometry(kv_end, p.splits, p.chunk_len, n, clen);
  if (split >= n) return 0;
  const int c0 = split * clen;
  const int c1 = split == n - 1 ? kv_end : c0 + clen;
  return (c1 - c0 + KT - 1) / KT;
}

__global__ __launch_bounds__(kPlanThreads) void prefill_plan_kernel(PrefillParams p, int bq) {
  __shared__ int hist[256];
  const int ntrip = p.num_reqs * p.nqb * p.splits;
  for (int b = threadIdx.x; b < 256; b += kPlanThreads) hist[b] = 0;
  __syncthreads();
  int req, qblk, split;
  for (int t = threadIdx.x; t < ntrip; t += kPlanThreads) {
    const int n = plan_tiles(p, bq, t, req, qblk, split);
    if (n > 0) atomicAdd(&hist[min(n, 255)], 1);
  }
  __syncthreads();
  if (threadIdx.x == 0) {  // exclusive offsets, longest bucket first
    int run = 0;
    for (int b = 255; b >= 1; --b) {
      const int c = hist[b];
      hist[b] = run;
      run += c;
    }
    *p.plan_count = run * p.hkv;
    p.plan_count[1] = p.num_reqs;  // the sizes this list is for (checked by every launch that reads it)
    p.plan_count[2] = p.num_tokens;
    p.plan_count[3] = p.splits;
    p.plan_count[4] = p.nqb;
    p.plan_count[5] = p.hkv;
    p.plan_count[6] = p.chunk_len;
  }
  __syncthreads();
  for (int t = threadIdx.x; t < ntrip; t += kPlanThreads) {
    const int n = plan_tiles(p, bq, t, req, qblk, split);
    if (n > 0) {
      const int pos = atomicAdd(&hist[min(n, 255)], 1);
      const int q0 = p.q_indptr[req];
      const int kv0 = p.kv_indptr[req];
      const int L = p.seq_lens ? p.seq_lens[req] : (p.kv_indptr[req + 1] - kv0);
      const int4 geo = make_int4(q0, p.q_indptr[req + 1] - q0, kv0, L);
      for (int h = 0; h < p.hkv; ++h) {
        p.plan[2 * (pos * p.hkv + h)] = make_int4(req, h, qblk, split);
        p.plan[2 * (pos * p.hkv + h) + 1] = geo;
      }
    }
  }
  if (p.splits > 1) {  // chunk count of every token's block, for the merge
    for (int tk = threadIdx.x; tk < p.num_tokens; tk += kPlanThreads) {
      int lo = 0, hi = p.num_reqs - 1;  // the last request r with q_indptr[r] <= tk
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (p.q_indptr[mid] <= tk) lo = mid; else hi = mid - 1;
      }
      const int q0 = p.q_indptr[lo];
      const int E = p.q_indptr[lo + 1] - q0;
      const int tok = tk - q0;
      int n = 0, clen;
      if (tok >= 0 && tok < E) {
        const int L = p.seq_lens ? p.seq_lens[lo] : (p.kv_indptr[lo + 1] - p.kv_indptr[lo]);
        chunk_geometry(block_kv_end(L, E, tok / bq * bq, bq), p.splits, p.chunk_len, n, clen);
      }
      p.merge_n[tk] = n;
    }
  }
}

int tokens_per_block16(int group) { return NWAVE16 * 32 / group; }

inline int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// Workspace of the 16-bit path: plan length, plan (two int4 per work item),
// then with splits > 1 each token's chunk count and the per-chunk (m, l) and O
// partials.
struct PrefillWorkspace {
  int64_t items, plan, merge_n, part_ml, part_o, bytes;
};
PrefillWorkspace prefill_workspace(int num_reqs, int num_tokens, int max_e, int hq, int hkv, int head_dim,
                                   int splits) {
  PrefillWorkspace w;
  const int bq = tokens_per_block16(hq / hkv) > 0 ? tokens_per_block16(hq / hkv) : 1;
  w.items = (int64_t)num_reqs * ((max_e + bq - 1) / bq) * splits * hkv;
  const int64_t rows = splits > 1 ? (int64_t)splits * num_tokens * hq : 0;
  w.plan = 256;
  w.merge_n = w.plan + align256(w.items * 32);
  w.part_ml = w.merge_n + align256(splits > 1 ? (int64_t)num_tokens * 4 : 0);
  w.part_o = w.part_ml + align256(rows * 8);
  w.bytes = w.part_o + align256(rows * head_dim * 4);
  return w;
}

}  // namespace
}  // namespace msgl

int msgl::pf::launch_prefill_plan(const PrefillParams& p, int bq, hipStream_t stream) {
  hipLaunchKernelGGL(prefill_plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, p, bq);
  MSGL_CHECK_LAUNCH("msgl_prefill_ragged (plan)");
  return MSGL_OK;
}

extern "C" int32_t msgl_prefill_default_splits(int32_t num_reqs, int32_t num_qo_heads, int32_t num_kv_heads,
                                               int32_t head_dim, int32_t max_extend_len, int32_t max_seq_len) {
  using namespace msgl;
  if (num_reqs <= 0 || num_kv_heads <= 0 || num_qo_heads < num_kv_heads || max_extend_len <= 0) return 1;
  const int group = num_qo_heads / num_kv_heads;
  const int bq = tokens_per_block16(group) > 0 ? tokens_per_block16(group) : 1;
  const int64_t base = (int64_t)num_reqs * num_kv_heads * ((max_extend_len + bq - 1) / bq);
  // about 6 workgroups per CU of the 256-CU device (two resident at a time):
  // enough items to balance, few enough partials to merge
  const int64_t target = 1536;
  int64_t s = (target + base - 1) / base;
  if (max_seq_len > 0) s = std::min<int64_t>(s, std::max<int64_t>(1, (max_seq_len + kMinChunk - 1) / kMinChunk));
  s = std::max<int64_t>(1, std::min<int64_t>(s, kMaxSplits));
  return (int32_t)s;
}

extern "C" int64_t msgl_prefill_workspace_size(int32_t num_reqs, int32_t num_tokens, int32_t max_extend_len,
                                               int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                               int32_t max_splits) {
  using namespace msgl;
  if (num_reqs <= 0 || num_tokens <= 0 || max_extend_len <= 0 || num_qo_heads <= 0 || num_kv_heads <= 0 ||
      head_dim <= 0 || num_qo_heads % num_kv_heads != 0 || max_splits < 1)
    return 0;
  return prefill_workspace(num_reqs, num_tokens, max_extend_len, num_qo_heads, num_kv_heads, head_dim,
                           std::min<int32_t>(max_splits, kMaxSplits))
      .bytes;
}

// Validates the arguments of a prefill call and fills p (the workspace regions
// included); empty: the batch has no query, nothing to launch.
int msgl::pf::prefill_params(const char* fn, int mode, const void* q, const void* k_pool, const void* v_pool,
                       const float* kv_scale, const int32_t* q_indptr, const int32_t* kv_indptr,
                       const int32_t* kv_indices, const int32_t* seq_lens, int32_t num_reqs, int32_t num_tokens,
                       int32_t max_extend_len, int32_t max_seq_len, int32_t num_qo_heads, int32_t num_kv_heads,
                       int32_t head_dim, int32_t page_size, int64_t num_slots, int32_t dtype, float scale,
                       int32_t max_splits, void* out, void* workspace, int64_t workspace_bytes, PrefillParams& p,
                       bool& empty) {
  clear_error();
  empty = false;
  MSGL_CHECK_ARG(num_reqs >= 0 && num_tokens >= 0 && max_extend_len >= 0, "%s: sizes must be >= 0", fn);
  if (num_reqs == 0 || max_extend_len == 0 || num_tokens == 0) {
    empty = true;
    return MSGL_OK;
  }
  MSGL_CHECK_ARG(num_qo_heads > 0 && num_kv_heads > 0 && head_dim > 0, "%s: sizes must be > 0", fn);
  MSGL_CHECK_ARG(num_qo_heads % num_kv_heads == 0, "%s: Hq (%d) must be a multiple of Hkv (%d)", fn, num_qo_heads,
                 num_kv_heads);
  MSGL_CHECK_ARG(max_splits >= 1 && max_splits <= kMaxSplits, "%s: max_splits must be in [1, %d]", fn, kMaxSplits);
  MSGL_CHECK_ARG(q_indptr && kv_indptr, "%s: null pointer", fn);
  if (mode != kPlanOnly) {
    MSGL_CHECK_ARG(page_size >= 1, "%s: page_size must be >= 1", fn);
    MSGL_CHECK_ARG(page_size == 1 || seq_lens != nullptr, "%s: page_size > 1 needs seq_lens", fn);
    MSGL_CHECK_ARG(num_slots > 0 && num_slots <= ((int64_t)1 << 31) - 1, "%s: num_slots must be in [1, 2^31)", fn);
    MSGL_CHECK_ARG(scale > 0.f && scale < INFINITY, "%s: scale must be positive and finite", fn);
    MSGL_CHECK_ARG(q && k_pool && v_pool && kv_indices && out, "%s: null pointer", fn);
    MSGL_CHECK_ARG(((uintptr_t)q | (uintptr_t)k_pool | (uintptr_t)v_pool | (uintptr_t)out) % 16 == 0,
                   "%s: q, pools and out must be 16-byte aligned", fn);
    MSGL_CHECK_ARG((uintptr_t)kv_scale % 8 == 0, "%s: kv_scale must be 8-byte aligned", fn);
  }
  if (dtype_size(dtype) == 0) {
    set_error("%s: unknown dtype %d", fn, dtype);
    return MSGL_ERR_UNSUPPORTED;
  }
  p.q = q;
  p.k_pool = k_pool;
  p.v_pool = v_pool;
  p.kv_scale = kv_scale;
  p.q_indptr = q_indptr;
  p.kv_indptr = kv_indptr;
  p.kv_indices = kv_indices;
  p.seq_lens = seq_lens;
  p.out = out;
  p.part_o = nullptr;
  p.part_ml = nullptr;
  p.plan = nullptr;
  p.plan_count = nullptr;
  p.merge_n = nullptr;
  p.plan_capacity = 0;
  p.num_slots = num_slots;
  p.hq = num_qo_heads;
  p.hkv = num_kv_heads;
  p.page_size = page_size;
  p.num_reqs = num_reqs;
  p.num_tokens = num_tokens;
  p.splits = dtype == MSGL_F32 ? 1 : max_splits;  // fp32 runs one pass per block
  p.chunk_len = 0;
  if (p.splits > 1 && max_seq_len > 0) {
    const int per = (max_seq_len + p.splits - 1) / p.splits;
    p.chunk_len = std::max(kMinChunk, (per + KT - 1) / KT * KT);
  }
  p.nqb = 0;
  p.items = 0;
  p.scale_log2 = scale * kLog2eP;
  p.mode = mode;
  if (dtype != MSGL_F32) {
    const PrefillWorkspace w =
        prefill_workspace(num_reqs, num_tokens, max_extend_len, num_qo_heads, num_kv_heads, head_dim, p.splits);
    if (workspace == nullptr || workspace_bytes < w.bytes) {
      set_error("%s: workspace of %lld bytes needed (%d splits), got %lld", fn, (long long)w.bytes, p.splits,
                (long long)workspace_bytes);
      return MSGL_ERR_WORKSPACE;
    }
    MSGL_CHECK_ARG((uintptr_t)workspace % 256 == 0, "%s: workspace must be 256-byte aligned", fn);
    MSGL_CHECK_ARG(w.items <= INT32_MAX, "%s: too many work items", fn);
    uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
    p.plan_count = reinterpret_cast<int*>(ws);
    p.plan = reinterpret_cast<int4*>(ws + w.plan);
    p.plan_capacity = (int)w.items;
    if (p.splits > 1) {
      p.merge_n = reinterpret_cast<int*>(ws + w.merge_n);
      p.part_ml = reinterpret_cast<float2*>(ws + w.part_ml);
      p.part_o = reinterpret_cast<float*>(ws + w.part_o);
    }
  }
  return MSGL_OK;
}

namespace {
int prefill_impl(const char* fn, int mode, const void* q, const void* k_pool, const void* v_pool,
                 const float* kv_scale, const int32_t* q_indptr, const int32_t* kv_indptr, const int32_t* kv_indices,
                 const int32_t* seq_lens, int32_t num_reqs, int32_t num_tokens, int32_t max_extend_len,
                 int32_t max_seq_len, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                 int64_t num_slots, int32_t dtype, float scale, int32_t max_splits, void* out, void* workspace,
                 int64_t workspace_bytes, void* stream) {
  using namespace msgl;
  PrefillParams p;
  bool empty = false;
  const int st = pf::prefill_params(fn, mode, q, k_pool, v_pool, kv_scale, q_indptr, kv_indptr, kv_indices, seq_lens,
                                    num_reqs, num_tokens, max_extend_len, max_seq_len, num_qo_heads, num_kv_heads,
                                    head_dim, page_size, num_slots, dtype, scale, max_splits, out, workspace,
                                    workspace_bytes, p, empty);
  if (st != MSGL_OK || empty) return st;
  const int group = num_qo_heads / num_kv_heads;
  hipStream_t s = (hipStream_t)stream;
  if (kv_scale != nullptr) {  // fp8 e4m3 pools with per-(slot, kv head) scales
    switch (dtype) {
      case MSGL_BF16: return pf::prefill_launch_bf16_fp8(p, max_extend_len, head_dim, group, s);
      case MSGL_F16: return pf::prefill_launch_f16_fp8(p, max_extend_len, head_dim, group, s);
    }
    set_error("%s: fp8 pools take bf16 or fp16 queries (dtype %d)", fn, dtype);
    return MSGL_ERR_UNSUPPORTED;
  }
  switch (dtype) {
    case MSGL_F32: return pf::prefill_launch_f32(p, max_extend_len, head_dim, group, s);
    case MSGL_BF16: return pf::prefill_launch_bf16(p, max_extend_len, head_dim, group, s);
    case MSGL_F16: return pf::prefill_launch_f16(p, max_extend_len, head_dim, group, s);
  }
  return MSGL_ERR_UNSUPPORTED;
}
}  // namespace

extern "C" int msgl_prefill_ragged(const void* q, const void* k_pool, const void* v_pool, const int32_t* q_indptr,
                                   const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                                   int32_t num_reqs, int32_t num_tokens, int32_t max_extend_len, int32_t max_seq_len,
                                   int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                   int64_t num_slots, int32_t dtype, float scale, int32_t max_splits, void* out,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
  return prefill_impl("msgl_prefill_ragged", msgl::kPlanAndRun, q, k_pool, v_pool, nullptr, q_indptr, kv_indptr,
                      kv_indices,
                      seq_lens, num_reqs, num_tokens, max_extend_len, max_seq_len, num_qo_heads, num_kv_heads,
                      head_dim, page_size, num_slots, dtype, scale, max_splits, out, workspace, workspace_bytes,
                      stream);
}

extern "C" int msgl_prefill_ragged_planned(const void* q, const void* k_pool, const void* v_pool,
                                           const int32_t* q_indptr, const int32_t* kv_indptr,
                                           const int32_t* kv_indices, const int32_t* seq_lens, int32_t num_reqs,
                                           int32_t num_tokens, int32_t max_extend_len, int32_t max_seq_len,
                                           int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                           int32_t page_size, int64_t num_slots, int32_t dtype, float scale,
                                           int32_t max_splits, void* out, void* workspace, int64_t workspace_bytes,
                                           void* stream) {
  return prefill_impl("msgl_prefill_ragged_planned", msgl::kRunPlanned, q, k_pool, v_pool, nullptr, q_indptr,
                      kv_indptr,
                      kv_indices, seq_lens, num_reqs, num_tokens, max_extend_len, max_seq_len, num_qo_heads,
                      num_kv_heads, head_dim, page_size, num_slots, dtype, scale, max_splits, out, workspace,
                      workspace_bytes, stream);
}

extern "C" int msgl_prefill_plan(const int32_t* q_indptr, const int32_t* kv_indptr, const int32_t* seq_lens,
                                 int32_t num_reqs, int32_t num_tokens, int32_t max_extend_len, int32_t max_seq_len,
                                 int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                                 int32_t max_splits, void* workspace, int64_t workspace_bytes, void* stream) {
  return prefill_impl("msgl_prefill_plan", msgl::kPlanOnly, nullptr, nullptr, nullptr, nullptr, q_indptr, kv_indptr,
                      nullptr,
                      seq_lens, num_reqs, num_tokens, max_extend_len, max_seq_len, num_qo_heads, num_kv_heads,
                      head_dim, 1, 1, dtype, 1.f, max_splits, nullptr, workspace, workspace_bytes, stream);
}

extern "C" int msgl_prefill_ragged_fp8(const void* q, const void* k_pool, const void* v_pool, const float* kv_scale,
                                       const int32_t* q_indptr, const int32_t* kv_indptr, const int32_t* kv_indices,
                                       const int32_t* seq_lens, int32_t num_reqs, int32_t num_tokens,
                                       int32_t max_extend_len, int32_t max_seq_len, int32_t num_qo_heads,
                                       int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int64_t num_slots,
                                       int32_t dtype, float scale, int32_t max_splits, void* out, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(kv_scale != nullptr, "msgl_prefill_ragged_fp8: null kv_scale");
  return prefill_impl("msgl_prefill_ragged_fp8", kPlanAndRun, q, k_pool, v_pool, kv_scale, q_indptr, kv_indptr,
                      kv_indices, seq_lens, num_reqs, num_tokens, max_extend_len, max_seq_len, num_qo_heads,
                      num_kv_heads, head_dim, page_size, num_slots, dtype, scale, max_splits, out, workspace,
                      workspace_bytes, stream);
}

extern "C" int msgl_prefill_ragged_fp8_planned(const void* q, const void* k_pool, const void* v_pool,
                                               const float* kv_scale, const int32_t* q_indptr,
                                               const int32_t* kv_indptr, const int32_t* kv_indices,
                                               const int32_t* seq_lens, int32_t num_reqs, int32_t num_tokens,
                                               int32_t max_extend_len, int32_t max_seq_len, int32_t num_qo_heads,
                                               int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                               int64_t num_slots, int32_t dtype, float scale, int32_t max_splits,
                                               void* out, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(kv_scale != nullptr, "msgl_prefill_ragged_fp8_planned: null kv_scale");
  return prefill_impl("msgl_prefill_ragged_fp8_planned", kRunPlanned, q, k_pool, v_pool, kv_scale, q_indptr,
                      kv_indptr, kv_indices, seq_lens, num_reqs, num_tokens, max_extend_len, max_seq_len,
                      num_qo_heads, num_kv_heads, head_dim, page_size, num_slots, dtype, scale, max_splits, out,
                      workspace, workspace_bytes, stream);
}
