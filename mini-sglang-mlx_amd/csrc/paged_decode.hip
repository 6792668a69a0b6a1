// Paged decode attention for gfx950 (one query token per request).
//
// Semantics: attention/naive.py:50-60 (gather by page table + masked SDPA) and
// attention/metal.py:112-131 (paged_decode_attention over CSR indices):
//   o[b, h] = softmax_j(scale * q[b,h] . K[slot_b(j), h/G]) V[slot_b(j), h/G],  j < L_b
//
// Design (MI355X-first, not a translation of the Metal kernel):
//  * Work unit = one wavefront per (request b, split s, kv head); a workgroup
//    holds the MSGL_DECODE_WAVES_PER_WG (4) neighbouring kv heads of one
//    (b, s) -- measured faster than 1 or 2 -- and the kv-head groups of a
//    (b, s) are neighbouring workgroups, so the rows of a slot (Hkv * D
//    contiguous elements) are read close in time. A workgroup gathers its
//    token slots once into LDS.
//  * Split-K, two forms. Per-request chunks: every request is cut into chunks
//    of one batch-wide length, ceil(max_b L_b / s) rounded to 16 tokens
//    (>= kMinChunk), and a one-workgroup plan kernel lists the (request,
//    chunk, kv-head group) items longest first, so the grid has no empty
//    workgroups and the long items start first. Equal key ranges (long
//    contexts: at least MSGL_DECODE_BALANCED_MIN_RANGE keys per range): the
//    batch's keys, requests concatenated in order, are cut into as many
//    ranges of one length as the device holds workgroups at once (per kv-head
//    group), so every workgroup gathers the same number of keys and no tail
//    of long chunks is left running on a few CUs; a range that crosses request
//    boundaries runs one chunk per request it touches, and the range length
//    is at least ceil(max_b L_b / (max_splits - 1)), so a request overlaps at
//    most max_splits ranges. The plan writes the requests' key offsets (a
//    prefix sum of L) as well as the list; the decode launch picks the form.
//    A request in one chunk writes its final row; otherwise each chunk writes
//    fp32 partials (acc, m, l) and a merge kernel with one wavefront per
//    (request, kv head) combines them. Merging inside the decode launch was
//    measured slower on MI355X: a device-scope fence per chunk writes back and
//    invalidates the XCD's L2, and even fence-free agent-coherent partials
//    leave every chunk waiting on write-through stores and an atomic round
//    trip before its slot frees -- more than the second launch costs.
//  * Q.K^T runs on the matrix cores: v_mfma_f32_16x16x32_{bf16,f16} (or
//    16x16x4 f32), A = the G query heads of the kv head (rows >= G are zero),
//    B = 16 K rows (no conversion). Output: lane (t = l%16, row group l/16)
//    holds 4 scores. K rows are fetched like V rows -- each 16-lane group reads
//    one whole row -- and re-laid into the B layout through a padded per-wave
//    LDS tile: on MI355X a load instruction spanning 4 rows x 256 B streams far
//    faster than one spanning 16 rows x 64 B (the B layout's own shape).
//  * Online softmax in the exp2 domain (scale*log2(e) folded into the score)
//    with the tile max over 16 tokens from 4 DPP steps inside a 16-lane row;
//    only the MFMA rows that hold query heads are processed. The reference
//    maximum moves lazily (only when a tile's exceeds it by 2^8), so most
//    tiles skip the accumulators' rescale.
//  * Virtual kv heads: a group above 8 that is a multiple of 8 runs as groups
//    of 8, and a group of 8 over one or two kv heads as groups of 4, over
//    Hq/G' virtual kv heads that read their pool head's rows (neighbouring
//    wavefronts, so the second read comes from L2); see head_map.
//  * P.V on the VALU: lane (token sub-row, 16-byte d chunk) accumulates
//    G x (16/sizeof T) fp32 outputs; P and the rescale factors go through a
//    small per-wave LDS tile.
//  * fp8 pools (e4m3 codes, one fp32 K and V scale per slot and kv head): K
//    codes widen exactly to the query's 16-bit type for the same MFMA, a key's
//    K scale multiplies its score and its V scale folds into its softmax
//    weight. A token's scales sit in a 128-byte line of their own, so the
//    workgroup stages each segment's scales of its kv heads into LDS with LDS
//    DMA (one request per token and workgroup rather than per wavefront), and
//    the kv-head groups of one work item run on one XCD, where the second
//    group finds the line in L2.
//  * The tile loop is software pipelined: the K/V loads of the next NST-1
//    tiles are in flight (a ring of register buffers) while one tile is
//    computed, which is what it takes to keep ~200 KiB of loads in flight per
//    CU at 2 wavefronts per SIMD. K/V rows
//    are read exactly once per launch, so they use nontemporal (streaming)
//    loads, which sustain markedly more HBM bandwidth for random row gathers
//    on MI355X than default-policy loads.
#include <atomic>

#include "decode_device.h"

namespace msgl {
using namespace dec;

// Plan for paged_decode_kernel, one workgroup. When key ranges are allowed
// (max_splits > 1): tok_off[b] = sum of L over the requests before b
// (tok_off[B] = all keys) and meta[3] = max_b L_b. Always the work list (the
// decode launch picks the form from tok_off[B]): the batch-wide chunk length
// ceil(max_b L_b / s) (s = max_splits, or chunk_splits when key ranges are
// allowed; a multiple of 16, >= kMinChunk), then every
// (request, chunk) counting-sorted by its 16-token tile count, longest first,
// each expanded to the kv-head groups as consecutive items. Every workgroup
// then gathers at most one chunk, the long ones are dispatched first and no
// empty workgroup sits between real ones; a request with L = 0 keeps its
// (zero-output) chunk 0. The order does not change any result.
constexpr int kPlanThreads = 1024;

constexpr int kPlanLds = 8192;  // request lengths staged in LDS (larger batches read them again)

__device__ __forceinline__ int decode_item_tiles(int L, int max_splits, int split, int chunk_len) {
  if (L <= 0) return split == 0 ? 1 : 0;
  int n, chunk;
  split_geometry(L, max_splits, chunk_len, n, chunk);
  if (split >= n) return 0;
  const int len = split == n - 1 ? L - split * chunk : chunk;
  return (len + 15) / 16;
}

// Chunks per request of the work list when the launch may also split by key
// ranges (max_splits then bounds the ranges, not the chunks): ~4096
// wavefronts in all, a bit over one round of MI355X at 3 per SIMD, enough
// units for ragged lengths to balance and few enough that the partials and
// the merge stay small; no chunk shorter than kMinChunk and none longer than
// 2048 keys (long contexts need more items than resident slots).
__device__ __forceinline__ int chunk_splits(int batch, int hkv, int max_len, int max_splits) {
  const int64_t units = (int64_t)batch * hkv;
  int64_t s = (4096 + units - 1) / units;
  s = min(s, (int64_t)(max_len + kMinChunk - 1) / kMinChunk);
  s = max(s, (int64_t)(max_len + 2047) / 2048);
  return (int)max((int64_t)1, min(s, (int64_t)max_splits));
}

__global__ __launch_bounds__(kPlanThreads) void paged_decode_plan_kernel(DecodeParams p) {
  __shared__ int lens[kPlanLds];
  __shared__ int hist[256];
  __shared__ int wmax[kPlanThreads / 64];
  __shared__ int64_t wsum[kPlanThreads / 64];
  __shared__ int chunk_s;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (p.max_splits > 1) {
    // thread i sums the lengths of a contiguous block of requests; a block
    // scan turns the sums into exclusive offsets
    const int per = (p.batch + kPlanThreads - 1) / kPlanThreads;
    const int b0 = min(p.batch, (int)threadIdx.x * per), b1 = min(p.batch, b0 + per);
    auto len = [&](int b) { return p.seq_lens ? p.seq_lens[b] : p.kv_indptr[b + 1] - p.kv_indptr[b]; };
    int64_t sum = 0;
    int mx = 0;
    for (int b = b0; b < b1; ++b) {
      const int L = max(0, len(b));
      sum += L;
      mx = max(mx, L);
    }
    int64_t incl = sum;
    for (int d = 1; d < 64; d <<= 1) {
      const int64_t y = __shfl_up(incl, d);
      if (lane >= d) incl += y;
    }
    for (int d = 32; d >= 1; d >>= 1) mx = max(mx, __shfl_xor(mx, d));
    if (lane == 63) wsum[wave] = incl;
    if (lane == 0) wmax[wave] = mx;
    __syncthreads();
    int64_t off = incl - sum;
    for (int w = 0; w < wave; ++w) off += wsum[w];
    for (int b = b0; b < b1; ++b) {
      p.tok_off[b] = off;
      off += max(0, len(b));
    }
    if (threadIdx.x == kPlanThreads - 1) p.tok_off[p.batch] = off;  // b1 == batch for the last thread
    if (threadIdx.x == 0) {
      int m = 0;
      for (int w = 0; w < kPlanThreads / 64; ++w) m = max(m, wmax[w]);
      p.meta[3] = m;
      p.meta[2] = p.max_splits;  // key offsets written for this bound
    }
    __syncthreads();  // wmax is reused below
  }
  const bool staged = p.batch <= kPlanLds;
  auto len_of = [&](int b) {
    return staged ? lens[b] : (p.seq_lens ? p.seq_lens[b] : p.kv_indptr[b + 1] - p.kv_indptr[b]);
  };
  int m = 0;
  for (int b = threadIdx.x; b < p.batch; b += kPlanThreads) {
    const int L = p.seq_lens ? p.seq_lens[b] : p.kv_indptr[b + 1] - p.kv_indptr[b];
    if (staged) lens[b] = L;
    m = max(m, L);
  }
  for (int d = 32; d >= 1; d >>= 1) m = max(m, __shfl_xor(m, d));
  if (lane == 0) wmax[wave] = m;
  for (int i = threadIdx.x; i < 256; i += kPlanThreads) hist[i] = 0;
  __syncthreads();
  if (threadIdx.x == 0) {
    if (p.max_splits <= 1) p.meta[2] = 0;  // no key offsets
    int mx = 0;
    for (int w = 0; w < kPlanThreads / 64; ++w) mx = max(mx, wmax[w]);
    const int s = MSGL_DECODE_BALANCED && p.max_splits > 1 ? chunk_splits(p.batch, p.hkv, mx, p.max_splits)
                                                            : p.max_splits;
    int c = (mx + s - 1) / s;
    c = max(kMinChunk, (c + 15) & ~15);
    chunk_s = c;
    p.meta[1] = c;
  }
  __syncthreads();
  const int chunk_len = chunk_s;
  const int ncand = p.batch * p.max_splits;
  for (int t = threadIdx.x; t < ncand; t += kPlanThreads) {
    const int n = decode_item_tiles(len_of(t / p.max_splits), p.max_splits, t % p.max_splits, chunk_len);
    if (n > 0) atomicAdd(&hist[min(n, 255)], 1);
  }
  __syncthreads();
  if (threadIdx.x == 0) {  // exclusive offsets, longest bucket first
    int run = 0;
    for (int i = 255; i >= 1; --i) {
      const int c = hist[i];
      hist[i] = run;
      run += c;
    }
    p.meta[0] = run * p.ngrp;
    p.meta[4] = p.batch;  // the sizes this list is for (checked by every launch that reads it)
    p.meta[5] = p.max_splits;
    p.meta[6] = p.ngrp;
  }
  __syncthreads();
  for (int t = threadIdx.x; t < ncand; t += kPlanThreads) {
    const int b = t / p.max_splits, split = t % p.max_splits;
    const int n = decode_item_tiles(len_of(b), p.max_splits, split, chunk_len);
    if (n > 0) {
      const int pos = atomicAdd(&hist[min(n, 255)], 1);
      for (int g = 0; g < p.ngrp; ++g) p.plan[pos * p.ngrp + g] = make_int4(b, split, g, 0);
    }
  }
}

int dec::launch_decode_plan(const DecodeParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(paged_decode_plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, p);
  MSGL_CHECK_LAUNCH("msgl_paged_decode (plan)");
  return MSGL_OK;
}

// The instantiation of (dtype, fp8 pool, head_dim, group) applied to op; each
// (query, pool) type pair is built in a translation unit of its own.
static int dispatch(const DecodeOp& op, int dtype, bool q8, int head_dim, int group, const char* fn) {
  if (q8) {  // fp8 e4m3 pools with per-(slot, kv head) scales
    switch (dtype) {
      case MSGL_BF16: return decode_op_bf16_fp8(op, head_dim, group);
      case MSGL_F16: return decode_op_f16_fp8(op, head_dim, group);
    }
    set_error("%s: fp8 pools take bf16 or fp16 queries (dtype %d)", fn, dtype);
    return MSGL_ERR_UNSUPPORTED;
  }
  switch (dtype) {
    case MSGL_F32: return decode_op_f32(op, head_dim, group);
    case MSGL_BF16: return decode_op_bf16(op, head_dim, group);
    case MSGL_F16: return decode_op_f16(op, head_dim, group);
  }
  set_error("%s: unknown dtype %d", fn, dtype);
  return MSGL_ERR_UNSUPPORTED;
}

// A launch request over p, and a query of the instantiation's properties.
static DecodeOp launch_op(DecodeOpKind kind, const DecodeParams& p, int batch, hipStream_t stream) {
  return DecodeOp{kind, &p, batch, stream, 0, nullptr, nullptr};
}
static DecodeOp query_op(DecodeOpKind kind, int nwaves, int* resident, bool* flag) {
  return DecodeOp{kind, nullptr, 0, nullptr, nwaves, resident, flag};
}

// Workspace layout, each region 256-byte aligned: [meta | plan B*S*ngrp int4 |
// key offsets (B+1) i64 | (S > 1) m,l B*S*Hq*2 f32 | acc B*S*Hq*D f32].
static inline int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

static inline int decode_groups(int hkv) {
  const int nwaves = hkv < MSGL_DECODE_WAVES_PER_WG ? hkv : MSGL_DECODE_WAVES_PER_WG;
  return (hkv + nwaves - 1) / nwaves;
}

// Query-head groups above 8 that are multiples of 8 run as groups of 8 over
// virtual kv heads: virtual head v holds query heads 8v .. 8v+7 and reads pool
// head v / rep (rep = G / 8). A workgroup's wavefronts hold neighbouring
// virtual heads, so the rep wavefronts of one pool head read the same K/V rows
// at about the same time and all but the first find them in L2, while the
// group-8 kernel keeps its P.V accumulators in registers (a group of 16 needs
// twice as many and spills). A group of 8 over one or two pool heads runs as
// groups of 4 over twice the heads: more wavefronts per token where there are
// few (measured faster with the default split bound). Every call maps its heads through this, so the
// workspace, the plan, the decode and the merge agree; the map does not depend
// on the pool type (the plan call does not know it). fp8 pools read their
// scales by pool head too.
struct HeadMap {
  int hkv;    // kv heads the kernels see
  int group;  // query heads per such kv head
  int rep;    // such kv heads per pool kv head
};
static inline HeadMap head_map(int hq, int hkv) {
  const int g = hkv > 0 ? hq / hkv : 0;
  if (g > 8 && g % 8 == 0) return HeadMap{hkv * (g / 8), 8, g / 8};
  if (g == 8 && hkv <= 2) return HeadMap{hkv * 2, 4, 2};
  return HeadMap{hkv, g, 1};
}

struct DecodeWorkspace {
  int64_t plan, tok_off, part_ml, part_o, bytes;
};
static inline DecodeWorkspace decode_workspace(int batch, int hq, int hkv, int head_dim, int splits) {
  DecodeWorkspace w;
  const int64_t units = splits > 1 ? (int64_t)batch * splits * hq : 0;
  w.plan = 256;
  w.tok_off = w.plan + align256((int64_t)batch * splits * decode_groups(head_map(hq, hkv).hkv) * 16);
  w.part_ml = w.tok_off + align256(((int64_t)batch + 1) * 8);
  w.part_o = w.part_ml + align256(units * 2 * 4);
  w.bytes = w.part_o + align256(units * head_dim * 4);
  return w;
}

// Key ranges of a balanced launch: one per workgroup the device holds at once,
// per kv-head group.
#ifndef MSGL_DECODE_RANGE_ROUNDS
#define MSGL_DECODE_RANGE_ROUNDS 1
#endif


}  // namespace msgl

int64_t msgl::dec::decode_items(const DecodeParams& p) {
  // a balanced launch is chosen on the device (balanced_launch), so the grid
  // covers both forms; workgroups past the chosen one's items exit at once
  const int64_t list = (int64_t)p.batch * p.max_splits * p.ngrp;
  return p.balanced ? std::max<int64_t>((int64_t)p.nranges * p.ngrp, list) : list;
}

extern "C" int32_t msgl_paged_decode_default_splits(int32_t batch, int32_t num_kv_heads, int32_t max_seq_len) {
  // max_splits bounds both split forms. Key ranges (one per resident
  // workgroup, about 256 per kv-head group on MI355X) are at least
  // ceil(max_b L_b / (max_splits - 1)) keys long: S = 2 + ceil(8192 / (B Hkv)),
  // at least 4, leaves room for the longest request to be ~8x the average
  // before its ranges must grow, and a request of max_seq_len keys overlaps at
  // most ceil(max_seq_len / kMinChunk) + 1 ranges. Per-request chunks take the
  // plan's chunk count (~4096 wavefronts, chunks of kMinChunk..2048 keys),
  // which S must not cap.
  if (batch <= 0 || num_kv_heads <= 0) return 1;
  const int64_t units = (int64_t)batch * num_kv_heads;
  int64_t s = 2 + (8192 + units - 1) / units;
  if (s < 4) s = 4;
  int64_t c = (4096 + units - 1) / units;
  if (max_seq_len > 0) {
    const int64_t cap = (max_seq_len + msgl::kMinChunk - 1) / msgl::kMinChunk;
    if (s > cap + 1) s = cap + 1;
    if (c > cap) c = cap;
    const int64_t floor_c = (max_seq_len + 2047) / 2048;
    if (c < floor_c) c = floor_c;
  }
  if (s < c) s = c;
  // One or two kv heads over contexts of at most 4096 keys: 16 chunks per
  // request measured faster than the bound above (batch 16 and 64, L up to
  // 3072: 5-21%; batch 256: no change), where 4096 wavefronts are two rounds of
  // their 2-wavefront workgroups. Longer contexts keep it (a small batch of
  // long requests needs the chunks to fill the device).
  if (num_kv_heads <= 2 && max_seq_len > 0 && max_seq_len <= 4096 && s > 16) s = 16;
  if (s > msgl::kMaxSplits) s = msgl::kMaxSplits;
  return (int32_t)s;
}

extern "C" int64_t msgl_paged_decode_workspace_size(int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                                                    int32_t head_dim, int32_t max_splits) {
  if (batch <= 0 || num_qo_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0) return 0;
  if (max_splits > msgl::kMaxSplits) max_splits = msgl::kMaxSplits;
  if (max_splits < 1) max_splits = 1;
  return msgl::decode_workspace(batch, num_qo_heads, num_kv_heads, head_dim, max_splits).bytes;
}

enum DecodeMode { kPlanAndRun, kRunPlanned };

static int paged_decode_impl(const char* fn, DecodeMode mode, const void* q, const void* k_new, const void* v_new,
                             const int32_t* out_loc, const void* k_pool, const void* v_pool, const float* kv_scale,
                             const int32_t* kv_indptr, const int32_t* kv_indices,
                             const int32_t* seq_lens,
                             int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t page_size, int64_t num_slots, int32_t dtype, float scale, int32_t max_splits,
                             void* out, void* workspace, int64_t workspace_bytes, void* stream, uint32_t flags = 0);

extern "C" int msgl_paged_decode(const void* q, const void* k_pool, const void* v_pool, const int32_t* kv_indptr,
                                 const int32_t* kv_indices, const int32_t* seq_lens, int32_t batch,
                                 int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                 int64_t num_slots, int32_t dtype, float scale, int32_t max_splits, void* out,
                                 void* workspace, int64_t workspace_bytes, void* stream) {
  return paged_decode_impl("msgl_paged_decode", kPlanAndRun, q, nullptr, nullptr, nullptr, k_pool, v_pool, nullptr,
                           kv_indptr,
                           kv_indices, seq_lens, batch, num_qo_heads, num_kv_heads, head_dim, page_size, num_slots,
                           dtype, scale, max_splits, out, workspace, workspace_bytes, stream);
}

extern "C" int msgl_paged_decode_plan(const int32_t* kv_indptr, const int32_t* seq_lens, int32_t batch,
                                      int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                      int32_t max_splits, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(batch >= 0 && batch <= 65535, "msgl_paged_decode_plan: batch must be in [0, 65535]");
  if (batch == 0) return MSGL_OK;
  MSGL_CHECK_ARG(num_qo_heads > 0 && num_kv_heads > 0 && head_dim > 0 && num_qo_heads % num_kv_heads == 0,
                 "msgl_paged_decode_plan: bad head counts");
  MSGL_CHECK_ARG(kv_indptr != nullptr, "msgl_paged_decode_plan: null kv_indptr");
  if (max_splits <= 0) max_splits = msgl_paged_decode_default_splits(batch, num_kv_heads, 0);
  if (max_splits > kMaxSplits) max_splits = kMaxSplits;
  const int64_t need = msgl_paged_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim, max_splits);
  if (workspace == nullptr || workspace_bytes < need || (uintptr_t)workspace % 256 != 0) {
    set_error("msgl_paged_decode_plan: 256-byte aligned workspace of %lld bytes needed, %lld given",
              (long long)need, (long long)workspace_bytes);
    return MSGL_ERR_WORKSPACE;
  }
  DecodeParams p{};
  const DecodeWorkspace w = decode_workspace(batch, num_qo_heads, num_kv_heads, head_dim, max_splits);
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  p.kv_indptr = kv_indptr;
  p.seq_lens = seq_lens;
  p.meta = reinterpret_cast<int*>(ws);
  p.plan = reinterpret_cast<int4*>(ws + w.plan);
  p.tok_off = reinterpret_cast<int64_t*>(ws + w.tok_off);
  const HeadMap hm = head_map(num_qo_heads, num_kv_heads);
  p.hq = num_qo_heads;
  p.hkv = hm.hkv;
  p.hkv_pool = num_kv_heads;
  p.kv_rep = hm.rep;
  p.max_splits = max_splits;
  p.batch = batch;
  p.ngrp = decode_groups(hm.hkv);
  hipLaunchKernelGGL(paged_decode_plan_kernel, dim3(1), dim3(kPlanThreads), 0, (hipStream_t)stream, p);
  MSGL_CHECK_LAUNCH("msgl_paged_decode_plan");
  return MSGL_OK;
}

extern "C" int msgl_paged_decode_planned(const void* q, const void* k_pool, const void* v_pool,
                                         const int32_t* kv_indptr, const int32_t* kv_indices,
                                         const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                                         int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int64_t num_slots,
                                         int32_t dtype, float scale, int32_t max_splits, void* out, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  return paged_decode_impl("msgl_paged_decode_planned", kRunPlanned, q, nullptr, nullptr, nullptr, k_pool, v_pool,
                           nullptr, kv_indptr, kv_indices, seq_lens, batch, num_qo_heads, num_kv_heads, head_dim, page_size,
                           num_slots, dtype, scale, max_splits, out, workspace, workspace_bytes, stream);
}

extern "C" int msgl_paged_decode_store(const void* q, const void* k_new, const void* v_new, const int32_t* out_loc,
                                       void* k_pool, void* v_pool, const int32_t* kv_indptr,
                                       const int32_t* kv_indices, const int32_t* seq_lens, int32_t batch,
                                       int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                       int32_t page_size, int64_t num_slots, int32_t dtype, float scale,
                                       int32_t max_splits, void* out, void* workspace, int64_t workspace_bytes,
                                       void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(k_new && v_new && out_loc, "msgl_paged_decode_store: null k_new, v_new or out_loc");
  MSGL_CHECK_ARG(((uintptr_t)k_new | (uintptr_t)v_new) % 16 == 0,
                 "msgl_paged_decode_store: k_new and v_new must be 16-byte aligned");
  return paged_decode_impl("msgl_paged_decode_store", kPlanAndRun, q, k_new, v_new, out_loc, k_pool, v_pool,
                           nullptr, kv_indptr, kv_indices, seq_lens, batch, num_qo_heads, num_kv_heads, head_dim, page_size,
                           num_slots, dtype, scale, max_splits, out, workspace, workspace_bytes, stream);
}

extern "C" int msgl_paged_decode_store_planned(const void* q, const void* k_new, const void* v_new,
                                               const int32_t* out_loc, void* k_pool, void* v_pool,
                                               const int32_t* kv_indptr, const int32_t* kv_indices,
                                               const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                                               int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                               int64_t num_slots, int32_t dtype, float scale, int32_t max_splits,
                                               void* out, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(k_new && v_new && out_loc, "msgl_paged_decode_store_planned: null k_new, v_new or out_loc");
  MSGL_CHECK_ARG(((uintptr_t)k_new | (uintptr_t)v_new) % 16 == 0,
                 "msgl_paged_decode_store_planned: k_new and v_new must be 16-byte aligned");
  return paged_decode_impl("msgl_paged_decode_store_planned", kRunPlanned, q, k_new, v_new, out_loc, k_pool, v_pool,
                           nullptr, kv_indptr, kv_indices, seq_lens, batch, num_qo_heads, num_kv_heads, head_dim, page_size,
                           num_slots, dtype, scale, max_splits, out, workspace, workspace_bytes, stream);
}

extern "C" int msgl_paged_decode_fp8(const void* q, const void* k_pool, const void* v_pool, const float* kv_scale,
                                     const int32_t* kv_indptr, const int32_t* kv_indices,
                                     const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                                     int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int64_t num_slots,
                                     int32_t dtype, float scale, int32_t max_splits, void* out, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(kv_scale != nullptr, "msgl_paged_decode_fp8: null kv_scale");
  return paged_decode_impl("msgl_paged_decode_fp8", kPlanAndRun, q, nullptr, nullptr, nullptr, k_pool, v_pool, kv_scale,
                           kv_indptr, kv_indices, seq_lens, batch, num_qo_heads, num_kv_heads, head_dim,
                           page_size, num_slots, dtype, scale, max_splits, out, workspace, workspace_bytes, stream);
}

extern "C" int msgl_paged_decode_fp8_planned(const void* q, const void* k_pool, const void* v_pool,
                                             const float* kv_scale, const int32_t* kv_indptr,
                                             const int32_t* kv_indices, const int32_t* seq_lens, int32_t batch,
                                             int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                             int32_t page_size, int64_t num_slots, int32_t dtype, float scale,
                                             int32_t max_splits, void* out, void* workspace, int64_t workspace_bytes,
                                             void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(kv_scale != nullptr, "msgl_paged_decode_fp8_planned: null kv_scale");
  return paged_decode_impl("msgl_paged_decode_fp8_planned", kRunPlanned, q, nullptr, nullptr, nullptr, k_pool, v_pool,
                           kv_scale, kv_indptr, kv_indices, seq_lens, batch, num_qo_heads, num_kv_heads,
                           head_dim, page_size, num_slots, dtype, scale, max_splits, out, workspace, workspace_bytes,
                           stream);
}

extern "C" int msgl_paged_decode_store_fp8(const void* q, const void* k_new, const void* v_new,
                                           const int32_t* out_loc, void* k_pool, void* v_pool, float* kv_scale,
                                           const int32_t* kv_indptr, const int32_t* kv_indices,
                                           const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                                           int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                           int64_t num_slots, int32_t dtype, float scale, int32_t max_splits,
                                           void* out, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(kv_scale != nullptr, "msgl_paged_decode_store_fp8: null kv_scale");
  MSGL_CHECK_ARG(k_new && v_new && out_loc, "msgl_paged_decode_store_fp8: null k_new, v_new or out_loc");
  MSGL_CHECK_ARG(((uintptr_t)k_new | (uintptr_t)v_new) % 16 == 0,
                 "msgl_paged_decode_store_fp8: k_new and v_new must be 16-byte aligned");
  return paged_decode_impl("msgl_paged_decode_store_fp8", kPlanAndRun, q, k_new, v_new, out_loc, k_pool, v_pool,
                           kv_scale, kv_indptr, kv_indices, seq_lens, batch, num_qo_heads, num_kv_heads, head_dim,
                           page_size, num_slots, dtype, scale, max_splits, out, workspace, workspace_bytes, stream);
}

extern "C" int msgl_paged_decode_store_fp8_planned(const void* q, const void* k_new, const void* v_new,
                                                   const int32_t* out_loc, void* k_pool, void* v_pool,
                                                   float* kv_scale, const int32_t* kv_indptr,
                                                   const int32_t* kv_indices, const int32_t* seq_lens, int32_t batch,
                                                   int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                                   int32_t page_size, int64_t num_slots, int32_t dtype, float scale,
                                                   int32_t max_splits, void* out, void* workspace,
                                                   int64_t workspace_bytes, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(kv_scale != nullptr, "msgl_paged_decode_store_fp8_planned: null kv_scale");
  MSGL_CHECK_ARG(k_new && v_new && out_loc, "msgl_paged_decode_store_fp8_planned: null k_new, v_new or out_loc");
  MSGL_CHECK_ARG(((uintptr_t)k_new | (uintptr_t)v_new) % 16 == 0,
                 "msgl_paged_decode_store_fp8_planned: k_new and v_new must be 16-byte aligned");
  return paged_decode_impl("msgl_paged_decode_store_fp8_planned", kRunPlanned, q, k_new, v_new, out_loc, k_pool,
                           v_pool, kv_scale, kv_indptr, kv_indices, seq_lens, batch, num_qo_heads, num_kv_heads,
                           head_dim, page_size, num_slots, dtype, scale, max_splits, out, workspace, workspace_bytes,
                           stream);
}

// Validates the arguments of a decode call and fills p (workspace regions
// included); empty: batch 0, nothing to launch.
int msgl::dec::decode_params(const char* fn, bool planned, const void* q, const void* k_new, const void* v_new,
                             const int32_t* out_loc, const void* k_pool, const void* v_pool, const float* kv_scale,
                             const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                             int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t page_size, int64_t num_slots, int32_t dtype, float scale, int32_t max_splits,
                             void* out, void* workspace, int64_t workspace_bytes, DecodeParams& p, bool& empty) {
  clear_error();
  empty = false;
  MSGL_CHECK_ARG(batch >= 0 && batch <= 65535, "%s: batch must be in [0, 65535]", fn);
  if (batch == 0) {
    empty = true;
    return MSGL_OK;
  }
  MSGL_CHECK_ARG(num_qo_heads > 0 && num_kv_heads > 0 && head_dim > 0, "%s: sizes must be > 0", fn);
  MSGL_CHECK_ARG(num_qo_heads % num_kv_heads == 0, "%s: Hq (%d) must be a multiple of Hkv (%d)",
                 fn, num_qo_heads, num_kv_heads);
  MSGL_CHECK_ARG(page_size >= 1, "%s: page_size must be >= 1", fn);
  MSGL_CHECK_ARG(page_size == 1 || seq_lens != nullptr, "%s: page_size > 1 needs seq_lens", fn);
  MSGL_CHECK_ARG(num_slots > 0 && num_slots <= ((int64_t)1 << 31) - 1,
                 "%s: num_slots must be in [1, 2^31)", fn);
  MSGL_CHECK_ARG(q && k_pool && v_pool && kv_indptr && kv_indices && out, "%s: null pointer", fn);
  MSGL_CHECK_ARG(((uintptr_t)q | (uintptr_t)k_pool | (uintptr_t)v_pool | (uintptr_t)out) % 16 == 0,
                 "%s: q, pools and out must be 16-byte aligned", fn);
  MSGL_CHECK_ARG((uintptr_t)kv_scale % 8 == 0, "%s: kv_scale must be 8-byte aligned", fn);
  if (dtype_size(dtype) == 0) {
    set_error("%s: unknown dtype %d", fn, dtype);
    return MSGL_ERR_UNSUPPORTED;
  }
  if (max_splits <= 0) max_splits = msgl_paged_decode_default_splits(batch, num_kv_heads, 0);
  if (max_splits > kMaxSplits) max_splits = kMaxSplits;
  const int64_t need =
      msgl_paged_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim, max_splits);
  if (workspace == nullptr || workspace_bytes < need || (uintptr_t)workspace % 256 != 0) {
    set_error("%s: 256-byte aligned workspace of %lld bytes needed, %lld given", fn, (long long)need,
              (long long)workspace_bytes);
    return MSGL_ERR_WORKSPACE;
  }
  p.q = q;
  p.k_pool = k_pool;
  p.v_pool = v_pool;
  p.kv_scale = kv_scale;
  p.kv_indptr = kv_indptr;
  p.kv_indices = kv_indices;
  p.seq_lens = seq_lens;
  p.out = out;
  p.k_new = k_new;
  p.v_new = v_new;
  p.out_loc = out_loc;
  p.k_pool_w = const_cast<void*>(k_pool);
  p.v_pool_w = const_cast<void*>(v_pool);
  p.kv_scale_w = const_cast<float*>(kv_scale);
  const DecodeWorkspace w = decode_workspace(batch, num_qo_heads, num_kv_heads, head_dim, max_splits);
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  p.meta = reinterpret_cast<int*>(ws);
  p.plan = reinterpret_cast<int4*>(ws + w.plan);
  p.tok_off = reinterpret_cast<int64_t*>(ws + w.tok_off);
  p.part_ml = max_splits > 1 ? reinterpret_cast<float*>(ws + w.part_ml) : nullptr;
  p.part_o = max_splits > 1 ? reinterpret_cast<float*>(ws + w.part_o) : nullptr;
  const HeadMap hm = head_map(num_qo_heads, num_kv_heads);
  p.batch = batch;
  p.ngrp = decode_groups(hm.hkv);
  p.planned = planned;
  p.num_slots = num_slots;
  p.hq = num_qo_heads;
  p.hkv = hm.hkv;
  p.hkv_pool = num_kv_heads;
  p.kv_rep = hm.rep;
  p.page_size = page_size;
  p.max_splits = max_splits;
  p.scale_log2 = scale * kLog2e;
  p.balanced = false;
  p.skip_merge = false;
  p.nranges = 1;
  p.shared_head = false;
  p.hpg = hm.hkv < MSGL_DECODE_WAVES_PER_WG ? hm.hkv : MSGL_DECODE_WAVES_PER_WG;
  if (max_splits == 1) {
    bool shared = false;
    const int st = dispatch(query_op(kOpShared, 0, nullptr, &shared), dtype, kv_scale != nullptr, head_dim,
                            hm.group, fn);
    if (st != MSGL_OK) return st;
    // With virtual kv heads the per-head-group form keeps the virtual heads of
    // a pool head in one workgroup, so its rows are fetched once; the
    // shared-head form gives each its own workgroup on another XCD.
    p.shared_head = shared && hm.rep == 1;
  }
  if (max_splits > 1) {
    const int nwaves = hm.hkv < MSGL_DECODE_WAVES_PER_WG ? hm.hkv : MSGL_DECODE_WAVES_PER_WG;
    int resident = 0;
    bool ranges = false;
    const int st = dispatch(query_op(kOpResident, nwaves, &resident, &ranges), dtype, kv_scale != nullptr, head_dim,
                            hm.group, fn);
    if (st != MSGL_OK) return st;
    p.balanced = ranges;
    p.nranges = std::max(1, resident * MSGL_DECODE_RANGE_ROUNDS / p.ngrp);
  }
  return MSGL_OK;
}

static int paged_decode_impl(const char* fn, DecodeMode mode, const void* q, const void* k_new, const void* v_new,
                             const int32_t* out_loc, const void* k_pool, const void* v_pool, const float* kv_scale,
                             const int32_t* kv_indptr, const int32_t* kv_indices,
                             const int32_t* seq_lens,
                             int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t page_size, int64_t num_slots, int32_t dtype, float scale, int32_t max_splits,
                             void* out, void* workspace, int64_t workspace_bytes, void* stream, uint32_t flags) {
  using namespace msgl;
  DecodeParams p;
  bool empty = false;
  const int st = dec::decode_params(fn, mode == kRunPlanned, q, k_new, v_new, out_loc, k_pool, v_pool, kv_scale,
                                    kv_indptr, kv_indices, seq_lens, batch, num_qo_heads, num_kv_heads, head_dim,
                                    page_size, num_slots, dtype, scale, max_splits, out, workspace, workspace_bytes, p,
                                    empty);
  if (st != MSGL_OK || empty) return st;
  p.skip_merge = (flags & MSGL_DECODE_NO_MERGE) != 0;
  return dispatch(launch_op(kOpLaunch, p, batch, (hipStream_t)stream), dtype, kv_scale != nullptr, head_dim,
                  p.hq / p.hkv, fn);
}

extern "C" int msgl_paged_decode_planned_ex(const void* q, const void* k_new, const void* v_new,
                                            const int32_t* out_loc, void* k_pool, void* v_pool, float* kv_scale,
                                            const int32_t* kv_indptr, const int32_t* kv_indices,
                                            const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                                            int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                            int64_t num_slots, int32_t dtype, float scale, int32_t max_splits,
                                            uint32_t flags, void* out, void* workspace, int64_t workspace_bytes,
                                            void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG((flags & ~(uint32_t)MSGL_DECODE_NO_MERGE) == 0, "msgl_paged_decode_planned_ex: unknown flags 0x%x",
                 flags);
  MSGL_CHECK_ARG((k_new == nullptr) == (v_new == nullptr) && (k_new == nullptr) == (out_loc == nullptr),
                 "msgl_paged_decode_planned_ex: k_new, v_new and out_loc go together");
  MSGL_CHECK_ARG(((uintptr_t)k_new | (uintptr_t)v_new) % 16 == 0,
                 "msgl_paged_decode_planned_ex: k_new and v_new must be 16-byte aligned");
  return paged_decode_impl("msgl_paged_decode_planned_ex", kRunPlanned, q, k_new, v_new, out_loc, k_pool, v_pool,
                           kv_scale, kv_indptr, kv_indices, seq_lens, batch, num_qo_heads, num_kv_heads, head_dim,
                           page_size, num_slots, dtype, scale, max_splits, out, workspace, workspace_bytes, stream,
                           flags);
}

extern "C" int msgl_paged_decode_merge(const int32_t* kv_indptr, const int32_t* seq_lens, int32_t batch,
                                       int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                                       int32_t kv_fp8, int32_t max_splits, void* out, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(batch >= 0 && batch <= 65535, "msgl_paged_decode_merge: batch must be in [0, 65535]");
  if (batch == 0) return MSGL_OK;
  MSGL_CHECK_ARG(num_qo_heads > 0 && num_kv_heads > 0 && head_dim > 0 && num_qo_heads % num_kv_heads == 0,
                 "msgl_paged_decode_merge: bad head counts");
  MSGL_CHECK_ARG(kv_indptr != nullptr && out != nullptr, "msgl_paged_decode_merge: null kv_indptr or out");
  MSGL_CHECK_ARG((uintptr_t)out % 16 == 0, "msgl_paged_decode_merge: out must be 16-byte aligned");
  if (dtype_size(dtype) == 0) {
    set_error("msgl_paged_decode_merge: unknown dtype %d", dtype);
    return MSGL_ERR_UNSUPPORTED;
  }
  if (max_splits <= 0) max_splits = msgl_paged_decode_default_splits(batch, num_kv_heads, 0);
  if (max_splits > kMaxSplits) max_splits = kMaxSplits;
  const int64_t need = msgl_paged_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim, max_splits);
  if (workspace == nullptr || workspace_bytes < need || (uintptr_t)workspace % 256 != 0) {
    set_error("msgl_paged_decode_merge: 256-byte aligned workspace of %lld bytes needed, %lld given",
              (long long)need, (long long)workspace_bytes);
    return MSGL_ERR_WORKSPACE;
  }
  if (max_splits == 1) return MSGL_OK;  // every request was written by the decode launch
  DecodeParams p{};
  const DecodeWorkspace w = decode_workspace(batch, num_qo_heads, num_kv_heads, head_dim, max_splits);
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  p.kv_indptr = kv_indptr;
  p.seq_lens = seq_lens;
  p.out = out;
  p.meta = reinterpret_cast<int*>(ws);
  p.plan = reinterpret_cast<int4*>(ws + w.plan);
  p.tok_off = reinterpret_cast<int64_t*>(ws + w.tok_off);
  p.part_ml = reinterpret_cast<float*>(ws + w.part_ml);
  p.part_o = reinterpret_cast<float*>(ws + w.part_o);
  const HeadMap hm = head_map(num_qo_heads, num_kv_heads);
  p.batch = batch;
  p.hq = num_qo_heads;
  p.hkv = hm.hkv;
  p.hkv_pool = num_kv_heads;
  p.kv_rep = hm.rep;
  p.max_splits = max_splits;
  p.ngrp = decode_groups(hm.hkv);
  // the split form the decode launch chose: key ranges are sized by that
  // kernel's residency, so it is derived the way the decode call derives it
  const int nwaves = hm.hkv < MSGL_DECODE_WAVES_PER_WG ? hm.hkv : MSGL_DECODE_WAVES_PER_WG;
  int resident = 0;
  bool ranges = false;
  const int st = dispatch(query_op(kOpResident, nwaves, &resident, &ranges), dtype, kv_fp8 != 0, head_dim,
                          hm.group, "msgl_paged_decode_merge");
  if (st != MSGL_OK) return st;
  p.balanced = ranges;
  p.nranges = std::max(1, resident * MSGL_DECODE_RANGE_ROUNDS / p.ngrp);
  return dispatch(launch_op(kOpMerge, p, batch, (hipStream_t)stream), dtype, false, head_dim,
                  hm.group,
                  "msgl_paged_decode_merge");
}

// ---------------------------------------------------------------------------
// Allocation-free decode: msgl_paged_decode_store with its workspace (the work
// list and the split-K partials) in a file-scope device array instead of a
// caller buffer. Each device holds its own copy of the array from the first
// call on it until the process ends; its address on the current device comes
// from hipGetSymbolAddress, looked up once per device (the array's name in
// host code is only a host-side stand-in for it). Every call on a device uses
// that device's one copy, so calls that overlap in time on one device (other
// streams, other threads) race; calls in order on one stream do not. The
// workspace needs no clearing: the plan kernel writes everything the decode
// and merge kernels read.
// ---------------------------------------------------------------------------
namespace msgl {
namespace {

constexpr int64_t kNoAllocScratchBytes = MSGL_NOALLOC_WORKSPACE_BYTES;  // per device
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

std::atomic<void*> g_scratch_ptr[kMaxDevices];

// The device address of `scratch` on the current device.
int scratch_on_current_device(void** ptr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("msgl_paged_decode_store_noalloc: no usable current device");
    return MSGL_ERR_HIP;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr) {
      set_error("msgl_paged_decode_store_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(err));
      return MSGL_ERR_HIP;
    }
    g_scratch_ptr[dev].store(p, std::memory_order_release);  // racing first calls store the same address
  }
  *ptr = p;
  return MSGL_OK;
}

}  // namespace
}  // namespace msgl

extern "C" int msgl_paged_decode_store_noalloc(const void* q, const void* k_new, const void* v_new,
                                               const int32_t* out_loc, void* k_pool, void* v_pool,
                                               const int32_t* kv_indptr, const int32_t* kv_indices,
                                               const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                                               int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                               int64_t num_slots, int32_t dtype, float scale, int32_t max_splits,
                                               void* out, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(k_new && v_new && out_loc, "msgl_paged_decode_store_noalloc: null k_new, v_new or out_loc");
  MSGL_CHECK_ARG(((uintptr_t)k_new | (uintptr_t)v_new) % 16 == 0,
                 "msgl_paged_decode_store_noalloc: k_new and v_new must be 16-byte aligned");
  MSGL_CHECK_ARG(batch >= 0 && batch <= 65535, "msgl_paged_decode_store_noalloc: batch must be in [0, 65535]");
  if (batch == 0) return MSGL_OK;
  MSGL_CHECK_ARG(num_qo_heads > 0 && num_kv_heads > 0 && head_dim > 0,
                 "msgl_paged_decode_store_noalloc: sizes must be > 0");
  int32_t splits = max_splits;
  if (splits <= 0) splits = msgl_paged_decode_default_splits(batch, num_kv_heads, 0);
  if (splits > kMaxSplits) splits = kMaxSplits;
  const int64_t need = msgl_paged_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim, splits);
  if (need > kNoAllocScratchBytes) {
    set_error("msgl_paged_decode_store_noalloc: these sizes need %lld bytes of workspace, more than the %lld the "
              "library holds per device (fewer max_splits or a smaller batch fit; msgl_paged_decode_store takes "
              "any workspace)",
              (long long)need, (long long)kNoAllocScratchBytes);
    return MSGL_ERR_WORKSPACE;
  }
  void* ws = nullptr;
  const int st = scratch_on_current_device(&ws);
  if (st != MSGL_OK) return st;
  return paged_decode_impl("msgl_paged_decode_store_noalloc", kPlanAndRun, q, k_new, v_new, out_loc, k_pool, v_pool,
                           nullptr, kv_indptr, kv_indices, seq_lens, batch, num_qo_heads, num_kv_heads, head_dim,
                           page_size, num_slots, dtype, scale, splits, out, ws, kNoAllocScratchBytes, stream);
}
