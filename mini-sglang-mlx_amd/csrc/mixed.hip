// Single-launch mixed step: the paged decode of a batch's decode requests and
// the ragged prefill of its prefill chunks as one grid, then one merge launch.
//
// The reference dispatches a whole batch to one phase (attention/base.py:49-60,
// core.py:111-116); per request the results here are exactly those of the
// decode path (attention/naive.py:50-60 / attention/metal.py:112-131, with the
// new token's store of kvcache/pool.py:47-50 fused in) or of the prefill path
// (attention/base.py:85-105): each workgroup runs the unchanged decode or
// prefill body on one work item of the lists msgl_paged_decode_plan and
// msgl_prefill_plan built (the decode part always runs per-request chunks).
//
// The grid is cut into groups of 8 workgroups (workgroup i runs on XCD i % 8).
// Group c is a prefill group when floor(c P / (P + Q)) steps up at c (P, Q:
// the prefill and decode lists' lengths in groups of 8, from the list lengths
// the plans left in the workspaces), otherwise a decode group; workgroup j of
// the k-th group of a kind takes item 8k + j of that list. The two
// longest-first lists interleave in proportion, so CUs hold HBM-bound decode
// and matrix-core-bound prefill workgroups side by side from the first wave of
// dispatch on, and each item runs on the XCD it runs on in its own kernel
// (item % 8: a prefill head's query blocks share one L2). Both bodies run as
// 4-wavefront workgroups; the launch takes the larger LDS of the two (the
// prefill ring) and the prefill's register budget.
#include "mixed_launch.h"

extern "C" int msgl_paged_decode_planned(const void* q, const void* k_pool, const void* v_pool,
                                         const int32_t* kv_indptr, const int32_t* kv_indices,
                                         const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                                         int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int64_t num_slots,
                                         int32_t dtype, float scale, int32_t max_splits, void* out, void* workspace,
                                         int64_t workspace_bytes, void* stream);
extern "C" int msgl_paged_decode_store_planned(const void* q, const void* k_new, const void* v_new,
                                               const int32_t* out_loc, void* k_pool, void* v_pool,
                                               const int32_t* kv_indptr, const int32_t* kv_indices,
                                               const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                                               int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                               int64_t num_slots, int32_t dtype, float scale, int32_t max_splits,
                                               void* out, void* workspace, int64_t workspace_bytes, void* stream);
extern "C" int msgl_prefill_ragged_planned(const void* q, const void* k_pool, const void* v_pool,
                                           const int32_t* q_indptr, const int32_t* kv_indptr,
                                           const int32_t* kv_indices, const int32_t* seq_lens, int32_t num_reqs,
                                           int32_t num_tokens, int32_t max_extend_len, int32_t max_seq_len,
                                           int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                           int32_t page_size, int64_t num_slots, int32_t dtype, float scale,
                                           int32_t max_splits, void* out, void* workspace, int64_t workspace_bytes,
                                           void* stream);

extern "C" int msgl_mixed_attention(const void* q_dec, const void* k_new, const void* v_new, const int32_t* out_loc,
                                    const int32_t* dec_kv_indptr, const int32_t* dec_kv_indices,
                                    const int32_t* dec_seq_lens, int32_t num_decode, int32_t dec_max_splits,
                                    void* out_dec, void* dec_workspace, int64_t dec_workspace_bytes,
                                    const void* q_pf, const int32_t* q_indptr, const int32_t* pf_kv_indptr,
                                    const int32_t* pf_kv_indices, const int32_t* pf_seq_lens, int32_t num_prefill,
                                    int32_t num_tokens, int32_t max_extend_len, int32_t max_seq_len,
                                    int32_t pf_max_splits, void* out_pf, void* pf_workspace,
                                    int64_t pf_workspace_bytes, void* k_pool, void* v_pool, int32_t num_qo_heads,
                                    int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int64_t num_slots,
                                    int32_t dtype, float scale, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(num_decode >= 0 && num_prefill >= 0, "msgl_mixed_attention: request counts must be >= 0");
  // The single launch is built for 16-bit q, head_dim 64 and 128 and Hq/Hkv 1
  // to 8 (a larger group's decode accumulators do not fit beside the prefill
  // body's registers); its decode body takes the decode's group (4 where the
  // decode runs 8 over virtual kv heads). Other shapes, and batches of one phase, run the phases
  // as launches of their own on the stream: the same results as the decode and
  // prefill calls, which touch disjoint slots (a request is in one phase).
  const int group = num_kv_heads > 0 && num_qo_heads % num_kv_heads == 0 ? num_qo_heads / num_kv_heads : 0;
  const bool one_launch = (dtype == MSGL_BF16 || dtype == MSGL_F16) && (head_dim == 64 || head_dim == 128) &&
                          group >= 1 && group <= 8;
  if (num_decode == 0 || num_prefill == 0 || max_extend_len == 0 || num_tokens == 0 || !one_launch) {
    int st = MSGL_OK;
    if (num_prefill > 0)
      st = msgl_prefill_ragged_planned(q_pf, k_pool, v_pool, q_indptr, pf_kv_indptr, pf_kv_indices, pf_seq_lens,
                                       num_prefill, num_tokens, max_extend_len, max_seq_len, num_qo_heads,
                                       num_kv_heads, head_dim, page_size, num_slots, dtype, scale, pf_max_splits,
                                       out_pf, pf_workspace, pf_workspace_bytes, stream);
    if (st == MSGL_OK && num_decode > 0)
      st = k_new != nullptr
               ? msgl_paged_decode_store_planned(q_dec, k_new, v_new, out_loc, k_pool, v_pool, dec_kv_indptr,
                                                 dec_kv_indices, dec_seq_lens, num_decode, num_qo_heads, num_kv_heads,
                                                 head_dim, page_size, num_slots, dtype, scale, dec_max_splits,
                                                 out_dec, dec_workspace, dec_workspace_bytes, stream)
               : msgl_paged_decode_planned(q_dec, k_pool, v_pool, dec_kv_indptr, dec_kv_indices, dec_seq_lens,
                                           num_decode, num_qo_heads, num_kv_heads, head_dim, page_size, num_slots,
                                           dtype, scale, dec_max_splits, out_dec, dec_workspace, dec_workspace_bytes,
                                           stream);
    return st;
  }
  MSGL_CHECK_ARG((k_new == nullptr) == (v_new == nullptr) && (k_new == nullptr || out_loc != nullptr),
                 "msgl_mixed_attention: k_new, v_new and out_loc go together");
  MSGL_CHECK_ARG(((uintptr_t)k_new | (uintptr_t)v_new) % 16 == 0,
                 "msgl_mixed_attention: k_new and v_new must be 16-byte aligned");
  pf::PrefillParams pp;
  bool empty = false;
  int st = pf::prefill_params("msgl_mixed_attention", pf::kRunPlanned, q_pf, k_pool, v_pool, nullptr, q_indptr,
                              pf_kv_indptr, pf_kv_indices, pf_seq_lens, num_prefill, num_tokens, max_extend_len,
                              max_seq_len, num_qo_heads, num_kv_heads, head_dim, page_size, num_slots, dtype, scale,
                              pf_max_splits, out_pf, pf_workspace, pf_workspace_bytes, pp, empty);
  if (st != MSGL_OK) return st;
  dec::DecodeParams dp;
  st = dec::decode_params("msgl_mixed_attention", true, q_dec, k_new, v_new, out_loc, k_pool, v_pool, nullptr,
                          dec_kv_indptr, dec_kv_indices, dec_seq_lens, num_decode, num_qo_heads, num_kv_heads,
                          head_dim, page_size, num_slots, dtype, scale, dec_max_splits, out_dec, dec_workspace,
                          dec_workspace_bytes, dp, empty);
  if (st != MSGL_OK) return st;
  // The decode part follows the per-request work list: key ranges sized for
  // the decode kernel's own residency would not all fit beside the prefill
  // items (measured slower), and the list keeps the longest items first.
  dp.balanced = false;
  dp.shared_head = false;  // one workgroup per work item here (max_splits == 1 runs the per-head-group form)
  hipStream_t s = (hipStream_t)stream;
  return dtype == MSGL_BF16 ? mixed_launch_bf16(pp, dp, num_decode, max_extend_len, head_dim, group, s)
                            : mixed_launch_f16(pp, dp, num_decode, max_extend_len, head_dim, group, s);
}
