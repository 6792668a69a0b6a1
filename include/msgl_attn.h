/*
 * msgl_attn.h -- C ABI of the MI355X (gfx950) attention backend for
 * mini-sglang-mlx's attention hot path.
 *
 * Every entry point takes plain device pointers and sizes (no framework
 * types), enqueues work on the caller's HIP stream (`stream` is a hipStream_t,
 * NULL = the null stream), never synchronises and never allocates: scratch
 * memory is passed in by the caller. All functions return 0 on success or a
 * MSGL_ERR_* code, with a message for the calling thread in msgl_last_error().
 *
 * Reference interfaces replaced (paths relative to the reference's
 * python/minisgl_mlx/):
 *   msgl_store_kv            kvcache/pool.py:47-50        MHAKVCache.store_kv
 *   msgl_paged_decode        attention/metal.py:112-131   paged_decode_attention
 *                            (semantics of attention/naive.py:50-60 forward_decode)
 *   msgl_paged_decode_store  kvcache/pool.py:47-50 + attention/metal.py:112-131 in one launch
 *                            (+ _plan / _planned / _store_planned: plan once per step;
 *                            _planned_ex + _merge: the decode and split-K merge launches apart)
 *   msgl_prefill_ragged      attention/base.py:85-105     BaseAttnBackend._forward_prefill
 *                            (+ _default_splits, _workspace_size; _plan / _planned: plan once per step)
 *   msgl_build_step_indices  scheduler/scheduler.py:154-157 + attention/metal.py:145-152
 *                            + attention/base.py:70-83 (index metadata, on the GPU)
 *   msgl_table_scatter       device mirror of scheduler/cache.py:53-72's page-table writes
 *   msgl_rope                layers.py:45-56 (RotaryEmbedding.__call__, rotate-half mx.fast.rope)
 *   msgl_rope_store_kv       layers.py:107-109 (rotate q and k, then store_kv) in one launch
 *   msgl_store_kv_fp8,       the fp8 KV cache of docs/09-exercises.md:81-82 (store_kv and paged
 *   msgl_paged_decode_fp8,   decode over pools of e4m3 codes with one scale per slot and kv head,
 *   msgl_paged_decode_store_fp8  the two in one launch,
 *   msgl_prefill_ragged_fp8  and the ragged prefill over them)
 *   msgl_mixed_attention     a batch's decode requests (attention/metal.py:112-131 + the store of
 *                            kvcache/pool.py:47-50) and prefill chunks (attention/base.py:85-105)
 *                            in one launch
 *   msgl_validate_metadata   attention/metal.py:122's precondition checks, for device-built indices
 *
 * Layouts (identical to the reference, no transposes at the boundary):
 *   q, out   [T, Hq, D]   row-major, dtype `dtype`
 *   k, v     [T, Hkv, D]
 *   pools    [num_slots, Hkv, D] one K and one V buffer per layer
 *   indices  int32; q head h reads kv head h / (Hq / Hkv)
 */
#ifndef MSGL_ATTN_H_
#define MSGL_ATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MSGL_ABI_VERSION 2

enum msgl_status {
  MSGL_OK = 0,
  MSGL_ERR_INVALID = 1,     /* bad argument (shape, null pointer, range)  */
  MSGL_ERR_UNSUPPORTED = 2, /* valid but not built (dtype/head_dim/group) */
  MSGL_ERR_WORKSPACE = 3,   /* workspace too small                        */
  MSGL_ERR_HIP = 4          /* the HIP runtime reported an error          */
};

enum msgl_dtype { MSGL_F32 = 0, MSGL_BF16 = 1, MSGL_F16 = 2 };

/* Violations msgl_validate_metadata reports (status[0]). */
enum msgl_meta_error {
  MSGL_META_OK = 0,
  MSGL_META_KV_INDPTR = 1, /* kv_indptr[0] < 0 or kv_indptr decreasing              */
  MSGL_META_KV_RANGE = 2,  /* kv_indptr[R] beyond the entries kv_indices holds       */
  MSGL_META_SEQ_LEN = 3,   /* a length < 0, or needing more entries than its row has */
  MSGL_META_SLOT = 4,      /* an entry read names a slot (page) outside the pool     */
  MSGL_META_Q_INDPTR = 5,  /* q_indptr not 0 .. num_tokens, or decreasing            */
  MSGL_META_EXTEND = 6     /* an extend length E_r > L_r                             */
};

/* ABI version of the loaded library (MSGL_ABI_VERSION). */
int msgl_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* msgl_last_error(void);

/*
 * KV store: k_pool[out_loc[t]] = k[t]; v_pool[out_loc[t]] = v[t] for t < num_tokens.
 * Replaces kvcache/pool.py:47-50 (called before attention, layers.py:109).
 * Bit-exact row copy of Hkv*D elements. out_loc entries must be distinct
 * (the allocator's invariant, scheduler/cache.py:124-132); an entry outside
 * [0, num_slots) is skipped, never written.
 */
int msgl_store_kv(const void* k, const void* v, const int32_t* out_loc, void* k_pool, void* v_pool,
                  int64_t num_tokens, int32_t num_kv_heads, int32_t head_dim, int64_t num_slots,
                  int32_t dtype, void* stream);

/* Default split count for msgl_paged_decode (max_splits <= 0 picks this);
 * max_seq_len (0: unknown) caps it at what a request of that length can use. */
int32_t msgl_paged_decode_default_splits(int32_t batch, int32_t num_kv_heads, int32_t max_seq_len);

/*
 * Bytes of workspace msgl_paged_decode needs for these sizes: the plan (work
 * list and per-request key offsets) and, when max_splits > 1, fp32 split-K
 * partials (m, l and the unnormalised output per chunk and query head). Its
 * contents need no initialisation. Calls that overlap in time must not share a
 * workspace; calls in order on one stream may.
 */
int64_t msgl_paged_decode_workspace_size(int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t max_splits);

/*
 * Paged decode attention, one query token per request.
 * Replaces attention/metal.py:112-131 (paged_decode_attention); the result
 * equals attention/naive.py:50-60 (gather + masked SDPA) within fp tolerance.
 *
 *   q          [B, Hq, D]
 *   kv_indptr  CSR offsets into kv_indices ([B+1]); kv_indptr[B] is the number
 *              of entries kv_indices holds (reads stop there); with seq_lens the
 *              rows' start offsets may come in any order
 *   kv_indices page_size == 1: token slots (attention/metal.py:150);
 *              page_size  > 1: page ids; token t of a request lives at slot
 *              kv_indices[kv_indptr[b] + t / page_size] * page_size + t % page_size
 *   seq_lens   [B] tokens per request, or NULL (then L_b = indptr[b+1]-indptr[b],
 *              page_size must be 1)
 *   scale      softmax scale (attention/base.py:45: head_dim ** -0.5)
 *   max_splits split-K bound (<= 0: msgl_paged_decode_default_splits): the most
 *              partials one request's keys are cut into, whether by per-request
 *              chunks or (long-context batches) by equal key ranges of the
 *              batch's concatenated keys
 *   out        [B, Hq, D]
 *   workspace  >= msgl_paged_decode_workspace_size(B, Hq, Hkv, D, max_splits)
 *              bytes, 256-byte aligned
 * Launches the decode kernel and, when max_splits > 1, the split-K merge.
 * Hq/Hkv 1 to 8, or a multiple of 8 (16 for Qwen3-235B-A22B's 64/4): a larger
 * multiple runs as groups of 8 over Hq/8 virtual kv heads, the Hq/(8 Hkv) of
 * one pool head reading its rows together; head_dim 64/128/256.
 * A request with L_b == 0 gets a zero output row. Memory-safe for any
 * metadata: index entries past kv_indptr[B] are not read and slots outside
 * [0, num_slots) read slot 0 (the result is then unspecified;
 * msgl_validate_metadata reports such metadata as an error).
 */
int msgl_paged_decode(const void* q, const void* k_pool, const void* v_pool, const int32_t* kv_indptr,
                      const int32_t* kv_indices, const int32_t* seq_lens, int32_t batch,
                      int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                      int64_t num_slots, int32_t dtype, float scale, int32_t max_splits, void* out,
                      void* workspace, int64_t workspace_bytes, void* stream);

/*
 * KV store fused into paged decode: msgl_store_kv(k_new, v_new, out_loc, ...)
 * followed by msgl_paged_decode(...), in one decode launch (+ the split-K
 * merge). Replaces the per-layer pair kvcache/pool.py:47-50 +
 * attention/metal.py:112-131 as called at layers.py:109-110.
 *   k_new, v_new  [B, Hkv, D] this step's rows, one new token per request
 *   out_loc       [B] slot of each request's newest token; it must be the slot
 *                 of position L_b - 1 (always the case in decode: the new
 *                 token is the last position, scheduler/scheduler.py:154-157)
 * The pools are written only at out_loc (entries outside [0, num_slots) are
 * skipped). Output and pool contents equal the two-call sequence bit for bit.
 */
int msgl_paged_decode_store(const void* q, const void* k_new, const void* v_new, const int32_t* out_loc,
                            void* k_pool, void* v_pool, const int32_t* kv_indptr, const int32_t* kv_indices,
                            const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                            int32_t head_dim, int32_t page_size, int64_t num_slots, int32_t dtype, float scale,
                            int32_t max_splits, void* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Key-range splits for msgl_prefill_ragged: enough workgroups for the 256-CU
 * device, each query block's keys cut into at most this many chunks of at
 * least 256 keys. max_seq_len (max_i L_i, 0 = unknown) caps the count.
 * No reference counterpart (MLX runs one SDPA per request).
 */
int32_t msgl_prefill_default_splits(int32_t num_reqs, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                    int32_t max_extend_len, int32_t max_seq_len);

/* Bytes of workspace msgl_prefill_ragged needs for bf16/fp16 (fp32 needs
 * none): the work list of (request, query block, chunk, kv head) items, and
 * with max_splits > 1 the fp32 (m, l) and unnormalised O per chunk and query
 * row. 0 for invalid sizes. */
int64_t msgl_prefill_workspace_size(int32_t num_reqs, int32_t num_tokens, int32_t max_extend_len,
                                    int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t max_splits);

/*
 * Plan/run split of the decode calls above, for callers that run many layers
 * over the same indices (one decode step of a model):
 * msgl_paged_decode_plan writes the work list of (request, chunk) items for
 * (kv_indptr, seq_lens, batch, heads, max_splits) into the workspace;
 * msgl_paged_decode_planned / msgl_paged_decode_store_planned take the same
 * arguments as msgl_paged_decode / msgl_paged_decode_store and use that plan
 * instead of building it (one launch fewer per call). The plan must have been
 * built on the same stream, for the same index data, workspace and sizes, and
 * the workspace must not be re-planned before the calls that use it. The plan
 * records the batch, max_splits and kv-head count it was built for; a planned
 * launch whose sizes differ does nothing (no work item is read). No
 * reference counterpart (MLX decodes layer by layer, attention/metal.py:112-131).
 */
int msgl_paged_decode_plan(const int32_t* kv_indptr, const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                           int32_t num_kv_heads, int32_t head_dim, int32_t max_splits, void* workspace,
                           int64_t workspace_bytes, void* stream);
int msgl_paged_decode_planned(const void* q, const void* k_pool, const void* v_pool, const int32_t* kv_indptr,
                              const int32_t* kv_indices, const int32_t* seq_lens, int32_t batch,
                              int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                              int64_t num_slots, int32_t dtype, float scale, int32_t max_splits, void* out,
                              void* workspace, int64_t workspace_bytes, void* stream);
int msgl_paged_decode_store_planned(const void* q, const void* k_new, const void* v_new, const int32_t* out_loc,
                                    void* k_pool, void* v_pool, const int32_t* kv_indptr, const int32_t* kv_indices,
                                    const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                                    int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int64_t num_slots,
                                    int32_t dtype, float scale, int32_t max_splits, void* out, void* workspace,
                                    int64_t workspace_bytes, void* stream);

/*
 * The planned decode family in one entry point, with launch flags:
 * k_new/v_new/out_loc all NULL (msgl_paged_decode_planned) or all set
 * (msgl_paged_decode_store_planned), kv_scale NULL (unquantised pools) or the
 * fp8 pools' scales (the _fp8_ forms). MSGL_DECODE_NO_MERGE launches the
 * decode kernel only: requests in one chunk get their output rows, the others
 * leave split-K partials in the workspace for msgl_paged_decode_merge (the two
 * calls on one stream equal the call without the flag, bit for bit). No
 * reference counterpart; it lets a caller time or schedule the two launches
 * apart.
 */
#define MSGL_DECODE_NO_MERGE 1u
int msgl_paged_decode_planned_ex(const void* q, const void* k_new, const void* v_new, const int32_t* out_loc,
                                 void* k_pool, void* v_pool, float* kv_scale, const int32_t* kv_indptr,
                                 const int32_t* kv_indices, const int32_t* seq_lens, int32_t batch,
                                 int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                 int64_t num_slots, int32_t dtype, float scale, int32_t max_splits, uint32_t flags,
                                 void* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The split-K merge of a planned decode launched with MSGL_DECODE_NO_MERGE:
 * out[b] = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s over the chunks of
 * every request cut into more than one (the combine of the Metal kernel's
 * simdgroup merge, attention/metal.py:75-94). Same indices, sizes, dtype,
 * max_splits and workspace as the decode call, and kv_fp8 = 1 when that call
 * ran over fp8 pools (its split form depends on the kernel it ran); nothing to
 * do when max_splits == 1.
 */
int msgl_paged_decode_merge(const int32_t* kv_indptr, const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                            int32_t num_kv_heads, int32_t head_dim, int32_t dtype, int32_t kv_fp8, int32_t max_splits,
                            void* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Ragged chunked-prefill attention over a paged pool, one launch per batch.
 * Replaces attention/base.py:85-105 (BaseAttnBackend._forward_prefill, a
 * per-request MLX SDPA loop).
 *
 *   q          [T, Hq, D] packed extend tokens; request i owns rows
 *              q_indptr[i] .. q_indptr[i+1]-1 (E_i rows); T = num_tokens =
 *              q_indptr[R]
 *   kv_indptr  offsets into kv_indices ([R+1]; kv_indptr[R] = entries of
 *              kv_indices, where reads stop)
 *   kv_indices slots (page ids when page_size > 1) of request i's full KV:
 *              the cached prefix followed by this step's E_i rows, which the
 *              caller stored with msgl_store_kv first
 *   seq_lens   [R] L_i = P_i + E_i, or NULL (L_i = kv_indptr[i+1]-kv_indptr[i])
 *   max_extend_len  max_i E_i (sizes the grid)
 *   max_seq_len     max_i L_i, or 0 if unknown: with max_splits > 1 the key
 *              chunk length is ceil(max_seq_len / max_splits) (>= 256) for the
 *              whole batch, so only long query blocks are split; with 0 every
 *              block is cut evenly. Only the speed depends on it.
 *   scale      softmax scale, > 0 (attention/base.py:45: head_dim^-0.5)
 *   max_splits chunks per query block's key range, 1..16 (bf16/fp16; fp32
 *              always runs one pass)
 *   workspace  bf16/fp16: msgl_prefill_workspace_size(num_reqs, num_tokens,
 *              max_extend_len, Hq, Hkv, D, max_splits) bytes, 256-byte aligned
 *              (fp32: may be NULL). Consecutive calls on one stream may share it.
 *   out        [T, Hq, D]
 * Query t of request i sees keys j <= P_i + t (MLX's bottom-right causal
 * mask, docs/04-attention.md:35-36); E_i <= L_i is required. Memory-safe for
 * any metadata (q rows outside [0, num_tokens) are neither read nor written,
 * index reads stop at kv_indptr[R]); msgl_validate_metadata checks it.
 */
int msgl_prefill_ragged(const void* q, const void* k_pool, const void* v_pool, const int32_t* q_indptr,
                        const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                        int32_t num_reqs, int32_t num_tokens, int32_t max_extend_len, int32_t max_seq_len,
                        int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                        int64_t num_slots, int32_t dtype, float scale, int32_t max_splits, void* out,
                        void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The ragged prefill in two parts, for callers that run it once per layer over
 * the same batch: msgl_prefill_plan writes the work list (which depends only
 * on q_indptr, kv_indptr / seq_lens and the sizes) into the workspace, then
 * msgl_prefill_ragged_planned (the arguments of msgl_prefill_ragged) runs the
 * attention from it, skipping one launch per layer. Same workspace, sizes,
 * dtype and max_splits in both calls, on one stream; fp32 has no work list
 * (the plan is a no-op). The plan records the sizes it was built for; a
 * planned launch whose sizes differ does nothing.
 */
int msgl_prefill_plan(const int32_t* q_indptr, const int32_t* kv_indptr, const int32_t* seq_lens, int32_t num_reqs,
                      int32_t num_tokens, int32_t max_extend_len, int32_t max_seq_len, int32_t num_qo_heads,
                      int32_t num_kv_heads, int32_t head_dim, int32_t dtype, int32_t max_splits, void* workspace,
                      int64_t workspace_bytes, void* stream);
int msgl_prefill_ragged_planned(const void* q, const void* k_pool, const void* v_pool, const int32_t* q_indptr,
                                const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                                int32_t num_reqs, int32_t num_tokens, int32_t max_extend_len, int32_t max_seq_len,
                                int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                int64_t num_slots, int32_t dtype, float scale, int32_t max_splits, void* out,
                                void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Per-step index construction on the GPU from a device copy of the page table
 * req_to_token [num_rows, row_stride] (token-granular slots, as the
 * scheduler's page_table, engine/engine.py:74). Per request r (device int32
 * arrays of num_reqs): row table_idx[r], tokens [cached_len[r], device_len[r])
 * are this step's. Writes, bit-exact with:
 *   q_indptr [R+1], last_indices [R]   attention/base.py:70-83 (q_offsets, last_indices)
 *   positions, out_loc [T]             scheduler/scheduler.py:154-157
 *   kv_indptr [R+1], kv_indices        attention/metal.py:145-152 (token slots of
 *                                      [0, device_len)); with page_size > 1 page
 *                                      ids of ceil(device_len / page_size) pages
 * T = q_indptr[R] and kv_indptr[R] are left on the device; outputs stop at
 * token_capacity / kv_capacity, and the offsets written (q_indptr, kv_indptr,
 * last_indices) are clamped to those capacities, so a launch that reads them
 * next stays inside the outputs (undersized capacities give truncated, not
 * out-of-bounds, metadata; size them from the host-known lengths).
 * positions, out_loc and last_indices may be NULL. Table entries outside the
 * table read as -1. Two launches.
 */
int msgl_build_step_indices(const int32_t* req_to_token, int64_t num_rows, int64_t row_stride,
                            const int32_t* table_idx, const int32_t* cached_len, const int32_t* device_len,
                            int32_t num_reqs, int32_t page_size, int32_t* q_indptr, int32_t* positions,
                            int32_t* out_loc, int32_t* last_indices, int64_t token_capacity, int32_t* kv_indptr,
                            int32_t* kv_indices, int64_t kv_capacity, void* stream);

/*
 * req_to_token[rows[i], cols[i]] = values[i] for i < n (entries outside the
 * table are skipped): keeps the device copy of the page table in step with the
 * slots the scheduler allocates on the host (scheduler/cache.py:53-72).
 */
int msgl_table_scatter(int32_t* req_to_token, int64_t num_rows, int64_t row_stride, const int32_t* rows,
                       const int32_t* cols, const int32_t* values, int64_t n, void* stream);

/*
 * Rotary position embedding, rotate-half layout (replaces RotaryEmbedding.__call__,
 * layers.py:45-56: mx.fast.rope(x[T,H,1,D], rotary_dim, traditional=False,
 * offset=positions)). For pair i < rotary_dim/2 of token t the angle is the
 * fp32 product positions[t] * inv_freq[i]; element i pairs with i + rotary_dim/2,
 * elements >= rotary_dim are copied. inv_freq ([rotary_dim/2] fp32, device)
 * holds the angular frequencies with any scaling folded in: default
 * base^(-2i/rotary_dim), linear (layers.py:37-38) times 1/factor, llama3 the
 * reciprocal of _llama3_freqs (layers.py:59-74).
 *   x, out     [T, H, D]; out may equal x (in place)
 *   rotary_dim multiple of 8, <= min(D, 256); D multiple of 4, <= 1024
 */
int msgl_rope(const void* x, void* out, const int32_t* positions, const float* inv_freq, int64_t num_tokens,
              int32_t num_heads, int32_t head_dim, int32_t rotary_dim, int32_t dtype, void* stream);

/*
 * layers.py:107-109 in one launch: q_out = rope(q), k_pool[out_loc[t]] = rope(k[t]),
 * v_pool[out_loc[t]] = v[t] (kvcache/pool.py:47-50), and k_out = rope(k) when
 * k_out is not null. q_out may equal q and k_out may equal k. num_qo_heads may
 * be 0 (q, q_out unused). Rows whose slot lies outside [0, num_slots) are not
 * stored.
 */
int msgl_rope_store_kv(const void* q, const void* k, const void* v, const int32_t* positions,
                       const int32_t* out_loc, const float* inv_freq, void* q_out, void* k_out, void* k_pool,
                       void* v_pool, int64_t num_tokens, int32_t num_qo_heads, int32_t num_kv_heads,
                       int32_t head_dim, int32_t rotary_dim, int64_t num_slots, int32_t dtype, void* stream);

/*
 * fp8 KV cache (docs/09-exercises.md:81-82: the pool stored as fp8 with one
 * scale per token and head, store_kv and paged decode changed accordingly).
 * Pools hold OCP fp8 e4m3 codes [num_slots, Hkv, D] (1 byte each) plus fp32
 * scales kv_scale [num_slots, Hkv, 2] = (K scale, V scale) of each slot and kv
 * head (adjacent, so decode reads both with one load); a stored element is
 * x ~ e4m3(code) * scale.
 *
 * msgl_store_kv_fp8 replaces kvcache/pool.py:47-50 for such a pool: for each
 * (token, kv head) row, amax = max |x|, codes = e4m3(x * (448 / amax)) rounded
 * to nearest even, scale = amax / 448 (all-zero rows: codes 0, scale 0); rows
 * whose slot is outside [0, num_slots) are skipped. k, v: [T, Hkv, D] of
 * `dtype` (16-byte aligned); D / (16 / sizeof(dtype)) must be a power of two <= 64.
 */
int msgl_store_kv_fp8(const void* k, const void* v, const int32_t* out_loc, void* k_pool, void* v_pool,
                      float* kv_scale, int64_t num_tokens, int32_t num_kv_heads, int32_t head_dim, int64_t num_slots,
                      int32_t dtype, void* stream);

/*
 * msgl_paged_decode over fp8 pools (attention/metal.py:112-131 semantics over
 * the dequantised pool): scores use e4m3(code) on the matrix core with the
 * row's K scale applied to the score, the V scale folds into the softmax
 * weight. q/out dtype bf16 or fp16; Hq/Hkv 1 to 8 or a multiple of 8 (as
 * msgl_paged_decode); head_dim 64/128/256.
 * Same workspace (msgl_paged_decode_workspace_size) and plan
 * (msgl_paged_decode_plan) as the unquantised decode; the _planned form skips
 * the plan like msgl_paged_decode_planned. The new token is stored first with
 * msgl_store_kv_fp8, or by the _store_fp8 forms below.
 */
int msgl_paged_decode_fp8(const void* q, const void* k_pool, const void* v_pool, const float* kv_scale,
                          const int32_t* kv_indptr, const int32_t* kv_indices,
                          const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                          int32_t head_dim, int32_t page_size, int64_t num_slots, int32_t dtype, float scale,
                          int32_t max_splits, void* out, void* workspace, int64_t workspace_bytes, void* stream);
int msgl_paged_decode_fp8_planned(const void* q, const void* k_pool, const void* v_pool, const float* kv_scale,
                                  const int32_t* kv_indptr, const int32_t* kv_indices,
                                  const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                                  int32_t head_dim, int32_t page_size, int64_t num_slots, int32_t dtype, float scale,
                                  int32_t max_splits, void* out, void* workspace, int64_t workspace_bytes,
                                  void* stream);

/*
 * msgl_store_kv_fp8(k_new, v_new, out_loc, ...) followed by
 * msgl_paged_decode_fp8(...) in one decode launch (kvcache/pool.py:47-50 +
 * attention/metal.py:112-131 over fp8 pools): the unit that holds request b's
 * last position quantises its kv head's new K and V rows (k_new/v_new
 * [B, Hkv, D] of q's dtype, 16-byte aligned) with the store's arithmetic, writes
 * codes and scales at out_loc[b], then reads them back like every other token;
 * pools and kv_scale end up bit-identical to the two-call sequence. _planned as
 * msgl_paged_decode_fp8_planned.
 */
int msgl_paged_decode_store_fp8(const void* q, const void* k_new, const void* v_new, const int32_t* out_loc,
                                void* k_pool, void* v_pool, float* kv_scale, const int32_t* kv_indptr,
                                const int32_t* kv_indices, const int32_t* seq_lens, int32_t batch,
                                int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                int64_t num_slots, int32_t dtype, float scale, int32_t max_splits, void* out,
                                void* workspace, int64_t workspace_bytes, void* stream);
int msgl_paged_decode_store_fp8_planned(const void* q, const void* k_new, const void* v_new, const int32_t* out_loc,
                                        void* k_pool, void* v_pool, float* kv_scale, const int32_t* kv_indptr,
                                        const int32_t* kv_indices, const int32_t* seq_lens, int32_t batch,
                                        int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                        int32_t page_size, int64_t num_slots, int32_t dtype, float scale,
                                        int32_t max_splits, void* out, void* workspace, int64_t workspace_bytes,
                                        void* stream);

/*
 * msgl_prefill_ragged over fp8 pools (the same kv_scale [num_slots, Hkv, 2]
 * layout): K tiles are widened to the query type for the matrix core and each
 * key's K scale multiplies its score, V rows are read transposed as bytes and
 * widened, and each key's V scale folds into its softmax weight. q/out bf16 or
 * fp16; the workspace, default splits and msgl_prefill_plan are those of the
 * unquantised prefill.
 */
int msgl_prefill_ragged_fp8(const void* q, const void* k_pool, const void* v_pool, const float* kv_scale,
                            const int32_t* q_indptr, const int32_t* kv_indptr, const int32_t* kv_indices,
                            const int32_t* seq_lens, int32_t num_reqs, int32_t num_tokens, int32_t max_extend_len,
                            int32_t max_seq_len, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                            int32_t page_size, int64_t num_slots, int32_t dtype, float scale, int32_t max_splits,
                            void* out, void* workspace, int64_t workspace_bytes, void* stream);
int msgl_prefill_ragged_fp8_planned(const void* q, const void* k_pool, const void* v_pool, const float* kv_scale,
                                    const int32_t* q_indptr, const int32_t* kv_indptr, const int32_t* kv_indices,
                                    const int32_t* seq_lens, int32_t num_reqs, int32_t num_tokens,
                                    int32_t max_extend_len, int32_t max_seq_len, int32_t num_qo_heads,
                                    int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int64_t num_slots,
                                    int32_t dtype, float scale, int32_t max_splits, void* out, void* workspace,
                                    int64_t workspace_bytes, void* stream);

/*
 * Mixed step in one launch: the paged decode of num_decode requests (one new
 * token each; with k_new/v_new/out_loc the new token's KV store fused in, as in
 * msgl_paged_decode_store) and the ragged prefill of num_prefill chunks, run
 * by one grid whose workgroups take decode and prefill work items in
 * proportion, then one merge launch for both split-K parts. The reference
 * dispatches a whole batch to one phase (attention/base.py:49-60); per request
 * the results are bit-identical to msgl_paged_decode_store_planned /
 * msgl_prefill_ragged_planned with the same arguments, whose work lists
 * msgl_paged_decode_plan (into dec_workspace) and msgl_prefill_plan (into
 * pf_workspace) must have built for these indices and sizes. Both parts share
 * the pools, head counts, head_dim, page size, dtype and scale; q_dec/out_dec
 * are [num_decode, Hq, D], q_pf/out_pf the packed [num_tokens, Hq, D] the
 * prefill's q_indptr indexes (they may be views of one packed batch). The one
 * launch is built for bf16/fp16, head_dim 64 and 128 and Hq/Hkv 1 to 8; other
 * shapes, and batches with no request of one phase, run the two planned calls
 * in turn on the stream (the same results).
 */
int msgl_mixed_attention(const void* q_dec, const void* k_new, const void* v_new, const int32_t* out_loc,
                         const int32_t* dec_kv_indptr, const int32_t* dec_kv_indices, const int32_t* dec_seq_lens,
                         int32_t num_decode, int32_t dec_max_splits, void* out_dec, void* dec_workspace,
                         int64_t dec_workspace_bytes, const void* q_pf, const int32_t* q_indptr,
                         const int32_t* pf_kv_indptr, const int32_t* pf_kv_indices, const int32_t* pf_seq_lens,
                         int32_t num_prefill, int32_t num_tokens, int32_t max_extend_len, int32_t max_seq_len,
                         int32_t pf_max_splits, void* out_pf, void* pf_workspace, int64_t pf_workspace_bytes,
                         void* k_pool, void* v_pool, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                         int32_t page_size, int64_t num_slots, int32_t dtype, float scale, void* stream);

/*
 * msgl_paged_decode_store without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * The work list and split-K partials live in a device array the library holds
 * on each device it runs on (MSGL_NOALLOC_WORKSPACE_BYTES, from the first call
 * on that device until the process ends); sizes whose workspace
 * (msgl_paged_decode_workspace_size) exceeds it are rejected with
 * MSGL_ERR_WORKSPACE. The call allocates nothing. Every call on one device
 * shares that array: calls that overlap in time on a device (other streams or
 * threads) race; calls in order on one stream do not. Same arguments, results
 * and pool contents as msgl_paged_decode_store.
 */
#define MSGL_NOALLOC_WORKSPACE_BYTES ((int64_t)32 << 20)
int msgl_paged_decode_store_noalloc(const void* q, const void* k_new, const void* v_new, const int32_t* out_loc,
                                    void* k_pool, void* v_pool, const int32_t* kv_indptr, const int32_t* kv_indices,
                                    const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                                    int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int64_t num_slots,
                                    int32_t dtype, float scale, int32_t max_splits, void* out, void* stream);

/*
 * Instrumentation: the calling thread's next main-kernel launch -- the decode
 * kernel of a decode call, the merge of msgl_paged_decode_merge, the attention
 * kernel of a prefill call or the mixed-step kernel -- records start_event and
 * stop_event (hipEvent_t, created by the caller) at its own dispatch start and
 * end (hipExtLaunchKernel), so hipEventElapsedTime gives that kernel's
 * duration without the queue barrier an event record before the call adds.
 * One launch consumes them; NULL, NULL disarms. No reference counterpart.
 */
int msgl_profile_next_launch(void* start_event, void* stop_event);

/*
 * Opt-in check of the index metadata of a decode (q_indptr NULL) or prefill
 * call, on the device, before the attention launches read it. Counterpart of
 * the reference's host-side preconditions (attention/metal.py:122) for indices
 * that never reach the host. Walks exactly the entries the attention kernels
 * read (request r: kv_indices[kv_indptr[r] .. + L_r, or ceil(L_r / page_size)
 * page ids]) and never reads past num_indices entries of kv_indices or the
 * [R+1] offsets; page_size > 1 needs seq_lens, as the attention calls do
 * (MSGL_ERR_INVALID otherwise). status: int64[3] device words, cleared by the call, then
 * {msgl_meta_error code, request or entry index, offending value} of one
 * violation found (0 = none). Two launches; the caller reads status after
 * synchronising.
 */
int msgl_validate_metadata(const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                           const int32_t* q_indptr, int32_t num_reqs, int32_t page_size, int64_t num_indices,
                           int64_t num_slots, int32_t num_tokens, int64_t* status, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MSGL_ATTN_H_ */
