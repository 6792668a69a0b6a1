// Device side of the paged decode (paged_decode.hip): parameters, the decode
// and split-K merge bodies, shared with the single-launch mixed step
// (mixed.hip). The design notes are at the top of paged_decode.hip.
#pragma once
#include <type_traits>

#include "msgl_common.h"

namespace msgl {
namespace dec {

#ifndef MSGL_DECODE_MIN_CHUNK
#define MSGL_DECODE_MIN_CHUNK 64
#endif
constexpr int kMinChunk = MSGL_DECODE_MIN_CHUNK;  // smallest split-K chunk (tokens)
constexpr int kMaxSplits = 64;  // bound on splits per request
constexpr int kSeg = 512;       // token slots staged in LDS at a time
constexpr int kSlotPad = 16 * 7;  // room for up to 7 padding tiles of prefetch
constexpr float kLog2e = 1.4426950408889634f;

// ---- per-dtype matrix-core step for S = Q K^T over one 16-byte chunk ------
template <typename T>
struct QK;

template <>
struct QK<bf16_t> {
  static constexpr int VEC = 8;  // elements per 16-byte lane chunk
  __device__ __forceinline__ static f32x4 step(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
};

template <>
struct QK<f16_t> {
  static constexpr int VEC = 8;
  __device__ __forceinline__ static f32x4 step(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
};

template <>
struct QK<float> {
  static constexpr int VEC = 4;
  __device__ __forceinline__ static f32x4 step(const u32x4& a, const u32x4& b, f32x4 c) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[e]), __uint_as_float(b[e]), c, 0, 0, 0);
    return c;
  }
};

// fp8 K elements -> the 16-bit MFMA B operand of the query's type. Every e4m3
// value is exactly representable in bf16 and fp16, so the products on the
// matrix core are those of the dequantised row up to its per-row scale.
template <typename T>
__device__ __forceinline__ u32x4 fp8x8_to(uint32_t w0, uint32_t w1);
template <>
__device__ __forceinline__ u32x4 fp8x8_to<bf16_t>(uint32_t w0, uint32_t w1) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return u32x4{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true))};
}
template <>
__device__ __forceinline__ u32x4 fp8x8_to<f16_t>(uint32_t w0, uint32_t w1) {
  return u32x4{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true))};
}

// Split geometry of one request: chunks of the batch-wide length chunk_len
// (the plan kernel's ceil(max_b L_b / max_splits), a multiple of 16 tokens),
// at most max_splits of them, the last one taking the rest. Used identically
// by the plan, decode and merge kernels.
__device__ __forceinline__ void split_geometry(int L, int max_splits, int chunk_len, int& n, int& chunk) {
  if (L <= 0) {
    n = 0;
    chunk = 0;
    return;
  }
  chunk = chunk_len;
  n = min(max_splits, (L + chunk - 1) / chunk);
}

// Pool slot of token `tok` of the request whose indices start at kv_indices[start].
// Memory-safe for any metadata: an index entry outside [0, nidx) (nidx =
// kv_indptr[B], the entries kv_indices holds) is not read, and a slot outside
// [0, num_slots) is replaced by slot 0 (the result is then unspecified; the
// metadata validation reports both).
__device__ __forceinline__ int slot_of(const int32_t* __restrict__ kv_indices, int64_t nidx, int start, int tok,
                                       int page_size, int64_t num_slots) {
  const int64_t i = (int64_t)start + (page_size == 1 ? tok : tok / page_size);
  if (i < 0 || i >= nidx) return 0;
  const int64_t s = page_size == 1 ? (int64_t)kv_indices[i] : (int64_t)kv_indices[i] * page_size + tok % page_size;
  return (s >= 0 && s < num_slots) ? (int)s : 0;
}

// Balanced split: the length of one key range of the batch's concatenated
// token stream (requests in order, ttot keys in all) when nranges ranges cover
// it: ceil(ttot / nranges), but at least ceil(max_len / (max_splits - 1)) so no
// request overlaps more than max_splits ranges (the partials the workspace
// holds per request) and at least kMinChunk keys. Used identically by the
// decode and merge kernels.
__device__ __forceinline__ int64_t balanced_range(int64_t ttot, int max_len, int nranges, int max_splits) {
  int64_t r = (ttot + nranges - 1) / nranges;
  r = max(r, ((int64_t)max_len + max_splits - 2) / (max_splits - 1));
  return max(r, (int64_t)kMinChunk);
}

// 0: no key-range form; split per request in chunks of one batch-wide length.
#ifndef MSGL_DECODE_BALANCED
#define MSGL_DECODE_BALANCED 1
#endif

// A balanced launch is used when the ranges average at least this many keys:
// shorter ranges measured slower on MI355X than per-request chunks (each chunk
// pays its slot staging, fold and partial store, and the merge reads more
// partials), longer ones faster (ragged long contexts leave no tail).
#ifndef MSGL_DECODE_BALANCED_MIN_RANGE
#define MSGL_DECODE_BALANCED_MIN_RANGE 2048
#endif

struct DecodeParams {
  const void* q;
  const void* k_pool;
  const void* v_pool;
  const float* kv_scale;  // fp8 pools: [num_slots, Hkv, 2] (K, V) scales per slot and kv head
  float* kv_scale_w;      // the same, written by the fused store of an fp8 decode
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* seq_lens;
  void* out;
  float* part_ml;     // [B, S, Hq, 2]
  float* part_o;      // [B, S, Hq, D]
  // fused KV store (all null for plain decode): this step's rows [B, Hkv, D]
  const void* k_new;
  const void* v_new;
  const int32_t* out_loc;  // [B] slot of each request's newest token (position L_b - 1)
  void* k_pool_w;
  void* v_pool_w;
  // work list (plan kernel output, in the workspace)
  int* meta;        // [0] items in the plan, [1] batch-wide chunk length, [2] the plan's max_splits
                    // (with key offsets), [3] max_b L_b, [4..6] the batch, max_splits and kv-head
                    // groups the plan was built for
  int4* plan;       // (request, split, kv-head group, 0), longest first
  int64_t* tok_off; // balanced split: [B+1] tokens of the requests before b (tok_off[B] = all)
  int nranges;      // balanced split: key ranges of the launch (grid / ngrp)
  int64_t num_slots;
  int hq, hkv, page_size, max_splits, batch, ngrp;
  // Some query-head groups run over hkv = hkv_pool * kv_rep virtual kv heads
  // (G above 8 as groups of 8; G 8 over one or two pool heads as groups of 4):
  // virtual head v holds query heads [v G, v G + G) and reads pool head
  // v / kv_rep. The pools, k_new, v_new and kv_scale have hkv_pool heads.
  int hkv_pool, kv_rep;
  bool planned;   // the workspace already holds this call's plan
  bool balanced;  // equal key ranges of the batch's token stream allowed (else per-request chunks)
  bool shared_head;  // max_splits == 1: one (request, kv head) per 4-wavefront workgroup, tiles split over the waves
  int hpg;           // kv heads per work-list group (the list's items are (request, group))
  bool skip_merge;  // host side: launch the decode kernel only (msgl_paged_decode_merge follows)
  float scale_log2;
};

// The work list in the workspace was built for this call's batch, split bound
// and kv-head groups (the plan kernel stamps them into meta[4..6]). A launch
// over a plan of other sizes does nothing: its items would index other
// requests and workspace regions.
__device__ __forceinline__ bool plan_matches(const DecodeParams& p) {
  return p.meta[4] == p.batch && p.meta[5] == p.max_splits && p.meta[6] == p.ngrp && p.meta[1] >= 16;
}

// Whether this launch splits by equal key ranges: allowed, the plan wrote key
// offsets for this max_splits, and the batch's keys (tok_off[B]) average at
// least MSGL_DECODE_BALANCED_MIN_RANGE per range. Used identically by the
// decode and merge kernels; otherwise both follow the per-request work list.
__device__ __forceinline__ bool balanced_launch(const DecodeParams& p) {
  return p.balanced && plan_matches(p) && p.meta[2] == p.max_splits &&
         p.tok_off[p.batch] >= (int64_t)MSGL_DECODE_BALANCED_MIN_RANGE * p.nranges;
}

// Lazy online softmax: a row's reference maximum moves only when a tile's
// maximum exceeds it by more than 2^kLazyLog2, so most tiles skip the rescale
// of the G x (16 / sizeof T) accumulators.
constexpr float kLazyLog2 = 8.f;

// LDS per wavefront: P tile [16 tokens][16 rows] + alpha[16] + (m, l)[16 rows].
constexpr int kLdsPerWave = 16 * 16 + 16 + 32;

// One 16-token tile of K and V rows as loaded: both in row layout (LPR
// consecutive lanes read one whole row, R rows per instruction). KV is the
// pool's storage type; an fp8 tile also carries the scales of the token this
// lane's MFMA column holds.
template <typename KV, int D>
struct TileBuf {
  static constexpr int VEC = 16 / (int)sizeof(KV);
  static constexpr int NL = 16 / (64 / (D / VEC));
  u32x4 k[NL];
  u32x4 v[NL];
  float ks, vs;
};

// Per-wave LDS K tile: 16 rows of D elements, row stride padded by 16 bytes so
// row-wise writes and 16-row column reads are both free of bank conflicts.
template <typename KV, int D>
constexpr int k_lds_stride() { return D * (int)sizeof(KV) + 16; }

// Dynamic LDS floats of a decode workgroup of nwaves wavefronts: the staged
// slots, then per wave the P/alpha/(m, l) tiles and the K re-layout tile, then
// (fp8 pools) the staged tokens' (K, V) scales of the workgroup's kv heads.
template <typename KV, int D>
__host__ __device__ constexpr int decode_lds_floats(int nwaves) {
  return kSeg + kSlotPad + nwaves * (kLdsPerWave + 16 * k_lds_stride<KV, D>() / 4) +
         (std::is_same<KV, fp8e4m3>::value ? (kSeg + kSlotPad) * nwaves * 2 : 0);
}

// Minimum wavefronts per SIMD the register allocator must allow (occupancy).
#ifndef MSGL_DECODE_MIN_WAVES
#define MSGL_DECODE_MIN_WAVES 2
#endif
// Tiles of K/V held in registers per wavefront (1 computing + NST-1 in flight).
#ifndef MSGL_DECODE_STAGES
#define MSGL_DECODE_STAGES 2
#endif
#ifndef MSGL_DECODE_FP8_STAGES
#define MSGL_DECODE_FP8_STAGES 2
#endif

// Tiles of K/V each wavefront holds in registers (its register budget; fp8
// tiles are half the bytes, so they keep more in flight).
template <typename T, typename KV, int D, int G>
constexpr int decode_stages() {
  return std::is_same<KV, fp8e4m3>::value ? (G <= 2 && D <= 128 ? MSGL_DECODE_FP8_STAGES : 2)
                                          : ((sizeof(T) == 4 || D > 128 || G > 4) ? 2 : MSGL_DECODE_STAGES);
}

// The shared-head form (max_splits == 1): the 4 wavefronts of a workgroup take
// every 4th tile of one (request, kv head) and combine their partial softmax
// states in LDS, so the output is written by the one launch (no split-K
// partials, no merge launch). Built where its strided prefetch fits the slot
// padding (two register stages).
constexpr int kSharedWaves = 4;
template <typename T, typename KV, int D, int G>
constexpr bool decode_shared() {
  return (decode_stages<T, KV, D, G>() - 1) * kSharedWaves * 16 <= kSlotPad &&
         (decode_lds_floats<KV, D>(kSharedWaves) + kSharedWaves * (G * D + 2 * G)) * 4 <= 65536;
}

// Workgroup order of a launch whose items are ngrp consecutive kv-head groups
// (n workgroups, a multiple of ngrp): the command processor hands workgroups
// to the 8 XCDs of MI355X round-robin, so item i's groups are given ids that
// differ by 8 inside a block of 8*ngrp workgroups (the last block: its m
// items' groups m apart) and run on one XCD at about the same time. Over fp8
// pools a token's 128-byte scale line (all kv heads of the slot) is then
// fetched from HBM once and hit in that XCD's L2 by the other groups.
#ifndef MSGL_DECODE_FP8_XCD_GROUPS
#define MSGL_DECODE_FP8_XCD_GROUPS 1
#endif
__device__ __forceinline__ int xcd_group_order(int wg, int n, int ngrp) {
  const int blk = 8 * ngrp;
  const int kb = wg / blk, j = wg - kb * blk;
  const int m = max(1, min(8, (n - kb * blk) / ngrp));  // items in this block
  return (kb * 8 + j % m) * ngrp + j / m;
}

// T: the query/output type; KV: the pool's storage type (T itself, or fp8e4m3
// for a quantised pool with per-(slot, kv head) scales). RANGES: the key-range
// form is built in (its chunk loop costs registers; without it every
// workgroup runs one work-list item and p.balanced must be false). SHARED:
// the shared-head form only (its own kernel, so the split forms keep their
// register allocation).
template <typename T, typename KV, int D, int G, bool RANGES, bool SHARED_FORM = false>
__device__ __forceinline__ void paged_decode_body(const DecodeParams& p, int wg) {
  constexpr bool Q8 = std::is_same<KV, fp8e4m3>::value;
  constexpr int VEC = QK<T>::VEC;   // query elements per 16-byte chunk (MFMA operand)
  constexpr int ES = sizeof(T);
  constexpr int VKV = 16 / (int)sizeof(KV);  // pool elements per 16-byte chunk
  constexpr int EKV = sizeof(KV);
  constexpr int KCHUNK = 4 * VEC;   // d covered by one MFMA step across the 4 row groups
  constexpr int NLK = D / KCHUNK;   // MFMA steps per 16-token tile
  constexpr int LPR = D / VKV;      // lanes per K/V row
  constexpr int R = 64 / LPR;       // K/V rows per wave load
  constexpr int NLV = 16 / R;       // K/V loads per lane per tile
  constexpr int NR = G < 4 ? G : 4; // MFMA accumulator rows holding query heads
  constexpr int NST = decode_stages<T, KV, D, G>();
  static_assert(NST >= 2 && (NST - 1) * 16 <= kSlotPad, "pipeline depth");
  static_assert(D % KCHUNK == 0 && 64 % LPR == 0 && 16 % R == 0, "unsupported head_dim");
  static_assert(G >= 1 && G <= 16, "unsupported group size");
  static_assert(!Q8 || (sizeof(T) == 2 && G <= 8), "fp8 pools take 16-bit queries and groups up to 8");

  extern __shared__ float lds_all[];
  int* slots_lds = reinterpret_cast<int*>(lds_all);  // [kSeg + kSlotPad]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  constexpr int KRS = k_lds_stride<KV, D>();
  float* lds = lds_all + kSeg + kSlotPad + wave * (kLdsPerWave + 16 * KRS / 4);
  // fp8 pools, split form: [staged token][workgroup head][K, V] scales
  float* scale_lds = lds_all + kSeg + kSlotPad + nwaves * (kLdsPerWave + 16 * KRS / 4);
  float* P_lds = lds;              // [16][16]
  float* A_lds = lds + 256;        // [16]
  float* ML_lds = lds + 256 + 16;  // [16][2]
  uint8_t* K_lds = reinterpret_cast<uint8_t*>(lds + kLdsPerWave);  // [16][KRS bytes]

  const int64_t row_stride = (int64_t)p.hkv_pool * D * EKV;  // bytes per slot
  const int64_t nidx = p.kv_indptr[p.batch];             // entries of kv_indices

  // One chunk: keys [t0, t1) of request b (L keys, kv_indices from start),
  // partial `split` of its n; the kv-head group kgrp is this workgroup's waves.
  // Shared-head form (SHARED): kgrp is the one kv head of every wave, wave w
  // takes tiles w, w + 4, ... of each segment, and the waves' partial states
  // are combined in LDS into the output rows.
  auto run_chunk = [&](const int b, const int start, const int L, const int t0, const int t1, const int split,
                       const int n, const int kgrp, auto shared_t) {
  constexpr bool SHARED = decltype(shared_t)::value;
  constexpr int TS = SHARED ? kSharedWaves : 1;  // tile stride of one wavefront
  static_assert(!SHARED || (NST - 1) * TS * 16 <= kSlotPad, "strided prefetch past the slot padding");
  {
    // lane-derived indices are recomputed per chunk from an opaque copy of
    // the lane id: hoisted out of the chunk loop they would hold registers
    // through the whole tile loop
    int lid = lane;
    if constexpr (RANGES) asm volatile("" : "+v"(lid));
    const int r = lid & 15;    // MFMA column (token in tile) / A row
    const int g4 = lid >> 4;   // MFMA row group
    const int vc = lid % LPR;  // V: 16-byte chunk within the row
    const int vr = lid / LPR;  // V: token sub-row
    const int kvh = SHARED ? kgrp : kgrp * nwaves + wave;
    const int tile0 = SHARED ? wave : 0;  // this wavefront's first tile of a segment
    const bool active = kvh < p.hkv;
    const int kvh_c = active ? kvh : 0;

    // Q fragment: A operand, row r = query head kvh*G + r (zero when r >= G).
    u32x4 qa[NLK];
    {
      const uint8_t* qrow =
          reinterpret_cast<const uint8_t*>(p.q) + ((int64_t)b * p.hq + kvh_c * G + r) * D * ES + g4 * VEC * ES;
#pragma unroll
      for (int j = 0; j < NLK; ++j) {
        qa[j] = (r < G) ? ld16(qrow + j * KCHUNK * ES) : u32x4{0u, 0u, 0u, 0u};
      }
    }
    float m_run[NR], l_run[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      m_run[i] = -INFINITY;
      l_run[i] = 0.f;
    }
    float acc[G][VKV];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < VKV; ++e) acc[g][e] = 0.f;

    const int ph = kvh_c / p.kv_rep;  // the pool head this (virtual) kv head reads
    const uint8_t* kbase_p = reinterpret_cast<const uint8_t*>(p.k_pool) + (int64_t)ph * D * EKV + vc * 16;
    const uint8_t* vbase_p = reinterpret_cast<const uint8_t*>(p.v_pool) + (int64_t)ph * D * EKV + vc * 16;

    // Fused KV store (unquantised pools): the chunk holding position L-1 (the
    // new token) writes its rows to the pool and reads them from k_new/v_new
    // instead -- no other unit reads that slot, so the write needs no ordering
    // inside the launch.
    const bool fused = !Q8 && p.k_new != nullptr;
    const int new_pos = fused && t1 == L ? L - 1 : 0x7fffffff;  // absolute position, or never
    const int64_t new_off = ((int64_t)b * p.hkv_pool + ph) * D * ES + vc * VEC * ES;
    const uint8_t* knew_p = fused ? reinterpret_cast<const uint8_t*>(p.k_new) + new_off : nullptr;
    const uint8_t* vnew_p = fused ? reinterpret_cast<const uint8_t*>(p.v_new) + new_off : nullptr;
    // (one virtual head of each pool head writes the row)
    if (active && kvh_c % p.kv_rep == 0 && new_pos != 0x7fffffff && lane < LPR && (!SHARED || wave == 0)) {
      const int64_t slot = p.out_loc[b];
      if (slot >= 0 && slot < p.num_slots) {
        const int64_t dst = slot * row_stride + (int64_t)ph * D * ES + vc * VEC * ES;
        st16(reinterpret_cast<uint8_t*>(p.k_pool_w) + dst, ld16(knew_p));
        st16(reinterpret_cast<uint8_t*>(p.v_pool_w) + dst, ld16(vnew_p));
      }
    }
    // Fused store over fp8 pools: the chunk holding the new token quantises its
    // K and V rows exactly like msgl_store_kv_fp8 (lanes [0, LQ) the K row,
    // [LQ, 2 LQ) the V row, one 16-byte chunk of T each) and writes codes and
    // scales before any load of the chunk is issued; the loop then reads the
    // new token from the pool like every other token. Every virtual head of a
    // pool head writes the same bytes, and each reads back only after its own
    // writes have landed, so none reads a slot half written.
    if constexpr (Q8) {
      if (active && p.k_new != nullptr && t1 == L) {
        constexpr int LQ = D / VEC;  // lanes per input row
        static_assert(2 * LQ <= 64, "a wavefront quantises the K and V rows together");
        const int sub = lane % LQ;
        const bool is_v = (lane / LQ) & 1;  // lanes >= 2 LQ repeat the rows and write nothing
        const uint8_t* src = reinterpret_cast<const uint8_t*>(is_v ? p.v_new : p.k_new) +
                             (((int64_t)b * p.hkv_pool + ph) * D + sub * VEC) * ES;
        uint32_t w[VEC / 4];
        const float amax = fp8_quantize_chunk<T>(ld16(src), LQ, w);
        const int64_t slot = p.out_loc[b];
        if (lane < 2 * LQ && slot >= 0 && slot < p.num_slots) {
          uint8_t* dst = reinterpret_cast<uint8_t*>(is_v ? p.v_pool_w : p.k_pool_w) +
                         (slot * p.hkv_pool + ph) * D + sub * VEC;
          static_assert(VEC == 8, "16-bit queries: eight codes per lane");
          *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
          if (sub == 0) p.kv_scale_w[(slot * p.hkv_pool + ph) * 2 + (is_v ? 1 : 0)] = amax / 448.f;
        }
        // the stores have completed before this wavefront loads the slot back
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
    }

    for (int s0 = t0; s0 < t1; s0 += kSeg) {
      const int seg_len = min(kSeg, t1 - s0);
      const int ntile = (seg_len + 15) >> 4;
      // ---- stage this segment's slots, padded by NST-1 tiles; positions past
      //      the end repeat the last valid slot ----
      __syncthreads();
      for (int i = threadIdx.x; i < (ntile + (NST - 1) * TS) * 16; i += blockDim.x) {
        const int tok = s0 + min(i, seg_len - 1);
        slots_lds[i] = slot_of(p.kv_indices, nidx, start, tok, p.page_size, p.num_slots);
      }
      __syncthreads();
      // fp8 pools, split form: the (K, V) scales of the workgroup's kv heads for
      // every staged token, one 4-byte LDS DMA per lane -- each token's scale
      // line is requested once per workgroup instead of once per wavefront (the
      // heads of a slot are neighbours, [slot][head][K, V]). The transfers land
      // while the first tiles load; the waves wait for them (and meet at a
      // barrier) just before their first compute of the segment.
      constexpr bool SCL = Q8 && !SHARED;
      if constexpr (SCL) {
        const int nd = 2 * nwaves;  // dwords per token
        const int total = (ntile + NST - 1) * 16 * nd;
        const int h0 = kgrp * nwaves;
        const uint32_t sbase = (uint32_t)(uintptr_t)((MSGL_LDS float*)scale_lds);
        if (nwaves == 4 && (p.hkv & 3) == 0 && p.kv_rep == 1) {
          // four heads, all present: a token's 32 bytes are two aligned 16-byte transfers
          const int total16 = total >> 2;
          for (int c = wave; c * 64 < total16; c += nwaves) {
            const int idx = c * 64 + lane;
            if (idx < total16)
              dma16(p.kv_scale + ((int64_t)slots_lds[idx >> 1] * p.hkv + h0) * 2 + (idx & 1) * 4,
                    __builtin_amdgcn_readfirstlane(sbase + c * 1024));
          }
        } else {
          for (int c = wave; c * 64 < total; c += nwaves) {
            const int idx = c * 64 + lane;
            if (idx < total) {
              const int t = idx / nd, d = idx - t * nd;
              const int h = min(h0 + (d >> 1), p.hkv - 1);  // heads past hkv: an inactive wave's, never read
              dma4(p.kv_scale + ((int64_t)slots_lds[t] * p.hkv_pool + h / p.kv_rep) * 2 + (d & 1),
                   __builtin_amdgcn_readfirstlane(sbase + c * 256));
            }
          }
        }
      }
      if (!active) {
        if constexpr (SCL) {  // this wave's transfers landed; meet the others' first-compute barrier
          vm_wait<0>();
          __syncthreads();
        }
        continue;
      }

      // Prefetches past the segment end read the padded slot list (the last
      // valid slot, one row per tile, already fetched): every path through the
      // loop keeps the same loads in flight, so the compiler waits for exactly
      // one tile instead of draining the pipeline at each branch.
      auto issue = [&](TileBuf<KV, D>& buf, int tile) {
        const int base = tile * 16;
#pragma unroll
        for (int i = 0; i < NLV; ++i) {
          const int pos = base + vr + R * i;
          const int64_t off = (int64_t)slots_lds[pos] * row_stride;
          const bool is_new = s0 + pos >= new_pos;  // the new token and the padding that repeats it
          buf.k[i] = ld16_stream(is_new ? knew_p : kbase_p + off);
          buf.v[i] = ld16_stream(is_new ? vnew_p : vbase_p + off);
        }
        if (Q8 && !SCL) {  // the K and V scales of the token in this lane's MFMA column: one 8-byte load
          const float2 sc = reinterpret_cast<const float2*>(p.kv_scale)[(int64_t)slots_lds[base + r] * p.hkv_pool + ph];
          buf.ks = sc.x;
          buf.vs = sc.y;
        }
      };

      auto compute = [&](const TileBuf<KV, D>& buf, int tile) {
        // K rows -> LDS -> MFMA B layout (lane: token r, d chunk j*KCHUNK + g4*VEC)
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < NLV; ++i) *reinterpret_cast<u32x4*>(K_lds + (vr + R * i) * KRS + vc * 16) = buf.k[i];
        wave_lds_sync();
        // S = Q K^T on the matrix core
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NLK; ++j) {
          if constexpr (Q8) {
            const uint2 k8 = *reinterpret_cast<const uint2*>(K_lds + r * KRS + (j * KCHUNK + g4 * VEC));
            s = QK<T>::step(qa[j], fp8x8_to<T>(k8.x, k8.y), s);
          } else {
            s = QK<T>::step(qa[j], *reinterpret_cast<const u32x4*>(K_lds + r * KRS + (j * KCHUNK + g4 * VEC) * ES),
                            s);
          }
        }
        // online softmax (exp2 domain); a quantised row's scale multiplies its scores
        float ks = buf.ks, vs = buf.vs;
        if constexpr (SCL) {
          const float2 kv = *reinterpret_cast<const float2*>(scale_lds + ((tile * 16 + r) * nwaves + wave) * 2);
          ks = kv.x;
          vs = kv.y;
        }
        const float sc = Q8 ? p.scale_log2 * ks : p.scale_log2;
        const bool valid = tile * 16 + r < seg_len;
        float pr[4] = {0.f, 0.f, 0.f, 0.f}, al[4] = {1.f, 1.f, 1.f, 1.f};
        bool moved = false;  // some row's reference maximum moved (its accumulators need al)
#pragma unroll
        for (int i = 0; i < NR; ++i) {
          const float x = valid ? s[i] * sc : -INFINITY;
          const float mt = row16_max(x);  // finite: key 0 of every tile is valid
          // the reference maximum moves only when the tile's exceeds it by more
          // than 2^kLazyLog2 (a weight stays below 2^kLazyLog2; l and O share the
          // reference, so the result is the same up to rounding)
          const bool mv = mt > m_run[i] + kLazyLog2;
          const float m_new = mv ? mt : m_run[i];
          al[i] = mv ? __builtin_amdgcn_exp2f(m_run[i] - m_new) : 1.f;
          moved |= mv;
          pr[i] = __builtin_amdgcn_exp2f(x - m_new);
          l_run[i] = l_run[i] * al[i] + pr[i];
          m_run[i] = m_new;
        }
        wave_lds_sync();  // previous tile's LDS reads are done
        // P V weights; a quantised V row's scale is folded into its weight (l keeps the plain weights)
        const float vsc = Q8 ? vs : 1.f;
        *reinterpret_cast<f32x4*>(P_lds + r * 16 + 4 * g4) = f32x4{pr[0] * vsc, pr[1] * vsc, pr[2] * vsc, pr[3] * vsc};
        if (r == 0) *reinterpret_cast<f32x4*>(A_lds + 4 * g4) = f32x4{al[0], al[1], al[2], al[3]};
        wave_lds_sync();
        // O = alpha * O + P V on the VALU (alpha only when a row's reference moved)
        if (__builtin_amdgcn_ballot_w64(moved) != 0) {
          float alpha[G];
#pragma unroll
          for (int g = 0; g < G; ++g) alpha[g] = A_lds[g];
#pragma unroll
          for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < VKV; ++e) acc[g][e] *= alpha[g];
        }
#pragma unroll
        for (int i = 0; i < NLV; ++i) {
          const int tl = vr + R * i;
          float vf[VKV];
          Vec16<KV>::to_f32(buf.v[i], vf);
          float pv[G];
#pragma unroll
          for (int g = 0; g < G; ++g) pv[g] = P_lds[tl * 16 + g];
#pragma unroll
          for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < VKV; ++e) acc[g][e] = fmaf(pv[g], vf[e], acc[g][e]);
        }
      };

      // NST-stage register pipeline: this wavefront's next NST-1 tiles are in
      // flight while one computes (tiles tile0, tile0 + TS, ...; past ntile: padding)
      const int nloc = ntile > tile0 ? (ntile - tile0 + TS - 1) / TS : 0;
      TileBuf<KV, D> buf[NST];
#pragma unroll
      for (int i = 0; i < NST - 1; ++i) issue(buf[i], tile0 + i * TS);
      for (int j0 = 0; j0 < nloc; j0 += NST) {
#pragma unroll
        for (int k = 0; k < NST; ++k) {
          const int j = j0 + k;
          if (j >= nloc) break;
          issue(buf[(k + NST - 1) % NST], tile0 + (j + NST - 1) * TS);
          if constexpr (SCL) {
            if (j == 0) {  // the scale transfers, issued before every row load, and tile 0 have landed
              vm_wait<(NST - 1) * 2 * NLV>();
              __syncthreads();
            }
          }
          compute(buf[k], tile0 + j * TS);
        }
      }
    }
    if (!active) return;

    // ---- fold: l over the 16 token lanes, acc over the R token sub-rows ----
#pragma unroll
    for (int i = 0; i < NR; ++i) l_run[i] = row16_sum(l_run[i]);
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1)
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < VKV; ++e) acc[g][e] += __shfl_xor(acc[g][e], off);
    wave_lds_sync();
    if (r == 0) {
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        ML_lds[(4 * g4 + i) * 2 + 0] = m_run[i];
        ML_lds[(4 * g4 + i) * 2 + 1] = l_run[i];
      }
    }
    wave_lds_sync();
    const int d0 = vc * VKV;
    if constexpr (SHARED) {
      // every wave's (acc, m, l) of the G heads into the combine region, then the
      // workgroup folds the four: o = sum_w 2^(m_w - M) acc_w / sum_w 2^(m_w - M) l_w
      constexpr int CW = G * D + 2 * G;  // floats per wave
      float* comb = lds_all + decode_lds_floats<KV, D>(kSharedWaves);
      float* mine = comb + wave * CW;
      if (lane < LPR) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int e = 0; e < VKV; ++e) mine[g * D + d0 + e] = acc[g][e];
      }
      if (lane < G) {
        mine[G * D + 2 * lane] = ML_lds[lane * 2 + 0];
        mine[G * D + 2 * lane + 1] = ML_lds[lane * 2 + 1];
      }
      __syncthreads();
      T* o = reinterpret_cast<T*>(p.out) + ((int64_t)b * p.hq + kvh * G) * D;
      for (int idx = threadIdx.x; idx < G * D; idx += kSharedWaves * 64) {
        const int g = idx / D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kSharedWaves; ++w) M = fmaxf(M, comb[w * CW + G * D + 2 * g]);
        float num = 0.f, den = 0.f;
#pragma unroll
        for (int w = 0; w < kSharedWaves; ++w) {
          const float f = __builtin_amdgcn_exp2f(comb[w * CW + G * D + 2 * g] - M);
          num += f * comb[w * CW + idx];
          den += f * comb[w * CW + G * D + 2 * g + 1];
        }
        o[idx] = from_f32<T>(num / den);
      }
      return;
    }
    if (n == 1) {
      if (lane < LPR) {
        T* o = reinterpret_cast<T*>(p.out) + ((int64_t)b * p.hq + kvh * G) * D + d0;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float inv = 1.f / ML_lds[g * 2 + 1];
#pragma unroll
          for (int c = 0; c < VKV; c += VEC) {
            T tmp[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) tmp[e] = from_f32<T>(acc[g][c + e] * inv);
            u32x4 packed;
            __builtin_memcpy(&packed, tmp, 16);
            st16(o + g * D + c, packed);
          }
        }
      }
      return;
    }

    // ---- split-K: publish this chunk's partials for the merge kernel ----
    const int64_t base = ((int64_t)b * p.max_splits + split) * p.hq + kvh * G;
    if (lane < LPR) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float* po = p.part_o + (base + g) * D + d0;
#pragma unroll
        for (int e = 0; e < VKV; e += 4)
          *reinterpret_cast<f32x4*>(po + e) = f32x4{acc[g][e], acc[g][e + 1], acc[g][e + 2], acc[g][e + 3]};
      }
    }
    if (lane < G) {
      p.part_ml[(base + lane) * 2 + 0] = ML_lds[lane * 2 + 0];
      p.part_ml[(base + lane) * 2 + 1] = ML_lds[lane * 2 + 1];
    }
  }
  };

  // This workgroup's chunks, run one after another through one call site.
  // Balanced: key range k of the batch's token stream (requests concatenated
  // in order), all ranges of one length, for kv-head group kgrp -- every
  // workgroup gets the same number of keys, so the launch ends when the
  // average one does. A range can span request boundaries: each request's part
  // is a chunk of its own, partial (k - the request's first range) of the
  // ranges it overlaps. Otherwise: one work item of the plan (workgroups past
  // its end have nothing to do).
  if constexpr (SHARED_FORM) {
    static_assert(decode_shared<T, KV, D, G>(), "no shared-head form for this instantiation");
    {  // workgroup wg: head wg % hpg of the list's item wg / hpg
      const int item_i = wg / p.hpg;
      if (item_i >= p.meta[0] || !plan_matches(p)) return;
      const int4 item = p.plan[item_i];
      const int b = item.x;
      const int head = item.z * p.hpg + wg % p.hpg;
      if (head >= p.hkv) return;
      const int start = p.kv_indptr[b];
      const int L = p.seq_lens ? p.seq_lens[b] : p.kv_indptr[b + 1] - start;
      if (L <= 0) {  // defined zero output for this head's query rows
        T* o = reinterpret_cast<T*>(p.out) + ((int64_t)b * p.hq + head * G) * D;
        for (int i = threadIdx.x; i < G * D; i += blockDim.x) o[i] = from_f32<T>(0.f);
        return;
      }
      run_chunk(b, start, L, 0, L, 0, 1, head, std::true_type{});
      return;
    }
  }
  const bool bal = RANGES && balanced_launch(p);
  if constexpr (Q8 && MSGL_DECODE_FP8_XCD_GROUPS) {
    // fp8 pools: the kv-head groups of one item on one XCD (see xcd_group_order)
    const int nw = bal ? p.nranges * p.ngrp : p.meta[0];
    if (p.ngrp > 1 && wg < nw) wg = xcd_group_order(wg, nw, p.ngrp);
  }
  int b, kgrp, start = 0, L = 0, t0 = 0, t1 = 0, split = 0, n = 1;
  int64_t k = 0, rl = 1, g0 = 0, g1 = 0;
  if (bal) {
    kgrp = wg % p.ngrp;
    k = wg / p.ngrp;
    const int64_t ttot = p.tok_off[p.batch];
    rl = balanced_range(ttot, p.meta[3], p.nranges, p.max_splits);
    g0 = k * rl;
    g1 = min(ttot, g0 + rl);
    if (g0 >= g1) return;
    // the last request starting at or before key g0 (it holds key g0): a
    // 64-way search, every lane probes one offset per round, so a batch of up
    // to 4096 requests takes two dependent loads
    int lo = 0, hi = p.batch - 1;
    while (lo < hi) {
      const int step = (hi - lo + 64) >> 6;
      const int idx = lo + lane * step;
      const uint64_t ok = __ballot(idx <= hi && p.tok_off[idx] <= g0);  // a prefix of the lanes, lane 0 included
      lo += (63 - __clzll((long long)ok)) * step;
      hi = min(hi, lo + step - 1);
    }
    b = lo;
  } else {
    if (wg >= p.meta[0] || !plan_matches(p)) return;
    const int4 item = p.plan[wg];
    b = item.x;
    split = item.y;
    kgrp = item.z;
    start = p.kv_indptr[b];
    L = p.seq_lens ? p.seq_lens[b] : p.kv_indptr[b + 1] - start;
    int chunk;
    split_geometry(L, p.max_splits, p.meta[1], n, chunk);
    if (split >= n) {
      if (split == 0) {  // L == 0: defined zero output for this group's heads
        const int h0 = kgrp * nwaves * G;
        const int h1 = min(p.hq, h0 + nwaves * G);
        T* o = reinterpret_cast<T*>(p.out) + (int64_t)b * p.hq * D;
        for (int i = h0 * D + threadIdx.x; i < h1 * D; i += blockDim.x) o[i] = from_f32<T>(0.f);
      }
      return;
    }
    t0 = split * chunk;
    t1 = split == n - 1 ? L : t0 + chunk;
  }
  for (;; ++b) {
    if (bal) {
      if (g0 >= g1 || b >= p.batch) return;
      const int64_t ob = p.tok_off[b], ob1 = p.tok_off[b + 1];
      if (ob1 <= g0) continue;  // no key of b in the range (L = 0)
      const int64_t s1 = min(g1, ob1);
      start = p.kv_indptr[b];
      L = (int)(ob1 - ob);
      t0 = (int)(g0 - ob);
      t1 = (int)(s1 - ob);
      split = (int)(k - ob / rl);
      n = (int)((ob1 - 1) / rl - ob / rl + 1);
      g0 = s1;
    }
    run_chunk(b, start, L, t0, t1, split, n, kgrp, std::false_type{});
    if constexpr (!RANGES) return;
    if (!bal) return;
  }
}

// Merge split-K partials, one wavefront per (request, kv head):
//   o = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s
// (the combine of the Metal kernel's simdgroup merge, attention/metal.py:75-94).
// Lanes own float4 chunks of the G*D outputs; the partials of up to 8 splits
// are loaded in one batch (one memory round trip) and combined online.
template <typename T, int D, int G>
__device__ __forceinline__ void paged_decode_merge_body(const DecodeParams& p, int batch, int wg) {
  const int unit = wg * (blockDim.x >> 6) + (threadIdx.x >> 6);  // (b, kvh)
  const int lane = threadIdx.x & 63;
  if (unit >= batch * p.hkv) return;
  const int b = unit / p.hkv, kvh = unit % p.hkv;
  if (!plan_matches(p)) return;
  int n, chunk;
  if (balanced_launch(p)) {  // the ranges request b overlaps; no key: the defined zero output
    const int64_t ob = p.tok_off[b], ob1 = p.tok_off[b + 1];
    if (ob1 == ob) {
      T* o = reinterpret_cast<T*>(p.out) + ((int64_t)b * p.hq + kvh * G) * D;
      for (int i = lane; i < G * D; i += 64) o[i] = from_f32<T>(0.f);
      return;
    }
    const int64_t rl = balanced_range(p.tok_off[p.batch], p.meta[3], p.nranges, p.max_splits);
    n = (int)((ob1 - 1) / rl - ob / rl + 1);
  } else {
    const int L = p.seq_lens ? p.seq_lens[b] : p.kv_indptr[b + 1] - p.kv_indptr[b];
    split_geometry(L, p.max_splits, p.meta[1], n, chunk);
  }
  if (n <= 1) return;
  const int64_t bbase = (int64_t)b * p.max_splits * p.hq + kvh * G;
  constexpr int C4 = D / 4;
  constexpr int NB = 8;  // splits whose partials are loaded in one batch
  T* o = reinterpret_cast<T*>(p.out) + ((int64_t)b * p.hq + kvh * G) * D;
  for (int c = lane; c < G * C4; c += 64) {
    const int g = c / C4, d4 = c % C4;
    const float2* ml = reinterpret_cast<const float2*>(p.part_ml) + bbase + g;
    const float* po = p.part_o + (bbase + g) * D + d4 * 4;
    const int64_t mstride = p.hq;  // float2 units
    const int64_t ostride = (int64_t)p.hq * D;
    float M = -INFINITY, Lsum = 0.f;
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < n; s0 += NB) {
      // issue every load of this batch before using any of them
      float2 mlv[NB];
      f32x4 xv[NB];
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int sp = min(s0 + i, n - 1);
        mlv[i] = ml[sp * mstride];
        xv[i] = *reinterpret_cast<const f32x4*>(po + sp * ostride);
      }
      float Mb = M;
#pragma unroll
      for (int i = 0; i < NB; ++i)
        if (s0 + i < n) Mb = fmaxf(Mb, mlv[i].x);
      const float r = __builtin_amdgcn_exp2f(M - Mb);  // rescale what was combined so far
      Lsum *= r;
      a *= r;
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        if (s0 + i < n) {
          const float f = __builtin_amdgcn_exp2f(mlv[i].x - Mb);
          Lsum += f * mlv[i].y;
          a += f * xv[i];
        }
      }
      M = Mb;
    }
    const float inv = 1.f / Lsum;
    T tmp[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) tmp[e] = from_f32<T>(a[e] * inv);
    T* dst = o + g * D + d4 * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[e] = tmp[e];
  }
}

// Wavefronts per workgroup of the decode kernel (kv heads handled by one
// workgroup); 4 measured faster than 1 or 2 on MI355X.
#ifndef MSGL_DECODE_WAVES_PER_WG
#define MSGL_DECODE_WAVES_PER_WG 4
#endif

// Dynamic LDS bytes of a decode workgroup of nwaves wavefronts, and of a
// shared-head workgroup (plus the region where its waves combine).
template <typename KV, int D>
inline size_t decode_lds_bytes(int nwaves) {
  return (size_t)decode_lds_floats<KV, D>(nwaves) * sizeof(float);
}
template <typename KV, int D, int G>
inline size_t decode_shared_lds_bytes() {
  return ((size_t)decode_lds_floats<KV, D>(kSharedWaves) + (size_t)kSharedWaves * (G * D + 2 * G)) * sizeof(float);
}

// Validates the arguments of a decode call and fills p (workspace regions
// included); empty: batch 0, nothing to launch. (paged_decode.hip)
int decode_params(const char* fn, bool planned, const void* q, const void* k_new, const void* v_new,
                  const int32_t* out_loc, const void* k_pool, const void* v_pool, const float* kv_scale,
                  const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens, int32_t batch,
                  int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int64_t num_slots,
                  int32_t dtype, float scale, int32_t max_splits, void* out, void* workspace, int64_t workspace_bytes,
                  DecodeParams& p, bool& empty);

// Workgroups of the decode launch (p.nranges key ranges x p.ngrp kv-head
// groups when balanced, else one per plan item). (paged_decode.hip)
int64_t decode_items(const DecodeParams& p);

// The work-list launch (paged_decode.hip).
int launch_decode_plan(const DecodeParams& p, hipStream_t stream);

// A request to the instantiation that (query type, pool type, head_dim, query-
// head group) selects: the decode launch (plan unless p->planned, attention,
// merge), the merge launch alone, or a property of the instantiation.
enum DecodeOpKind { kOpLaunch = 0, kOpMerge = 1, kOpShared = 2, kOpResident = 3 };
struct DecodeOp {
  DecodeOpKind kind;
  const DecodeParams* p;  // kOpLaunch, kOpMerge
  int batch;              // kOpLaunch, kOpMerge
  hipStream_t stream;     // kOpLaunch, kOpMerge
  int nwaves;             // kOpResident: wavefronts per workgroup
  int* resident;          // kOpResident: workgroups the device holds at once
  bool* flag;             // kOpShared: the shared-head form is built; kOpResident: the key-range form is built
};

// op applied to the instantiations of one (query, pool) type pair, each pair
// built in a translation unit of its own (inst/decode_*.hip over
// decode_launch.h).
int decode_op_f32(const DecodeOp& op, int head_dim, int group);
int decode_op_bf16(const DecodeOp& op, int head_dim, int group);
int decode_op_f16(const DecodeOp& op, int head_dim, int group);
int decode_op_bf16_fp8(const DecodeOp& op, int head_dim, int group);
int decode_op_f16_fp8(const DecodeOp& op, int head_dim, int group);

}  // namespace dec
}  // namespace msgl
