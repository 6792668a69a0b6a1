// Paged decode attention for gfx950 (one query token per request).
//
// Semantics: attention/naive.py:50-60 (gather by page table + masked SDPA) and
// attention/metal.py:112-131 (paged_decode_attention over CSR indices):
//   o[b, h] = softmax_j(scale * q[b,h] . K[slot_b(j), h/G]) V[slot_b(j), h/G],  j < L_b
//
// Design (MI355X-first, not a translation of the Metal kernel):
//  * Work unit = one wavefront per (request b, split s, kv head). Workgroups
//    are small (one wavefront by default) so a CU refills as soon as any unit
//    finishes; the kv heads of one (b, s) are neighbouring workgroups, so the
//    rows of a slot (Hkv * D contiguous elements) are read close in time. A
//    workgroup gathers its token slots once into LDS.
//  * Split-K: every request is cut into chunks of one batch-wide length,
//    ceil(max_b L_b / max_splits) rounded to 16 tokens (>= kMinChunk), so a
//    workgroup never gathers more than one chunk; a one-workgroup plan kernel
//    lists the (request, chunk, kv-head group) items longest first, so the
//    grid has no empty workgroups and the long items start first. A
//    single-chunk request writes its final row. Otherwise every chunk writes
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
//    only the MFMA rows that hold query heads are processed.
//  * P.V on the VALU: lane (token sub-row, 16-byte d chunk) accumulates
//    G x (16/sizeof T) fp32 outputs; P and the rescale factors go through a
//    small per-wave LDS tile.
//  * The tile loop is software pipelined: the K/V loads of the next NST-1
//    tiles are in flight (a ring of register buffers) while one tile is
//    computed, which is what it takes to keep ~200 KiB of loads in flight per
//    CU at 2 wavefronts per SIMD. K/V rows
//    are read exactly once per launch, so they use nontemporal (streaming)
//    loads, which sustain markedly more HBM bandwidth for random row gathers
//    on MI355X than default-policy loads.
#include <type_traits>

#include "msgl_common.h"

namespace msgl {

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

__device__ __forceinline__ int slot_of(const int32_t* __restrict__ kv_indices, int start, int tok, int page_size,
                                       int64_t num_slots) {
  int64_t s;
  if (page_size == 1) {
    s = kv_indices[start + tok];
  } else {
    s = (int64_t)kv_indices[start + tok / page_size] * page_size + tok % page_size;
  }
  return (s >= 0 && s < num_slots) ? (int)s : 0;
}

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
  int* meta;        // [0] items in the plan, [1] batch-wide chunk length
  int4* plan;       // (request, split, kv-head group, 0), longest first
  int64_t num_slots;
  int hq, hkv, page_size, max_splits, batch, ngrp;
  bool planned;  // the workspace already holds this call's plan
  float scale_log2;
};

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

// T: the query/output type; KV: the pool's storage type (T itself, or fp8e4m3
// for a quantised pool with per-(slot, kv head) scales).
template <typename T, typename KV, int D, int G>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(MSGL_DECODE_MIN_WAVES)))
void paged_decode_kernel(DecodeParams p) {
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
  // register budget; fp8 tiles are half the bytes, so they keep more in flight
  constexpr int NST = Q8 ? (G <= 2 && D <= 128 ? MSGL_DECODE_FP8_STAGES : 2)
                         : ((sizeof(T) == 4 || D > 128 || G > 4) ? 2 : MSGL_DECODE_STAGES);
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
  float* P_lds = lds;              // [16][16]
  float* A_lds = lds + 256;        // [16]
  float* ML_lds = lds + 256 + 16;  // [16][2]
  uint8_t* K_lds = reinterpret_cast<uint8_t*>(lds + kLdsPerWave);  // [16][KRS bytes]

  // work item from the plan (workgroups past its end have nothing to do); a
  // kv-head group is this workgroup's waves
  if ((int)blockIdx.x >= p.meta[0]) return;
  const int4 item = p.plan[blockIdx.x];
  const int b = item.x;
  const int split = item.y;
  const int kgrp = item.z;
  const int start = p.kv_indptr[b];
  const int L = p.seq_lens ? p.seq_lens[b] : p.kv_indptr[b + 1] - start;
  int n, chunk;
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
  const int t0 = split * chunk;
  const int t1 = split == n - 1 ? L : t0 + chunk;

  const int r = lane & 15;    // MFMA column (token in tile) / A row
  const int g4 = lane >> 4;   // MFMA row group
  const int vc = lane % LPR;  // V: 16-byte chunk within the row
  const int vr = lane / LPR;  // V: token sub-row

  const int64_t row_stride = (int64_t)p.hkv * D * EKV;  // bytes per slot

  {
    const int kvh = kgrp * nwaves + wave;
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

    const uint8_t* kbase_p = reinterpret_cast<const uint8_t*>(p.k_pool) + (int64_t)kvh_c * D * EKV + vc * 16;
    const uint8_t* vbase_p = reinterpret_cast<const uint8_t*>(p.v_pool) + (int64_t)kvh_c * D * EKV + vc * 16;

    // Fused KV store (unquantised pools): the chunk holding position L-1 (the
    // new token) writes its rows to the pool and reads them from k_new/v_new
    // instead -- no other unit reads that slot, so the write needs no ordering
    // inside the launch.
    const bool fused = !Q8 && p.k_new != nullptr;
    const int new_pos = fused && t1 == L ? L - 1 : 0x7fffffff;  // absolute position, or never
    const int64_t new_off = ((int64_t)b * p.hkv + kvh_c) * D * ES + vc * VEC * ES;
    const uint8_t* knew_p = fused ? reinterpret_cast<const uint8_t*>(p.k_new) + new_off : nullptr;
    const uint8_t* vnew_p = fused ? reinterpret_cast<const uint8_t*>(p.v_new) + new_off : nullptr;
    if (active && new_pos != 0x7fffffff && lane < LPR) {
      const int64_t slot = p.out_loc[b];
      if (slot >= 0 && slot < p.num_slots) {
        const int64_t dst = slot * row_stride + (int64_t)kvh * D * ES + vc * VEC * ES;
        st16(reinterpret_cast<uint8_t*>(p.k_pool_w) + dst, ld16(knew_p));
        st16(reinterpret_cast<uint8_t*>(p.v_pool_w) + dst, ld16(vnew_p));
      }
    }
    // Fused store over fp8 pools: the chunk holding the new token quantises its
    // K and V rows exactly like msgl_store_kv_fp8 (lanes [0, LQ) the K row,
    // [LQ, 2 LQ) the V row, one 16-byte chunk of T each) and writes codes and
    // scales before any load of the chunk is issued; the loop then reads the
    // new token from the pool like every other token.
    if constexpr (Q8) {
      if (active && p.k_new != nullptr && t1 == L) {
        constexpr int LQ = D / VEC;  // lanes per input row
        static_assert(2 * LQ <= 64, "a wavefront quantises the K and V rows together");
        const int sub = lane % LQ;
        const bool is_v = (lane / LQ) & 1;  // lanes >= 2 LQ repeat the rows and write nothing
        const uint8_t* src = reinterpret_cast<const uint8_t*>(is_v ? p.v_new : p.k_new) +
                             (((int64_t)b * p.hkv + kvh) * D + sub * VEC) * ES;
        uint32_t w[VEC / 4];
        const float amax = fp8_quantize_chunk<T>(ld16(src), LQ, w);
        const int64_t slot = p.out_loc[b];
        if (lane < 2 * LQ && slot >= 0 && slot < p.num_slots) {
          uint8_t* dst = reinterpret_cast<uint8_t*>(is_v ? p.v_pool_w : p.k_pool_w) +
                         (slot * p.hkv + kvh) * D + sub * VEC;
          static_assert(VEC == 8, "16-bit queries: eight codes per lane");
          *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
          if (sub == 0) p.kv_scale_w[(slot * p.hkv + kvh) * 2 + (is_v ? 1 : 0)] = amax / 448.f;
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
      for (int i = threadIdx.x; i < (ntile + NST - 1) * 16; i += blockDim.x) {
        const int tok = s0 + min(i, seg_len - 1);
        slots_lds[i] = slot_of(p.kv_indices, start, tok, p.page_size, p.num_slots);
      }
      __syncthreads();
      if (!active) continue;

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
        if (Q8) {  // the K and V scales of the token in this lane's MFMA column: one 8-byte load
          const float2 sc = reinterpret_cast<const float2*>(p.kv_scale)[(int64_t)slots_lds[base + r] * p.hkv + kvh_c];
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
        const float sc = Q8 ? p.scale_log2 * buf.ks : p.scale_log2;
        const bool valid = tile * 16 + r < seg_len;
        float pr[4] = {0.f, 0.f, 0.f, 0.f}, al[4] = {1.f, 1.f, 1.f, 1.f};
#pragma unroll
        for (int i = 0; i < NR; ++i) {
          const float x = valid ? s[i] * sc : -INFINITY;
          const float mt = row16_max(x);
          const float m_new = fmaxf(m_run[i], mt);
          al[i] = __builtin_amdgcn_exp2f(m_run[i] - m_new);
          pr[i] = __builtin_amdgcn_exp2f(x - m_new);
          l_run[i] = l_run[i] * al[i] + pr[i];
          m_run[i] = m_new;
        }
        wave_lds_sync();  // previous tile's LDS reads are done
        // P V weights; a quantised V row's scale is folded into its weight (l keeps the plain weights)
        const float vsc = Q8 ? buf.vs : 1.f;
        *reinterpret_cast<f32x4*>(P_lds + r * 16 + 4 * g4) = f32x4{pr[0] * vsc, pr[1] * vsc, pr[2] * vsc, pr[3] * vsc};
        if (r == 0) *reinterpret_cast<f32x4*>(A_lds + 4 * g4) = f32x4{al[0], al[1], al[2], al[3]};
        wave_lds_sync();
        // O = alpha * O + P V on the VALU
        float alpha[G];
#pragma unroll
        for (int g = 0; g < G; ++g) alpha[g] = A_lds[g];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int e = 0; e < VKV; ++e) acc[g][e] *= alpha[g];
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

      // NST-stage register pipeline: tiles t+1 .. t+NST-1 are in flight while t computes
      TileBuf<KV, D> buf[NST];
#pragma unroll
      for (int i = 0; i < NST - 1; ++i) issue(buf[i], i);  // tiles past ntile are padding
      for (int tile = 0; tile < ntile; tile += NST) {
#pragma unroll
        for (int k = 0; k < NST; ++k) {
          const int t = tile + k;
          if (t >= ntile) break;
          issue(buf[(k + NST - 1) % NST], t + NST - 1);
          compute(buf[k], t);
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
}

// Merge split-K partials, one wavefront per (request, kv head):
//   o = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s
// (the combine of the Metal kernel's simdgroup merge, attention/metal.py:75-94).
// Lanes own float4 chunks of the G*D outputs; the partials of up to 8 splits
// are loaded in one batch (one memory round trip) and combined online.
template <typename T, int D, int G>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(DecodeParams p, int batch) {
  const int unit = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);  // (b, kvh)
  const int lane = threadIdx.x & 63;
  if (unit >= batch * p.hkv) return;
  const int b = unit / p.hkv, kvh = unit % p.hkv;
  const int L = p.seq_lens ? p.seq_lens[b] : p.kv_indptr[b + 1] - p.kv_indptr[b];
  int n, chunk;
  split_geometry(L, p.max_splits, p.meta[1], n, chunk);
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

// Wavefronts per workgroup (kv heads handled by one workgroup). Small
// workgroups let a CU start new work as soon as any wave finishes.
#ifndef MSGL_DECODE_WAVES_PER_WG
#define MSGL_DECODE_WAVES_PER_WG 4
#endif

// Work list for paged_decode_kernel, one workgroup: the batch-wide chunk length
// ceil(max_b L_b / max_splits) (a multiple of 16, >= kMinChunk), then every
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

__global__ __launch_bounds__(kPlanThreads) void paged_decode_plan_kernel(DecodeParams p) {
  __shared__ int lens[kPlanLds];
  __shared__ int hist[256];
  __shared__ int wmax[kPlanThreads / 64];
  __shared__ int chunk_s;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
    int mx = 0;
    for (int w = 0; w < kPlanThreads / 64; ++w) mx = max(mx, wmax[w]);
    int c = (mx + p.max_splits - 1) / p.max_splits;
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

template <typename T, typename KV, int D, int G>
static int launch_decode(const DecodeParams& p, int batch, hipStream_t stream) {
  const int nwaves = p.hkv < MSGL_DECODE_WAVES_PER_WG ? p.hkv : MSGL_DECODE_WAVES_PER_WG;
  const size_t lds = ((size_t)kSeg + kSlotPad + (size_t)nwaves * (kLdsPerWave + 16 * k_lds_stride<KV, D>() / 4)) *
                     sizeof(float);
  if (!p.planned) {
    hipLaunchKernelGGL(paged_decode_plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, p);
    MSGL_CHECK_LAUNCH("msgl_paged_decode (plan)");
  }
  hipLaunchKernelGGL((paged_decode_kernel<T, KV, D, G>), dim3(batch * p.max_splits * p.ngrp), dim3(64 * nwaves),
                     lds, stream, p);
  MSGL_CHECK_LAUNCH("msgl_paged_decode");
  if (p.max_splits > 1) {
    const int units = batch * p.hkv;
    hipLaunchKernelGGL((paged_decode_merge_kernel<T, D, G>), dim3((units + 3) / 4), dim3(256), 0, stream, p, batch);
    MSGL_CHECK_LAUNCH("msgl_paged_decode (merge)");
  }
  return MSGL_OK;
}

template <typename T, typename KV, int D>
static int dispatch_group(const DecodeParams& p, int batch, int group, hipStream_t stream) {
  constexpr bool Q8 = std::is_same<KV, fp8e4m3>::value;
  switch (group) {
    case 1: return launch_decode<T, KV, D, 1>(p, batch, stream);
    case 2: return launch_decode<T, KV, D, 2>(p, batch, stream);
    case 4: return launch_decode<T, KV, D, 4>(p, batch, stream);
    case 8: return launch_decode<T, KV, D, 8>(p, batch, stream);
    case 16:
      if constexpr (!Q8) return launch_decode<T, KV, D, 16>(p, batch, stream);
      [[fallthrough]];
    default:
      set_error("msgl_paged_decode: Hq/Hkv = %d not built (1, 2, 4, 8%s)", group, Q8 ? " for fp8 pools" : ", 16");
      return MSGL_ERR_UNSUPPORTED;
  }
}

template <typename T, typename KV = T>
static int dispatch_dim(const DecodeParams& p, int batch, int head_dim, int group, hipStream_t stream) {
  switch (head_dim) {
    case 64: return dispatch_group<T, KV, 64>(p, batch, group, stream);
    case 128: return dispatch_group<T, KV, 128>(p, batch, group, stream);
    case 256: return dispatch_group<T, KV, 256>(p, batch, group, stream);
    default:
      set_error("msgl_paged_decode: head_dim %d not built (64, 128, 256)", head_dim);
      return MSGL_ERR_UNSUPPORTED;
  }
}

// Workspace layout, each region 256-byte aligned: [meta | plan B*S*ngrp int4 |
// (S > 1) m,l B*S*Hq*2 f32 | acc B*S*Hq*D f32].
static inline int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

static inline int decode_groups(int hkv) {
  const int nwaves = hkv < MSGL_DECODE_WAVES_PER_WG ? hkv : MSGL_DECODE_WAVES_PER_WG;
  return (hkv + nwaves - 1) / nwaves;
}

struct DecodeWorkspace {
  int64_t plan, part_ml, part_o, bytes;
};
static inline DecodeWorkspace decode_workspace(int batch, int hq, int hkv, int head_dim, int splits) {
  DecodeWorkspace w;
  const int64_t units = splits > 1 ? (int64_t)batch * splits * hq : 0;
  w.plan = 256;
  w.part_ml = w.plan + align256((int64_t)batch * splits * decode_groups(hkv) * 16);
  w.part_o = w.part_ml + align256(units * 2 * 4);
  w.bytes = w.part_o + align256(units * head_dim * 4);
  return w;
}

}  // namespace msgl

extern "C" int32_t msgl_paged_decode_default_splits(int32_t batch, int32_t num_kv_heads, int32_t max_seq_len) {
  // Aim for ~4096 wavefronts (a bit over one round of MI355X at 3 waves/SIMD):
  // enough units for ragged lengths to balance, few enough that the split-K
  // partials and the merge stay small. No chunk is shorter than kMinChunk.
  // Chunks of at most kMaxChunk tokens keep long-context batches balanced
  // (the dispatcher needs more items than resident slots).
  if (batch <= 0 || num_kv_heads <= 0) return 1;
  constexpr int64_t kMaxChunk = 2048;
  const int64_t target_waves = 4096;
  int64_t s = (target_waves + (int64_t)batch * num_kv_heads - 1) / ((int64_t)batch * num_kv_heads);
  if (max_seq_len > 0) {
    const int64_t cap = (max_seq_len + msgl::kMinChunk - 1) / msgl::kMinChunk;
    if (s > cap) s = cap;
    const int64_t floor_s = (max_seq_len + kMaxChunk - 1) / kMaxChunk;
    if (s < floor_s) s = floor_s;
  }
  if (s < 1) s = 1;
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
                             void* out, void* workspace, int64_t workspace_bytes, void* stream);

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
  p.hq = num_qo_heads;
  p.hkv = num_kv_heads;
  p.max_splits = max_splits;
  p.batch = batch;
  p.ngrp = decode_groups(num_kv_heads);
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

static int paged_decode_impl(const char* fn, DecodeMode mode, const void* q, const void* k_new, const void* v_new,
                             const int32_t* out_loc, const void* k_pool, const void* v_pool, const float* kv_scale,
                             const int32_t* kv_indptr, const int32_t* kv_indices,
                             const int32_t* seq_lens,
                             int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t page_size, int64_t num_slots, int32_t dtype, float scale, int32_t max_splits,
                             void* out, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(batch >= 0 && batch <= 65535, "%s: batch must be in [0, 65535]", fn);
  if (batch == 0) return MSGL_OK;
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
  DecodeParams p;
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
  p.part_ml = max_splits > 1 ? reinterpret_cast<float*>(ws + w.part_ml) : nullptr;
  p.part_o = max_splits > 1 ? reinterpret_cast<float*>(ws + w.part_o) : nullptr;
  p.batch = batch;
  p.ngrp = decode_groups(num_kv_heads);
  p.planned = mode == kRunPlanned;
  p.num_slots = num_slots;
  p.hq = num_qo_heads;
  p.hkv = num_kv_heads;
  p.page_size = page_size;
  p.max_splits = max_splits;
  p.scale_log2 = scale * kLog2e;
  const int group = num_qo_heads / num_kv_heads;
  hipStream_t s = (hipStream_t)stream;
  if (kv_scale != nullptr) {  // fp8 e4m3 pools with per-(slot, kv head) scales
    switch (dtype) {
      case MSGL_BF16: return dispatch_dim<bf16_t, fp8e4m3>(p, batch, head_dim, group, s);
      case MSGL_F16: return dispatch_dim<f16_t, fp8e4m3>(p, batch, head_dim, group, s);
    }
    set_error("%s: fp8 pools take bf16 or fp16 queries (dtype %d)", fn, dtype);
    return MSGL_ERR_UNSUPPORTED;
  }
  switch (dtype) {
    case MSGL_F32: return dispatch_dim<float>(p, batch, head_dim, group, s);
    case MSGL_BF16: return dispatch_dim<bf16_t>(p, batch, head_dim, group, s);
    case MSGL_F16: return dispatch_dim<f16_t>(p, batch, head_dim, group, s);
  }
  return MSGL_ERR_UNSUPPORTED;
}
