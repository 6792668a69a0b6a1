// Device side of the ragged prefill (prefill.hip): parameters, geometry
// helpers and the bf16/fp16 attention and split-K merge bodies, shared with
// the single-launch mixed step (mixed.hip). The design notes are at the top of
// prefill.hip.
#pragma once
#include <algorithm>
#include <type_traits>

#include "msgl_common.h"

namespace msgl {
namespace pf {


constexpr float kLog2eP = 1.4426950408889634f;
constexpr int KT = 32;           // keys per tile
constexpr int NWAVE = 4;         // wavefronts per workgroup (fp32 kernel)
#ifndef MSGL_PREFILL_WAVES
#define MSGL_PREFILL_WAVES 4
#endif
constexpr int NWAVE16 = MSGL_PREFILL_WAVES;  // wavefronts per workgroup of the 16-bit kernel
constexpr int THREADS16 = NWAVE16 * 64;
constexpr int kWin = 1024;       // keys whose slots are staged in LDS at a time
constexpr int kMinChunk = 256;   // smallest key range given its own workgroup
constexpr int kMaxSplits = 16;

struct PrefillParams {
  const void* q;
  const void* k_pool;
  const void* v_pool;
  const float* kv_scale;  // fp8 pools: [num_slots, Hkv, 2] (K, V) scales, else null
  const int32_t* q_indptr;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* seq_lens;
  void* out;
  float* part_o;     // [splits][num_tokens][hq][D]
  float2* part_ml;   // [splits][num_tokens][hq]
  int4* plan;        // work list, longest first: per item (request, kv head, query block, chunk)
                     // then (first token, extend length E, first kv index, kv length L)
  int* plan_count;   // its length, then the sizes the list was built for (plan_matches)
  int* merge_n;      // [num_tokens] chunks of each token's block (<= 1: nothing to merge)
  int64_t num_slots;
  int hq, hkv, page_size;
  int num_reqs, num_tokens;
  int splits;     // key chunks per block (grid dimension)
  int chunk_len;  // keys per chunk, 0 = per block
  int nqb;      // query blocks per request (grid dimension)
  int items;    // (request, query block, chunk) triples x kv heads: the grid
  int plan_capacity;  // work items the plan area holds
  float scale_log2;
  int mode;  // host side only: which launches a call makes (PrefillMode)
};

// Launches of one call: the work list and the attention (+ merge), only the
// attention with a work list already in the workspace, or only the work list.
enum PrefillMode { kPlanAndRun = 0, kRunPlanned = 1, kPlanOnly = 2 };

// Pool slot of token `tok` of the request whose indices start at
// kv_indices[start]; memory-safe for any metadata: an index entry outside
// [0, nidx) (nidx = kv_indptr[R], the entries kv_indices holds) is not read,
// and a slot outside [0, num_slots) becomes slot 0.
__device__ __forceinline__ int64_t kv_slot(const PrefillParams& p, int64_t nidx, int start, int tok) {
  const int64_t i = (int64_t)start + (p.page_size == 1 ? tok : tok / p.page_size);
  if (i < 0 || i >= nidx) return 0;
  const int64_t s = p.page_size == 1 ? (int64_t)p.kv_indices[i] : (int64_t)p.kv_indices[i] * p.page_size + tok % p.page_size;
  return (s >= 0 && s < p.num_slots) ? s : 0;
}

// The work list in the workspace was built for this call's sizes: the plan
// kernel stamps (requests, tokens, splits, query blocks, kv heads, chunk
// length) after its length. A launch over a plan of other sizes does nothing.
__device__ __forceinline__ bool plan_matches(const PrefillParams& p) {
  const int* st = p.plan_count;
  return st[1] == p.num_reqs && st[2] == p.num_tokens && st[3] == p.splits && st[4] == p.nqb && st[5] == p.hkv &&
         st[6] == p.chunk_len;
}

// Keys a block of query tokens [qb, qb + bq) can see.
__device__ __forceinline__ int block_kv_end(int L, int E, int qb, int bq) {
  return min(L, L - E + min(E, qb + bq));
}

// Split of [0, kv_end) into n <= splits chunks of clen keys (a multiple of
// the tile; the last chunk takes the rest), used identically by the attention
// and merge kernels. With a batch-wide chunk length (from the longest
// sequence) only long blocks are split; without one each block is cut evenly.
__device__ __forceinline__ void chunk_geometry(int kv_end, int splits, int chunk_len, int& n, int& clen) {
  if (chunk_len > 0) {
    clen = chunk_len;
  } else {
    const int n0 = max(1, min(splits, (kv_end + kMinChunk - 1) / kMinChunk));
    clen = ((kv_end + n0 - 1) / n0 + KT - 1) / KT * KT;
  }
  n = min(splits, (kv_end + clen - 1) / clen);
}

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __fp16 f16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// ds_read_b64_tr_b16: within each 16-lane group, source lane j's 4 elements
// X[j][0..3] are redistributed so lane i receives Y[i][e] = X[4e + i/4][i%4]
// (lane-layout measured on gfx950). If source lane j points at row key_{j/4},
// columns c0 + 4*(j%4), lane i receives rows key_0..key_3 of column c0 + i.
template <typename T>
__device__ __forceinline__ uint2 lds_read_tr16(const uint8_t* p);
template <>
__device__ __forceinline__ uint2 lds_read_tr16<bf16_t>(const uint8_t* p) {
  MSGL_LDS bf16x4_t* lp = (MSGL_LDS bf16x4_t*)(p);
  return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(lp));
}
template <>
__device__ __forceinline__ uint2 lds_read_tr16<f16_t>(const uint8_t* p) {
  MSGL_LDS f16x4_t* lp = (MSGL_LDS f16x4_t*)(p);
  return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4f16(lp));
}

// The value of lane l ^ 32 combined with this lane's, on the VALU:
// v_permlane32_swap of x with itself leaves (x[l % 32], x[l % 32 + 32]) in
// every lane (checked on gfx950), so max / sum of the pair needs no LDS
// round trip as a lane shuffle would.
__device__ __forceinline__ f32x2_t halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return f32x2_t{__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ float xor32_max(float x) {
  const f32x2_t h = halves(x);
  return fmaxf(h[0], h[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
  const f32x2_t h = halves(x);
  return h[0] + h[1];
}

// ds_read_b64_tr_b8: within each 16-lane group, lane i receives byte i%8 of
// source lanes i/8 + 2e at position e (e = 0..7; lane layout measured on
// gfx950). If source lane s points at row key(s/2), columns c0 + 8(s%2) ..+7,
// lane i receives rows key(0..7) of column c0 + i.
__device__ __forceinline__ uint2 lds_read_tr8(const uint8_t* p) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((MSGL_LDS v2i*)(p)));
}

// 8 fp8 e4m3 values -> the 16-bit MFMA operand (exact: every e4m3 value is a
// bf16 and an fp16 value).
template <typename T>
__device__ __forceinline__ u32x4 fp8x8(uint32_t w0, uint32_t w1);
template <>
__device__ __forceinline__ u32x4 fp8x8<bf16_t>(uint32_t w0, uint32_t w1) {
  return u32x4{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true))};
}
template <>
__device__ __forceinline__ u32x4 fp8x8<f16_t>(uint32_t w0, uint32_t w1) {
  return u32x4{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true))};
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

// v_mfma_f32_32x32x16_{bf16,f16}: A [32 x 16] lane l holds row l%32, k
// 8*(l/32)..+7; B [16 x 32] lane l holds column l%32, the same k; C [32 x 32]
// lane l holds column l%32, rows 8*(i/4) + 4*(l/32) + i%4 for i = 0..15.
// (The 16x16x32 form runs at half this rate on gfx950.)
template <typename T>
struct MMA32;

// Wave priorities (s_setprio) inside the key loop, so that of the two
// wavefronts of a SIMD the one issuing a tile's LDS transfers goes first, then
// the one in its P.V block (the P.V MFMAs with the next tile's exp/pack between
// them), then the one in its S block. Measured on the 16-request workload
// (same box, alternating runs; no priorities: bf16 73.6, fp8 88.5 us/layer):
//   P.V 1:                 bf16 73.2, fp8 80.9
//   S 1, P.V 2:            bf16 73.0, fp8 80.4
//   P.V 1, transfers 3:    bf16 71.9, fp8 80.8   (bf16 pools)
//   S 1, P.V 2, transfers 3: bf16 72.6, fp8 79.9 (fp8 pools)
//   each MFMA's issue 1:   bf16 74.4, fp8 83.2
// 0 turns them off.
#ifndef MSGL_PREFILL_SKIP_DEAD
#define MSGL_PREFILL_SKIP_DEAD 1
#endif
#ifndef MSGL_PREFILL_SETPRIO
#define MSGL_PREFILL_SETPRIO 1
#endif
template <>
struct MMA32<bf16_t> {
  __device__ __forceinline__ static f32x16 mma(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  // v_cvt_pk_bf16_f32: round-to-nearest-even, like f32_to_bf16
  __device__ __forceinline__ static uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
  }
  __device__ __forceinline__ static uint32_t scale2(uint32_t w, float a) {
    return pack2(__uint_as_float(w << 16) * a, __uint_as_float(w & 0xffff0000u) * a);
  }
  // acc + the two packed values (v_dot2c_f32_bf16 with (1, 1))
  __device__ __forceinline__ static float sum2(uint32_t w, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), bf16x2_t{(__bf16)1.f, (__bf16)1.f}, acc,
                                           false);
  }
};
template <>
struct MMA32<f16_t> {
  __device__ __forceinline__ static f32x16 mma(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
  __device__ __forceinline__ static uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, f16x2_t));
  }
  __device__ __forceinline__ static uint32_t scale2(uint32_t w, float a) {
    const f16x2_t v = __builtin_bit_cast(f16x2_t, w);
    return pack2((float)v[0] * a, (float)v[1] * a);
  }
  __device__ __forceinline__ static float sum2(uint32_t w, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w), f16x2_t{(_Float16)1.f, (_Float16)1.f}, acc, false);
  }
};

// Geometry of the 16-bit kernel for one head_dim and pool element size KB
// (2: bf16/fp16 pools; 1: fp8 pools, whose stages also hold the tile's scales).
template <int D, int KB = 2>
struct G16 {
  static constexpr int ROWS = NWAVE16 * 32;        // query rows per workgroup (32 per wavefront)
  static constexpr int RBYTES = D * KB;             // bytes per K/V row
  static constexpr int CPR = RBYTES / 16;           // 16-byte chunks per row
  static constexpr int SWZ = CPR >= 16 ? 15 : CPR - 1;
  static constexpr int TILE_BYTES = KT * RBYTES;    // K (or V) tile
  static constexpr int SCALE_BYTES = KB == 1 ? KT * 8 : 0;  // (K, V) scale of each key
  static constexpr int STAGE_BYTES = 2 * TILE_BYTES + SCALE_BYTES;
  static constexpr int SPW = 2 * KT / NWAVE16;      // scale dwords each wavefront transfers per tile
  // The occupancy the register budget is built for: two workgroups per CU at
  // head_dim <= 128 (LDS: 2 x 68 KiB of the 160 KiB at 128; <= 256 VGPRs),
  // one at 256 (132 KiB, 512 VGPRs).
  static constexpr int NS = 4;  // V of tile t-1, tiles t and t+1 resident, tile t+2 in flight
  static constexpr int WAVES = D <= 128 ? 2 : 1;
  static constexpr int NXFER = TILE_BYTES / 1024;                // 1 KiB transfers per tile, each of K and V
  static constexpr int IPW = (NXFER + NWAVE16 - 1) / NWAVE16;     // of them per wavefront (all or none)
  static constexpr int LDS_BYTES = NS * STAGE_BYTES + kWin * 4;
  static_assert(NXFER % NWAVE16 == 0 || NXFER < NWAVE16, "a tile must split evenly over the wavefronts");
  static_assert(KB == 2 || (2 * KT) % NWAVE16 == 0, "a tile's scales must split evenly over the wavefronts");
};

// XOR swizzle of a row's 16-byte chunks: a bijection on r % 16, so 16
// consecutive rows place one logical chunk in 16 different bank groups, and
// rows 4g..4g+3 x chunks {2t, 2t+1} land in 8 different ones.
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 1) | (((r >> 2) & 1) << 3) | ((r >> 3) & 1); }

// KV: the pools' storage type, T itself or fp8e4m3 (codes plus the per-slot,
// per-kv-head (K, V) scales of p.kv_scale).
template <typename T, typename KV, int D, int G>
__device__ __forceinline__ void prefill16_body(const PrefillParams& p, int wg) {
  constexpr bool Q8 = std::is_same<KV, fp8e4m3>::value;
  using Geo = G16<D, (int)sizeof(KV)>;
  constexpr int ROWS = Geo::ROWS;
  static_assert(G >= 1 && G <= 32, "unsupported group size");
  constexpr int BQ = ROWS / G;     // query tokens per workgroup
  constexpr int RROWS = BQ * G;    // rows holding (token, head) pairs; any rest pads the block
  constexpr int NQF = D / 16;   // 16-wide d steps of the S^T product
  constexpr int NDT = D / 32;   // 32-wide output column tiles
  constexpr int NS = Geo::NS;
  constexpr int IPW = Geo::IPW;
  constexpr int RBYTES = Geo::RBYTES;
  constexpr int CPR = Geo::CPR;
  constexpr int SWZ = Geo::SWZ;

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  int* slots = reinterpret_cast<int*>(smem + NS * Geo::STAGE_BYTES);
  const uint32_t lds0 = (uint32_t)(uintptr_t)((MSGL_LDS uint8_t*)smem);

  // ---- work item from the plan (workgroups past its end have nothing to do) ----
  if (wg >= *p.plan_count || !plan_matches(p)) return;
  const int4 item = p.plan[2 * wg];
  const int4 geo = p.plan[2 * wg + 1];  // the request's geometry, loaded with the item
  const int kvh = item.y, qblk = item.z, split = item.w;
  const int q0 = geo.x, E = geo.y, kv_start = geo.z, L = geo.w;
  const int qb = qblk * BQ;
  if (qb >= E) return;
  const int P = L - E;
  const int kv_end = block_kv_end(L, E, qb, BQ);
  int nchunks, clen;
  chunk_geometry(kv_end, p.splits, p.chunk_len, nchunks, clen);
  if (split >= nchunks) return;
  const int c0 = split * clen;
  const int c1 = split == nchunks - 1 ? kv_end : c0 + clen;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int rl = lane & 31;  // this lane's query row within the wavefront's 32 (S^T column)
  const int h = lane >> 5;   // k half of the MFMA operands; row quarter of the results

  // this lane's query row, clamped into range so every row sees key 0; rows
  // past E are computed, not stored
  const int my_row = wave * 32 + rl;
  // A wavefront whose 32 rows all lie past the extend (the last query block of
  // a request) only moves tiles: it issues its share of the LDS transfers and
  // meets every barrier, but computes nothing.
  const bool live = !MSGL_PREFILL_SKIP_DEAD || (wave * 32 < RROWS && qb + wave * 32 / G < E);
  const int my_tok = min(qb + my_row / G, E - 1);
  const int limit = P + my_tok;
  const int lim_lo = __builtin_amdgcn_readfirstlane(limit);  // the wavefront's first row (lane 0)
  // Q fragment (B operand of S^T = K Q^T): d = 16j + 8h .. +7 (rows clamped
  // into [0, num_tokens): q holds num_tokens rows whatever the offsets say)
  u32x4 qf[NQF];
  {
    const int64_t qr = min((int64_t)max(q0 + my_tok, 0), (int64_t)p.num_tokens - 1);
    const uint8_t* qrow = reinterpret_cast<const uint8_t*>(p.q) + (qr * p.hq + kvh * G + my_row % G) * D * 2;
#pragma unroll
    for (int j = 0; j < NQF; ++j) qf[j] = ld16(qrow + (16 * j + 8 * h) * 2);
  }
  // O accumulators: acc[dt][i] = O[row 8(i/4) + 4h + i%4][column 32 dt + rl]
  f32x16 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[dt][i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;  // of this lane's row (l_run: this lane's keys only)

  const uint8_t* kp = reinterpret_cast<const uint8_t*>(p.k_pool);
  const uint8_t* vp = reinterpret_cast<const uint8_t*>(p.v_pool);
  const int64_t row_stride = (int64_t)p.hkv * RBYTES;
  const int64_t head_off = (int64_t)kvh * RBYTES;
  const int64_t nidx = p.kv_indptr[p.num_reqs];  // entries of kv_indices

  // This wavefront's IPW transfers of each of K and V per tile. Transfer qi
  // covers LDS bytes [qi KiB, (qi+1) KiB) of the tile: lane l fills physical
  // chunk (qi*64 + l) % CPR of row (qi*64 + l) / CPR with logical chunk
  // pc ^ swz(row). The rows' slots are read from LDS one tile ahead (load_slots)
  // so the issue itself waits on nothing; rows past the window repeat its last key.
  int dma_row[IPW], nslot[IPW];
  const uint8_t* kcol[IPW];
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int flat = (wave + NWAVE16 * i) * 64 + lane;
    dma_row[i] = flat / CPR;
    kcol[i] = kp + head_off + (((flat % CPR) ^ (swz(dma_row[i]) & SWZ)) << 4);
  }
  const int64_t vk = vp - kp;  // V rows sit at the same offsets in the V pool
  // a wavefront issues all its row transfers of a tile or none (wave-uniform)
  const bool kv_issuer = Geo::NXFER >= NWAVE16 || wave < Geo::NXFER;
  // fp8: lane j < SPW of wavefront w moves scale dword d = SPW w + j of the
  // tile's [K scales of its KT keys | V scales]: (K or V = d / KT, key d % KT)
  const int sc_dw = wave * Geo::SPW + lane;
  const float* sc_src = Q8 ? p.kv_scale + (int64_t)kvh * 2 + sc_dw / KT : nullptr;
  int sslot = 0;
  auto load_slots = [&](int t, int nw) {
#pragma unroll
    for (int i = 0; i < IPW; ++i) nslot[i] = slots[min(t * KT + dma_row[i], nw - 1)];
    if (Q8) sslot = slots[min(t * KT + sc_dw % KT, nw - 1)];
  };
  auto issue = [&](int st) {
    const uint32_t sb = lds0 + st * Geo::STAGE_BYTES;
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      // slots are clamped into [0, num_slots) and a row stride fits 32 bits: one 32 x 32 -> 64-bit multiply-add
      const uint8_t* g = kcol[i] + (uint64_t)(uint32_t)nslot[i] * (uint32_t)row_stride;
      if (kv_issuer) {
        const uint32_t lk = __builtin_amdgcn_readfirstlane(sb + (wave + NWAVE16 * i) * 1024);
        dma16(g, lk);
        dma16(g + vk, lk + Geo::TILE_BYTES);
      }
    }
    if (Q8 && lane < Geo::SPW)  // one transfer per wavefront and tile, SPW lanes active
      dma4(sc_src + (int64_t)sslot * p.hkv * 2,
           __builtin_amdgcn_readfirstlane(sb + 2 * Geo::TILE_BYTES + wave * Geo::SPW * 4));
  };
  // Wait until this wavefront's transfers of a tile have landed, `after`
  // (0 or 1) tiles having been issued behind it.
  auto wait_tile = [&](int after) {
    if (after <= 0) {
      vm_wait<0>();
    } else if (kv_issuer) {
      vm_wait<2 * IPW + (Q8 ? 1 : 0)>();
    } else {
      vm_wait<Q8 ? 1 : 0>();
    }
  };

  // K operands (A of S^T = K Q^T) of the tile in stage st, all read before
  // the first MFMA: d step j takes key row rl, d = 16j + 8h .. +7 (fp8: half h
  // of chunk j, widened when used)
  struct KOps {
    u32x4 w[Q8 ? 1 : NQF];
    uint2 b[Q8 ? NQF : 1];
  };
  auto k_read = [&](int st, KOps& ko) {
    const uint8_t* krow = smem + st * Geo::STAGE_BYTES + rl * RBYTES;
    const int sw = swz(rl) & SWZ;
#pragma unroll
    for (int j = 0; j < NQF; ++j) {
      if constexpr (Q8) {
        ko.b[j] = *reinterpret_cast<const uint2*>(krow + ((j ^ sw) << 4) + 8 * h);
      } else {
        ko.w[j] = *reinterpret_cast<const u32x4*>(krow + (((2 * j + h) ^ sw) << 4));
      }
    }
  };
  auto k_operand = [&](const KOps& ko, int j) -> u32x4 {
    if constexpr (Q8) {
      return fp8x8<T>(ko.b[j].x, ko.b[j].y);
    } else {
      return ko.w[j];
    }
  };
  // S^T = K Q^T of the tile in ring stage st: lane l gets the scores of row rl
  // against keys 8c + 4h + r (c, r = 0..3) in sdst[4c + r] (one MFMA chain over d)
  auto scores = [&](int st, f32x16& sdst) {
    KOps ko;
    k_read(st, ko);
    f32x16 acc_s = {};
#pragma unroll
    for (int j = 0; j < NQF; ++j) acc_s = MMA32<T>::mma(k_operand(ko, j), qf[j], acc_s);
    sdst = acc_s;
  };
  // Row max of the scores of tile t (keys kbase..), raw (scale > 0, so the raw
  // max orders like the scaled one); x gets the scores, -inf where masked.
  // fp8: the K (which = 0) or V (1) scales of this lane's 16 keys 8c + 4h + r
  // of the tile in ring stage st (four consecutive keys per c: one 16-byte read)
  auto tile_scales = [&](int st, int which, float (&sc)[16]) {
    const f32x4* sp =
        reinterpret_cast<const f32x4*>(smem + st * Geo::STAGE_BYTES + 2 * Geo::TILE_BYTES + which * KT * 4);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const f32x4 a = sp[2 * c + h];
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[4 * c + r] = a[r];
    }
  };
  // Block A of an iteration: the S^T MFMAs of the tile in stage st (one chain
  // over d) with the row max of the current tile's scores sc between them,
  // 16 / NQF scores per MFMA, in this order (sched_barrier: the matrix core
  // runs each MFMA while the wavefront issues the VALU work behind it).
  // x gets the scores (a quantised key's scale applied), -inf where masked:
  // key 8(i/4) + 4h + i%4 of the tile is visible iff it is <= thr.
  auto scores_rowmax = [&](int st, f32x16& sdst, const f32x16& sc, const float (&ks)[16], float (&x)[16], int thr,
                           auto masked) -> float {
    constexpr bool MASKED = decltype(masked)::value;
    constexpr int EPM = 16 / NQF;
    KOps ko;
    k_read(st, ko);
    float m = -INFINITY;
    f32x16 acc_s = {};
    if (MSGL_PREFILL_SETPRIO && Q8) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int j = 0; j < NQF; ++j) {
      acc_s = MMA32<T>::mma(k_operand(ko, j), qf[j], acc_s);
#pragma unroll
      for (int e = 0; e < EPM; ++e) {
        const int i = j * EPM + e;
        float v = Q8 ? sc[i] * ks[i] : sc[i];
        if (MASKED && 8 * (i >> 2) + (i & 3) > thr) v = -INFINITY;
        x[i] = v;
        m = fmaxf(m, v);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (MSGL_PREFILL_SETPRIO && Q8) __builtin_amdgcn_s_setprio(0);
    sdst = acc_s;
    return m;
  };
  // Lazy rescale: a row's reference m_run (log2 domain) moves only when its max
  // exceeds it by more than 8, so P <= 2^8 and most tiles leave the
  // accumulators alone. Exact up to rounding: P, l and O share the reference.
  // The P of the previous tile, whose P V is still to come, is rescaled with
  // them (in this lane: it holds its own row's P).
  auto rescale = [&](float mloc, u32x4 (&pa_prev)[2], bool has_prev) {
    const float mcand = mloc * p.scale_log2;
    const bool grow = mcand > m_run + 8.f;
    if (__ballot(grow) != 0) {
      const float m_new = grow ? mcand : m_run;
      const float alpha = grow ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.f;
      l_run *= alpha;
      m_run = m_new;
      // accumulator i holds row 8(i/4) + 4h + i%4, whose factor is in that lane
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float ar = __shfl(alpha, 8 * (i >> 2) + 4 * h + (i & 3));
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) acc[dt][i] *= ar;
      }
      if (has_prev) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int w = 0; w < 4; ++w) pa_prev[ks][w] = MMA32<T>::scale2(pa_prev[ks][w], alpha);
      }
    }
  };
  // O += P V with the V tile in ring stage st
  auto pv = [&](int st, const u32x4 (&pa)[2]) {
    const uint8_t* Vb = smem + st * Geo::STAGE_BYTES + Geo::TILE_BYTES;
    // B operand (keys of the same slots x 32 columns) by transposing reads: in
    // 16-lane group g (columns 16(g%2).., key half h = g/2) source lane i16 reads
    // row 16ks + 4h + i16/4 (+8 for slots e >= 4), columns 32dt + 16(g%2) + 4(i16%4)
    // .. +3 = logical chunk 4dt + 2(g%2) + (i16%4)/2, half i16%2
    const int i16 = lane & 15;
    const int gs = (lane >> 4) & 1;
    if constexpr (Q8) {
      // fp8: one transposing 8-bit read per (ks, dt). Source lane s = i16 reads
      // row 16ks + 8(s/8) + 4h + (s/2)%4 (the key of slot e = s/2), columns
      // 32dt + 16(g%2) + 8(s%2) .. +7 = half s%2 of logical chunk 2dt + g%2;
      // lane i then holds that slot order for column 32dt + 16(g%2) + i.
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int r = 16 * ks + 8 * (i16 >> 3) + 4 * h + ((i16 >> 1) & 3);
        const uint8_t* vr = Vb + r * RBYTES + ((i16 & 1) << 3);
        const int sw = swz(r) & SWZ;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const uint2 v8 = lds_read_tr8(vr + (((2 * dt + gs) ^ sw) << 4));
          acc[dt] = MMA32<T>::mma(pa[ks], fp8x8<T>(v8.x, v8.y), acc[dt]);
        }
      }
      return;
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int r0 = 16 * ks + 4 * h + (i16 >> 2);
      const int r1 = r0 + 8;
      const uint8_t* v0 = Vb + r0 * RBYTES + ((i16 & 1) << 3);
      const uint8_t* v1 = Vb + r1 * RBYTES + ((i16 & 1) << 3);
      const int sw0 = swz(r0) & SWZ, sw1 = swz(r1) & SWZ;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const int c = 4 * dt + 2 * gs + ((i16 & 3) >> 1);
        const uint2 lo = lds_read_tr16<T>(v0 + ((c ^ sw0) << 4));
        const uint2 hi = lds_read_tr16<T>(v1 + ((c ^ sw1) << 4));
        const u32x4 bop = {lo.x, lo.y, hi.x, hi.y};
        acc[dt] = MMA32<T>::mma(pa[ks], bop, acc[dt]);
      }
    }
  };
  // Block C: O += P V for the tile in stage st (MFMA k: 16-key step k / NDT,
  // column tile k % NDT, so consecutive MFMAs are independent) with this
  // tile's P = exp2(x * scale - m_run) between them, 16 / (2 NDT) keys per
  // MFMA, packed into the A operands of the next P V (slot (h, e) of step ks =
  // key 16ks + 8(e/4) + 4h + e%4, i.e. this lane's scores 8ks .. 8ks+7 in order).
  // fp8: a quantised V row's scale folds into its weight in P; l keeps the plain weights.
  auto pv_probs = [&](int st, const u32x4 (&pa)[2], const float (&x)[16], const float (&vs)[16],
                      u32x4 (&pa_new)[2], auto do_pv) {
    constexpr bool DO_PV = decltype(do_pv)::value;
    if (MSGL_PREFILL_SETPRIO) __builtin_amdgcn_s_setprio(Q8 ? 2 : 1);
    constexpr int NMF = 2 * NDT;
    constexpr int EPM = 16 / NMF;
    const uint8_t* Vb = smem + st * Geo::STAGE_BYTES + Geo::TILE_BYTES;
    const int i16 = lane & 15;
    const int gs = (lane >> 4) & 1;
    // B operands, read in the order of use (layouts as in pv)
    u32x4 bop[2][NDT];
    uint2 b8[2][NDT];
    if constexpr (DO_PV) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if constexpr (Q8) {
          const int r = 16 * ks + 8 * (i16 >> 3) + 4 * h + ((i16 >> 1) & 3);
          const uint8_t* vr = Vb + r * RBYTES + ((i16 & 1) << 3);
          const int sw = swz(r) & SWZ;
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) b8[ks][dt] = lds_read_tr8(vr + (((2 * dt + gs) ^ sw) << 4));
        } else {
          const int r0 = 16 * ks + 4 * h + (i16 >> 2);
          const uint8_t* v0 = Vb + r0 * RBYTES + ((i16 & 1) << 3);
          const uint8_t* v1 = v0 + 8 * RBYTES;
          const int sw0 = swz(r0) & SWZ, sw1 = swz(r0 + 8) & SWZ;
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            const int c = 4 * dt + 2 * gs + ((i16 & 3) >> 1);
            const uint2 lo = lds_read_tr16<T>(v0 + ((c ^ sw0) << 4));
            const uint2 hi = lds_read_tr16<T>(v1 + ((c ^ sw1) << 4));
            bop[ks][dt] = u32x4{lo.x, lo.y, hi.x, hi.y};
          }
        }
      }
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;  // a row may see nothing yet
    float pr[16];
    float ls[2] = {0.f, 0.f};  // fp8: the row sum of the plain weights (P carries the V scales)
    float lp = 0.f;            // otherwise: of the rounded weights the P V products use
#pragma unroll
    for (int k = 0; k < NMF; ++k) {
      if constexpr (DO_PV) {
        const int ks = k / NDT, dt = k % NDT;
        if constexpr (Q8) {
          acc[dt] = MMA32<T>::mma(pa[ks], fp8x8<T>(b8[ks][dt].x, b8[ks][dt].y), acc[dt]);
        } else {
          acc[dt] = MMA32<T>::mma(pa[ks], bop[ks][dt], acc[dt]);
        }
      }
#pragma unroll
      for (int e = 0; e < EPM; ++e) {
        const int i = k * EPM + e;
        pr[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[i], p.scale_log2, -m_use));
        if (Q8) {
          ls[i & 1] += pr[i];
          pr[i] *= vs[i];
        }
        if (i & 1) {
          const uint32_t w = MMA32<T>::pack2(pr[i - 1], pr[i]);
          pa_new[i >> 3][(i & 7) >> 1] = w;
          if (!Q8) lp = MMA32<T>::sum2(w, lp);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    l_run += Q8 ? ls[0] + ls[1] : lp;
    if (MSGL_PREFILL_SETPRIO) __builtin_amdgcn_s_setprio(0);
  };
  // Software pipeline per window, three tiles deep. Iteration t:
  //   A: the S MFMAs of tile t+1 interleaved with tile t's masked row max;
  //   B: (rare) the rescale when a row's max moved;
  //   C: the P V MFMAs of tile t-1 interleaved with tile t's exp/sum/pack.
  // (gfx950 overlaps MFMA with VALU work of the same wavefront, not of other
  // wavefronts on the SIMD.) V of tile t-1, tile t and K of tile t+1 stay
  // resident, so iteration t's transfer (tile t+2) fills the stage of tile
  // t-2: a ring of NS >= 4.
  static_assert(NS >= 4, "the pipeline keeps three tiles resident");
  for (int w0 = c0; w0 < c1; w0 += kWin) {
    const int nw = min(kWin, c1 - w0);
    const int ntiles = (nw + KT - 1) / KT;
    const int kend = w0 + nw;
    __syncthreads();  // every wavefront is done with the previous window
    {  // the window's slots: every gather load in flight before the first LDS store
      constexpr int SPT = kWin / THREADS16;
      int sv[SPT];
#pragma unroll
      for (int k = 0; k < SPT; ++k) {  // kv_slot in two passes: every load before any use
        const int tok = w0 + min(tid + k * THREADS16, nw - 1);
        const int64_t ix = (int64_t)kv_start + (p.page_size == 1 ? tok : tok / p.page_size);
        sv[k] = (ix >= 0 && ix < nidx) ? p.kv_indices[ix] : -1;  // -1: outside kv_indices, becomes slot 0
      }
#pragma unroll
      for (int k = 0; k < SPT; ++k) {
        const int tok = w0 + min(tid + k * THREADS16, nw - 1);
        const int64_t sl = p.page_size == 1 ? (int64_t)sv[k] : (int64_t)sv[k] * p.page_size + tok % p.page_size;
        sv[k] = (sl >= 0 && sl < p.num_slots) ? (int)sl : 0;
      }
#pragma unroll
      for (int k = 0; k < SPT; ++k) {
        const int i = tid + k * THREADS16;
        if (i < nw) slots[i] = sv[k];
      }
    }
    // Q must have arrived before the key loop: otherwise the compiler's wait
    // for it lands inside the loop (its wait analysis merges the loop entry),
    // where a vmcnt would also drain the LDS transfers in flight. Waiting here,
    // with the first window's slot gather, makes the two share a round trip.
#pragma unroll
    for (int j = 0; j < NQF; ++j) asm volatile("" ::"v"(qf[j]));
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 2; ++s)
      if (s < ntiles) {
        load_slots(s, nw);
        issue(s);
      }
    load_slots(2, nw);  // clamped into the window: harmless when unused
    wait_tile(min(1, ntiles - 1));
    __syncthreads();  // tile 0 visible to all
    f32x16 s_cur;
    if (live) scores(0, s_cur);
    u32x4 pa_prev[2];

    // stc: tile t's ring stage as a compile-time constant (the main loop runs
    // NS iterations per trip, so every LDS address offset folds into the
    // instructions), or -1 for one computed at run time
    auto iteration = [&](int t, auto first, auto stc) {
      constexpr bool FIRST = decltype(first)::value;
      constexpr int SC = decltype(stc)::value;
      const int st = SC >= 0 ? SC : t % NS;
      const int st1 = SC >= 0 ? (SC + 1) % NS : (t + 1) % NS;
      const int st2 = SC >= 0 ? (SC + 2) % NS : (t + 2) % NS;
      const int stp = SC >= 0 ? (SC + NS - 1) % NS : (t + NS - 1) % NS;
      if (t + 1 < ntiles) vm_wait<0>();  // tile t+1, the only one in flight, landed
      __syncthreads();  // tile t+1 visible; everyone is done with tile t-2's stage
      if (MSGL_PREFILL_SETPRIO) __builtin_amdgcn_s_setprio(3);
      if (t + 2 < ntiles) issue(st2);
      if (MSGL_PREFILL_SETPRIO) __builtin_amdgcn_s_setprio(0);
      const int kbase = w0 + t * KT;
      // A (past the last tile, scores reads a stage whose transfers have all landed; unused)
      f32x16 s_next;
      float x[16];
      float ksc[16];  // fp8: tile t's K scales
      if constexpr (Q8) tile_scales(st, 0, ksc);
      if (!live) {
        load_slots(t + 3, nw);
        return;
      }
      float mloc;
      if (kbase + KT <= kend && kbase + KT - 1 <= lim_lo) {
        mloc = scores_rowmax(st1, s_next, s_cur, ksc, x, 0, std::false_type{});
      } else {
        mloc = scores_rowmax(st1, s_next, s_cur, ksc, x, min(limit, kend - 1) - kbase - 4 * h,
                             std::true_type{});
      }
      mloc = xor32_max(mloc);  // with the row's other 16 keys
      // B
      rescale(mloc, pa_prev, !FIRST);
      // C
      float vsc[16];  // fp8: tile t's V scales
      if constexpr (Q8) tile_scales(st, 1, vsc);
      load_slots(t + 3, nw);  // for the next iteration's issue (clamped: harmless when unused)
      u32x4 pa_new[2];
      pv_probs(stp, pa_prev, x, vsc, pa_new, std::integral_constant<bool, !FIRST>{});
      pa_prev[0] = pa_new[0];
      pa_prev[1] = pa_new[1];
      s_cur = s_next;
    };
    static_assert(NS == 4, "the main loop is unrolled for a four-stage ring");
    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, 1>;
    using C2 = std::integral_constant<int, 2>;
    using C3 = std::integral_constant<int, 3>;
    iteration(0, std::true_type{}, C0{});
    int t = 1;
    if constexpr (D <= 128) {  // (at 256 the unrolled body would spill)
      for (; t + 3 < ntiles; t += 4) {  // tiles 1..4 mod 4: stages 1, 2, 3, 0
        iteration(t, std::false_type{}, C1{});
        iteration(t + 1, std::false_type{}, C2{});
        iteration(t + 2, std::false_type{}, C3{});
        iteration(t + 3, std::false_type{}, C0{});
      }
    }
    for (; t < ntiles; ++t) iteration(t, std::false_type{}, std::integral_constant<int, -1>{});
    if (live) pv((ntiles - 1) % NS, pa_prev);
  }

  // ---- results: accumulator i is WG row wave*32 + 8(i/4) + 4h + i%4, column 32dt + rl ----
  const float l_row = xor32_sum(l_run);  // both halves of this lane's row
  if (nchunks == 1) {
    const float inv = 1.f / l_row;
    T* out = reinterpret_cast<T*>(p.out);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int m = 8 * (i >> 2) + 4 * h + (i & 3);
      const int row = wave * 32 + m;
      const int tok = qb + row / G;
      const float rinv = __shfl(inv, m);
      if (row < RROWS && tok < E && q0 + tok >= 0 && q0 + tok < p.num_tokens) {
        T* orow = out + ((int64_t)(q0 + tok) * p.hq + kvh * G + row % G) * D;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) orow[32 * dt + rl] = from_f32<T>(acc[dt][i] * rinv);
      }
    }
  } else {
    const int64_t base = (int64_t)split * p.num_tokens;
    if (h == 0) {
      const int tok = qb + my_row / G;
      if (my_row < RROWS && tok < E && q0 + tok >= 0 && q0 + tok < p.num_tokens)
        p.part_ml[(base + q0 + tok) * p.hq + kvh * G + my_row % G] = make_float2(m_run, l_row);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = wave * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
      const int tok = qb + row / G;
      if (row < RROWS && tok < E && q0 + tok >= 0 && q0 + tok < p.num_tokens) {  // the workspace holds num_tokens rows
        float* orow = p.part_o + ((base + q0 + tok) * p.hq + kvh * G + row % G) * D;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) orow[32 * dt + rl] = acc[dt][i];
      }
    }
  }
}

// Combines the chunks of every query row whose block was split: one thread
// per 4 output columns of one (token, head). The plan kernel left each token's
// chunk count in merge_n, so the (m, l) and O partials of up to kMergeUnroll
// chunks are loaded at once, with no lookup in front of them.
constexpr int kMergeUnroll = 4;

template <typename T, int D>
__device__ __forceinline__ void prefill_merge_body(const PrefillParams& p, int tk, int hy) {
  constexpr int TPH = D / 4;
  constexpr int HPB = 256 / TPH;
  if (!plan_matches(p)) return;
  const int n = min(p.merge_n[tk], p.splits);
  if (n <= 1) return;  // written by the attention kernel (or not a token of any request)
  const int h = hy * HPB + threadIdx.x / TPH;
  const int d = (threadIdx.x % TPH) * 4;
  if (h >= p.hq) return;
  const int64_t stride = (int64_t)p.num_tokens * p.hq;
  const int64_t idx = (int64_t)tk * p.hq + h;
  // out = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c over the chunks, M = max_c m_c
  // (kMergeUnroll chunks per pass, the running M rescaling earlier passes)
  float M = -INFINITY, lsum = 0.f;
  float o[4] = {0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < n; c0 += kMergeUnroll) {
    float2 ml[kMergeUnroll];
    float4 v[kMergeUnroll];
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
      const int64_t e = (int64_t)min(c0 + u, n - 1) * stride + idx;
      ml[u] = p.part_ml[e];
      v[u] = *reinterpret_cast<const float4*>(p.part_o + e * D + d);
      if (c0 + u >= n) ml[u] = make_float2(-INFINITY, 0.f);
    }
    float Mn = M;
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) Mn = fmaxf(Mn, ml[u].x);
    const float a = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - Mn);
    lsum *= a;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] *= a;
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
      const float w = ml[u].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml[u].x - Mn);
      lsum += ml[u].y * w;
      o[0] += w * v[u].x;
      o[1] += w * v[u].y;
      o[2] += w * v[u].z;
      o[3] += w * v[u].w;
    }
    M = Mn;
  }
  const float inv = 1.f / lsum;
  T* dst = reinterpret_cast<T*>(p.out) + idx * D + d;
  T r[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = from_f32<T>(o[e] * inv);
  *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(r);
}

// Validates the arguments of a prefill call and fills p (the workspace regions
// included); empty: the batch has no query, nothing to launch. (prefill.hip)
int prefill_params(const char* fn, int mode, const void* q, const void* k_pool, const void* v_pool,
                   const float* kv_scale, const int32_t* q_indptr, const int32_t* kv_indptr, const int32_t* kv_indices,
                   const int32_t* seq_lens, int32_t num_reqs, int32_t num_tokens, int32_t max_extend_len,
                   int32_t max_seq_len, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                   int32_t page_size, int64_t num_slots, int32_t dtype, float scale, int32_t max_splits, void* out,
                   void* workspace, int64_t workspace_bytes, PrefillParams& p, bool& empty);

// The work-list launch of the 16-bit path, bq query tokens per block
// (prefill.hip).
int launch_prefill_plan(const PrefillParams& p, int bq, hipStream_t stream);

// The launches of one (query, pool) type pair -- the work list unless p.mode
// runs a stored one, the attention grid, the split-K merge -- for the
// instantiation that head_dim and the query-head group select. Each is built in
// a translation unit of its own (inst/prefill_*.hip over prefill_launch.h).
int prefill_launch_f32(const PrefillParams& p, int max_e, int head_dim, int group, hipStream_t stream);
int prefill_launch_bf16(const PrefillParams& p, int max_e, int head_dim, int group, hipStream_t stream);
int prefill_launch_f16(const PrefillParams& p, int max_e, int head_dim, int group, hipStream_t stream);
int prefill_launch_bf16_fp8(const PrefillParams& p, int max_e, int head_dim, int group, hipStream_t stream);
int prefill_launch_f16_fp8(const PrefillParams& p, int max_e, int head_dim, int group, hipStream_t stream);

}  // namespace pf
}  // namespace msgl
