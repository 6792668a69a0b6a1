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
#include <algorithm>
#include <type_traits>

#include "msgl_common.h"

namespace msgl {

namespace {

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
  int* plan_count;   // its length
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

__device__ __forceinline__ int64_t kv_slot(const PrefillParams& p, int start, int tok) {
  int64_t s;
  if (p.page_size == 1) {
    s = p.kv_indices[start + tok];
  } else {
    s = (int64_t)p.kv_indices[start + tok / p.page_size] * p.page_size + tok % p.page_size;
  }
  return (s >= 0 && s < p.num_slots) ? s : 0;
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

#define MSGL_LDS __attribute__((address_space(3)))
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

// 16 bytes per lane from global memory into LDS at m0 + 16 * lane. Issued as
// inline assembly so the compiler does not drain every outstanding transfer
// before the next LDS read; the caller waits with vm_wait.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds_addr) {
  // m0 is reserved by the compiler, so it cannot be listed as clobbered; the
  // kernels using this helper have no other m0 user.
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_addr) : "memory");
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

// 4 bytes per active lane from global memory into LDS at m0 + 4 * lane.
__device__ __forceinline__ void dma4(const void* g, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds_addr) : "memory");
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

template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

// v_mfma_f32_32x32x16_{bf16,f16}: A [32 x 16] lane l holds row l%32, k
// 8*(l/32)..+7; B [16 x 32] lane l holds column l%32, the same k; C [32 x 32]
// lane l holds column l%32, rows 8*(i/4) + 4*(l/32) + i%4 for i = 0..15.
// (The 16x16x32 form runs at half this rate on gfx950.)
template <typename T>
struct MMA32;
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
__global__ __launch_bounds__(THREADS16) __attribute__((amdgpu_waves_per_eu(G16<D>::WAVES))) void prefill16_kernel(
    PrefillParams p) {
  constexpr bool Q8 = std::is_same<KV, fp8e4m3>::value;
  using Geo = G16<D, (int)sizeof(KV)>;
  constexpr int ROWS = Geo::ROWS;
  static_assert(ROWS % G == 0, "group must divide the row block");
  constexpr int BQ = ROWS / G;  // query tokens per workgroup
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
  if ((int)blockIdx.x >= *p.plan_count) return;
  const int4 item = p.plan[2 * blockIdx.x];
  const int4 geo = p.plan[2 * blockIdx.x + 1];  // the request's geometry, loaded with the item
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
  const int my_tok = min(qb + my_row / G, E - 1);
  const int limit = P + my_tok;
  const int lim_lo = __builtin_amdgcn_readfirstlane(limit);  // the wavefront's first row (lane 0)
  // Q fragment (B operand of S^T = K Q^T): d = 16j + 8h .. +7
  u32x4 qf[NQF];
  {
    const uint8_t* qrow =
        reinterpret_cast<const uint8_t*>(p.q) + ((int64_t)(q0 + my_tok) * p.hq + kvh * G + my_row % G) * D * 2;
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
        sv[k] = p.kv_indices[kv_start + (p.page_size == 1 ? tok : tok / p.page_size)];
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
    scores(0, s_cur);
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
      if (t + 2 < ntiles) issue(st2);
      const int kbase = w0 + t * KT;
      // A (past the last tile, scores reads a stage whose transfers have all landed; unused)
      f32x16 s_next;
      float x[16];
      float ksc[16];  // fp8: tile t's K scales
      if constexpr (Q8) tile_scales(st, 0, ksc);
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
    pv((ntiles - 1) % NS, pa_prev);
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
      if (tok < E) {
        T* orow = out + ((int64_t)(q0 + tok) * p.hq + kvh * G + row % G) * D;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) orow[32 * dt + rl] = from_f32<T>(acc[dt][i] * rinv);
      }
    }
  } else {
    const int64_t base = (int64_t)split * p.num_tokens;
    if (h == 0) {
      const int tok = qb + my_row / G;
      if (tok < E && q0 + tok < p.num_tokens)
        p.part_ml[(base + q0 + tok) * p.hq + kvh * G + my_row % G] = make_float2(m_run, l_row);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = wave * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
      const int tok = qb + row / G;
      if (tok < E && q0 + tok < p.num_tokens) {  // the workspace holds num_tokens rows
        float* orow = p.part_o + ((base + q0 + tok) * p.hq + kvh * G + row % G) * D;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) orow[32 * dt + rl] = acc[dt][i];
      }
    }
  }
}

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

// Combines the chunks of every query row whose block was split: one thread
// per 4 output columns of one (token, head). The plan kernel left each token's
// chunk count in merge_n, so the (m, l) and O partials of up to kMergeUnroll
// chunks are loaded at once, with no lookup in front of them.
constexpr int kMergeUnroll = 4;

template <typename T, int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillParams p) {
  constexpr int TPH = D / 4;
  constexpr int HPB = 256 / TPH;
  const int tk = blockIdx.x;
  const int n = p.merge_n[tk];
  if (n <= 1) return;  // written by the attention kernel (or not a token of any request)
  const int h = blockIdx.y * HPB + threadIdx.x / TPH;
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

// ---------------------------------------------------------------------------
// fp32: one pass per block, register-staged gather
// ---------------------------------------------------------------------------
constexpr int QROWS32 = 16;  // query rows per wavefront

template <int D>
struct G32 {
  static constexpr int KS = D + 4;  // padded row stride (floats)
  static constexpr int BUF_BYTES = 2 * KT * KS * 4;
  static constexpr int NBUF = 2 * BUF_BYTES <= 65536 ? 2 : 1;
  static constexpr int LDS_BYTES = NBUF * BUF_BYTES;
};

template <int D, int G>
__global__ __launch_bounds__(256) void prefill_f32_kernel(PrefillParams p) {
  constexpr int ROWS = NWAVE * QROWS32;
  static_assert(ROWS % G == 0, "group must divide the row block");
  constexpr int BQ = ROWS / G;
  constexpr int NDT = D / 16;
  constexpr int KS = G32<D>::KS;
  constexpr int BUF_BYTES = G32<D>::BUF_BYTES;
  constexpr int NBUF = G32<D>::NBUF;

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;
  const int grp = lane >> 4;

  const int req = blockIdx.y / p.hkv;
  const int kvh = blockIdx.y % p.hkv;
  const int q0 = p.q_indptr[req];
  const int E = p.q_indptr[req + 1] - q0;
  const int qb = blockIdx.x * BQ;
  if (qb >= E) return;
  const int kv_start = p.kv_indptr[req];
  const int Lkv = p.seq_lens ? p.seq_lens[req] : (p.kv_indptr[req + 1] - kv_start);
  const int P = Lkv - E;
  const int kv_end = block_kv_end(Lkv, E, qb, BQ);

  const int my_row = wave * QROWS32 + col;
  const int my_tok = min(qb + my_row / G, E - 1);
  const int my_limit = P + my_tok;
  const int my_head = kvh * G + my_row % G;

  // Q fragment (B operand of 16x16x4): d = 16*j + 4*grp + e
  constexpr int NQF = D / 16;
  u32x4 qf[NQF];
  {
    const uint8_t* qrow = reinterpret_cast<const uint8_t*>(p.q) + ((int64_t)(q0 + my_tok) * p.hq + my_head) * D * 4;
#pragma unroll
    for (int j = 0; j < NQF; ++j) qf[j] = ld16(qrow + (16 * j + 4 * grp) * 4);
  }

  f32x4 acc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  const uint8_t* kp = reinterpret_cast<const uint8_t*>(p.k_pool);
  const uint8_t* vp = reinterpret_cast<const uint8_t*>(p.v_pool);
  const int64_t row_stride = (int64_t)p.hkv * D * 4;
  const int64_t head_off = (int64_t)kvh * D * 4;

  // slots two tiles ahead, rows one tile ahead (registers), compute from LDS
  constexpr int CPR = D / 4;
  constexpr int CH = KT * CPR / 256;
  static_assert((KT * CPR) % 256 == 0, "a tile must split evenly over 256 threads");
  int nslot[CH];
  u32x4 kreg[CH], vreg[CH];
  auto slots_for = [&](int kt0) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int j = kt0 + (tid + 256 * i) / CPR;
      nslot[i] = j < kv_end ? (int)kv_slot(p, kv_start, j) : -1;
    }
  };
  auto gload = [&]() {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int ch = (tid + 256 * i) % CPR;
      if (nslot[i] >= 0) {
        const int64_t off = (int64_t)nslot[i] * row_stride + head_off + ch * 16;
        kreg[i] = ld16(kp + off);
        vreg[i] = ld16(vp + off);
      } else {
        kreg[i] = u32x4{0u, 0u, 0u, 0u};
        vreg[i] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto lstore = [&](int buf) {
    float* Kb = reinterpret_cast<float*>(smem + buf * BUF_BYTES);
    float* Vb = Kb + KT * KS;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int key = (tid + 256 * i) / CPR, ch = (tid + 256 * i) % CPR;
      *reinterpret_cast<u32x4*>(Kb + key * KS + ch * 4) = kreg[i];
      *reinterpret_cast<u32x4*>(Vb + key * KS + ch * 4) = vreg[i];
    }
  };
  slots_for(0);
  gload();
  lstore(0);
  slots_for(KT);
  __syncthreads();

  int buf = 0;
  for (int kt0 = 0; kt0 < kv_end; kt0 += KT) {
    const bool more = kt0 + KT < kv_end;
    if (more) {
      gload();
      slots_for(kt0 + 2 * KT);
    }
    const float* Ks = reinterpret_cast<const float*>(smem + buf * BUF_BYTES);
    const float* Vs = Ks + KT * KS;

    f32x4 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
      const float* krow = Ks + (kt * 16 + col) * KS;
#pragma unroll
      for (int j = 0; j < NQF; ++j) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(krow + 16 * j + 4 * grp);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[e]), __uint_as_float(qf[j][e]), s[kt], 0, 0,
                                                       0);
      }
    }
    float x[2][4];
    float mloc = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kt0 + kt * 16 + 4 * grp + i;
        const bool vis = key <= my_limit && key < kv_end;
        x[kt][i] = vis ? s[kt][i] * p.scale_log2 : -INFINITY;
        mloc = fmaxf(mloc, x[kt][i]);
      }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    const float m_new = fmaxf(m_run, mloc);  // key 0 is visible to every row: finite from the first tile
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float pr[2][4];
    float lsum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[kt][i] = __builtin_amdgcn_exp2f(x[kt][i] - m_new);
        lsum += pr[kt][i];
      }
    l_run = l_run * alpha + lsum;
    m_run = m_new;

    float arow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, 4 * grp + i);
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][i] *= arow[i];

#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float* vrow = Vs + (kt * 16 + 4 * grp + i) * KS;
#pragma unroll
        for (int t = 0; t < NDT; ++t)
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[kt][i], vrow[t * 16 + col], acc[t], 0, 0, 0);
      }
    if constexpr (NBUF == 2) {
      if (more) lstore(buf ^ 1);  // the other buffer was last read before the previous barrier
      __syncthreads();
      buf ^= 1;
    } else {
      __syncthreads();
      if (more) lstore(0);
      __syncthreads();
    }
  }

  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  const float inv = 1.f / l_run;
  float* out = reinterpret_cast<float*>(p.out);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = wave * QROWS32 + 4 * grp + i;
    const int tok = qb + row / G;
    const float rinv = __shfl(inv, 4 * grp + i);
    if (tok < E) {
      float* orow = out + ((int64_t)(q0 + tok) * p.hq + kvh * G + row % G) * D;
#pragma unroll
      for (int t = 0; t < NDT; ++t) orow[t * 16 + col] = acc[t][i] * rinv;
    }
  }
}

// ---------------------------------------------------------------------------
// launch
// ---------------------------------------------------------------------------
int tokens_per_block16(int group) { return NWAVE16 * 32 / group; }

template <typename T, typename KV, int D, int G>
int launch16(PrefillParams p, int max_e, hipStream_t stream) {
  using Geo = G16<D, (int)sizeof(KV)>;
  constexpr int BQ = Geo::ROWS / G;
  p.nqb = (max_e + BQ - 1) / BQ;
  const int64_t items = (int64_t)p.hkv * p.num_reqs * p.splits * p.nqb;
  p.items = (int)items;
  if (items > (int64_t)p.plan_capacity) {
    set_error("msgl_prefill_ragged: workspace holds %d work items, %lld needed", p.plan_capacity, (long long)items);
    return MSGL_ERR_WORKSPACE;
  }
  if (p.mode != kRunPlanned) {
    hipLaunchKernelGGL(prefill_plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, p, BQ);
    MSGL_CHECK_LAUNCH("msgl_prefill_ragged (plan)");
  }
  if (p.mode == kPlanOnly) return MSGL_OK;
  const int grid = (int)items;
  static bool attr_set = false;  // per process; the attribute is per function
  if (Geo::LDS_BYTES > 65536 && !attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill16_kernel<T, KV, D, G>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, Geo::LDS_BYTES) != hipSuccess) {
      set_error("msgl_prefill_ragged: cannot raise the LDS limit to %d bytes", Geo::LDS_BYTES);
      return MSGL_ERR_HIP;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL((prefill16_kernel<T, KV, D, G>), dim3(grid), dim3(THREADS16), Geo::LDS_BYTES, stream, p);
  MSGL_CHECK_LAUNCH("msgl_prefill_ragged");
  if (p.splits > 1) {
    constexpr int HPB = 256 / (D / 4);
    hipLaunchKernelGGL((prefill_merge_kernel<T, D>), dim3(p.num_tokens, (p.hq + HPB - 1) / HPB), dim3(256), 0,
                       stream, p);
    MSGL_CHECK_LAUNCH("msgl_prefill_ragged (merge)");
  }
  return MSGL_OK;
}

template <int D, int G>
int launch32(const PrefillParams& p, int max_e, hipStream_t stream) {
  constexpr int BQ = NWAVE * QROWS32 / G;
  const int qblocks = (max_e + BQ - 1) / BQ;
  hipLaunchKernelGGL((prefill_f32_kernel<D, G>), dim3(qblocks, p.num_reqs * p.hkv), dim3(256), G32<D>::LDS_BYTES,
                     stream, p);
  MSGL_CHECK_LAUNCH("msgl_prefill_ragged");
  return MSGL_OK;
}

template <typename T, typename KV, int D, int G>
int launch_prefill(const PrefillParams& p, int max_e, hipStream_t s) {
  if constexpr (sizeof(T) == 4) {
    if (p.mode == kPlanOnly) return MSGL_OK;  // the fp32 path has no work list
    return launch32<D, G>(p, max_e, s);
  } else {
    return launch16<T, KV, D, G>(p, max_e, s);
  }
}

template <typename T, typename KV, int D>
int prefill_group(const PrefillParams& p, int max_e, int group, hipStream_t s) {
  switch (group) {
    case 1: return launch_prefill<T, KV, D, 1>(p, max_e, s);
    case 2: return launch_prefill<T, KV, D, 2>(p, max_e, s);
    case 4: return launch_prefill<T, KV, D, 4>(p, max_e, s);
    case 8: return launch_prefill<T, KV, D, 8>(p, max_e, s);
    case 16: return launch_prefill<T, KV, D, 16>(p, max_e, s);
    default:
      set_error("msgl_prefill_ragged: Hq/Hkv = %d not built (1, 2, 4, 8, 16)", group);
      return MSGL_ERR_UNSUPPORTED;
  }
}

template <typename T, typename KV = T>
int prefill_dim(const PrefillParams& p, int max_e, int head_dim, int group, hipStream_t s) {
  switch (head_dim) {
    case 64: return prefill_group<T, KV, 64>(p, max_e, group, s);
    case 128: return prefill_group<T, KV, 128>(p, max_e, group, s);
    case 256: return prefill_group<T, KV, 256>(p, max_e, group, s);
    default:
      set_error("msgl_prefill_ragged: head_dim %d not built (64, 128, 256)", head_dim);
      return MSGL_ERR_UNSUPPORTED;
  }
}

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

namespace {
int prefill_impl(const char* fn, int mode, const void* q, const void* k_pool, const void* v_pool,
                 const float* kv_scale, const int32_t* q_indptr, const int32_t* kv_indptr, const int32_t* kv_indices,
                 const int32_t* seq_lens, int32_t num_reqs, int32_t num_tokens, int32_t max_extend_len,
                 int32_t max_seq_len, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                 int64_t num_slots, int32_t dtype, float scale, int32_t max_splits, void* out, void* workspace,
                 int64_t workspace_bytes, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(num_reqs >= 0 && num_tokens >= 0 && max_extend_len >= 0, "%s: sizes must be >= 0", fn);
  if (num_reqs == 0 || max_extend_len == 0 || num_tokens == 0) return MSGL_OK;
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
  PrefillParams p;
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
  const int group = num_qo_heads / num_kv_heads;
  hipStream_t s = (hipStream_t)stream;
  if (kv_scale != nullptr) {  // fp8 e4m3 pools with per-(slot, kv head) scales
    switch (dtype) {
      case MSGL_BF16: return prefill_dim<bf16_t, fp8e4m3>(p, max_extend_len, head_dim, group, s);
      case MSGL_F16: return prefill_dim<f16_t, fp8e4m3>(p, max_extend_len, head_dim, group, s);
    }
    set_error("%s: fp8 pools take bf16 or fp16 queries (dtype %d)", fn, dtype);
    return MSGL_ERR_UNSUPPORTED;
  }
  switch (dtype) {
    case MSGL_F32: return prefill_dim<float>(p, max_extend_len, head_dim, group, s);
    case MSGL_BF16: return prefill_dim<bf16_t>(p, max_extend_len, head_dim, group, s);
    case MSGL_F16: return prefill_dim<f16_t>(p, max_extend_len, head_dim, group, s);
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
