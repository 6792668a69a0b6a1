// Ragged chunked-prefill attention for gfx950, one launch per packed batch.
//
// Semantics: attention/base.py:85-105 (_forward_prefill): request i's E_i
// extend queries q[q_indptr[i] : q_indptr[i+1]] attend to its first L_i =
// P_i + E_i tokens of KV (the cached prefix plus this step's rows, already
// stored in the pool) with MLX's bottom-right causal mask
// (docs/04-attention.md:35-36): query t sees key j iff j <= P_i + t. With
// E_i == 1 the mask keeps every key (attention/base.py:103, mask=None).
//
// Design (flash-attention forward, MFMA throughout):
//  * Workgroup = (request, kv head, block of query rows); query rows are
//    (token, grouped head) pairs, so the G query heads of one kv head share
//    every K/V tile (GQA). 4 wavefronts x 16 query rows each.
//  * Per iteration a 32-key tile is gathered from the pool through the slot
//    indices into LDS: K row-major (A operand of S^T = K Q^T), V transposed
//    (B operand of O = P V) so the key dimension is contiguous per lane.
//  * S^T = K Q^T with v_mfma_f32_16x16x32_{bf16,f16}: lane (query col l%16,
//    key group l/16) holds 4 keys of each 16-key tile, which is exactly the A
//    operand layout P needs for O += P V (converted in registers, no shuffle).
//    fp32 uses v_mfma_f32_16x16x4f32 and row-major V.
//  * Online softmax per query row in the exp2 domain; row max/sum across the 4
//    key groups by two xor shuffles; per-row rescale factors are broadcast to
//    the accumulator layout with ds_bpermute.
//  * Causal tiles past a block's last visible key are never loaded.
#include "msgl_common.h"

namespace msgl {

namespace {

constexpr float kLog2eP = 1.4426950408889634f;
constexpr int KT = 32;      // keys per iteration
constexpr int NWAVE = 4;    // wavefronts per workgroup
constexpr int QROWS = 16;   // query rows per wavefront

struct PrefillParams {
  const void* q;
  const void* k_pool;
  const void* v_pool;
  const int32_t* q_indptr;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* seq_lens;
  void* out;
  int64_t num_slots;
  int hq, hkv, page_size;
  float scale_log2;
};

__device__ __forceinline__ int64_t kv_slot(const PrefillParams& p, int start, int tok) {
  int64_t s;
  if (p.page_size == 1) {
    s = p.kv_indices[start + tok];
  } else {
    s = (int64_t)p.kv_indices[start + tok / p.page_size] * p.page_size + tok % p.page_size;
  }
  return (s >= 0 && s < p.num_slots) ? s : 0;
}

template <typename T>
struct PF;

// 16-bit types: K row-major [KT][D+8], V transposed [D][KT+4] in LDS.
template <typename T>
struct PF16 {
  static constexpr int VEC = 8;
  template <int D>
  static constexpr int k_stride() { return D + 8; }       // elements
  static constexpr int vt_stride() { return KT + 4; }     // elements
  template <int D>
  static constexpr int lds_bytes() { return (KT * (D + 8) + D * (KT + 4)) * 2; }
};

template <>
struct PF<bf16_t> : PF16<bf16_t> {
  __device__ __forceinline__ static f32x4 mma(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack2(float lo, float hi) {
    return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
  }
};

template <>
struct PF<f16_t> : PF16<f16_t> {
  __device__ __forceinline__ static f32x4 mma(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
  __device__ __forceinline__ static uint32_t pack2(float lo, float hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
  }
};

template <>
struct PF<float> {
  static constexpr int VEC = 4;
  template <int D>
  static constexpr int k_stride() { return D + 4; }
  template <int D>
  static constexpr int lds_bytes() { return 2 * KT * (D + 4) * 4; }
};

template <typename T, int D, int G>
__global__ __launch_bounds__(256) void prefill_kernel(PrefillParams p) {
  constexpr int ES = sizeof(T);
  constexpr int VEC = PF<T>::VEC;
  constexpr int ROWS = NWAVE * QROWS;   // query rows per workgroup
  static_assert(ROWS % G == 0, "group must divide the row block");
  constexpr int BQ = ROWS / G;          // query tokens per workgroup
  constexpr int NDT = D / 16;           // 16-wide output column tiles
  constexpr int KS = PF<T>::template k_stride<D>();

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  T* Ks = reinterpret_cast<T*>(smem);                 // [KT][KS]
  T* Vs = Ks + KT * KS;                               // 16-bit: Vt[D][KT+4]; fp32: V[KT][KS]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;   // S^T column = query row within the wave tile
  const int grp = lane >> 4;   // key group

  const int req = blockIdx.y / p.hkv;
  const int kvh = blockIdx.y % p.hkv;
  const int q0 = p.q_indptr[req];
  const int E = p.q_indptr[req + 1] - q0;
  const int qb = blockIdx.x * BQ;
  if (qb >= E) return;
  const int kv_start = p.kv_indptr[req];
  const int Lkv = p.seq_lens ? p.seq_lens[req] : (p.kv_indptr[req + 1] - kv_start);
  const int P = Lkv - E;
  const int kv_end = min(Lkv, P + min(E, qb + BQ));  // keys this block can see

  // this lane's query row (as S^T column) and its token (clamped into range so
  // every row has at least key 0 visible; rows past E are computed, not stored)
  const int my_row = wave * QROWS + col;
  const int my_tok = min(qb + my_row / G, E - 1);
  const int my_limit = P + my_tok;  // last visible key
  const int my_head = kvh * G + my_row % G;

  // Q fragment (B operand): d = 4*VEC*j + VEC*grp + e
  constexpr int NQF = D / (4 * VEC);
  u32x4 qf[NQF];
  {
    const uint8_t* qrow = reinterpret_cast<const uint8_t*>(p.q) + ((int64_t)(q0 + my_tok) * p.hq + my_head) * D * ES;
#pragma unroll
    for (int j = 0; j < NQF; ++j) qf[j] = ld16(qrow + (4 * VEC * j + VEC * grp) * ES);
  }

  f32x4 acc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;  // per query row (this lane's column)

  const uint8_t* kp = reinterpret_cast<const uint8_t*>(p.k_pool);
  const uint8_t* vp = reinterpret_cast<const uint8_t*>(p.v_pool);
  const int64_t row_stride = (int64_t)p.hkv * D * ES;
  const int64_t head_off = (int64_t)kvh * D * ES;

  for (int kt0 = 0; kt0 < kv_end; kt0 += KT) {
    // ---- gather the key tile into LDS ----
    __syncthreads();
    constexpr int CPR = D / VEC;  // 16-byte chunks per row
    for (int c = tid; c < KT * CPR; c += 256) {
      const int key = c / CPR, ch = c % CPR;
      const int j = kt0 + key;
      u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
      if (j < kv_end) {
        const int64_t s = kv_slot(p, kv_start, j);
        kv = ld16(kp + s * row_stride + head_off + ch * 16);
        vv = ld16(vp + s * row_stride + head_off + ch * 16);
      }
      *reinterpret_cast<u32x4*>(Ks + key * KS + ch * VEC) = kv;
      if constexpr (ES == 2) {
        constexpr int VTS = KT + 4;
        const uint16_t* e16 = reinterpret_cast<const uint16_t*>(&vv);
#pragma unroll
        for (int e = 0; e < 8; ++e) reinterpret_cast<uint16_t*>(Vs)[(ch * 8 + e) * VTS + key] = e16[e];
      } else {
        *reinterpret_cast<u32x4*>(Vs + key * KS + ch * VEC) = vv;
      }
    }
    __syncthreads();

    // ---- S^T = K Q^T for two 16-key tiles ----
    f32x4 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
      const T* krow = Ks + (kt * 16 + col) * KS;
#pragma unroll
      for (int j = 0; j < NQF; ++j) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(krow + 4 * VEC * j + VEC * grp);
        if constexpr (ES == 2) {
          s[kt] = PF<T>::mma(a, qf[j], s[kt]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[e]), __uint_as_float(qf[j][e]), s[kt], 0,
                                                         0, 0);
        }
      }
    }
    // ---- online softmax for this lane's query row ----
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
    const float m_new = fmaxf(m_run, mloc);
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

    // ---- rescale accumulators: row 4*grp+i takes alpha of column 4*grp+i ----
    float arow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, 4 * grp + i);
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][i] *= arow[i];

    // ---- O += P V ----
    if constexpr (ES == 2) {
      // A operand: slot (grp, e<4) = key 4*grp+e of tile 0, (grp, e>=4) = key 16+4*grp+e-4
      u32x4 pa;
      pa[0] = PF<T>::pack2(pr[0][0], pr[0][1]);
      pa[1] = PF<T>::pack2(pr[0][2], pr[0][3]);
      pa[2] = PF<T>::pack2(pr[1][0], pr[1][1]);
      pa[3] = PF<T>::pack2(pr[1][2], pr[1][3]);
      constexpr int VTS = KT + 4;
#pragma unroll
      for (int t = 0; t < NDT; ++t) {
        const uint16_t* vt = reinterpret_cast<const uint16_t*>(Vs) + (t * 16 + col) * VTS;
        const uint2 lo = *reinterpret_cast<const uint2*>(vt + 4 * grp);
        const uint2 hi = *reinterpret_cast<const uint2*>(vt + 16 + 4 * grp);
        const u32x4 b = {lo.x, lo.y, hi.x, hi.y};
        acc[t] = PF<T>::mma(pa, b, acc[t]);
      }
    } else {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float* vrow = reinterpret_cast<const float*>(Vs) + (kt * 16 + 4 * grp + i) * KS;
#pragma unroll
          for (int t = 0; t < NDT; ++t)
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[kt][i], vrow[t * 16 + col], acc[t], 0, 0, 0);
        }
    }
  }

  // ---- normalise and store: acc row 4*grp+i is query row wave*16 + 4*grp + i ----
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  const float inv = 1.f / l_run;
  T* out = reinterpret_cast<T*>(p.out);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = wave * QROWS + 4 * grp + i;
    const int tok = qb + row / G;
    const float rinv = __shfl(inv, 4 * grp + i);
    if (tok < E) {
      T* orow = out + ((int64_t)(q0 + tok) * p.hq + kvh * G + row % G) * D;
#pragma unroll
      for (int t = 0; t < NDT; ++t) orow[t * 16 + col] = from_f32<T>(acc[t][i] * rinv);
    }
  }
}

template <typename T, int D, int G>
int launch_prefill(const PrefillParams& p, int num_reqs, int max_extend_len, hipStream_t stream) {
  constexpr int BQ = NWAVE * QROWS / G;
  const int qblocks = (max_extend_len + BQ - 1) / BQ;
  const size_t lds = PF<T>::template lds_bytes<D>();
  hipLaunchKernelGGL((prefill_kernel<T, D, G>), dim3(qblocks, num_reqs * p.hkv), dim3(256), lds, stream, p);
  MSGL_CHECK_LAUNCH("msgl_prefill_ragged");
  return MSGL_OK;
}

template <typename T, int D>
int prefill_group(const PrefillParams& p, int num_reqs, int max_e, int group, hipStream_t s) {
  switch (group) {
    case 1: return launch_prefill<T, D, 1>(p, num_reqs, max_e, s);
    case 2: return launch_prefill<T, D, 2>(p, num_reqs, max_e, s);
    case 4: return launch_prefill<T, D, 4>(p, num_reqs, max_e, s);
    case 8: return launch_prefill<T, D, 8>(p, num_reqs, max_e, s);
    case 16: return launch_prefill<T, D, 16>(p, num_reqs, max_e, s);
    default:
      set_error("msgl_prefill_ragged: Hq/Hkv = %d not built (1, 2, 4, 8, 16)", group);
      return MSGL_ERR_UNSUPPORTED;
  }
}

template <typename T>
int prefill_dim(const PrefillParams& p, int num_reqs, int max_e, int head_dim, int group, hipStream_t s) {
  switch (head_dim) {
    case 64: return prefill_group<T, 64>(p, num_reqs, max_e, group, s);
    case 128: return prefill_group<T, 128>(p, num_reqs, max_e, group, s);
    case 256: return prefill_group<T, 256>(p, num_reqs, max_e, group, s);
    default:
      set_error("msgl_prefill_ragged: head_dim %d not built (64, 128, 256)", head_dim);
      return MSGL_ERR_UNSUPPORTED;
  }
}

}  // namespace
}  // namespace msgl

extern "C" int msgl_prefill_ragged(const void* q, const void* k_pool, const void* v_pool, const int32_t* q_indptr,
                                   const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                                   int32_t num_reqs, int32_t max_extend_len, int32_t num_qo_heads,
                                   int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int64_t num_slots,
                                   int32_t dtype, float scale, void* out, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(num_reqs >= 0 && max_extend_len >= 0, "msgl_prefill_ragged: sizes must be >= 0");
  if (num_reqs == 0 || max_extend_len == 0) return MSGL_OK;
  MSGL_CHECK_ARG(num_qo_heads > 0 && num_kv_heads > 0 && head_dim > 0, "msgl_prefill_ragged: sizes must be > 0");
  MSGL_CHECK_ARG(num_qo_heads % num_kv_heads == 0, "msgl_prefill_ragged: Hq (%d) must be a multiple of Hkv (%d)",
                 num_qo_heads, num_kv_heads);
  MSGL_CHECK_ARG(page_size >= 1, "msgl_prefill_ragged: page_size must be >= 1");
  MSGL_CHECK_ARG(page_size == 1 || seq_lens != nullptr, "msgl_prefill_ragged: page_size > 1 needs seq_lens");
  MSGL_CHECK_ARG(num_slots > 0 && num_slots <= ((int64_t)1 << 31) - 1,
                 "msgl_prefill_ragged: num_slots must be in [1, 2^31)");
  MSGL_CHECK_ARG((int64_t)num_reqs * num_kv_heads <= 65535, "msgl_prefill_ragged: num_reqs * Hkv must be <= 65535");
  MSGL_CHECK_ARG(q && k_pool && v_pool && q_indptr && kv_indptr && kv_indices && out,
                 "msgl_prefill_ragged: null pointer");
  MSGL_CHECK_ARG(((uintptr_t)q | (uintptr_t)k_pool | (uintptr_t)v_pool | (uintptr_t)out) % 16 == 0,
                 "msgl_prefill_ragged: q, pools and out must be 16-byte aligned");
  if (dtype_size(dtype) == 0) {
    set_error("msgl_prefill_ragged: unknown dtype %d", dtype);
    return MSGL_ERR_UNSUPPORTED;
  }
  PrefillParams p;
  p.q = q;
  p.k_pool = k_pool;
  p.v_pool = v_pool;
  p.q_indptr = q_indptr;
  p.kv_indptr = kv_indptr;
  p.kv_indices = kv_indices;
  p.seq_lens = seq_lens;
  p.out = out;
  p.num_slots = num_slots;
  p.hq = num_qo_heads;
  p.hkv = num_kv_heads;
  p.page_size = page_size;
  p.scale_log2 = scale * kLog2eP;
  const int group = num_qo_heads / num_kv_heads;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MSGL_F32: return prefill_dim<float>(p, num_reqs, max_extend_len, head_dim, group, s);
    case MSGL_BF16: return prefill_dim<bf16_t>(p, num_reqs, max_extend_len, head_dim, group, s);
    case MSGL_F16: return prefill_dim<f16_t>(p, num_reqs, max_extend_len, head_dim, group, s);
  }
  return MSGL_ERR_UNSUPPORTED;
}
