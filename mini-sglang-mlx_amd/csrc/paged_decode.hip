// Paged decode attention for gfx950 (one query token per request).
//
// Semantics: attention/naive.py:50-60 (gather by page table + masked SDPA) and
// attention/metal.py:112-131 (paged_decode_attention over CSR indices):
//   o[b, h] = softmax_j(scale * q[b,h] . K[slot_b(j), h/G]) V[slot_b(j), h/G],  j < L_b
//
// Design (MI355X-first, not a translation of the Metal kernel):
//  * Work unit = one wavefront per (request b, split s, kv head). A workgroup
//    holds the Hkv wavefronts of one (b, s), so the rows of a token slot
//    (Hkv * D contiguous elements) are read by neighbouring waves together.
//  * Split-K: request b is cut into n_b <= max_splits chunks of a multiple of
//    16 tokens (>= kMinChunk), decided on the device from L_b alone, so the
//    launch needs no host-side lengths. Single-chunk requests write the final
//    row; others write fp32 partials (acc, m, l) merged by a second kernel.
//  * Q.K^T runs on the matrix cores: v_mfma_f32_16x16x32_{bf16,f16} (or
//    16x16x4 f32), A = the G query heads of the kv head (rows >= G are zero),
//    B = 16 K rows straight from the pool (one 16-byte load per lane per MFMA,
//    no conversion). Output: lane (t = l%16, row group l/16) holds 4 scores.
//  * Online softmax in the exp2 domain (scale*log2(e) folded into the score)
//    with the tile max over the 16 tokens from 4 DPP steps inside a 16-lane row.
//  * P.V on the VALU: lane (token sub-row, 16-byte d chunk) accumulates
//    G x (16/sizeof T) fp32 outputs; P and the rescale factors go through a
//    1 KiB per-wave LDS tile. Partial sums over token sub-rows are folded once
//    per work unit.
//  * Slot indices: one coalesced load of 64 slots per 64 tokens, handed to the
//    lanes that need them with ds_bpermute; out-of-range slots are clamped.
#include "msgl_common.h"

namespace msgl {

constexpr int kMinChunk = 64;   // smallest split-K chunk (tokens)
constexpr int kMaxSplits = 64;  // merge kernel's LDS bound
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

// Split geometry of one request; identical in the decode and merge kernels.
__device__ __forceinline__ void split_geometry(int L, int max_splits, int& n, int& chunk) {
  if (L <= 0) {
    n = 0;
    chunk = 0;
    return;
  }
  int want = (L + kMinChunk - 1) / kMinChunk;
  if (want > max_splits) want = max_splits;
  chunk = (L + want - 1) / want;
  chunk = (chunk + 15) & ~15;
  n = (L + chunk - 1) / chunk;
}

__device__ __forceinline__ int64_t slot_of(const int32_t* __restrict__ kv_indices, int start, int tok, int page_size,
                                           int64_t num_slots) {
  int64_t s;
  if (page_size == 1) {
    s = kv_indices[start + tok];
  } else {
    s = (int64_t)kv_indices[start + tok / page_size] * page_size + tok % page_size;
  }
  return (s >= 0 && s < num_slots) ? s : 0;
}

struct DecodeParams {
  const void* q;
  const void* k_pool;
  const void* v_pool;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* seq_lens;
  void* out;
  float* part_o;   // [B, S, Hq, D]
  float* part_ml;  // [B, S, Hq, 2]
  int64_t num_slots;
  int hq, hkv, page_size, max_splits;
  float scale_log2;
};

// LDS per wavefront: P tile [16 tokens][16 rows] + alpha[16] + (m, l)[16 rows].
constexpr int kLdsPerWave = 16 * 16 + 16 + 32;

template <typename T, int D, int G>
__global__ __launch_bounds__(512) void paged_decode_kernel(DecodeParams p) {
  constexpr int VEC = QK<T>::VEC;   // elements per 16-byte chunk
  constexpr int ES = sizeof(T);
  constexpr int KCHUNK = 4 * VEC;   // d covered by one K load across the 4 row groups
  constexpr int NLK = D / KCHUNK;   // K loads per lane per 16-token tile
  constexpr int LPR = D / VEC;      // lanes per V row
  constexpr int R = 64 / LPR;       // V rows per wave load
  constexpr int NLV = 16 / R;       // V loads per lane per tile
  static_assert(D % KCHUNK == 0 && 64 % LPR == 0 && 16 % R == 0, "unsupported head_dim");
  static_assert(G >= 1 && G <= 16, "unsupported group size");

  extern __shared__ float lds_all[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  float* lds = lds_all + wave * kLdsPerWave;
  float* P_lds = lds;              // [16][16]
  float* A_lds = lds + 256;        // [16]
  float* ML_lds = lds + 256 + 16;  // [16][2]

  const int b = blockIdx.y;
  const int split = blockIdx.x;
  int start, L;
  if (p.seq_lens) {
    start = p.kv_indptr[b];
    L = p.seq_lens[b];
  } else {
    start = p.kv_indptr[b];
    L = p.kv_indptr[b + 1] - start;
  }
  int n, chunk;
  split_geometry(L, p.max_splits, n, chunk);
  if (split >= n) {
    if (split == 0) {  // L == 0: defined zero output
      T* o = reinterpret_cast<T*>(p.out) + (int64_t)b * p.hq * D;
      for (int i = threadIdx.x; i < p.hq * D; i += blockDim.x) o[i] = from_f32<T>(0.f);
    }
    return;
  }
  const int t0 = split * chunk;
  const int t1 = min(L, t0 + chunk);

  const int r = lane & 15;  // MFMA column (token in tile) / A row
  const int g4 = lane >> 4;  // MFMA row group
  const int vc = lane % LPR;  // V: 16-byte chunk within the row
  const int vr = lane / LPR;  // V: token sub-row

  const uint8_t* kp = reinterpret_cast<const uint8_t*>(p.k_pool);
  const uint8_t* vp = reinterpret_cast<const uint8_t*>(p.v_pool);
  const int64_t row_stride = (int64_t)p.hkv * D * ES;  // bytes per slot

  for (int kvh = wave; kvh < p.hkv; kvh += nwaves) {
    // Q fragment: A operand, row r = query head kvh*G + r (zero when r >= G).
    u32x4 qa[NLK];
    {
      const uint8_t* qrow =
          reinterpret_cast<const uint8_t*>(p.q) + ((int64_t)b * p.hq + kvh * G + r) * D * ES + g4 * VEC * ES;
#pragma unroll
      for (int j = 0; j < NLK; ++j) {
        qa[j] = (r < G) ? ld16(qrow + j * KCHUNK * ES) : u32x4{0u, 0u, 0u, 0u};
      }
    }
    float m_run[4], l_run[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      m_run[i] = -INFINITY;
      l_run[i] = 0.f;
    }
    float acc[G][VEC];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[g][e] = 0.f;

    const int64_t head_off = (int64_t)kvh * D * ES;

    for (int tb = t0; tb < t1; tb += 64) {
      const int my_tok = tb + lane;
      const int64_t my_slot = (my_tok < t1) ? slot_of(p.kv_indices, start, my_tok, p.page_size, p.num_slots) : 0;
      const int my_slot32 = (int)my_slot;  // slots < 2^31 (checked on the host)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int tt = tb + 16 * k;
        if (tt >= t1) break;
        // ---- loads: K rows for the MFMA, V rows for the PV lanes ----
        const int ks = __shfl(my_slot32, 16 * k + r);
        u32x4 kb[NLK];
        {
          const uint8_t* krow = kp + (int64_t)ks * row_stride + head_off + g4 * VEC * ES;
#pragma unroll
          for (int j = 0; j < NLK; ++j) kb[j] = ld16(krow + j * KCHUNK * ES);
        }
        u32x4 vb[NLV];
#pragma unroll
        for (int i = 0; i < NLV; ++i) {
          const int tl = vr + R * i;
          const int vs = __shfl(my_slot32, 16 * k + tl);
          const u32x4 x = ld16(vp + (int64_t)vs * row_stride + head_off + vc * VEC * ES);
          vb[i] = (tt + tl < t1) ? x : u32x4{0u, 0u, 0u, 0u};
        }
        // ---- S = Q K^T on the matrix core ----
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NLK; ++j) s = QK<T>::step(qa[j], kb[j], s);
        // ---- online softmax (exp2 domain) ----
        const bool valid = (tt + r) < t1;
        float pr[4], al[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float x = valid ? s[i] * p.scale_log2 : -INFINITY;
          const float mt = row16_max(x);
          const float m_new = fmaxf(m_run[i], mt);
          al[i] = __builtin_amdgcn_exp2f(m_run[i] - m_new);
          pr[i] = __builtin_amdgcn_exp2f(x - m_new);
          l_run[i] = l_run[i] * al[i] + pr[i];
          m_run[i] = m_new;
        }
        wave_lds_sync();  // previous tile's LDS reads are done
        *reinterpret_cast<f32x4*>(P_lds + r * 16 + 4 * g4) = f32x4{pr[0], pr[1], pr[2], pr[3]};
        if (r == 0) *reinterpret_cast<f32x4*>(A_lds + 4 * g4) = f32x4{al[0], al[1], al[2], al[3]};
        wave_lds_sync();
        // ---- O = alpha * O + P V on the VALU ----
        float alpha[G];
#pragma unroll
        for (int g = 0; g < G; ++g) alpha[g] = A_lds[g];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[g][e] *= alpha[g];
#pragma unroll
        for (int i = 0; i < NLV; ++i) {
          const int tl = vr + R * i;
          float vf[VEC];
          Vec16<T>::to_f32(vb[i], vf);
          float pv[G];
#pragma unroll
          for (int g = 0; g < G; ++g) pv[g] = P_lds[tl * 16 + g];
#pragma unroll
          for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[g][e] = fmaf(pv[g], vf[e], acc[g][e]);
        }
      }
    }

    // ---- fold: l over the 16 token lanes, acc over the R token sub-rows ----
#pragma unroll
    for (int i = 0; i < 4; ++i) l_run[i] = row16_sum(l_run[i]);
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1)
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[g][e] += __shfl_xor(acc[g][e], off);
    wave_lds_sync();
    if (r == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ML_lds[(4 * g4 + i) * 2 + 0] = m_run[i];
        ML_lds[(4 * g4 + i) * 2 + 1] = l_run[i];
      }
    }
    wave_lds_sync();
    if (lane < LPR) {
      const int d0 = vc * VEC;
      if (n == 1) {
        T* o = reinterpret_cast<T*>(p.out) + ((int64_t)b * p.hq + kvh * G) * D + d0;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float inv = 1.f / ML_lds[g * 2 + 1];
          T tmp[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e) tmp[e] = from_f32<T>(acc[g][e] * inv);
          u32x4 packed;
          __builtin_memcpy(&packed, tmp, 16);
          st16(o + g * D, packed);
        }
      } else {
        const int64_t base = ((int64_t)b * p.max_splits + split) * p.hq + kvh * G;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float* po = p.part_o + (base + g) * D + d0;
#pragma unroll
          for (int e = 0; e < VEC; e += 4)
            *reinterpret_cast<f32x4*>(po + e) = f32x4{acc[g][e], acc[g][e + 1], acc[g][e + 2], acc[g][e + 3]};
          if (vc == 0) {
            p.part_ml[(base + g) * 2 + 0] = ML_lds[g * 2 + 0];
            p.part_ml[(base + g) * 2 + 1] = ML_lds[g * 2 + 1];
          }
        }
      }
    }
  }
}

// Merge split-K partials: o = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s
// (the same combine as the Metal kernel's simdgroup merge, attention/metal.py:75-94).
template <typename T, int D>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(DecodeParams p) {
  __shared__ float w[kMaxSplits * 64];  // [Hq (<= 64)][splits] weights
  const int b = blockIdx.x;
  int L;
  if (p.seq_lens) {
    L = p.seq_lens[b];
  } else {
    L = p.kv_indptr[b + 1] - p.kv_indptr[b];
  }
  int n, chunk;
  split_geometry(L, p.max_splits, n, chunk);
  if (n <= 1) return;
  const int64_t base = (int64_t)b * p.max_splits * p.hq;
  for (int h = threadIdx.x; h < p.hq; h += blockDim.x) {
    float M = -INFINITY;
    for (int s = 0; s < n; ++s) M = fmaxf(M, p.part_ml[(base + (int64_t)s * p.hq + h) * 2]);
    float Lsum = 0.f;
    for (int s = 0; s < n; ++s) {
      const float* ml = p.part_ml + (base + (int64_t)s * p.hq + h) * 2;
      const float f = __builtin_amdgcn_exp2f(ml[0] - M);
      w[h * kMaxSplits + s] = f;
      Lsum += ml[1] * f;
    }
    const float inv = 1.f / Lsum;
    for (int s = 0; s < n; ++s) w[h * kMaxSplits + s] *= inv;
  }
  __syncthreads();
  constexpr int C = D / 4;  // float4 chunks per head row
  T* o = reinterpret_cast<T*>(p.out) + (int64_t)b * p.hq * D;
  for (int i = threadIdx.x; i < p.hq * C; i += blockDim.x) {
    const int h = i / C, c = i % C;
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < n; ++s) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(p.part_o + (base + (int64_t)s * p.hq + h) * D + c * 4);
      a += w[h * kMaxSplits + s] * x;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) o[h * D + c * 4 + e] = from_f32<T>(a[e]);
  }
}

template <typename T, int D, int G>
static int launch_decode(const DecodeParams& p, int batch, hipStream_t stream) {
  const int nwaves = p.hkv < 8 ? p.hkv : 8;
  const size_t lds = (size_t)nwaves * kLdsPerWave * sizeof(float);
  hipLaunchKernelGGL((paged_decode_kernel<T, D, G>), dim3(p.max_splits, batch), dim3(64 * nwaves), lds, stream, p);
  MSGL_CHECK_LAUNCH("msgl_paged_decode");
  if (p.max_splits > 1) {
    hipLaunchKernelGGL((paged_decode_merge_kernel<T, D>), dim3(batch), dim3(256), 0, stream, p);
    MSGL_CHECK_LAUNCH("msgl_paged_decode (merge)");
  }
  return MSGL_OK;
}

template <typename T, int D>
static int dispatch_group(const DecodeParams& p, int batch, int group, hipStream_t stream) {
  switch (group) {
    case 1: return launch_decode<T, D, 1>(p, batch, stream);
    case 2: return launch_decode<T, D, 2>(p, batch, stream);
    case 4: return launch_decode<T, D, 4>(p, batch, stream);
    case 8: return launch_decode<T, D, 8>(p, batch, stream);
    case 16: return launch_decode<T, D, 16>(p, batch, stream);
    default:
      set_error("msgl_paged_decode: Hq/Hkv = %d not built (1, 2, 4, 8, 16)", group);
      return MSGL_ERR_UNSUPPORTED;
  }
}

template <typename T>
static int dispatch_dim(const DecodeParams& p, int batch, int head_dim, int group, hipStream_t stream) {
  switch (head_dim) {
    case 64: return dispatch_group<T, 64>(p, batch, group, stream);
    case 128: return dispatch_group<T, 128>(p, batch, group, stream);
    case 256: return dispatch_group<T, 256>(p, batch, group, stream);
    default:
      set_error("msgl_paged_decode: head_dim %d not built (64, 128, 256)", head_dim);
      return MSGL_ERR_UNSUPPORTED;
  }
}

}  // namespace msgl

extern "C" int32_t msgl_paged_decode_default_splits(int32_t batch, int32_t num_kv_heads, int32_t max_seq_len) {
  // Aim for ~16k wavefronts (about 4 rounds of a full MI355X at 4 waves/SIMD)
  // so ragged lengths balance, without chunks shorter than kMinChunk.
  if (batch <= 0 || num_kv_heads <= 0) return 1;
  const int64_t target_waves = 16384;
  int64_t s = (target_waves + (int64_t)batch * num_kv_heads - 1) / ((int64_t)batch * num_kv_heads);
  if (max_seq_len > 0) {
    const int64_t cap = (max_seq_len + msgl::kMinChunk - 1) / msgl::kMinChunk;
    if (s > cap) s = cap;
  }
  if (s < 1) s = 1;
  if (s > msgl::kMaxSplits) s = msgl::kMaxSplits;
  return (int32_t)s;
}

extern "C" int64_t msgl_paged_decode_workspace_size(int32_t batch, int32_t num_qo_heads, int32_t head_dim,
                                                    int32_t max_splits) {
  if (batch <= 0 || num_qo_heads <= 0 || head_dim <= 0) return 0;
  if (max_splits <= 1) return 0;
  const int64_t units = (int64_t)batch * max_splits * num_qo_heads;
  const int64_t o_bytes = units * head_dim * 4;
  const int64_t ml_bytes = units * 2 * 4;
  return ((o_bytes + 255) / 256) * 256 + ml_bytes;
}

extern "C" int msgl_paged_decode(const void* q, const void* k_pool, const void* v_pool, const int32_t* kv_indptr,
                                 const int32_t* kv_indices, const int32_t* seq_lens, int32_t batch,
                                 int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                 int64_t num_slots, int32_t dtype, float scale, int32_t max_splits, void* out,
                                 void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(batch >= 0 && batch <= 65535, "msgl_paged_decode: batch must be in [0, 65535]");
  if (batch == 0) return MSGL_OK;
  MSGL_CHECK_ARG(num_qo_heads > 0 && num_kv_heads > 0 && head_dim > 0, "msgl_paged_decode: sizes must be > 0");
  MSGL_CHECK_ARG(num_qo_heads % num_kv_heads == 0, "msgl_paged_decode: Hq (%d) must be a multiple of Hkv (%d)",
                 num_qo_heads, num_kv_heads);
  MSGL_CHECK_ARG(num_qo_heads <= 64, "msgl_paged_decode: Hq must be <= 64 (got %d)", num_qo_heads);
  MSGL_CHECK_ARG(page_size >= 1, "msgl_paged_decode: page_size must be >= 1");
  MSGL_CHECK_ARG(page_size == 1 || seq_lens != nullptr, "msgl_paged_decode: page_size > 1 needs seq_lens");
  MSGL_CHECK_ARG(num_slots > 0 && num_slots <= ((int64_t)1 << 31) - 1,
                 "msgl_paged_decode: num_slots must be in [1, 2^31)");
  MSGL_CHECK_ARG(q && k_pool && v_pool && kv_indptr && kv_indices && out, "msgl_paged_decode: null pointer");
  MSGL_CHECK_ARG(((uintptr_t)q | (uintptr_t)k_pool | (uintptr_t)v_pool | (uintptr_t)out) % 16 == 0,
                 "msgl_paged_decode: q, pools and out must be 16-byte aligned");
  if (dtype_size(dtype) == 0) {
    set_error("msgl_paged_decode: unknown dtype %d", dtype);
    return MSGL_ERR_UNSUPPORTED;
  }
  if (max_splits <= 0) max_splits = msgl_paged_decode_default_splits(batch, num_kv_heads, 0);
  if (max_splits > kMaxSplits) max_splits = kMaxSplits;
  const int64_t need = msgl_paged_decode_workspace_size(batch, num_qo_heads, head_dim, max_splits);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_error("msgl_paged_decode: workspace of %lld bytes needed, %lld given", (long long)need,
              (long long)workspace_bytes);
    return MSGL_ERR_WORKSPACE;
  }
  DecodeParams p;
  p.q = q;
  p.k_pool = k_pool;
  p.v_pool = v_pool;
  p.kv_indptr = kv_indptr;
  p.kv_indices = kv_indices;
  p.seq_lens = seq_lens;
  p.out = out;
  const int64_t units = (int64_t)batch * max_splits * num_qo_heads;
  p.part_o = reinterpret_cast<float*>(workspace);
  p.part_ml = need > 0 ? reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) +
                                                  ((units * head_dim * 4 + 255) / 256) * 256)
                       : nullptr;
  p.num_slots = num_slots;
  p.hq = num_qo_heads;
  p.hkv = num_kv_heads;
  p.page_size = page_size;
  p.max_splits = max_splits;
  p.scale_log2 = scale * kLog2e;
  const int group = num_qo_heads / num_kv_heads;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MSGL_F32: return dispatch_dim<float>(p, batch, head_dim, group, s);
    case MSGL_BF16: return dispatch_dim<bf16_t>(p, batch, head_dim, group, s);
    case MSGL_F16: return dispatch_dim<f16_t>(p, batch, head_dim, group, s);
  }
  return MSGL_ERR_UNSUPPORTED;
}
