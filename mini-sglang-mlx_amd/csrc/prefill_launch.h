// Kernel templates and launches of the ragged prefill (the design is described
// at the top of prefill.hip). Included by the translation units under inst/,
// each of which instantiates one (query, pool) type pair, so the instantiations
// compile in parallel.
// The templates have internal linkage (anonymous namespace): a kernel that
// several of those units instantiate -- the merge kernels, which do not depend
// on the pool type -- gets its own copy and registration in each unit rather
// than one external symbol registered by several code objects.
#pragma once

#include "prefill_device.h"

namespace msgl {

namespace {
using namespace pf;

template <typename T, typename KV, int D, int G>
__global__ __launch_bounds__(THREADS16) __attribute__((amdgpu_waves_per_eu(G16<D>::WAVES))) void prefill16_kernel(
    PrefillParams p) {
  prefill16_body<T, KV, D, G>(p, blockIdx.x);
}

template <typename T, int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillParams p) {
  prefill_merge_body<T, D>(p, blockIdx.x, blockIdx.y);
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
  static_assert(G >= 1 && G <= ROWS, "unsupported group size");
  constexpr int BQ = ROWS / G;   // query tokens per workgroup; rows past BQ * G pad the block
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
  const int64_t nidx = p.kv_indptr[p.num_reqs];  // entries of kv_indices
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
    const int64_t qr = min((int64_t)max(q0 + my_tok, 0), (int64_t)p.num_tokens - 1);  // q holds num_tokens rows
    const uint8_t* qrow = reinterpret_cast<const uint8_t*>(p.q) + (qr * p.hq + my_head) * D * 4;
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
      nslot[i] = j < kv_end ? (int)kv_slot(p, nidx, kv_start, j) : -1;
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
    if (row < BQ * G && tok < E && q0 + tok >= 0 && q0 + tok < p.num_tokens) {
      float* orow = out + ((int64_t)(q0 + tok) * p.hq + kvh * G + row % G) * D;
#pragma unroll
      for (int t = 0; t < NDT; ++t) orow[t * 16 + col] = acc[t][i] * rinv;
    }
  }
}

// ---------------------------------------------------------------------------
// launch
// ---------------------------------------------------------------------------

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
    const int st = launch_prefill_plan(p, BQ, stream);
    if (st != MSGL_OK) return st;
  }
  if (p.mode == kPlanOnly) return MSGL_OK;
  const int grid = (int)items;
  static std::atomic<uint64_t> lds_raised{0};  // per device, for this instantiation
  const int lst = ensure_lds_limit(reinterpret_cast<const void*>(&prefill16_kernel<T, KV, D, G>), Geo::LDS_BYTES,
                                   lds_raised, "msgl_prefill_ragged");
  if (lst != MSGL_OK) return lst;
  launch_main(prefill16_kernel<T, KV, D, G>, dim3(grid), dim3(THREADS16), Geo::LDS_BYTES, stream, p);
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
  launch_main(prefill_f32_kernel<D, G>, dim3(qblocks, p.num_reqs * p.hkv), dim3(256), G32<D>::LDS_BYTES, stream, p);
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
    case 3: return launch_prefill<T, KV, D, 3>(p, max_e, s);
    case 4: return launch_prefill<T, KV, D, 4>(p, max_e, s);
    case 5: return launch_prefill<T, KV, D, 5>(p, max_e, s);
    case 6: return launch_prefill<T, KV, D, 6>(p, max_e, s);
    case 7: return launch_prefill<T, KV, D, 7>(p, max_e, s);
    case 8: return launch_prefill<T, KV, D, 8>(p, max_e, s);
    case 16: return launch_prefill<T, KV, D, 16>(p, max_e, s);
    default:
      set_error("msgl_prefill_ragged: Hq/Hkv = %d not built (1-8, 16)", group);
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

}  // namespace
}  // namespace msgl
