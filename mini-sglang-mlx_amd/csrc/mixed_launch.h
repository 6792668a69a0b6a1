// Kernel templates and launch of the single-launch mixed step (the design is
// described at the top of mixed.hip). Included by the translation units under
// inst/, each of which instantiates one query type, so the instantiations
// compile in parallel.
// The templates have internal linkage (anonymous namespace), like those of
// decode_launch.h and prefill_launch.h.
#pragma once

#include "decode_device.h"
#include "prefill_device.h"

namespace msgl {

// The single launch for 16-bit queries of type bf16 / fp16 over a pool of the
// same type (inst/mixed_*.hip): head_dim and the query-head group pick the
// instantiation.
int mixed_launch_bf16(const pf::PrefillParams& pp, const dec::DecodeParams& dp, int batch, int max_e, int head_dim,
                      int group, hipStream_t stream);
int mixed_launch_f16(const pf::PrefillParams& pp, const dec::DecodeParams& dp, int batch, int max_e, int head_dim,
                     int group, hipStream_t stream);

}  // namespace msgl

namespace msgl {
namespace {

// G: query heads per kv head of the prefill body; GD: of the decode body, which
// runs the decode's kv heads (virtual ones where it maps G 8 over Hkv <= 2 to
// groups of 4).
template <typename T, int D, int G, int GD>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(pf::G16<D>::WAVES))) void mixed_attention_kernel(
    pf::PrefillParams pp, dec::DecodeParams dp) {
  const int np = *pp.plan_count;
  const int nd = dp.meta[0];
  const int gp = (np + 7) >> 3, gd = (nd + 7) >> 3;
  const int c = blockIdx.x >> 3, j = blockIdx.x & 7;
  if (c >= gp + gd) return;
  const int64_t tot = (int64_t)gp + gd;
  const int a = (int)((int64_t)c * gp / tot);
  const int a1 = (int)((int64_t)(c + 1) * gp / tot);
  if (a1 > a) {
    const int item = 8 * a + j;
    if (item < np) pf::prefill16_body<T, T, D, G>(pp, item);
  } else {
    const int item = 8 * (c - a) + j;
    if (item < nd) dec::paged_decode_body<T, T, D, GD, false>(dp, item);
  }
}

// The split-K merges of both parts: the first npm workgroups are the prefill
// merge's (token tk = i % ntok, head block i / ntok), the rest the decode merge's.
template <typename T, int D, int GD>
__global__ __launch_bounds__(256) void mixed_merge_kernel(pf::PrefillParams pp, dec::DecodeParams dp, int batch,
                                                          int ntok, int npm) {
  const int i = blockIdx.x;
  if (i < npm) {
    pf::prefill_merge_body<T, D>(pp, i % ntok, i / ntok);
  } else {
    dec::paged_decode_merge_body<T, D, GD>(dp, batch, i - npm);
  }
}

template <typename T, int D, int G, int GD = G>
int launch_mixed(pf::PrefillParams pp, const dec::DecodeParams& dp, int batch, int max_e, hipStream_t stream) {
  using Geo = pf::G16<D, (int)sizeof(T)>;
  constexpr int BQ = Geo::ROWS / G;  // as in the prefill body: rows past BQ * G pad the block
  static_assert(pf::THREADS16 == 256 && G <= Geo::ROWS, "both bodies run as 4-wavefront workgroups");
  pp.nqb = (max_e + BQ - 1) / BQ;
  const int64_t items_pf = (int64_t)pp.hkv * pp.num_reqs * pp.splits * pp.nqb;
  if (items_pf > (int64_t)pp.plan_capacity) {
    set_error("msgl_mixed_attention: prefill workspace holds %d work items, %lld needed", pp.plan_capacity,
              (long long)items_pf);
    return MSGL_ERR_WORKSPACE;
  }
  pp.items = (int)items_pf;
  const int64_t items_dec = dec::decode_items(dp);
  const size_t lds = std::max<size_t>(Geo::LDS_BYTES, dec::decode_lds_bytes<T, D>(4));
  static std::atomic<uint64_t> lds_raised{0};  // per device, for this instantiation
  const int lst = ensure_lds_limit(reinterpret_cast<const void*>(&mixed_attention_kernel<T, D, G, GD>), (int)lds,
                                   lds_raised, "msgl_mixed_attention");
  if (lst != MSGL_OK) return lst;
  const int64_t groups = (items_pf + 7) / 8 + (items_dec + 7) / 8;
  launch_main(mixed_attention_kernel<T, D, G, GD>, dim3((unsigned)(8 * groups)), dim3(256), lds, stream, pp, dp);
  MSGL_CHECK_LAUNCH("msgl_mixed_attention");
  constexpr int HPB = 256 / (D / 4);  // heads per prefill-merge workgroup
  const int npm = pp.splits > 1 ? pp.num_tokens * ((pp.hq + HPB - 1) / HPB) : 0;
  const int ndm = dp.max_splits > 1 ? (batch * dp.hkv + 3) / 4 : 0;
  if (npm + ndm > 0) {
    hipLaunchKernelGGL((mixed_merge_kernel<T, D, GD>), dim3(npm + ndm), dim3(256), 0, stream, pp, dp, batch,
                       pp.num_tokens, npm);
    MSGL_CHECK_LAUNCH("msgl_mixed_attention (merge)");
  }
  return MSGL_OK;
}

template <typename T, int D>
int mixed_group(const pf::PrefillParams& pp, const dec::DecodeParams& dp, int batch, int max_e, int group,
                hipStream_t s) {
  switch (group) {
    case 1: return launch_mixed<T, D, 1>(pp, dp, batch, max_e, s);
    case 2: return launch_mixed<T, D, 2>(pp, dp, batch, max_e, s);
    case 3: return launch_mixed<T, D, 3>(pp, dp, batch, max_e, s);
    case 4: return launch_mixed<T, D, 4>(pp, dp, batch, max_e, s);
    case 5: return launch_mixed<T, D, 5>(pp, dp, batch, max_e, s);
    case 6: return launch_mixed<T, D, 6>(pp, dp, batch, max_e, s);
    case 7: return launch_mixed<T, D, 7>(pp, dp, batch, max_e, s);
    case 8:  // the decode may run it as groups of 4 over twice the kv heads
      return dp.hq == dp.hkv * 4 ? launch_mixed<T, D, 8, 4>(pp, dp, batch, max_e, s)
                                 : launch_mixed<T, D, 8>(pp, dp, batch, max_e, s);
    default:
      set_error("msgl_mixed_attention: Hq/Hkv = %d not built (1-8)", group);
      return MSGL_ERR_UNSUPPORTED;
  }
}

template <typename T>
int mixed_dim(const pf::PrefillParams& pp, const dec::DecodeParams& dp, int batch, int max_e, int head_dim, int group,
              hipStream_t s) {
  switch (head_dim) {
    case 64: return mixed_group<T, 64>(pp, dp, batch, max_e, group, s);
    case 128: return mixed_group<T, 128>(pp, dp, batch, max_e, group, s);
    default:
      set_error("msgl_mixed_attention: head_dim %d not built (64, 128)", head_dim);
      return MSGL_ERR_UNSUPPORTED;
  }
}

}  // namespace
}  // namespace msgl
