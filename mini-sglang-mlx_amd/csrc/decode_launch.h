// Kernel templates and launches of paged decode (the design is described at the
// top of paged_decode.hip). Included by the translation units under inst/,
// each of which instantiates one (query, pool) type pair, so the instantiations
// compile in parallel.
// The templates have internal linkage (anonymous namespace): a kernel that
// several of those units instantiate -- the merge kernels, which do not depend
// on the pool type -- gets its own copy and registration in each unit rather
// than one external symbol registered by several code objects.
#pragma once

#include <atomic>

#include "decode_device.h"

namespace msgl {
namespace {
using namespace dec;

// Occupancy floor: 16-bit queries with D <= 128 and up to 2 query heads per kv
// head fit 3 wavefronts per SIMD (168 VGPRs) without spilling, which keeps
// more K/V loads in flight per CU; the rest keep MSGL_DECODE_MIN_WAVES.
#ifndef MSGL_DECODE_G2_MIN_WAVES
#define MSGL_DECODE_G2_MIN_WAVES 3
#endif
template <typename T, int D, int G>
constexpr int decode_min_waves() {
  return (sizeof(T) == 2 && D <= 128 && G <= 2 && MSGL_DECODE_MIN_WAVES < MSGL_DECODE_G2_MIN_WAVES)
             ? MSGL_DECODE_G2_MIN_WAVES
             : MSGL_DECODE_MIN_WAVES;
}

// Instantiations with the key-range form built in: the shapes where its chunk
// loop (10-25 more VGPRs) leaves the occupancy as it is -- 16-bit queries,
// head_dim 128, up to 8 query heads per kv head (2 or 4 over fp8 pools).
template <typename T, typename KV, int D, int G>
constexpr bool decode_ranges() {
  constexpr bool q8 = std::is_same<KV, fp8e4m3>::value;
  return MSGL_DECODE_BALANCED && sizeof(T) == 2 && D == 128 && (q8 ? (G == 2 || G == 4) : G <= 8);
}

template <typename T, typename KV, int D, int G>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(decode_min_waves<T, D, G>())))
void paged_decode_kernel(DecodeParams p) {
  paged_decode_body<T, KV, D, G, decode_ranges<T, KV, D, G>()>(p, blockIdx.x);
}

// The shared-head form (max_splits == 1): kSharedWaves wavefronts per
// (request, kv head), no merge.
template <typename T, typename KV, int D, int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(decode_min_waves<T, D, G>())))
void paged_decode_shared_kernel(DecodeParams p) {
  if constexpr (decode_shared<T, KV, D, G>()) paged_decode_body<T, KV, D, G, false, true>(p, blockIdx.x);
}

template <typename T, int D, int G>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(DecodeParams p, int batch) {
  paged_decode_merge_body<T, D, G>(p, batch, blockIdx.x);
}
template <typename T, typename KV, int D, int G>
int launch_decode(const DecodeParams& p_in, int batch, hipStream_t stream) {
  DecodeParams p = p_in;
  const int nwaves = p.hkv < MSGL_DECODE_WAVES_PER_WG ? p.hkv : MSGL_DECODE_WAVES_PER_WG;
  const size_t lds = decode_lds_bytes<KV, D>(nwaves);
  if (!p.planned) {
    const int st = launch_decode_plan(p, stream);
    if (st != MSGL_OK) return st;
  }
  if constexpr (decode_shared<T, KV, D, G>()) {
    if (p.shared_head) {  // one launch, no merge: kSharedWaves wavefronts per (request, kv head)
      if (std::is_same<KV, fp8e4m3>::value && p.k_new != nullptr) {
        // fp8 pools: the quantising store first (the waves of a workgroup do not
        // read back a slot another of them wrote), then the decode reads it
        const int st = msgl_store_kv_fp8(p.k_new, p.v_new, p.out_loc, p.k_pool_w, p.v_pool_w, p.kv_scale_w, batch,
                                         p.hkv_pool, D, p.num_slots,
                                         std::is_same<T, bf16_t>::value ? MSGL_BF16 : MSGL_F16,
                                         stream);
        if (st != MSGL_OK) return st;
        p.k_new = p.v_new = nullptr;
        p.out_loc = nullptr;
      }
      launch_main(paged_decode_shared_kernel<T, KV, D, G>, dim3((unsigned)(dec::decode_items(p) * p.hpg)),
                  dim3(64 * kSharedWaves), decode_shared_lds_bytes<KV, D, G>(), stream, p);
      MSGL_CHECK_LAUNCH("msgl_paged_decode");
      return MSGL_OK;
    }
  }
  launch_main(paged_decode_kernel<T, KV, D, G>, dim3((unsigned)dec::decode_items(p)), dim3(64 * nwaves), lds, stream,
              p);
  MSGL_CHECK_LAUNCH("msgl_paged_decode");
  if (p.max_splits > 1 && !p.skip_merge) {
    const int units = batch * p.hkv;
    hipLaunchKernelGGL((paged_decode_merge_kernel<T, D, G>), dim3((units + 3) / 4), dim3(256), 0, stream, p, batch);
    MSGL_CHECK_LAUNCH("msgl_paged_decode (merge)");
  }
  return MSGL_OK;
}

// Workgroups of paged_decode_kernel<T, KV, D, G> the device holds at once
// (occupancy x CUs), measured once per process and shape.
struct Resident {
  int nwaves;
  int* out;
  bool* ranges;  // the instantiation has the key-range form
  template <typename T, typename KV, int D, int G>
  int run() const {
    *ranges = decode_ranges<T, KV, D, G>();
    static std::atomic<int> cached[MSGL_DECODE_WAVES_PER_WG + 1];  // per process: one device type
    int c = cached[nwaves].load(std::memory_order_relaxed);
    if (c == 0) {
      int per_cu = 0, dev = 0, cus = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
              &per_cu, reinterpret_cast<const void*>(&paged_decode_kernel<T, KV, D, G>), 64 * nwaves,
              decode_lds_bytes<KV, D>(nwaves)) != hipSuccess ||
          hipGetDevice(&dev) != hipSuccess ||
          hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
        set_error("msgl_paged_decode: occupancy query failed: %s", hipGetErrorString(hipGetLastError()));
        return MSGL_ERR_HIP;
      }
      c = per_cu * cus > 0 ? per_cu * cus : 1;
      cached[nwaves].store(c, std::memory_order_relaxed);
    }
    *out = c;
    return MSGL_OK;
  }
};

// Groups 1 to 8; the host runs larger multiples of 8 as groups of 8 over
// virtual kv heads, so no instantiation needs more.
template <typename T, typename KV, int D, typename F>
int dispatch_group(const F& f, int group) {
  constexpr bool Q8 = std::is_same<KV, fp8e4m3>::value;
  switch (group) {
    case 1: return f.template run<T, KV, D, 1>();
    case 2: return f.template run<T, KV, D, 2>();
    case 3: return f.template run<T, KV, D, 3>();
    case 4: return f.template run<T, KV, D, 4>();
    case 5: return f.template run<T, KV, D, 5>();
    case 6: return f.template run<T, KV, D, 6>();
    case 7: return f.template run<T, KV, D, 7>();
    case 8: return f.template run<T, KV, D, 8>();
    default:
      set_error("msgl_paged_decode: Hq/Hkv = %d not built (1-8%s)", group,
                Q8 ? " for fp8 pools" : ", and multiples of 8 as groups of 8");
      return MSGL_ERR_UNSUPPORTED;
  }
}

template <typename T, typename KV = T, typename F>
int dispatch_dim(const F& f, int head_dim, int group) {
  switch (head_dim) {
    case 64: return dispatch_group<T, KV, 64>(f, group);
    case 128: return dispatch_group<T, KV, 128>(f, group);
    case 256: return dispatch_group<T, KV, 256>(f, group);
    default:
      set_error("msgl_paged_decode: head_dim %d not built (64, 128, 256)", head_dim);
      return MSGL_ERR_UNSUPPORTED;
  }
}

// One request (decode launch, merge launch, or a property of the instantiation)
// applied to the instantiation of <T, KV, D, G>.
struct OpRun {
  const DecodeOp& op;
  template <typename T, typename KV, int D, int G>
  int run() const {
    switch (op.kind) {
      case kOpLaunch: return launch_decode<T, KV, D, G>(*op.p, op.batch, op.stream);
      case kOpMerge: {
        const int units = op.batch * op.p->hkv;
        launch_main(paged_decode_merge_kernel<T, D, G>, dim3((units + 3) / 4), dim3(256), 0, op.stream, *op.p,
                    op.batch);
        MSGL_CHECK_LAUNCH("msgl_paged_decode_merge");
        return MSGL_OK;
      }
      case kOpShared:
        *op.flag = decode_shared<T, KV, D, G>();
        return MSGL_OK;
      case kOpResident: return Resident{op.nwaves, op.resident, op.flag}.template run<T, KV, D, G>();
    }
    set_error("msgl_paged_decode: unknown request %d", (int)op.kind);
    return MSGL_ERR_UNSUPPORTED;
  }
};

}  // namespace
}  // namespace msgl
