// Shared device helpers and host error channel for the gfx950 attention kernels.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <cstdio>
#include <string>

#include "msgl_attn.h"

namespace msgl {

// ---------------------------------------------------------------------------
// host: per-thread error message and status helpers
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
void clear_error();

// The events msgl_profile_next_launch armed for this thread, if any (disarms them).
bool take_profile_events(hipEvent_t& start, hipEvent_t& stop);

// Launch of an entry point's main kernel: with events armed by
// msgl_profile_next_launch, through hipExtLaunchKernel, which records them at
// the dispatch's own start and end (no queue barrier in front of the kernel).
template <typename K, typename... Args>
inline void launch_main(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream, Args... args) {
  hipEvent_t e0, e1;
  if (take_profile_events(e0, e1)) {
    hipExtLaunchKernelGGL(kernel, grid, block, (std::uint32_t)lds, stream, e0, e1, 0u, args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
  }
}

#define MSGL_CHECK_ARG(cond, ...)            \
  do {                                       \
    if (!(cond)) {                           \
      ::msgl::set_error(__VA_ARGS__);        \
      return MSGL_ERR_INVALID;               \
    }                                        \
  } while (0)

#define MSGL_CHECK_LAUNCH(what)                                                          \
  do {                                                                                   \
    hipError_t err__ = hipGetLastError();                                                \
    if (err__ != hipSuccess) {                                                           \
      ::msgl::set_error("%s: HIP launch failed: %s", what, hipGetErrorString(err__));    \
      return MSGL_ERR_HIP;                                                               \
    }                                                                                    \
  } while (0)

// Raises `fn`'s dynamic-LDS limit to `bytes` once per device: `done` (one per
// kernel function) holds a bit per device id that already has it. Concurrent
// first calls may both set the attribute, which is harmless (it is idempotent).
inline int ensure_lds_limit(const void* fn, int bytes, std::atomic<uint64_t>& done, const char* what) {
  if (bytes <= 65536) return MSGL_OK;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    set_error("%s: hipGetDevice failed", what);
    return MSGL_ERR_HIP;
  }
  const uint64_t bit = dev < 64 ? (uint64_t)1 << dev : 0;
  if (bit != 0 && (done.load(std::memory_order_acquire) & bit)) return MSGL_OK;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) {
    set_error("%s: cannot raise the LDS limit to %d bytes", what, bytes);
    return MSGL_ERR_HIP;
  }
  done.fetch_or(bit, std::memory_order_acq_rel);
  return MSGL_OK;
}

inline int dtype_size(int32_t dtype) {
  switch (dtype) {
    case MSGL_F32: return 4;
    case MSGL_BF16: return 2;
    case MSGL_F16: return 2;
    default: return 0;
  }
}

// ---------------------------------------------------------------------------
// device: element types
// ---------------------------------------------------------------------------
typedef uint16_t bf16_t;  // raw bfloat16 bits
typedef _Float16 f16_t;

// OCP fp8 e4m3 ("e4m3fn": bias 7, largest finite 448), the KV-cache storage
// format of the quantised pool; a distinct type so templates can select on it.
struct fp8e4m3 {
  uint8_t bits;
};

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// float -> bfloat16, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Unpack the 8 elements of a 16-byte chunk to fp32, for each storage type.
template <typename T>
struct Vec16;

template <>
struct Vec16<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void to_f32(const u32x4& r, float* out) {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(r[i]);
  }
};

template <>
struct Vec16<bf16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void to_f32(const u32x4& r, float* out) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(r[i] << 16);
      out[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
    }
  }
};

template <>
struct Vec16<f16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void to_f32(const u32x4& r, float* out) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r[i] & 0xffffu));
      out[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r[i] >> 16));
    }
  }
};

template <>
struct Vec16<fp8e4m3> {
  static constexpr int N = 16;
  __device__ __forceinline__ static void to_f32(const u32x4& r, float* out) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)r[i], false);
      const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)r[i], true);
      out[4 * i] = lo.x;
      out[4 * i + 1] = lo.y;
      out[4 * i + 2] = hi.x;
      out[4 * i + 3] = hi.y;
    }
  }
};

template <typename T>
__device__ __forceinline__ T from_f32(float f);
template <>
__device__ __forceinline__ float from_f32<float>(float f) { return f; }
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float f) { return f32_to_bf16(f); }
template <>
__device__ __forceinline__ f16_t from_f32<f16_t>(float f) { return (_Float16)f; }

template <typename T>
__device__ __forceinline__ float to_f32(T x);
template <>
__device__ __forceinline__ float to_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ float to_f32<bf16_t>(bf16_t x) { return bf16_to_f32(x); }
template <>
__device__ __forceinline__ float to_f32<f16_t>(f16_t x) { return (float)x; }

// 16-byte global load / store (dwordx4).
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
// Streaming 16-byte load for data read exactly once (nontemporal cache policy).
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }

// ---------------------------------------------------------------------------
// device: cross-lane reductions inside one 16-lane DPP row
// ---------------------------------------------------------------------------
// DPP controls: quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E,
// row_half_mirror = 0x141, row_mirror = 0x140. After the four steps every
// lane of a 16-lane row holds the row's reduction.
#define MSGL_DPP(v, ctrl) \
  __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, (v)), (ctrl), 0xF, 0xF, true))

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, MSGL_DPP(v, 0xB1));
  v = fmaxf(v, MSGL_DPP(v, 0x4E));
  v = fmaxf(v, MSGL_DPP(v, 0x141));
  v = fmaxf(v, MSGL_DPP(v, 0x140));
  return v;
}

__device__ __forceinline__ float row16_sum(float v) {
  v += MSGL_DPP(v, 0xB1);
  v += MSGL_DPP(v, 0x4E);
  v += MSGL_DPP(v, 0x141);
  v += MSGL_DPP(v, 0x140);
  return v;
}

// OCP fp8 e4m3 quantisation of one row of a KV pool, shared by the
// quantising store and the decode launch that stores the new token itself
// (so both write the same codes): the row is lpr consecutive lanes, each
// holding one 16-byte chunk `in` of VEC elements of T. amax = max |x| over the
// row (lane exchanges), codes = e4m3(x * (448 / amax)) rounded to nearest even
// into w (byte e of the chunk in byte e % 4 of w[e / 4]), +0 codes for a row
// of zeros; the row's scale is amax / 448. Returns amax. Every lane of an
// lpr-group must take part (the exchanges read its neighbours).
template <typename T>
__device__ __forceinline__ float fp8_quantize_chunk(const u32x4& in, int lpr, uint32_t (&w)[16 / sizeof(T) / 4]) {
  constexpr int VEC = 16 / (int)sizeof(T);
  float x[VEC];
  Vec16<T>::to_f32(in, x);
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < VEC; ++e) amax = fmaxf(amax, fabsf(x[e]));
  for (int off = 1; off < lpr; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  const float inv = amax > 0.f ? 448.f / amax : 0.f;
#pragma unroll
  for (int i = 0; i < VEC / 4; ++i) {
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * i] * inv, x[4 * i + 1] * inv, 0, false);
    w[i] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x[4 * i + 2] * inv, x[4 * i + 3] * inv, lo, true);
  }
  if (amax == 0.f) {
#pragma unroll
    for (int i = 0; i < VEC / 4; ++i) w[i] = 0u;  // +0 codes, also for -0 inputs
  }
  return amax;
}

#define MSGL_LDS __attribute__((address_space(3)))

// LDS DMA (global_load_lds_dword{,x4}): `bytes` per lane from global memory
// into LDS at lds_addr + bytes * lane (lds_addr wave-uniform, in m0). The
// caller waits for the transfer with vm_wait and makes it visible to the
// other wavefronts with a barrier.
//
// Issued as inline assembly: with __builtin_amdgcn_global_load_lds the
// compiler cannot tell which LDS bytes a transfer in flight writes (it has no
// alias scopes for them), so it drains every transfer (vmcnt(0)) before each
// LDS read of a ring, which serialises a pipeline over one. The statement is
// self-contained: it saves m0, sets it, waits the one wait state an SALU write
// of m0 needs before an LDS DMA reads it (GFX9 family), issues the transfer
// and restores m0, so whatever the compiler keeps in m0 survives it.
// MSGL_DMA_BUILTIN=1 builds the builtin form instead.
#ifndef MSGL_DMA_BUILTIN
#define MSGL_DMA_BUILTIN 0
#endif
__device__ __forceinline__ void dma16(const void* g, uint32_t lds_addr) {
#if MSGL_DMA_BUILTIN
  __builtin_amdgcn_global_load_lds(g, (MSGL_LDS void*)(uintptr_t)lds_addr, 16, 0, 0);
#else
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(lds_addr)
      : "memory");
#endif
}

// 4 bytes per active lane (see dma16).
__device__ __forceinline__ void dma4(const void* g, uint32_t lds_addr) {
#if MSGL_DMA_BUILTIN
  __builtin_amdgcn_global_load_lds(g, (MSGL_LDS void*)(uintptr_t)lds_addr, 4, 0, 0);
#else
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(lds_addr)
      : "memory");
#endif
}

// Wait until at most N vector memory operations of this wavefront are in
// flight (they complete in issue order).
template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Ordering point for LDS traffic between lanes of one wavefront.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace msgl
