// Rotary position embedding (rotate-half layout) and its fusion with the KV
// store.
//
// Restates layers.py:45-56 (RotaryEmbedding.__call__: mx.fast.rope with
// traditional=False, one position per token) and the caller order of
// layers.py:107-109 (rotate q and k, then store rotated k and raw v into the
// pool at out_loc, kvcache/pool.py:47-50) as a single launch.
//
// For pair i < rotary_dim/2 the angle is positions[t] * inv_freq[i], one fp32
// product (inv_freq carries the base, linear or llama3 scaling, and the
// position scale); element i pairs with element i + rotary_dim/2:
//   out[i]        = x[i] * cos - x[i + half] * sin
//   out[i + half] = x[i] * sin + x[i + half] * cos
// and elements >= rotary_dim pass through. Arithmetic is fp32 for every
// storage type; results are rounded once to the storage type.
//
// One workgroup of 128 lanes per token (grid-stride over tokens). Items are
// 16 bytes (8 bf16/fp16 or 4 fp32 elements) when the rotated half and the
// pass-through tail split into such pieces, else 8 bytes: a rotated row costs
// one pair item per item of its lower half (it reads and writes that item in
// both halves) plus one copy item per item of the tail; a v row is all copy
// items. Per token each lane first issues the loads of up to K items (they do
// not depend on the position), then the position and slot arrive as scalar
// loads and the cos/sin table is computed once into LDS, shared by all q and k
// heads; rotation and stores follow. q is read and written, k and v read and
// written once each. At a few thousand tokens the whole chunk is in flight at
// once: the launch runs at ~3 TB/s (33 MB in ~11 µs), against ~4.2 TB/s for a
// device copy of the same bytes timed the same way (28 launches back to back).
// The slot order of the stores does not change the time, nor do 2 or 4 tokens
// per workgroup: every token's loads land before its stores start, so the
// chunk's reads and writes overlap little, where a copy streams both.
#include "msgl_common.h"

namespace msgl {
namespace {

constexpr int kRopeThreads = 128;
constexpr int kRopeMaxHalf = 128;  // rotary_dim <= 256
constexpr int64_t kRopeMaxBlocks = 8192;

struct RopeParams {
  const uint8_t* q;
  uint8_t* q_out;
  const uint8_t* k;
  uint8_t* k_out;
  const uint8_t* v;
  const int32_t* positions;
  const int32_t* out_loc;
  const float* inv_freq;
  uint8_t* k_pool;
  uint8_t* v_pool;
  int64_t num_slots;
  int64_t num_tokens;
  int hq;
  int hkv;
  int head_dim;
  int rotary_dim;
};

// IB bytes of storage type T (E = IB / sizeof(T) consecutive elements) as fp32:
// one 16-byte or 8-byte load or store.
template <typename T, int IB>
struct Item;

template <int IB>
struct Item<float, IB> {
  static_assert(IB == 16, "fp32 items are four elements");
  static constexpr int E = 4;
  typedef u32x4 raw_t;
  __device__ __forceinline__ static void unpack(const raw_t& r, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(r[i]);
  }
  __device__ __forceinline__ static raw_t pack(const float* f) {
    raw_t r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = __float_as_uint(f[i]);
    return r;
  }
};

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
template <int W>
struct RawWords;
template <>
struct RawWords<2> {
  typedef u32x2 type;
};
template <>
struct RawWords<4> {
  typedef u32x4 type;
};

template <int IB>
struct Item<bf16_t, IB> {
  static constexpr int E = IB / 2;
  typedef typename RawWords<IB / 4>::type raw_t;
  __device__ __forceinline__ static void unpack(const raw_t& r, float* f) {
#pragma unroll
    for (int i = 0; i < IB / 4; ++i) {
      f[2 * i] = __uint_as_float(r[i] << 16);
      f[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static raw_t pack(const float* f) {
    raw_t r;
#pragma unroll
    for (int i = 0; i < IB / 4; ++i)
      r[i] = (uint32_t)f32_to_bf16(f[2 * i]) | ((uint32_t)f32_to_bf16(f[2 * i + 1]) << 16);
    return r;
  }
};

template <int IB>
struct Item<f16_t, IB> {
  static constexpr int E = IB / 2;
  typedef typename RawWords<IB / 4>::type raw_t;
  __device__ __forceinline__ static void unpack(const raw_t& r, float* f) {
#pragma unroll
    for (int i = 0; i < IB / 4; ++i) {
      f[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r[i] & 0xffffu));
      f[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r[i] >> 16));
    }
  }
  __device__ __forceinline__ static raw_t pack(const float* f) {
    raw_t r;
#pragma unroll
    for (int i = 0; i < IB / 4; ++i)
      r[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f[2 * i]) |
             ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f[2 * i + 1]) << 16);
    return r;
  }
};

template <typename T, int IB>
__device__ __forceinline__ typename Item<T, IB>::raw_t ldi(const uint8_t* p) {
  return *reinterpret_cast<const typename Item<T, IB>::raw_t*>(p);
}
template <typename T, int IB>
__device__ __forceinline__ void sti(uint8_t* p, const typename Item<T, IB>::raw_t& r) {
  *reinterpret_cast<typename Item<T, IB>::raw_t*>(p) = r;
}

// Where item i of a token reads and writes: a pair item rotates item j of the
// lower half with item j of the upper half of one q or k row, a copy item
// moves one item of the pass-through tail of a q or k row or of a v row.
struct RopeItem {
  const uint8_t* src;
  uint8_t* d0;  // q_out / k_out row (or null)
  uint8_t* d1;  // pool row (or null)
  int64_t o;    // byte offset of the (lower) item inside the row
  bool pair;
};

template <typename T, int IB>
__device__ __forceinline__ RopeItem rope_item(const RopeParams& p, int64_t t, int64_t slot, int i, int pairs,
                                              int per_row, int nrot, int vq) {
  const int64_t row_bytes = (int64_t)p.head_dim * sizeof(T);
  RopeItem it;
  if (i < nrot) {
    const int row = i / per_row;
    const int j = i - row * per_row;
    const bool isq = row < p.hq;
    const int h = isq ? row : row - p.hq;
    const int64_t off = (t * (isq ? p.hq : p.hkv) + h) * row_bytes;
    it.src = (isq ? p.q : p.k) + off;
    it.d0 = isq ? p.q_out + off : (p.k_out ? p.k_out + off : nullptr);
    it.d1 = (!isq && slot >= 0) ? p.k_pool + (slot * p.hkv + h) * row_bytes : nullptr;
    it.pair = j < pairs;
    it.o = it.pair ? (int64_t)j * IB : (int64_t)p.rotary_dim * sizeof(T) + (int64_t)(j - pairs) * IB;
  } else {
    const int idx = i - nrot;
    const int h = idx / vq;
    it.src = p.v + (t * p.hkv + h) * row_bytes;
    it.d0 = nullptr;
    it.d1 = slot >= 0 ? p.v_pool + (slot * p.hkv + h) * row_bytes : nullptr;
    it.pair = false;
    it.o = (int64_t)(idx - h * vq) * IB;
  }
  return it;
}

// IB-byte items (16 bytes when the rotated half and the tail split into
// 16-byte pieces, else 8), K per lane whose loads are all issued before the
// first store. The data loads do not depend on the position, so they are
// issued before the token's cos/sin table is built: the two memory round
// trips (position, data) overlap.
template <typename T, int IB, int K>
__global__ __launch_bounds__(kRopeThreads) void rope_store_kernel(RopeParams p,
                                                                  const int32_t* __restrict__ positions,
                                                                  const int32_t* __restrict__ slots) {
  typedef Item<T, IB> I;
  typedef typename I::raw_t raw_t;
  constexpr int E = I::E;
  __shared__ float2 cs[kRopeMaxHalf];
  const int half = p.rotary_dim >> 1;
  const int pairs = half / E;  // pair items per rotated row
  const int per_row = pairs + (p.head_dim - p.rotary_dim) / E;
  const int nrot = (p.hq + p.hkv) * per_row;
  const int vq = p.head_dim / E;
  // v rows are only touched to store them
  const int n = nrot + ((p.out_loc && p.v_pool) ? p.hkv * vq : 0);
  const int64_t half_bytes = (int64_t)half * sizeof(T);
  // this lane's frequency (half <= kRopeMaxHalf < kRopeThreads), loaded once
  const float freq = (int)threadIdx.x < half ? p.inv_freq[threadIdx.x] : 0.f;
  for (int64_t t = blockIdx.x; t < p.num_tokens; t += gridDim.x) {
    for (int base = 0; base < n; base += kRopeThreads * K) {
      // 1. every load of this lane in flight before any store (items never
      //    overlap, so an in-place q_out/k_out is written only after all reads
      //    of the same elements)
      raw_t lo[K], hi[K];
#pragma unroll
      for (int r = 0; r < K; ++r) {
        const int i = base + r * kRopeThreads + (int)threadIdx.x;
        if (i < n) {
          const RopeItem it = rope_item<T, IB>(p, t, -1, i, pairs, per_row, nrot, vq);
          lo[r] = ldi<T, IB>(it.src + it.o);
          if (it.pair) hi[r] = ldi<T, IB>(it.src + half_bytes + it.o);
        }
      }
      // 2. the token's position and slot (read-only and uniform: scalar loads;
      //    slots aliases positions when nothing is stored), and on the first
      //    pass its cos/sin table
      const float pos = (float)positions[t];
      const int32_t raw_slot = slots[t];
      if (base == 0 && half > 0) {
        __syncthreads();  // the previous token's readers of cs are done
        if ((int)threadIdx.x < half) {
          float sn, cn;
          sincosf(pos * freq, &sn, &cn);
          cs[threadIdx.x] = make_float2(cn, sn);
        }
        __syncthreads();
      }
      // never write outside the pool
      const int64_t slot = (p.out_loc && raw_slot >= 0 && raw_slot < p.num_slots) ? (int64_t)raw_slot : -1;
      // 3. rotate and store
#pragma unroll
      for (int r = 0; r < K; ++r) {
        const int i = base + r * kRopeThreads + (int)threadIdx.x;
        if (i >= n) continue;
        const RopeItem it = rope_item<T, IB>(p, t, slot, i, pairs, per_row, nrot, vq);
        if (it.pair) {
          float x0[E], x1[E], a[E], b[E];
          I::unpack(lo[r], x0);
          I::unpack(hi[r], x1);
          const int e0 = (int)(it.o / IB) * E;
#pragma unroll
          for (int e = 0; e < E; ++e) {
            const float2 w = cs[e0 + e];
            a[e] = x0[e] * w.x - x1[e] * w.y;
            b[e] = x0[e] * w.y + x1[e] * w.x;
          }
          const raw_t ra = I::pack(a), rb = I::pack(b);
          if (it.d0) {
            sti<T, IB>(it.d0 + it.o, ra);
            sti<T, IB>(it.d0 + half_bytes + it.o, rb);
          }
          if (it.d1) {
            sti<T, IB>(it.d1 + it.o, ra);
            sti<T, IB>(it.d1 + half_bytes + it.o, rb);
          }
        } else {
          if (it.d0) sti<T, IB>(it.d0 + it.o, lo[r]);
          if (it.d1) sti<T, IB>(it.d1 + it.o, lo[r]);
        }
      }
    }
  }
}

int launch_rope(const RopeParams& p, int32_t dtype, void* stream, const char* what) {
  const int es = dtype_size(dtype);
  if (es == 0) {
    set_error("%s: unknown dtype %d", what, dtype);
    return MSGL_ERR_UNSUPPORTED;
  }
  MSGL_CHECK_ARG(p.num_tokens >= 0, "%s: num_tokens must be >= 0", what);
  MSGL_CHECK_ARG(p.hq >= 0 && p.hkv >= 0, "%s: head counts must be >= 0", what);
  MSGL_CHECK_ARG(p.head_dim >= 4 && p.head_dim <= 1024 && p.head_dim % 4 == 0,
                 "%s: head_dim must be a multiple of 4 in [4, 1024] (got %d)", what, p.head_dim);
  MSGL_CHECK_ARG(p.rotary_dim >= 0 && p.rotary_dim <= p.head_dim && p.rotary_dim % 8 == 0 &&
                     p.rotary_dim / 2 <= kRopeMaxHalf,
                 "%s: rotary_dim must be a multiple of 8 in [0, min(head_dim, %d)] (got %d)", what,
                 2 * kRopeMaxHalf, p.rotary_dim);
  if (p.num_tokens == 0 || p.hq + p.hkv == 0) return MSGL_OK;
  MSGL_CHECK_ARG(p.positions && (p.rotary_dim == 0 || p.inv_freq), "%s: positions or inv_freq is null", what);
  MSGL_CHECK_ARG(p.hq == 0 || (p.q && p.q_out), "%s: q or q_out is null", what);
  MSGL_CHECK_ARG(p.hkv == 0 || p.k, "%s: k is null", what);
  if (p.out_loc) {
    MSGL_CHECK_ARG(p.hkv > 0 && p.v && p.k_pool && p.v_pool, "%s: the KV store needs k, v and both pools", what);
    MSGL_CHECK_ARG(p.num_slots > 0, "%s: num_slots must be > 0", what);
  }
  const uintptr_t quad = 4 * (uintptr_t)es;
  MSGL_CHECK_ARG(((uintptr_t)p.q | (uintptr_t)p.q_out | (uintptr_t)p.k | (uintptr_t)p.k_out | (uintptr_t)p.v |
                  (uintptr_t)p.k_pool | (uintptr_t)p.v_pool) % quad == 0,
                 "%s: tensors must be aligned to 4 elements (%d bytes)", what, (int)quad);
  const int64_t blocks = p.num_tokens < kRopeMaxBlocks ? p.num_tokens : kRopeMaxBlocks;
  const int32_t* slots = p.out_loc ? p.out_loc : p.positions;
  hipStream_t s = (hipStream_t)stream;
  // 16-byte items when the rotated half and the pass-through tail split into
  // 16-byte pieces (and the tensors allow it), else 8-byte items
  const bool wide = es == 4 || ((p.rotary_dim / 2) % 8 == 0 && (p.head_dim - p.rotary_dim) % 8 == 0 &&
                                ((uintptr_t)p.q | (uintptr_t)p.q_out | (uintptr_t)p.k | (uintptr_t)p.k_out |
                                 (uintptr_t)p.v | (uintptr_t)p.k_pool | (uintptr_t)p.v_pool) % 16 == 0);
  const dim3 g((unsigned)blocks), b(kRopeThreads);
  switch (dtype) {
    case MSGL_F32: hipLaunchKernelGGL((rope_store_kernel<float, 16, 4>), g, b, 0, s, p, p.positions, slots); break;
    case MSGL_BF16:
      if (wide) hipLaunchKernelGGL((rope_store_kernel<bf16_t, 16, 4>), g, b, 0, s, p, p.positions, slots);
      else hipLaunchKernelGGL((rope_store_kernel<bf16_t, 8, 5>), g, b, 0, s, p, p.positions, slots);
      break;
    default:
      if (wide) hipLaunchKernelGGL((rope_store_kernel<f16_t, 16, 4>), g, b, 0, s, p, p.positions, slots);
      else hipLaunchKernelGGL((rope_store_kernel<f16_t, 8, 5>), g, b, 0, s, p, p.positions, slots);
      break;
  }
  MSGL_CHECK_LAUNCH(what);
  return MSGL_OK;
}

}  // namespace
}  // namespace msgl

extern "C" int msgl_rope(const void* x, void* out, const int32_t* positions, const float* inv_freq,
                         int64_t num_tokens, int32_t num_heads, int32_t head_dim, int32_t rotary_dim, int32_t dtype,
                         void* stream) {
  using namespace msgl;
  clear_error();
  RopeParams p = {};
  p.q = (const uint8_t*)x;
  p.q_out = (uint8_t*)out;
  p.positions = positions;
  p.inv_freq = inv_freq;
  p.num_tokens = num_tokens;
  p.hq = num_heads;
  p.head_dim = head_dim;
  p.rotary_dim = rotary_dim;
  return launch_rope(p, dtype, stream, "msgl_rope");
}

extern "C" int msgl_rope_store_kv(const void* q, const void* k, const void* v, const int32_t* positions,
                                  const int32_t* out_loc, const float* inv_freq, void* q_out, void* k_out,
                                  void* k_pool, void* v_pool, int64_t num_tokens, int32_t num_qo_heads,
                                  int32_t num_kv_heads, int32_t head_dim, int32_t rotary_dim, int64_t num_slots,
                                  int32_t dtype, void* stream) {
  using namespace msgl;
  clear_error();
  MSGL_CHECK_ARG(out_loc != nullptr, "msgl_rope_store_kv: out_loc is null");
  MSGL_CHECK_ARG(num_kv_heads > 0, "msgl_rope_store_kv: num_kv_heads must be > 0");
  RopeParams p = {};
  p.q = (const uint8_t*)q;
  p.q_out = (uint8_t*)q_out;
  p.k = (const uint8_t*)k;
  p.k_out = (uint8_t*)k_out;
  p.v = (const uint8_t*)v;
  p.positions = positions;
  p.out_loc = out_loc;
  p.inv_freq = inv_freq;
  p.k_pool = (uint8_t*)k_pool;
  p.v_pool = (uint8_t*)v_pool;
  p.num_slots = num_slots;
  p.num_tokens = num_tokens;
  p.hq = num_qo_heads;
  p.hkv = num_kv_heads;
  p.head_dim = head_dim;
  p.rotary_dim = rotary_dim;
  return launch_rope(p, dtype, stream, "msgl_rope_store_kv");
}
