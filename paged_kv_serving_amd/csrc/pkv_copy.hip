// Byte-moving kernels of the KV data path: the slot-mapped append and the batched copy-on-write
// block copy. Both are pure HBM streams: every thread moves one 16-byte vector, and the grid is
// laid out so that one workgroup covers a contiguous 4 KiB (append) or 8 KiB (copy) stretch of a
// token row or a block.
#include "pkv_common.h"

namespace pkv {
namespace {

constexpr int kCopyThreads = 256;

// 16-byte unit of the byte-moving kernels, as a vector type the non-temporal builtins accept.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

#ifndef PKV_APPEND_UNROLL
#define PKV_APPEND_UNROLL 1
#endif
#ifndef PKV_APPEND_NT
#define PKV_APPEND_NT 0  // bit 0: non-temporal loads of the new rows; bit 1: of the pool stores
#endif
constexpr int kAppendUnroll = PKV_APPEND_UNROLL;

__device__ __forceinline__ u32x4 append_load(const void* p) {
  const auto* q = static_cast<const u32x4*>(p);
  if constexpr ((PKV_APPEND_NT & 1) != 0) return __builtin_nontemporal_load(q);
  return *q;
}
__device__ __forceinline__ void append_store(void* p, u32x4 v) {
  auto* q = static_cast<u32x4*>(p);
  if constexpr ((PKV_APPEND_NT & 2) != 0) {
    __builtin_nontemporal_store(v, q);
  } else {
    *q = v;
  }
}

// --------------------------------------------------------------------------------------------
// Append. grid = (tokens * chunks of a token row, 2); y selects keys (0) or values (1).
// Each thread moves kAppendUnroll vectors of VEC consecutive elements of one token's
// [heads * head_dim] row, all loads issued before the stores.
// --------------------------------------------------------------------------------------------
template <typename SrcT, typename DstT>
struct Mover;

// float32 -> float32, 4 elements (16 bytes).
template <>
struct Mover<float, float> {
  static constexpr int kVec = 4;
  struct In {
    u32x4 v;
  };
  __device__ static In load(const float* src) { return {append_load(src)}; }
  __device__ static void store(float* dst, In in) { append_store(dst, in.v); }
};

// bfloat16 -> bfloat16, 8 elements (16 bytes); bits are copied unchanged.
template <>
struct Mover<uint16_t, uint16_t> {
  static constexpr int kVec = 8;
  struct In {
    u32x4 v;
  };
  __device__ static In load(const uint16_t* src) { return {append_load(src)}; }
  __device__ static void store(uint16_t* dst, In in) { append_store(dst, in.v); }
};

// float32 -> bfloat16, 8 elements (32 bytes in, 16 bytes out), round to nearest even.
template <>
struct Mover<float, uint16_t> {
  static constexpr int kVec = 8;
  struct In {
    u32x4 a, b;
  };
  __device__ static In load(const float* src) { return {append_load(src), append_load(src + 4)}; }
  __device__ static void store(uint16_t* dst, In in) {
    const auto bits = [](unsigned int x) { return f32_to_bf16_bits(__uint_as_float(x)); };
    u32x4 o;
    o.x = bits(in.a.x) | (bits(in.a.y) << 16);
    o.y = bits(in.a.z) | (bits(in.a.w) << 16);
    o.z = bits(in.b.x) | (bits(in.b.y) << 16);
    o.w = bits(in.b.z) | (bits(in.b.w) << 16);
    append_store(dst, o);
  }
};

__device__ __forceinline__ void move_one(float* d, const float* s) { *d = *s; }
__device__ __forceinline__ void move_one(uint16_t* d, const uint16_t* s) { *d = *s; }
__device__ __forceinline__ void move_one(uint16_t* d, const float* s) {
  *d = static_cast<uint16_t>(f32_to_bf16_bits(*s));
}

template <typename SrcT, typename DstT, bool kVectorized>
__global__ __launch_bounds__(kCopyThreads) void append_kernel(
    DstT* __restrict__ key_pool, DstT* __restrict__ value_pool, int64_t num_slots,
    const SrcT* __restrict__ new_keys, const SrcT* __restrict__ new_values, int64_t key_stride,
    int64_t value_stride, const int64_t* __restrict__ slots, int64_t row_elems, int64_t chunks) {
  const int64_t token = blockIdx.x / chunks;
  const int64_t chunk = blockIdx.x - token * chunks;
  const int64_t slot = slots[token];
  if (slot < 0 || slot >= num_slots) return;
  const bool is_value = blockIdx.y != 0;
  const SrcT* src = is_value ? new_values + token * value_stride : new_keys + token * key_stride;
  DstT* dst = (is_value ? value_pool : key_pool) + slot * row_elems;
  if constexpr (kVectorized) {
    using M = Mover<SrcT, DstT>;
    constexpr int64_t kStep = static_cast<int64_t>(kCopyThreads) * M::kVec;
    const int64_t first = chunk * kStep * kAppendUnroll + threadIdx.x * M::kVec;
    typename M::In buf[kAppendUnroll];
#pragma unroll
    for (int u = 0; u < kAppendUnroll; ++u) {
      const int64_t e = first + u * kStep;
      if (e < row_elems) buf[u] = M::load(src + e);
    }
#pragma unroll
    for (int u = 0; u < kAppendUnroll; ++u) {
      const int64_t e = first + u * kStep;
      if (e < row_elems) M::store(dst + e, buf[u]);
    }
  } else {
    const int64_t e = chunk * kCopyThreads + threadIdx.x;
    if (e < row_elems) move_one(dst + e, src + e);
  }
}

template <typename SrcT, typename DstT>
int launch_append(void* key_pool, void* value_pool, int64_t num_slots, const void* new_keys,
                  const void* new_values, int64_t key_stride, int64_t value_stride,
                  const int64_t* slots, int64_t num_tokens, int64_t row_elems,
                  hipStream_t stream) {
  constexpr int kVec = Mover<SrcT, DstT>::kVec;
  const bool vectorized = row_elems % kVec == 0 && key_stride % kVec == 0 &&
                          value_stride % kVec == 0 &&
                          aligned16(key_pool) && aligned16(value_pool) && aligned16(new_keys) &&
                          aligned16(new_values);
  const int64_t per_block = static_cast<int64_t>(kCopyThreads) * (vectorized ? kVec * kAppendUnroll : 1);
  const int64_t chunks = (row_elems + per_block - 1) / per_block;
  if (chunks * num_tokens > 0x7fffffff) return PKV_EUNSUPPORTED;
  const dim3 grid(static_cast<uint32_t>(chunks * num_tokens), 2);
  auto* kp = static_cast<DstT*>(key_pool);
  auto* vp = static_cast<DstT*>(value_pool);
  const auto* kn = static_cast<const SrcT*>(new_keys);
  const auto* vn = static_cast<const SrcT*>(new_values);
  if (vectorized) {
    hipLaunchKernelGGL((append_kernel<SrcT, DstT, true>), grid, dim3(kCopyThreads), 0, stream, kp,
                       vp, num_slots, kn, vn, key_stride, value_stride, slots, row_elems, chunks);
  } else {
    hipLaunchKernelGGL((append_kernel<SrcT, DstT, false>), grid, dim3(kCopyThreads), 0, stream, kp,
                       vp, num_slots, kn, vn, key_stride, value_stride, slots, row_elems, chunks);
  }
  return check_launch();
}

// --------------------------------------------------------------------------------------------
// Copy-on-write. grid = (pairs * chunks of one block, layers * 2); y = layer * 2 + (0 keys,
// 1 values). Unit is the widest of 16/4/1 bytes that divides the block; each of kCowThreads
// threads moves kUnroll units, issuing every load before the first store.
//
// Layout measured on MI355X (256 distinct random pairs of 256 KiB float32 blocks, K and V, i.e.
// 128 MiB read + 128 MiB written; mean of 50 launches, three rounds): one 16-byte unit per
// thread in 512-thread workgroups (8 KiB each) with non-temporal stores 40.2-40.6 us (6.6-6.7
// TB/s); the same with ordinary stores 41.6-42.9 us; 256 threads 42.6 us (non-temporal stores)
// and 44.4 us; 1024 threads 41.0 us; two units per thread 41.4-41.6 us; four units per thread
// in 256-thread workgroups with non-temporal loads (16 KiB each, the earlier layout) 46.5-47.3
// us; non-temporal loads cost 2-4 us at every layout. One unit per thread keeps the most
// independent 16-byte transfers in flight across the chip for a copy this small.
// --------------------------------------------------------------------------------------------
#ifndef PKV_COPY_NT_LOAD
#define PKV_COPY_NT_LOAD 0
#endif
#ifndef PKV_COPY_NT_STORE
#define PKV_COPY_NT_STORE 1
#endif
#ifndef PKV_COPY_UNROLL
#define PKV_COPY_UNROLL 1
#endif
#ifndef PKV_COPY_THREADS
#define PKV_COPY_THREADS 512
#endif
constexpr int kCowThreads = PKV_COPY_THREADS;

template <typename UnitT>
__device__ __forceinline__ UnitT load_unit(const UnitT* p) {
#if PKV_COPY_NT_LOAD
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}
template <typename UnitT>
__device__ __forceinline__ void store_unit(UnitT* p, UnitT v) {
#if PKV_COPY_NT_STORE
  __builtin_nontemporal_store(v, p);
#else
  *p = v;
#endif
}

template <typename UnitT, int kUnroll>
__global__ __launch_bounds__(kCowThreads) void copy_blocks_kernel(
    char* __restrict__ key_pool, char* __restrict__ value_pool, const int64_t* __restrict__ pairs,
    int64_t num_blocks, int64_t block_units, int64_t chunks) {
  const int64_t pair = blockIdx.x / chunks;
  const int64_t chunk = blockIdx.x - pair * chunks;
  const int64_t src = pairs[2 * pair];
  const int64_t dst = pairs[2 * pair + 1];
  if (src == dst || src < 0 || dst < 0 || src >= num_blocks || dst >= num_blocks) return;
  const int64_t layer = blockIdx.y >> 1;
  char* pool = (blockIdx.y & 1) ? value_pool : key_pool;
  UnitT* base = reinterpret_cast<UnitT*>(pool) + layer * num_blocks * block_units;
  const UnitT* from = base + src * block_units;
  UnitT* to = base + dst * block_units;
  const int64_t first = chunk * (kCowThreads * kUnroll) + threadIdx.x;
  UnitT buf[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = first + static_cast<int64_t>(u) * kCowThreads;
    if (i < block_units) buf[u] = load_unit(from + i);
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = first + static_cast<int64_t>(u) * kCowThreads;
    if (i < block_units) store_unit(to + i, buf[u]);
  }
}

template <typename UnitT>
int launch_copy(void* key_pool, void* value_pool, const int64_t* pairs, int64_t num_pairs,
                int32_t num_layers, int64_t num_blocks, int64_t block_bytes, hipStream_t stream) {
  constexpr int kUnroll = PKV_COPY_UNROLL;
  const int64_t units = block_bytes / static_cast<int64_t>(sizeof(UnitT));
  const int64_t per_group = static_cast<int64_t>(kCowThreads) * kUnroll;
  const int64_t chunks = (units + per_group - 1) / per_group;
  if (chunks * num_pairs > 0x7fffffff || 2 * static_cast<int64_t>(num_layers) > 65535) {
    return PKV_EUNSUPPORTED;
  }
  const dim3 grid(static_cast<uint32_t>(chunks * num_pairs), static_cast<uint32_t>(2 * num_layers));
  hipLaunchKernelGGL((copy_blocks_kernel<UnitT, kUnroll>), grid, dim3(kCowThreads), 0, stream,
                     static_cast<char*>(key_pool), static_cast<char*>(value_pool), pairs,
                     num_blocks, units, chunks);
  return check_launch();
}

}  // namespace
}  // namespace pkv

extern "C" const char* pkv_version(void) { return "pkv 0.1"; }

extern "C" const char* pkv_error_string(int code) {
  switch (code) {
    case PKV_OK:
      return "ok";
    case PKV_EINVAL:
      return "invalid argument";
    case PKV_EUNSUPPORTED:
      return "unsupported shape or dtype";
    case PKV_EHIP:
      return "HIP runtime error while enqueueing";
    case PKV_ETOOBIG:
      return "the batch needs more split-context scratch than the library's static buffer holds";
    default:
      return "unknown error code";
  }
}

extern "C" int pkv_append(void* key_pool, void* value_pool, pkv_dtype pool_dtype,
                          int64_t num_slots, const void* new_keys, const void* new_values,
                          pkv_dtype src_dtype, int64_t key_token_stride,
                          int64_t value_token_stride, const int64_t* slot_mapping,
                          int64_t num_tokens, int32_t num_heads, int32_t head_dim, int device,
                          void* stream) {
  using namespace pkv;
  if (num_tokens < 0 || num_heads < 1 || head_dim < 1 || num_slots < 1) return PKV_EINVAL;
  if (dtype_size(pool_dtype) == 0 || dtype_size(src_dtype) == 0) return PKV_EINVAL;
  if (src_dtype == PKV_BF16 && pool_dtype == PKV_F32) return PKV_EUNSUPPORTED;
  const int64_t row = static_cast<int64_t>(num_heads) * head_dim;
  if (key_token_stride < row || value_token_stride < row) return PKV_EINVAL;
  if (num_tokens == 0) return PKV_OK;
  if (!key_pool || !value_pool || !new_keys || !new_values || !slot_mapping) return PKV_EINVAL;
  DeviceGuard guard(device);
  if (!guard.ok()) return PKV_EHIP;
  (void)hipGetLastError();
  auto s = static_cast<hipStream_t>(stream);
  if (pool_dtype == PKV_F32) {
    return launch_append<float, float>(key_pool, value_pool, num_slots, new_keys, new_values,
                                       key_token_stride, value_token_stride, slot_mapping,
                                       num_tokens, row, s);
  }
  if (src_dtype == PKV_F32) {
    return launch_append<float, uint16_t>(key_pool, value_pool, num_slots, new_keys, new_values,
                                          key_token_stride, value_token_stride, slot_mapping,
                                          num_tokens, row, s);
  }
  return launch_append<uint16_t, uint16_t>(key_pool, value_pool, num_slots, new_keys, new_values,
                                           key_token_stride, value_token_stride, slot_mapping,
                                           num_tokens, row, s);
}

extern "C" int pkv_copy_blocks(void* key_pool, void* value_pool, pkv_dtype dtype,
                               const int64_t* pairs, int64_t num_pairs, int32_t num_layers,
                               int64_t num_blocks, int64_t block_elems, int device,
                               void* stream) {
  using namespace pkv;
  if (num_pairs < 0 || num_layers < 1 || num_blocks < 1 || block_elems < 1) return PKV_EINVAL;
  if (dtype_size(dtype) == 0) return PKV_EINVAL;
  if (num_pairs == 0) return PKV_OK;
  if (!key_pool || !value_pool || !pairs) return PKV_EINVAL;
  DeviceGuard guard(device);
  if (!guard.ok()) return PKV_EHIP;
  (void)hipGetLastError();
  auto s = static_cast<hipStream_t>(stream);
  const int64_t bytes = block_elems * dtype_size(dtype);
  const bool base_aligned = aligned16(key_pool) && aligned16(value_pool);
  if (bytes % 16 == 0 && base_aligned) {
    return launch_copy<u32x4>(key_pool, value_pool, pairs, num_pairs, num_layers, num_blocks,
                              bytes, s);
  }
  if (bytes % 4 == 0 && (reinterpret_cast<uintptr_t>(key_pool) & 3u) == 0 &&
      (reinterpret_cast<uintptr_t>(value_pool) & 3u) == 0) {
    return launch_copy<uint32_t>(key_pool, value_pool, pairs, num_pairs, num_layers, num_blocks,
                                 bytes, s);
  }
  return launch_copy<uint8_t>(key_pool, value_pool, pairs, num_pairs, num_layers, num_blocks,
                              bytes, s);
}
