// Fused rotary embedding + slot-mapped append: one pass over a layer's fresh q, k, v rows that
// rotates q (written to a caller buffer) and k (written into the key pool at the token's slot),
// and copies v into the value pool. It replaces the two rotations and the append of one layer,
// so the rotated keys never make a round trip through HBM before reaching the pool.
//
// Rotation (half-split, per head): with c = cos[pos][i], s = sin[pos][i], i < D/2,
//     out[i]       = x[i] * c - x[i + D/2] * s
//     out[i + D/2] = x[i + D/2] * c + x[i] * s
// Each product and each sum is rounded separately (no fused multiply-add), so the results are
// bit-identical to the same expressions evaluated elementwise in float32.
#include "pkv_common.h"

// Tuning switches (config 3's 4,216 tokens, 32 heads x 128, float32 pool, MI355X):
//   PKV_ROPE_NT    bit 0: non-temporal loads of q, k, v (they are read once); bit 1: of the pool
//                  stores; bit 2: of the rotated-query store. Default 1: 64.2 us = 6.49 TB/s in
//                  place (the runner's use), 65.1 us with a separate output; with cached loads
//                  64.9 and 80.2 us. Bit 1 costs 3-9%; bit 2 gains under 1%, and the attention
//                  call that follows reads the rotated queries, so they stay cacheable.
//   PKV_ROPE_ITEMS (token, fragment) items per thread, all loads issued before any store.
//                  Default 1: 2 and 4 items per thread took 65.7 and 70.6 us.
#ifndef PKV_ROPE_NT
#define PKV_ROPE_NT 1
#endif
#ifndef PKV_ROPE_ITEMS
#define PKV_ROPE_ITEMS 1
#endif

namespace pkv {
namespace {

constexpr int kRopeThreads = 256;
constexpr int kRopeItems = PKV_ROPE_ITEMS;

// float32 row fragments are stored unchanged; into a bfloat16 pool they are rounded to nearest
// even. kVec elements at a time (4: one 16-byte float load, 8-byte bf16 store; 1: scalar).
template <int kVec>
struct Frag {
  float v[kVec];
};

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int kVec, bool kNt = false>
__device__ __forceinline__ Frag<kVec> load_frag(const float* p) {
  Frag<kVec> f;
  if constexpr (kVec == 4) {
    f32x4 x;
    if constexpr (kNt) {
      x = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    } else {
      x = *reinterpret_cast<const f32x4*>(p);
    }
    f.v[0] = x.x;
    f.v[1] = x.y;
    f.v[2] = x.z;
    f.v[3] = x.w;
  } else if constexpr (kNt) {
    f.v[0] = __builtin_nontemporal_load(p);
  } else {
    f.v[0] = *p;
  }
  return f;
}

template <int kVec, bool kNt = false>
__device__ __forceinline__ void store_frag(float* p, const Frag<kVec>& f) {
  if constexpr (kVec == 4) {
    const f32x4 x = {f.v[0], f.v[1], f.v[2], f.v[3]};
    if constexpr (kNt) {
      __builtin_nontemporal_store(x, reinterpret_cast<f32x4*>(p));
    } else {
      *reinterpret_cast<f32x4*>(p) = x;
    }
  } else if constexpr (kNt) {
    __builtin_nontemporal_store(f.v[0], p);
  } else {
    *p = f.v[0];
  }
}

template <int kVec, bool kNt = false>
__device__ __forceinline__ void store_frag(uint16_t* p, const Frag<kVec>& f) {
  if constexpr (kVec == 4) {
    const u32x2 o = {f32_to_bf16_bits(f.v[0]) | (f32_to_bf16_bits(f.v[1]) << 16),
                     f32_to_bf16_bits(f.v[2]) | (f32_to_bf16_bits(f.v[3]) << 16)};
    if constexpr (kNt) {
      __builtin_nontemporal_store(o, reinterpret_cast<u32x2*>(p));
    } else {
      *reinterpret_cast<u32x2*>(p) = o;
    }
  } else {
    const auto bits = static_cast<uint16_t>(f32_to_bf16_bits(f.v[0]));
    if constexpr (kNt) {
      __builtin_nontemporal_store(bits, p);
    } else {
      *p = bits;
    }
  }
}

// lo' = lo * c - hi * s ; hi' = hi * c + lo * s, every operation rounded on its own.
template <int kVec>
__device__ __forceinline__ void rotate(Frag<kVec>& lo, Frag<kVec>& hi, const Frag<kVec>& c,
                                       const Frag<kVec>& s) {
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < kVec; ++e) {
    const float a = lo.v[e];
    const float b = hi.v[e];
    const float ac = a * c.v[e];
    const float bs = b * s.v[e];
    const float bc = b * c.v[e];
    const float as = a * s.v[e];
    lo.v[e] = ac - bs;
    hi.v[e] = bc + as;
  }
}

// One work item per (token, head, fragment of kVec elements of the lower half); its thread also
// owns the matching fragment of the upper half. Flattened 1-D item space, fragment index fastest,
// so a wavefront reads contiguous stretches of each head row. A thread takes kRopeItems items a
// grid apart and issues all their loads before any store.
template <typename PoolT, int kVec>
__global__ __launch_bounds__(kRopeThreads) void rope_append_kernel(
    float* rotated, int64_t rotated_stride, const float* queries, const float* keys,
    const float* values, int64_t q_stride, int64_t k_stride, int64_t v_stride,
    const int64_t* __restrict__ positions, const float* __restrict__ cos_table,
    const float* __restrict__ sin_table, int64_t table_rows, PoolT* __restrict__ key_pool,
    PoolT* __restrict__ value_pool, int64_t num_slots, const int64_t* __restrict__ slots,
    int64_t num_tokens, int num_heads, int head_dim) {
  constexpr bool kNtLoad = (PKV_ROPE_NT & 1) != 0;
  constexpr bool kNtPool = (PKV_ROPE_NT & 2) != 0;
  constexpr bool kNtRot = (PKV_ROPE_NT & 4) != 0;
  const int half = head_dim / 2;
  const int frags = half / kVec;
  const int64_t per_token = static_cast<int64_t>(num_heads) * frags;
  const int64_t total = num_tokens * per_token;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kRopeThreads + threadIdx.x;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kRopeThreads;

  int64_t token[kRopeItems], head[kRopeItems];
  bool live[kRopeItems];
  Frag<kVec> qlo[kRopeItems], qhi[kRopeItems], klo[kRopeItems], khi[kRopeItems];
  Frag<kVec> vlo[kRopeItems], vhi[kRopeItems], c[kRopeItems], s[kRopeItems];
#pragma unroll
  for (int k = 0; k < kRopeItems; ++k) {
    const int64_t item = first + k * step;
    token[k] = item / per_token;
    live[k] = item < total;
    if (!live[k]) continue;
    const int64_t rest = item - token[k] * per_token;
    const int h = static_cast<int>(rest / frags);
    const int i = static_cast<int>(rest - static_cast<int64_t>(h) * frags) * kVec;
    const int64_t pos = positions[token[k]];
    live[k] = pos >= 0 && pos < table_rows;  // the host validates positions first
    if (!live[k]) continue;
    head[k] = static_cast<int64_t>(h) * head_dim + i;
    c[k] = load_frag<kVec>(cos_table + pos * half + i);
    s[k] = load_frag<kVec>(sin_table + pos * half + i);
    const int64_t t = token[k];
    qlo[k] = load_frag<kVec, kNtLoad>(queries + t * q_stride + head[k]);
    qhi[k] = load_frag<kVec, kNtLoad>(queries + t * q_stride + head[k] + half);
    klo[k] = load_frag<kVec, kNtLoad>(keys + t * k_stride + head[k]);
    khi[k] = load_frag<kVec, kNtLoad>(keys + t * k_stride + head[k] + half);
    vlo[k] = load_frag<kVec, kNtLoad>(values + t * v_stride + head[k]);
    vhi[k] = load_frag<kVec, kNtLoad>(values + t * v_stride + head[k] + half);
  }
#pragma unroll
  for (int k = 0; k < kRopeItems; ++k) {
    if (!live[k]) continue;
    const int64_t t = token[k];
    rotate(qlo[k], qhi[k], c[k], s[k]);
    rotate(klo[k], khi[k], c[k], s[k]);
    // The rotated queries may overwrite the queries in place: this thread read them above.
    store_frag<kVec, kNtRot>(rotated + t * rotated_stride + head[k], qlo[k]);
    store_frag<kVec, kNtRot>(rotated + t * rotated_stride + head[k] + half, qhi[k]);
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= num_slots) continue;  // as pkv_append: a bad slot is skipped
    const int64_t row = slot * num_heads * static_cast<int64_t>(head_dim) + head[k];
    store_frag<kVec, kNtPool>(key_pool + row, klo[k]);
    store_frag<kVec, kNtPool>(key_pool + row + half, khi[k]);
    store_frag<kVec, kNtPool>(value_pool + row, vlo[k]);
    store_frag<kVec, kNtPool>(value_pool + row + half, vhi[k]);
  }
}

template <typename PoolT>
int launch_rope_append(float* rotated, int64_t rotated_stride, const float* queries,
                       const float* keys, const float* values, int64_t q_stride,
                       int64_t k_stride, int64_t v_stride, const int64_t* positions,
                       const float* cos_table, const float* sin_table, int64_t table_rows,
                       void* key_pool, void* value_pool, int64_t num_slots, const int64_t* slots,
                       int64_t num_tokens, int num_heads, int head_dim, hipStream_t stream) {
  const int half = head_dim / 2;
  // 16-byte loads need every row start, the half offset and the table rows on 4-float bounds.
  const bool vectorized = half % 4 == 0 && q_stride % 4 == 0 && k_stride % 4 == 0 &&
                          v_stride % 4 == 0 && rotated_stride % 4 == 0 && aligned16(rotated) &&
                          aligned16(queries) && aligned16(keys) && aligned16(values) &&
                          aligned16(cos_table) && aligned16(sin_table) && aligned16(key_pool) &&
                          aligned16(value_pool);
  const int vec = vectorized ? 4 : 1;
  const int64_t items = num_tokens * num_heads * (half / vec);
  const int64_t threads = (items + kRopeItems - 1) / kRopeItems;
  const int64_t groups = (threads + kRopeThreads - 1) / kRopeThreads;
  if (groups > 0x7fffffff) return PKV_EUNSUPPORTED;
  const dim3 grid(static_cast<uint32_t>(groups));
  auto* kp = static_cast<PoolT*>(key_pool);
  auto* vp = static_cast<PoolT*>(value_pool);
  if (vectorized) {
    hipLaunchKernelGGL((rope_append_kernel<PoolT, 4>), grid, dim3(kRopeThreads), 0, stream,
                       rotated, rotated_stride, queries, keys, values, q_stride, k_stride,
                       v_stride, positions, cos_table, sin_table, table_rows, kp, vp, num_slots,
                       slots, num_tokens, num_heads, head_dim);
  } else {
    hipLaunchKernelGGL((rope_append_kernel<PoolT, 1>), grid, dim3(kRopeThreads), 0, stream,
                       rotated, rotated_stride, queries, keys, values, q_stride, k_stride,
                       v_stride, positions, cos_table, sin_table, table_rows, kp, vp, num_slots,
                       slots, num_tokens, num_heads, head_dim);
  }
  return check_launch();
}

}  // namespace
}  // namespace pkv

extern "C" int pkv_rope_append(float* rotated_queries, int64_t rotated_token_stride,
                               const float* queries, const float* keys, const float* values,
                               int64_t query_token_stride, int64_t key_token_stride,
                               int64_t value_token_stride, const int64_t* positions,
                               const float* cos_table, const float* sin_table,
                               int64_t table_rows, void* key_pool, void* value_pool,
                               pkv_dtype pool_dtype, int64_t num_slots,
                               const int64_t* slot_mapping, int64_t num_tokens,
                               int32_t num_heads, int32_t head_dim, int device, void* stream) {
  using namespace pkv;
  if (num_tokens < 0 || num_heads < 1 || head_dim < 2 || head_dim % 2 != 0 || num_slots < 0 ||
      table_rows < 0) {
    return PKV_EINVAL;
  }
  if (pool_dtype != PKV_F32 && pool_dtype != PKV_BF16) return PKV_EINVAL;
  if (num_tokens == 0) return PKV_OK;
  if (!rotated_queries || !queries || !keys || !values || !positions || !cos_table ||
      !sin_table || !key_pool || !value_pool || !slot_mapping) {
    return PKV_EINVAL;
  }
  const int64_t row = static_cast<int64_t>(num_heads) * head_dim;
  // Rows may be strided views (a fused QKV output) but must not overlap their neighbours. The
  // rotated queries may alias the queries exactly (in place), not partially.
  if (query_token_stride < row || key_token_stride < row || value_token_stride < row ||
      rotated_token_stride < row) {
    return PKV_EINVAL;
  }
  if (rotated_queries == queries && rotated_token_stride != query_token_stride) return PKV_EINVAL;
  DeviceGuard guard(device);
  if (!guard.ok()) return PKV_EHIP;
  auto s = static_cast<hipStream_t>(stream);
  if (pool_dtype == PKV_F32) {
    return launch_rope_append<float>(rotated_queries, rotated_token_stride, queries, keys, values,
                                     query_token_stride, key_token_stride, value_token_stride,
                                     positions, cos_table, sin_table, table_rows, key_pool,
                                     value_pool, num_slots, slot_mapping, num_tokens, num_heads,
                                     head_dim, s);
  }
  return launch_rope_append<uint16_t>(rotated_queries, rotated_token_stride, queries, keys,
                                      values, query_token_stride, key_token_stride,
                                      value_token_stride, positions, cos_table, sin_table,
                                      table_rows, key_pool, value_pool, num_slots, slot_mapping,
                                      num_tokens, num_heads, head_dim, s);
}
