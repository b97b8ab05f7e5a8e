// Paged causal attention over block tables, for ragged batches (decode rows and prefill-chunk
// rows alike), as two passes:
//
//  1. partial: one workgroup of kWaves wavefronts per (query row, head, context partition).
//     The partition's block-table slice is staged in LDS; each wavefront streams whole key and
//     value token rows of its share of the partition with 16-byte loads (kLpt lanes cover one
//     token's head row, so one load instruction reads kTpr rows of up to 128 contiguous bytes),
//     and keeps an online softmax (running max m, running sum l, unnormalised accumulator) per
//     lane group in registers. The groups are merged through LDS at the end. A query whose
//     visible context fits one partition writes its final output here.
//  2. reduce: for queries spanning several partitions, merge the per-partition (m, l, acc)
//     with the same max-rescaled sum and write the normalised output.
//
// Scores are kept in base 2: q is pre-multiplied by scale * log2(e), so every exponential is a
// single v_exp_f32. Softmax is invariant under that change of base.
//
// Every key position a query may read is below min(context_len, position + 1); rows at or
// beyond it are never loaded, and table entries past the last visible block are never read.
#include <math.h>

#include "pkv_common.h"

namespace pkv {
namespace {

// Tunables (compile-time): wavefronts per workgroup, key rows loaded per wavefront before any
// of them is used, and whether K/V rows are loaded non-temporally (read-once streams).
#ifndef PKV_ATTN_WAVES
#define PKV_ATTN_WAVES 4
#endif
#ifndef PKV_ATTN_ITER_TOKENS
#define PKV_ATTN_ITER_TOKENS 32
#endif
#ifndef PKV_ATTN_NONTEMPORAL
#define PKV_ATTN_NONTEMPORAL 1
#endif

constexpr int kWaves = PKV_ATTN_WAVES;  // wavefronts per workgroup
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxPartition = 1024;   // keys per partition, upper bound
constexpr int kDefaultPartition = 512;
constexpr int kTableSlots = kMaxPartition + 4;  // ceil(P / B) + 1 entries at most

template <typename KVT>
struct KVTraits;
template <>
struct KVTraits<float> {
  static constexpr int kEsize = 4;
};
template <>
struct KVTraits<uint16_t> {  // bfloat16 bits
  static constexpr int kEsize = 2;
};

// How one wavefront maps onto token rows of a head: kLpt lanes per row, kVpl 16-byte vectors per
// lane, so each lane owns kDpl = D / kLpt dimensions and a wavefront covers kTpr rows per load
// round. kRounds rounds (kIterTok rows) are loaded before any of them is used.
template <typename KVT, int D>
struct Layout {
  static constexpr int kEsize = KVTraits<KVT>::kEsize;
  static constexpr int kRowBytes = D * kEsize;
  static_assert(kRowBytes >= 16 && kRowBytes % 16 == 0, "head row must be whole 16-byte vectors");
  static constexpr int kLpt = kRowBytes / 16 < 8 ? kRowBytes / 16 : 8;
  static constexpr int kVpl = kRowBytes / (16 * kLpt);
  static constexpr int kEpv = 16 / kEsize;  // elements per 16-byte vector
  static constexpr int kDpl = kVpl * kEpv;
  static constexpr int kTpr = kWave / kLpt;
  static constexpr int kRounds = kTpr >= PKV_ATTN_ITER_TOKENS ? 1 : PKV_ATTN_ITER_TOKENS / kTpr;
  static constexpr int kIterTok = kTpr * kRounds;
  static constexpr int kGroups = kWaves * kTpr;  // lane groups per workgroup
};

// Widen one 16-byte vector into kEpv floats.
__device__ __forceinline__ void widen(const uint4& raw, float* out, float) {
  out[0] = __uint_as_float(raw.x);
  out[1] = __uint_as_float(raw.y);
  out[2] = __uint_as_float(raw.z);
  out[3] = __uint_as_float(raw.w);
}
__device__ __forceinline__ void widen(const uint4& raw, float* out, uint16_t) {
  out[0] = bf16_lo(raw.x);
  out[1] = bf16_hi(raw.x);
  out[2] = bf16_lo(raw.y);
  out[3] = bf16_hi(raw.y);
  out[4] = bf16_lo(raw.z);
  out[5] = bf16_hi(raw.z);
  out[6] = bf16_lo(raw.w);
  out[7] = bf16_hi(raw.w);
}

// One 16-byte vector of a key or value row.
__device__ __forceinline__ uint4 load_row(const uint4* p) {
#if PKV_ATTN_NONTEMPORAL
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
#else
  return *p;
#endif
}

// Visible key count of a query: keys at positions 0 .. min(context_len, position + 1) - 1.
__device__ __forceinline__ int visible_len(int ctx, int pos) {
  if (pos < 0) return 0;
  return pos >= ctx ? ctx : pos + 1;
}

template <typename KVT, int D, bool kPow2Block>
__global__ __launch_bounds__(kThreads) void attention_partial_kernel(
    float* __restrict__ out, float* __restrict__ ws_acc, float* __restrict__ ws_ml,
    const float* __restrict__ queries, int64_t q_stride, const int32_t* __restrict__ q_pos,
    const int32_t* __restrict__ q_seq, const KVT* __restrict__ kcache,
    const KVT* __restrict__ vcache, int64_t num_blocks, int32_t block_size, int32_t block_shift,
    const int32_t* __restrict__ tables, int32_t table_stride, const int32_t* __restrict__ ctx_lens,
    int32_t num_seqs, int32_t num_heads, float scale_log2, int32_t part_size, int32_t max_parts,
    int32_t max_ctx) {
  using L = Layout<KVT, D>;
  __shared__ int s_table[kTableSlots];
  __shared__ float s_m[L::kGroups];
  __shared__ float s_l[L::kGroups];
  __shared__ float s_acc[L::kGroups * D];

  // Grid: heads fastest, then partitions, then query rows.
  const int64_t bid = blockIdx.x;
  const int h = static_cast<int>(bid % num_heads);
  const int64_t rest = bid / num_heads;
  const int p = static_cast<int>(rest % max_parts);
  const int64_t t = rest / max_parts;

  const int seq = q_seq[t];
  const bool seq_ok = seq >= 0 && seq < num_seqs;
  const int kv_len = seq_ok ? min(visible_len(ctx_lens[seq], q_pos[t]), max_ctx) : 0;
  const int nparts = kv_len > part_size ? (kv_len + part_size - 1) / part_size : 1;
  if (p >= nparts) return;
  const int kbeg = p * part_size;
  const int kend = min(kbeg + part_size, kv_len);

  // Stage the partition's slice of the block table.
  const int b0 = kPow2Block ? (kbeg >> block_shift) : (kbeg / block_size);
  const int nb = kend > kbeg ? (kPow2Block ? ((kend - 1) >> block_shift) : ((kend - 1) / block_size)) - b0 + 1 : 0;
  if (nb > 0) {
    const int32_t* table = tables + static_cast<int64_t>(seq) * table_stride + b0;
    for (int i = threadIdx.x; i < nb; i += kThreads) s_table[i] = table[i];
  }
  __syncthreads();

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int g = lane / L::kLpt;  // token slot inside a load round
  const int j = lane % L::kLpt;  // position inside the row

  float qv[L::kDpl];
  {
    const float* qrow = queries + t * q_stride + static_cast<int64_t>(h) * D;
#pragma unroll
    for (int i = 0; i < L::kVpl; ++i) {
#pragma unroll
      for (int e = 0; e < L::kEpv; ++e) {
        qv[i * L::kEpv + e] = qrow[(i * L::kLpt + j) * L::kEpv + e] * scale_log2;
      }
    }
  }

  float m = -INFINITY;
  float l = 0.f;
  float acc[L::kDpl];
#pragma unroll
  for (int d = 0; d < L::kDpl; ++d) acc[d] = 0.f;

  const int64_t head_off = static_cast<int64_t>(h) * D;
  const int64_t row_stride = static_cast<int64_t>(num_heads) * D;  // elements per token row
  const int n_iter = (kend - kbeg + L::kIterTok - 1) / L::kIterTok;

  for (int it = wave; it < n_iter; it += kWaves) {
    const int base = kbeg + it * L::kIterTok;
    uint4 kraw[L::kRounds][L::kVpl];
    uint4 vraw[L::kRounds][L::kVpl];
    bool valid[L::kRounds];
#pragma unroll
    for (int r = 0; r < L::kRounds; ++r) {
      const int kpos = base + r * L::kTpr + g;
      bool ok = kpos < kend;
      int64_t row = 0;
      if (ok) {
        const int lb = (kPow2Block ? (kpos >> block_shift) : (kpos / block_size)) - b0;
        const int off = kPow2Block ? (kpos & (block_size - 1)) : (kpos - (lb + b0) * block_size);
        const int blk = s_table[lb];
        ok = blk >= 0 && blk < num_blocks;
        row = (static_cast<int64_t>(blk) * block_size + off) * row_stride + head_off;
      }
      valid[r] = ok;
      if (ok) {
        const uint4* kp = reinterpret_cast<const uint4*>(kcache + row);
        const uint4* vp = reinterpret_cast<const uint4*>(vcache + row);
#pragma unroll
        for (int i = 0; i < L::kVpl; ++i) kraw[r][i] = load_row(kp + i * L::kLpt + j);
#pragma unroll
        for (int i = 0; i < L::kVpl; ++i) vraw[r][i] = load_row(vp + i * L::kLpt + j);
      } else {
#pragma unroll
        for (int i = 0; i < L::kVpl; ++i) {
          kraw[r][i] = make_uint4(0, 0, 0, 0);
          vraw[r][i] = make_uint4(0, 0, 0, 0);
        }
      }
    }

    // Scores of this lane group's rows (base-2 units), reduced over the kLpt lanes of a row.
    float s[L::kRounds];
#pragma unroll
    for (int r = 0; r < L::kRounds; ++r) {
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < L::kVpl; ++i) {
        float kf[L::kEpv];
        widen(kraw[r][i], kf, KVT{});
#pragma unroll
        for (int e = 0; e < L::kEpv; ++e) dot = fmaf(qv[i * L::kEpv + e], kf[e], dot);
      }
      dot = group_sum<L::kLpt>(dot);
      s[r] = valid[r] ? dot : -INFINITY;
    }

    // Online softmax update.
    float mx = m;
#pragma unroll
    for (int r = 0; r < L::kRounds; ++r) mx = fmaxf(mx, s[r]);
    const float shift = mx == -INFINITY ? 0.f : mx;
    const float alpha = fast_exp2(m - shift);
    float pr[L::kRounds];
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < L::kRounds; ++r) {
      pr[r] = fast_exp2(s[r] - shift);
      psum += pr[r];
    }
    l = fmaf(l, alpha, psum);
#pragma unroll
    for (int d = 0; d < L::kDpl; ++d) acc[d] *= alpha;
#pragma unroll
    for (int r = 0; r < L::kRounds; ++r) {
#pragma unroll
      for (int i = 0; i < L::kVpl; ++i) {
        float vf[L::kEpv];
        widen(vraw[r][i], vf, KVT{});
#pragma unroll
        for (int e = 0; e < L::kEpv; ++e) {
          acc[i * L::kEpv + e] = fmaf(pr[r], vf[e], acc[i * L::kEpv + e]);
        }
      }
    }
    m = mx;
  }

  // Merge the kGroups partial states of the workgroup.
  const int grp = wave * L::kTpr + g;
  if (j == 0) {
    s_m[grp] = m;
    s_l[grp] = l;
  }
#pragma unroll
  for (int i = 0; i < L::kVpl; ++i) {
#pragma unroll
    for (int e = 0; e < L::kEpv; ++e) {
      s_acc[grp * D + (i * L::kLpt + j) * L::kEpv + e] = acc[i * L::kEpv + e];
    }
  }
  __syncthreads();

  for (int d = threadIdx.x; d < D; d += kThreads) {
    float big = -INFINITY;
    for (int k = 0; k < L::kGroups; ++k) big = fmaxf(big, s_m[k]);
    const float shift = big == -INFINITY ? 0.f : big;
    float lsum = 0.f;
    float a = 0.f;
    for (int k = 0; k < L::kGroups; ++k) {
      const float w = fast_exp2(s_m[k] - shift);
      lsum = fmaf(s_l[k], w, lsum);
      a = fmaf(s_acc[k * D + d], w, a);
    }
    const int64_t qh = t * num_heads + h;
    if (nparts == 1) {
      out[qh * D + d] = a / (lsum > 0.f ? lsum : 1.f);
    } else {
      const int64_t slot = qh * max_parts + p;
      ws_acc[slot * D + d] = a;
      if (d == 0) {
        ws_ml[2 * slot] = big;
        ws_ml[2 * slot + 1] = lsum;
      }
    }
  }
}

// One workgroup per (query row, head); thread d owns output dimension d.
template <int D>
__global__ __launch_bounds__(D < kWave ? kWave : D) void attention_reduce_kernel(
    float* __restrict__ out, const float* __restrict__ ws_acc, const float* __restrict__ ws_ml,
    const int32_t* __restrict__ q_pos, const int32_t* __restrict__ q_seq,
    const int32_t* __restrict__ ctx_lens, int32_t num_seqs, int32_t num_heads, int32_t part_size,
    int32_t max_parts, int32_t max_ctx) {
  const int64_t qh = blockIdx.x;
  const int64_t t = qh / num_heads;
  const int seq = q_seq[t];
  const bool seq_ok = seq >= 0 && seq < num_seqs;
  const int kv_len = seq_ok ? min(visible_len(ctx_lens[seq], q_pos[t]), max_ctx) : 0;
  const int nparts = kv_len > part_size ? (kv_len + part_size - 1) / part_size : 1;
  if (nparts == 1) return;  // written by the partial pass
  const int d = threadIdx.x;
  if (d >= D) return;
  const float* ml = ws_ml + 2 * qh * max_parts;
  float big = -INFINITY;
  for (int k = 0; k < nparts; ++k) big = fmaxf(big, ml[2 * k]);
  const float shift = big == -INFINITY ? 0.f : big;
  float lsum = 0.f;
  float a = 0.f;
  const float* acc = ws_acc + qh * max_parts * D;
  for (int k = 0; k < nparts; ++k) {
    const float w = fast_exp2(ml[2 * k] - shift);
    lsum = fmaf(ml[2 * k + 1], w, lsum);
    a = fmaf(acc[static_cast<int64_t>(k) * D + d], w, a);
  }
  out[qh * D + d] = a / (lsum > 0.f ? lsum : 1.f);
}

struct AttnArgs {
  float* out;
  const float* queries;
  int64_t q_stride;
  const int32_t* q_pos;
  const int32_t* q_seq;
  int64_t num_queries;
  const void* kcache;
  const void* vcache;
  int64_t num_blocks;
  int32_t block_size;
  const int32_t* tables;
  int32_t table_stride;
  const int32_t* ctx_lens;
  int32_t num_seqs;
  int32_t num_heads;
  float scale_log2;
  int32_t part_size;
  int32_t max_parts;
  int32_t max_ctx;
  float* ws_acc;
  float* ws_ml;
};

template <typename KVT, int D>
int launch_attention(const AttnArgs& a, hipStream_t stream) {
  const int64_t groups = a.num_queries * a.max_parts * a.num_heads;
  if (groups > 0x7fffffff) return PKV_EUNSUPPORTED;
  const int bs = a.block_size;
  const bool pow2 = (bs & (bs - 1)) == 0;
  int shift = 0;
  while ((1 << shift) < bs) ++shift;
  const auto* kc = static_cast<const KVT*>(a.kcache);
  const auto* vc = static_cast<const KVT*>(a.vcache);
  if (pow2) {
    hipLaunchKernelGGL((attention_partial_kernel<KVT, D, true>), dim3(static_cast<uint32_t>(groups)),
                       dim3(kThreads), 0, stream, a.out, a.ws_acc, a.ws_ml, a.queries, a.q_stride,
                       a.q_pos, a.q_seq, kc, vc, a.num_blocks, bs, shift, a.tables,
                       a.table_stride, a.ctx_lens, a.num_seqs, a.num_heads, a.scale_log2,
                       a.part_size, a.max_parts, a.max_ctx);
  } else {
    hipLaunchKernelGGL((attention_partial_kernel<KVT, D, false>),
                       dim3(static_cast<uint32_t>(groups)), dim3(kThreads), 0, stream, a.out,
                       a.ws_acc, a.ws_ml, a.queries, a.q_stride, a.q_pos, a.q_seq, kc, vc,
                       a.num_blocks, bs, 0, a.tables, a.table_stride, a.ctx_lens, a.num_seqs,
                       a.num_heads, a.scale_log2, a.part_size, a.max_parts, a.max_ctx);
  }
  int rc = check_launch();
  if (rc != PKV_OK || a.max_parts == 1) return rc;
  const int64_t rows = a.num_queries * a.num_heads;
  hipLaunchKernelGGL((attention_reduce_kernel<D>), dim3(static_cast<uint32_t>(rows)),
                     dim3(D < kWave ? kWave : D), 0, stream, a.out, a.ws_acc, a.ws_ml, a.q_pos,
                     a.q_seq, a.ctx_lens, a.num_seqs, a.num_heads, a.part_size, a.max_parts,
                     a.max_ctx);
  return check_launch();
}

template <typename KVT>
int dispatch_head_dim(int head_dim, const AttnArgs& a, hipStream_t stream) {
  switch (head_dim) {
    case 8:
      return launch_attention<KVT, 8>(a, stream);
    case 16:
      return launch_attention<KVT, 16>(a, stream);
    case 32:
      return launch_attention<KVT, 32>(a, stream);
    case 64:
      return launch_attention<KVT, 64>(a, stream);
    case 128:
      return launch_attention<KVT, 128>(a, stream);
    case 256:
      return launch_attention<KVT, 256>(a, stream);
    default:
      return PKV_EUNSUPPORTED;
  }
}

int resolve_partition(int32_t partition_size) {
  if (partition_size == 0) return kDefaultPartition;
  if (partition_size < 16 || partition_size > kMaxPartition || partition_size % 16 != 0) return -1;
  return partition_size;
}

int64_t parts_for(int32_t max_context_len, int part) {
  if (max_context_len <= part) return 1;
  return (static_cast<int64_t>(max_context_len) + part - 1) / part;
}

}  // namespace
}  // namespace pkv

extern "C" int64_t pkv_attention_workspace_bytes(int64_t num_queries, int32_t num_heads,
                                                 int32_t head_dim, int32_t max_context_len,
                                                 int32_t partition_size) {
  using namespace pkv;
  const int part = resolve_partition(partition_size);
  if (part < 0 || num_queries < 0 || num_heads < 1 || head_dim < 1 || max_context_len < 0) {
    return -1;
  }
  const int64_t parts = parts_for(max_context_len, part);
  if (parts == 1) return 0;
  return num_queries * num_heads * parts * (static_cast<int64_t>(head_dim) + 2) *
         static_cast<int64_t>(sizeof(float));
}

extern "C" int pkv_paged_attention(float* out, const float* queries, int64_t query_token_stride,
                                   const int32_t* query_positions, const int32_t* query_seq,
                                   int64_t num_queries, const void* key_cache,
                                   const void* value_cache, pkv_dtype kv_dtype, int64_t num_blocks,
                                   int32_t block_size, const int32_t* block_tables,
                                   int32_t block_table_stride, const int32_t* context_lens,
                                   int32_t num_seqs, int32_t num_heads, int32_t head_dim,
                                   float scale, int32_t max_context_len, int32_t partition_size,
                                   float* workspace, int64_t workspace_bytes, int device,
                                   void* stream) {
  using namespace pkv;
  const int part = resolve_partition(partition_size);
  if (part < 0) return PKV_EINVAL;
  if (num_queries < 0 || num_blocks < 1 || block_size < 1 || block_table_stride < 0 ||
      num_seqs < 0 || num_heads < 1 || head_dim < 1 || max_context_len < 0) {
    return PKV_EINVAL;
  }
  if (dtype_size(kv_dtype) == 0) return PKV_EINVAL;
  if (query_token_stride < static_cast<int64_t>(num_heads) * head_dim) return PKV_EINVAL;
  // Every visible key position is < max_context_len (the kernels clamp to it), so a table this
  // wide covers every block id the kernels can read.
  if (static_cast<int64_t>(block_table_stride) * block_size < max_context_len) return PKV_EINVAL;
  if (num_queries == 0) return PKV_OK;
  if (!out || !queries || !query_positions || !query_seq || !key_cache || !value_cache ||
      !block_tables || !context_lens || num_seqs == 0) {
    return PKV_EINVAL;
  }
  if (!aligned16(key_cache) || !aligned16(value_cache)) return PKV_EINVAL;
  const int64_t parts = parts_for(max_context_len, part);
  if (parts > 0x7fffffff) return PKV_EUNSUPPORTED;
  float* ws_acc = nullptr;
  float* ws_ml = nullptr;
  if (parts > 1) {
    const int64_t need =
        pkv_attention_workspace_bytes(num_queries, num_heads, head_dim, max_context_len, part);
    if (!workspace || workspace_bytes < need) return PKV_EINVAL;
    ws_acc = workspace;
    ws_ml = workspace + num_queries * num_heads * parts * head_dim;
  }
  DeviceGuard guard(device);
  if (!guard.ok()) return PKV_EHIP;
  (void)hipGetLastError();
  const double log2e = 1.4426950408889634;
  AttnArgs a{out,
             queries,
             query_token_stride,
             query_positions,
             query_seq,
             num_queries,
             key_cache,
             value_cache,
             num_blocks,
             block_size,
             block_tables,
             block_table_stride,
             context_lens,
             num_seqs,
             num_heads,
             static_cast<float>(static_cast<double>(scale) * log2e),
             part,
             static_cast<int32_t>(parts),
             max_context_len,
             ws_acc,
             ws_ml};
  auto s = static_cast<hipStream_t>(stream);
  if (kv_dtype == PKV_F32) return dispatch_head_dim<float>(head_dim, a, s);
  return dispatch_head_dim<uint16_t>(head_dim, a, s);
}
