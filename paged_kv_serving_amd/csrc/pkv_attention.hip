// Paged causal attention over block tables for ragged batches: decode rows and prefill-chunk
// rows of many sequences in one call. Three kernels; passes 1 and 2 cover disjoint query rows and
// run side by side (pass 2 on a second stream forked from and joined back to the caller's), and
// pass 3 runs on the caller's stream after both:
//
//  1. row_partial (memory-bound rows, e.g. decode): one workgroup of kWaves wavefronts per
//     (query row, group of HPW adjacent heads, context partition), HPW = 2 where one head row is
//     at most 256 bytes. The partition's slice of the block table is staged in LDS; each
//     wavefront streams the group's slice of whole key and value token rows of its share of the
//     partition with non-temporal 16-byte loads (kLpt lanes cover one slice) and keeps an online
//     softmax (running max, running sum, unnormalised accumulator) per lane group and head in
//     registers. The lane groups are merged through LDS at the end.
//  2. tile_partial (compute-bound rows: a run of consecutive prefill rows of one sequence, or
//     decode rows of several sequences over the partitions of a prefix they share): one
//     workgroup per (tile of <= 64 rows, head, context partition). Keys are read through the
//     table of the tile's first row, which the planner only allows where every row of the tile
//     has the same blocks. Key and value tiles of 32 rows
//     (16 at head_dim 256) are staged in LDS and shared by 4 wavefronts of 16 queries each:
//     through registers into padded rows, or, for float32 pools beside the row pass, straight
//     from HBM into three swizzled LDS stages (global_load_lds_dwordx4, two tiles in flight);
//     the scores are computed as S^T = K Q^T and the output as O = P V with
//     v_mfma_f32_16x16x4f32, so every lane owns four scores of one query per 16 keys and the P
//     operand of the second product is the lane's own registers.
//  3. reduce: rows whose visible context spans several partitions merge the per-partition
//     (max, sum, acc) and write the normalised output. Rows that fit one partition were written
//     by pass 1 or 2 directly.
//
// Scores are kept in base 2: q is pre-multiplied by scale * log2(e), so every exponential is a
// single v_exp_f32; softmax is invariant under the change of base.
//
// Every key position a query may read is below min(context_len, position + 1), clamped to
// max_context_len; rows at or beyond it are never loaded, and table entries past the last
// visible block are never read.
#include <math.h>

#include <atomic>
#include <mutex>
#include <type_traits>

#include "pkv_common.h"

// The split-context workspace of pkv_paged_attention_noalloc: a file-scope device array, one copy
// per GPU (each device's address is looked up with hipGetSymbolAddress, with that device current,
// and kept per device; host code never passes the array's own name to a kernel).
static __device__ __align__(256) float scratch[PKV_STATIC_SCRATCH_BYTES / sizeof(float)];

// Sixteen zero bytes in global memory: the tile pass loads the key and value vectors of a key
// past the end, or in a block outside the pool, from here. Such a key's probability is 0, and
// 0 times whatever a pool row holds (inf or NaN included) would not be 0.
static __device__ __align__(16) uint4 zero_vector = {0u, 0u, 0u, 0u};

namespace pkv {
namespace {

// Tunables (compile-time): wavefronts per row_partial workgroup; bytes of one head row each lane
// covers; bytes of key rows a wavefront loads (and as many value bytes) before it uses any of
// them; and whether row_partial loads K/V rows non-temporally (each row is read once there).
#ifndef PKV_ATTN_WAVES
#define PKV_ATTN_WAVES 4
#endif
#ifndef PKV_ATTN_LANE_BYTES
#define PKV_ATTN_LANE_BYTES 16
#endif
#ifndef PKV_ATTN_ITER_BYTES
#define PKV_ATTN_ITER_BYTES 16384
#endif
#ifndef PKV_ATTN_NONTEMPORAL
#define PKV_ATTN_NONTEMPORAL 1
#endif
// Run the tile pass on a second stream beside the row pass when a call has both.
#ifndef PKV_ATTN_OVERLAP
#define PKV_ATTN_OVERLAP 1
#endif
// Launch order of an overlapped call: 0 = the tile pass first (on the second stream), 1 = the
// row pass first (the fork event is recorded before it, so the tile pass still waits only for
// the work queued before the call). Measured with the current passes, same box, two alternating
// runs: config 3's mixed call 1.4795-1.4814 ms rows first against 1.4787-1.4794 tiles first,
// config 4's attention 0.2386-0.2387 against 0.2337-0.2399 ms; rows first starts the device on
// the row pass before the host's two stream waits (about 9.5 us each), so config 4's runner
// step takes 0.398-0.399 instead of 0.419-0.427 ms. (Before the tile grid rules, tiles first
// had been 40 us faster on config 3.)
#ifndef PKV_ATTN_ROWS_FIRST
#define PKV_ATTN_ROWS_FIRST 1
#endif
// Workgroup order of the row pass: 0 = the hardware's round robin over the 8 XCDs (consecutive
// workgroups, i.e. neighbouring heads of one token, on different XCDs); 1 = each XCD walks one
// contiguous eighth of the grid. Measured on MI355X (64 x 4k decode): 0 reads at 6.79 TB/s,
// 1 at 6.26 TB/s.
#ifndef PKV_ATTN_XCD_REMAP
#define PKV_ATTN_XCD_REMAP 0
#endif
// Tile pass beside the row pass, float32 pools: 1 = key and value tiles go from HBM straight into
// LDS (global_load_lds_dwordx4) through PKV_TILE_STAGES buffers, all but one in flight while one
// is multiplied; 0 = through registers, one tile ahead. A tile pass on its own (one workgroup per
// item) and the bfloat16 path always go through registers: the 96 KiB of stages allow one
// workgroup per CU, where the register path runs three (measured: 0.86 vs 0.68 ms for config 3's
// tiles alone; beside its row pass the direct path takes the call 1.56 -> 1.53 ms).
#ifndef PKV_TILE_DMA
#define PKV_TILE_DMA 1
#endif
// Direct-to-LDS path: LDS stages (2..5; 32 KiB each at head_dim 128: three leave room for two
// row-pass workgroups on the CU).
#ifndef PKV_TILE_STAGES
#define PKV_TILE_STAGES 3
#endif
// Register path at head_dim 128: the occupancy target in waves per SIMD (its VGPR budget).
// Measured on config 3's tiles alone: 3 waves (168 VGPRs) 0.68-0.70 ms, 2 waves (190 VGPRs,
// value reads double-buffered) 0.73 ms.
#ifndef PKV_TILE_REG_WAVES
#define PKV_TILE_REG_WAVES 3
#endif

constexpr int kWaves = PKV_ATTN_WAVES;  // wavefronts per row_partial workgroup
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxPartition = 1024;     // keys per partition, upper bound
constexpr int kDefaultPartition = 512;
constexpr int kTableSlots = kMaxPartition + 4;  // ceil(P / B) + 1 entries at most
constexpr int kTileRows = 64;           // query rows per tile_partial workgroup (4 x 16)
constexpr int kTileThreads = 256;
constexpr int kTileStages = PKV_TILE_STAGES;  // LDS key/value stages of the direct-to-LDS path
static_assert(kTileStages >= 2 && kTileStages <= 5, "2..5 direct-to-LDS stages");
constexpr int kTileWhole = PKV_TILE_WHOLE;  // tile end partition: every key in one workgroup
constexpr int kReduceThreads = 256;

typedef float floatx4 __attribute__((ext_vector_type(4)));

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

// Everything the three kernels read, passed by value.
struct Params {
  float* out;              // [T, H, D]
  float* ws_acc;           // [T, H, max_parts, D]
  float* ws_ml;            // [T, H, max_parts, 2]
  const float* queries;    // row q_rows[t] (t without q_rows) at that row * q_stride
  int64_t q_stride;
  const int32_t* q_rows;   // [T] or null: the row of queries / out / new_keys / new_values of
                           // planner row t (null: t itself); every other [T] array is by t
  const int32_t* q_pos;    // [T]
  const int32_t* q_seq;    // [T]
  const int32_t* rows;     // row_partial: [R, 2] = (query row, partition) items; null: every
                           // partition of every query row
  const int32_t* tiles;    // tile_partial: [n, 4] = (first row, row count <= 64, first
                           // partition, end partition; end <= first: through the last;
                           // kTileWhole: one workgroup covers every key and writes final rows)
  const int32_t* merge_rows;  // reduce: the query rows whose partials are merged
  int64_t num_merge;       // entries of merge_rows; negative: every query row instead
  int64_t num_tiles;       // entries of tiles
  int32_t flags;           // PKV_ATTN_* launch hints
  const void* kcache;      // [N, B, H, D]
  const void* vcache;
  int64_t num_queries;
  int64_t num_blocks;
  const int32_t* tables;   // [S, table_stride]
  const int32_t* ctx_lens; // [S]
  int32_t table_stride;
  int32_t num_seqs;
  int32_t num_heads;
  int32_t block_size;
  int32_t block_shift;     // log2(block_size) when it is a power of two
  int32_t part_size;
  int32_t max_parts;
  int32_t max_ctx;
  float scale_log2;        // scale * log2(e)
  // The decode append fused into the row pass (new_keys null: none). Query row t's own key and
  // value row (row r = io_row(t) of new_keys / new_values) is written to pool slot new_slots[r]
  // by the row-pass workgroups whose partition holds position q_pos[t], which also use it as
  // that key.
  const void* new_keys;    // [T, H, D] of new_dtype, row r at r * new_key_stride elements
  const void* new_values;
  int64_t new_key_stride;
  int64_t new_value_stride;
  const int64_t* new_slots;  // [T], by io_row like new_keys
  int64_t num_slots;       // pool token rows (num_blocks * block_size)
  int32_t new_dtype;       // PKV_F32 or PKV_BF16 (bfloat16 only into a bfloat16 pool)
};

constexpr uint32_t kXcds = 8;  // MI355X: workgroup i runs on XCD i % 8

// Logical workgroup index of this workgroup under the XCD order chosen above.
__device__ __forceinline__ uint32_t logical_block() {
  const uint32_t bid = blockIdx.x;
  if constexpr (PKV_ATTN_XCD_REMAP) {
    const uint32_t full = gridDim.x - gridDim.x % kXcds;
    if (bid < full) return (bid % kXcds) * (full / kXcds) + bid / kXcds;
  }
  return bid;
}

// How one wavefront of row_partial maps onto token rows. A workgroup serves HPW consecutive
// heads, so each token row it reads is one contiguous slice of HPW * D elements. kLpt lanes
// cover a slice (about PKV_ATTN_LANE_BYTES each, 1 to 8 lanes, never more than the 16-byte
// vectors of one head), each with kVpl 16-byte vectors: lane j's vector i is vector i * kLpt + j
// of the slice and belongs to head i / kVph. A lane therefore owns kDph dimensions of each of
// the HPW heads, and a wavefront covers kTpr token rows per load round. kRounds rounds (kIterTok
// rows, about PKV_ATTN_ITER_BYTES of keys, at most 64 rows) are loaded before any is used.
// Measured on MI355X: 16-byte lanes beat 64-byte lanes for bfloat16 by 18% (register pressure
// halves occupancy otherwise); 16 KiB per round is within 1-3% of 8 and 24 KiB on configs 2-5
// and best overall. Slices of at least 512 contiguous bytes per token row stream faster than
// 256-byte ones from a shuffled pool (a load-only probe of the bfloat16 head_dim-128 pattern:
// 6.65 TB/s at one head per workgroup, 6.97 TB/s at two), which is what HPW = 2 is for.
template <typename KVT, int D, int HPW, int kIterBytes = PKV_ATTN_ITER_BYTES>
struct Layout {
  static constexpr int kEsize = KVTraits<KVT>::kEsize;
  static constexpr int kHeadBytes = D * kEsize;
  static_assert(kHeadBytes >= 16 && kHeadBytes % 16 == 0, "head row must be whole 16-byte vectors");
  static constexpr int kVecPerHead = kHeadBytes / 16;
  static constexpr int kSliceBytes = HPW * kHeadBytes;
  static constexpr int kLptWanted = kSliceBytes / PKV_ATTN_LANE_BYTES;
  static constexpr int kLptCap = kVecPerHead < 8 ? kVecPerHead : 8;
  static constexpr int kLpt = kLptWanted < 1 ? 1 : (kLptWanted > kLptCap ? kLptCap : kLptWanted);
  static_assert(kVecPerHead % kLpt == 0, "the lanes of a row split every head alike");
  static constexpr int kVph = kVecPerHead / kLpt;  // vectors per lane per head
  static constexpr int kVpl = HPW * kVph;
  static constexpr int kEpv = 16 / kEsize;  // elements per 16-byte vector
  static constexpr int kDph = kVph * kEpv;  // dimensions per lane per head
  static constexpr int kDpl = kVpl * kEpv;
  static constexpr int kTpr = kWave / kLpt;
  static constexpr int kIterWanted = kIterBytes / kSliceBytes < 64 ? kIterBytes / kSliceBytes : 64;
  static constexpr int kRounds = kTpr >= kIterWanted ? 1 : kIterWanted / kTpr;
  static constexpr int kIterTok = kTpr * kRounds;
  static constexpr int kGroups = kWaves * kTpr;  // lane groups per workgroup
};

// Heads per row_partial workgroup: two when one head row is at most 256 bytes and the heads pair
// up, so every token row is read as a slice of at least 512 contiguous bytes.
template <typename KVT, int D>
constexpr bool kPairHeads = D * KVTraits<KVT>::kEsize <= 256;

// Widen one 16-byte vector into 4 (float) or 8 (bfloat16) floats.
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

// One 16-byte vector of a key or value row. Rows read once by the whole call stream past the
// caches (non-temporal); rows shared by several sequences of the batch are loaded normally so
// the other readers hit L2 / the Infinity Cache.
template <bool kStream>
__device__ __forceinline__ uint4 load_row(const uint4* p) {
  if constexpr (kStream && PKV_ATTN_NONTEMPORAL) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *p;
  }
}

// One 16-byte pool vector (16 / sizeof(KVT) elements) of a new key or value row, from element
// `elem` of the append source, in the pool's element type: equal types copy bits, float32 into a
// bfloat16 pool rounds to nearest even, exactly what pkv_append stores.
__device__ __forceinline__ uint4 new_row_vector(const Params&, const void* src, int64_t elem, float) {
  return *reinterpret_cast<const uint4*>(static_cast<const float*>(src) + elem);
}
__device__ __forceinline__ uint4 new_row_vector(const Params& a, const void* src, int64_t elem, uint16_t) {
  if (a.new_dtype == PKV_BF16) return *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(src) + elem);
  const float4 x = reinterpret_cast<const float4*>(static_cast<const float*>(src) + elem)[0];
  const float4 y = reinterpret_cast<const float4*>(static_cast<const float*>(src) + elem)[1];
  return make_uint4(f32_to_bf16_bits(x.x) | (f32_to_bf16_bits(x.y) << 16),
                    f32_to_bf16_bits(x.z) | (f32_to_bf16_bits(x.w) << 16),
                    f32_to_bf16_bits(y.x) | (f32_to_bf16_bits(y.y) << 16),
                    f32_to_bf16_bits(y.z) | (f32_to_bf16_bits(y.w) << 16));
}

// Visible key count of a query: keys at positions 0 .. min(context_len, position + 1) - 1.
__device__ __forceinline__ int visible_len(int ctx, int pos) {
  if (pos < 0) return 0;
  return pos >= ctx ? ctx : pos + 1;
}

__device__ __forceinline__ int row_visible(const Params& a, int64_t t) {
  const int seq = a.q_seq[t];
  if (seq < 0 || seq >= a.num_seqs) return 0;
  return min(visible_len(a.ctx_lens[seq], a.q_pos[t]), a.max_ctx);
}

// Row of the caller's queries / out / new key and value arrays that planner row t reads and
// writes (t itself without q_rows); -1 when q_rows names a row outside the batch, which the
// kernels then skip.
__device__ __forceinline__ int64_t io_row(const Params& a, int64_t t) {
  if (a.q_rows == nullptr) return t;
  const int64_t r = a.q_rows[t];
  return r >= 0 && r < a.num_queries ? r : -1;
}

__device__ __forceinline__ int parts_of(int visible, int part_size) {
  return visible > part_size ? (visible + part_size - 1) / part_size : 1;
}

template <bool kPow2Block>
__device__ __forceinline__ int block_of(int pos, const Params& a) {
  return kPow2Block ? (pos >> a.block_shift) : (pos / a.block_size);
}

// Stage table entries of blocks [b0, b0 + nb) of sequence `seq` into LDS.
__device__ __forceinline__ void stage_table(int* s_table, const Params& a, int seq, int b0, int nb,
                                            int threads) {
  const int32_t* table = a.tables + static_cast<int64_t>(seq) * a.table_stride + b0;
  for (int i = threadIdx.x; i < nb; i += threads) s_table[i] = table[i];
}

// Write one query row's partition result: final output (row r of out) when the row fits one
// partition, otherwise the unnormalised (max, sum, acc) of planner row t for the reduce pass.
__device__ __forceinline__ void store_result(const Params& a, int64_t t, int64_t r, int h, int p,
                                             int nparts, int d, int D, float acc, float big,
                                             float sum, bool write_ml) {
  const int64_t qh = t * a.num_heads + h;
  if (nparts == 1) {
    a.out[(r * a.num_heads + h) * D + d] = acc / (sum > 0.f ? sum : 1.f);
  } else {
    const int64_t slot = qh * a.max_parts + p;
    a.ws_acc[slot * D + d] = acc;
    if (write_ml) {
      a.ws_ml[2 * slot] = big;
      a.ws_ml[2 * slot + 1] = sum;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Pass 1: row_partial.
// ---------------------------------------------------------------------------------------------
// kLean: half the bytes in flight per wavefront (112 instead of 176 VGPRs at float32 head_dim
// 128), so twice as many workgroups fit on a CU; chosen for batches whose row-pass items are
// short, where the workgroups' set-up and latency, not their streaming, dominate (measured: the
// 256-sequence prefix-sharing step's attention 0.242 -> 0.228 ms; long items are unchanged or
// slower beside the tile pass).
// kAppend: the decode append fused into the pass (pkv_paged_attention_append); a separate
// instantiation, so the plain pass keeps its register budget.
template <typename KVT, int D, int HPW, bool kPow2Block, bool kStream, bool kLean, bool kAppend>
__global__ __launch_bounds__(kThreads) void row_partial_kernel(const Params a) {
  using L = Layout<KVT, D, HPW, kLean ? PKV_ATTN_ITER_BYTES / 2 : PKV_ATTN_ITER_BYTES>;
  constexpr int kSlice = HPW * D;  // elements of the token-row slice this workgroup reads
  __shared__ int s_table[kTableSlots];
  __shared__ float s_m[L::kGroups * HPW];
  __shared__ float s_l[L::kGroups * HPW];
  __shared__ float s_acc[L::kGroups * kSlice];

  // Grid: head groups fastest, then partitions, then rows.
  const uint32_t bid = logical_block();
  const uint32_t head_groups = static_cast<uint32_t>(a.num_heads / HPW);
  const int h = static_cast<int>(bid % head_groups) * HPW;  // first head of the group
  const uint32_t rest = bid / head_groups;
  // With a plan, work item `rest` names its (query row, partition); without one, every
  // partition of every row.
  int64_t t;
  int p;
  if (a.rows) {
    t = a.rows[2 * static_cast<int64_t>(rest)];
    p = a.rows[2 * static_cast<int64_t>(rest) + 1];
  } else {
    t = rest / static_cast<uint32_t>(a.max_parts);
    p = static_cast<int>(rest % static_cast<uint32_t>(a.max_parts));
  }
  if (t < 0 || t >= a.num_queries || p < 0) return;  // an item outside the batch is skipped
  const int64_t r = io_row(a, t);
  if (r < 0) return;

  const int seq = a.q_seq[t];
  const int kv_len = row_visible(a, t);
  const int nparts = parts_of(kv_len, a.part_size);
  if (p >= nparts) return;
  const int kbeg = p * a.part_size;
  const int kend = min(kbeg + a.part_size, kv_len);

  const int b0 = block_of<kPow2Block>(kbeg, a);
  const int nb = kend > kbeg ? block_of<kPow2Block>(kend - 1, a) - b0 + 1 : 0;
  if (nb > 0) stage_table(s_table, a, seq, b0, nb, kThreads);
  __syncthreads();

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int g = lane / L::kLpt;  // token slot inside a load round
  const int j = lane % L::kLpt;  // position inside the slice

  // Element (i * kLpt + j) * kEpv + e of the slice is dimension ((i % kVph) * kLpt + j) * kEpv +
  // e of head h + i / kVph; the heads of a group are adjacent in both queries and pools.
  float qv[L::kDpl];
  {
    const float* qrow = a.queries + r * a.q_stride + static_cast<int64_t>(h) * D;
#pragma unroll
    for (int i = 0; i < L::kVpl; ++i) {
#pragma unroll
      for (int e = 0; e < L::kEpv; ++e) {
        qv[i * L::kEpv + e] = qrow[(i * L::kLpt + j) * L::kEpv + e] * a.scale_log2;
      }
    }
  }

  float m[HPW];
  float l[HPW];
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) {
    m[hh] = -INFINITY;
    l[hh] = 0.f;
  }
  float acc[L::kDpl];
#pragma unroll
  for (int d = 0; d < L::kDpl; ++d) acc[d] = 0.f;

  const KVT* kcache = static_cast<const KVT*>(a.kcache);
  const KVT* vcache = static_cast<const KVT*>(a.vcache);
  const int64_t head_off = static_cast<int64_t>(h) * D;
  const int64_t row_stride = static_cast<int64_t>(a.num_heads) * D;  // elements per token row
  // With the fused append, the key position of this row's own new token. It is the row's last
  // visible key (the query sits at its own position), so it lies in the row's last partition.
  // The full-size workgroups take it from the append source inside the loop, in the load round
  // that reaches it. The lean ones, whose workgroups must keep to the plain lean pass's
  // registers to fit three of them beside a tile workgroup (3 x 112 + 168 <= 512 per SIMD), stop
  // the loop one key short and take it before the loop in one lane group: a branch inside the
  // loop takes them to 124 registers (measured: config 4's attention 0.22 -> 0.30 ms), while the
  // full-size pass is quicker with the branch (config 2: 0.722 against 0.732 ms).
  const int own_pos = kAppend ? a.q_pos[t] : -1;
  const bool own_here = kAppend && own_pos >= kbeg && own_pos < kend;
  const int kloop = kLean && own_here ? own_pos : kend;
  const int n_iter = (kloop - kbeg + L::kIterTok - 1) / L::kIterTok;
  const int64_t own_key = r * a.new_key_stride + head_off;
  const int64_t own_value = r * a.new_value_stride + head_off;

  if constexpr (kAppend && kLean) {
    // The row's own new token, in its last partition: before the loop (few registers are live
    // yet), lane group 0 of the last wavefront (the one the loop's round robin gives the fewest
    // steps) takes its key and value from the append source (in the pool's element type, as
    // pkv_append stores them), writes them to the token's slot (the workgroup of each head group
    // writes its slice) and starts its softmax state with them. A block id outside the pool
    // masks the key and writes nothing (its slot, formed from the same table, lies outside too).
    if (own_here && wave == kWaves - 1) {
      const int lb = block_of<kPow2Block>(own_pos, a) - b0;
      const int blk = s_table[lb];
      const bool ok = g == 0 && blk >= 0 && blk < a.num_blocks;
      uint4 kr[L::kVpl];
      uint4 vr[L::kVpl];
#pragma unroll
      for (int i = 0; i < L::kVpl; ++i) {
        const int64_t e = static_cast<int64_t>(i * L::kLpt + j) * L::kEpv;
        kr[i] = ok ? new_row_vector(a, a.new_keys, own_key + e, KVT{}) : make_uint4(0, 0, 0, 0);
        vr[i] = ok ? new_row_vector(a, a.new_values, own_value + e, KVT{}) : make_uint4(0, 0, 0, 0);
      }
      const int64_t slot = a.new_slots[r];
      if (ok && slot >= 0 && slot < a.num_slots) {
        uint4* kd = reinterpret_cast<uint4*>(const_cast<KVT*>(kcache) + slot * row_stride + head_off);
        uint4* vd = reinterpret_cast<uint4*>(const_cast<KVT*>(vcache) + slot * row_stride + head_off);
#pragma unroll
        for (int i = 0; i < L::kVpl; ++i) {
          kd[i * L::kLpt + j] = kr[i];
          vd[i * L::kLpt + j] = vr[i];
        }
      }
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) {
        float dot = 0.f;
#pragma unroll
        for (int i = hh * L::kVph; i < (hh + 1) * L::kVph; ++i) {
          float kf[L::kEpv];
          widen(kr[i], kf, KVT{});
#pragma unroll
          for (int e = 0; e < L::kEpv; ++e) dot = fmaf(qv[i * L::kEpv + e], kf[e], dot);
        }
        dot = group_sum<L::kLpt>(dot);
        const float sc = ok ? dot : -INFINITY;
        const float mx = fmaxf(m[hh], sc);
        const float shift = mx == -INFINITY ? 0.f : mx;
        const float alpha = fast_exp2(m[hh] - shift);
        const float pr = fast_exp2(sc - shift);
        l[hh] = fmaf(l[hh], alpha, pr);
        m[hh] = mx;
#pragma unroll
        for (int i = hh * L::kVph; i < (hh + 1) * L::kVph; ++i) {
          float vf[L::kEpv];
          widen(vr[i], vf, KVT{});
#pragma unroll
          for (int e = 0; e < L::kEpv; ++e) acc[i * L::kEpv + e] = fmaf(pr, vf[e], acc[i * L::kEpv + e] * alpha);
        }
      }
    }
  }

  for (int it = wave; it < n_iter; it += kWaves) {
    const int base = kbeg + it * L::kIterTok;
    uint4 kraw[L::kRounds][L::kVpl];
    uint4 vraw[L::kRounds][L::kVpl];
    bool valid[L::kRounds];
#pragma unroll
    for (int rr = 0; rr < L::kRounds; ++rr) {
      const int kpos = base + rr * L::kTpr + g;
      bool ok = kpos < kloop;
      int64_t row = 0;
      if (ok) {
        const int lb = block_of<kPow2Block>(kpos, a) - b0;
        const int off = kpos - (lb + b0) * a.block_size;
        const int blk = s_table[lb];
        ok = blk >= 0 && blk < a.num_blocks;
        row = (static_cast<int64_t>(blk) * a.block_size + off) * row_stride + head_off;
      }
      valid[rr] = ok;
      if (kAppend && !kLean && kpos == own_pos && kpos < kend) {
        // This row's own new token: its key and value come from the append source and are
        // written to the token's slot here (the workgroup of each head group writes its slice).
#pragma unroll
        for (int i = 0; i < L::kVpl; ++i) {
          const int64_t e = static_cast<int64_t>(i * L::kLpt + j) * L::kEpv;
          kraw[rr][i] = new_row_vector(a, a.new_keys, own_key + e, KVT{});
          vraw[rr][i] = new_row_vector(a, a.new_values, own_value + e, KVT{});
        }
        const int64_t slot = a.new_slots[r];
        if (slot >= 0 && slot < a.num_slots) {
          uint4* kd = reinterpret_cast<uint4*>(const_cast<KVT*>(kcache) + slot * row_stride + head_off);
          uint4* vd = reinterpret_cast<uint4*>(const_cast<KVT*>(vcache) + slot * row_stride + head_off);
#pragma unroll
          for (int i = 0; i < L::kVpl; ++i) {
            kd[i * L::kLpt + j] = kraw[rr][i];
            vd[i * L::kLpt + j] = vraw[rr][i];
          }
        }
        if (!ok) {  // a block id outside the pool masks the key, as it would after pkv_append
#pragma unroll
          for (int i = 0; i < L::kVpl; ++i) {
            kraw[rr][i] = make_uint4(0, 0, 0, 0);
            vraw[rr][i] = make_uint4(0, 0, 0, 0);
          }
        }
      } else if (ok) {
        const uint4* kp = reinterpret_cast<const uint4*>(kcache + row);
        const uint4* vp = reinterpret_cast<const uint4*>(vcache + row);
#pragma unroll
        for (int i = 0; i < L::kVpl; ++i) kraw[rr][i] = load_row<kStream>(kp + i * L::kLpt + j);
#pragma unroll
        for (int i = 0; i < L::kVpl; ++i) vraw[rr][i] = load_row<kStream>(vp + i * L::kLpt + j);
      } else {
#pragma unroll
        for (int i = 0; i < L::kVpl; ++i) {
          kraw[rr][i] = make_uint4(0, 0, 0, 0);
          vraw[rr][i] = make_uint4(0, 0, 0, 0);
        }
      }
    }

    // Scores of this lane group's rows (base-2 units) for each head, reduced over the kLpt lanes
    // of a row.
    float s[L::kRounds][HPW];
#pragma unroll
    for (int rr = 0; rr < L::kRounds; ++rr) {
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) {
        float dot = 0.f;
#pragma unroll
        for (int i = hh * L::kVph; i < (hh + 1) * L::kVph; ++i) {
          float kf[L::kEpv];
          widen(kraw[rr][i], kf, KVT{});
#pragma unroll
          for (int e = 0; e < L::kEpv; ++e) dot = fmaf(qv[i * L::kEpv + e], kf[e], dot);
        }
        dot = group_sum<L::kLpt>(dot);
        s[rr][hh] = valid[rr] ? dot : -INFINITY;
      }
    }

    // Online softmax update, per head.
    float pr[L::kRounds][HPW];
    float alpha[HPW];
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
      float mx = m[hh];
#pragma unroll
      for (int rr = 0; rr < L::kRounds; ++rr) mx = fmaxf(mx, s[rr][hh]);
      const float shift = mx == -INFINITY ? 0.f : mx;
      alpha[hh] = fast_exp2(m[hh] - shift);
      float psum = 0.f;
#pragma unroll
      for (int rr = 0; rr < L::kRounds; ++rr) {
        pr[rr][hh] = fast_exp2(s[rr][hh] - shift);
        psum += pr[rr][hh];
      }
      l[hh] = fmaf(l[hh], alpha[hh], psum);
      m[hh] = mx;
    }
#pragma unroll
    for (int d = 0; d < L::kDpl; ++d) acc[d] *= alpha[d / L::kDph];
#pragma unroll
    for (int rr = 0; rr < L::kRounds; ++rr) {
#pragma unroll
      for (int i = 0; i < L::kVpl; ++i) {
        float vf[L::kEpv];
        widen(vraw[rr][i], vf, KVT{});
        const float w = pr[rr][i / L::kVph];
#pragma unroll
        for (int e = 0; e < L::kEpv; ++e) {
          acc[i * L::kEpv + e] = fmaf(w, vf[e], acc[i * L::kEpv + e]);
        }
      }
    }
  }

  // Merge the kGroups partial states of the workgroup, head by head.
  const int grp = wave * L::kTpr + g;
  if (j == 0) {
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
      s_m[grp * HPW + hh] = m[hh];
      s_l[grp * HPW + hh] = l[hh];
    }
  }
#pragma unroll
  for (int i = 0; i < L::kVpl; ++i) {
#pragma unroll
    for (int e = 0; e < L::kEpv; ++e) {
      s_acc[grp * kSlice + (i * L::kLpt + j) * L::kEpv + e] = acc[i * L::kEpv + e];
    }
  }
  __syncthreads();

  for (int x = threadIdx.x; x < kSlice; x += kThreads) {
    const int hh = x / D;
    const int d = x - hh * D;
    float big = -INFINITY;
    for (int k = 0; k < L::kGroups; ++k) big = fmaxf(big, s_m[k * HPW + hh]);
    const float shift = big == -INFINITY ? 0.f : big;
    float lsum = 0.f;
    float sum_acc = 0.f;
    for (int k = 0; k < L::kGroups; ++k) {
      const float w = fast_exp2(s_m[k * HPW + hh] - shift);
      lsum = fmaf(s_l[k * HPW + hh], w, lsum);
      sum_acc = fmaf(s_acc[k * kSlice + x], w, sum_acc);
    }
    store_result(a, t, r, h + hh, p, nparts, d, D, sum_acc, big, lsum, d == 0);
  }
}

// ---------------------------------------------------------------------------------------------
// Pass 2: tile_partial (fp32 MFMA). Lane l of a wavefront is (c = l / 16, n = l % 16); wavefront
// w owns the tile's queries 16w .. 16w + 15. Keys are staged in LDS kKeys at a time, as kSub
// column blocks of 16 keys.
//
//   S^T = K Q^T  with v_mfma_f32_16x16x4f32, kD4 = D / 4 steps per 16-key block j. In step s, the
//                k index of lane group c stands for head dimension c * kD4 + s, so lane (c, n)
//                supplies A = K[key 16j + n][c * kD4 + s] (from LDS) and B = Q[query n][c * kD4
//                + s] (from registers). Register r of block j holds S[query n][key 16j + 4c + r].
//                The kSub chains are independent and interleaved.
//   O^T = V^T P^T  four steps per 16-key block; in step m the k index of lane group c stands for
//                key 16j + 4c + m. Output tile b = kW g + e (kW = 4, or 2 at head_dim 32) covers
//                dims 16 kW g + kW i + e, i = 0..15, so lane (c, n) supplies A = V[key 16j + 4c +
//                m][16 kW g + kW n + e] for the kW tiles of group g from one LDS read of kW
//                adjacent floats, and B = P[query n][key 16j + 4c + m], its own register m.
//                Register r of tile b holds O[query n][16 kW g + kW (4c + r) + e]: every lane owns
//                dimensions of its own query's output row only, so rescaling a row needs only the
//                lane's own factor.
//
// Online softmax with a lazy reference: probabilities are exp2(s - m_ref), where m_ref is a
// running maximum that is only raised when some score of a query exceeds it by more than
// kLazyLog2 (then every p stays <= 2^kLazyLog2, far from float overflow). Raising it rescales the
// query's output row and sum; the branch is taken by the whole wavefront only when one of its
// queries needs it, which after the first key tile is rare. A query's four lanes keep partial
// sums of their own keys, summed once at the end. The result is acc / l relative to the same
// m_ref, which the reduce pass merges like any other (max, sum, acc) triple.
// ---------------------------------------------------------------------------------------------
constexpr float kLazyLog2 = 8.f;

// Maximum / sum over the four lanes {n, n + 16, n + 32, n + 48} of a wavefront. With the same
// register as both operands, v_permlane16_swap returns in each lane the two values of the lane
// pair {l, l ^ 16} (one per result) and v_permlane32_swap those of {l, l ^ 32}.
__device__ __forceinline__ float column_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float column_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// One 16-byte global load per lane written straight into LDS (global_load_lds_dwordx4): lane l
// of the wavefront writes LDS bytes [lds + 16 l, lds + 16 l + 16). `lds` is the wavefront-uniform
// LDS byte address, which the instruction takes in M0, set in the same statement (with the one
// wait state GFX9 requires between an SALU write of M0 and an LDS DMA). The compiler does not
// see these loads, so their completion is waited for explicitly (wait_vmcnt) before the barrier
// that publishes the data.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void load_to_lds16(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(N), leaving the other counters alone (gfx9 encoding: vmcnt in bits 3:0 and
// 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// A workgroup barrier that orders LDS accesses only: unlike __syncthreads it does not wait for
// outstanding global loads, so loads into the other LDS stages stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int D>
struct TileShape {
  static constexpr int kKeys = D <= 128 ? 32 : 16;  // keys per LDS tile (registers bound D = 256)
  static constexpr int kSub = kKeys / 16;
  static constexpr int kRow = D + 4;                 // padded LDS row (floats): conflict-free reads
  static constexpr int kD4 = D / 4;
  static constexpr int kNb = D / 16;
  // Output dims of the O^T products: MFMA row i of output tile b = kW g + e holds dimension
  // 16 kW g + kW i + e. Lane n's A operands of the kW tiles of group g are then kW adjacent
  // floats of a value row (one LDS vector read feeds kW products), and registers r of those
  // tiles in lane (c, n) are the kW adjacent output dims 16 kW g + kW (4 c + r) + [0, kW).
  static constexpr int kW = kNb >= 4 ? 4 : kNb;
  static constexpr int kGroups = kNb / kW;
  // Direct-to-LDS stages: unpadded rows of D floats whose 16-byte chunks are XOR-swizzled by
  // (row & 7): chunk q of key row r sits at chunk q ^ (r & 7). The S^T reads (16 rows, one
  // chunk each) and the PV reads (4 rows, 16 adjacent chunks each) then spread over all LDS
  // banks, as the padded rows do, while every 16-byte chunk stays whole for the DMA.
  static constexpr int kChunks = kKeys * D / 4;            // 16-byte chunks of one K (or V) tile
  static constexpr int kTileFloats = kKeys * D;
  static constexpr int kStageFloats = 2 * kTileFloats;     // K tile then V tile
};

// LDS float offset of element `col` of key row `row` in a swizzled direct-to-LDS tile.
template <int D>
__device__ __forceinline__ int swz(int row, int col) {
  return row * D + ((((col >> 2) ^ (row & 7))) << 2) + (col & 3);
}

// kW adjacent floats, the unit of one value-operand read and one output store of the tile pass.
template <int W>
using floatw = float __attribute__((ext_vector_type(W)));

// One query row of the tile pass's O^T products, divided by `sum` (1 for the unnormalised
// workspace rows), stored at `dst` (the row's dimension 0) when output tile W g + e holds dims
// 16 W g + W i + e: lane (c, n) writes the W adjacent dims of each (group, register) pair.
template <int D, int W>
__device__ __forceinline__ void store_out_row(float* dst, const floatx4 (&o)[D / 16], int c, float sum) {
  constexpr int kGroups = D / 16 / W;
#pragma unroll
  for (int g = 0; g < kGroups; ++g) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      floatw<W> x;
#pragma unroll
      for (int e = 0; e < W; ++e) x[e] = o[W * g + e][r] / sum;
      *reinterpret_cast<floatw<W>*>(dst + 16 * W * g + W * (4 * c + r)) = x;
    }
  }
}

// One work item of the tile pass staged through registers: item `bid` = (partition, tile, head),
// heads fastest, partitions slowest (a whole tile's work is all in partition 0, so those items
// come first). Every thread of the workgroup calls it with the same item; it returns early
// (uniformly) for items outside the tile's partitions.
template <typename KVT, int D, bool kPow2Block>
__device__ __forceinline__ void tile_item(const Params& a, uint32_t bid, int* s_table, float* s_k,
                                          float* s_v, int* s_vis) {
  static_assert(D % 16 == 0 && D >= 32, "the MFMA tile needs whole 16-wide output tiles");
  using S = TileShape<D>;
  constexpr int kKeys = S::kKeys;
  constexpr int kSub = S::kSub;
  constexpr int kRow = S::kRow;
  constexpr int kD4 = S::kD4;
  constexpr int kNb = S::kNb;
  constexpr int kEsize = KVTraits<KVT>::kEsize;
  constexpr int kEpv = 16 / kEsize;  // elements per 16-byte vector
  constexpr int kVecPerRow = D / kEpv;

  const int h = static_cast<int>(bid % static_cast<uint32_t>(a.num_heads));
  const uint32_t rest = bid / static_cast<uint32_t>(a.num_heads);
  const int64_t tile = rest % static_cast<uint32_t>(a.num_tiles);
  const int p = static_cast<int>(rest / static_cast<uint32_t>(a.num_tiles));
  const int32_t* entry = a.tiles + 4 * tile;
  const int64_t t0 = entry[0];
  if (t0 < 0 || t0 >= a.num_queries) return;  // a tile outside the batch is skipped
  // A whole tile is computed by its partition-0 workgroup alone, over every visible key.
  const bool whole = entry[3] == kTileWhole;
  if (whole ? p != 0 : (p < entry[2] || (entry[3] > entry[2] && p >= entry[3]))) return;
  const int nrows = static_cast<int>(min<int64_t>(min(entry[1], kTileRows), a.num_queries - t0));
  const int seq = a.q_seq[t0];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  if (threadIdx.x < kTileRows) {
    s_vis[threadIdx.x] = static_cast<int>(threadIdx.x) < nrows ? row_visible(a, t0 + threadIdx.x) : 0;
  }
  __syncthreads();
  // The tile's longest visible row bounds its partitions (every wavefront reads all 64 entries).
  int tile_vis = s_vis[lane];
#pragma unroll
  for (int mask = 32; mask > 0; mask >>= 1) tile_vis = max(tile_vis, __shfl_xor(tile_vis, mask));
  tile_vis = __builtin_amdgcn_readfirstlane(tile_vis);  // the same in every lane: keep it scalar
  const int nparts = parts_of(tile_vis, a.part_size);
  if (!whole && p >= nparts) return;
  const int kbeg = whole ? 0 : p * a.part_size;
  const int kend = whole ? tile_vis : min(kbeg + a.part_size, tile_vis);
  // The table entries of blocks [b0, b0 + kTableSlots) are staged in LDS. A partition always
  // fits; a whole tile moves the window forward when the next key tile would leave it.
  const int last_block = kend > kbeg ? block_of<kPow2Block>(kend - 1, a) : -1;
  int b0 = block_of<kPow2Block>(kbeg, a);
  auto stage_window = [&]() {
    const int nb = min(last_block - b0 + 1, kTableSlots);
    if (nb > 0) stage_table(s_table, a, seq, b0, nb, kTileThreads);
  };
  stage_window();

  const int c = lane >> 4;
  const int n = lane & 15;
  const int qi = wave * 16 + n;  // this lane's query in the S^T layout
  const int my_vis = s_vis[qi];
  const bool q_ok = qi < nrows;

  // This lane's row of queries and out (-1: a caller row outside the batch, skipped).
  const int io = static_cast<int>(io_row(a, t0 + (q_ok ? qi : 0)));
  float qreg[kD4];
  {
    // Lanes past the tile read row t0 (always in the batch) and drop it, so every load is
    // unconditional and the 32 loads of a lane can all be in flight together.
    const float* qrow =
        a.queries + static_cast<int64_t>(io < 0 ? 0 : io) * a.q_stride + static_cast<int64_t>(h) * D + c * kD4;
    float raw[kD4];
#pragma unroll
    for (int s = 0; s < kD4; ++s) raw[s] = qrow[s];
#pragma unroll
    for (int s = 0; s < kD4; ++s) qreg[s] = q_ok ? raw[s] * a.scale_log2 : 0.f;
  }

  floatx4 o[kNb];
#pragma unroll
  for (int b = 0; b < kNb; ++b) o[b] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_ref = -INFINITY;  // the same in the four lanes of a query
  float l_part = 0.f;       // this lane's share of the query's sum

  const KVT* kcache = static_cast<const KVT*>(a.kcache);
  const KVT* vcache = static_cast<const KVT*>(a.vcache);
  const int64_t head_off = static_cast<int64_t>(h) * D;
  const int64_t row_stride = static_cast<int64_t>(a.num_heads) * D;
  __syncthreads();  // s_table ready

  const int lim = min(my_vis, kend);
  int wave_lim = lim;  // the wavefront's last key + 1: key tiles from there on are all masked
#pragma unroll
  for (int mask = 32; mask > 0; mask >>= 1) wave_lim = max(wave_lim, __shfl_xor(wave_lim, mask));
  wave_lim = __builtin_amdgcn_readfirstlane(wave_lim);
  // Every row of the wavefront sees the keys below wave_full: a key tile that ends by then, with
  // every key in a block inside the pool (all bits of its key mask set), needs no per-key mask.
  int wave_full = q_ok ? lim : INT32_MAX;
#pragma unroll
  for (int mask = 32; mask > 0; mask >>= 1) wave_full = min(wave_full, __shfl_xor(wave_full, mask));
  wave_full = __builtin_amdgcn_readfirstlane(wave_full);
  constexpr uint32_t kAllKeys = static_cast<uint32_t>((uint64_t{1} << kKeys) - 1u);

  // One key tile's scores st -> probabilities pr, updating the running reference and sum. A key
  // counts when it is below the lane's limit and its bit in kmask is set.
  auto softmax_step = [&](floatx4 (&st)[kSub], int k0, uint32_t kmask, float (&pr)[kSub][4]) {
    float sc[kSub][4];
    float mx = -INFINITY;
    if (k0 + kKeys <= wave_full && kmask == kAllKeys) {  // wavefront-uniform: nothing masked
#pragma unroll
      for (int j = 0; j < kSub; ++j) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[j][r] = st[j][r];
          mx = fmaxf(mx, sc[j][r]);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < kSub; ++j) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int kk = 16 * j + 4 * c + r;
          sc[j][r] = (k0 + kk) < lim && ((kmask >> kk) & 1u) ? st[j][r] : -INFINITY;
          mx = fmaxf(mx, sc[j][r]);
        }
      }
    }
    mx = column_max(mx);
    // Raise the reference only when a score passes it by more than kLazyLog2 (or it is unset).
    const bool raise = mx > m_ref + kLazyLog2 || (m_ref == -INFINITY && mx > -INFINITY);
    // Skip the multiplies when no lane raises (fewer VGPRs than a branch-free rescale).
    if (__builtin_amdgcn_ballot_w64(raise) != 0) {
      const float m_next = raise ? mx : m_ref;
      const float alpha = raise ? fast_exp2(m_ref - m_next) : 1.f;  // exp2(-inf) = 0
      l_part *= alpha;
#pragma unroll
      for (int b = 0; b < kNb; ++b) o[b] *= alpha;
      m_ref = m_next;
    }
    const float shift = m_ref == -INFINITY ? 0.f : m_ref;
#pragma unroll
    for (int j = 0; j < kSub; ++j) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pr[j][r] = fast_exp2(sc[j][r] - shift);
        l_part += pr[j][r];
      }
    }
  };

  // Software pipeline: the raw vectors of key tile k0 + kKeys are loaded into registers while
  // tile k0 is being multiplied; at the top of each step they are widened into LDS.
  constexpr int kVecs = kKeys * kVecPerRow;  // 16-byte vectors per K (or V) tile
  constexpr int kPerThread = (kVecs + kTileThreads - 1) / kTileThreads;
  uint4 kraw[kPerThread];
  uint4 vraw[kPerThread];
  // The prefetched tile's key mask (keys before kend in blocks inside the pool), a wavefront
  // ballot kept in scalar registers until the tile's scores are masked.
  uint32_t mask_next = 0u;
  const uint32_t pool_blocks = static_cast<uint32_t>(min<int64_t>(a.num_blocks, INT32_MAX));
  auto prefetch = [&](int k0) {
    {
      const int kpos = k0 + lane;
      const int lb = min(max(block_of<kPow2Block>(kpos, a) - b0, 0), kTableSlots - 1);
      const int blk = s_table[lb];
      const bool ok = (lane < kKeys) & (kpos < kend) & (static_cast<uint32_t>(blk) < pool_blocks);
      mask_next = static_cast<uint32_t>(__builtin_amdgcn_ballot_w64(ok));
    }
    // One branch per vector: a key past kend or in a block outside the pool keeps zeros (its
    // table entry is read at a clamped index and not used).
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) {
      const int v = threadIdx.x + u * kTileThreads;
      const int row = v / kVecPerRow;
      const int col = (v - row * kVecPerRow) * kEpv;
      const int kpos = k0 + row;
      const int lb = min(max(block_of<kPow2Block>(kpos, a) - b0, 0), kTableSlots - 1);
      const int blk = s_table[lb];
      const bool ok = (kVecs % kTileThreads == 0 || v < kVecs) & (kpos < kend) &
                      (static_cast<uint32_t>(blk) < pool_blocks);
      kraw[u] = make_uint4(0, 0, 0, 0);
      vraw[u] = make_uint4(0, 0, 0, 0);
      if (ok) {
        const int64_t off =
            (static_cast<int64_t>(blk) * a.block_size + (kpos - (lb + b0) * a.block_size)) * row_stride +
            head_off + col;
        kraw[u] = *reinterpret_cast<const uint4*>(kcache + off);
        vraw[u] = *reinterpret_cast<const uint4*>(vcache + off);
      }
    }
  };
  if (kbeg < kend) prefetch(kbeg);

  for (int k0 = kbeg; k0 < kend; k0 += kKeys) {
    const uint32_t kmask = mask_next;  // this tile's, from its prefetch
    // Every read of s_table by the last prefetch happened before the previous barrier, so the
    // window can move here; the barrier below publishes it before the next prefetch reads it.
    const int next = k0 + kKeys;
    if (next < kend && block_of<kPow2Block>(min(next + kKeys, kend) - 1, a) >= b0 + kTableSlots) {
      b0 = block_of<kPow2Block>(next, a);
      stage_window();
    }
    // Widen the prefetched tile (zeros for keys past kend or outside the pool) into LDS as float32.
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) {
      const int v = threadIdx.x + u * kTileThreads;
      if (v < kVecs) {
        const int row = v / kVecPerRow;
        const int col = (v - row * kVecPerRow) * kEpv;
        float kf[kEpv];
        float vf[kEpv];
        widen(kraw[u], kf, KVT{});
        widen(vraw[u], vf, KVT{});
#pragma unroll
        for (int e = 0; e < kEpv; e += 4) {
          *reinterpret_cast<float4*>(&s_k[row * kRow + col + e]) =
              make_float4(kf[e], kf[e + 1], kf[e + 2], kf[e + 3]);
          *reinterpret_cast<float4*>(&s_v[row * kRow + col + e]) =
              make_float4(vf[e], vf[e + 1], vf[e + 2], vf[e + 3]);
        }
      }
    }
    __syncthreads();
    if (k0 + kKeys < kend) prefetch(k0 + kKeys);
    // A wavefront whose rows all end before this key tile skips its products: every score would
    // be masked and every probability 0, so nothing it holds would change.
    if (k0 >= wave_lim) {
      __syncthreads();
      continue;
    }

    // S^T blocks: register r of st[j] = S[query n][key k0 + 16j + 4c + r].
    floatx4 st[kSub];
#pragma unroll
    for (int j = 0; j < kSub; ++j) st[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kD4; ++s) {
#pragma unroll
      for (int j = 0; j < kSub; ++j) {
        st[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(s_k[(16 * j + n) * kRow + c * kD4 + s], qreg[s], st[j], 0, 0, 0);
      }
    }

    float pr[kSub][4];
    softmax_step(st, k0, kmask, pr);

    // O^T += V^T P^T: lane (c, n) reads the kW adjacent floats of group g of value row
    // 16 j + 4 c + step in one LDS read.
#pragma unroll
    for (int j = 0; j < kSub; ++j) {
#pragma unroll
      for (int step = 0; step < 4; ++step) {
        const float* vrow = &s_v[(16 * j + 4 * c + step) * kRow + S::kW * n];
#pragma unroll
        for (int g = 0; g < S::kGroups; ++g) {
          const floatw<S::kW> x = *reinterpret_cast<const floatw<S::kW>*>(vrow + 16 * S::kW * g);
#pragma unroll
          for (int e = 0; e < S::kW; ++e) {
            const int b = S::kW * g + e;
            o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[e], pr[j][step], o[b], 0, 0, 0);
          }
        }
      }
    }
    __syncthreads();
  }

  // Epilogue: register r of tile kW g + e is O[query n][16 kW g + kW (4c + r) + e].
  const float l = column_sum(l_part);
  if (!q_ok) return;
  // A whole tile covered every visible key of its rows: their outputs are final.
  const int row_parts = whole ? 1 : parts_of(my_vis, a.part_size);
  if (p >= row_parts) return;
  const int64_t qh = (t0 + qi) * a.num_heads + h;
  if (row_parts == 1) {
    if (io >= 0) {
      store_out_row<D, S::kW>(a.out + (static_cast<int64_t>(io) * a.num_heads + h) * D, o, c, l > 0.f ? l : 1.f);
    }
  } else {
    const int64_t slot = qh * a.max_parts + p;
    store_out_row<D, S::kW>(a.ws_acc + slot * D, o, c, 1.f);
    if (c == 0) {
      a.ws_ml[2 * slot] = m_ref;
      a.ws_ml[2 * slot + 1] = l;
    }
  }
}

// One work item of the tile pass beside the row pass, float32 pools: the same item as tile_item,
// with the key and value tiles moved from HBM straight into LDS (global_load_lds_dwordx4)
// through kTileStages buffers, all but one in flight while one is multiplied, so no register
// holds a tile on its way. In every step a wavefront whose rows all end before the step's first
// key skips both products: its keys would all be masked (every score -inf, every probability
// 0), so its registers would not change.
template <int D, bool kPow2Block>
__device__ __forceinline__ void tile_item_dma(const Params& a, uint32_t bid, int* s_table, float* s_kv,
                                              int* s_vis) {
  static_assert(D % 16 == 0 && D >= 32, "the MFMA tile needs whole 16-wide output tiles");
  using S = TileShape<D>;
  constexpr int kKeys = S::kKeys;
  constexpr int kSub = S::kSub;
  constexpr int kD4 = S::kD4;
  constexpr int kNb = S::kNb;
  constexpr int kPer = S::kChunks / kTileThreads;  // DMA loads per lane per K (or V) tile
  static_assert(kPer >= 1 && S::kChunks % kTileThreads == 0, "whole wavefront DMA loads per tile");
  constexpr int kCpr = D / 4;  // 16-byte chunks per key row
  constexpr int kAhead = kTileStages - 1;
  constexpr int kVw = S::kW;  // output tile kVw g + e holds dims 16 kVw g + kVw i + e

  const int h = static_cast<int>(bid % static_cast<uint32_t>(a.num_heads));
  const uint32_t rest = bid / static_cast<uint32_t>(a.num_heads);
  const int64_t tile = rest % static_cast<uint32_t>(a.num_tiles);
  const int p = static_cast<int>(rest / static_cast<uint32_t>(a.num_tiles));
  const int32_t* entry = a.tiles + 4 * tile;
  const int64_t t0 = entry[0];
  if (t0 < 0 || t0 >= a.num_queries) return;  // a tile outside the batch is skipped
  // A whole tile is computed by its partition-0 workgroup alone, over every visible key.
  const bool whole = entry[3] == kTileWhole;
  if (whole ? p != 0 : (p < entry[2] || (entry[3] > entry[2] && p >= entry[3]))) return;
  const int nrows = static_cast<int>(min<int64_t>(min(entry[1], kTileRows), a.num_queries - t0));
  const int seq = a.q_seq[t0];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  if (threadIdx.x < kTileRows) {
    s_vis[threadIdx.x] = static_cast<int>(threadIdx.x) < nrows ? row_visible(a, t0 + threadIdx.x) : 0;
  }
  __syncthreads();
  // The tile's longest visible row bounds its partitions (every wavefront reads all 64 entries).
  int tile_vis = s_vis[lane];
#pragma unroll
  for (int mask = 32; mask > 0; mask >>= 1) tile_vis = max(tile_vis, __shfl_xor(tile_vis, mask));
  tile_vis = __builtin_amdgcn_readfirstlane(tile_vis);  // the same in every lane: keep it scalar
  if (!whole && p >= parts_of(tile_vis, a.part_size)) return;
  const int s_beg = whole ? 0 : p * a.part_size;
  const int s_end = whole ? tile_vis : min(s_beg + a.part_size, tile_vis);

  const float* kcache = static_cast<const float*>(a.kcache);
  const float* vcache = static_cast<const float*>(a.vcache);
  const int64_t head_off = static_cast<int64_t>(h) * D;
  const int64_t row_stride = static_cast<int64_t>(a.num_heads) * D;
  const uint32_t lds_kv = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(s_kv));
  // Branch-free address arithmetic (selects, no divergent branches). A block's elements and a
  // token row's fit 31 bits (launch_tiles takes this path only when block_size * num_heads *
  // head_dim does).
  const uint64_t block_elems = static_cast<uint64_t>(a.block_size) * static_cast<uint64_t>(row_stride);
  const uint32_t row_elems = static_cast<uint32_t>(row_stride);
  const uint32_t pool_blocks = static_cast<uint32_t>(min<int64_t>(a.num_blocks, INT32_MAX));
  const int c = lane >> 4;
  const int n = lane & 15;
  const int qi = wave * 16 + n;  // this lane's query in the S^T layout

  // The table entries of blocks [b0, b0 + kTableSlots) are staged in LDS. A partition always
  // fits; a whole tile moves the window forward when the next key tile would leave it.
  const int last_block = s_end > s_beg ? block_of<kPow2Block>(s_end - 1, a) : -1;
  int b0 = block_of<kPow2Block>(s_beg, a);
  auto stage_window = [&]() {
    const int nb = min(last_block - b0 + 1, kTableSlots);
    if (nb > 0) stage_table(s_table, a, seq, b0, nb, kTileThreads);
  };
  stage_window();

  const int my_vis = s_vis[qi];
  const bool q_ok = qi < nrows;
  // This lane's row of queries and out (-1: a caller row outside the batch, skipped).
  const int io = static_cast<int>(io_row(a, t0 + (q_ok ? qi : 0)));
  float qreg[kD4];
  {
    // Lanes past the tile read row t0 (always in the batch) and drop it, so every load is
    // unconditional and the loads of a lane can all be in flight together.
    const float* qrow =
        a.queries + static_cast<int64_t>(io < 0 ? 0 : io) * a.q_stride + static_cast<int64_t>(h) * D + c * kD4;
    float raw[kD4];
#pragma unroll
    for (int i = 0; i < kD4; ++i) raw[i] = qrow[i];
#pragma unroll
    for (int i = 0; i < kD4; ++i) qreg[i] = q_ok ? raw[i] * a.scale_log2 : 0.f;
  }
  floatx4 o[kNb];
#pragma unroll
  for (int b = 0; b < kNb; ++b) o[b] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_ref = -INFINITY;  // the same in the four lanes of a query
  float l_part = 0.f;       // this lane's share of the query's sum
  const int lim = min(my_vis, s_end);
  int wave_lim = lim;  // the wavefront's last key + 1: steps from there on are all masked
#pragma unroll
  for (int mask = 32; mask > 0; mask >>= 1) wave_lim = max(wave_lim, __shfl_xor(wave_lim, mask));
  wave_lim = __builtin_amdgcn_readfirstlane(wave_lim);
  // Every row of the wavefront sees the keys below wave_full: a key tile that ends by then, with
  // every key in a block inside the pool (all bits of its key mask set), needs no per-key mask.
  int wave_full = q_ok ? lim : INT32_MAX;
#pragma unroll
  for (int mask = 32; mask > 0; mask >>= 1) wave_full = min(wave_full, __shfl_xor(wave_full, mask));
  wave_full = __builtin_amdgcn_readfirstlane(wave_full);
  constexpr uint32_t kAllKeys = static_cast<uint32_t>((uint64_t{1} << kKeys) - 1u);
  __syncthreads();  // s_table ready

  // Table entry of key kpos (clamped into the window; callers discard it when kpos is out).
  auto table_at = [&](int kpos) {
    const int lb = min(max(block_of<kPow2Block>(kpos, a) - b0, 0), kTableSlots - 1);
    return s_table[lb];
  };
  // Element offsets of this lane's kPer chunks of key tile k0 (bit u of `valid`: chunk u's key
  // is before the end and in the pool), and the tile's key mask.
  auto prepare = [&](int k0, int lane_v, int64_t (&off)[kPer], uint32_t& valid) -> uint32_t {
    valid = 0u;
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int chunk = (wave * kPer + u) * kWave + lane_v;
      const int row = chunk / kCpr;
      const int col = ((chunk % kCpr) ^ (row & 7)) * 4;
      const int kpos = k0 + row;
      const int blk = table_at(kpos);
      const bool ok = (kpos < s_end) & (static_cast<uint32_t>(blk) < pool_blocks);
      const uint32_t within = kPow2Block ? (kpos & (a.block_size - 1)) : kpos % a.block_size;
      const uint32_t blk_u = ok ? static_cast<uint32_t>(blk) : 0u;
      const uint32_t row_off = ok ? within * row_elems : 0u;
      off[u] = static_cast<int64_t>(blk_u * block_elems) + static_cast<int64_t>(row_off) + head_off + col;
      valid |= ok ? 1u << u : 0u;
    }
    const int kpos = k0 + lane_v;
    const bool ok = (lane_v < kKeys) & (kpos < s_end) &
                    (static_cast<uint32_t>(table_at(kpos)) < pool_blocks);
    return static_cast<uint32_t>(__builtin_amdgcn_ballot_w64(ok));
  };
  // Queue the chunks' loads into stage `buf`; an invalid chunk loads zero_vector.
  auto fire = [&](int buf, const int64_t (&off)[kPer], uint32_t valid) {
    const uint32_t dst = lds_kv + static_cast<uint32_t>(buf * S::kStageFloats * 4 + wave * kPer * 1024);
    const float* zero = reinterpret_cast<const float*>(&zero_vector);
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const bool ok = (valid >> u) & 1u;
      load_to_lds16(ok ? kcache + off[u] : zero, dst + u * 1024);
      load_to_lds16(ok ? vcache + off[u] : zero, dst + u * 1024 + S::kTileFloats * 4);
    }
  };
  // One key tile's scores st -> probabilities pr, updating the running reference and sum. A
  // key counts when it is below the lane's limit and its bit in kmask is set. The rescale is
  // branch-free (alpha is exactly 1 in lanes that keep their reference), so the step stays
  // one block of straight-line code the compiler can interleave.
  auto softmax_step = [&](floatx4 (&st)[kSub], int k0, uint32_t kmask, float (&pr)[kSub][4]) {
    float sc[kSub][4];
    float mx = -INFINITY;
    if (k0 + kKeys <= wave_full && kmask == kAllKeys) {  // wavefront-uniform: nothing masked
#pragma unroll
      for (int j = 0; j < kSub; ++j) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[j][r] = st[j][r];
          mx = fmaxf(mx, sc[j][r]);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < kSub; ++j) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int kk = 16 * j + 4 * c + r;
          sc[j][r] = (k0 + kk) < lim && ((kmask >> kk) & 1u) ? st[j][r] : -INFINITY;
          mx = fmaxf(mx, sc[j][r]);
        }
      }
    }
    mx = column_max(mx);
    // Raise the reference only when a score passes it by more than kLazyLog2 (or it is unset).
    const bool raise = mx > m_ref + kLazyLog2 || (m_ref == -INFINITY && mx > -INFINITY);
    const float m_next = raise ? mx : m_ref;
    const float alpha = raise ? fast_exp2(m_ref - m_next) : 1.f;  // exp2(-inf) = 0
    l_part *= alpha;
#pragma unroll
    for (int b = 0; b < kNb; ++b) o[b] *= alpha;
    m_ref = m_next;
    const float shift = m_ref == -INFINITY ? 0.f : m_ref;
#pragma unroll
    for (int j = 0; j < kSub; ++j) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pr[j][r] = fast_exp2(sc[j][r] - shift);
        l_part += pr[j][r];
      }
    }
  };

  // The pipeline: step i waits for its own loads (vmcnt), then one barrier publishes every
  // wavefront's share and also closes step i - 1, whose buffer the loads of step
  // i + kTileStages - 1 then fill. Those are queued between the step's two products. Every
  // lane issues the same loads in every step, past the last step too: a lane whose key is past
  // the end or in a block outside the pool loads zero_vector instead, and the key's bit in the
  // step's mask stays clear.
  const int nsteps = s_end > s_beg ? (s_end - s_beg + kKeys - 1) / kKeys : 0;
  uint32_t kmask[kAhead];  // key masks of steps i .. i + kAhead - 1
  wait_vmcnt<0>();  // the query loads (and earlier stores) complete before the pipeline's loads
  if (nsteps > 0) {
#pragma unroll
    for (int st = 0; st < kAhead; ++st) {
      int64_t off[kPer];
      uint32_t valid;
      kmask[st] = prepare(s_beg + st * kKeys, lane, off, valid);
      fire(st, off, valid);
    }
  }
  int buf = 0;
  for (int i = 0; i < nsteps; ++i) {
    const int k0 = s_beg + i * kKeys;
    wait_vmcnt<(kAhead - 1) * 2 * kPer>();  // this step's loads have landed
    lds_barrier();
    const int k_next = k0 + kAhead * kKeys;  // the tile whose loads this step queues
    if (block_of<kPow2Block>(min(k_next + kKeys, s_end) - 1, a) >= b0 + kTableSlots) {
      // A whole tile moves its table window; no wavefront reads the table between the barrier
      // above and the one below.
      b0 = block_of<kPow2Block>(k_next, a);
      stage_window();
      lds_barrier();
    }
    const bool work = k0 < wave_lim;  // wavefront-uniform
    // The swizzled LDS addresses are lane constants; they are recomputed from an opaque copy
    // of the lane index each step (a few VALU operations) instead of being hoisted out of the
    // loop, which would hold about 20 more VGPRs and cost the CU a row-pass workgroup.
    int lane_o = lane;
    asm volatile("" : "+v"(lane_o));
    const int cl = lane_o >> 4;
    const int nl = lane_o & 15;
    const float* sk = s_kv + buf * S::kStageFloats;
    const float* sv = sk + S::kTileFloats;

    // S^T blocks: register r of st[j] = S[query n][key k0 + 16j + 4c + r]. Lane (c, n) reads
    // chunk c * kD4 / 4 + q of key row 16 j + n, swizzled by n & 7.
    floatx4 st[kSub];
#pragma unroll
    for (int j = 0; j < kSub; ++j) st[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (work) {
#pragma unroll
      for (int q = 0; q < kD4 / 4; ++q) {
#pragma unroll
        for (int j = 0; j < kSub; ++j) {
          const float4 kv = *reinterpret_cast<const float4*>(
              sk + (16 * j + nl) * D + (((cl * (kD4 / 4) + q) ^ (nl & 7)) << 2));
          st[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.x, qreg[4 * q], st[j], 0, 0, 0);
          st[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.y, qreg[4 * q + 1], st[j], 0, 0, 0);
          st[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.z, qreg[4 * q + 2], st[j], 0, 0, 0);
          st[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.w, qreg[4 * q + 3], st[j], 0, 0, 0);
        }
      }
    }
    // Queue step i + kAhead's loads into the buffer step i - 1 used. Their address arithmetic
    // is scheduled among the PV products below, not the S^T products above (which would keep
    // more registers live across the S^T loop).
    __builtin_amdgcn_sched_barrier(0);
    uint32_t next_mask;
    {
      int64_t off[kPer];
      uint32_t valid;
      next_mask = prepare(k_next, lane_o, off, valid);
      fire(buf == 0 ? kAhead : buf - 1, off, valid);
    }
    if (work) {
      float pr[kSub][4];
      softmax_step(st, k0, kmask[0], pr);
      // O^T += V^T P^T. Lane (c, n) reads the kVw adjacent floats at column 16 kVw g + kVw n
      // of row 16 j + 4 c + step: part of chunk 4 g + n (kVw = 4: the whole chunk) or
      // g + n / 2 (kVw = 2), swizzled by (4 c + step) & 7, so each step needs one lane base and
      // j and g are immediate offsets. The products are accumulated in the register path's
      // order (j, then step, then output tile), so both paths round identically.
#pragma unroll
      for (int j = 0; j < kSub; ++j) {
#pragma unroll
        for (int step = 0; step < 4; ++step) {
          const int swz_row = 4 * (cl & 1) + step;  // (16 j + 4 c + step) & 7
          const int col = kVw * nl;
          const float* vbase = sv + 4 * cl * D + ((((col >> 2) ^ swz_row)) << 2) + (col & 3);
#pragma unroll
          for (int g = 0; g < kNb / kVw; ++g) {
            const floatw<kVw> x =
                *reinterpret_cast<const floatw<kVw>*>(vbase + (16 * j + step) * D + 16 * kVw * g);
#pragma unroll
            for (int e = 0; e < kVw; ++e) {
              const int b = kVw * g + e;
              o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[e], pr[j][step], o[b], 0, 0, 0);
            }
          }
        }
      }
    }
#pragma unroll
    for (int st2 = 0; st2 + 1 < kAhead; ++st2) kmask[st2] = kmask[st2 + 1];
    kmask[kAhead - 1] = next_mask;
    buf = buf == kTileStages - 1 ? 0 : buf + 1;
  }
  wait_vmcnt<0>();  // the loads queued past the last step land before the LDS is reused

  // Epilogue: register r of tile kVw g + e is O[query n][16 kVw g + kVw (4c + r) + e].
  const float l = column_sum(l_part);
  // A whole tile covered every visible key of its rows: their outputs are final.
  const int row_parts = whole ? 1 : parts_of(my_vis, a.part_size);
  if (!q_ok || p >= row_parts) return;
  const int64_t qh = (t0 + qi) * a.num_heads + h;
  if (row_parts == 1) {
    if (io >= 0) {
      store_out_row<D, kVw>(a.out + (static_cast<int64_t>(io) * a.num_heads + h) * D, o, c, l > 0.f ? l : 1.f);
    }
  } else {
    const int64_t slot = qh * a.max_parts + p;
    store_out_row<D, kVw>(a.ws_acc + slot * D, o, c, 1.f);
    if (c == 0) {
      a.ws_ml[2 * slot] = m_ref;
      a.ws_ml[2 * slot + 1] = l;
    }
  }
}

// The tile pass: workgroup w computes items w, w + gridDim.x, ... of the num_items (tile,
// partition, head) items. With one item per workgroup the grid is the item count; beside the
// row pass the host launches one workgroup per CU instead, so the tile pass holds one wave per
// SIMD and leaves the rest of each CU to the memory-bound row pass. The register path at
// head_dim 128 is held to 168 VGPRs (three waves per SIMD; it needs about 170 unconstrained,
// which allows two); the other instantiations have no occupancy target. Its wavefronts run at
// instruction-arbiter priority 1 (the row pass keeps 0): beside the row pass the tile items are
// the ones that finish last, and the memory-bound row wavefronts lose little by yielding issue
// slots (measured: the prefix-sharing step's call 0.2333-0.2369 -> 0.2311-0.2335 ms, the mixed
// bfloat16 call 1.105-1.110 -> 1.102-1.107 ms; alone, where every wavefront is a tile's, it
// changes nothing). The reverse, the row pass at priority 1, starves the tiles (the mixed
// float32 call 1.48 -> 1.97 ms).
template <typename KVT, int D, bool kPow2Block, bool kDma>
__global__ __launch_bounds__(kTileThreads)
__attribute__((amdgpu_waves_per_eu(!kDma && D == 128 ? PKV_TILE_REG_WAVES : 1)))
void tile_partial_kernel(const Params a, uint32_t num_items) {
  using S = TileShape<D>;
  __builtin_amdgcn_s_setprio(1);
  __shared__ int s_table[kTableSlots];
  __shared__ int s_vis[kTileRows];
  if constexpr (kDma) {
    static_assert(std::is_same_v<KVT, float>, "the direct-to-LDS tiles are float32");
    // The stages are dynamic LDS (kTileStages * S::kStageFloats floats, sized at launch). From
    // a static array of their size the compiler would infer one wave per SIMD and reserve the
    // registers of that occupancy (257 instead of the 152 used), which leaves room for one
    // row-pass workgroup per CU instead of two.
    extern __shared__ __align__(16) float s_kv[];
    for (uint32_t item = blockIdx.x; item < num_items; item += gridDim.x) {
      __syncthreads();  // the previous item's reads of LDS are done
      tile_item_dma<D, kPow2Block>(a, item, s_table, s_kv, s_vis);
    }
  } else {
    __shared__ float s_k[S::kKeys * S::kRow];
    __shared__ float s_v[S::kKeys * S::kRow];
    for (uint32_t item = blockIdx.x; item < num_items; item += gridDim.x) {
      __syncthreads();  // the previous item's reads of LDS are done
      tile_item<KVT, D, kPow2Block>(a, item, s_table, s_k, s_v, s_vis);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Pass 3: reduce. Item i = (entry i / H of the merge list, or query row i / H without one; head
// i % H). D / 4 threads per item, four output dimensions each, so a workgroup of kReduceThreads
// merges several (row, head) items; kVec selects 16-byte accesses (out and workspace aligned).
// ---------------------------------------------------------------------------------------------
template <int D, bool kVec>
__global__ __launch_bounds__(kReduceThreads) void reduce_kernel(const Params a, int64_t num_items) {
  static_assert(D % 4 == 0 && D / 4 <= kReduceThreads, "four dimensions per thread");
  constexpr int kTpi = D / 4;                       // threads per item
  constexpr int kItems = kReduceThreads / kTpi;     // items per workgroup
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kItems + threadIdx.x / kTpi;
  if (item >= num_items) return;
  const int h = static_cast<int>(item % a.num_heads);
  const int64_t idx = item / a.num_heads;
  const int64_t t = a.num_merge >= 0 ? a.merge_rows[idx] : idx;
  if (t < 0 || t >= a.num_queries) return;  // a row outside the batch is skipped
  const int nparts = parts_of(row_visible(a, t), a.part_size);
  if (nparts == 1) return;  // written by the partial pass
  const int64_t r = io_row(a, t);
  if (r < 0) return;
  const int d = (static_cast<int>(threadIdx.x) % kTpi) * 4;
  const int64_t qh = t * a.num_heads + h;
  const float* ml = a.ws_ml + 2 * qh * a.max_parts;
  // Unrolled so that several partitions' loads are in flight at once (a long context has tens).
  float big = -INFINITY;
#pragma unroll 8
  for (int k = 0; k < nparts; ++k) big = fmaxf(big, ml[2 * k]);
  const float shift = big == -INFINITY ? 0.f : big;
  float lsum = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const float* part = a.ws_acc + qh * a.max_parts * D + d;
#pragma unroll 8
  for (int k = 0; k < nparts; ++k) {
    const float w = fast_exp2(ml[2 * k] - shift);
    lsum = fmaf(ml[2 * k + 1], w, lsum);
    float v[4];
    if constexpr (kVec) {
      const float4 x = *reinterpret_cast<const float4*>(part + static_cast<int64_t>(k) * D);
      v[0] = x.x;
      v[1] = x.y;
      v[2] = x.z;
      v[3] = x.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = part[static_cast<int64_t>(k) * D + e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = fmaf(v[e], w, acc[e]);
  }
  const float sum = lsum > 0.f ? lsum : 1.f;
  float* dst = a.out + (r * a.num_heads + h) * D + d;
  if constexpr (kVec) {
    *reinterpret_cast<float4*>(dst) = make_float4(acc[0] / sum, acc[1] / sum, acc[2] / sum, acc[3] / sum);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[e] = acc[e] / sum;
  }
}

// The library's per-device resources, created by pkv_init and kept for the life of the process:
// a second stream (default priority, non-blocking) with fork and join events, so the
// compute-bound tile pass of a call runs beside its memory-bound row pass. The compute entry
// points never create anything; on a device pkv_init has not set up, they run both passes on the
// caller's stream. Each device has its own mutex: it serialises the fork/join enqueue sequence
// of calls from several host threads on that device (calls on other devices do not wait).
constexpr int kMaxDevices = 64;
constexpr int64_t kOverlapMinRowGroups = 2048;  // 8 row-pass workgroups per CU

struct DeviceResources {
  std::mutex mu;
  std::atomic<bool> ready{false};            // stream and events exist
  std::atomic<float*> scratch_ptr{nullptr};  // this device's copy of `scratch`
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr;
  hipEvent_t join = nullptr;
  int64_t cus = 0;  // compute units (the tile pass's persistent grid beside the row pass)
};

DeviceResources g_devices[kMaxDevices];

// Looks up the current device's copy of `scratch` into r.scratch_ptr. Caller holds r.mu and has
// made the device current.
int resolve_scratch_locked(DeviceResources& r) {
  if (r.scratch_ptr.load(std::memory_order_relaxed) != nullptr) return PKV_OK;
  void* ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
    (void)hipGetLastError();
    return PKV_EHIP;
  }
  r.scratch_ptr.store(static_cast<float*>(ptr), std::memory_order_release);
  return PKV_OK;
}

// The device's overlap resources, or null when pkv_init has not created them.
DeviceResources* overlap_for(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  DeviceResources& r = g_devices[device];
  return r.ready.load(std::memory_order_acquire) ? &r : nullptr;
}

// cus == 0: one workgroup per item (the tile pass alone). cus > 0: a persistent grid beside the
// row pass, of one workgroup per CU staged straight into LDS (float32 pools beside full-size row
// workgroups), else of two register-staged workgroups per CU, or of three with
// PKV_ATTN_DOMINANT_TILES. Measured on MI355X (config 3's shape, 30-240 decode rows):
//  - float32 beside full rows: one direct-to-LDS workgroup per CU is best while the tile pass's
//    time is below about 1.1 times the row pass's (1.44 ms against 1.57 / 1.46 ms with two /
//    three register-staged ones at 120 decode rows), three register-staged ones above it
//    (0.86 against 0.99 ms at 30 rows);
//  - bfloat16 (always register-staged): one per CU leaves the tile pass far behind (1.82 ms at
//    120 decode rows), two are best below the same crossover (1.11 ms), three above it;
//  - beside lean row workgroups the 100 KiB of direct-to-LDS stages would crowd them out (the
//    prefix-sharing step's attention took 0.30 instead of 0.23 ms); one, two or three
//    register-staged workgroups per CU tie there in float32, and two are best in bfloat16
//    (0.146 against 0.173 ms with one).
template <typename KVT, int D>
int launch_tiles(const Params& a, int64_t num_tiles, int64_t cus, bool lean_rows, hipStream_t stream) {
  if constexpr (D % 16 == 0 && D >= 32) {
    const int64_t items = num_tiles * static_cast<int64_t>(a.max_parts) * a.num_heads;
    if (items > 0x7fffffff) return PKV_EUNSUPPORTED;
    const bool pow2 = (a.block_size & (a.block_size - 1)) == 0;
    constexpr bool kDmaType = PKV_TILE_DMA && std::is_same_v<KVT, float>;
    const bool block_fits = static_cast<int64_t>(a.block_size) * a.num_heads * D <= INT32_MAX;
    const bool dominant = (a.flags & PKV_ATTN_DOMINANT_TILES) != 0;
    const bool dma = kDmaType && cus > 0 && !lean_rows && !dominant && block_fits;
    const int64_t max_groups = cus * (dma ? 1 : dominant ? 3 : 2);
    const int64_t groups = max_groups > 0 && max_groups < items ? max_groups : items;
    const dim3 grid(static_cast<uint32_t>(groups));
    const auto n = static_cast<uint32_t>(items);
    const size_t stage_bytes = kTileStages * TileShape<D>::kStageFloats * sizeof(float);
    if (dma && pow2) {
      hipLaunchKernelGGL((tile_partial_kernel<KVT, D, true, kDmaType>), grid, dim3(kTileThreads), stage_bytes,
                         stream, a, n);
    } else if (dma) {
      hipLaunchKernelGGL((tile_partial_kernel<KVT, D, false, kDmaType>), grid, dim3(kTileThreads), stage_bytes,
                         stream, a, n);
    } else if (pow2) {
      hipLaunchKernelGGL((tile_partial_kernel<KVT, D, true, false>), grid, dim3(kTileThreads), 0, stream, a, n);
    } else {
      hipLaunchKernelGGL((tile_partial_kernel<KVT, D, false, false>), grid, dim3(kTileThreads), 0, stream, a, n);
    }
    return check_launch();
  } else {
    return PKV_EUNSUPPORTED;
  }
}

template <typename KVT, int D>
int launch_all(const Params& a, int64_t num_queries, int64_t num_rows, int64_t num_tiles,
               bool stream_kv, int device, hipStream_t stream) {
  const bool pow2 = (a.block_size & (a.block_size - 1)) == 0;
  const bool short_rows = (a.flags & PKV_ATTN_SHORT_ROWS) != 0;
  const bool append = a.new_keys != nullptr;
  std::unique_lock<std::mutex> overlap_lock;
  DeviceResources* overlap = nullptr;
  // The second stream pays off only when the row pass alone would keep the GPU busy long enough
  // to hide the tile pass: its fork and join cost about 40 us of host time per call (two event
  // records, two stream waits), more than a small call's whole device time. Below
  // kOverlapMinRowGroups row-pass workgroups both passes run on the caller's stream, tiles first.
  const int64_t row_groups = (a.rows ? num_rows : num_rows * static_cast<int64_t>(a.max_parts)) *
                             (kPairHeads<KVT, D> && a.num_heads % 2 == 0 ? a.num_heads / 2 : a.num_heads);
  if (PKV_ATTN_OVERLAP && num_tiles > 0 && num_rows > 0 && row_groups >= kOverlapMinRowGroups) {
    overlap = overlap_for(device);
    if (overlap != nullptr) overlap_lock = std::unique_lock<std::mutex>(overlap->mu);
  }
  auto launch_rows_hpw = [&](auto hpw_tag, hipStream_t rs) -> int {
    constexpr int HPW = decltype(hpw_tag)::value;
    const int64_t items = a.rows ? num_rows : num_rows * static_cast<int64_t>(a.max_parts);
    const int64_t groups = items * (a.num_heads / HPW);
    if (groups > 0x7fffffff) return PKV_EUNSUPPORTED;
    const dim3 grid(static_cast<uint32_t>(groups));
    // The lean and the appending variants exist for power-of-two block sizes only (the others
    // ignore the hint; attention_call appends separately for them).
    if (pow2 && append && short_rows && stream_kv) {
      hipLaunchKernelGGL((row_partial_kernel<KVT, D, HPW, true, true, true, true>), grid, dim3(kThreads), 0, rs, a);
    } else if (pow2 && append && short_rows) {
      hipLaunchKernelGGL((row_partial_kernel<KVT, D, HPW, true, false, true, true>), grid, dim3(kThreads), 0, rs, a);
    } else if (pow2 && append && stream_kv) {
      hipLaunchKernelGGL((row_partial_kernel<KVT, D, HPW, true, true, false, true>), grid, dim3(kThreads), 0, rs, a);
    } else if (pow2 && append) {
      hipLaunchKernelGGL((row_partial_kernel<KVT, D, HPW, true, false, false, true>), grid, dim3(kThreads), 0, rs, a);
    } else if (pow2 && short_rows && stream_kv) {
      hipLaunchKernelGGL((row_partial_kernel<KVT, D, HPW, true, true, true, false>), grid, dim3(kThreads), 0, rs, a);
    } else if (pow2 && short_rows) {
      hipLaunchKernelGGL((row_partial_kernel<KVT, D, HPW, true, false, true, false>), grid, dim3(kThreads), 0, rs, a);
    } else if (pow2 && stream_kv) {
      hipLaunchKernelGGL((row_partial_kernel<KVT, D, HPW, true, true, false, false>), grid, dim3(kThreads), 0, rs, a);
    } else if (pow2) {
      hipLaunchKernelGGL((row_partial_kernel<KVT, D, HPW, true, false, false, false>), grid, dim3(kThreads), 0, rs, a);
    } else if (stream_kv) {
      hipLaunchKernelGGL((row_partial_kernel<KVT, D, HPW, false, true, false, false>), grid, dim3(kThreads), 0, rs, a);
    } else {
      hipLaunchKernelGGL((row_partial_kernel<KVT, D, HPW, false, false, false, false>), grid, dim3(kThreads), 0, rs, a);
    }
    return check_launch();
  };
  auto launch_rows = [&](hipStream_t rs) -> int {
    if (num_rows == 0) return PKV_OK;
    if constexpr (kPairHeads<KVT, D>) {
      if (a.num_heads % 2 == 0) return launch_rows_hpw(std::integral_constant<int, 2>{}, rs);
    }
    return launch_rows_hpw(std::integral_constant<int, 1>{}, rs);
  };
  if (PKV_ATTN_ROWS_FIRST || overlap == nullptr) {
    // Without overlap the order does not matter; with it, rows first takes the CUs first.
    if (overlap != nullptr && hipEventRecord(overlap->fork, stream) != hipSuccess) return PKV_EHIP;
    const int rc = launch_rows(stream);
    if (rc != PKV_OK) return rc;
  } else if (hipEventRecord(overlap->fork, stream) != hipSuccess) {
    return PKV_EHIP;
  }
  if (num_tiles > 0) {
    if (overlap != nullptr) {
      // fork: the tile pass starts when the caller's stream reaches the fork point
      if (hipStreamWaitEvent(overlap->stream, overlap->fork, 0) != hipSuccess) return PKV_EHIP;
      const int rc = launch_tiles<KVT, D>(a, num_tiles, overlap->cus, short_rows, overlap->stream);
      if (rc != PKV_OK) return rc;
      if (hipEventRecord(overlap->join, overlap->stream) != hipSuccess) return PKV_EHIP;
    } else {
      const int rc = launch_tiles<KVT, D>(a, num_tiles, 0, short_rows, stream);
      if (rc != PKV_OK) return rc;
    }
  }
  if (!PKV_ATTN_ROWS_FIRST && overlap != nullptr) {
    const int rc = launch_rows(stream);
    if (rc != PKV_OK) return rc;
  }
  if (overlap != nullptr) {
    // join: everything after this (the reduce, the caller's next work) waits for the tile pass
    if (hipStreamWaitEvent(stream, overlap->join, 0) != hipSuccess) return PKV_EHIP;
    overlap_lock.unlock();
  }
  const int64_t merge = a.num_merge >= 0 ? a.num_merge : num_queries;
  if (a.max_parts > 1 && merge > 0) {
    constexpr int kItems = kReduceThreads / (D / 4);
    const int64_t items = merge * a.num_heads;
    const int64_t groups = (items + kItems - 1) / kItems;
    if (groups > 0x7fffffff) return PKV_EUNSUPPORTED;
    const dim3 grid(static_cast<uint32_t>(groups));
    if (aligned16(a.out) && aligned16(a.ws_acc)) {
      hipLaunchKernelGGL((reduce_kernel<D, true>), grid, dim3(kReduceThreads), 0, stream, a, items);
    } else {
      hipLaunchKernelGGL((reduce_kernel<D, false>), grid, dim3(kReduceThreads), 0, stream, a, items);
    }
    if (check_launch() != PKV_OK) return PKV_EHIP;
  }
  return PKV_OK;
}

template <typename KVT>
int dispatch_head_dim(int head_dim, const Params& a, int64_t num_queries, int64_t num_rows,
                      int64_t num_tiles, bool stream_kv, int device, hipStream_t stream) {
  switch (head_dim) {
    case 8:
      return launch_all<KVT, 8>(a, num_queries, num_rows, num_tiles, stream_kv, device, stream);
    case 16:
      return launch_all<KVT, 16>(a, num_queries, num_rows, num_tiles, stream_kv, device, stream);
    case 32:
      return launch_all<KVT, 32>(a, num_queries, num_rows, num_tiles, stream_kv, device, stream);
    case 64:
      return launch_all<KVT, 64>(a, num_queries, num_rows, num_tiles, stream_kv, device, stream);
    case 128:
      return launch_all<KVT, 128>(a, num_queries, num_rows, num_tiles, stream_kv, device, stream);
    case 256:
      return launch_all<KVT, 256>(a, num_queries, num_rows, num_tiles, stream_kv, device, stream);
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

extern "C" int pkv_tile_head_dim_supported(int32_t head_dim) {
  return head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256;
}

extern "C" int pkv_init(int device) {
  using namespace pkv;
  if (device < 0 || device >= kMaxDevices) return PKV_EINVAL;
  DeviceResources& r = g_devices[device];
  std::lock_guard<std::mutex> lock(r.mu);
  if (r.ready.load(std::memory_order_relaxed)) return PKV_OK;
  DeviceGuard guard(device);
  if (!guard.ok()) return PKV_EHIP;
  const int found = resolve_scratch_locked(r);
  if (found != PKV_OK) return found;
  int cus = 0;
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr;
  hipEvent_t join = nullptr;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      hipStreamCreateWithFlags(&stream, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&fork, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&join, hipEventDisableTiming) != hipSuccess) {
    if (join != nullptr) (void)hipEventDestroy(join);
    if (fork != nullptr) (void)hipEventDestroy(fork);
    if (stream != nullptr) (void)hipStreamDestroy(stream);
    (void)hipGetLastError();
    return PKV_EHIP;
  }
  r.stream = stream;
  r.fork = fork;
  r.join = join;
  r.cus = cus;
  r.ready.store(true, std::memory_order_release);
  return PKV_OK;
}

namespace pkv {
namespace {

// The source of a decode append fused into the row pass (pkv_paged_attention_append).
struct AppendSource {
  const void* keys;
  const void* values;
  pkv_dtype dtype;
  int64_t key_stride;
  int64_t value_stride;
  const int64_t* slots;
};

int attention_call(float* out, const float* queries, int64_t query_token_stride,
                   const int32_t* query_positions, const int32_t* query_seq, int64_t num_queries,
                   const int32_t* caller_rows, const int32_t* rows, int64_t num_rows, const int32_t* tiles, int64_t num_tiles,
                   const int32_t* merge_rows, int64_t num_merge_rows, const void* key_cache,
                   const void* value_cache, pkv_dtype kv_dtype, int64_t num_blocks,
                   int32_t block_size, const int32_t* block_tables, int32_t block_table_stride,
                   const int32_t* context_lens, int32_t num_seqs, int32_t num_heads,
                   int32_t head_dim, float scale, int32_t max_context_len, int32_t partition_size,
                   int32_t flags, float* workspace, int64_t workspace_bytes, int device,
                   void* stream, const AppendSource* append) {
  const int part = resolve_partition(partition_size);
  if (part < 0) return PKV_EINVAL;
  if (flags & ~(PKV_ATTN_SHARED_KV | PKV_ATTN_SHORT_ROWS | PKV_ATTN_DOMINANT_TILES)) return PKV_EINVAL;
  const bool stream_kv = (flags & PKV_ATTN_SHARED_KV) == 0;
  if (num_queries < 0 || num_rows < 0 || num_tiles < 0 || num_merge_rows < -1 || num_blocks < 1 ||
      block_size < 1 ||
      block_table_stride < 0 || num_seqs < 0 || num_heads < 1 || head_dim < 1 ||
      max_context_len < 0) {
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
  // Without a plan (rows and tiles both null) every query goes through the row pass.
  if (!rows && !tiles) {
    num_rows = num_queries;
    num_tiles = 0;
  }
  if ((num_rows > 0 && !rows && num_rows != num_queries) || (num_tiles > 0 && !tiles) ||
      (num_merge_rows > 0 && !merge_rows)) {
    return PKV_EINVAL;
  }
  if (num_tiles > 0 && !pkv_tile_head_dim_supported(head_dim)) return PKV_EUNSUPPORTED;
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
  // The tile pass writes four dimensions of a row at a time.
  if (num_tiles > 0 && (!aligned16(out) || (ws_acc && !aligned16(ws_acc)))) return PKV_EINVAL;
  if (append != nullptr) {
    // Only the row pass appends (tiles may cover partitions that hold no new position: a shared
    // prefix); the source rows are read as 16-byte vectors.
    const int src_size = dtype_size(append->dtype);
    if (src_size == 0 || !append->keys || !append->values || !append->slots) {
      return PKV_EINVAL;
    }
    if (append->dtype == PKV_BF16 && kv_dtype == PKV_F32) return PKV_EUNSUPPORTED;
    const int64_t row = static_cast<int64_t>(num_heads) * head_dim;
    if (append->key_stride < row || append->value_stride < row) return PKV_EINVAL;
    if (!aligned16(append->keys) || !aligned16(append->values) ||
        (append->key_stride * src_size) % 16 != 0 || (append->value_stride * src_size) % 16 != 0 ||
        (static_cast<int64_t>(head_dim) * src_size) % 16 != 0) {
      return PKV_EUNSUPPORTED;
    }
  }
  DeviceGuard guard(device);
  if (!guard.ok()) return PKV_EHIP;
  (void)hipGetLastError();
  int shift = 0;
  while ((1 << shift) < block_size) ++shift;
  Params a{};
  a.out = out;
  a.ws_acc = ws_acc;
  a.ws_ml = ws_ml;
  a.queries = queries;
  a.q_stride = query_token_stride;
  a.q_pos = query_positions;
  a.q_seq = query_seq;
  a.q_rows = caller_rows;
  a.rows = rows;
  a.tiles = tiles;
  a.merge_rows = merge_rows;
  a.num_merge = num_merge_rows;
  a.num_tiles = tiles ? num_tiles : 0;
  a.flags = flags;
  a.kcache = key_cache;
  a.vcache = value_cache;
  a.num_queries = num_queries;
  a.num_blocks = num_blocks;
  a.tables = block_tables;
  a.ctx_lens = context_lens;
  a.table_stride = block_table_stride;
  a.num_seqs = num_seqs;
  a.num_heads = num_heads;
  a.block_size = block_size;
  a.block_shift = shift;
  a.part_size = part;
  a.max_parts = static_cast<int32_t>(parts);
  a.max_ctx = max_context_len;
  a.scale_log2 = static_cast<float>(static_cast<double>(scale) * 1.4426950408889634);
  if (append != nullptr && (block_size & (block_size - 1)) != 0) {
    // No fused instantiation for this block size: the same two steps as separate launches.
    const int rc = pkv_append(const_cast<void*>(key_cache), const_cast<void*>(value_cache), kv_dtype, num_blocks * block_size,
                              append->keys, append->values, append->dtype, append->key_stride,
                              append->value_stride, append->slots, num_queries, num_heads,
                              head_dim, device, stream);
    if (rc != PKV_OK) return rc;
    append = nullptr;
  }
  if (append != nullptr) {
    a.new_keys = append->keys;
    a.new_values = append->values;
    a.new_key_stride = append->key_stride;
    a.new_value_stride = append->value_stride;
    a.new_slots = append->slots;
    a.num_slots = num_blocks * block_size;
    a.new_dtype = append->dtype;
  }
  auto s = static_cast<hipStream_t>(stream);
  if (kv_dtype == PKV_F32) {
    return dispatch_head_dim<float>(head_dim, a, num_queries, num_rows, num_tiles, stream_kv, device, s);
  }
  return dispatch_head_dim<uint16_t>(head_dim, a, num_queries, num_rows, num_tiles, stream_kv, device, s);
}

}  // namespace
}  // namespace pkv

extern "C" int pkv_paged_attention(float* out, const float* queries, int64_t query_token_stride,
                                   const int32_t* query_positions, const int32_t* query_seq,
                                   int64_t num_queries, const int32_t* caller_rows,
                                   const int32_t* rows, int64_t num_rows,
                                   const int32_t* tiles, int64_t num_tiles,
                                   const int32_t* merge_rows, int64_t num_merge_rows,
                                   const void* key_cache, const void* value_cache,
                                   pkv_dtype kv_dtype, int64_t num_blocks,
                                   int32_t block_size, const int32_t* block_tables,
                                   int32_t block_table_stride, const int32_t* context_lens,
                                   int32_t num_seqs, int32_t num_heads, int32_t head_dim,
                                   float scale, int32_t max_context_len, int32_t partition_size,
                                   int32_t flags, float* workspace, int64_t workspace_bytes,
                                   int device, void* stream) {
  return pkv::attention_call(out, queries, query_token_stride, query_positions, query_seq,
                             num_queries, caller_rows, rows, num_rows, tiles, num_tiles, merge_rows,
                             num_merge_rows, key_cache, value_cache, kv_dtype, num_blocks,
                             block_size, block_tables, block_table_stride, context_lens, num_seqs,
                             num_heads, head_dim, scale, max_context_len, partition_size, flags,
                             workspace, workspace_bytes, device, stream, nullptr);
}

extern "C" int pkv_paged_attention_noalloc(
    float* out, const float* queries, int64_t query_token_stride, const int32_t* query_positions,
    const int32_t* query_seq, int64_t num_queries, const int32_t* caller_rows, const int32_t* rows,
    int64_t num_rows,
    const int32_t* tiles, int64_t num_tiles, const int32_t* merge_rows, int64_t num_merge_rows,
    const void* key_cache, const void* value_cache, pkv_dtype kv_dtype, int64_t num_blocks,
    int32_t block_size, const int32_t* block_tables, int32_t block_table_stride,
    const int32_t* context_lens, int32_t num_seqs, int32_t num_heads, int32_t head_dim,
    float scale, int32_t max_context_len, int32_t partition_size, int32_t flags, int device,
    void* stream) {
  using namespace pkv;
  if (device < 0 || device >= kMaxDevices) return PKV_EINVAL;
  const int64_t need = pkv_attention_workspace_bytes(num_queries, num_heads, head_dim,
                                                     max_context_len, partition_size);
  if (need < 0) return PKV_EINVAL;
  if (need > PKV_STATIC_SCRATCH_BYTES) return PKV_ETOOBIG;
  float* workspace = nullptr;
  if (need > 0) {
    DeviceResources& r = g_devices[device];
    workspace = r.scratch_ptr.load(std::memory_order_acquire);
    if (workspace == nullptr) {  // the device's first use: find its copy of the array
      std::lock_guard<std::mutex> lock(r.mu);
      DeviceGuard guard(device);
      if (!guard.ok()) return PKV_EHIP;
      const int rc = resolve_scratch_locked(r);
      if (rc != PKV_OK) return rc;
      workspace = r.scratch_ptr.load(std::memory_order_relaxed);
    }
  }
  return pkv::attention_call(out, queries, query_token_stride, query_positions, query_seq,
                             num_queries, caller_rows, rows, num_rows, tiles, num_tiles, merge_rows,
                             num_merge_rows, key_cache, value_cache, kv_dtype, num_blocks,
                             block_size, block_tables, block_table_stride, context_lens, num_seqs,
                             num_heads, head_dim, scale, max_context_len, partition_size, flags,
                             workspace, need > 0 ? PKV_STATIC_SCRATCH_BYTES : 0, device, stream,
                             nullptr);
}

extern "C" int pkv_paged_attention_append(
    float* out, const float* queries, int64_t query_token_stride, const int32_t* query_positions,
    const int32_t* query_seq, int64_t num_queries, const int32_t* caller_rows, const int32_t* rows,
    int64_t num_rows, const int32_t* tiles, int64_t num_tiles,
    const int32_t* merge_rows, int64_t num_merge_rows, void* key_cache, void* value_cache,
    pkv_dtype kv_dtype, int64_t num_blocks, int32_t block_size, const int32_t* block_tables,
    int32_t block_table_stride, const int32_t* context_lens, int32_t num_seqs, int32_t num_heads,
    int32_t head_dim, float scale, int32_t max_context_len, int32_t partition_size, int32_t flags,
    float* workspace, int64_t workspace_bytes, const void* new_keys, const void* new_values,
    pkv_dtype new_dtype, int64_t new_key_token_stride, int64_t new_value_token_stride,
    const int64_t* slot_mapping, int device, void* stream) {
  const pkv::AppendSource append{new_keys, new_values, new_dtype, new_key_token_stride,
                                 new_value_token_stride, slot_mapping};
  return pkv::attention_call(out, queries, query_token_stride, query_positions, query_seq,
                             num_queries, caller_rows, rows, num_rows, tiles, num_tiles, merge_rows,
                             num_merge_rows,
                             key_cache, value_cache, kv_dtype, num_blocks, block_size,
                             block_tables, block_table_stride, context_lens, num_seqs, num_heads,
                             head_dim, scale, max_context_len, partition_size, flags, workspace,
                             workspace_bytes, device, stream, &append);
}
