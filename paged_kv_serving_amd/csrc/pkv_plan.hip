// Host-side planner of a ragged attention call (pkv_plan_batch): which (query row, context
// partition) goes to the row-streaming pass and which to the MFMA tile pass, the reduce's merge
// list, the partition size and the launch flags. Host code only: it reads host arrays, writes
// host arrays and never touches a device, so it runs (and is tested) on any machine.
//
// The rules, in order (each a measured launch choice on MI355X; none changes a result):
//   1. Runs of >= min_tile_rows consecutive rows of one sequence become tiles of <= 64 rows
//      (head_dim 32, 64, 128 or 256); every other row goes to the row pass.
//   2. With >= 1024 (tile, head) pairs, tiles are whole (one workgroup per tile and head over
//      every visible key). Beside row-pass rows they are grouped by chunk, longest chunk
//      first; a chunk's tiles run from its last row's to its first row's in even-ranked chunks
//      and the other way in odd-ranked ones, so the persistent workgroups that share a head
//      alternate long and short tiles and reach every second chunk together (sharing its keys
//      through their XCD's L2). Without row-pass rows the longest tile comes first (stable), so
//      the grid ends on its shortest workgroups.
//   3. >= 16 consecutive row-pass rows whose tables agree over >= 512 leading tokens form a
//      shared-prefix group; its whole partitions become 64-row tiles read through the first
//      row's table (a tile never starts at a member whose table ends inside the prefix), and
//      the rows start the row pass after the prefix.
//   4. Partition size: the one whose whole partitions (<= 1024 keys) cover the largest group's
//      prefix with about 512 tile workgroups; without groups 1024 when rows x heads x
//      ceil(context / 1024) >= 8192, else 512. An explicit size is kept.
//   5. PKV_ATTN_SHARED_KV when >= 25% of the block ids the row pass still reads repeat;
//      PKV_ATTN_SHORT_ROWS when the row-pass items average < 256 keys; PKV_ATTN_DOMINANT_TILES
//      when the call has both passes and the tile pass's estimated time is at least 1.1 times
//      the row pass's: a tile key costs 4 * head_dim products at about 100 TFLOP/s, a row key
//      2 * head_dim * element-size bytes at about 6.8 TB/s, i.e.
//      tile_keys * 34 >= row_keys * element_size * 275 (measured crossover on MI355X, config 3's
//      chunks beside 30-240 decode rows in float32 and bfloat16).
//   6. Row-pass items: every partition a row still needs, longest first (stable), so the grid
//      ends on its shortest workgroups.
#include <stdint.h>

#include <algorithm>
#include <cstring>
#include <vector>

#include "pkv_common.h"

namespace pkv {
namespace {

constexpr int kTileRows = 64;
constexpr int64_t kWidePartitionItems = 8192;
constexpr double kSharedKvFraction = 0.25;
constexpr int kMinSharedTokens = 512;
constexpr int64_t kMinSharedRows = 16;
constexpr int64_t kTargetPrefixGroups = 512;
constexpr int kMinPrefixPartition = 256;
constexpr int64_t kWholeTileGroups = 1024;
constexpr int64_t kShortRowKeys = 256;
constexpr int64_t kDominantTileWeight = 34;  // rule 5: tile_keys * 34 >= row_keys * esize * 275
constexpr int64_t kDominantRowWeight = 275;
constexpr int kDefaultPlanPartition = 512;

struct Tile {
  int32_t first, count, begin, end;
};

struct Group {
  int64_t start, count, common;
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }  // a >= 0, b > 0

bool tiled_head_dim(int32_t d) { return d == 32 || d == 64 || d == 128 || d == 256; }

// The batch's block tables: entry c of sequence s, or -1 past its used blocks.
struct Tables {
  const int32_t* base;
  int32_t stride;
  const int64_t* used;
  int32_t at(int64_t s, int64_t c) const { return c < used[s] ? base[s * stride + c] : -1; }
};

// First column in [0, limit) where the tables of sequences a and b differ, or limit. Sharers
// agree over their whole prefix, so the common answer comes from one memcmp.
int64_t common_prefix(const Tables& t, int64_t a, int64_t b, int64_t limit) {
  const int32_t* x = t.base + a * t.stride;
  const int32_t* y = t.base + b * t.stride;
  if (limit <= 0 || std::memcmp(x, y, static_cast<size_t>(limit) * sizeof(int32_t)) == 0) {
    return std::max<int64_t>(limit, 0);
  }
  int64_t c = 0;
  while (x[c] == y[c]) ++c;
  return c;
}

// Rule 2: whole prefill tiles. Beside row-pass rows, chunk by chunk; without them (the tile pass
// runs one workgroup per item, handed out in item order as workgroups finish), longest first.
void make_whole(std::vector<Tile>& tiles, const int32_t* seq, const std::vector<int64_t>& vis,
                int32_t num_heads, bool has_rows) {
  const int64_t n = static_cast<int64_t>(tiles.size());
  if (n == 0 || n * num_heads < kWholeTileGroups) return;
  std::vector<int64_t> longest(n);
  for (int64_t t = 0; t < n; ++t) {
    int64_t m = vis[tiles[t].first];
    for (int32_t r = 1; r < tiles[t].count; ++r) m = std::max(m, vis[tiles[t].first + r]);
    longest[t] = m;
  }
  if (!has_rows) {
    std::vector<int64_t> order(n);
    for (int64_t t = 0; t < n; ++t) order[t] = t;
    std::stable_sort(order.begin(), order.end(),
                     [&](int64_t a, int64_t b) { return longest[a] > longest[b]; });
    std::vector<Tile> whole;
    whole.reserve(n);
    for (int64_t t : order) {
      Tile w = tiles[t];
      w.begin = 0;
      w.end = PKV_TILE_WHOLE;
      whole.push_back(w);
    }
    tiles.swap(whole);
    return;
  }
  std::vector<int64_t> starts;  // a chunk starts where a tile does not continue the previous one
  for (int64_t t = 0; t < n; ++t) {
    if (t == 0 || tiles[t].first != tiles[t - 1].first + tiles[t - 1].count ||
        seq[tiles[t].first] != seq[tiles[t - 1].first]) {
      starts.push_back(t);
    }
  }
  const int64_t chunks = static_cast<int64_t>(starts.size());
  std::vector<int64_t> chunk_longest(chunks);
  for (int64_t c = 0; c < chunks; ++c) {
    const int64_t end = c + 1 < chunks ? starts[c + 1] : n;
    int64_t m = longest[starts[c]];
    for (int64_t t = starts[c] + 1; t < end; ++t) m = std::max(m, longest[t]);
    chunk_longest[c] = m;
  }
  std::vector<int64_t> order(chunks);
  for (int64_t c = 0; c < chunks; ++c) order[c] = c;
  std::stable_sort(order.begin(), order.end(),
                   [&](int64_t a, int64_t b) { return chunk_longest[a] > chunk_longest[b]; });
  std::vector<Tile> whole;
  whole.reserve(n);
  for (int64_t rank = 0; rank < chunks; ++rank) {
    const int64_t c = order[rank];
    const int64_t begin = starts[c];
    const int64_t size = (c + 1 < chunks ? starts[c + 1] : n) - begin;
    const bool reverse = rank % 2 == 0;  // even ranks last row first, odd ranks first row first
    for (int64_t i = 0; i < size; ++i) {
      Tile t = tiles[begin + (reverse ? size - 1 - i : i)];
      t.begin = 0;
      t.end = PKV_TILE_WHOLE;
      whole.push_back(t);
    }
  }
  tiles.swap(whole);
}

// Rule 3: shared-prefix groups over the row-pass rows (rows[k] = query row, in order).
std::vector<Group> prefix_groups(const std::vector<int32_t>& rows, const int32_t* seq,
                                 const Tables& t, int64_t min_blocks) {
  std::vector<Group> groups;
  const int64_t count = static_cast<int64_t>(rows.size());
  if (count < kMinSharedRows) return groups;
  std::vector<int64_t> sid(count), used(count);
  int64_t width = 0;
  for (int64_t k = 0; k < count; ++k) {
    sid[k] = seq[rows[k]];
    used[k] = t.used[sid[k]];
    width = std::max(width, used[k]);
  }
  if (width < min_blocks) return groups;
  // consecutive[k]: row k + 1 continues row k; lead[k]: their tables' common prefix (<= both)
  std::vector<char> consecutive(count > 0 ? count - 1 : 0);
  std::vector<int64_t> stops;
  for (int64_t k = 0; k + 1 < count; ++k) {
    consecutive[k] = rows[k + 1] == rows[k] + 1;
    if (!consecutive[k]) stops.push_back(k);
  }
  int64_t next_free = 0;  // rows before this one already belong to a group
  for (int64_t k = 0; k + 1 < count; ++k) {
    if (k < next_free || !consecutive[k]) continue;
    const int64_t both = std::min(used[k], used[k + 1]);
    const int64_t lead = common_prefix(t, sid[k], sid[k + 1], both);
    // A run can start at k only if row k + 1 joins it: it shares enough, or its whole table is
    // a prefix of row k's.
    if (!(lead >= min_blocks || lead == used[k + 1])) continue;
    const auto stop = std::lower_bound(stops.begin(), stops.end(), k);
    const int64_t after = stop != stops.end() ? *stop + 1 : count;
    int64_t common = used[k];
    int64_t joined = 0;
    for (int64_t r = k + 1; r < after; ++r) {
      // Row r keeps the common prefix unless its table leaves row k's before both it ends and
      // the prefix does (a member whose whole table is a prefix of row k's constrains nothing).
      // common <= used[k], so comparing up to min(common, used[r]) decides it.
      const int64_t limit = std::min(common, used[r]);
      const int64_t lead_r = common_prefix(t, sid[r], sid[k], limit);
      const int64_t next = lead_r < limit ? lead_r : common;
      if (next < min_blocks) break;
      common = next;
      ++joined;
    }
    if (joined + 1 >= kMinSharedRows && common >= min_blocks) {
      groups.push_back({k, joined + 1, common});
      next_free = k + joined + 1;
    }
  }
  return groups;
}

// Number of distinct values. Block ids of one pool span a small range, so a bitmap over it is
// much cheaper than sorting (a 256-row decode batch reads about 3,000 ids: 2 us against 70 us);
// a range too wide for that falls back to a sort.
int64_t distinct_count(std::vector<int32_t>& ids) {
  const auto [lo, hi] = std::minmax_element(ids.begin(), ids.end());
  const int64_t low = *lo;
  const int64_t range = static_cast<int64_t>(*hi) - low + 1;
  if (range <= 64 * std::max<int64_t>(4096, 16 * static_cast<int64_t>(ids.size()))) {
    std::vector<uint64_t> seen((range + 63) / 64, 0);
    int64_t distinct = 0;
    for (const int32_t id : ids) {
      const int64_t bit = id - low;
      uint64_t& word = seen[bit >> 6];
      const uint64_t mask = uint64_t{1} << (bit & 63);
      distinct += (word & mask) == 0;
      word |= mask;
    }
    return distinct;
  }
  std::sort(ids.begin(), ids.end());
  return std::unique(ids.begin(), ids.end()) - ids.begin();
}

int32_t prefix_partition(int64_t shared_tokens, int64_t tiles, int32_t num_heads) {
  int32_t best = 0;
  for (int64_t k = std::max<int64_t>(1, ceil_div(shared_tokens, 1024));; ++k) {
    const int64_t size = std::min<int64_t>(1024, (shared_tokens / k) / 16 * 16);
    if (size < kMinPrefixPartition) break;
    best = static_cast<int32_t>(size);
    if (tiles * num_heads * k >= kTargetPrefixGroups) break;
  }
  return best;
}

}  // namespace
}  // namespace pkv

extern "C" int pkv_plan_batch(const int32_t* query_seq, const int32_t* query_positions,
                              int64_t num_queries, const int32_t* block_tables,
                              int32_t block_table_stride, const int32_t* context_lens,
                              int32_t num_seqs, int32_t block_size, int32_t num_heads,
                              int32_t head_dim, pkv_dtype kv_dtype, int32_t partition_size,
                              int32_t min_tile_rows,
                              int32_t* rows_out, int64_t rows_capacity, int32_t* tiles_out,
                              int64_t tiles_capacity, int32_t* merge_out, int64_t merge_capacity,
                              int64_t* counts_out, int32_t* launch_out) {
  using namespace pkv;
  const int esize = dtype_size(kv_dtype);
  if (num_queries < 0 || num_seqs < 0 || block_size < 1 || num_heads < 1 || head_dim < 1 ||
      esize == 0 || partition_size < 0 || min_tile_rows < 1 || block_table_stride < 0 ||
      !counts_out || !launch_out) {
    return PKV_EINVAL;
  }
  if (num_queries > 0 && (!query_seq || !context_lens || !block_tables || num_seqs == 0)) {
    return PKV_EINVAL;
  }
  const int32_t* seq = query_seq;
  // Used blocks of every sequence a query names; each must fit its table row.
  std::vector<int64_t> used(num_seqs, 0);
  std::vector<char> present(num_seqs, 0);
  for (int64_t q = 0; q < num_queries; ++q) {
    const int32_t s = seq[q];
    if (s < 0 || s >= num_seqs) return PKV_EINVAL;
    if (!present[s]) {
      if (context_lens[s] < 0) return PKV_EINVAL;
      used[s] = ceil_div(context_lens[s], block_size);
      if (used[s] > block_table_stride) return PKV_EINVAL;
      present[s] = 1;
    }
  }
  const Tables tables{block_tables, block_table_stride, used.data()};

  // Rule 1: the row/tile split.
  std::vector<int32_t> row_pass;  // query rows of the row pass
  std::vector<int32_t> row_first;  // first partition each starts at
  std::vector<Tile> tiles;
  const bool tiled = tiled_head_dim(head_dim);
  for (int64_t start = 0; start < num_queries;) {
    int64_t end = start + 1;
    while (end < num_queries && seq[end] == seq[start]) ++end;
    if (tiled && end - start >= min_tile_rows) {
      for (int64_t f = start; f < end; f += kTileRows) {
        tiles.push_back({static_cast<int32_t>(f), static_cast<int32_t>(std::min<int64_t>(kTileRows, end - f)), 0, 0});
      }
    } else {
      for (int64_t q = start; q < end; ++q) row_pass.push_back(static_cast<int32_t>(q));
    }
    start = end;
  }
  if (num_queries == 0) {
    counts_out[0] = counts_out[1] = counts_out[2] = 0;
    launch_out[0] = partition_size;
    launch_out[1] = 0;
    return PKV_OK;
  }
  row_first.assign(row_pass.size(), 0);
  std::vector<int64_t> vis(num_queries);  // visible keys of every query row
  for (int64_t q = 0; q < num_queries; ++q) {
    const int64_t ctx = context_lens[seq[q]];
    if (!query_positions) {
      vis[q] = ctx;
    } else {
      const int64_t p = query_positions[q];
      vis[q] = p < 0 ? 0 : std::min(ctx, p + 1);
    }
  }
  make_whole(tiles, seq, vis, num_heads, !row_pass.empty());

  // Do two row-pass sequences start with the same block? Without that there is neither a
  // shared-prefix group nor a repeated block to look for.
  bool may_share = false;
  {
    std::vector<char> listed(num_seqs, 0);  // each row-pass sequence's first block, once
    std::vector<int32_t> firsts;
    firsts.reserve(row_pass.size());
    for (int32_t q : row_pass) {
      const int32_t s = seq[q];
      if (listed[s] || used[s] == 0) continue;
      listed[s] = 1;
      firsts.push_back(block_tables[static_cast<int64_t>(s) * block_table_stride]);
    }
    may_share = !firsts.empty() && distinct_count(firsts) < static_cast<int64_t>(firsts.size());
  }
  std::vector<Group> groups;
  if (may_share && static_cast<int64_t>(row_pass.size()) >= kMinSharedRows && tiled) {
    groups = prefix_groups(row_pass, seq, tables, ceil_div(kMinSharedTokens, block_size));
  }

  // Rule 4: the partition size.
  int32_t partition = partition_size;
  if (partition == 0) {
    if (!groups.empty()) {
      const Group* largest = &groups[0];
      int64_t tile_count = 0;
      for (const Group& g : groups) {
        if (g.count * g.common > largest->count * largest->common) largest = &g;
        tile_count += ceil_div(g.count, kTileRows);
      }
      partition = prefix_partition(largest->common * block_size, tile_count, num_heads);
    }
    if (partition == 0) {
      int64_t n_present = 0, wide = 0;
      for (int32_t s = 0; s < num_seqs; ++s) {
        if (!present[s]) continue;
        ++n_present;
        wide += ceil_div(context_lens[s], 1024);
      }
      const int64_t per_seq = std::max<int64_t>(1, num_queries / n_present);
      partition = wide * per_seq * num_heads >= kWidePartitionItems ? 1024 : 512;
    }
  }

  // Rule 3 continued: prefix tiles.
  for (const Group& g : groups) {
    const int64_t parts = g.common * block_size / partition;
    if (parts < 1) continue;
    const int64_t need = ceil_div(parts * partition, block_size);
    int64_t count = g.count;
    for (int64_t offset = kTileRows; offset < count; offset += kTileRows) {
      if (used[seq[row_pass[g.start + offset]]] < need) {
        count = offset;
        break;
      }
    }
    for (int64_t i = g.start; i < g.start + count; ++i) row_first[i] = static_cast<int32_t>(parts);
    const int32_t first_row = row_pass[g.start];
    for (int64_t offset = 0; offset < count; offset += kTileRows) {
      tiles.push_back({static_cast<int32_t>(first_row + offset),
                       static_cast<int32_t>(std::min<int64_t>(kTileRows, count - offset)), 0,
                       static_cast<int32_t>(parts)});
    }
  }

  // Rule 5: the load hint, over what the row pass still reads.
  bool shared_kv = false;
  if (!row_pass.empty() && may_share) {
    // The ids of every distinct (sequence, first block) the row pass reads from: a sequence's
    // first such pair is found through a per-sequence slot, any further one (a sequence whose
    // rows start at different partitions) through a sorted list.
    std::vector<int64_t> first_of(num_seqs, -1);
    std::vector<std::pair<int32_t, int64_t>> segments, more;  // (sequence, first column) read
    for (size_t i = 0; i < row_pass.size(); ++i) {
      const int32_t s = seq[row_pass[i]];
      const int64_t first = static_cast<int64_t>(row_first[i]) * partition / block_size;
      if (first_of[s] < 0) {
        first_of[s] = first;
        segments.emplace_back(s, first);
      } else if (first_of[s] != first) {
        more.emplace_back(s, first);
      }
    }
    std::sort(more.begin(), more.end());
    more.erase(std::unique(more.begin(), more.end()), more.end());
    segments.insert(segments.end(), more.begin(), more.end());
    // The ids are counted where they lie in the tables: their number and range first, then one
    // bit per id of the range (distinct_count's rule, without gathering them).
    int64_t n = 0;
    int32_t low = INT32_MAX, high = INT32_MIN;
    for (const auto& [s, first] : segments) {
      const int32_t* row = tables.base + static_cast<int64_t>(s) * tables.stride;
      for (int64_t c = first; c < used[s]; ++c) {
        low = std::min(low, row[c]);
        high = std::max(high, row[c]);
      }
      n += std::max<int64_t>(used[s] - first, 0);
    }
    if (n > 0) {
      const int64_t range = static_cast<int64_t>(high) - low + 1;
      int64_t distinct = 0;
      if (range <= 64 * std::max<int64_t>(4096, 16 * n)) {
        std::vector<uint64_t> seen((range + 63) / 64, 0);
        for (const auto& [s, first] : segments) {
          const int32_t* row = tables.base + static_cast<int64_t>(s) * tables.stride;
          for (int64_t c = first; c < used[s]; ++c) {
            const int64_t bit = static_cast<int64_t>(row[c]) - low;
            uint64_t& word = seen[bit >> 6];
            const uint64_t mask = uint64_t{1} << (bit & 63);
            distinct += (word & mask) == 0;
            word |= mask;
          }
        }
      } else {
        std::vector<int32_t> ids;
        ids.reserve(static_cast<size_t>(n));
        for (const auto& [s, first] : segments) {
          const int32_t* row = tables.base + static_cast<int64_t>(s) * tables.stride;
          ids.insert(ids.end(), row + first, row + std::max<int64_t>(used[s], first));
        }
        distinct = distinct_count(ids);
      }
      shared_kv = static_cast<double>(n - distinct) >= kSharedKvFraction * static_cast<double>(n);
    }
  }

  // The merge list: rows no whole tile covers whose visible keys span several partitions.
  std::vector<char> keep(num_queries, 1);
  for (const Tile& t : tiles) {
    if (t.end == PKV_TILE_WHOLE) std::fill(keep.begin() + t.first, keep.begin() + t.first + t.count, 0);
  }
  int64_t num_merge = 0;
  for (int64_t q = 0; q < num_queries; ++q) {
    if (keep[q] && (partition <= 0 || vis[q] > partition)) ++num_merge;
  }

  // Rule 6: row-pass items, longest first (stable), by a counting sort on their key count.
  const int64_t part = partition > 0 ? partition : kDefaultPlanPartition;
  int64_t num_items = 0;
  for (size_t i = 0; i < row_pass.size(); ++i) {
    const int64_t nparts = std::max<int64_t>(1, ceil_div(vis[row_pass[i]], part));
    num_items += std::max<int64_t>(nparts - row_first[i], 0);
  }
  counts_out[0] = num_items;
  counts_out[1] = static_cast<int64_t>(tiles.size());
  counts_out[2] = num_merge;
  if (num_items > rows_capacity || counts_out[1] > tiles_capacity || num_merge > merge_capacity) {
    return PKV_ETOOBIG;
  }
  if ((num_items > 0 && !rows_out) || (!tiles.empty() && !tiles_out) || (num_merge > 0 && !merge_out)) {
    return PKV_EINVAL;
  }
  std::vector<int64_t> bucket(part + 2, 0);  // items per key count (0 .. part)
  int64_t key_sum = 0;
  for (size_t i = 0; i < row_pass.size(); ++i) {
    const int64_t v = vis[row_pass[i]];
    const int64_t nparts = std::max<int64_t>(1, ceil_div(v, part));
    for (int64_t p = row_first[i]; p < nparts; ++p) {
      const int64_t keys = std::min<int64_t>(part, v - p * part);
      ++bucket[part - keys];  // longest first
      key_sum += std::max<int64_t>(keys, 0);
    }
  }
  for (int64_t k = 0, at = 0; k <= part; ++k) {  // bucket start offsets
    const int64_t n = bucket[k];
    bucket[k] = at;
    at += n;
  }
  for (size_t i = 0; i < row_pass.size(); ++i) {
    const int64_t v = vis[row_pass[i]];
    const int64_t nparts = std::max<int64_t>(1, ceil_div(v, part));
    for (int64_t p = row_first[i]; p < nparts; ++p) {
      const int64_t keys = std::min<int64_t>(part, v - p * part);
      const int64_t at = bucket[part - keys]++;
      rows_out[2 * at] = row_pass[i];
      rows_out[2 * at + 1] = static_cast<int32_t>(p);
    }
  }
  for (size_t i = 0; i < tiles.size(); ++i) {
    tiles_out[4 * i] = tiles[i].first;
    tiles_out[4 * i + 1] = tiles[i].count;
    tiles_out[4 * i + 2] = tiles[i].begin;
    tiles_out[4 * i + 3] = tiles[i].end;
  }
  for (int64_t q = 0, at = 0; q < num_queries; ++q) {
    if (keep[q] && (partition <= 0 || vis[q] > partition)) merge_out[at++] = static_cast<int32_t>(q);
  }
  const bool short_rows = num_items > 0 && key_sum < kShortRowKeys * num_items;
  // The keys the tile pass reads per head: a whole tile every visible key of its rows, a
  // partitioned one those in its partitions.
  int64_t tile_keys = 0;
  for (const Tile& t : tiles) {
    const int64_t lo = t.end == PKV_TILE_WHOLE ? 0 : static_cast<int64_t>(t.begin) * part;
    const bool to_last = t.end == PKV_TILE_WHOLE || t.end <= t.begin;
    for (int32_t r = 0; r < t.count; ++r) {
      const int64_t v = vis[t.first + r];
      const int64_t hi = to_last ? v : std::min<int64_t>(v, static_cast<int64_t>(t.end) * part);
      tile_keys += std::max<int64_t>(hi - lo, 0);
    }
  }
  const bool dominant = num_items > 0 && !tiles.empty() &&
                        tile_keys * kDominantTileWeight >= key_sum * esize * kDominantRowWeight;
  launch_out[0] = partition;
  launch_out[1] = (shared_kv ? PKV_ATTN_SHARED_KV : 0) | (short_rows ? PKV_ATTN_SHORT_ROWS : 0) |
                  (dominant ? PKV_ATTN_DOMINANT_TILES : 0);
  return PKV_OK;
}
