/*
 * pkv.h -- C ABI of the MI355X (gfx950) KV-cache data path.
 *
 * The reference (rouviere-german/paged-kv-serving) is pure Python + NumPy and has no FFI of its
 * own. Each entry point below replaces one NumPy operation of the reference's data path; the
 * comment above each names the reference code it replaces (paths are relative to the reference
 * repository root).
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers (HIP global memory) unless stated otherwise. The caller owns
 *     every buffer, including the attention workspace. No compute entry point allocates memory
 *     or creates a stream or event: the only resources the library makes are the per-device
 *     ones pkv_init creates, once, when the caller asks for them.
 *   - `device` is the HIP device ordinal the pointers live on. The library makes it current for
 *     the duration of the call and restores the caller's device afterwards, so calls may come
 *     from any host thread (the library keeps no per-thread state; per-device state is guarded
 *     by a per-device mutex).
 *   - `stream` is a hipStream_t passed as void*; NULL means the default stream. All work is
 *     enqueued on it, asynchronously; nothing synchronises the host.
 *   - Return value: PKV_OK (0) on success, a negative PKV_E* code otherwise. pkv_error_string()
 *     maps a code to a constant message. Argument errors are detected before anything is
 *     enqueued.
 *   - Pools are laid out [num_layers, num_blocks, block_size, num_heads, head_dim], row-major,
 *     exactly the shape of the reference's pools (src/paged_kv_serving/engine/runner.py:112-114).
 *     A "slot" is block_id * block_size + offset (runner.py:158), so token row `slot` of layer l
 *     starts at element ((l * num_blocks * block_size) + slot) * num_heads * head_dim.
 */
#ifndef PKV_H_
#define PKV_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type of a pool or of an input buffer. */
typedef enum pkv_dtype {
  PKV_F32 = 0,  /* IEEE binary32 */
  PKV_BF16 = 1, /* bfloat16; written from float32 with round-to-nearest-even */
} pkv_dtype;

/* pkv_paged_attention flags. */
#define PKV_ATTN_SHARED_KV 1 /* blocks are shared between sequences of the batch (a common
                                prefix): load K/V rows through the caches instead of streaming
                                them past, so the other readers hit L2 / the Infinity Cache */

#define PKV_ATTN_SHORT_ROWS 2 /* the row pass's items are short (a few hundred keys): launch a
                                lighter workgroup so more of them are in flight at once */

#define PKV_ATTN_DOMINANT_TILES 4 /* the tile pass carries more of the call's time than the row
                                    pass beside it: run it as three register-staged workgroups
                                    per CU (the row workgroups fill in around them) instead of
                                    one (float32, staged straight into LDS) or two per CU */

/* pkv_paged_attention tile record: end partition of a tile computed whole by one workgroup. */
#define PKV_TILE_WHOLE (-1)

#define PKV_OK 0
#define PKV_EINVAL (-1)       /* a size, stride, pointer or enum argument is out of range */
#define PKV_EUNSUPPORTED (-2) /* a valid but unimplemented shape (e.g. head_dim 96) */
#define PKV_EHIP (-3)         /* the HIP runtime reported an error while enqueueing */
#define PKV_ETOOBIG (-4)      /* the call needs more scratch than PKV_STATIC_SCRATCH_BYTES */

/* Size of the library's static per-device scratch (pkv_paged_attention_noalloc). */
#define PKV_STATIC_SCRATCH_BYTES (64LL << 20)

/*
 * Creates the library's resources on `device`: a second stream (default priority, non-blocking)
 * and two events, used by pkv_paged_attention to run the MFMA tile pass of a call beside its
 * row-streaming pass. Idempotent and thread-safe; the resources live until the process ends.
 * Call it once per device before the first attention call that should overlap its passes, and
 * before capturing attention calls into a HIP graph. Without it, calls run both passes one
 * after the other on the caller's stream (same results). Calls whose row pass has fewer than
 * 2,048 workgroups (row items x head groups) also run both passes on the caller's stream: the
 * fork and join onto the second stream cost more host time than such a call's device time.
 *
 * No counterpart in the reference (it has no device); the resources replace nothing there.
 */
int pkv_init(int device);

/* Version string of the library ("pkv <major>.<minor>"). Host-only, never fails. */
const char* pkv_version(void);

/* Constant, NUL-terminated description of a PKV_* return code. Host-only. */
const char* pkv_error_string(int code);

/*
 * Slot-mapped append of one layer's new keys and values into the pools.
 *
 * Replaces src/paged_kv_serving/engine/runner.py:195-196:
 *     key_pool.reshape(-1, H, D)[slots] = keys ; value_pool.reshape(-1, H, D)[slots] = values
 *
 *   key_pool, value_pool : the layer's pools, [num_slots, num_heads, head_dim] of pool_dtype
 *                          (num_slots = num_blocks * block_size).
 *   new_keys, new_values : [num_tokens, num_heads, head_dim] of src_dtype; token t of the keys
 *                          starts at element t * key_token_stride, of the values at
 *                          t * value_token_stride (each H*D row itself is contiguous), so views
 *                          into a fused QKV output need no copy.
 *   slot_mapping         : int64 [num_tokens]. A slot outside [0, num_slots) is skipped (the
 *                          host validates slots first; this only keeps a bad slot in bounds).
 * A float32 source into a bfloat16 pool is rounded to nearest even; equal types copy bits.
 * Duplicate slots in one call leave an unspecified one of the duplicate rows (the reference's
 * fancy-index assignment keeps the last; the engine never produces duplicates).
 */
int pkv_append(void* key_pool, void* value_pool, pkv_dtype pool_dtype, int64_t num_slots,
               const void* new_keys, const void* new_values, pkv_dtype src_dtype,
               int64_t key_token_stride, int64_t value_token_stride,
               const int64_t* slot_mapping, int64_t num_tokens, int32_t num_heads,
               int32_t head_dim, int device, void* stream);

/*
 * Copy-on-write block copies, batched: for every pair (src, dst), block src is copied over block
 * dst in every layer, for keys and values.
 *
 * Replaces src/paged_kv_serving/engine/runner.py:128-133 (ModelRunner.copy_block), called once
 * per pair by BlockManager.prepare_for_write (src/paged_kv_serving/engine/blocks.py:162-164).
 *
 *   key_pool, value_pool : whole pools, [num_layers, num_blocks, block_elems] of dtype.
 *   pairs                : int64 [num_pairs, 2] = (src, dst), device memory.
 * All pairs of one call run concurrently, so no dst may appear twice and no dst may be the src
 * of another pair in the same call (the Python host splits dependent sequences into several
 * calls). Pairs with an id outside [0, num_blocks) or with src == dst are skipped.
 */
int pkv_copy_blocks(void* key_pool, void* value_pool, pkv_dtype dtype, const int64_t* pairs,
                    int64_t num_pairs, int32_t num_layers, int64_t num_blocks, int64_t block_elems,
                    int device, void* stream);

/*
 * Rotary embedding of one layer's queries and keys fused with the slot-mapped append of the
 * rotated keys and the values.
 *
 * Replaces src/paged_kv_serving/engine/model.py:251-252 (apply_rope, model.py:70-81, on the q
 * and k of the fused projection) followed by runner.py:195-196 (the append), for float32
 * activations:
 *     q' = rope(q, positions) ; key_pool[slots] = rope(k, positions) ; value_pool[slots] = v
 * with rope(x)[i] = x[i]*cos - x[i+D/2]*sin and rope(x)[i+D/2] = x[i+D/2]*cos + x[i]*sin,
 * cos/sin = table[position][i]; each product and sum is rounded separately, so the results
 * equal the reference's float32 NumPy expressions bit for bit.
 *
 *   rotated_queries      : float32 [num_tokens, num_heads, head_dim], token stride
 *                          rotated_token_stride. May be `queries` itself (same stride) to rotate
 *                          in place; must not otherwise overlap an input.
 *   queries, keys, values: float32 [num_tokens, num_heads, head_dim] with their own token
 *                          strides (>= num_heads * head_dim), e.g. the three slices of a fused
 *                          [num_tokens, 3, num_heads, head_dim] projection output.
 *   positions            : int64 [num_tokens], absolute token positions.
 *   cos_table, sin_table : float32 [table_rows, head_dim / 2] (model.py:60-67).
 *   key_pool, value_pool : the layer's pools, [num_slots, num_heads, head_dim] of pool_dtype.
 *   slot_mapping         : int64 [num_tokens].
 * head_dim must be even. A token whose position is outside [0, table_rows) is skipped entirely
 * (its rotated query is not written); a slot outside [0, num_slots) skips only that token's
 * pool writes. The host validates both first; the checks only keep a bad index in bounds.
 * Into a bfloat16 pool the rotated keys and the values are rounded to nearest even.
 */
int pkv_rope_append(float* rotated_queries, int64_t rotated_token_stride, const float* queries,
                    const float* keys, const float* values, int64_t query_token_stride,
                    int64_t key_token_stride, int64_t value_token_stride,
                    const int64_t* positions, const float* cos_table, const float* sin_table,
                    int64_t table_rows, void* key_pool, void* value_pool, pkv_dtype pool_dtype,
                    int64_t num_slots, const int64_t* slot_mapping, int64_t num_tokens,
                    int32_t num_heads, int32_t head_dim, int device, void* stream);

/*
 * Bytes of float32 workspace pkv_paged_attention needs for a batch (0 when no query can span
 * more than one partition). Host-only.
 */
int64_t pkv_attention_workspace_bytes(int64_t num_queries, int32_t num_heads, int32_t head_dim,
                                      int32_t max_context_len, int32_t partition_size);

/*
 * Nonzero when the MFMA tile path of pkv_paged_attention supports this head_dim (32, 64, 128,
 * 256). Host-only.
 */
int pkv_tile_head_dim_supported(int32_t head_dim);

/*
 * Paged causal attention of a ragged batch over one layer's pools: every query row attends to
 * the keys at positions [0, min(context_len, position + 1)) of its sequence, read through the
 * sequence's block table.
 *
 * Replaces src/paged_kv_serving/engine/attention.py:42-121 (paged_attention) together with the
 * per-sequence loop of src/paged_kv_serving/engine/runner.py:198-212: one call covers every
 * sequence of the batch, decode rows and prefill-chunk rows alike.
 *
 *   out              : float32 [num_queries, num_heads, head_dim], contiguous; 16-byte aligned
 *                      when num_tiles > 0.
 *   queries          : float32; query t starts at element t * query_token_stride, and its
 *                      [num_heads, head_dim] block is contiguous.
 *   query_positions  : int32 [num_queries], absolute position of each query (the causal mask:
 *                      key position > query position is masked, attention.py:102-104).
 *   query_seq        : int32 [num_queries], index of the sequence each query belongs to.
 *   caller_rows      : int32 [num_queries] or NULL. Query t's row of `queries` and of `out`
 *                      (and of the new keys, values and slots of pkv_paged_attention_append) is
 *                      caller_rows[t]; NULL means t. Every other per-query array (positions,
 *                      sequences, the plan's rows, tiles and merge list) is indexed by t. This
 *                      lets a plan order the queries its own way (rows sharing a prefix next to
 *                      each other) while the caller keeps its token order: no copy of the
 *                      queries in and of the outputs back. caller_rows must be a permutation of
 *                      [0, num_queries); a query whose entry lies outside that range is skipped
 *                      (its output row is not written).
 *   rows, num_rows   : the plan's row-pass work items, int32 [num_rows, 2] = (query row,
 *                      partition): one workgroup per item and group of heads computes that
 *                      partition of that row with the row-streaming pass (the right pass for
 *                      decode rows). Items past a row's last partition are skipped, so listing
 *                      partitions up to an upper bound of the row's visible length is safe.
 *   tiles, num_tiles : the plan's tile list, int32 [num_tiles, 4] = (first row, row count <= 64,
 *                      first partition, end partition; end <= first means through the last):
 *                      runs of consecutive rows computed by the fp32 MFMA tile pass over those
 *                      partitions, one workgroup per (tile, head, partition). Keys are read
 *                      through the table of the tile's first row, so the rows are either one
 *                      sequence's (a prefill chunk) or rows of several sequences whose tables
 *                      hold the same block ids over the tile's partitions (a shared prefix;
 *                      those rows then also appear in the row list with the first partition
 *                      after the tile's). End partition PKV_TILE_WHOLE: one workgroup per
 *                      (tile, head) covers every visible key of the tile's rows and writes
 *                      their final outputs (the first partition is then ignored; such rows must
 *                      not be in the merge list). Needs pkv_tile_head_dim_supported(head_dim).
 *                      Every (query row, partition) must be covered exactly once. With rows and
 *                      tiles both NULL, every partition of every row goes through the
 *                      row-streaming pass.
 *   merge_rows,
 *   num_merge_rows   : int32 [num_merge_rows], the query rows whose per-partition results the
 *                      reduce pass merges: every row whose visible context spans more than one
 *                      partition and that no whole tile covers (listing a row that fits one
 *                      partition is harmless; merge_rows may be NULL when the count is 0).
 *                      num_merge_rows = -1: every row of the batch, which is only correct
 *                      without whole tiles.
 *   key_cache,
 *   value_cache      : the layer's pools, [num_blocks, block_size, num_heads, head_dim], kv_dtype,
 *                      16-byte aligned.
 *   block_tables     : int32 [num_seqs, block_table_stride], physical block ids in logical order.
 *   context_lens     : int32 [num_seqs], valid cached tokens of each sequence (runner.py:66-68).
 *   max_context_len  : an upper bound of every context_len; it sizes the grid, and visible
 *                      lengths are clamped to it, so block_table_stride * block_size must be
 *                      >= max_context_len (checked).
 *   partition_size   : keys per split-context partition, a positive multiple of 16, <= 1024;
 *                      0 selects the library default (512).
 *   flags            : PKV_ATTN_SHARED_KV, PKV_ATTN_SHORT_ROWS and/or PKV_ATTN_DOMINANT_TILES,
 *                      or 0. They only choose how the kernels run; the results agree within
 *                      float32 rounding (PKV_ATTN_DOMINANT_TILES: bit for bit).
 *   workspace        : float32 scratch of pkv_attention_workspace_bytes(...) bytes (may be
 *                      NULL when that is 0); 16-byte aligned when num_tiles > 0.
 * A query whose every key is masked gets a zero output (attention.py:120-121).
 * Block ids are read only for positions below the query's visible length, so table entries
 * past a sequence's last used block may hold anything. A block id outside [0, num_blocks) at a
 * visible position is not read either: its keys take no part in the softmax (the reference
 * would raise on such a table; every pass here skips them alike). Supported head_dim: 8, 16, 32, 64, 128,
 * 256; any block_size >= 1; kv_dtype F32 or BF16 (accumulation is float32 either way).
 */
int pkv_paged_attention(float* out, const float* queries, int64_t query_token_stride,
                        const int32_t* query_positions, const int32_t* query_seq,
                        int64_t num_queries, const int32_t* caller_rows, const int32_t* rows,
                        int64_t num_rows,
                        const int32_t* tiles, int64_t num_tiles, const int32_t* merge_rows,
                        int64_t num_merge_rows, const void* key_cache,
                        const void* value_cache, pkv_dtype kv_dtype, int64_t num_blocks,
                        int32_t block_size, const int32_t* block_tables,
                        int32_t block_table_stride, const int32_t* context_lens,
                        int32_t num_seqs, int32_t num_heads, int32_t head_dim, float scale,
                        int32_t max_context_len, int32_t partition_size, int32_t flags,
                        float* workspace, int64_t workspace_bytes, int device, void* stream);

/*
 * pkv_paged_attention without a workspace argument, for callers that cannot allocate: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 *
 * No counterpart in the reference. Arguments, plan, results and errors are pkv_paged_attention's;
 * the split-context workspace is instead a static device array of PKV_STATIC_SCRATCH_BYTES
 * (64 MiB) in the library, one copy per GPU, held until the process ends. The call allocates
 * nothing and creates nothing: on a device's first use it only looks up that device's copy of
 * the array (pkv_init does the same). A batch whose workspace
 * (pkv_attention_workspace_bytes) exceeds the buffer is refused with PKV_ETOOBIG before anything
 * is enqueued. Nothing in the buffer needs to start at zero: every entry a call reads, the same
 * call has written before. Every call on one GPU shares that GPU's buffer, so two calls whose
 * execution overlaps on one GPU (on different streams, without ordering between them) race;
 * calls on one stream, or ordered by events, do not.
 */
int pkv_paged_attention_noalloc(float* out, const float* queries, int64_t query_token_stride,
                                const int32_t* query_positions, const int32_t* query_seq,
                                int64_t num_queries, const int32_t* caller_rows,
                                const int32_t* rows, int64_t num_rows,
                                const int32_t* tiles, int64_t num_tiles,
                                const int32_t* merge_rows, int64_t num_merge_rows,
                                const void* key_cache, const void* value_cache,
                                pkv_dtype kv_dtype, int64_t num_blocks, int32_t block_size,
                                const int32_t* block_tables, int32_t block_table_stride,
                                const int32_t* context_lens, int32_t num_seqs, int32_t num_heads,
                                int32_t head_dim, float scale, int32_t max_context_len,
                                int32_t partition_size, int32_t flags, int device, void* stream);

/*
 * A decode step's append and attention in one pass: pkv_append of every query row's own new key
 * and value row followed by pkv_paged_attention, with the append done by the row-streaming pass
 * itself. The workgroups whose partition holds a row's position take that row's key and value
 * from new_keys / new_values, use them for that position and write them to slot_mapping[t], so
 * the pools end exactly as after pkv_append and the outputs are those of the two calls.
 *
 * Replaces src/paged_kv_serving/engine/runner.py:195-196 (the append) and :198-212 (the
 * per-entry attention loop, attention.py:42-121) for a batch of decode rows.
 *
 * Arguments are pkv_paged_attention's plus new_keys / new_values ([num_queries, num_heads,
 * head_dim] of new_dtype with token strides
 * new_key_token_stride / new_value_token_stride, 16-byte aligned rows; bfloat16 only into a
 * bfloat16 pool) and slot_mapping (int64 [num_queries]), as for pkv_append; all three in the
 * caller's row order, like queries and out (with caller_rows, query t's new token is row
 * caller_rows[t] of new_keys / new_values and goes to slot_mapping[caller_rows[t]]). Query t's
 * new token sits at query_positions[t]. Only the row pass appends, so the tiles may cover only
 * partitions that hold no row's new position: shared-prefix tiles over blocks no row writes,
 * which the last rule below guarantees (a written block that one row alone reads lies in no
 * shared prefix). Preconditions, which the caller checks: each sequence has exactly one query
 * row in the call, that row's position is below its context_len and below max_context_len, and slot_mapping[t] is the slot the block table gives that position (as in
 * runner.py:149-159). A slot outside the pool is not written, as in pkv_append. No row may read a
 * block another row writes: the block holding each row's new slot must occur exactly once among
 * the blocks every row reads (table entries [0, ceil(visible length / block_size)) of each row's
 * sequence), namely in its own row's table at that position. A written key reaches only its own
 * row, so a second reader of the block (the same sequence twice, tables sharing the block being
 * written, a table naming it twice) would race with the write; such a batch takes pkv_append
 * followed by pkv_paged_attention, which the Python runner chooses by this rule.
 */
int pkv_paged_attention_append(
    float* out, const float* queries, int64_t query_token_stride, const int32_t* query_positions,
    const int32_t* query_seq, int64_t num_queries, const int32_t* caller_rows, const int32_t* rows,
    int64_t num_rows, const int32_t* tiles, int64_t num_tiles, const int32_t* merge_rows,
    int64_t num_merge_rows, void* key_cache, void* value_cache,
    pkv_dtype kv_dtype, int64_t num_blocks, int32_t block_size, const int32_t* block_tables,
    int32_t block_table_stride, const int32_t* context_lens, int32_t num_seqs, int32_t num_heads,
    int32_t head_dim, float scale, int32_t max_context_len, int32_t partition_size, int32_t flags,
    float* workspace, int64_t workspace_bytes, const void* new_keys, const void* new_values,
    pkv_dtype new_dtype, int64_t new_key_token_stride, int64_t new_value_token_stride,
    const int64_t* slot_mapping, int device, void* stream);

/*
 * The host plan of one pkv_paged_attention call (host-only: reads and writes host memory, never
 * touches a device).
 *
 * Replaces nothing in the reference, whose runner loops over sequences
 * (src/paged_kv_serving/engine/runner.py:198-212); it decides how this library's one ragged call
 * covers them: rows (the row pass's (query row, partition) items), tiles (runs of rows for the
 * MFMA tile pass, including whole prefill tiles and shared-prefix tiles), the merge list, the
 * partition size and the flags. Results never depend on the plan, only the launch does.
 *
 *   query_seq, query_positions : int32 [num_queries] (positions may be NULL: every row then
 *                                sees its whole context), host memory.
 *   block_tables               : int32 [num_seqs, block_table_stride], host; every sequence a
 *                                query names must hold ceil(context / block_size) entries.
 *   context_lens               : int32 [num_seqs], host.
 *   kv_dtype                   : the pools' element type; it weighs the row pass's bytes
 *                                against the tile pass's products for PKV_ATTN_DOMINANT_TILES.
 *   partition_size             : 0 lets the planner choose; a positive value is kept.
 *   min_tile_rows              : the shortest run of one sequence's rows made into tiles (8).
 *   rows_out [rows_capacity, 2], tiles_out [tiles_capacity, 4], merge_out [merge_capacity] :
 *                                int32 outputs in pkv_paged_attention's layout.
 *   counts_out                 : int64 [3] = rows, tiles, merge rows written (or needed).
 *   launch_out                 : int32 [2] = partition size, flags for pkv_paged_attention.
 * Returns PKV_ETOOBIG, with counts_out holding the sizes needed and nothing else written, when a
 * capacity is too small.
 */
int pkv_plan_batch(const int32_t* query_seq, const int32_t* query_positions, int64_t num_queries,
                   const int32_t* block_tables, int32_t block_table_stride,
                   const int32_t* context_lens, int32_t num_seqs, int32_t block_size,
                   int32_t num_heads, int32_t head_dim, pkv_dtype kv_dtype, int32_t partition_size,
                   int32_t min_tile_rows, int32_t* rows_out, int64_t rows_capacity,
                   int32_t* tiles_out, int64_t tiles_capacity, int32_t* merge_out,
                   int64_t merge_capacity, int64_t* counts_out, int32_t* launch_out);

/*
 * RMSNorm of rows of float32 activations, optionally after the residual add that feeds it.
 *
 * Replaces src/paged_kv_serving/engine/model.py:43-46 (rms_norm) as the runner applies it
 * (model.py:256-264: before the QKV projection, before the SwiGLU block and before the logits),
 * and the residual adds in front of the second and third (hidden = hidden + ...):
 *     if delta: hidden[r] = hidden[r] + delta[r]
 *     out[r] = hidden[r] / sqrt(mean(hidden[r] ** 2) + eps) * weight
 *
 *   out    : float32 [num_rows, dim], row r at r * out_stride. May be `hidden` itself.
 *   hidden : float32 [num_rows, dim], row r at r * hidden_stride; updated in place when delta is
 *            given.
 *   delta  : float32 [num_rows, dim] at r * delta_stride, or NULL (no residual add).
 *   weight : float32 [dim].
 * Each product, quotient and square root is the correctly rounded float32 operation; the sum of
 * squares is accumulated in float32 in a different order than NumPy's pairwise sum.
 */
int pkv_rms_norm(float* out, int64_t out_stride, float* hidden, int64_t hidden_stride,
                 const float* delta, int64_t delta_stride, const float* weight, int64_t num_rows,
                 int32_t dim, float eps, int device, void* stream);

/*
 * The SwiGLU gate product: out[r, j] = silu(gate[r, j]) * up[r, j] with
 * silu(x) = x * (1 / (1 + exp(-clip(x, -60, 60)))).
 *
 * Replaces src/paged_kv_serving/engine/model.py:49-51 (silu) and the product at model.py:256-259
 * (silu(normed @ gate_proj) * (normed @ up_proj)). gate and up are float32 [num_rows, width]
 * with row r at r * in_stride (for one [num_rows, 2 * width] product of [gate | up] weights: up =
 * gate + width, in_stride = 2 * width); out is float32 [num_rows, width] at r * out_stride.
 */
int pkv_silu_mul(float* out, int64_t out_stride, const float* gate, const float* up,
                 int64_t in_stride, int64_t num_rows, int32_t width, int device, void* stream);

/*
 * Row gather: out[r, :] = src[index[r], :] for r < num_rows, float32 rows of `width` values;
 * a row whose index lies outside [0, src_rows) is written as zeros.
 *
 * Replaces the two row lookups of the reference's forward pass: the embedding lookup
 * (src/paged_kv_serving/engine/model.py:262-263, token_embedding[token_ids]) and the choice of
 * the rows that ask for logits (runner.py:215-227, hidden[wanted]). The runner validates token ids
 * before the call, as the reference does (runner.py:175-176).
 *
 *   out   : float32, row r at r * out_stride (out_stride >= width).
 *   src   : float32 [src_rows, ...], row i at i * src_stride (src_stride >= width).
 *   index : int64 [num_rows], device memory.
 */
int pkv_gather_rows(float* out, int64_t out_stride, const float* src, int64_t src_stride,
                    int64_t src_rows, const int64_t* index, int64_t num_rows, int32_t width,
                    int device, void* stream);

/*
 * Greedy sampling: the argmax of each logits row, on the device.
 *
 * Replaces src/paged_kv_serving/engine/sampling.py:28-30 (greedy_token: int(np.argmax(logits)))
 * applied to every row the engine samples from, so one int32 per row crosses PCIe instead of
 * the whole row. NumPy's rules: ties resolve to the lowest id; a NaN beats every number and the
 * first NaN wins; -0.0 and +0.0 tie.
 *
 *   token_ids  : int32 [num_rows], output.
 *   logits     : float32 rows of vocab_size values; row r starts at element r * row_stride
 *                (row_stride >= vocab_size).
 */
int pkv_greedy_tokens(int32_t* token_ids, const float* logits, int64_t row_stride,
                      int64_t num_rows, int64_t vocab_size, int device, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PKV_H_ */
