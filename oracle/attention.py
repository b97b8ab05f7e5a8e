"""Paged attention on the CPU -- test infrastructure only (see ``oracle/__init__.py``).

``paged_attention`` restates src/paged_kv_serving/engine/attention.py:42-121: the block table is
walked in tiles of ``tile_blocks`` blocks and every tile is folded into an online softmax
(running max, running sum, unnormalised accumulator) with the guarded shift of attention.py:111
and the empty-sum guard of attention.py:120. ``dense_attention`` is the textbook closed form
(one softmax over the whole score row) in float64, used to pin the restatement.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "DEFAULT_TILE_BLOCKS",
    "dense_attention",
    "gather_context",
    "paged_attention",
]

#: attention.py:39
DEFAULT_TILE_BLOCKS = 8


def _check(queries, query_positions, key_cache, value_cache, block_table, context_len, tile_blocks):
    """Argument checks in the order and with the messages of attention.py:67-80."""
    if queries.ndim != 3:
        raise ValueError("queries must have shape (num_queries, num_heads, head_dim)")
    if queries.shape[0] != query_positions.shape[0]:
        raise ValueError("one position per query is required")
    if key_cache.shape != value_cache.shape:
        raise ValueError("key and value caches must have the same shape")
    if tile_blocks < 1:
        raise ValueError("tile_blocks must be >= 1")
    if context_len < 1:
        raise ValueError("context_len must be >= 1")
    if -(-context_len // key_cache.shape[1]) > block_table.shape[0]:
        raise ValueError("context_len exceeds the blocks listed in the block table")


def paged_attention(
    queries: np.ndarray,
    query_positions: np.ndarray,
    key_cache: np.ndarray,
    value_cache: np.ndarray,
    block_table: np.ndarray,
    context_len: int,
    scale: float,
    *,
    tile_blocks: int = DEFAULT_TILE_BLOCKS,
    dtype: type = np.float32,
) -> np.ndarray:
    """Tiled online-softmax attention over a paged cache (attention.py:42-121).

    ``queries`` (nq, H, D); ``query_positions`` (nq,); caches (N, B, H, D); ``block_table``
    physical ids in logical order. Returns (nq, H, D) in ``dtype`` (float32 reproduces the
    reference's arithmetic type; float64 gives a high-precision version of the same recurrence).
    """
    query_positions = np.asarray(query_positions)
    block_table = np.asarray(block_table)
    _check(queries, query_positions, key_cache, value_cache, block_table, context_len, tile_blocks)
    block = key_cache.shape[1]
    nq, heads, dim = queries.shape
    used = -(-context_len // block)
    # Head-major query block, so each tile is one batched BLAS product per operand
    # (the reference contracts with np.matmul for the same reason, attention.py:24-25, 101, 117).
    q = np.ascontiguousarray(queries.astype(dtype).transpose(1, 0, 2))  # (H, nq, D)
    pos = query_positions.astype(np.int64)
    big = np.full((heads, nq), -np.inf, dtype=dtype)  # running max
    total = np.zeros((heads, nq), dtype=dtype)  # running sum
    acc = np.zeros((heads, nq, dim), dtype=dtype)
    for first in range(0, used, tile_blocks):
        ids = block_table[first : min(first + tile_blocks, used)]
        start = first * block
        width = min(len(ids) * block, context_len - start)
        k = key_cache[ids].reshape(len(ids) * block, heads, dim)[:width].astype(dtype)
        v = value_cache[ids].reshape(len(ids) * block, heads, dim)[:width].astype(dtype)
        # scores[h, i, j] = q[i, h] . k[j, h] * scale
        scores = np.matmul(q, k.transpose(1, 2, 0)) * dtype(scale)
        hidden = (start + np.arange(width))[None, :] > pos[:, None]  # (nq, width)
        scores = np.where(hidden[None], dtype(-np.inf), scores)
        new_big = np.maximum(big, scores.max(axis=2))
        shift = np.where(np.isfinite(new_big), new_big, dtype(0))
        weights = np.exp(scores - shift[:, :, None])
        carry = np.exp(big - shift)
        total = total * carry + weights.sum(axis=2)
        acc = acc * carry[:, :, None] + np.matmul(weights, v.transpose(1, 0, 2))
        big = new_big
    denom = np.where(total > 0, total, dtype(1))
    return (acc / denom[:, :, None]).transpose(1, 0, 2).astype(dtype)


def gather_context(cache: np.ndarray, block_table: np.ndarray, context_len: int) -> np.ndarray:
    """The first ``context_len`` token rows of a sequence, in logical order: (ctx, H, D)."""
    block = cache.shape[1]
    used = -(-context_len // block)
    rows = cache[np.asarray(block_table[:used])]
    return rows.reshape(used * block, *cache.shape[2:])[:context_len]


def dense_attention(
    queries: np.ndarray,
    keys: np.ndarray,
    values: np.ndarray,
    scale: float,
    query_positions: np.ndarray,
) -> np.ndarray:
    """Closed form in float64: softmax over keys 0..min(ctx, pos+1)-1 of each query.

    ``keys``/``values`` are contiguous (ctx, H, D). A query that sees no key returns zeros (the
    reference's empty-sum guard, attention.py:120-121).
    """
    q = queries.astype(np.float64)
    k = keys.astype(np.float64)
    v = values.astype(np.float64)
    nq, heads, dim = q.shape
    out = np.zeros((nq, heads, dim), dtype=np.float64)
    for i, position in enumerate(np.asarray(query_positions, dtype=np.int64)):
        visible = min(k.shape[0], int(position) + 1) if position >= 0 else 0
        if visible <= 0:
            continue
        scores = np.einsum("hd,jhd->hj", q[i], k[:visible]) * float(scale)
        scores -= scores.max(axis=1, keepdims=True)
        weights = np.exp(scores)
        weights /= weights.sum(axis=1, keepdims=True)
        out[i] = np.einsum("hj,jhd->hd", weights, v[:visible])
    return out
