"""Slots, append, copy-on-write and the paged forward on the CPU -- test infrastructure only.

Restates src/paged_kv_serving/engine/runner.py:95-227: a zeroed float32 pool per layer shaped
(num_blocks, block_size, heads, head_dim); ``slot = block_table[p // B] * B + p % B`` for every
token (runner.py:149-159); keys (after RoPE) and values scattered to their slots before attention
(runner.py:195-196); one paged attention call per batch entry (runner.py:198-212); the block copy
of copy-on-write across every layer (runner.py:128-133).

Batches are duck-typed: ``batch.entries`` with ``seq_id, token_ids, positions, block_table,
logits_index`` as in the reference's BatchEntry (runner.py:33-68).
"""

from __future__ import annotations

import numpy as np

from oracle.attention import DEFAULT_TILE_BLOCKS, paged_attention

__all__ = ["OracleRunner", "append", "copy_block", "slots_for"]


def slots_for(seq_id: str, positions, block_table, block_size: int) -> list[int]:
    """Flat slot of every position, raising the reference's message for a missing block
    (runner.py:149-159)."""
    out = []
    for position in positions:
        index = position // block_size
        if index >= len(block_table):
            raise ValueError(f"sequence {seq_id}: position {position} has no block in the table")
        out.append(block_table[index] * block_size + position % block_size)
    return out


def append(key_pool: np.ndarray, value_pool: np.ndarray, slots, keys, values) -> None:
    """Scatter token rows into one layer's pools by flat slot (runner.py:195-196)."""
    heads, dim = key_pool.shape[-2:]
    key_pool.reshape(-1, heads, dim)[np.asarray(slots, dtype=np.int64)] = keys
    value_pool.reshape(-1, heads, dim)[np.asarray(slots, dtype=np.int64)] = values


def copy_block(keys: np.ndarray, values: np.ndarray, source: int, destination: int) -> None:
    """Byte copy of one block across every layer (runner.py:128-133)."""
    if source == destination:
        raise ValueError("copy-on-write must not copy a block onto itself")
    keys[:, destination] = keys[:, source]
    values[:, destination] = values[:, source]


class OracleRunner:
    """NumPy counterpart of the reference ModelRunner, driving an ``OracleModel``."""

    def __init__(self, model, *, num_blocks: int, block_size: int, tile_blocks: int = DEFAULT_TILE_BLOCKS):
        if num_blocks < 1 or block_size < 1:
            raise ValueError("num_blocks and block_size must be >= 1")
        if tile_blocks < 1:
            raise ValueError("tile_blocks must be >= 1")
        c = model.config
        self.model = model
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.tile_blocks = tile_blocks
        shape = (c.n_layers, num_blocks, block_size, c.n_heads, c.head_dim)
        self.keys = np.zeros(shape, dtype=np.float32)
        self.values = np.zeros(shape, dtype=np.float32)

    def copy_block(self, source: int, destination: int) -> None:
        copy_block(self.keys, self.values, source, destination)

    def execute(self, batch) -> dict[str, np.ndarray]:
        """One ragged forward; logits rows of the entries that ask for them (runner.py:161-227)."""
        entries = batch.entries
        if not entries:
            return {}
        c = self.model.config
        tokens = np.asarray([t for e in entries for t in e.token_ids], dtype=np.int64)
        if np.any(tokens < 0) or np.any(tokens >= c.vocab_size):
            raise ValueError("token id outside the vocabulary")
        positions = np.asarray([p for e in entries for p in e.positions], dtype=np.int64)
        if np.any(positions >= c.max_seq_len):
            raise ValueError("position beyond max_seq_len")
        slots = [s for e in entries for s in slots_for(e.seq_id, e.positions, e.block_table, self.block_size)]
        hidden = self.model.embed(tokens)
        total = tokens.size
        for index, layer in enumerate(self.model.weights.layers):
            q, k, v = self.model.project_qkv(hidden, layer, positions)
            append(self.keys[index], self.values[index], slots, k, v)
            attended = np.empty_like(q)
            offset = 0
            for entry in entries:
                stop = offset + len(entry.token_ids)
                attended[offset:stop] = paged_attention(
                    q[offset:stop],
                    positions[offset:stop],
                    self.keys[index],
                    self.values[index],
                    np.asarray(entry.block_table, dtype=np.int64),
                    entry.positions[-1] + 1,
                    self.model.attention_scale,
                    tile_blocks=self.tile_blocks,
                )
                offset = stop
            hidden = hidden + attended.reshape(total, c.d_model) @ layer.out_proj
            hidden = (hidden + self.model.feed_forward(hidden, layer)).astype(np.float32)
        wanted, names, offset = [], [], 0
        for entry in entries:
            if entry.logits_index is not None:
                wanted.append(offset + entry.logits_index)
                names.append(entry.seq_id)
            offset += len(entry.token_ids)
        if not wanted:
            return {}
        logits = self.model.logits_from_hidden(hidden[wanted])
        return dict(zip(names, logits))
