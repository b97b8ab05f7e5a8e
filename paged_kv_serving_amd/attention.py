"""``paged_attention`` with the reference's signature and errors, computed by the HIP kernel.

Mirrors src/paged_kv_serving/engine/attention.py:42-121: causal attention of ``queries`` over
the first ``context_len`` cached tokens of one sequence, masked by absolute position. Arguments
are checked in the reference's order with its messages (attention.py:67-80). Inputs may be
torch device tensors (the result stays on the device) or NumPy arrays (they are copied to the
current HIP device and the result comes back as a NumPy array). ``tile_blocks`` is validated
and otherwise ignored: the kernel's own tiling never changes the result beyond rounding.
"""

from __future__ import annotations

import numpy as np
import torch

from paged_kv_serving_amd import ops

__all__ = ["DEFAULT_TILE_BLOCKS", "paged_attention"]

DEFAULT_TILE_BLOCKS = 8


def _to_device(value, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    if isinstance(value, torch.Tensor):
        return value.to(device=device, dtype=dtype)
    return torch.as_tensor(np.asarray(value), dtype=dtype).to(device)


def paged_attention(
    queries,
    query_positions,
    key_cache,
    value_cache,
    block_table,
    context_len: int,
    scale: float,
    *,
    tile_blocks: int = DEFAULT_TILE_BLOCKS,
):
    """``(num_queries, num_heads, head_dim)`` attention output for one sequence.

    ``key_cache``/``value_cache``: ``(num_blocks, block_size, num_heads, head_dim)`` pools,
    float32 or bfloat16; ``block_table``: physical ids in logical order.
    """
    if queries.ndim != 3:
        raise ValueError("queries must have shape (num_queries, num_heads, head_dim)")
    if queries.shape[0] != query_positions.shape[0]:
        raise ValueError("one position per query is required")
    if tuple(key_cache.shape) != tuple(value_cache.shape):
        raise ValueError("key and value caches must have the same shape")
    if tile_blocks < 1:
        raise ValueError("tile_blocks must be >= 1")
    block_size = key_cache.shape[1]
    if context_len < 1:
        raise ValueError("context_len must be >= 1")
    if -(-context_len // block_size) > block_table.shape[0]:
        raise ValueError("context_len exceeds the blocks listed in the block table")

    host = not isinstance(queries, torch.Tensor)
    if isinstance(key_cache, torch.Tensor):
        device = key_cache.device
    elif isinstance(queries, torch.Tensor):
        device = queries.device
    else:
        device = torch.device("cuda", torch.cuda.current_device())
    if isinstance(key_cache, torch.Tensor):
        keys, values = key_cache, value_cache
    else:
        keys = _to_device(key_cache, torch.float32, device)
        values = _to_device(value_cache, torch.float32, device)
    keys, values = keys.contiguous(), values.contiguous()
    q = _to_device(queries, torch.float32, device).contiguous()
    num_queries = q.shape[0]
    positions = _to_device(query_positions, torch.int32, device)
    query_seq = torch.zeros(num_queries, dtype=torch.int32, device=device)
    used = -(-context_len // block_size)
    table = _to_device(block_table, torch.int32, device)[:used].reshape(1, used).contiguous()
    context = torch.full((1,), int(context_len), dtype=torch.int32, device=device)  # no host copy
    out = ops.paged_attention_ragged(
        q, positions, query_seq, keys, values, table, context, scale,
        max_context_len=int(context_len),
    )  # fmt: skip
    return out.cpu().numpy() if host else out
