"""``paged_attention`` with the reference's signature and errors, computed by the HIP kernel.

Mirrors src/paged_kv_serving/engine/attention.py:42-121: causal attention of ``queries`` over
the first ``context_len`` cached tokens of one sequence, masked by absolute position. Arguments
are checked in the reference's order with its messages (attention.py:67-80). Inputs may be
torch device tensors (the result stays on the device) or NumPy arrays (they are copied to the
current HIP device and the result comes back as a NumPy array). ``tile_blocks`` is validated
and otherwise ignored: the kernel's own tiling never changes the result beyond rounding.
"""

from __future__ import annotations

import threading

import numpy as np
import torch

from paged_kv_serving_amd import ops

__all__ = ["DEFAULT_TILE_BLOCKS", "paged_attention"]

DEFAULT_TILE_BLOCKS = 8


#: Per device, a pinned host buffer that NumPy inputs are packed into for one transfer. It is
#: reused by the next call only after the call that filled it has copied its result back (a
#: synchronising copy), and the lock keeps two threads from filling it at once.
_STAGES: dict[int, torch.Tensor] = {}
_STAGE_LOCK = threading.Lock()
_TORCH_TYPES = {np.dtype(np.float32): torch.float32, np.dtype(np.int32): torch.int32}


def _staged(arrays: list[np.ndarray], device: torch.device) -> list[torch.Tensor]:
    """Device copies of contiguous float32/int32 host arrays, packed at 256-byte offsets into
    the device's pinned buffer and sent in one transfer. The caller holds ``_STAGE_LOCK``."""
    offsets, total = [], 0
    for array in arrays:
        offsets.append(total)
        total += -(-max(array.nbytes, 1) // 256) * 256
    stage = _STAGES.get(device.index)
    if stage is None or stage.numel() < total:
        stage = torch.empty(max(total, 1 << 20), dtype=torch.uint8, pin_memory=True)
        _STAGES[device.index] = stage
    host = stage.numpy()
    for array, offset in zip(arrays, offsets):
        host[offset : offset + array.nbytes] = array.reshape(-1).view(np.uint8)
    moved = stage[:total].to(device, non_blocking=True)
    return [
        moved[offset : offset + array.nbytes].view(_TORCH_TYPES[array.dtype]).view(array.shape)
        for array, offset in zip(arrays, offsets)
    ]


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
    if host and not any(isinstance(a, torch.Tensor) for a in (query_positions, key_cache, value_cache, block_table)):
        return _paged_attention_from_host(queries, query_positions, key_cache, value_cache, block_table,
                                          context_len, scale, block_size)  # fmt: skip
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


def _paged_attention_from_host(queries, query_positions, key_cache, value_cache, block_table,
                               context_len: int, scale: float, block_size: int) -> np.ndarray:  # fmt: skip
    """The reference's call on NumPy arrays: every input in one pinned transfer, the result
    copied back as a new float32 array."""
    device = torch.device("cuda", torch.cuda.current_device())
    used = -(-context_len // block_size)
    queries = np.ascontiguousarray(queries, dtype=np.float32)
    arrays = [
        np.ascontiguousarray(key_cache, dtype=np.float32),
        np.ascontiguousarray(value_cache, dtype=np.float32),
        queries,
        np.ascontiguousarray(query_positions, dtype=np.int32),
        np.zeros(queries.shape[0], dtype=np.int32),  # every query belongs to sequence 0
        np.ascontiguousarray(np.asarray(block_table)[:used], dtype=np.int32).reshape(1, used),
        np.asarray([context_len], dtype=np.int32),
    ]
    with _STAGE_LOCK:
        keys, values, q, positions, query_seq, table, context = _staged(arrays, device)
        out = ops.paged_attention_ragged(
            q, positions, query_seq, keys, values, table, context, scale,
            max_context_len=int(context_len),
        )  # fmt: skip
        return out.cpu().numpy()
