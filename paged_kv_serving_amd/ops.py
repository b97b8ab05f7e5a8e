"""Tensor-level entry points of the data path: torch device tensors in, HIP kernels out.

Each function checks shapes, dtypes, devices and layouts on the host, then calls the matching
``pkv_*`` function of ``libpkv.so`` on the caller's current HIP stream (torch's current stream of
the tensors' device). Nothing here computes on the CPU: a missing library raises
:class:`~paged_kv_serving_amd._native.NativeLibraryError`.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from paged_kv_serving_amd import _native

__all__ = [
    "AttentionPlan",
    "MIN_TILE_ROWS",
    "TILE_ROWS",
    "append_kv",
    "attention_workspace_bytes",
    "copy_blocks",
    "expand_rows",
    "greedy_tokens",
    "independent_groups",
    "kv_dtype_code",
    "kv_dtype_size",
    "merge_rows_for",
    "paged_attention_ragged",
    "BatchPlan",
    "batch_hints",
    "NativePlanner",
    "plan_batch",
    "plan_batch_native",
    "plan_rows",
    "tiles_supported",
    "upload_batch_plan",
    "rms_norm",
    "rope_append",
    "silu_mul",
    "upload_plan",
]

#: Rows per MFMA tile (4 wavefronts x 16 queries).
TILE_ROWS = 64
#: A run of at least this many consecutive rows of one sequence is computed as MFMA tiles; the
#: row-streaming pass reads a sequence's keys once per row, the tile pass once per 64 rows.
MIN_TILE_ROWS = 8

_DTYPE_CODES = {torch.float32: _native.PKV_F32, torch.bfloat16: _native.PKV_BF16}


def kv_dtype_code(dtype: torch.dtype) -> int:
    """``pkv_dtype`` of a torch dtype (float32 or bfloat16)."""
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported KV dtype {dtype}; use float32 or bfloat16") from None


def _device_index(*tensors: torch.Tensor) -> int:
    device = tensors[0].device
    if device.type != "cuda":
        raise ValueError("the KV data path runs on a HIP device; got a tensor on " + str(device))
    for tensor in tensors[1:]:
        if tensor.device != device:
            raise ValueError("all tensors must be on the same device")
    return device.index if device.index is not None else torch.cuda.current_device()


def _stream(device: int) -> int:
    """The raw handle of ``device``'s current stream (torch's own accessor, without building a
    Stream object)."""
    return torch._C._cuda_getCurrentRawStream(device)


def _rows_contiguous(tensor: torch.Tensor, name: str) -> int:
    """Token stride (elements) of a [T, H, D] tensor whose [H, D] block is contiguous."""
    if tensor.dim() != 3:
        raise ValueError(f"{name} must have shape (tokens, heads, head_dim)")
    _, heads, dim = tensor.shape
    if tensor.stride(2) != 1 or (heads > 1 and tensor.stride(1) != dim):
        raise ValueError(f"{name}: each token's (heads, head_dim) block must be contiguous")
    return tensor.stride(0) if tensor.shape[0] > 1 else heads * dim


def append_kv(
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> None:
    """Write ``keys[t]`` / ``values[t]`` to token row ``slot_mapping[t]`` of one layer's pools.

    ``key_pool``/``value_pool``: contiguous ``[num_blocks, block_size, heads, head_dim]`` (or any
    contiguous shape whose trailing dims are ``heads, head_dim``), float32 or bfloat16.
    ``keys``/``values``: ``[T, heads, head_dim]`` float32 (or bfloat16 for a bfloat16 pool),
    token-strided views allowed. ``slot_mapping``: int64 ``[T]`` on the same device.
    Mirrors ``key_pool.reshape(-1, H, D)[slots] = keys`` (reference runner.py:195-196).
    """
    device = _device_index(key_pool, value_pool, keys, values, slot_mapping)
    if key_pool.shape != value_pool.shape or key_pool.dtype != value_pool.dtype:
        raise ValueError("key and value pools must have the same shape and dtype")
    if not (key_pool.is_contiguous() and value_pool.is_contiguous()):
        raise ValueError("pools must be contiguous")
    if keys.shape != values.shape or keys.dtype != values.dtype:
        raise ValueError("keys and values must have the same shape and dtype")
    heads, dim = keys.shape[1], keys.shape[2]
    if tuple(key_pool.shape[-2:]) != (heads, dim):
        raise ValueError("pool rows and keys disagree on (heads, head_dim)")
    key_stride = _rows_contiguous(keys, "keys")
    value_stride = _rows_contiguous(values, "values")
    if slot_mapping.dtype != torch.int64 or slot_mapping.shape != (keys.shape[0],):
        raise ValueError("slot_mapping must be int64 with one slot per token")
    pool_code = kv_dtype_code(key_pool.dtype)
    src_code = kv_dtype_code(keys.dtype)
    num_slots = key_pool.numel() // (heads * dim)
    rc = _native.library().pkv_append(
        key_pool.data_ptr(), value_pool.data_ptr(), pool_code, num_slots,
        keys.data_ptr(), values.data_ptr(), src_code, key_stride, value_stride,
        slot_mapping.data_ptr(), keys.shape[0], heads, dim,
        device, _stream(device),
    )  # fmt: skip
    _native.check(rc, "pkv_append")


def rope_append(
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    queries: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    positions: torch.Tensor,
    cos_table: torch.Tensor,
    sin_table: torch.Tensor,
    slot_mapping: torch.Tensor,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Rotate ``queries`` and ``keys`` by their positions and append the rotated keys and the
    ``values`` to one layer's pools, in one kernel; returns the rotated queries.

    Mirrors ``apply_rope`` on q and k (reference model.py:70-81, 251-252) followed by
    ``key_pool.reshape(-1, H, D)[slots] = k; value_pool...[slots] = v`` (runner.py:195-196), bit
    for bit in float32. ``queries``/``keys``/``values``: float32 ``[T, heads, head_dim]``,
    token-strided views allowed (the slices of a fused projection). ``positions``, ``slot_mapping``:
    int64 ``[T]``. ``cos_table``/``sin_table``: float32 ``[rows, head_dim / 2]``. ``out``: where
    to write the rotated queries (``[T, heads, head_dim]`` float32 with contiguous rows; may be
    ``queries`` itself); a new contiguous tensor when None.
    """
    device = _device_index(key_pool, value_pool, queries, keys, values, positions, cos_table, sin_table, slot_mapping)
    if key_pool.shape != value_pool.shape or key_pool.dtype != value_pool.dtype:
        raise ValueError("key and value pools must have the same shape and dtype")
    if not (key_pool.is_contiguous() and value_pool.is_contiguous()):
        raise ValueError("pools must be contiguous")
    if queries.dim() != 3 or queries.shape != keys.shape or keys.shape != values.shape:
        raise ValueError("queries, keys and values must all be [T, heads, head_dim]")
    if any(t.dtype != torch.float32 for t in (queries, keys, values, cos_table, sin_table)):
        raise ValueError("queries, keys, values and the rope tables must be float32")
    tokens, heads, dim = queries.shape
    if dim % 2:
        raise ValueError("head_dim must be even for rotary embeddings")
    if tuple(key_pool.shape[-2:]) != (heads, dim):
        raise ValueError("pool rows and keys disagree on (heads, head_dim)")
    if cos_table.shape != sin_table.shape or cos_table.dim() != 2 or cos_table.shape[1] != dim // 2:
        raise ValueError("rope tables must both be [rows, head_dim / 2]")
    if not (cos_table.is_contiguous() and sin_table.is_contiguous()):
        raise ValueError("rope tables must be contiguous")
    for name, index in (("positions", positions), ("slot_mapping", slot_mapping)):
        if index.dtype != torch.int64 or index.shape != (tokens,):
            raise ValueError(f"{name} must be int64 with one entry per token")
    q_stride = _rows_contiguous(queries, "queries")
    k_stride = _rows_contiguous(keys, "keys")
    v_stride = _rows_contiguous(values, "values")
    if out is None:
        out = torch.empty((tokens, heads, dim), dtype=torch.float32, device=queries.device)
    elif out.shape != queries.shape or out.dtype != torch.float32 or out.device != queries.device:
        raise ValueError("out must be float32 [T, heads, head_dim] on the queries' device")
    out_stride = _rows_contiguous(out, "out")
    if tokens == 0:
        return out
    num_slots = key_pool.numel() // (heads * dim)
    rc = _native.library().pkv_rope_append(
        out.data_ptr(), out_stride, queries.data_ptr(), keys.data_ptr(), values.data_ptr(),
        q_stride, k_stride, v_stride, positions.data_ptr(), cos_table.data_ptr(),
        sin_table.data_ptr(), cos_table.shape[0], key_pool.data_ptr(), value_pool.data_ptr(),
        kv_dtype_code(key_pool.dtype), num_slots, slot_mapping.data_ptr(), tokens, heads, dim,
        device, _stream(device),
    )  # fmt: skip
    _native.check(rc, "pkv_rope_append")
    return out


def _rows_2d(tensor: torch.Tensor, name: str, width: int) -> int:
    """Row stride (elements) of a float32 ``[rows, >= width]`` tensor with contiguous rows."""
    if tensor.dim() != 2 or tensor.dtype != torch.float32 or tensor.shape[1] < width:
        raise ValueError(f"{name} must be float32 [rows, {width}]")
    if tensor.stride(1) != 1:
        raise ValueError(f"{name} rows must be contiguous")
    return tensor.stride(0) if tensor.shape[0] > 1 else tensor.shape[1]


def rms_norm(
    hidden: torch.Tensor, weight: torch.Tensor, eps: float, *, delta: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:  # fmt: skip
    """``hidden / sqrt(mean(hidden ** 2) + eps) * weight`` over the last axis of float32
    ``hidden [rows, dim]`` (reference model.py:43-46). With ``delta``, ``hidden += delta`` first,
    in place (the residual add before the norm, model.py:256-264). ``out`` may be ``hidden``."""
    device = _device_index(hidden, weight)
    rows, dim = hidden.shape if hidden.dim() == 2 else (-1, -1)
    h_stride = _rows_2d(hidden, "hidden", dim)
    if weight.shape != (dim,) or weight.dtype != torch.float32 or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous float32 [dim] tensor")
    d_stride = 0
    if delta is not None:
        if delta.shape != hidden.shape or delta.device != hidden.device:
            raise ValueError("delta must match hidden")
        d_stride = _rows_2d(delta, "delta", dim)
    if out is None:
        out = torch.empty((rows, dim), dtype=torch.float32, device=hidden.device)
    elif out.shape != hidden.shape or out.device != hidden.device:
        raise ValueError("out must match hidden")
    o_stride = _rows_2d(out, "out", dim)
    rc = _native.library().pkv_rms_norm(
        out.data_ptr(), o_stride, hidden.data_ptr(), h_stride, None if delta is None else delta.data_ptr(),
        d_stride, weight.data_ptr(), rows, dim, float(eps), device, _stream(device),
    )  # fmt: skip
    _native.check(rc, "pkv_rms_norm")
    return out


def silu_mul(gate_up: torch.Tensor, width: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(gate) * up`` for float32 ``gate_up [rows, 2 * width]`` holding ``[gate | up]`` (one
    product with the concatenated weights), as float32 ``[rows, width]`` (reference
    model.py:49-51 and 256-259)."""
    device = _device_index(gate_up)
    if width < 1 or gate_up.dim() != 2 or gate_up.shape[1] != 2 * width:
        raise ValueError("gate_up must be [rows, 2 * width]")
    stride = _rows_2d(gate_up, "gate_up", 2 * width)
    rows = gate_up.shape[0]
    if out is None:
        out = torch.empty((rows, width), dtype=torch.float32, device=gate_up.device)
    elif out.shape != (rows, width) or out.device != gate_up.device:
        raise ValueError("out must be [rows, width] on gate_up's device")
    o_stride = _rows_2d(out, "out", width)
    rc = _native.library().pkv_silu_mul(
        out.data_ptr(), o_stride, gate_up.data_ptr(), gate_up.data_ptr() + 4 * width, stride, rows, width,
        device, _stream(device),
    )  # fmt: skip
    _native.check(rc, "pkv_silu_mul")
    return out


def greedy_tokens(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Argmax of each row of float32 ``logits [rows, vocab]`` as int32 ``[rows]``, on the device.

    Mirrors ``int(np.argmax(row))`` (reference sampling.py:28-30) row by row: ties go to the
    lowest id, the first NaN wins.
    """
    device = _device_index(logits)
    if logits.dim() != 2 or logits.dtype != torch.float32:
        raise ValueError("logits must be float32 of shape (rows, vocab)")
    rows, vocab = logits.shape
    if vocab < 1:
        raise ValueError("logits need at least one column")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    if out is None:
        out = torch.empty(rows, dtype=torch.int32, device=logits.device)
    elif out.shape != (rows,) or out.dtype != torch.int32 or not out.is_contiguous():
        raise ValueError("out must be a contiguous int32 tensor with one entry per row")
    if rows == 0:
        return out
    stride = logits.stride(0) if rows > 1 else vocab
    rc = _native.library().pkv_greedy_tokens(
        out.data_ptr(), logits.data_ptr(), stride, rows, vocab, device, _stream(device)
    )
    _native.check(rc, "pkv_greedy_tokens")
    return out


def copy_blocks(key_pool: torch.Tensor, value_pool: torch.Tensor, pairs: torch.Tensor) -> None:
    """Copy block ``src`` over block ``dst`` in every layer for each row ``(src, dst)`` of pairs.

    ``key_pool``/``value_pool``: contiguous ``[layers, num_blocks, ...]``. ``pairs``: int64
    ``[n, 2]`` on the device. The pairs must be independent (no repeated dst, no dst that is also
    a src); :func:`independent_groups` splits an ordered list into such groups.
    Mirrors ``K[:, dst] = K[:, src]; V[:, dst] = V[:, src]`` (reference runner.py:132-133).
    """
    device = _device_index(key_pool, value_pool, pairs)
    if key_pool.shape != value_pool.shape or key_pool.dtype != value_pool.dtype:
        raise ValueError("key and value pools must have the same shape and dtype")
    if not (key_pool.is_contiguous() and value_pool.is_contiguous()):
        raise ValueError("pools must be contiguous")
    if pairs.dtype != torch.int64 or pairs.dim() != 2 or pairs.shape[1] != 2:
        raise ValueError("pairs must be int64 of shape (n, 2)")
    pairs = pairs.contiguous()
    layers, num_blocks = key_pool.shape[0], key_pool.shape[1]
    block_elems = key_pool[0, 0].numel()
    rc = _native.library().pkv_copy_blocks(
        key_pool.data_ptr(), value_pool.data_ptr(), kv_dtype_code(key_pool.dtype),
        pairs.data_ptr(), pairs.shape[0], layers, num_blocks, block_elems,
        device, _stream(device),
    )  # fmt: skip
    _native.check(rc, "pkv_copy_blocks")


def independent_groups(pairs: list[tuple[int, int]]) -> list[list[tuple[int, int]]]:
    """Split an ordered list of block copies into groups that may each run concurrently.

    Applying the groups one after another gives the same pool as applying the copies one at a
    time in list order: a copy starts a new group when it reads a block an earlier copy of the
    group writes, or writes a block an earlier copy of the group reads or writes.
    """
    if not pairs:
        return []
    # The common case -- every destination distinct and none of them also a source (a batch of
    # forks copying shared blocks into fresh ones) -- is one group.
    destinations = {dst for _, dst in pairs}
    if len(destinations) == len(pairs) and destinations.isdisjoint(src for src, _ in pairs):
        return [list(pairs)]
    groups: list[list[tuple[int, int]]] = []
    reads: set[int] = set()
    writes: set[int] = set()
    for src, dst in pairs:
        if not groups or src in writes or dst in reads or dst in writes:
            groups.append([])
            reads, writes = set(), set()
        groups[-1].append((src, dst))
        reads.add(src)
        writes.add(dst)
    return groups


@dataclass(frozen=True)
class AttentionPlan:
    """Which (query row, partition) goes to which attention pass, as int32 device tensors, plus
    the launch hints.

    ``rows``: ``[R, 2]`` = (query row, partition) work items of the row-streaming pass
    (:func:`expand_rows` makes them from each row's first partition). ``tiles``:
    ``[n, 4]`` = (first row, row count, first partition, end partition; end <= first: through
    the last; ``TILE_WHOLE``: one workgroup per head over every visible key) for the MFMA tile
    pass: a run of consecutive rows of one sequence, or decode rows of several sequences over
    the partitions of a prefix whose blocks they share. Every (row, partition) is covered
    exactly once. ``merge``: int32 ``[M]``, the rows whose partition results the reduce pass
    merges (None: every row, which is only correct without whole tiles). ``partition_size``
    (0: library default), ``shared_kv``, ``short_rows`` (the lighter row-pass workgroup for
    short items) and ``dominant_tiles`` (three tile-pass workgroups per CU beside the rows)
    choose the launch.
    """

    rows: torch.Tensor
    tiles: torch.Tensor
    partition_size: int = 0
    shared_kv: bool = False
    merge: torch.Tensor | None = None
    short_rows: bool = False
    dominant_tiles: bool = False

    @property
    def num_rows(self) -> int:
        return int(self.rows.shape[0])

    @property
    def num_tiles(self) -> int:
        return int(self.tiles.shape[0])


def tiles_supported(head_dim: int) -> bool:
    """Whether the MFMA tile pass exists for this head_dim."""
    return bool(_native.library().pkv_tile_head_dim_supported(head_dim))


def plan_rows(
    query_seq: np.ndarray, head_dim: int, *, min_tile_rows: int = MIN_TILE_ROWS
) -> tuple[np.ndarray, np.ndarray]:
    """Split a ragged batch's rows between the two attention passes (host, int32).

    Runs of at least ``min_tile_rows`` consecutive rows with the same sequence index become
    tiles of at most ``TILE_ROWS`` rows over all partitions (when the head_dim has a tile
    kernel); every other row goes to the row-streaming pass from partition 0. Returns
    ``(rows [R, 2], tiles [n, 4])``.
    """
    seq = np.asarray(query_seq, dtype=np.int64)
    total = seq.size
    if total == 0:
        return np.zeros((0, 2), np.int32), np.zeros((0, 4), np.int32)
    tiled = tiles_supported(head_dim)
    starts = np.flatnonzero(np.concatenate([[True], seq[1:] != seq[:-1]]))
    ends = np.concatenate([starts[1:], [total]])
    rows, tiles = [], []
    for start, end in zip(starts.tolist(), ends.tolist()):
        if tiled and end - start >= min_tile_rows:
            for first in range(start, end, TILE_ROWS):
                tiles.append((first, min(TILE_ROWS, end - first), 0, 0))
        else:
            rows.extend(range(start, end))
    row_array = np.zeros((len(rows), 2), dtype=np.int32)
    row_array[:, 0] = rows
    return row_array, np.asarray(tiles, dtype=np.int32).reshape(-1, 4)


#: Partition work items (row x head x partition) above which 1024-key partitions pay off: fewer,
#: longer workgroups amortise their set-up and the reduce, while the grid still fills the GPU.
WIDE_PARTITION_ITEMS = 8192
#: Fraction of a batch's used table entries that repeat across sequences above which the K/V
#: rows are loaded through the caches (PKV_ATTN_SHARED_KV) rather than streamed past them.
SHARED_KV_FRACTION = 0.25
#: Row-pass rows of different sequences whose tables share at least this many leading tokens'
#: blocks, at least MIN_SHARED_ROWS of them in a row, compute that prefix as MFMA tiles.
MIN_SHARED_TOKENS = 512
MIN_SHARED_ROWS = 16
#: Shared-prefix tile workgroups the partition choice aims for (two per CU of 256), and the
#: smallest partition it will choose for them.
TARGET_PREFIX_GROUPS = 512
MIN_PREFIX_PARTITION = 256
#: Prefill tiles are computed whole (one workgroup per tile and head over every visible key,
#: final rows written directly, nothing for the reduce) once the call has at least this many
#: (tile, head) workgroups: four per CU of 256 keeps the chip full without splitting contexts.
WHOLE_TILE_GROUPS = 1024
#: Tile record end partition of a whole tile (include/pkv.h PKV_TILE_WHOLE).
TILE_WHOLE = -1
#: Row-pass items shorter than this many keys on average launch the lighter row-pass workgroup
#: (PKV_ATTN_SHORT_ROWS): with half the bytes in flight per wavefront, twice as many fit on a CU.
SHORT_ROW_KEYS = 256


def _wide_partition(contexts: np.ndarray, num_heads: int, rows_per_seq: int) -> int:
    wide = int(np.sum(-(-contexts // 1024))) * rows_per_seq * num_heads
    return 1024 if wide >= WIDE_PARTITION_ITEMS else 512


def _repeated_fraction_reached(ids: np.ndarray) -> bool:
    if ids.size == 0:
        return False
    low, high = int(ids.min()), int(ids.max())
    if 0 <= low and high < (1 << 26):  # block ids: a histogram is cheaper than a sort
        distinct = int(np.count_nonzero(np.bincount(ids, minlength=0)))
    else:
        distinct = int(np.unique(ids).size)
    return ids.size - distinct >= SHARED_KV_FRACTION * ids.size


def batch_hints(
    tables: list | None, context_lens: np.ndarray, num_heads: int, block_size: int,
    num_rows: int | None = None, *, used_ids: np.ndarray | None = None,
) -> tuple[int, bool]:  # fmt: skip
    """``(partition_size, shared_kv)`` for a batch, from its host block tables and contexts.

    ``used_ids`` (every sequence's first ``ceil(context / block_size)`` table entries,
    concatenated) may be passed instead of ``tables``.

    Partition size: 1024 when ``rows x heads x ceil(context / 1024)`` reaches
    ``WIDE_PARTITION_ITEMS``, else 512 (measured on MI355X: long contexts and large batches gain
    3-10% from the wider partitions; 64 x 4k decode is flat). ``shared_kv`` is set when at least
    ``SHARED_KV_FRACTION`` of the used block ids appear in more than one sequence's table (a
    shared prefix), which makes cached loads 1.8x faster than streaming on the 256-sequence
    prefix-sharing workload.
    """
    contexts = np.asarray(context_lens, dtype=np.int64)
    if contexts.size == 0:
        return 0, False
    per_seq_rows = 1 if num_rows is None else max(1, num_rows // contexts.size)
    partition = _wide_partition(contexts, num_heads, per_seq_rows)
    if used_ids is None:
        used = [np.asarray(t[: -(-int(c) // block_size)]) for t, c in zip(tables, contexts)]
        used_ids = np.concatenate(used) if used else np.zeros(0, np.int64)
    return partition, _repeated_fraction_reached(np.asarray(used_ids))


@dataclass(frozen=True)
class BatchPlan:
    """A host plan: ``rows [R, 2]``, ``tiles [n, 4]`` and ``merge [M]`` (int32, the
    :class:`AttentionPlan` layout), the partition size and the launch hints."""

    rows: np.ndarray
    tiles: np.ndarray
    partition_size: int
    shared_kv: bool
    merge: np.ndarray | None = None
    short_rows: bool = False
    dominant_tiles: bool = False


def _padded_tables(tables, sid: np.ndarray, used: np.ndarray, width: int) -> np.ndarray:
    """``[len(sid), width]`` int64 matrix of the used table entries of sequences ``sid``, -1 past
    each one's used length. A 2-D table array (the runner's arena) is gathered in one step."""
    if isinstance(tables, np.ndarray) and tables.ndim == 2 and tables.shape[1] >= width:
        out = tables[sid, :width].astype(np.int64)
    else:
        out = np.full((sid.size, width), -1, dtype=np.int64)
        for r, (s, n) in enumerate(zip(sid.tolist(), used.tolist())):
            out[r, :n] = np.asarray(tables[s][:n])
    out[np.arange(width)[None, :] >= used[:, None]] = -1
    return out


def _prefix_groups(
    rows: np.ndarray, seq: np.ndarray, tables, used_blocks: np.ndarray, min_blocks: int,
    padded: tuple | None = None,
) -> list:
    """Runs of consecutive row-pass rows whose sequences' used tables agree over a common
    prefix of at least ``min_blocks`` blocks. Returns
    ``[(first index into rows, row count, common blocks)]``; a member whose whole used table is
    a prefix of the first row's constrains nothing (its visible keys end inside the prefix).

    Vectorised: one comparison of every row with the one before finds where a run can start;
    from each such start the rows that follow are compared with it a chunk at a time until one
    fails, so a batch without sharing costs one pass over its tables. ``padded`` (sorted
    sequence ids, their :func:`_padded_tables` matrix) reuses tables the caller already padded."""
    count = rows.shape[0]
    if count < MIN_SHARED_ROWS:
        return []
    qrow = np.asarray(rows[:, 0], dtype=np.int64)
    sid = np.asarray(seq, dtype=np.int64)[qrow]
    used = np.asarray(used_blocks, dtype=np.int64)[sid]
    width = int(used.max())
    if width < min_blocks:
        return []
    if padded is None:
        table = _padded_tables(tables, sid, used, width)
    else:
        table = padded[1][np.searchsorted(padded[0], sid), :width]
    col = np.arange(width)
    consecutive = qrow[1:] == qrow[:-1] + 1  # row k + 1 continues row k
    both = np.minimum(used[1:], used[:-1])
    same = (table[1:] == table[:-1]) & (col[None, :] < both[:, None])
    lead_prev = np.where(same.all(axis=1), both, same.argmin(axis=1))
    # A run can start at k only if row k + 1 joins it: it shares enough, or its whole table is
    # a prefix of row k's.
    starts = np.flatnonzero(consecutive & ((lead_prev >= min_blocks) | (lead_prev == used[1:])))
    stops = np.flatnonzero(~consecutive)  # row k + 1 does not continue row k
    groups = []
    free = 0  # rows before this index already belong to a group
    chunk = 32
    for k in starts.tolist():
        if k < free:
            continue
        after = stops[np.searchsorted(stops, k)] + 1 if stops.size and stops[-1] >= k else count
        first = table[k]
        common = int(used[k])
        joined = 0
        for lo in range(k + 1, after, chunk):
            hi = min(lo + chunk, after)
            eq = (table[lo:hi] == first) & (col[None, :] < used[k])
            lead = np.where(eq.all(axis=1), width, eq.argmin(axis=1))
            limit = np.where(lead >= used[lo:hi], common, lead)  # a whole-prefix member: no limit
            running = np.minimum.accumulate(np.minimum(limit, common))
            bad = np.flatnonzero(running < min_blocks)
            take = int(bad[0]) if bad.size else hi - lo
            if take:
                common = int(running[take - 1])
            joined += take
            if bad.size:
                break
        if joined + 1 >= MIN_SHARED_ROWS and common >= min_blocks:
            groups.append((k, joined + 1, common))
            free = k + joined + 1
    return groups


def _prefix_partition(shared_tokens: int, tiles: int, num_heads: int) -> int:
    """Partition size for a shared prefix: whole partitions should cover the prefix (at most
    1024 keys each) and give the tile pass about TARGET_PREFIX_GROUPS workgroups."""
    best = 0
    k = max(1, -(-shared_tokens // 1024))
    while True:
        size = min(1024, (shared_tokens // k) // 16 * 16)
        if size < MIN_PREFIX_PARTITION:
            break
        best = size
        if tiles * num_heads * k >= TARGET_PREFIX_GROUPS:
            break
        k += 1
    return best


def _visible(seq: np.ndarray, contexts: np.ndarray, positions: np.ndarray | None) -> np.ndarray:
    """Visible key count of every query row, min(context, position + 1) (the context when the
    positions are not known: an upper bound)."""
    ctx = contexts[seq]
    if positions is None:
        return ctx
    pos = np.asarray(positions, dtype=np.int64)
    return np.where(pos < 0, 0, np.minimum(ctx, pos + 1))


def _whole_tiles(
    tiles: np.ndarray, seq: np.ndarray, visible: np.ndarray, num_heads: int, has_rows: bool = True
) -> np.ndarray:
    """Prefill tiles as whole tiles when there are enough of them to fill the GPU.

    Order beside row-pass rows (``has_rows``; the tile pass then runs as one persistent
    workgroup per CU, each taking every 256th item): the tiles of one chunk (a run of one
    sequence's rows) stay together, longest chunk first; an even-ranked chunk's tiles run from
    its last rows' tile to its first rows', an odd-ranked chunk's the other way. The tile pass
    hands its (tile, head) items out heads fastest, so with a multiple of 8 heads one head's
    tiles of a chunk run side by side on one XCD and share its L2 reads of that chunk's keys;
    with the causal mask a chunk's later tiles are its longer ones, so each persistent workgroup
    alternates long and short tiles, and the workgroups of a head reach every second chunk
    together. Measured on the mixed 8 x 512 prefill + 120 decode batch: 1.47-1.48 ms, against
    1.49-1.52 ms with each chunk's tiles rotated by its rank, 1.51-1.54 ms in row order and
    1.65 ms longest tile first.

    Without row-pass rows the tile pass runs one workgroup per item, started in item order as
    others finish, and the longest tile comes first (stable): the grid then ends on its
    shortest workgroups. Measured on the same 8 chunks alone: 0.614 ms, against 0.66-0.69 ms
    in the chunk order above.
    """
    if tiles.shape[0] == 0 or tiles.shape[0] * num_heads < WHOLE_TILE_GROUPS:
        return tiles
    first, count = tiles[:, 0].astype(np.int64), tiles[:, 1].astype(np.int64)
    longest = np.fromiter(
        (visible[f : f + c].max() for f, c in zip(first.tolist(), count.tolist())),
        dtype=np.int64, count=tiles.shape[0],
    )  # fmt: skip
    if not has_rows:
        whole = tiles[np.argsort(-longest, kind="stable")].copy()
        whole[:, 2] = 0
        whole[:, 3] = TILE_WHOLE
        return whole
    # a chunk starts where a tile does not continue the previous tile's rows of one sequence
    new_chunk = np.ones(tiles.shape[0], dtype=bool)
    new_chunk[1:] = (first[1:] != first[:-1] + count[:-1]) | (seq[first[1:]] != seq[first[:-1]])
    starts = np.flatnonzero(new_chunk)
    ends = np.append(starts[1:], tiles.shape[0])
    chunk_longest = np.maximum.reduceat(longest, starts)
    order = []
    for rank, c in enumerate(np.argsort(-chunk_longest, kind="stable").tolist()):
        members = np.arange(starts[c], ends[c])
        order.append(members[::-1] if rank % 2 == 0 else members)
    whole = tiles[np.concatenate(order)].copy()
    whole[:, 2] = 0
    whole[:, 3] = TILE_WHOLE
    return whole


def expand_rows(rows: np.ndarray, visible: np.ndarray, partition_size: int) -> np.ndarray:
    """Row-pass work items ``[W, 2]`` = (query row, partition) from ``rows [R, 2]`` = (query
    row, first partition): partitions first .. ceil(visible / partition_size) - 1 of each row
    (at least its first). Full partitions come first in row order, then every row's shorter last
    partition, longest first, so the grid ends on its shortest workgroups. ``partition_size`` 0
    is the library default (512). ``visible`` may overstate a row (the kernel skips partitions
    past the row's visible length), never understate it."""
    rows = np.asarray(rows, dtype=np.int64).reshape(-1, 2)
    if rows.shape[0] == 0:
        return np.zeros((0, 2), np.int32)
    part = partition_size or 512
    vis = np.asarray(visible, dtype=np.int64)[rows[:, 0]]
    nparts = np.maximum(1, -(-vis // part))
    first = rows[:, 1]
    count = np.maximum(nparts - first, 0)  # a row whose keys all lie in a prefix tile has none
    row_of = np.repeat(rows[:, 0], count)
    offsets = np.arange(count.sum()) - np.repeat(np.cumsum(count) - count, count)
    p_of = np.repeat(first, count) + offsets
    keys = np.minimum(part, np.repeat(vis, count) - p_of * part)  # keys in each item
    order = np.lexsort((np.arange(keys.size), -keys))  # longest first, stable
    return np.stack([row_of[order], p_of[order]], axis=1).astype(np.int32)


def merge_rows_for(
    num_queries: int, tiles: np.ndarray, visible: np.ndarray | None = None, partition_size: int = 0
) -> np.ndarray:
    """The rows the reduce pass merges: every row no whole tile covers, and of those only the
    ones whose visible length spans more than one partition when ``visible`` is known."""
    keep = np.ones(num_queries, dtype=bool)
    for first, count, _, end in np.asarray(tiles, dtype=np.int64).reshape(-1, 4).tolist():
        if end == TILE_WHOLE:
            keep[first : first + count] = False
    if visible is not None and partition_size > 0:
        keep &= np.asarray(visible) > partition_size
    return np.flatnonzero(keep).astype(np.int32)


def plan_batch(
    query_seq: np.ndarray, head_dim: int, num_heads: int, tables, context_lens: np.ndarray,
    block_size: int, *, partition_size: int = 0, min_tile_rows: int = MIN_TILE_ROWS,
    query_positions: np.ndarray | None = None, kv_dtype: torch.dtype = torch.float32,
) -> BatchPlan:  # fmt: skip
    """The full host plan of a ragged call: the row/tile split of :func:`plan_rows`, shared-prefix
    tiles, whole prefill tiles, the reduce's merge list, the partition size and the load hint.

    ``tables[s]`` / ``context_lens[s]``: block table (any int sequence) and context length of
    the sequence index ``s`` used in ``query_seq``. Row-pass rows of consecutive queries whose
    sequences share at least MIN_SHARED_TOKENS of leading blocks, MIN_SHARED_ROWS or more of
    them, read that prefix once per head as MFMA tiles over its whole partitions, and start the
    row pass at the first partition after it. Prefill tiles become whole tiles when there are at
    least WHOLE_TILE_GROUPS (tile, head) pairs. ``query_positions`` (optional) narrows the merge
    list to rows that span several partitions. A nonzero ``partition_size`` is kept as given.
    Shared-prefix groups and the load hint are only searched for when two row-pass sequences
    start with the same block; tables that repeat ids only past their first block get the
    streaming hint (the hint chooses a load path, never a result). ``kv_dtype`` (the pools'
    element type) weighs the row pass's bytes against the tile pass's products for the
    ``dominant_tiles`` hint (:func:`_dominant_tiles`).
    """
    seq = np.asarray(query_seq, dtype=np.int64)
    contexts = np.asarray(context_lens, dtype=np.int64)
    rows, tiles = plan_rows(seq, head_dim, min_tile_rows=min_tile_rows)
    if seq.size == 0:
        return BatchPlan(rows, tiles, partition_size or 0, False, np.zeros(0, np.int32))
    visible = _visible(seq, contexts, query_positions)
    tiles = _whole_tiles(tiles, seq, visible, num_heads, rows.size > 0)
    used_blocks = -(-contexts // block_size)
    # Prefix sharing gives sequences the same first block (a shared block's whole prefix is
    # shared), so when the row pass's sequences all start in different blocks there is neither a
    # shared-prefix group nor a repeated block to look for: the common decode step skips both.
    row_seqs = np.unique(seq[rows[:, 0]]) if rows.size else np.zeros(0, np.int64)
    starting = row_seqs[used_blocks[row_seqs] > 0]
    if starting.size == 0:
        first_blocks = np.zeros(0, np.int64)
    elif isinstance(tables, np.ndarray) and tables.ndim == 2:
        first_blocks = tables[starting, 0]
    else:
        first_blocks = np.fromiter((tables[s][0] for s in starting.tolist()), dtype=np.int64,
                                   count=starting.size)  # fmt: skip
    may_share = np.unique(first_blocks).size < first_blocks.size
    padded = None  # the row pass's sequences' used tables, padded once for both searches below
    if may_share:
        held = used_blocks[row_seqs]
        padded = (row_seqs, _padded_tables(tables, row_seqs, held, int(held.max())))
    groups = []
    if may_share and rows.shape[0] >= MIN_SHARED_ROWS and tiles_supported(head_dim):
        groups = _prefix_groups(rows, seq, tables, used_blocks, -(-MIN_SHARED_TOKENS // block_size),
                                padded)  # fmt: skip
    present = np.unique(seq)
    partition = partition_size
    if partition == 0:
        if groups:
            largest = max(groups, key=lambda g: g[1] * g[2])
            tile_count = sum(-(-g[1] // TILE_ROWS) for g in groups)
            partition = _prefix_partition(largest[2] * block_size, tile_count, num_heads)
        if partition == 0:
            partition = _wide_partition(contexts[present], num_heads, max(1, seq.size // present.size))
    prefix_tiles = []
    for start, count, common in groups:
        parts = common * block_size // partition
        if parts < 1:
            continue
        # A tile reads its keys through its first row's table, so every 64-row tile must start at
        # a row whose table covers the parts * partition prefix keys. A member whose whole table
        # ends inside the prefix may sit inside a tile, never at its start: the group ends before
        # such a row, and the rows from there on stay in the row pass from partition 0.
        need = -(-parts * partition // block_size)
        for offset in range(TILE_ROWS, count, TILE_ROWS):
            if used_blocks[seq[rows[start + offset, 0]]] < need:
                count = offset
                break
        rows[start : start + count, 1] = parts
        first_row = int(rows[start, 0])
        for offset in range(0, count, TILE_ROWS):
            prefix_tiles.append((first_row + offset, min(TILE_ROWS, count - offset), 0, parts))
    if prefix_tiles:
        tiles = np.concatenate([tiles, np.asarray(prefix_tiles, dtype=np.int32)])
    # The load hint looks at what the row pass still reads: each row-pass sequence's blocks from
    # its first partition on (tiles read their keys once per 64 rows either way).
    ids = np.zeros(0, np.int64)
    if rows.size and may_share:
        firsts = rows[:, 1].astype(np.int64) * partition // block_size
        span = int(firsts.max()) + 1
        pair = np.unique(seq[rows[:, 0]] * span + firsts)  # distinct (sequence, first block)
        pair_seq, pair_first = pair // span, pair % span
        reads = used_blocks[pair_seq]
        table = padded[1][np.searchsorted(padded[0], pair_seq)]
        col = np.arange(table.shape[1])[None, :]
        ids = table[(col >= pair_first[:, None]) & (col < reads[:, None])]
    merge = merge_rows_for(seq.size, tiles, visible, int(partition))
    items = expand_rows(rows, visible, int(partition))
    short = dominant = False
    if items.shape[0]:
        keys = np.maximum(np.minimum(partition, visible[items[:, 0]] - items[:, 1].astype(np.int64) * partition), 0)
        short = bool(np.mean(keys) < SHORT_ROW_KEYS)
        dominant = _dominant_tiles(tiles, visible, int(partition), int(keys.sum()), kv_dtype_size(kv_dtype))
    return BatchPlan(items, tiles, int(partition), _repeated_fraction_reached(ids), merge, short, dominant)


#: The dominant-tiles hint: a call with both passes sets it when the tile pass's estimated time
#: is at least 1.1 times the row pass's. A tile key costs 4 * head_dim products at about
#: 100 TFLOP/s, a row key 2 * head_dim * element-size bytes at about 6.8 TB/s, so the test is
#: tile_keys * DOMINANT_TILE_WEIGHT >= row_keys * element_size * DOMINANT_ROW_WEIGHT. Measured
#: crossover on MI355X: config 3's chunks beside 30-240 decode rows, float32 and bfloat16.
DOMINANT_TILE_WEIGHT = 34
DOMINANT_ROW_WEIGHT = 275


def kv_dtype_size(dtype: torch.dtype) -> int:
    """Bytes per element of a KV pool dtype (float32 or bfloat16)."""
    kv_dtype_code(dtype)  # validates
    return 2 if dtype == torch.bfloat16 else 4


def _dominant_tiles(tiles: np.ndarray, visible: np.ndarray, partition: int, row_keys: int, esize: int) -> bool:
    """Whether the tile pass dominates a call whose row pass reads ``row_keys`` keys per head:
    a whole tile reads every visible key of its rows, a partitioned one the keys in its
    partitions."""
    if tiles.shape[0] == 0 or row_keys == 0:
        return False
    tile_keys = 0
    for first, count, begin, end in tiles.tolist():
        v = visible[first : first + count]
        lo = 0 if end == TILE_WHOLE else begin * partition
        hi = v if end == TILE_WHOLE or end <= begin else np.minimum(v, end * partition)
        tile_keys += int(np.maximum(hi - lo, 0).sum())
    return tile_keys * DOMINANT_TILE_WEIGHT >= row_keys * esize * DOMINANT_ROW_WEIGHT


class NativePlanner:
    """:func:`plan_batch` computed by the library's host planner (``pkv_plan_batch``), with
    output buffers kept between calls. The same plan, bit for bit (tests/test_host_plan_native.py),
    at a few microseconds per decode batch instead of a hundred. One instance per caller: the
    buffers are reused."""

    def __init__(self) -> None:
        self._rows = np.zeros((4096, 2), np.int32)
        self._tiles = np.zeros((256, 4), np.int32)
        self._merge = np.zeros(1024, np.int32)
        self._counts = np.zeros(3, np.int64)
        self._launch = np.zeros(2, np.int32)
        self._host = None

    def plan_views(
        self, query_seq: np.ndarray, query_positions: np.ndarray | None, tables: np.ndarray,
        context_lens: np.ndarray, block_size: int, num_heads: int, head_dim: int, partition_size: int = 0,
        min_tile_rows: int = MIN_TILE_ROWS, kv_dtype: torch.dtype = torch.float32,
    ) -> tuple[np.ndarray, np.ndarray, np.ndarray, int, int]:  # fmt: skip
        """:meth:`plan` for callers that hand over int32 C-contiguous arrays (``tables`` 2-D) and
        use the result at once: ``(rows [R, 2], tiles [n, 4], merge [M], partition size, flags)``,
        where the arrays are views of this planner's buffers, valid until its next call. The
        library is reached through ``_pkvhost.plan`` rather than ctypes."""
        host = self._host
        if host is None:
            host = self._host = _native.bound_host()
        while True:
            rc = host.plan(query_seq, query_positions, tables, context_lens, block_size, num_heads, head_dim,
                           kv_dtype_code(kv_dtype), partition_size, min_tile_rows, self._rows, self._tiles,
                           self._merge, self._counts, self._launch)  # fmt: skip
            if rc != _native.PKV_ETOOBIG:
                break
            rows, tiles, merge = (int(c) for c in self._counts)
            self._rows = np.zeros((max(rows, 2 * self._rows.shape[0]), 2), np.int32)
            self._tiles = np.zeros((max(tiles, 2 * self._tiles.shape[0]), 4), np.int32)
            self._merge = np.zeros(max(merge, 2 * self._merge.size), np.int32)
        _native.check(rc, "pkv_plan_batch")
        rows, tiles, merge = self._counts.tolist()
        partition, flags = self._launch.tolist()
        return self._rows[:rows], self._tiles[:tiles], self._merge[:merge], partition, flags

    def plan(
        self, query_seq: np.ndarray, head_dim: int, num_heads: int, tables: np.ndarray,
        context_lens: np.ndarray, block_size: int, *, partition_size: int = 0,
        min_tile_rows: int = MIN_TILE_ROWS, query_positions: np.ndarray | None = None,
        kv_dtype: torch.dtype = torch.float32,
    ) -> BatchPlan:  # fmt: skip
        """Arguments as :func:`plan_batch`, except that ``tables`` is a 2-D int32 array (one
        padded row per sequence index, as the runner's block-table arena holds them)."""
        seq = np.ascontiguousarray(query_seq, dtype=np.int32)
        table = np.ascontiguousarray(tables, dtype=np.int32)
        if table.ndim != 2:
            raise ValueError("tables must be a 2-D int32 array")
        contexts = np.ascontiguousarray(context_lens, dtype=np.int32)
        positions = None if query_positions is None else np.ascontiguousarray(query_positions, dtype=np.int32)
        lib = _native.library()
        while True:
            rc = lib.pkv_plan_batch(
                seq.ctypes.data, None if positions is None else positions.ctypes.data, seq.size,
                table.ctypes.data, table.shape[1], contexts.ctypes.data, contexts.size,
                block_size, num_heads, head_dim, kv_dtype_code(kv_dtype), partition_size, min_tile_rows,
                self._rows.ctypes.data, self._rows.shape[0], self._tiles.ctypes.data, self._tiles.shape[0],
                self._merge.ctypes.data, self._merge.size, self._counts.ctypes.data, self._launch.ctypes.data,
            )  # fmt: skip
            if rc != _native.PKV_ETOOBIG:
                break
            rows, tiles, merge = (int(c) for c in self._counts)
            self._rows = np.zeros((max(rows, 2 * self._rows.shape[0]), 2), np.int32)
            self._tiles = np.zeros((max(tiles, 2 * self._tiles.shape[0]), 4), np.int32)
            self._merge = np.zeros(max(merge, 2 * self._merge.size), np.int32)
        _native.check(rc, "pkv_plan_batch")
        rows, tiles, merge = (int(c) for c in self._counts)
        partition, flags = (int(v) for v in self._launch)
        return BatchPlan(
            self._rows[:rows].copy(), self._tiles[:tiles].copy(), partition,
            bool(flags & _native.PKV_ATTN_SHARED_KV), self._merge[:merge].copy(),
            bool(flags & _native.PKV_ATTN_SHORT_ROWS), bool(flags & _native.PKV_ATTN_DOMINANT_TILES),
        )  # fmt: skip


def plan_batch_native(query_seq, head_dim, num_heads, tables, context_lens, block_size, **kwargs) -> BatchPlan:
    """:meth:`NativePlanner.plan` with a fresh planner; ``tables`` may also be a list of
    per-sequence tables (padded here)."""
    if not (isinstance(tables, np.ndarray) and tables.ndim == 2):
        width = max((len(t) for t in tables), default=0)
        padded = np.zeros((len(tables), max(width, 1)), np.int32)
        for i, t in enumerate(tables):
            padded[i, : len(t)] = np.asarray(t)
        tables = padded
    return NativePlanner().plan(query_seq, head_dim, num_heads, tables, context_lens, block_size, **kwargs)


def _plan_flags(plan: AttentionPlan | None, shared_kv: bool) -> int:
    """pkv_paged_attention flags of a call with ``plan``."""
    flags = _native.PKV_ATTN_SHARED_KV if shared_kv else 0
    if plan is not None and plan.short_rows:
        flags |= _native.PKV_ATTN_SHORT_ROWS
    if plan is not None and plan.dominant_tiles:
        flags |= _native.PKV_ATTN_DOMINANT_TILES
    return flags


def launch_paged_attention(
    out: torch.Tensor, queries: torch.Tensor, query_positions: torch.Tensor, query_seq: torch.Tensor,
    key_cache: torch.Tensor, value_cache: torch.Tensor, block_tables: torch.Tensor,
    context_lens: torch.Tensor, scale: float, max_context_len: int, plan: AttentionPlan,
    workspace: torch.Tensor, device: int, append: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
    caller_rows: torch.Tensor | None = None,
) -> None:  # fmt: skip
    """:func:`paged_attention_ragged` for callers that built every argument themselves (the
    runner): the same C call without re-validating shapes and dtypes on the host. Preconditions
    are the checked function's: contiguous float32 ``out`` ``[T, H, D]``; queries with
    contiguous rows; int32 positions, sequence indices, tables, contexts and plan tensors on the
    pools' device; a workspace of ``attention_workspace_bytes`` bytes; for ``append``, the decode
    shape. The library still validates sizes and pointers before enqueueing anything."""
    num_queries, heads, dim = out.shape
    flags = _plan_flags(plan, plan.shared_kv)
    merge = plan.merge
    num_merge = -1 if merge is None else int(merge.shape[0])
    num_rows, num_tiles = int(plan.rows.shape[0]), int(plan.tiles.shape[0])
    if num_queries == 0 or (num_rows == 0 and num_tiles == 0):
        return
    lib = _native.library()
    common = (
        out.data_ptr(), queries.data_ptr(), queries.stride(0), query_positions.data_ptr(), query_seq.data_ptr(),
        num_queries, None if caller_rows is None else caller_rows.data_ptr(),
        plan.rows.data_ptr() if num_rows else None, num_rows,
    )  # fmt: skip
    tail = (
        merge.data_ptr() if num_merge > 0 else None, num_merge, key_cache.data_ptr(), value_cache.data_ptr(),
        kv_dtype_code(key_cache.dtype), key_cache.shape[0], key_cache.shape[1], block_tables.data_ptr(),
        block_tables.shape[1], context_lens.data_ptr(), block_tables.shape[0], heads, dim, float(scale),
        max_context_len, plan.partition_size, flags, workspace.data_ptr(), workspace.numel() * workspace.element_size(),
    )  # fmt: skip
    if append is None:
        rc = lib.pkv_paged_attention(*common, plan.tiles.data_ptr() if num_tiles else None, num_tiles, *tail,
                                     device, _stream(device))  # fmt: skip
        _native.check(rc, "pkv_paged_attention")
        return
    new_keys, new_values, slot_mapping = append
    rc = lib.pkv_paged_attention_append(
        *common, plan.tiles.data_ptr() if num_tiles else None, num_tiles, *tail, new_keys.data_ptr(),
        new_values.data_ptr(), kv_dtype_code(new_keys.dtype),
        new_keys.stride(0), new_values.stride(0), slot_mapping.data_ptr(), device, _stream(device),
    )  # fmt: skip
    _native.check(rc, "pkv_paged_attention_append")


def upload_plan(
    rows: np.ndarray, tiles: np.ndarray, device: torch.device, *, partition_size: int = 0,
    shared_kv: bool = False, merge: np.ndarray | None = None, short_rows: bool = False,
    dominant_tiles: bool = False,
) -> AttentionPlan:
    """Copy a host plan (``rows [R, 2]``, ``tiles [n, 4]``, ``merge [M]``) to the device in one
    transfer. Without a merge list, one is derived when a tile is whole (every row no whole tile
    covers), since the reduce must not touch the rows those tiles finish."""
    rows = np.asarray(rows, dtype=np.int32).reshape(-1, 2)
    tiles = np.asarray(tiles, dtype=np.int32).reshape(-1, 4)
    if merge is None and tiles.size and np.any(tiles[:, 3] == TILE_WHOLE):
        num_queries = max(int(rows[:, 0].max()) + 1 if rows.size else 0,
                          int((tiles[:, 0] + tiles[:, 1]).max()))  # fmt: skip
        merge = merge_rows_for(num_queries, tiles)
    merge_arr = np.zeros(0, np.int32) if merge is None else np.asarray(merge, dtype=np.int32).ravel()
    packed = np.concatenate([rows.ravel(), tiles.ravel(), merge_arr])
    data = torch.from_numpy(packed).to(device)
    end_tiles = rows.size + tiles.size
    return AttentionPlan(
        rows=data[: rows.size].view(-1, 2), tiles=data[rows.size : end_tiles].view(-1, 4),
        partition_size=partition_size, shared_kv=shared_kv,
        merge=None if merge is None else data[end_tiles:], short_rows=short_rows,
        dominant_tiles=dominant_tiles,
    )  # fmt: skip


def upload_batch_plan(plan: BatchPlan, device: torch.device) -> AttentionPlan:
    return upload_plan(plan.rows, plan.tiles, device, partition_size=plan.partition_size,
                       shared_kv=plan.shared_kv, merge=plan.merge, short_rows=plan.short_rows,
                       dominant_tiles=plan.dominant_tiles)  # fmt: skip


def attention_workspace_bytes(
    num_queries: int, num_heads: int, head_dim: int, max_context_len: int, partition_size: int = 0
) -> int:
    """Bytes of float32 split-context workspace :func:`paged_attention_ragged` needs."""
    size = _native.library().pkv_attention_workspace_bytes(
        num_queries, num_heads, head_dim, max_context_len, partition_size
    )
    if size < 0:
        raise ValueError("invalid attention workspace query")
    return int(size)


def paged_attention_ragged(
    queries: torch.Tensor,
    query_positions: torch.Tensor,
    query_seq: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    *,
    max_context_len: int,
    partition_size: int = 0,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    plan: AttentionPlan | None = None,
    shared_kv: bool | None = None,
    append: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
    caller_rows: torch.Tensor | None = None,
) -> torch.Tensor:
    """Causal paged attention of every query row of a ragged batch, in one call.

    ``caller_rows`` (int32 ``[T]``, a permutation of ``range(T)``, or None): query t reads row
    ``caller_rows[t]`` of ``queries`` and writes that row of the output (and, with ``append``,
    takes that row of the new keys and values and of ``slot_mapping``), while the positions,
    sequence indices and plan are indexed by t. A plan can then order the rows its own way (rows
    sharing a prefix next to each other) without the caller reordering its tensors.

    ``append=(new_keys, new_values, slot_mapping)`` fuses a decode step's append into the call
    (``pkv_paged_attention_append``): row t's own key and value row (``[T, H, D]`` float32, or
    bfloat16 for a bfloat16 pool; token-strided views allowed) is written to slot
    ``slot_mapping[t]`` (int64) by the row pass itself, exactly as :func:`append_kv` followed by
    this call would. Every row then goes through the row pass (a plan must have no tiles), and the
    caller guarantees the decode shape: one query row per sequence, at a position below its
    context length, with the slot its block table gives (reference runner.py:149-159).

    ``queries``: float32 ``[T, H, D]`` (token-strided views allowed); ``query_positions`` and
    ``query_seq``: int32 ``[T]``; ``key_cache``/``value_cache``: one layer's pools
    ``[num_blocks, block_size, H, D]``; ``block_tables``: int32 ``[S, max_blocks]``;
    ``context_lens``: int32 ``[S]``; ``max_context_len`` bounds every context length.
    ``plan`` (from :func:`plan_batch` + :func:`upload_batch_plan`) routes prefill runs and shared
    prefixes to the MFMA tile
    pass; without one every row takes the row-streaming pass. An explicit ``partition_size``
    overrides the plan's; so does ``shared_kv`` when not None.
    Returns float32 ``[T, H, D]``. Semantics of reference attention.py:42-121 for each query.
    """
    device = _device_index(
        queries, query_positions, query_seq, key_cache, value_cache, block_tables, context_lens
    )
    _native.init_device(device)  # once per device: the stream the tile pass overlaps on
    if queries.dtype != torch.float32:
        raise ValueError("queries must be float32")
    stride = _rows_contiguous(queries, "queries")
    num_queries, heads, dim = queries.shape
    if key_cache.shape != value_cache.shape or key_cache.dtype != value_cache.dtype:
        raise ValueError("key and value caches must have the same shape")
    if key_cache.dim() != 4 or tuple(key_cache.shape[2:]) != (heads, dim):
        raise ValueError("caches must have shape (num_blocks, block_size, heads, head_dim)")
    if not (key_cache.is_contiguous() and value_cache.is_contiguous()):
        raise ValueError("caches must be contiguous")
    for name, tensor in (("query_positions", query_positions), ("query_seq", query_seq), ("caller_rows", caller_rows)):
        if tensor is not None and (tensor.dtype != torch.int32 or tensor.shape != (num_queries,)):
            raise ValueError(f"{name} must be int32 with one entry per query")
    if caller_rows is not None and (caller_rows.device != queries.device or not caller_rows.is_contiguous()):
        raise ValueError("caller_rows must be contiguous and on the queries' device")
    caller_ptr = None if caller_rows is None else caller_rows.data_ptr()
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2:
        raise ValueError("block_tables must be int32 of shape (num_seqs, max_blocks)")
    if not block_tables.is_contiguous():
        raise ValueError("block_tables must be contiguous")
    num_seqs = block_tables.shape[0]
    if context_lens.dtype != torch.int32 or context_lens.shape != (num_seqs,):
        raise ValueError("context_lens must be int32 with one entry per sequence")
    if block_tables.shape[1] * key_cache.shape[1] < max_context_len:
        raise ValueError("block_tables are too narrow for max_context_len")
    if out is None:
        out = torch.empty((num_queries, heads, dim), dtype=torch.float32, device=queries.device)
    elif out.shape != (num_queries, heads, dim) or out.dtype != torch.float32:
        raise ValueError("out must be float32 of shape (num_queries, heads, head_dim)")
    elif not out.is_contiguous():
        raise ValueError("out must be contiguous")
    if num_queries == 0:
        return out
    if plan is not None and plan.partition_size:
        if partition_size not in (0, plan.partition_size):
            raise ValueError(
                f"the plan's partitions were laid out for partition_size {plan.partition_size}, "
                f"not {partition_size}"
            )
        partition_size = plan.partition_size
    if shared_kv is None:
        shared_kv = plan.shared_kv if plan is not None else False
    need = attention_workspace_bytes(num_queries, heads, dim, max_context_len, partition_size)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need // 4, dtype=torch.float32, device=queries.device)
    ws_ptr = workspace.data_ptr() if need else None
    ws_bytes = workspace.numel() * workspace.element_size() if need else 0
    rows_ptr = tiles_ptr = merge_ptr = None
    num_rows = num_tiles = 0
    num_merge = -1  # every row
    if plan is not None:
        for name, tensor in (("rows", plan.rows), ("tiles", plan.tiles)):
            if tensor.dtype != torch.int32 or tensor.device != queries.device:
                raise ValueError(f"plan.{name} must be an int32 tensor on the queries' device")
        if plan.rows.dim() != 2 or plan.rows.shape[1] != 2 or not plan.rows.is_contiguous():
            raise ValueError("plan.rows must be contiguous int32 of shape (R, 2)")
        if plan.tiles.dim() != 2 or plan.tiles.shape[1] != 4 or not plan.tiles.is_contiguous():
            raise ValueError("plan.tiles must be contiguous int32 of shape (n, 4)")
        num_rows, num_tiles = plan.num_rows, plan.num_tiles
        rows_ptr = plan.rows.data_ptr() if num_rows else None
        tiles_ptr = plan.tiles.data_ptr() if num_tiles else None
        if append is not None and not num_rows:
            raise ValueError("a fused append needs a plan with row-pass rows (the row pass appends)")
        if num_rows == 0 and num_tiles == 0:
            return out
        if plan.merge is not None:
            merge = plan.merge
            if merge.dtype != torch.int32 or merge.device != queries.device or merge.dim() != 1:
                raise ValueError("plan.merge must be a 1-D int32 tensor on the queries' device")
            if not merge.is_contiguous():
                raise ValueError("plan.merge must be contiguous")
            num_merge = int(merge.shape[0])
            merge_ptr = merge.data_ptr() if num_merge else None
    flags = _plan_flags(plan, shared_kv)
    if append is not None:
        new_keys, new_values, slot_mapping = append
        if _device_index(new_keys, new_values, slot_mapping) != device:
            raise ValueError("the appended rows must be on the queries' device")
        if new_keys.shape != (num_queries, heads, dim) or new_values.shape != new_keys.shape:
            raise ValueError("new keys and values must be [num_queries, heads, head_dim]")
        if new_keys.dtype != new_values.dtype:
            raise ValueError("new keys and values must have the same dtype")
        if slot_mapping.dtype != torch.int64 or slot_mapping.shape != (num_queries,):
            raise ValueError("slot_mapping must be int64 with one slot per query row")
        rc = _native.library().pkv_paged_attention_append(
            out.data_ptr(), queries.data_ptr(), stride,
            query_positions.data_ptr(), query_seq.data_ptr(), num_queries, caller_ptr,
            rows_ptr, num_rows, tiles_ptr, num_tiles, merge_ptr, num_merge,
            key_cache.data_ptr(), value_cache.data_ptr(), kv_dtype_code(key_cache.dtype),
            key_cache.shape[0], key_cache.shape[1],
            block_tables.data_ptr(), block_tables.shape[1], context_lens.data_ptr(), num_seqs,
            heads, dim, float(scale), max_context_len, partition_size, flags,
            ws_ptr, ws_bytes, new_keys.data_ptr(), new_values.data_ptr(),
            kv_dtype_code(new_keys.dtype), _rows_contiguous(new_keys, "new keys"),
            _rows_contiguous(new_values, "new values"), slot_mapping.data_ptr(),
            device, _stream(device),
        )  # fmt: skip
        _native.check(rc, "pkv_paged_attention_append")
        return out
    rc = _native.library().pkv_paged_attention(
        out.data_ptr(), queries.data_ptr(), stride,
        query_positions.data_ptr(), query_seq.data_ptr(), num_queries, caller_ptr,
        rows_ptr, num_rows, tiles_ptr, num_tiles, merge_ptr, num_merge,
        key_cache.data_ptr(), value_cache.data_ptr(), kv_dtype_code(key_cache.dtype),
        key_cache.shape[0], key_cache.shape[1],
        block_tables.data_ptr(), block_tables.shape[1], context_lens.data_ptr(), num_seqs,
        heads, dim, float(scale), max_context_len, partition_size, flags,
        ws_ptr, ws_bytes, device, _stream(device),
    )  # fmt: skip
    _native.check(rc, "pkv_paged_attention")
    return out
