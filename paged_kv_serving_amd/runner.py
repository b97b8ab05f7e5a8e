"""GPU ModelRunner: the drop-in replacement of the reference's runner (runner.py:33-227).

It owns the K/V pools in HBM, shaped ``[layers, num_blocks, block_size, heads, head_dim]``
exactly like the reference's NumPy pools (runner.py:112-114), and is both the reference's
``EngineExecutor`` (``execute(batch) -> {seq_id: float32[vocab]}``, engine.py:64-73) and its
``BlockStore`` (``copy_block(src, dst)``, blocks.py:43-48). Per layer of :meth:`execute`:

    torch (hipBLASLt) : RMSNorm, fused QKV projection
    pkv_rope_append   : RoPE on q (in place) and k, and the scatter of the rotated keys and the
                        values into their slots, in one launch
    pkv_paged_attention : every query of the ragged batch against its block table in one call:
                          decode rows stream K/V per row, prefill runs go to the fp32 MFMA tile
                          pass, then the split-context reduce when a context spans partitions
    torch             : output projection, SwiGLU

Slot mappings are computed on the host with the reference's closed form and validation
(runner.py:149-159), so they are bit-exact with the reference by construction; they, the
positions and the block tables reach the device in two small copies per call.

Copy-on-write copies requested through :meth:`copy_block` are queued and flushed as batched
``pkv_copy_blocks`` launches before anything reads or writes the pool (the next
:meth:`execute`, :meth:`block_view`, :meth:`block_fingerprint`), on the same stream, so they land
before the append and attention of the step that scheduled them.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np
import torch

from paged_kv_serving_amd import ops
from paged_kv_serving_amd.tables import BlockTableArena

__all__ = ["DEFAULT_TILE_BLOCKS", "BatchEntry", "ExecutionBatch", "ModelRunner", "compute_slots"]

#: Accepted for API compatibility (reference attention.py:39). The kernels tile the context in
#: their own units, and results do not depend on this value.
DEFAULT_TILE_BLOCKS = 8


@dataclass(frozen=True)
class BatchEntry:
    """One sequence's slice of an iteration (runner.py:33-68)."""

    seq_id: str
    token_ids: tuple[int, ...]
    positions: tuple[int, ...]
    block_table: tuple[int, ...]
    logits_index: int | None = None

    def __post_init__(self) -> None:
        if not self.token_ids:
            raise ValueError("a batch entry must run at least one token")
        if len(self.token_ids) != len(self.positions):
            raise ValueError("token_ids and positions must have the same length")
        if self.logits_index is not None and not 0 <= self.logits_index < len(self.token_ids):
            raise ValueError("logits_index must point inside the slice")

    @property
    def needs_logits(self) -> bool:
        return self.logits_index is not None

    @property
    def num_tokens(self) -> int:
        return len(self.token_ids)

    @property
    def context_len(self) -> int:
        return self.positions[-1] + 1


@dataclass(frozen=True)
class ExecutionBatch:
    """The slices scheduled for one iteration (runner.py:71-87)."""

    entries: tuple[BatchEntry, ...]

    @property
    def num_tokens(self) -> int:
        return sum(entry.num_tokens for entry in self.entries)

    @property
    def num_sequences(self) -> int:
        return len(self.entries)

    @property
    def num_prefill_tokens(self) -> int:
        return sum(entry.num_tokens for entry in self.entries if entry.num_tokens > 1)


def compute_slots(entries, block_size: int) -> np.ndarray:
    """Flat slot ``block_table[p // B] * B + p % B`` of every token of a batch, int64.

    The slot mapping of runner.py:149-159 and :184-186, vectorised per entry; a position past
    the entry's table raises the reference's ValueError, naming the first such position.
    """
    total = sum(len(entry.positions) for entry in entries)
    out = np.empty(total, dtype=np.int64)
    offset = 0
    for entry in entries:
        positions, table = entry.positions, entry.block_table
        if len(positions) == 1:  # a decode row: one lookup, no array conversion of the table
            position = positions[0]
            index = position // block_size
            if index >= len(table):
                raise ValueError(f"sequence {entry.seq_id}: position {position} has no block in the table")
            out[offset] = table[index] * block_size + position % block_size
            offset += 1
            continue
        where = np.asarray(positions, dtype=np.int64)
        index = where // block_size
        missing = np.nonzero(index >= len(table))[0]
        if missing.size:
            position = int(where[missing[0]])
            raise ValueError(f"sequence {entry.seq_id}: position {position} has no block in the table")
        low = int(index.min())
        if low >= 0:  # convert only the stretch of the table the chunk touches
            blocks = np.asarray(table[low : int(index.max()) + 1], dtype=np.int64)
            index = index - low
        else:  # negative positions index from the end, as the reference's tuple lookup does
            blocks = np.asarray(table, dtype=np.int64)
        out[offset : offset + where.size] = blocks[index] * block_size + where % block_size
        offset += where.size
    return out


def shared_prefix_order(entries, block_size: int) -> list[int] | None:
    """A row order that puts decode entries whose block tables share their leading blocks next
    to each other, so ``ops.plan_batch`` can read a common prefix once per head as MFMA tiles
    (it looks for runs of consecutive rows). Decode entries (one token) with at least
    MIN_SHARED_TOKENS of table come first, stably sorted by those leading block ids; every other
    entry follows in batch order. None when the batch order already has every such run together
    or there are too few decode entries to form one."""
    lead = -(-ops.MIN_SHARED_TOKENS // block_size)
    decode = [i for i, e in enumerate(entries) if len(e.token_ids) == 1 and len(e.block_table) >= lead]
    if len(decode) < ops.MIN_SHARED_ROWS:
        return None
    keys = {i: tuple(entries[i].block_table[:lead]) for i in decode}
    grouped = sorted(decode, key=lambda i: keys[i])
    # Nothing to gain when no two decode entries share their leading blocks, or when the
    # entries that do are already adjacent in the batch.
    shared = sum(keys[a] == keys[b] for a, b in zip(grouped, grouped[1:]))
    adjacent = sum(keys[a] == keys[b] for a, b in zip(decode, decode[1:]) if b == a + 1)
    if shared == 0 or shared == adjacent:
        return None
    rest = [i for i in range(len(entries)) if i not in keys]
    return grouped + rest


def _rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    return x / torch.sqrt(torch.mean(x * x, dim=-1, keepdim=True) + eps) * weight


def _silu(x: torch.Tensor) -> torch.Tensor:
    return x * (1.0 / (1.0 + torch.exp(-torch.clamp(x, -60.0, 60.0))))


class _DeviceWeights:
    """Device copies of a model's weights and rotary tables, tied to one weights object."""

    def __init__(self, model, device: torch.device) -> None:
        def up(array: np.ndarray) -> torch.Tensor:
            return torch.from_numpy(np.ascontiguousarray(array, dtype=np.float32)).to(device)

        weights = model.weights
        self.source = weights
        self.embedding = up(weights.token_embedding)
        self.final_norm = up(weights.final_norm)
        self.layers = [
            tuple(
                up(getattr(layer, name))
                for name in (
                    "attn_norm", "qkv_proj", "out_proj", "ffn_norm",
                    "gate_proj", "up_proj", "down_proj",
                )  # fmt: skip
            )
            for layer in weights.layers
        ]
        cos, sin = model.rope
        self.cos = up(cos)
        self.sin = up(sin)


class ModelRunner:
    """Owns the K/V pools on one HIP device and executes ragged batches against them."""

    def __init__(
        self,
        model,
        *,
        num_blocks: int,
        block_size: int,
        tile_blocks: int = DEFAULT_TILE_BLOCKS,
        kv_dtype: torch.dtype = torch.float32,
        device: torch.device | str | int | None = None,
        partition_size: int = 0,
    ) -> None:
        """``partition_size`` 0 lets each call choose (``ops.plan_batch``)."""
        if num_blocks < 1 or block_size < 1:
            raise ValueError("num_blocks and block_size must be >= 1")
        if tile_blocks < 1:
            raise ValueError("tile_blocks must be >= 1")
        ops.kv_dtype_code(kv_dtype)
        config = model.config
        self.model = model
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.tile_blocks = tile_blocks
        self.partition_size = partition_size
        self.device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("ModelRunner keeps its pools on a HIP device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        shape = (config.n_layers, num_blocks, block_size, config.n_heads, config.head_dim)
        self._keys = torch.zeros(shape, dtype=kv_dtype, device=self.device)
        self._values = torch.zeros(shape, dtype=kv_dtype, device=self.device)
        self._pending: list[tuple[int, int]] = []
        self._weights: _DeviceWeights | None = None
        self._tables = BlockTableArena(self.device)
        #: The host plan of the last ``execute`` (rows, tiles, partition size, load hint).
        self.last_plan: ops.BatchPlan | None = None

    # --- pool ---------------------------------------------------------------------------

    @property
    def kv_dtype(self) -> torch.dtype:
        return self._keys.dtype

    @property
    def cache_bytes(self) -> int:
        return 2 * self._keys.numel() * self._keys.element_size()

    @property
    def capacity_tokens(self) -> int:
        return self.num_blocks * self.block_size

    @property
    def key_cache(self) -> torch.Tensor:
        """All layers' key pool (device tensor), after pending copies have landed."""
        self.flush_copies()
        return self._keys

    @property
    def value_cache(self) -> torch.Tensor:
        self.flush_copies()
        return self._values

    def block_view(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Key and value pools of one layer, as device tensor views (runner.py:124-126)."""
        self.flush_copies()
        return self._keys[layer], self._values[layer]

    def copy_block(self, source: int, destination: int) -> None:
        """Copy-on-write of one block across every layer (runner.py:128-133), queued.

        The copy is enqueued on the device before the pool is next read or written.
        """
        if source == destination:
            raise ValueError("copy-on-write must not copy a block onto itself")
        for block_id in (source, destination):
            if not 0 <= block_id < self.num_blocks:
                raise IndexError(f"block id {block_id} is outside the pool")
        self._pending.append((int(source), int(destination)))

    def flush_copies(self) -> int:
        """Launch every queued copy-on-write copy, in order. Returns the number of copies."""
        if not self._pending:
            return 0
        pending, self._pending = self._pending, []
        for group in ops.independent_groups(pending):
            pairs = torch.tensor(group, dtype=torch.int64).to(self.device, non_blocking=True)
            ops.copy_blocks(self._keys, self._values, pairs)
        return len(pending)

    def block_fingerprint(self, block_id: int) -> bytes:
        """BLAKE2b-16 of one block's bytes, keys then values (runner.py:135-142)."""
        self.flush_copies()
        digest = hashlib.blake2b(digest_size=16)
        for pool in (self._keys, self._values):
            data = pool[:, block_id].contiguous().cpu()
            digest.update(data.view(torch.uint8).numpy().tobytes())
        return digest.digest()

    def reset_cache(self) -> None:
        """Zero the whole pool; queued copies are dropped (runner.py:144-147)."""
        self._pending.clear()
        self._keys.zero_()
        self._values.zero_()

    # --- forward ------------------------------------------------------------------------

    def _device_weights(self) -> _DeviceWeights:
        # Keyed on the weights object: an admin swap assigns a new one (reference api.py:577-584).
        if self._weights is None or self._weights.source is not self.model.weights:
            self._weights = _DeviceWeights(self.model, self.device)
        return self._weights

    def execute(self, batch: ExecutionBatch) -> dict[str, np.ndarray]:
        """Run one iteration; return host float32 logits for the entries that ask for them.

        Keys and values of every token are written into the pool as a side effect, so the
        blocks named by each entry's block table must have been allocated first.
        """
        names, logits = self._forward(batch)
        if not names:
            return {}
        host = logits.cpu().numpy()
        return {name: host[i] for i, name in enumerate(names)}

    def execute_greedy(self, batch: ExecutionBatch) -> dict[str, int]:
        """:meth:`execute` followed by greedy sampling on the device: the argmax token id of each
        logits row (reference sampling.py:28-30), one int32 per row copied to the host."""
        names, logits = self._forward(batch)
        if not names:
            return {}
        tokens = ops.greedy_tokens(logits).cpu().numpy()
        return {name: int(tokens[i]) for i, name in enumerate(names)}

    def _forward(self, batch: ExecutionBatch) -> tuple[list[str], torch.Tensor | None]:
        """The forward pass of one iteration: (seq ids, device logits [rows, vocab]) of the
        entries that ask for logits, in batch order."""
        entries = batch.entries
        if not entries:
            return [], None
        config = self.model.config
        total = sum(len(entry.token_ids) for entry in entries)
        tokens = np.fromiter((t for e in entries for t in e.token_ids), dtype=np.int64, count=total)
        if np.any(tokens < 0) or np.any(tokens >= config.vocab_size):
            raise ValueError("token id outside the vocabulary")
        positions = np.fromiter((p for e in entries for p in e.positions), dtype=np.int64, count=total)
        if np.any(positions >= config.max_seq_len):
            raise ValueError("position beyond max_seq_len")
        if np.any(positions < 0):
            raise ValueError("positions must be >= 0")
        slots = compute_slots(entries, self.block_size)
        if slots.size and (slots.min() < 0 or slots.max() >= self.capacity_tokens):
            raise IndexError("a block table names a block outside the pool")
        # Rows in the order the planner can use (validation above ran in batch order, so errors
        # name the same entry as the reference's); logits come back in batch order below.
        order = shared_prefix_order(entries, self.block_size)
        lengths = np.fromiter((len(e.token_ids) for e in entries), dtype=np.int64, count=len(entries))
        batch_starts = np.cumsum(lengths) - lengths
        if order is not None:
            token_order = np.concatenate([np.arange(batch_starts[i], batch_starts[i] + lengths[i]) for i in order])
            tokens, positions, slots = tokens[token_order], positions[token_order], slots[token_order]
            moved = np.cumsum(lengths[order]) - lengths[order]
            starts = np.empty_like(batch_starts)
            starts[order] = moved
            entries = [entries[i] for i in order]
        else:
            starts = batch_starts

        num_seqs = len(entries)
        # Block tables live in a device arena between calls; only changed entries travel.
        update = self._tables.update(entries)
        arena_rows = self._tables.num_rows
        context = np.fromiter((e.positions[-1] + 1 for e in entries), dtype=np.int32, count=num_seqs)
        contexts_by_row = np.zeros(arena_rows, dtype=np.int32)
        contexts_by_row[update.rows] = context
        per_entry = np.fromiter((len(e.token_ids) for e in entries), dtype=np.int64, count=num_seqs)
        query_seq = np.repeat(update.rows, per_entry)
        host_plan = ops.plan_batch(
            query_seq, config.head_dim, config.n_heads, self._tables.host, contexts_by_row,
            self.block_size, partition_size=self.partition_size, query_positions=positions,
        )  # fmt: skip
        self.last_plan = host_plan
        partition = host_plan.partition_size
        plan_rows, plan_tiles, plan_merge = host_plan.rows, host_plan.tiles, host_plan.merge
        changed = update.index.size
        meta64 = torch.from_numpy(np.concatenate([tokens, positions, slots, update.index])).to(self.device)
        meta32 = torch.from_numpy(
            np.concatenate([
                positions.astype(np.int32), query_seq, contexts_by_row, update.values,
                plan_rows.ravel(), plan_tiles.ravel(), plan_merge,
            ])  # fmt: skip
        ).to(self.device)
        tokens_d, positions_d = meta64[:total], meta64[total : 2 * total]
        slots_d = meta64[2 * total : 3 * total]
        qpos_d = meta32[:total]
        qseq_d = meta32[total : 2 * total]
        context_d = meta32[2 * total : 2 * total + arena_rows]
        end_values = 2 * total + arena_rows + changed
        self._tables.apply(meta64[3 * total :], meta32[2 * total + arena_rows : end_values])
        tables_d = self._tables.tables
        end_rows = end_values + plan_rows.size
        end_tiles = end_rows + plan_tiles.size
        plan = ops.AttentionPlan(
            rows=meta32[end_values:end_rows].view(-1, 2),
            tiles=meta32[end_rows:end_tiles].view(-1, 4),
            partition_size=partition,
            shared_kv=host_plan.shared_kv,
            merge=meta32[end_tiles:],
            short_rows=host_plan.short_rows,
        )
        max_context = int(context.max())

        self.flush_copies()
        w = self._device_weights()
        heads, dim, d_model = config.n_heads, config.head_dim, config.d_model
        eps = config.norm_eps
        scale = self.model.attention_scale
        hidden = w.embedding[tokens_d]
        workspace = None
        attended = torch.empty((total, heads, dim), dtype=torch.float32, device=self.device)
        for index, (attn_norm, qkv, out_proj, ffn_norm, gate, up, down) in enumerate(w.layers):
            fused = (_rms_norm(hidden, attn_norm, eps) @ qkv).view(total, 3, heads, dim)
            # RoPE on q (in place) and k, and the append of k and v, in one kernel
            # (reference model.py:251-252 then runner.py:195-196).
            queries = ops.rope_append(
                self._keys[index], self._values[index], fused[:, 0], fused[:, 1], fused[:, 2],
                positions_d, w.cos, w.sin, slots_d, out=fused[:, 0],
            )  # fmt: skip
            if workspace is None:
                need = ops.attention_workspace_bytes(total, heads, dim, max_context, partition)
                workspace = torch.empty(max(need // 4, 1), dtype=torch.float32, device=self.device)
            ops.paged_attention_ragged(
                queries, qpos_d, qseq_d, self._keys[index], self._values[index], tables_d,
                context_d, scale, max_context_len=max_context,
                partition_size=partition, out=attended, workspace=workspace, plan=plan,
            )  # fmt: skip
            hidden = hidden + attended.view(total, d_model) @ out_proj
            normed = _rms_norm(hidden, ffn_norm, eps)
            hidden = hidden + (_silu(normed @ gate) * (normed @ up)) @ down

        wanted, names = [], []
        for start, entry in zip(starts.tolist(), batch.entries):
            if entry.logits_index is not None:
                wanted.append(start + entry.logits_index)
                names.append(entry.seq_id)
        if not wanted:
            return [], None
        rows = torch.tensor(wanted, dtype=torch.int64).to(self.device)
        return names, _rms_norm(hidden[rows], w.final_norm, eps) @ w.embedding.T
