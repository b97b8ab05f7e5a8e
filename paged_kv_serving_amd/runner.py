"""GPU ModelRunner: the drop-in replacement of the reference's runner (runner.py:33-227).

It owns the K/V pools in HBM, shaped ``[layers, num_blocks, block_size, heads, head_dim]``
exactly like the reference's NumPy pools (runner.py:112-114), and is both the reference's
``EngineExecutor`` (``execute(batch) -> {seq_id: float32[vocab]}``, engine.py:64-73) and its
``BlockStore`` (``copy_block(src, dst)``, blocks.py:43-48). Per layer of :meth:`execute`, all
enqueued by one C++ call of the host extension:

    pkv_rms_norm        : RMSNorm, with the preceding residual add fused into it
    rocBLAS sgemm       : the fused QKV projection
    pkv_rope_append     : RoPE on q (in place) and k, and the scatter of the rotated keys and the
                          values into their slots, in one launch
    pkv_paged_attention : every query of the ragged batch against its block table in one call:
                          decode rows stream K/V per row, prefill runs go to the fp32 MFMA tile
                          pass, then the split-context reduce when a context spans partitions
    rocBLAS sgemm, pkv_silu_mul : the output projection and the SwiGLU block

Slot mappings are computed on the host with the reference's closed form and validation
(runner.py:149-159), so they are bit-exact with the reference by construction; they, the
positions and the changed block-table entries reach the device in one copy per call.

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

from paged_kv_serving_amd import _native, ops
from paged_kv_serving_amd.tables import BlockTableArena

__all__ = ["DEFAULT_TILE_BLOCKS", "BatchEntry", "ExecutionBatch", "ModelRunner", "compute_slots"]

#: Accepted for API compatibility (reference attention.py:39). The kernels tile the context in
#: their own units, and results do not depend on this value.
DEFAULT_TILE_BLOCKS = 8


_NO_ROWS = np.zeros(0, dtype=np.int64)  # no logits rows (read only)
_NO_ROWS.flags.writeable = False


@dataclass(frozen=True, slots=True)
class BatchEntry:
    """One sequence's slice of an iteration (runner.py:33-68), slotted as the reference's is. The
    host extension reads the fields at their slots' offsets when it walks a batch."""

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


@dataclass(frozen=True, slots=True)
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
    # Sharers have the same first block: when every decode entry starts elsewhere (the common
    # case of private sequences), there is nothing to group.
    if len({entries[i].block_table[0] for i in decode}) == len(decode):
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


class _Staging:
    """One call's integer metadata, sent in one asynchronous copy from pinned host memory.

    The sections (the int64 ones first, 8-byte aligned, then the int32 ones) are packed into a
    pinned host buffer and copied to a device buffer of the same layout on the runner's stream by
    one C++ call (``_pkvhost.stage``: the packing and one ``hipMemcpyAsync``); the host does not
    wait for the copy. Before a later call rewrites the host buffer it waits for the copy that
    last read it (a HIP event the same C++ call records), which has normally long finished. The
    device buffer is rewritten by the next call's copy, which the stream orders after this call's
    kernels."""

    def __init__(self, device: torch.device, host_ext) -> None:
        self.device = device
        self._ext = host_ext
        self.host: torch.Tensor | None = None
        self.dev: torch.Tensor | None = None
        self.base = 0  # device address of self.dev
        self._host_np = np.zeros(0, dtype=np.uint8)
        self._event = 0  # the HIP event recorded after each copy (created at the first send)

    def __del__(self) -> None:
        if self._event:
            # At interpreter exit the extension module's globals may already be cleared (None);
            # the process's end releases the event then.
            destroy = getattr(self._ext, "event_destroy", None)
            if callable(destroy):
                destroy(self._event)
            self._event = 0

    @property
    def host_array(self) -> np.ndarray:
        """The pinned host buffer as a NumPy uint8 array (empty until :meth:`grow`)."""
        return self._host_np

    def grow(self, nbytes: int) -> None:
        """Reallocate both buffers to hold at least ``nbytes``. The old ones are dropped after the
        device has drained: the last copy from the host buffer and the kernels reading the device
        buffer are raw HIP work that torch's allocators do not track."""
        torch.cuda.synchronize(self.device)
        size = max(nbytes, 2 * self._host_np.size, 1 << 16)
        self.host = torch.empty(size, dtype=torch.uint8, pin_memory=True)
        self.dev = torch.empty(size, dtype=torch.uint8, device=self.device)
        self.base = self.dev.data_ptr()
        self._host_np = self.host.numpy()

    def send(self, parts64: list[np.ndarray], parts32: list[np.ndarray], stream: int | None = None) -> list[int]:
        """Copy ``parts64`` (int64 arrays) then ``parts32`` (int32 arrays) to the device on
        ``stream`` (default: the device's current stream); returns each part's byte offset in the
        device buffer (see :meth:`tensor` and :attr:`base`)."""
        if stream is None:
            stream = ops._stream(self.device.index)
        if not self._event:
            self._event = self._ext.event_create(self.device.index)
        while True:
            offsets = self._ext.stage(parts64, parts32, self._host_np, self.base, stream, self._event)
            if offsets is not None:
                return offsets
            self.grow(8 * sum(p.size for p in parts64) + 4 * sum(p.size for p in parts32))

    def tensor(self, offset: int, count: int, dtype: torch.dtype) -> torch.Tensor:
        """A device tensor view of ``count`` elements of ``dtype`` (int32 or int64) at byte
        ``offset``."""
        size = 8 if dtype == torch.int64 else 4
        return self.dev[offset : offset + count * size].view(dtype)


@dataclass(slots=True)
class _Step:
    """One iteration's device-side metadata (from :meth:`ModelRunner._prepare`), in the planner's
    row order; ``token_order`` maps it back to batch order (None: the same), and when it is set
    the staging buffer also holds it as int32 (``caller_rows_at``: the attention call's
    caller_rows) and the slots in batch order (``batch_slots_at``). Every section lives
    in the staging buffer at ``staging.base`` + its byte offset; the ``*_at`` fields are those
    offsets, and :meth:`tensor` gives torch views where torch needs them."""

    total: int
    staging: _Staging
    tokens_at: int
    rope_at: int
    slots_at: int
    logits_at: int
    qpos_at: int
    qseq_at: int
    contexts_at: int
    plan_rows_at: int
    plan_tiles_at: int
    merge_at: int
    num_plan_rows: int
    num_tiles: int
    num_merge: int
    num_wanted: int
    partition: int
    flags: int
    max_context: int
    token_order: np.ndarray | None
    caller_rows_at: int
    batch_slots_at: int
    entries: tuple
    decode_only: bool

    def tensor(self, name: str) -> torch.Tensor:
        """int64 views: ``tokens``, ``rope_positions``, ``slots``, ``batch_slots`` (the slots in
        batch order), ``logits_rows``."""
        offset, count = {
            "tokens": (self.tokens_at, self.total), "rope_positions": (self.rope_at, self.total),
            "slots": (self.slots_at, self.total), "batch_slots": (self.batch_slots_at, self.total),
            "logits_rows": (self.logits_at, self.num_wanted),
        }[name]  # fmt: skip
        return self.staging.tensor(offset, count, torch.int64)

    def ptr(self, offset: int) -> int:
        return self.staging.base + offset


class _DeviceWeights:
    """Device copies of a model's weights and rotary tables, tied to one weights object. Each
    layer's gate and up projections are stored side by side as one ``[d_model, 2 * d_ff]`` matrix,
    so the SwiGLU block runs one product for both."""

    def __init__(self, model, device: torch.device) -> None:
        def up(array: np.ndarray) -> torch.Tensor:
            return torch.from_numpy(np.ascontiguousarray(array, dtype=np.float32)).to(device)

        weights = model.weights
        self.source = weights
        self.embedding = up(weights.token_embedding)
        self.final_norm = up(weights.final_norm)
        self.layers = [
            (
                up(layer.attn_norm), up(layer.qkv_proj), up(layer.out_proj), up(layer.ffn_norm),
                up(np.concatenate([layer.gate_proj, layer.up_proj], axis=1)), up(layer.down_proj),
            )
            for layer in weights.layers
        ]
        cos, sin = model.rope
        self.cos = up(cos)
        self.sin = up(sin)
        #: Per layer the six addresses the host extension's forward pass reads.
        self.addresses = [tuple(t.data_ptr() for t in layer) for layer in self.layers]


class ModelRunner:
    """Owns the K/V pools on one HIP device and executes ragged batches against them.

    Work is enqueued on the caller's current stream of the runner's device. Consecutive calls
    reuse one device metadata buffer and one split-context workspace, so a runner's calls must be
    ordered on the device (one stream, as the reference engine's serialised steps are); calls of
    one runner overlapping on two streams would race on those buffers."""

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
        self._weights: _DeviceWeights | None = None
        self._tables = BlockTableArena(self.device)
        self._planner = ops.NativePlanner()
        self._host = _native.bound_host()
        self._staging = _Staging(self.device, self._host)
        self._device_index = self.device.index
        self._stats = np.zeros(9, np.int64)
        self._contexts_by_row = np.zeros(0, np.int32)  # a call's context lengths by arena row
        self._kv_code = ops.kv_dtype_code(kv_dtype)
        self._marks = np.zeros(num_blocks, np.uint8)  # one per pool block, for exclusive_writes
        self._order = np.zeros(256, np.int64)  # a call's planner row order (prefix_order_rows)
        # Queued copy-on-write copies live in C++ (_pkvhost.CopyQueue); copy_block is its push,
        # so a scheduler's per-block calls cost no Python frame. Their pairs travel through a
        # pinned buffer of their own.
        self._copies = self._host.CopyQueue(num_blocks)
        self.copy_block = self._copies.push
        self._cow_staging = _Staging(self.device, self._host)
        self._workspace: torch.Tensor | None = None
        self._forward_ws: torch.Tensor | None = None  # the forward pass's activations
        self._greedy_out: torch.Tensor | None = None  # its greedy token ids
        _native.init_device(self._device_index)  # the library's overlap stream on this device
        self._per_token = (np.zeros(1024, np.int64), np.zeros(1024, np.int64), np.zeros(1024, np.int64))
        self._per_entry = (np.zeros(256, np.int64), np.zeros(256, np.int32), np.zeros(256, np.int64))
        self._last_plan: tuple | None = None  # the last call's plan pieces (see last_plan)
        #: Whether the last step's append rode inside its attention call (the decode rule of
        #: _pkvhost.exclusive_writes), rather than a pkv_append launch before it.
        self.last_append_fused = False
        self._layer_bytes = self._keys[0].numel() * self._keys.element_size()
        self._block_elems = self._keys[0, 0].numel()

    @property
    def last_plan(self) -> ops.BatchPlan | None:
        """The host plan of the last call (rows, tiles, merge list, partition size, hints); its
        arrays are views of the planner's buffers, rewritten by the next call."""
        if self._last_plan is None:
            return None
        plan_rows, plan_tiles, partition, flags, merge = self._last_plan
        return ops.BatchPlan(
            plan_rows, plan_tiles, partition, bool(flags & _native.PKV_ATTN_SHARED_KV), merge,
            bool(flags & _native.PKV_ATTN_SHORT_ROWS), bool(flags & _native.PKV_ATTN_DOMINANT_TILES),
        )  # fmt: skip

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

        The copy is enqueued on the device before the pool is next read or written. A runner's
        ``copy_block`` attribute is its C++ queue's ``push``, which makes these same checks
        (ValueError for a copy onto itself, IndexError naming a block id outside the pool);
        this method is what the class exposes.
        """
        self._copies.push(source, destination)

    @property
    def pending_copies(self) -> list[tuple[int, int]]:
        """The queued (source, destination) copies, in queue order."""
        return self._copies.items()

    def flush_copies(self) -> int:
        """Launch every queued copy-on-write copy, in order: one ``pkv_copy_blocks`` launch per
        group of independent copies (``ops.independent_groups``'s rule), their pairs sent in one
        asynchronous copy of their own, all from one C++ call (``CopyQueue.flush``). Returns the
        number of copies. A failed launch raises and leaves every copy queued (a group reads no
        block it writes, so a group that ran already leaves the same bytes when it runs again)."""
        copies = self._copies
        if not len(copies):
            return 0
        keys, staging = self._keys, self._cow_staging
        while True:
            rc, count = copies.flush(
                keys.data_ptr(), self._values.data_ptr(), self._kv_code, keys.shape[0], self._block_elems,
                staging.host_array, staging.base, self._device_index, ops._stream(self._device_index),
            )  # fmt: skip
            if count >= 0:
                break
            staging.grow(-count)
        _native.check(rc, "pkv_copy_blocks")
        return count

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
        self._copies.clear()
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
        host = logits.cpu().numpy()  # a copy: the next call rewrites the device rows
        return {name: host[i] for i, name in enumerate(names)}

    def execute_greedy(self, batch: ExecutionBatch) -> dict[str, int]:
        """:meth:`execute` followed by greedy sampling on the device: the argmax token id of each
        logits row (reference sampling.py:28-30), one int32 per row copied to the host."""
        names, tokens = self._forward(batch, greedy=True)
        if not names:
            return {}
        picked = tokens.cpu().numpy()
        return {name: int(picked[i]) for i, name in enumerate(names)}

    def _gather(self, entries):
        """One C++ walk over the entries (``_pkvhost.gather``): token ids, positions and slots
        (batch order, int64), per-entry lengths, context lengths (int32) and flat logits rows (-1:
        none), and the first slot problem (0 none, 1 past the table, 2 before its start) with its
        entry index and position."""
        count = len(entries)
        if self._per_entry[0].size < count:
            n = max(count, 2 * self._per_entry[0].size)
            self._per_entry = (np.zeros(n, np.int64), np.zeros(n, np.int32), np.zeros(n, np.int64))
        lengths, contexts, logits = self._per_entry
        while True:
            tokens, positions, slots = self._per_token
            total, problem, entry, position = self._host.gather(
                entries, self.block_size, tokens, positions, slots, lengths, contexts, logits, self._stats
            )
            if total >= 0:
                break
            n = max(-total, 2 * tokens.size)
            self._per_token = (np.zeros(n, np.int64), np.zeros(n, np.int64), np.zeros(n, np.int64))
        # Views of the reused buffers: they are consumed (copied into the staging buffer, or
        # reindexed) before the next call rewrites them.
        return (tokens[:total], positions[:total], slots[:total], lengths[:count], contexts[:count],
                logits[:count], (problem, entry, position))  # fmt: skip

    def _prepare(self, batch: ExecutionBatch, *, logits: bool = True) -> _Step | None:
        """Everything one iteration needs on the device before its first kernel: validation in
        the reference's order and with its messages, slots, the block-table arena update, the
        attention plan, and one asynchronous copy of all of it (None for an empty batch). Without
        ``logits`` (attend, which computes none) no logits rows are listed."""
        entries = batch.entries
        if not entries:
            return None
        # Copies queued by copy_block (the scheduler's copy-on-write, issued before this step in
        # the reference, blocks.py:162-164) start first, so the device copies while the host
        # prepares the step; the stream orders them before this step's appends and attention.
        self.flush_copies()
        config = self.model.config
        tokens, positions, slots, lengths, context, logits_rows, (problem, bad, position) = self._gather(entries)
        total = tokens.size
        low_token, high_token, low_pos, high_pos, low_slot, high_slot, low_ctx, repeats, high_ctx = self._stats.tolist()
        # The reference checks token ids, then positions, then forms the slots (runner.py:174-187).
        if low_token < 0 or high_token >= config.vocab_size:
            raise ValueError("token id outside the vocabulary")
        if high_pos >= config.max_seq_len:
            raise ValueError("position beyond max_seq_len")
        if problem == 1:
            raise ValueError(f"sequence {entries[bad].seq_id}: position {position} has no block in the table")
        if problem == 2:
            raise IndexError("tuple index out of range")
        if low_slot < 0 or high_slot >= self.capacity_tokens:
            raise IndexError("a block table names a block outside the pool")
        # Negative positions run as in the reference: their slot comes from the end of the table
        # (a Python index, runner.py:158), their rotary angle from the end of the tables (a NumPy
        # index, model.py:77-78), and every key is masked for them (a zero attention row,
        # attention.py:102-104, 120-121). An entry ending at one has context_len < 1, which the
        # reference's attention refuses (attention.py:76-77).
        rope_positions = positions
        if low_pos < 0:
            if low_pos < -config.max_seq_len:
                raise IndexError("position outside the rotary tables")
            if low_ctx < 1:
                raise ValueError("context_len must be >= 1")
            rope_positions = np.where(positions < 0, positions + config.max_seq_len, positions)
        # Logits rows, in batch order of the entries that ask for them.
        wanted = logits_rows[logits_rows >= 0] if logits else _NO_ROWS
        # Block tables live in a device arena between calls; only changed entries travel.
        update = self._tables.update(entries)
        rows = update.rows
        # Rows in the order the planner can use: decode entries sharing leading blocks together
        # (validation above ran in batch order, so errors name the reference's entry). Only a
        # batch where two decode entries start in the same block can have such entries; the
        # order is read from the arena's rows, which hold every table as int32 by now.
        order = None
        if repeats:
            if self._order.size < len(entries):
                self._order = np.zeros(max(len(entries), 2 * self._order.size), np.int64)
            if self._host.prefix_order_rows(
                rows, lengths, self._tables.host, self._tables.held_lengths,
                -(-ops.MIN_SHARED_TOKENS // self.block_size), ops.MIN_SHARED_ROWS, self._order,
            ):  # fmt: skip
                order = self._order[: len(entries)]  # rewritten by the next call
        token_order = None
        if order is not None:
            if total == len(entries):  # one token per entry: tokens move as their entries do
                token_order = order
            else:  # entry order[r]'s tokens, consecutively: token j of run r is start + (j - run offset)
                starts, runs = (np.cumsum(lengths) - lengths)[order], lengths[order]
                token_order = np.repeat(starts - (np.cumsum(runs) - runs), runs) + np.arange(total)
            batch_slots = slots
            tokens, positions, slots = tokens[token_order], positions[token_order], slots[token_order]
            rope_positions = rope_positions[token_order]
            planner_row = np.empty(total, dtype=np.int64)  # batch token index -> planner token index
            planner_row[token_order] = np.arange(total)
            wanted = planner_row[wanted]
            rows, lengths, context = rows[order], lengths[order], context[order]
        # Context lengths by arena row; only the batch's rows are read (by the planner and the
        # kernels), so the buffer is kept between calls and only those rows are written.
        if self._contexts_by_row.size != self._tables.num_rows:
            self._contexts_by_row = np.zeros(self._tables.num_rows, dtype=np.int32)
        contexts_by_row = self._contexts_by_row
        contexts_by_row[rows] = context
        query_seq = rows if total == len(entries) else np.repeat(rows, lengths)
        query_pos = positions.astype(np.int32)
        plan_rows, plan_tiles, merge, partition, flags = self._planner.plan_views(
            query_seq, query_pos, self._tables.host, contexts_by_row, self.block_size, config.n_heads,
            config.head_dim, self.partition_size, kv_dtype=self._keys.dtype,
        )  # fmt: skip
        self._last_plan = (plan_rows, plan_tiles, partition, flags, merge)
        parts64 = [tokens, rope_positions, slots, update.index, wanted]
        parts32 = [query_pos, query_seq, contexts_by_row, update.values, plan_rows.ravel(), plan_tiles.ravel(), merge]
        if token_order is not None:  # attend's caller rows, and its slots in batch order
            parts64.append(batch_slots)
            parts32.append(token_order.astype(np.int32))
        offsets = self._staging.send(parts64, parts32)
        tokens_at, rope_at, slots_at, index_at, logits_at = offsets[:5]
        qpos_at, qseq_at, context_at, values_at, rows_at, tiles_at, merge_at = offsets[len(parts64) : len(parts64) + 7]
        batch_slots_at, caller_rows_at = (offsets[5], offsets[-1]) if token_order is not None else (slots_at, -1)
        staging = self._staging
        if update.index.size:
            self._tables.apply(staging.tensor(index_at, update.index.size, torch.int64),
                               staging.tensor(values_at, update.values.size, torch.int32))  # fmt: skip
        else:
            self._tables.apply_nothing()
        # One token per entry: each is a decode row at its last position (context = position + 1).
        # Its append may ride inside the attention call only when no other row reads the block it
        # writes: the fused kernel hands a written key to its own row alone, while the reference
        # writes every slot before any attention (runner.py:195-212). A sequence twice in one
        # batch, or tables that share the block being written, take the append-then-attention
        # path. Tiles may stay: only the row pass appends, so no tile may cover a row's new
        # position, which exclusive_writes also checks (a decode batch's tiles are shared-prefix
        # tiles, and a written block that one row alone reads lies past every shared prefix).
        decode_only = len(entries) == total and self._host.exclusive_writes(
            rows, context, self._tables.host, self.block_size, self._marks, plan_tiles, partition
        )  # fmt: skip
        return _Step(
            total=total, staging=staging, tokens_at=tokens_at, rope_at=rope_at, slots_at=slots_at,
            logits_at=logits_at, qpos_at=qpos_at, qseq_at=qseq_at, contexts_at=context_at, plan_rows_at=rows_at,
            plan_tiles_at=tiles_at, merge_at=merge_at, num_plan_rows=plan_rows.shape[0],
            num_tiles=plan_tiles.shape[0], num_merge=merge.size, num_wanted=wanted.size, partition=partition,
            flags=flags, max_context=high_ctx, token_order=token_order, caller_rows_at=caller_rows_at,
            batch_slots_at=batch_slots_at, entries=entries, decode_only=decode_only,
        )  # fmt: skip

    def _attention(self, step: _Step, layer: int, queries: torch.Tensor, out: torch.Tensor, append=None) -> None:
        """Paged attention of one layer's rotated queries over the pools (and the decode append
        fused into it when ``append`` = (keys, values) rows is given), called through
        ``_pkvhost`` with the metadata's device addresses. ``queries``, ``out`` and the appended
        rows are in batch order: when the plan orders the rows its own way, the call's
        caller_rows (the staged token order) maps each planner row to its batch row."""
        config = self.model.config
        heads, dim = config.n_heads, config.head_dim
        # pkv_attention_workspace_bytes: (head_dim + 2) floats per (query, head, partition) once a
        # context can span more than one partition.
        part = step.partition or 512  # 0: the library's default
        parts = -(-step.max_context // part) if step.max_context > part else 1
        need = 0 if parts == 1 else step.total * heads * parts * (dim + 2) * 4
        workspace = self._workspace
        if workspace is None or workspace.numel() * 4 < need:
            workspace = self._workspace = torch.empty(max(need // 4, 1), dtype=torch.float32, device=self.device)
        if step.num_plan_rows == 0 and step.num_tiles == 0:
            return
        pools = self._keys
        key_at = pools.data_ptr() + layer * self._layer_bytes
        value_at = self._values.data_ptr() + layer * self._layer_bytes
        tables = self._tables.tables
        device = self._device_index
        stream = ops._stream(device)
        common = (
            out.data_ptr(), queries.data_ptr(), queries.stride(0), step.ptr(step.qpos_at), step.ptr(step.qseq_at),
            step.total, step.ptr(step.caller_rows_at) if step.caller_rows_at >= 0 else 0,
            step.ptr(step.plan_rows_at) if step.num_plan_rows else 0, step.num_plan_rows,
        )  # fmt: skip
        tail = (
            step.ptr(step.merge_at) if step.num_merge else 0, step.num_merge, key_at, value_at, self._kv_code,
            self.num_blocks, self.block_size, tables.data_ptr(), tables.shape[1], step.ptr(step.contexts_at),
            tables.shape[0], heads, dim,
            float(self.model.attention_scale), step.max_context, step.partition, step.flags, workspace.data_ptr(),
            workspace.numel() * 4,
        )  # fmt: skip
        if append is None:
            rc = self._host.paged_attention(*common, step.ptr(step.plan_tiles_at) if step.num_tiles else 0,
                                            step.num_tiles, *tail, device, stream)  # fmt: skip
            _native.check(rc, "pkv_paged_attention")
            return
        keys, values = append
        rc = self._host.paged_attention_append(
            *common, step.ptr(step.plan_tiles_at) if step.num_tiles else 0, step.num_tiles, *tail, keys.data_ptr(),
            values.data_ptr(), ops.kv_dtype_code(keys.dtype), keys.stride(0),
            values.stride(0), step.ptr(step.batch_slots_at), device, stream,
        )  # fmt: skip
        _native.check(rc, "pkv_paged_attention_append")

    def attend(
        self, batch: ExecutionBatch, queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
        *, layer: int = 0, out: torch.Tensor | None = None,
    ) -> torch.Tensor:  # fmt: skip
        """The KV data path of one layer for caller-computed projections: the batch's keys and
        values (float32 ``[T, heads, head_dim]``, rotated already, in batch token order) are
        written at its slots and every query attends over its entry's block table
        (reference runner.py:184-212 for one layer). Returns float32 ``[T, heads, head_dim]`` in
        batch order, on the device (asynchronous). A decode batch (one token per entry, at its
        last position) appends inside the attention call."""
        config = self.model.config
        if not 0 <= layer < config.n_layers:
            raise IndexError(f"layer {layer} is outside the model's {config.n_layers} layers")
        step = self._prepare(batch, logits=False)
        total = 0 if step is None else step.total
        shape = (total, config.n_heads, config.head_dim)
        if out is None:
            out = torch.empty(shape, dtype=torch.float32, device=self.device)
        if step is None:
            return out
        index = self._device_index
        for name, tensor in (("queries", queries), ("keys", keys), ("values", values), ("out", out)):
            if tensor.dtype is not torch.float32 or tensor.shape != shape or tensor.get_device() != index:
                raise ValueError(f"{name} must be float32 {list(shape)} on the runner's device")
        if not out.is_contiguous():
            raise ValueError("out must be contiguous")
        queries, keys, values = (t if t.is_contiguous() else t.contiguous() for t in (queries, keys, values))
        # Everything stays in batch order: a plan in its own row order reaches the batch rows
        # through the call's caller_rows.
        self.last_append_fused = step.decode_only
        if step.decode_only:
            self._attention(step, layer, queries, out, append=(keys, values))
        else:  # pkv_append of the batch's keys and values at their slots, then the attention
            offset = layer * self._layer_bytes
            rc = self._host.append(
                self._keys.data_ptr() + offset, self._values.data_ptr() + offset, self._kv_code,
                self.capacity_tokens, keys.data_ptr(), values.data_ptr(), _native.PKV_F32, keys.stride(0),
                values.stride(0), step.ptr(step.batch_slots_at), total, config.n_heads, config.head_dim,
                self._device_index, ops._stream(self._device_index),
            )  # fmt: skip
            _native.check(rc, "pkv_append")
            self._attention(step, layer, queries, out)
        return out

    def _forward(self, batch: ExecutionBatch, *, greedy: bool = False):
        """The forward pass of one iteration: (seq ids of the entries that ask for logits, in
        batch order; their device logits [rows, vocab], or with ``greedy`` their argmax token ids,
        int32 [rows]). Both are views of buffers the next call rewrites.

        Every launch is enqueued by one C++ call (``_pkvhost.forward``): per layer RMSNorm with the
        residual add fused into it, the QKV product, RoPE + append, paged attention, the output,
        [gate | up] and down products (rocBLAS) and the SwiGLU gate; then the logits rows and
        their product with the tied embedding (model.py:243-264, runner.py:189-227)."""
        step = self._prepare(batch)
        if step is None:
            return [], None
        config = self.model.config
        total, wanted = step.total, step.num_wanted
        w = self._device_weights()
        d, ff, vocab = config.d_model, config.d_ff, config.vocab_size
        # One float32 workspace, sections 64-float aligned: hidden, normed, fused q|k|v, attended,
        # the residual delta, [gate | up], the gate product, the logits rows and their logits.
        sizes = (total * d, total * d, 3 * total * d, total * d, total * d, 2 * total * ff, total * ff,
                 wanted * d, wanted * vocab)  # fmt: skip
        offsets, need = [], 0
        for size in sizes:
            offsets.append(need)
            need += -(-size // 64) * 64
        if self._forward_ws is None or self._forward_ws.numel() < need:
            self._forward_ws = torch.empty(max(need, 2 * (0 if self._forward_ws is None else self._forward_ws.numel())),
                                           dtype=torch.float32, device=self.device)  # fmt: skip
        if greedy and (self._greedy_out is None or self._greedy_out.numel() < wanted):
            self._greedy_out = torch.empty(max(wanted, 64), dtype=torch.int32, device=self.device)
        base = self._forward_ws.data_ptr()
        at = [base + 4 * o for o in offsets]
        heads, dim = config.n_heads, config.head_dim
        part = step.partition or 512  # 0: the library's default
        parts = -(-step.max_context // part) if step.max_context > part else 1
        ws_need = 0 if parts == 1 else total * heads * parts * (dim + 2) * 4
        workspace = self._workspace
        if workspace is None or workspace.numel() * 4 < ws_need:
            workspace = self._workspace = torch.empty(max(ws_need // 4, 1), dtype=torch.float32, device=self.device)
        tables = self._tables.tables
        fields = (
            self._device_index, ops._stream(self._device_index), total, wanted, d, heads, dim, ff, vocab,
            step.ptr(step.tokens_at), step.ptr(step.rope_at), step.ptr(step.slots_at), step.ptr(step.logits_at),
            w.embedding.data_ptr(), w.final_norm.data_ptr(), w.cos.data_ptr(), w.sin.data_ptr(), w.cos.shape[0],
            self._keys.data_ptr(), self._values.data_ptr(), self._layer_bytes, self._kv_code,
            self.num_blocks * self.block_size, *at,
            step.ptr(step.qpos_at), step.ptr(step.qseq_at),
            step.ptr(step.plan_rows_at) if step.num_plan_rows else 0, step.num_plan_rows,
            step.ptr(step.plan_tiles_at) if step.num_tiles else 0, step.num_tiles,
            step.ptr(step.merge_at) if step.num_merge else 0, step.num_merge,
            self.num_blocks, self.block_size, tables.data_ptr(), tables.shape[1], step.ptr(step.contexts_at),
            tables.shape[0], step.max_context, step.partition, step.flags, workspace.data_ptr(), workspace.numel() * 4,
            self._greedy_out.data_ptr() if greedy and wanted else 0,
        )  # fmt: skip
        self._host.forward(fields, w.addresses, float(config.norm_eps), float(self.model.attention_scale))
        if not wanted:
            return [], None
        names = [e.seq_id for e in step.entries if e.logits_index is not None]  # batch order
        if greedy:
            return names, self._greedy_out[:wanted]
        return names, self._forward_ws[offsets[-1] : offsets[-1] + wanted * vocab].view(wanted, vocab)
