"""Seeded synthetic batches for the data-path configurations (BASELINE.json ``configs``).

Host-side randomness (context lengths, offsets, block-table permutations) comes from one
``np.random.default_rng(seed)``, so block tables and slot mappings are reproducible and can be
recomputed exactly on the CPU; the bulk N(0, 1) data (pools, queries, new keys and values) is
drawn on the device from a seeded ``torch.Generator``, so a 20-40k-block pool never crosses
PCIe. ``host_rows`` copies back only the blocks of chosen sequences, for the CPU oracle.

Every batch follows the engine's order: the query tokens' new keys and values are appended to
their slots first (reference runner.py:195-196), then every query attends over its sequence's
first ``min(context_len, position + 1)`` keys (runner.py:198-212).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from paged_kv_serving_amd import ops

__all__ = [
    "AttentionBatch",
    "PrefixSharingStep",
    "decode_batch",
    "long_context_batch",
    "mixed_batch",
    "prefix_sharing_step",
]


@dataclass
class AttentionBatch:
    """One layer's pools plus a ragged batch of queries, on the device, with host metadata."""

    key_cache: torch.Tensor  # [N, B, H, D]
    value_cache: torch.Tensor
    queries: torch.Tensor  # [T, H, D] float32
    new_keys: torch.Tensor  # [T, H, D] float32, appended at slot_mapping before attention
    new_values: torch.Tensor
    slot_mapping: torch.Tensor  # int64 [T]
    query_positions: torch.Tensor  # int32 [T]
    query_seq: torch.Tensor  # int32 [T]
    block_tables: torch.Tensor  # int32 [S, W]
    context_lens: torch.Tensor  # int32 [S]
    max_context_len: int
    scale: float
    plan: ops.AttentionPlan | None = None  # prefill runs -> MFMA tiles, other rows -> row pass
    # Host copies of the integer metadata (bit-exact with the device tensors).
    host_tables: list[np.ndarray] = field(default_factory=list)
    host_context: np.ndarray | None = None
    host_positions: np.ndarray | None = None
    host_seq: np.ndarray | None = None
    host_slots: np.ndarray | None = None

    @property
    def num_queries(self) -> int:
        return int(self.queries.shape[0])

    def replan(self, partition_size: int) -> None:
        """Rebuild the plan for a given partition size (0: the planner's choice)."""
        heads, dim = self.key_cache.shape[2], self.key_cache.shape[3]
        host = ops.plan_batch_native(
            self.host_seq, dim, heads, self.host_tables, self.host_context, self.key_cache.shape[1],
            partition_size=partition_size, query_positions=self.host_positions, kv_dtype=self.key_cache.dtype,
        )  # fmt: skip
        self.plan = ops.upload_batch_plan(host, self.queries.device)

    @property
    def num_seqs(self) -> int:
        return int(self.context_lens.shape[0])

    def decode_rows_only(self) -> bool:
        """One query row per sequence, each at its sequence's last position: the decode shape
        whose append can ride in the attention call (pkv_paged_attention_append)."""
        seq = self.host_seq
        if seq is None or np.unique(seq).size != seq.size:
            return False
        return bool(np.all(self.host_positions == self.host_context[seq] - 1))

    def fusable_append(self) -> bool:
        """Whether the runner would fuse this batch's append into the attention call: the
        decode shape, each written block read by its own row alone, and no tile of the plan over
        a written position (the rule of ModelRunner's exclusive_writes check)."""
        if not self.decode_rows_only():
            return False
        block = self.key_cache.shape[1]
        tables = [np.asarray(self.host_tables[s]) for s in self.host_seq]
        contexts = self.host_context[self.host_seq]
        visible = np.concatenate([t[: -(-int(c) // block)] for t, c in zip(tables, contexts)])
        written = np.asarray([t[(int(c) - 1) // block] for t, c in zip(tables, contexts)])
        counts = dict(zip(*np.unique(visible, return_counts=True)))
        if any(counts.get(int(w), 0) != 1 for w in written):
            return False
        tiles = self.plan.tiles.cpu().numpy() if self.plan.num_tiles else np.zeros((0, 4), np.int32)
        part = self.plan.partition_size or 512
        own = contexts - 1
        for first, count, begin, end in tiles.tolist():
            lo = 0 if end == -1 else begin * part
            hi = np.inf if end == -1 or end <= begin else end * part
            if np.any((own[first : first + count] >= lo) & (own[first : first + count] < hi)):
                return False
        return True

    def context_bytes(self) -> int:
        """Algorithmic K+V bytes: each query row's visible keys and values, read once."""
        heads, dim = self.key_cache.shape[2], self.key_cache.shape[3]
        per_token = 2 * heads * dim * self.key_cache.element_size()
        visible = 0
        for s, ctx in enumerate(self.host_context):
            rows = self.host_positions[self.host_seq == s]
            # a sequence's rows share its key range; the union is read once per sequence
            visible += int(min(int(ctx), int(rows.max()) + 1)) if rows.size else 0
        return visible * per_token

    def host_rows(self, seq: int) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
        """(keys, values, queries, positions) of one sequence on the host, keys/values in
        logical order ``(ctx, H, D)`` as float32, after the append."""
        table = torch.from_numpy(self.host_tables[seq].astype(np.int64)).to(self.key_cache.device)
        ctx = int(self.host_context[seq])
        keys = self.key_cache[table].reshape(-1, *self.key_cache.shape[2:])[:ctx]
        values = self.value_cache[table].reshape(-1, *self.value_cache.shape[2:])[:ctx]
        rows = np.nonzero(self.host_seq == seq)[0]
        q = self.queries[torch.from_numpy(rows).to(self.queries.device)]
        return (
            keys.float().cpu().numpy(),
            values.float().cpu().numpy(),
            q.cpu().numpy(),
            self.host_positions[rows],
        )


def _tables_from_permutation(
    rng: np.random.Generator, num_blocks: int, blocks_per_seq: list[int]
) -> list[np.ndarray]:
    perm = rng.permutation(num_blocks)
    if sum(blocks_per_seq) > num_blocks:
        raise ValueError("the pool is too small for the requested contexts")
    tables, offset = [], 0
    for count in blocks_per_seq:
        tables.append(perm[offset : offset + count].astype(np.int32))
        offset += count
    return tables


def _assemble(
    *,
    rng_device: torch.Generator,
    device: torch.device,
    num_blocks: int,
    block_size: int,
    heads: int,
    head_dim: int,
    kv_dtype: torch.dtype,
    tables: list[np.ndarray],
    context: np.ndarray,
    positions: np.ndarray,
    seq: np.ndarray,
) -> AttentionBatch:
    """Draw pools and query/new-token data on the device and package the batch."""
    shape = (num_blocks, block_size, heads, head_dim)
    key_cache = torch.empty(shape, dtype=kv_dtype, device=device)
    value_cache = torch.empty(shape, dtype=kv_dtype, device=device)
    # Fill in slabs so a bfloat16 pool never needs a float32 copy of itself.
    slab = max(1, (1 << 28) // (block_size * heads * head_dim))
    for cache in (key_cache, value_cache):
        for start in range(0, num_blocks, slab):
            part = cache[start : start + slab]
            part.copy_(torch.randn(part.shape, generator=rng_device, device=device, dtype=torch.float32))
    total = positions.size
    queries = torch.randn((total, heads, head_dim), generator=rng_device, device=device)
    new_keys = torch.randn((total, heads, head_dim), generator=rng_device, device=device)
    new_values = torch.randn((total, heads, head_dim), generator=rng_device, device=device)
    slots = np.empty(total, dtype=np.int64)
    for t in range(total):
        table = tables[int(seq[t])]
        p = int(positions[t])
        slots[t] = int(table[p // block_size]) * block_size + p % block_size
    width = max(len(t) for t in tables)
    padded = np.zeros((len(tables), width), dtype=np.int32)
    for i, table in enumerate(tables):
        padded[i, : len(table)] = table
    plan = ops.upload_batch_plan(
        ops.plan_batch_native(seq, head_dim, heads, tables, context, block_size, query_positions=positions,
                              kv_dtype=kv_dtype),
        device,
    )  # fmt: skip
    return AttentionBatch(
        key_cache=key_cache,
        value_cache=value_cache,
        queries=queries,
        new_keys=new_keys,
        new_values=new_values,
        slot_mapping=torch.from_numpy(slots).to(device),
        query_positions=torch.from_numpy(positions.astype(np.int32)).to(device),
        query_seq=torch.from_numpy(seq.astype(np.int32)).to(device),
        block_tables=torch.from_numpy(padded).to(device),
        context_lens=torch.from_numpy(context.astype(np.int32)).to(device),
        max_context_len=int(context.max()),
        scale=float(head_dim) ** -0.5,
        plan=plan,
        host_tables=tables,
        host_context=context.astype(np.int64),
        host_positions=positions.astype(np.int64),
        host_seq=seq.astype(np.int64),
        host_slots=slots,
    )


def decode_batch(
    *,
    seed: int = 0,
    num_seqs: int = 64,
    context_low: int = 512,
    context_high: int = 4096,
    heads: int = 32,
    head_dim: int = 128,
    block_size: int = 16,
    num_blocks: int = 20_000,
    kv_dtype: torch.dtype = torch.float32,
    device: torch.device | str = "cuda",
) -> AttentionBatch:
    """Config 2: one decode row per sequence, contexts uniform in [low, high], tables drawn from
    a shuffled pool; the new token sits at position context - 1."""
    device = torch.device(device)
    rng = np.random.default_rng(seed)
    context = rng.integers(context_low, context_high + 1, num_seqs)
    tables = _tables_from_permutation(rng, num_blocks, [-(-int(c) // block_size) for c in context])
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    return _assemble(
        rng_device=gen, device=device, num_blocks=num_blocks, block_size=block_size, heads=heads,
        head_dim=head_dim, kv_dtype=kv_dtype, tables=tables, context=context,
        positions=context - 1, seq=np.arange(num_seqs),
    )  # fmt: skip


def mixed_batch(
    *,
    seed: int = 0,
    num_prefill: int = 8,
    chunk: int = 512,
    offset_high: int = 2048,
    num_decode: int = 120,
    decode_low: int = 256,
    decode_high: int = 4096,
    heads: int = 32,
    head_dim: int = 128,
    block_size: int = 16,
    num_blocks: int = 40_000,
    kv_dtype: torch.dtype = torch.float32,
    device: torch.device | str = "cuda",
) -> AttentionBatch:
    """Config 3: chunked-prefill rows (``chunk`` tokens from an existing offset, causal inside
    the chunk) followed by decode rows, in one ragged batch."""
    device = torch.device(device)
    rng = np.random.default_rng(seed)
    offsets = rng.integers(0, offset_high + 1, num_prefill)
    decode_ctx = rng.integers(decode_low, decode_high + 1, num_decode)
    context = np.concatenate([offsets + chunk, decode_ctx])
    tables = _tables_from_permutation(rng, num_blocks, [-(-int(c) // block_size) for c in context])
    positions = np.concatenate(
        [np.arange(o, o + chunk) for o in offsets] + [decode_ctx - 1]
    ).astype(np.int64)
    seq = np.concatenate(
        [np.full(chunk, i) for i in range(num_prefill)] + [np.arange(num_prefill, num_prefill + num_decode)]
    )
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    return _assemble(
        rng_device=gen, device=device, num_blocks=num_blocks, block_size=block_size, heads=heads,
        head_dim=head_dim, kv_dtype=kv_dtype, tables=tables, context=context,
        positions=positions, seq=seq,
    )  # fmt: skip


def long_context_batch(
    *,
    seed: int = 0,
    num_seqs: int = 16,
    context_len: int = 32_768,
    heads: int = 32,
    head_dim: int = 128,
    block_size: int = 16,
    num_blocks: int = 40_000,
    kv_dtype: torch.dtype = torch.bfloat16,
    device: torch.device | str = "cuda",
) -> AttentionBatch:
    """Config 5: decode rows at a long fixed context over a shuffled pool (bf16 KV)."""
    device = torch.device(device)
    rng = np.random.default_rng(seed)
    context = np.full(num_seqs, context_len, dtype=np.int64)
    tables = _tables_from_permutation(rng, num_blocks, [-(-context_len // block_size)] * num_seqs)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    return _assemble(
        rng_device=gen, device=device, num_blocks=num_blocks, block_size=block_size, heads=heads,
        head_dim=head_dim, kv_dtype=kv_dtype, tables=tables, context=context,
        positions=context - 1, seq=np.arange(num_seqs),
    )  # fmt: skip


@dataclass
class PrefixSharingStep:
    """Config 4: a shared prefix, one copy-on-write per sequence, then one decode step."""

    key_cache: torch.Tensor  # [1, N, B, H, D] (one layer, pools as copy_blocks expects)
    value_cache: torch.Tensor
    cow_pairs: torch.Tensor  # int64 [n, 2] (src, dst), in BlockManager order
    host_pairs: list[tuple[int, int]]
    decode: AttentionBatch  # views of the same pools (layer 0), one decode row per sequence
    shared_blocks: int
    prefix_tokens: int

    def cow_bytes(self) -> int:
        """Bytes one COW launch moves: each pair reads and writes a K and a V block."""
        block = self.key_cache[0, 0].numel() * self.key_cache.element_size()
        return 4 * block * len(self.host_pairs)

    def unique_context_bytes(self) -> int:
        """K+V bytes of distinct blocks the decode step reads (the shared prefix counted once)."""
        heads, dim = self.key_cache.shape[3], self.key_cache.shape[4]
        per_token = 2 * heads * dim * self.key_cache.element_size()
        shared = self.prefix_tokens - (self.prefix_tokens % self.key_cache.shape[2] or self.key_cache.shape[2])
        own = int(sum(int(c) - shared for c in self.decode.host_context))
        return (shared + own) * per_token


def prefix_sharing_step(
    *,
    seed: int = 0,
    num_seqs: int = 256,
    prefix_tokens: int = 1016,
    suffix_low: int = 32,
    suffix_high: int = 256,
    heads: int = 32,
    head_dim: int = 128,
    block_size: int = 16,
    num_blocks: int = 8192,
    device: torch.device | str = "cuda",
) -> PrefixSharingStep:
    """Config 4 through the host API: a parent prefills ``prefix_tokens`` (the last shared block
    is partial: 1016 = 63 x 16 + 8), ``num_seqs`` children fork from it while the parent keeps its
    reference, and each child reserves its suffix, so ``KVCacheManager.reserve`` copies-on-write
    the partial shared block once per child (reference kvcache.py:148-180, blocks.py:148-165).
    Suffix keys/values are then written (untimed set-up) and every child runs one decode token.
    """
    from paged_kv_serving_amd.blocks import BlockManager, RecordingBlockStore
    from paged_kv_serving_amd.kvcache import KVCacheManager
    from paged_kv_serving_amd.prefix_cache import PrefixCache
    from paged_kv_serving_amd.sequence import Request, Sequence

    device = torch.device(device)
    rng = np.random.default_rng(seed)
    store = RecordingBlockStore()
    blocks = BlockManager(num_blocks=num_blocks, block_size=block_size, store=store)
    cache = KVCacheManager(blocks, PrefixCache(blocks, enabled=False))
    prefix = [int(t) for t in rng.integers(0, 50_000, prefix_tokens)]
    parent = Sequence.from_request(Request("parent", tuple(prefix)), 0)
    cache.reserve(parent, prefix_tokens)
    parent.num_computed_tokens = prefix_tokens
    suffixes = rng.integers(suffix_low, suffix_high + 1, num_seqs)
    children = []
    for i in range(num_seqs):
        child = Sequence.from_request(Request(f"c{i}", tuple(prefix)), 0)
        cache.fork(parent, child)
        child.token_ids.extend(int(t) for t in rng.integers(0, 50_000, int(suffixes[i]) + 1))
        cache.reserve(child, prefix_tokens + int(suffixes[i]) + 1)  # suffix + the decode token
        children.append(child)
    pairs = list(store.copies)
    cache.check_invariants()

    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    shape = (1, num_blocks, block_size, heads, head_dim)
    key_cache = torch.randn(shape, generator=gen, device=device)
    value_cache = torch.randn(shape, generator=gen, device=device)
    contexts = prefix_tokens + suffixes + 1
    tables = [np.asarray(c.block_table, dtype=np.int32) for c in children]
    # Suffix rows (positions prefix .. ctx-2) get their own data; the pool's random fill stands
    # in for it, except that the COW destinations are overwritten by the timed copy.
    total = num_seqs
    width = max(len(t) for t in tables)
    padded = np.zeros((num_seqs, width), dtype=np.int32)
    for i, table in enumerate(tables):
        padded[i, : len(table)] = table
    positions = contexts - 1
    slots = np.asarray(
        [int(tables[i][p // block_size]) * block_size + p % block_size for i, p in enumerate(positions)],
        dtype=np.int64,
    )
    seq = np.arange(num_seqs)
    decode = AttentionBatch(
        key_cache=key_cache[0],
        value_cache=value_cache[0],
        queries=torch.randn((total, heads, head_dim), generator=gen, device=device),
        new_keys=torch.randn((total, heads, head_dim), generator=gen, device=device),
        new_values=torch.randn((total, heads, head_dim), generator=gen, device=device),
        slot_mapping=torch.from_numpy(slots).to(device),
        query_positions=torch.from_numpy(positions.astype(np.int32)).to(device),
        query_seq=torch.from_numpy(seq.astype(np.int32)).to(device),
        block_tables=torch.from_numpy(padded).to(device),
        context_lens=torch.from_numpy(contexts.astype(np.int32)).to(device),
        max_context_len=int(contexts.max()),
        scale=float(head_dim) ** -0.5,
        plan=ops.upload_batch_plan(
            ops.plan_batch_native(seq, head_dim, heads, tables, contexts, block_size, query_positions=positions), device
        ),
        host_tables=tables,
        host_context=contexts.astype(np.int64),
        host_positions=positions.astype(np.int64),
        host_seq=seq.astype(np.int64),
        host_slots=slots,
    )
    return PrefixSharingStep(
        key_cache=key_cache,
        value_cache=value_cache,
        cow_pairs=torch.tensor(pairs, dtype=torch.int64).to(device),
        host_pairs=pairs,
        decode=decode,
        shared_blocks=len(parent.block_table),
        prefix_tokens=prefix_tokens,
    )
