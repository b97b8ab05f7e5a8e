"""Per-sequence block tables, prefix reuse and copy-on-write, with the reference's API.

Mirrors src/paged_kv_serving/engine/kvcache.py:27-211. ``reserve`` is all-or-nothing: it counts
the shared blocks in the write range ``[num_computed // B, ceil(up_to / B))`` plus the missing
blocks, evicts cached blocks if the free list is short, raises before mutating anything when the
pool still cannot cover the request, then copies-on-write the shared blocks in index order and
finally appends the new blocks -- the order that determines every block id, so block tables
agree with the reference's for the same call sequence.
"""

from __future__ import annotations

from dataclasses import dataclass

from paged_kv_serving_amd.blocks import BlockAllocationError, BlockManager, InvariantError
from paged_kv_serving_amd.prefix_cache import PrefixCache, chain_seed, next_block_hash

__all__ = ["KVCacheManager", "PrefixReuse"]


@dataclass(frozen=True)
class PrefixReuse:
    blocks: int
    tokens: int
    queried_blocks: int


class KVCacheManager:
    """Block tables, prefix reuse and eviction for every live sequence."""

    def __init__(self, blocks: BlockManager, prefix_cache: PrefixCache) -> None:
        self.blocks = blocks
        self.prefix_cache = prefix_cache
        self.block_size = blocks.block_size

    @property
    def num_free_blocks(self) -> int:
        return self.blocks.num_free_blocks

    @property
    def utilization(self) -> float:
        return self.blocks.utilization

    def evictable_blocks(self) -> int:
        """Cached blocks that only the cache references (kvcache.py:56-62)."""
        return sum(1 for b in self.prefix_cache.cached_block_ids() if self.blocks.ref_count(b) == 1)

    def blocks_required(self, sequence, up_to_tokens: int) -> int:
        needed = -(-up_to_tokens // self.block_size)
        return max(0, needed - len(sequence.block_table))

    def can_reserve(self, count: int) -> bool:
        return count <= self.blocks.num_free_blocks + self.evictable_blocks()

    def attach_prefix(self, sequence, *, record: bool = True) -> PrefixReuse:
        """Adopt cached blocks for the longest matching prefix, leaving at least one token to
        compute (kvcache.py:75-107)."""
        if sequence.num_computed_tokens or sequence.block_table:
            raise InvariantError("attach_prefix runs before any block is allocated")
        if not self.prefix_cache.enabled:
            return PrefixReuse(0, 0, 0)
        reusable = (sequence.num_tokens - 1) // self.block_size
        if reusable < 1:
            return PrefixReuse(0, 0, 0)
        parent = chain_seed(self.prefix_cache.scope_bytes(sequence.request.key_id))
        hashes = []
        size = self.block_size
        for i in range(reusable):
            parent = next_block_hash(parent, sequence.token_ids[i * size : (i + 1) * size], size)
            hashes.append(parent)
        matched = self.prefix_cache.lookup(hashes, record=record)
        sequence.block_table.extend(matched)
        sequence.block_hashes.extend(hashes[: len(matched)])
        sequence.cached_prefix_blocks = len(matched)
        sequence.num_computed_tokens = len(matched) * size
        return PrefixReuse(len(matched), len(matched) * size, reusable)

    def record_prefix(self, reuse: PrefixReuse) -> None:
        self.prefix_cache.record_lookup(reuse.queried_blocks, reuse.blocks)

    def detach_prefix(self, sequence) -> None:
        if sequence.num_computed_tokens != len(sequence.block_table) * self.block_size:
            raise InvariantError("only a freshly attached prefix can be detached")
        self.free(sequence)
        sequence.num_computed_tokens = 0

    def publish_full_blocks(self, sequence) -> int:
        """Offer newly completed blocks to the prefix cache (kvcache.py:125-144)."""
        if not self.prefix_cache.enabled:
            return 0
        complete = sequence.num_computed_tokens // self.block_size
        scope = self.prefix_cache.scope_bytes(sequence.request.key_id)
        size = self.block_size
        published = 0
        while len(sequence.block_hashes) < complete:
            i = len(sequence.block_hashes)
            parent = sequence.block_hashes[-1] if sequence.block_hashes else chain_seed(scope)
            block_hash = next_block_hash(parent, sequence.token_ids[i * size : (i + 1) * size], size)
            sequence.block_hashes.append(block_hash)
            if self.prefix_cache.register(block_hash, sequence.block_table[i]):
                published += 1
        return published

    def reserve(self, sequence, up_to_tokens: int) -> None:
        """Make positions ``[num_computed_tokens, up_to_tokens)`` writable (kvcache.py:148-180)."""
        if up_to_tokens > sequence.num_tokens:
            raise ValueError("cannot reserve beyond the tokens the sequence has")
        table = sequence.block_table
        extra = self.blocks_required(sequence, up_to_tokens)
        first = sequence.num_computed_tokens // self.block_size
        last = min(-(-up_to_tokens // self.block_size), len(table))
        shared = [i for i in range(first, last) if self.blocks.ref_count(table[i]) > 1]
        needed = extra + len(shared)
        if needed:
            self.prefix_cache.evict_until_free(needed)
            free = self.blocks.num_free_blocks
            if free < needed:
                raise BlockAllocationError(f"need {needed} blocks, {free} free")
        for i in shared:
            table[i] = self.blocks.prepare_for_write(table[i])
        if extra:
            table.extend(self.blocks.allocate_many(extra))

    def fork(self, parent, child) -> None:
        """Share the parent's blocks with the child by reference (kvcache.py:182-195)."""
        if child.block_table:
            raise InvariantError("fork target already owns blocks")
        for block_id in parent.block_table:
            self.blocks.incref(block_id)
        child.block_table.extend(parent.block_table)
        child.block_hashes.extend(parent.block_hashes)
        child.num_computed_tokens = parent.num_computed_tokens
        child.cached_prefix_blocks = parent.cached_prefix_blocks

    def free(self, sequence) -> int:
        count = len(sequence.block_table)
        self.blocks.free_many(sequence.block_table)
        sequence.block_table.clear()
        sequence.block_hashes.clear()
        sequence.cached_prefix_blocks = 0
        return count

    def check_invariants(self) -> None:
        self.blocks.check_invariants()
        for block_id in self.prefix_cache.cached_block_ids():
            if self.blocks.ref_count(block_id) < 1:
                raise InvariantError(f"cached block {block_id} has no reference")
