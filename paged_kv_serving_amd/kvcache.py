"""Sequence-level KV cache: block tables, prefix reuse, copy-on-write and release.

Interface (kept so the reference's Scheduler and Engine drive it unchanged,
src/paged_kv_serving/engine/kvcache.py:27-211): ``KVCacheManager`` with ``reserve / fork / free /
attach_prefix / detach_prefix / record_prefix / publish_full_blocks / blocks_required /
can_reserve / evictable_blocks / check_invariants``, the ``num_free_blocks`` and ``utilization``
properties, ``PrefixReuse``, and the reference's error types and messages. A sequence is any
object with ``token_ids``, ``block_table``, ``block_hashes``, ``num_computed_tokens``,
``cached_prefix_blocks``, ``num_tokens`` and ``request.key_id``, like the reference's
``Sequence``; this class is the only writer of the first five.

Behaviour that fixes every block id, and so is the reference's exactly:

* ``reserve(seq, up_to)`` touches the blocks that hold positions
  ``[num_computed_tokens, up_to)``. It first counts what it will need -- one block per shared
  block in that range (each gets a private copy) plus the blocks the table lacks -- evicts cached
  blocks if the pool is short, and raises before changing anything if it is still short. Then it
  copies the shared blocks, lowest index first, and appends the new blocks.
* ``attach_prefix`` adopts the longest cached run of the sequence's full blocks, always leaving
  at least one token to compute; ``publish_full_blocks`` registers each block as soon as the
  computed tokens cover it.
* ``fork`` shares every block of the parent by ownership, not by copy.

What is this module's own: the shared blocks of a write range are found with one gather of owner
counts over the range, the cache's evictable count with one gather over the cached ids, and a
prefix lookup hashes the chain only up to its first miss.
"""

from __future__ import annotations

from dataclasses import dataclass

from paged_kv_serving_amd.blocks import BlockAllocationError, BlockManager, InvariantError
from paged_kv_serving_amd.prefix_cache import PrefixCache, chain_seed, next_block_hash

__all__ = ["KVCacheManager", "PrefixReuse"]


@dataclass(frozen=True)
class PrefixReuse:
    """What a prefix lookup gave one sequence: blocks adopted, tokens they cover, blocks asked."""

    blocks: int
    tokens: int
    queried_blocks: int


_NO_REUSE = PrefixReuse(blocks=0, tokens=0, queried_blocks=0)


class KVCacheManager:
    """Block tables of every live sequence over one pool and one prefix cache."""

    def __init__(self, blocks: BlockManager, prefix_cache: PrefixCache) -> None:
        self.blocks = blocks
        self.prefix_cache = prefix_cache
        self.block_size = blocks.block_size

    # --- capacity ------------------------------------------------------------------------

    @property
    def num_free_blocks(self) -> int:
        return self.blocks.num_free_blocks

    @property
    def utilization(self) -> float:
        return self.blocks.utilization

    def evictable_blocks(self) -> int:
        """Cached blocks no sequence reads: what eviction could give back."""
        return self.prefix_cache.sole_owner_count()

    def blocks_required(self, sequence, up_to_tokens: int) -> int:
        """Blocks the table still lacks to hold ``up_to_tokens`` tokens."""
        have = len(sequence.block_table)
        want = -(-up_to_tokens // self.block_size)
        return want - have if want > have else 0

    def can_reserve(self, count: int) -> bool:
        return count <= self.blocks.num_free_blocks + self.evictable_blocks()

    # --- prefix reuse --------------------------------------------------------------------

    def _seed(self, sequence) -> bytes:
        return chain_seed(self.prefix_cache.scope_bytes(sequence.request.key_id))

    def attach_prefix(self, sequence, *, record: bool = True) -> PrefixReuse:
        """Adopt the cached blocks of the sequence's longest cached prefix of full blocks, short
        of its last token (which must run to give logits). ``record=False`` leaves the hit
        counters to :meth:`record_prefix` (or :meth:`detach_prefix` when not admitted)."""
        if sequence.num_computed_tokens or sequence.block_table:
            raise InvariantError("attach_prefix runs before any block is allocated")
        if not self.prefix_cache.enabled:
            return _NO_REUSE
        size = self.block_size
        candidates = (sequence.num_tokens - 1) // size
        if candidates < 1:
            return _NO_REUSE
        blocks, hashes = self.prefix_cache.match(
            self._seed(sequence), sequence.token_ids, size, candidates, record=record
        )
        adopted = len(blocks)
        sequence.block_table.extend(blocks)
        sequence.block_hashes.extend(hashes)
        sequence.cached_prefix_blocks = adopted
        sequence.num_computed_tokens = adopted * size
        return PrefixReuse(blocks=adopted, tokens=adopted * size, queried_blocks=candidates)

    def record_prefix(self, reuse: PrefixReuse) -> None:
        """Count an unrecorded :meth:`attach_prefix` in the hit counters."""
        self.prefix_cache.record_lookup(reuse.queried_blocks, reuse.blocks)

    def detach_prefix(self, sequence) -> None:
        """Give back what :meth:`attach_prefix` adopted, for a sequence that was not admitted."""
        if sequence.num_computed_tokens != len(sequence.block_table) * self.block_size:
            raise InvariantError("only a freshly attached prefix can be detached")
        self.free(sequence)
        sequence.num_computed_tokens = 0

    def publish_full_blocks(self, sequence) -> int:
        """Register every block the computed tokens now fill; returns how many were new to the
        cache. A block is hashed once: ``block_hashes`` holds the chain so far."""
        if not self.prefix_cache.enabled:
            return 0
        size = self.block_size
        full = sequence.num_computed_tokens // size
        hashes = sequence.block_hashes
        done = len(hashes)
        if done >= full:
            return 0
        parent = hashes[-1] if hashes else self._seed(sequence)
        table, tokens = sequence.block_table, sequence.token_ids
        new = 0
        for index in range(done, full):
            parent = next_block_hash(parent, tokens[index * size : (index + 1) * size], size)
            hashes.append(parent)
            new += self.prefix_cache.register(parent, table[index])
        return new

    # --- allocation ----------------------------------------------------------------------

    def reserve(self, sequence, up_to_tokens: int) -> None:
        """Make positions ``[num_computed_tokens, up_to_tokens)`` writable: private copies of the
        shared blocks among them, then new blocks for the rest. All or nothing: on
        :class:`BlockAllocationError` the table and every owner count are unchanged (cache
        entries evicted while trying stay evicted: no sequence was reading them)."""
        if up_to_tokens > sequence.num_tokens:
            raise ValueError("cannot reserve beyond the tokens the sequence has")
        size = self.block_size
        table = sequence.block_table
        grow = self.blocks_required(sequence, up_to_tokens)
        lo = sequence.num_computed_tokens // size
        hi = min(-(-up_to_tokens // size), len(table))
        shared = self.blocks.shared_positions(table, lo, hi) if hi > lo else []
        needed = grow + len(shared)
        if needed:
            self.prefix_cache.evict_until_free(needed)
            free = self.blocks.num_free_blocks
            if free < needed:
                raise BlockAllocationError(f"need {needed} blocks, {free} free")
        for index in shared:
            table[index] = self.blocks.prepare_for_write(table[index])
        if grow:
            table.extend(self.blocks.allocate_many(grow))

    def fork(self, parent, child) -> None:
        """Give ``child`` the parent's blocks by ownership; the first write to a shared block
        (through :meth:`reserve`) copies just that block."""
        if child.block_table:
            raise InvariantError("fork target already owns blocks")
        for block_id in parent.block_table:
            self.blocks.incref(block_id)
        child.block_table.extend(parent.block_table)
        child.block_hashes.extend(parent.block_hashes)
        child.num_computed_tokens = parent.num_computed_tokens
        child.cached_prefix_blocks = parent.cached_prefix_blocks

    def free(self, sequence) -> int:
        """Give back every block of the sequence; returns how many it held."""
        table = sequence.block_table
        held = len(table)
        self.blocks.free_many(table)
        table.clear()
        sequence.block_hashes.clear()
        sequence.cached_prefix_blocks = 0
        return held

    def check_invariants(self) -> None:
        """The pool's invariants, and every cached block still owned."""
        self.blocks.check_invariants()
        cached = self.prefix_cache.cached_block_ids()
        if cached:
            owners = self.blocks.counts_of(cached)
            if (owners < 1).any():
                block = cached[int((owners < 1).nonzero()[0][0])]
                raise InvariantError(f"cached block {block} has no reference")
