"""Host-side memory management: BlockManager, KVCacheManager and PrefixCache.

These are the integer half of the data path: they decide every block id a table holds and every
copy-on-write pair the GPU executes. The assertions are the known answers of the reference's own
tests (tests/unit/test_blocks.py, test_kvcache.py, test_prefix_cache.py), run against this
package's implementation: exact copy pair lists, exact reference counts, FIFO reuse order and
all-or-nothing reservations. Block-table bit-exactness follows from matching them call for call.
"""

from __future__ import annotations

import pytest

from paged_kv_serving_amd.blocks import (
    BlockAllocationError,
    BlockManager,
    BlockStore,
    InvariantError,
    RecordingBlockStore,
)
from paged_kv_serving_amd.kvcache import KVCacheManager
from paged_kv_serving_amd.prefix_cache import (
    PrefixCache,
    block_hash_chain,
    chain_seed,
    next_block_hash,
)
from paged_kv_serving_amd.sequence import Request, Sequence

# --- BlockManager (reference tests/unit/test_blocks.py) -------------------------------------


def manager(num_blocks: int = 8, block_size: int = 4):
    store = RecordingBlockStore()
    return BlockManager(num_blocks=num_blocks, block_size=block_size, store=store), store


def test_reference_counting_returns_blocks_to_the_free_list() -> None:
    blocks, _ = manager()
    first = blocks.allocate()
    assert blocks.ref_count(first) == 1 and blocks.num_free_blocks == 7
    blocks.incref(first)
    assert blocks.ref_count(first) == 2
    assert blocks.free(first) == 1 and blocks.num_free_blocks == 7
    assert blocks.free(first) == 0 and blocks.num_free_blocks == 8
    blocks.check_invariants()


def test_allocation_is_fifo_and_a_freed_block_goes_to_the_back() -> None:
    blocks, _ = manager(num_blocks=4)
    assert [blocks.allocate() for _ in range(3)] == [0, 1, 2]
    blocks.free(1)
    assert blocks.allocate() == 3
    assert blocks.allocate() == 1


def test_allocate_many_is_all_or_nothing() -> None:
    blocks, _ = manager(num_blocks=4)
    with pytest.raises(BlockAllocationError, match="need 5 blocks"):
        blocks.allocate_many(5)
    assert blocks.num_free_blocks == 4
    assert len(blocks.allocate_many(4)) == 4
    with pytest.raises(BlockAllocationError):
        blocks.allocate()
    with pytest.raises(ValueError, match="count must be"):
        blocks.allocate_many(-1)
    assert blocks.allocate_many(0) == []


def test_copy_on_write_gives_the_writer_a_private_block() -> None:
    blocks, store = manager()
    shared = blocks.allocate()
    blocks.incref(shared)
    private = blocks.prepare_for_write(shared)
    assert private != shared
    assert store.copies == [(shared, private)]
    assert blocks.ref_count(shared) == 1 and blocks.ref_count(private) == 1
    blocks.check_invariants()


def test_an_unshared_block_is_written_in_place() -> None:
    blocks, store = manager()
    block = blocks.allocate()
    assert blocks.prepare_for_write(block) == block
    assert store.copies == []


def test_a_three_way_share_costs_one_copy_per_writer_but_the_last() -> None:
    blocks, store = manager()
    shared = blocks.allocate()
    blocks.incref(shared)
    blocks.incref(shared)
    first, second, third = (blocks.prepare_for_write(shared) for _ in range(3))
    assert third == shared
    assert len({first, second, third}) == 3
    assert store.copies == [(shared, first), (shared, second)]
    blocks.check_invariants()


def test_double_free_and_out_of_range_ids_are_refused() -> None:
    blocks, _ = manager()
    block = blocks.allocate()
    blocks.free(block)
    with pytest.raises(InvariantError, match="freed twice"):
        blocks.free(block)
    with pytest.raises(InvariantError, match="outside the pool"):
        blocks.ref_count(99)
    with pytest.raises(InvariantError, match="cannot gain a reference"):
        blocks.incref(block)
    with pytest.raises(InvariantError, match="cannot be written"):
        blocks.prepare_for_write(block)


def test_invariant_check_detects_a_corrupted_free_list() -> None:
    blocks, _ = manager(num_blocks=4)
    block = blocks.allocate()
    blocks._push(block)  # a held block back on the free ring
    with pytest.raises(InvariantError, match="owners but is on the free ring"):
        blocks.check_invariants()


def test_runs_of_blocks_take_the_vector_path_with_the_same_order() -> None:
    """allocate_many / free_many of many ids (one slice of the ring, one gather) hand out and
    take back ids in exactly the order one-at-a-time calls would, across the ring's wrap."""
    one, _ = manager(num_blocks=40)
    many, _ = manager(num_blocks=40)
    rng = __import__("numpy").random.default_rng(0)
    held_one, held_many = [], []
    for _ in range(30):
        take = int(rng.integers(0, 12))
        if take <= one.num_free_blocks:
            held_one.append([one.allocate() for _ in range(take)])
            held_many.append(many.allocate_many(take))
            assert held_one[-1] == held_many[-1]
        if held_one and rng.random() < 0.5:
            k = int(rng.integers(0, len(held_one)))
            for block in held_one.pop(k):
                one.free(block)
            many.free_many(held_many.pop(k))
        assert one.free_order() == many.free_order() and one.snapshot() == many.snapshot()
    many.check_invariants()


def test_free_many_fails_at_the_same_id_as_one_by_one() -> None:
    blocks, _ = manager(num_blocks=16)
    held = blocks.allocate_many(10)
    blocks.free(held[6])
    with pytest.raises(InvariantError, match=f"block {held[6]} was freed twice"):
        blocks.free_many(held)
    assert [blocks.ref_count(b) for b in held] == [0] * 7 + [1] * 3, "released up to the bad id"
    assert blocks.free_order()[-7:] == [held[6], *held[:6]]


def test_utilisation_and_snapshot() -> None:
    blocks, _ = manager(num_blocks=4)
    assert blocks.utilization == 0.0
    held = blocks.allocate_many(2)
    assert blocks.utilization == 0.5 and blocks.num_used_blocks == 2
    blocks.free_many(held)
    assert blocks.snapshot() == (0, 0, 0, 0)


@pytest.mark.parametrize(("num_blocks", "block_size"), [(0, 4), (4, 0)])
def test_degenerate_pools_are_refused(num_blocks: int, block_size: int) -> None:
    with pytest.raises(ValueError, match="must be >= 1"):
        BlockManager(num_blocks=num_blocks, block_size=block_size, store=RecordingBlockStore())


def test_recording_store_refuses_a_self_copy_and_satisfies_the_protocol() -> None:
    store = RecordingBlockStore()
    assert isinstance(store, BlockStore)
    with pytest.raises(InvariantError, match="onto itself"):
        store.copy_block(1, 1)


# --- KVCacheManager (reference tests/unit/test_kvcache.py) ----------------------------------

BLOCK = 4


def build(num_blocks: int = 16, *, prefix_cache: bool = True):
    store = RecordingBlockStore()
    blocks = BlockManager(num_blocks=num_blocks, block_size=BLOCK, store=store)
    return KVCacheManager(blocks, PrefixCache(blocks, enabled=prefix_cache)), store


def sequence(tokens, *, key: str = "tenant-a", index: int = 0) -> Sequence:
    return Sequence.from_request(Request(f"r{index}", tuple(tokens), key_id=key), 0)


def compute(cache: KVCacheManager, seq: Sequence, chunk: int) -> None:
    cache.reserve(seq, seq.num_computed_tokens + chunk)
    seq.num_computed_tokens += chunk
    cache.publish_full_blocks(seq)


def test_reserve_allocates_only_what_a_chunk_needs() -> None:
    cache, _ = build()
    seq = sequence(list(range(10)))
    compute(cache, seq, 4)
    assert seq.block_table == [0]
    compute(cache, seq, 5)
    assert seq.block_table == [0, 1, 2]
    assert cache.blocks_required(seq, 10) == 0
    cache.check_invariants()


def test_reserve_beyond_the_sequence_is_refused() -> None:
    cache, _ = build()
    with pytest.raises(ValueError, match="beyond the tokens"):
        cache.reserve(sequence([1, 2, 3]), 10)


def test_a_full_pool_raises_without_changing_the_table() -> None:
    cache, _ = build(num_blocks=2)
    seq = sequence(list(range(12)))
    with pytest.raises(BlockAllocationError):
        cache.reserve(seq, 12)
    assert seq.block_table == []
    cache.check_invariants()


def test_attach_prefix_reuses_published_blocks_and_leaves_a_token() -> None:
    cache, _ = build()
    first = sequence([1, 2, 3, 4, 5, 6, 7, 8])
    compute(cache, first, 8)
    assert len(cache.prefix_cache) == 2
    second = sequence([1, 2, 3, 4, 5, 6, 7, 8], index=1)
    reuse = cache.attach_prefix(second)
    assert (reuse.blocks, reuse.tokens) == (1, 4)
    assert second.num_computed_tokens == 4
    assert second.block_table == first.block_table[:1]
    assert cache.blocks.ref_count(first.block_table[0]) == 3


def test_prefix_reuse_is_scoped_to_the_calling_key() -> None:
    cache, _ = build()
    compute(cache, sequence([1, 2, 3, 4, 5, 6], key="tenant-a"), 6)
    assert cache.attach_prefix(sequence([1, 2, 3, 4, 5, 6], key="tenant-b", index=1)).blocks == 0
    assert cache.attach_prefix(sequence([1, 2, 3, 4, 5, 6], key="tenant-a", index=2)).blocks == 1


def test_attach_prefix_without_a_cache_or_a_full_block() -> None:
    disabled, _ = build(prefix_cache=False)
    assert disabled.attach_prefix(sequence(list(range(9)))).blocks == 0
    cache, _ = build()
    short = sequence([1, 2])
    assert cache.attach_prefix(short).blocks == 0
    compute(cache, short, 2)
    assert cache.publish_full_blocks(short) == 0
    with pytest.raises(InvariantError, match="before any block"):
        cache.attach_prefix(short)


def test_fork_shares_blocks_and_the_first_write_copies_only_the_partial_block() -> None:
    cache, store = build()
    parent = sequence([1, 2, 3, 4, 5, 6])
    compute(cache, parent, 6)
    partial = parent.block_table[1]
    child = sequence([1, 2, 3, 4, 5, 6], index=1)
    cache.fork(parent, child)
    assert child.block_table == parent.block_table
    assert cache.blocks.ref_count(partial) == 2 and store.copies == []
    child.token_ids.append(99)
    compute(cache, child, 1)
    assert child.block_table[1] != partial
    assert store.copies == [(partial, child.block_table[1])]
    assert parent.block_table[1] == partial
    assert child.block_table[0] == parent.block_table[0]
    cache.check_invariants()


def test_fork_into_an_owner_is_refused() -> None:
    cache, _ = build()
    parent = sequence([1, 2, 3, 4])
    compute(cache, parent, 4)
    child = sequence([1, 2, 3, 4], index=1)
    compute(cache, child, 4)
    with pytest.raises(InvariantError, match="already owns blocks"):
        cache.fork(parent, child)


def test_free_keeps_the_caches_reference() -> None:
    cache, _ = build()
    seq = sequence([1, 2, 3, 4, 5, 6, 7, 8])
    compute(cache, seq, 8)
    before = cache.num_free_blocks
    assert cache.free(seq) == 2 and seq.block_table == []
    assert cache.num_free_blocks == before
    assert cache.evictable_blocks() == 2
    assert cache.prefix_cache.flush() == 2
    assert cache.num_free_blocks == before + 2


def test_reserve_evicts_cached_blocks_under_pressure() -> None:
    cache, _ = build(num_blocks=4)
    first = sequence([1, 2, 3, 4, 5, 6, 7, 8])
    compute(cache, first, 8)
    cache.free(first)
    assert cache.num_free_blocks == 2
    hungry = sequence(list(range(16, 32)), index=1)
    cache.reserve(hungry, 16)
    assert len(hungry.block_table) == 4 and len(cache.prefix_cache) == 0
    cache.check_invariants()


def test_can_reserve_counts_evictable_blocks() -> None:
    cache, _ = build(num_blocks=4)
    seq = sequence([1, 2, 3, 4, 5, 6, 7, 8])
    compute(cache, seq, 8)
    cache.free(seq)
    assert cache.can_reserve(4) and not cache.can_reserve(5)
    assert 0.0 < cache.utilization <= 1.0


def test_a_cached_block_that_lost_its_reference_is_detected() -> None:
    cache, _ = build()
    seq = sequence([1, 2, 3, 4])
    compute(cache, seq, 4)
    cached = cache.prefix_cache.cached_block_ids()[0]
    cache.free(seq)
    cache.blocks.free(cached)
    with pytest.raises(InvariantError, match="has no reference"):
        cache.check_invariants()


def test_copy_and_growth_are_all_or_nothing_together() -> None:
    cache, store = build(num_blocks=3)
    parent = sequence([1, 2, 3, 4, 5, 6])
    compute(cache, parent, 6)
    child = sequence([1, 2, 3, 4, 5, 6], index=1)
    cache.fork(parent, child)
    child.token_ids.extend([7, 8, 9])
    table, refs = list(child.block_table), cache.blocks.snapshot()
    with pytest.raises(BlockAllocationError):
        cache.reserve(child, 9)
    assert child.block_table == table and cache.blocks.snapshot() == refs and store.copies == []
    cache.check_invariants()


def test_a_shared_partial_block_is_copied_before_the_first_write() -> None:
    cache, store = build(num_blocks=8)
    parent = sequence([1, 2, 3, 4, 5, 6])
    compute(cache, parent, 6)
    child = sequence([1, 2, 3, 4, 5, 6], index=1)
    cache.fork(parent, child)
    child.token_ids.extend([7, 8, 9])
    cache.reserve(child, 9)
    assert child.block_table[0] == parent.block_table[0]
    assert child.block_table[1] != parent.block_table[1]
    assert store.copies == [(parent.block_table[1], child.block_table[1])]
    assert len(child.block_table) == 3
    cache.check_invariants()


def test_detach_prefix_returns_the_matched_blocks() -> None:
    cache, _ = build()
    compute(cache, sequence([1, 2, 3, 4, 5, 6, 7, 8, 9]), 9)
    waiter = sequence([1, 2, 3, 4, 5, 6, 7, 8, 9], index=1)
    reuse = cache.attach_prefix(waiter, record=False)
    assert reuse.blocks == 2 and cache.prefix_cache.stats.queried_blocks == 0
    cache.detach_prefix(waiter)
    assert waiter.block_table == [] and waiter.num_computed_tokens == 0
    cache.record_prefix(reuse)
    assert cache.prefix_cache.stats.hit_blocks == 2
    cache.check_invariants()


# --- PrefixCache (reference tests/unit/test_prefix_cache.py) --------------------------------


def prefix(num_blocks: int = 8, scope: str = "per_key"):
    blocks = BlockManager(num_blocks=num_blocks, block_size=4, store=RecordingBlockStore())
    return PrefixCache(blocks, scope=scope), blocks


def test_the_chain_commits_to_the_whole_history() -> None:
    first = block_hash_chain([1, 1, 1, 1, 9, 9, 9, 9], block_size=4, num_blocks=2)
    second = block_hash_chain([2, 2, 2, 2, 9, 9, 9, 9], block_size=4, num_blocks=2)
    assert first[0] != second[0] and first[1] != second[1]
    assert first == block_hash_chain([1, 1, 1, 1, 9, 9, 9, 9], block_size=4, num_blocks=2)
    a = block_hash_chain([3] * 4, block_size=4, num_blocks=1, scope=b"tenant-a")
    assert a != block_hash_chain([3] * 4, block_size=4, num_blocks=1, scope=b"tenant-b")


def test_the_hash_bytes_follow_the_documented_format() -> None:
    """h0 = BLAKE2b-16(domain|scope); h1 = BLAKE2b-16(h0 + u32 block_size + u32 tokens)."""
    import hashlib
    import struct

    seed = hashlib.blake2b(b"paged-kv-serving/prefix-v1|t", digest_size=16).digest()
    assert chain_seed(b"t") == seed
    body = seed + struct.pack("<I", 4) + struct.pack("<4I", 5, 6, 7, 8)
    assert next_block_hash(seed, [5, 6, 7, 8], 4) == hashlib.blake2b(body, digest_size=16).digest()


def test_hash_chain_argument_validation() -> None:
    with pytest.raises(ValueError, match="block_size must be"):
        block_hash_chain([1], block_size=0, num_blocks=0)
    with pytest.raises(ValueError, match="num_blocks must be"):
        block_hash_chain([1], block_size=1, num_blocks=-1)
    with pytest.raises(ValueError, match="not enough tokens"):
        block_hash_chain([1, 2], block_size=4, num_blocks=1)
    with pytest.raises(ValueError, match="only full blocks"):
        next_block_hash(chain_seed(), [1, 2], 4)


def test_lookup_stops_at_the_first_miss() -> None:
    cache, blocks = prefix()
    hashes = block_hash_chain([1] * 4 + [2] * 4 + [3] * 4, block_size=4, num_blocks=3)
    first, second = blocks.allocate(), blocks.allocate()
    assert cache.register(hashes[0], first) and cache.register(hashes[2], second)
    assert cache.lookup(hashes) == [first]
    assert blocks.ref_count(first) == 3


def test_registering_a_hash_twice_keeps_the_first_block() -> None:
    cache, blocks = prefix()
    hashes = block_hash_chain([7] * 4, block_size=4, num_blocks=1)
    first, second = blocks.allocate(), blocks.allocate()
    assert cache.register(hashes[0], first)
    assert not cache.register(hashes[0], second)
    assert cache.cached_block_ids() == (first,)


def test_eviction_is_lru_and_skips_blocks_in_use() -> None:
    cache, blocks = prefix()
    ids, hashes = [], []
    for value in range(3):
        block = blocks.allocate()
        block_hash = block_hash_chain([value] * 4, block_size=4, num_blocks=1)[0]
        cache.register(block_hash, block)
        blocks.free(block)
        ids.append(block)
        hashes.append(block_hash)
    cache.lookup([hashes[0]])
    assert cache.evict(1) == 1
    assert ids[0] in cache.cached_block_ids() and ids[1] not in cache.cached_block_ids()
    assert cache.evict(5) == 1
    assert cache.cached_block_ids() == (ids[0],)
    blocks.free(ids[0])
    assert cache.evict(1) == 1 and cache.cached_block_ids() == ()


def test_evict_until_free_releases_only_what_is_needed() -> None:
    cache, blocks = prefix(num_blocks=4)
    for i, block in enumerate(blocks.allocate_many(2)):
        cache.register(block_hash_chain([i] * 4, block_size=4, num_blocks=1)[0], block)
        blocks.free(block)
    assert cache.evict_until_free(3) == 1 and blocks.num_free_blocks == 3
    assert cache.evict_until_free(1) == 0 and cache.evict(0) == 0


def test_a_disabled_cache_never_hits_or_registers() -> None:
    cache, blocks = prefix()
    cache.enabled = False
    hashes = block_hash_chain([1] * 4, block_size=4, num_blocks=1)
    assert not cache.register(hashes[0], blocks.allocate())
    assert cache.lookup(hashes) == []
    assert cache.stats.queried_blocks == 1 and cache.stats.hit_ratio == 0.0


def test_statistics_and_flush() -> None:
    cache, blocks = prefix()
    hashes = block_hash_chain([1] * 4 + [2] * 4, block_size=4, num_blocks=2)
    for block_hash in hashes:
        block = blocks.allocate()
        cache.register(block_hash, block)
        blocks.free(block)
    assert cache.lookup(hashes) == list(cache.cached_block_ids())
    assert cache.stats.hit_ratio == 1.0
    assert cache.lookup(block_hash_chain([9] * 8, block_size=4, num_blocks=2)) == []
    assert cache.stats.hit_ratio == 0.5
    for block in cache.cached_block_ids():
        blocks.free(block)
    assert cache.flush() == 2 and len(cache) == 0
    stats = cache.stats.as_dict()
    assert stats["registered_blocks"] == 2 and stats["evicted_blocks"] == 2


def test_scope_bytes() -> None:
    per_key, _ = prefix()
    shared, _ = prefix(scope="global")
    assert per_key.scope_bytes("alice") != per_key.scope_bytes("bob")
    assert shared.scope_bytes("alice") == shared.scope_bytes("bob")


def test_shared_positions_reads_short_and_long_stretches_alike() -> None:
    """BlockManager.shared_positions (reserve's check for blocks it must copy before writing):
    the scalar read of a few entries and the NumPy gather of a long stretch give the same
    indices, and an id outside the pool is an InvariantError on both paths."""
    import random

    from paged_kv_serving_amd.blocks import BlockManager, InvariantError, RecordingBlockStore

    rng = random.Random(3)
    pool = BlockManager(num_blocks=64, block_size=4, store=RecordingBlockStore())
    ids = pool.allocate_many(40)
    for block in rng.sample(ids, 15):
        pool.incref(block)
    table = [rng.choice(ids) for _ in range(30)]
    want = [i for i, b in enumerate(table) if pool.ref_count(b) > 1]
    for lo, hi in ((0, 30), (3, 9), (5, 6), (10, 30), (29, 30)):
        assert pool.shared_positions(table, lo, hi) == [i for i in want if lo <= i < hi], (lo, hi)
    for bad, hi in ((64, 2), (-1, 20)):
        with pytest.raises(InvariantError, match="outside the pool"):
            pool.shared_positions([ids[0], bad] + ids[:18], 0, hi)
