"""Stateful property test of the paged allocator, with a shadow store of token ids.

Follows the reference's tests/property/test_allocator_state.py: hypothesis drives this package's
KVCacheManager through interleavings of admit, prefill, decode, fork, preempt, finish and evict,
and after every step checks that

1. the allocator is consistent (free list, reference counts, totals);
2. every sequence reads back its own token at every computed position, through its block table
   and the slot formula -- this catches a missed copy-on-write or a block handed out twice;
3. a block registered in the prefix cache never changes;
4. nothing leaks once everything is freed and the cache is flushed.

The shadow store also replays every copy-on-write pair through ``independent_groups`` batching
(the GPU runner's flush), so the batched order is checked against the one-at-a-time order.
"""

from __future__ import annotations

import contextlib

from hypothesis import HealthCheck, settings
from hypothesis import strategies as st
from hypothesis.stateful import RuleBasedStateMachine, invariant, precondition, rule

from paged_kv_serving_amd.blocks import BlockAllocationError, BlockManager
from paged_kv_serving_amd.kvcache import KVCacheManager
from paged_kv_serving_amd.prefix_cache import PrefixCache
from paged_kv_serving_amd.sequence import Request, SamplingParams, Sequence

BLOCK = 4
NUM_BLOCKS = 24
KEYS = ("tenant-a", "tenant-b")


def independent_groups(pairs):
    """Same rule as paged_kv_serving_amd.ops.independent_groups (importing ops needs torch)."""
    from paged_kv_serving_amd.ops import independent_groups as groups

    return groups(pairs)


class ShadowStore:
    """What each block holds; copies are queued and applied as batched groups on demand."""

    def __init__(self) -> None:
        self.cells: list[list[int | None]] = [[None] * BLOCK for _ in range(NUM_BLOCKS)]
        self.pending: list[tuple[int, int]] = []

    def copy_block(self, source: int, destination: int) -> None:
        self.pending.append((source, destination))

    def flush(self) -> None:
        for group in independent_groups(self.pending):
            snapshot = [list(self.cells[src]) for src, _ in group]  # concurrent: read all first
            for (_, dst), data in zip(group, snapshot):
                self.cells[dst] = data
        self.pending.clear()

    def write(self, block: int, offset: int, token: int) -> None:
        self.flush()
        self.cells[block][offset] = token


class PagedCacheMachine(RuleBasedStateMachine):
    def __init__(self) -> None:
        super().__init__()
        self.store = ShadowStore()
        self.blocks = BlockManager(num_blocks=NUM_BLOCKS, block_size=BLOCK, store=self.store)
        self.cache = PrefixCache(self.blocks, scope="per_key")
        self.kv = KVCacheManager(self.blocks, self.cache)
        self.sequences: dict[str, Sequence] = {}
        self.snapshots: dict[bytes, tuple] = {}
        self.counter = 0

    def _pick(self, index: int) -> Sequence:
        keys = sorted(self.sequences)
        return self.sequences[keys[index % len(keys)]]

    def _write_chunk(self, seq: Sequence, chunk: int) -> None:
        self.kv.reserve(seq, seq.num_computed_tokens + chunk)
        for position in range(seq.num_computed_tokens, seq.num_computed_tokens + chunk):
            self.store.write(seq.block_table[position // BLOCK], position % BLOCK, seq.token_ids[position])
        seq.num_computed_tokens += chunk
        self.kv.publish_full_blocks(seq)
        self.store.flush()
        for block_hash, block_id in zip(self.cache._entries.keys(), self.cache.cached_block_ids()):
            self.snapshots.setdefault(block_hash, tuple(self.store.cells[block_id]))

    @rule(
        prompt=st.lists(st.integers(1, 12), min_size=1, max_size=14),
        key=st.sampled_from(KEYS),
        shared_prefix=st.booleans(),
    )
    def admit(self, prompt, key, shared_prefix) -> None:
        if len(self.sequences) >= 6:
            return
        self.counter += 1
        tokens = [1, 2, 3, 4, *prompt] if shared_prefix else prompt
        request = Request(f"r{self.counter}", tuple(tokens), SamplingParams(4, self.counter), key_id=key)
        seq = Sequence.from_request(request, 0)
        self.kv.attach_prefix(seq)
        self.sequences[seq.seq_id] = seq

    @precondition(lambda self: bool(self.sequences))
    @rule(index=st.integers(0, 100), chunk=st.integers(1, 6))
    def prefill_chunk(self, index, chunk) -> None:
        seq = self._pick(index)
        if seq.num_uncomputed_tokens >= 1:
            with contextlib.suppress(BlockAllocationError):
                self._write_chunk(seq, min(chunk, seq.num_uncomputed_tokens))

    @precondition(lambda self: bool(self.sequences))
    @rule(index=st.integers(0, 100), token=st.integers(1, 12))
    def decode(self, index, token) -> None:
        seq = self._pick(index)
        if seq.num_uncomputed_tokens != 0 or seq.num_output_tokens >= 6:
            return
        seq.append_token(token)
        try:
            self._write_chunk(seq, 1)
        except BlockAllocationError:
            seq.token_ids.pop()

    @precondition(lambda self: bool(self.sequences))
    @rule(index=st.integers(0, 100))
    def fork(self, index) -> None:
        parent = self._pick(index)
        if parent.num_computed_tokens < 1 or len(self.sequences) >= 8:
            return
        self.counter += 1
        child = Sequence.from_request(parent.request, self.counter)
        child.token_ids = list(parent.token_ids)
        child.seq_id = f"{parent.seq_id}-fork{self.counter}"
        self.kv.fork(parent, child)
        self.sequences[child.seq_id] = child

    @precondition(lambda self: bool(self.sequences))
    @rule(index=st.integers(0, 100))
    def preempt(self, index) -> None:
        seq = self._pick(index)
        self.kv.free(seq)
        seq.reset_for_recompute()

    @precondition(lambda self: bool(self.sequences))
    @rule(index=st.integers(0, 100))
    def finish(self, index) -> None:
        seq = self._pick(index)
        self.kv.free(seq)
        del self.sequences[seq.seq_id]

    @rule(count=st.integers(1, 4))
    def evict(self, count) -> None:
        assert self.cache.evict(count) <= count

    @invariant()
    def allocator_is_consistent(self) -> None:
        self.kv.check_invariants()

    @invariant()
    def sequences_read_back_their_own_tokens(self) -> None:
        self.store.flush()
        for seq in self.sequences.values():
            for position in range(seq.num_computed_tokens):
                block = seq.block_table[position // BLOCK]
                assert self.store.cells[block][position % BLOCK] == seq.token_ids[position], (
                    seq.seq_id, position, block
                )

    @invariant()
    def cached_blocks_are_never_mutated(self) -> None:
        for block_hash, block_id in zip(self.cache._entries.keys(), self.cache.cached_block_ids()):
            expected = self.snapshots.get(block_hash)
            if expected is not None:
                assert tuple(self.store.cells[block_id]) == expected

    def teardown(self) -> None:
        for seq in self.sequences.values():
            self.kv.free(seq)
        self.cache.flush()
        self.blocks.check_invariants()
        assert self.blocks.num_free_blocks == NUM_BLOCKS, "blocks leaked"


PagedCacheTest = PagedCacheMachine.TestCase
PagedCacheTest.settings = settings(
    max_examples=40,
    stateful_step_count=40,
    deadline=None,
    suppress_health_check=[HealthCheck.too_slow, HealthCheck.filter_too_much],
)
