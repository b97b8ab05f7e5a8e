"""The pool's bookkeeping checked against a ledger rebuilt from scratch after every operation.

Seeded random runs drive KVCacheManager the way a serving loop does -- admit with a prefix
lookup, compute chunks, decode, fork, free, evict -- over a block store that keeps the tokens
each block slot holds (so copy-on-write copies contents). After every operation the expected
state is recomputed from what is alive, independently of the allocator:

* every block's owner count = the live block tables naming it + one if the prefix cache holds it;
* the free ids are exactly the ownerless blocks, each once;
* every live sequence reads its own tokens back through its block table at every computed
  position (no block is shared with a writer, no copy is lost);
* a block the prefix cache holds never changes after it was registered.
"""

from __future__ import annotations

import numpy as np
import pytest

from paged_kv_serving_amd.blocks import BlockAllocationError, BlockManager
from paged_kv_serving_amd.kvcache import KVCacheManager
from paged_kv_serving_amd.prefix_cache import PrefixCache
from paged_kv_serving_amd.sequence import Request, Sequence


class ContentStore:
    """Token ids held by every slot of every block; copy_block copies a whole block."""

    def __init__(self, num_blocks: int, block_size: int) -> None:
        self.slots = np.full((num_blocks, block_size), -1, dtype=np.int64)
        self.copies = 0

    def copy_block(self, source: int, destination: int) -> None:
        assert source != destination
        self.slots[destination] = self.slots[source]
        self.copies += 1


class Run:
    def __init__(self, seed: int, *, num_blocks: int, block_size: int, enabled: bool) -> None:
        self.rng = np.random.default_rng(seed)
        self.size = block_size
        self.store = ContentStore(num_blocks, block_size)
        self.blocks = BlockManager(num_blocks=num_blocks, block_size=block_size, store=self.store)
        self.cache = KVCacheManager(self.blocks, PrefixCache(self.blocks, enabled=enabled))
        self.live: list[Sequence] = []
        # (chain hash, block) of every cache entry -> the block's contents when it was registered
        self.frozen: dict[tuple[bytes, int], np.ndarray] = {}
        self.stems = [list(self.rng.integers(0, 50, int(self.rng.integers(4, 30)))) for _ in range(3)]
        self.count = 0

    # --- operations ------------------------------------------------------------------------

    def admit(self) -> None:
        stem = self.stems[int(self.rng.integers(0, 3))] if self.rng.random() < 0.7 else []
        tokens = [int(t) for t in stem] + [int(t) for t in self.rng.integers(0, 50, int(self.rng.integers(1, 20)))]
        key = "a" if self.rng.random() < 0.8 else "b"
        seq = Sequence.from_request(Request(f"s{self.count}", tuple(tokens), key_id=key))
        self.count += 1
        self.cache.attach_prefix(seq)
        chunk = int(self.rng.integers(1, seq.num_uncomputed_tokens + 1))
        if not self.compute(seq, chunk):
            self.cache.detach_prefix(seq)
            return
        self.live.append(seq)

    def compute(self, seq: Sequence, chunk: int) -> bool:
        start = seq.num_computed_tokens
        try:
            self.cache.reserve(seq, start + chunk)
        except BlockAllocationError:
            return False
        for p in range(start, start + chunk):  # the append: write each token at its slot
            self.store.slots[seq.block_table[p // self.size], p % self.size] = seq.token_ids[p]
        seq.num_computed_tokens += chunk
        self.cache.publish_full_blocks(seq)
        self.freeze()
        return True

    def freeze(self) -> None:
        entries = set(self.cache.prefix_cache._blocks.items())
        for entry in entries:
            self.frozen.setdefault(entry, self.store.slots[entry[1]].copy())
        for entry in set(self.frozen) - entries:
            del self.frozen[entry]

    def step(self) -> None:
        if not self.live:
            return
        seq = self.live[int(self.rng.integers(0, len(self.live)))]
        if seq.num_uncomputed_tokens == 0:
            seq.token_ids.append(int(self.rng.integers(0, 50)))  # a sampled token
        chunk = int(self.rng.integers(1, seq.num_uncomputed_tokens + 1))
        if not self.compute(seq, chunk):
            self.finish(seq)  # preempted: its blocks go back, it starts over later

    def fork(self) -> None:
        done = [s for s in self.live if s.num_uncomputed_tokens == 0 and s.num_computed_tokens]
        if not done:
            return
        parent = done[int(self.rng.integers(0, len(done)))]
        child = Sequence(f"{parent.seq_id}f{self.count}", parent.request, list(parent.token_ids))
        self.count += 1
        self.cache.fork(parent, child)
        self.live.append(child)

    def finish(self, seq: Sequence) -> None:
        self.live.remove(seq)
        self.cache.free(seq)

    def evict(self) -> None:
        self.cache.prefix_cache.evict(int(self.rng.integers(0, 4)))
        self.freeze()

    # --- the ledger ----------------------------------------------------------------------

    def check(self) -> None:
        n = self.blocks.num_blocks
        owners = np.zeros(n, dtype=np.int64)
        for seq in self.live:
            np.add.at(owners, np.asarray(seq.block_table, dtype=np.int64), 1)
        cached = list(self.cache.prefix_cache.cached_block_ids())
        np.add.at(owners, np.asarray(cached, dtype=np.int64), 1)
        assert list(self.blocks.snapshot()) == owners.tolist()
        free = self.blocks.free_order()
        assert sorted(free) == np.flatnonzero(owners == 0).tolist()
        assert self.blocks.num_free_blocks == len(free)
        for seq in self.live:
            for p in range(seq.num_computed_tokens):
                assert self.store.slots[seq.block_table[p // self.size], p % self.size] == seq.token_ids[p]
        for (_, block), contents in self.frozen.items():
            assert np.array_equal(self.store.slots[block], contents), "a cached block changed"
        assert self.cache.evictable_blocks() == sum(1 for b in cached if owners[b] == 1)
        self.cache.check_invariants()


@pytest.mark.parametrize("seed", range(12))
@pytest.mark.parametrize(("num_blocks", "block_size", "enabled"), [(24, 4, True), (60, 2, True), (16, 8, False)])
def test_random_runs_keep_the_ledger(seed, num_blocks, block_size, enabled) -> None:
    run = Run(seed, num_blocks=num_blocks, block_size=block_size, enabled=enabled)
    operations = (run.admit, run.step, run.step, run.step, run.fork, run.evict)
    for _ in range(300):
        which = int(run.rng.integers(0, len(operations) + 1))
        if which == len(operations):
            if run.live:
                run.finish(run.live[int(run.rng.integers(0, len(run.live)))])
        else:
            operations[which]()
        run.check()
    for seq in list(run.live):
        run.finish(seq)
    run.cache.prefix_cache.flush()
    run.check()
    assert run.blocks.num_free_blocks == num_blocks
