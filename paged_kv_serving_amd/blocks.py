"""The block pool behind every block table: owner counts, a FIFO ring of free ids, copy-on-write.

Interface (kept so the reference's scheduler and tests run unchanged): ``BlockManager`` with
``allocate / allocate_many / incref / free / free_many / prepare_for_write / ref_count /
check_invariants / snapshot``, the ``BlockStore`` protocol, ``RecordingBlockStore`` and the two
error types, with the reference's messages (src/paged_kv_serving/engine/blocks.py:35-192).

Observable order (kept so block tables are bit-exact with the reference): ids start free in the
order ``0 .. N-1``; allocation takes the oldest free id; a block whose last owner leaves goes
behind every other free id; a write to a shared block allocates the destination, asks the store
for the copy, then drops the writer's ownership of the source (blocks.py:148-165).

Representation. The pool is two int32 buffers of ``num_blocks`` entries:

* ``_owners[b]`` -- how many block tables (and prefix-cache entries) hold block ``b``; 0 = free;
* ``_ring`` -- the free ids as a circular FIFO: the ``_nfree`` ids starting at ``_head``.

Each buffer is a ``array('i')`` with a NumPy view of the same memory (``_owners_v``,
``_ring_v``). Single-block calls (one allocate, one copy-on-write) index the array directly,
which costs about half what a NumPy scalar access does; calls over many blocks use the views:
a run of ``k`` ids leaves the ring as at most two slices, and a table's worth of blocks returns
with one gather of their counts, so the per-iteration work of a large batch (hundreds of tables,
thousands of blocks) is a few array operations instead of a Python loop per block. The views
also answer what the KV-cache manager asks of whole tables at once ("which blocks of this write
range are shared?", "which cached blocks does only the cache hold?") in one gather.
"""

from __future__ import annotations

from array import array
from collections.abc import Iterable
from typing import Protocol, runtime_checkable

import numpy as np

__all__ = [
    "BlockAllocationError",
    "BlockManager",
    "BlockStore",
    "InvariantError",
    "RecordingBlockStore",
]

# Below this many ids a batch call runs the scalar path: a handful of NumPy calls (about a
# microsecond each) costs more than a short Python loop (measured crossover: 40-60 ids).
_VECTOR_MIN = 64


class BlockAllocationError(RuntimeError):
    """The pool cannot supply the blocks asked for (reference blocks.py:35-36)."""


class InvariantError(AssertionError):
    """The pool's bookkeeping is inconsistent, or a call would make it so (blocks.py:39-40)."""


@runtime_checkable
class BlockStore(Protocol):
    """Whatever holds the bytes of the blocks (blocks.py:43-48): the GPU ModelRunner here."""

    def copy_block(self, source: int, destination: int) -> None:
        """Copy every byte of block ``source`` over block ``destination``."""


class RecordingBlockStore:
    """A store that keeps the list of requested copies and moves no bytes (blocks.py:51-60)."""

    def __init__(self) -> None:
        self.copies: list[tuple[int, int]] = []

    def copy_block(self, source: int, destination: int) -> None:
        if source == destination:
            raise InvariantError("copy-on-write must not copy a block onto itself")
        self.copies.append((source, destination))


class BlockManager:
    """Owner-counted pool of ``num_blocks`` KV blocks with FIFO reuse; see the module docstring."""

    def __init__(self, *, num_blocks: int, block_size: int, store: BlockStore) -> None:
        if num_blocks < 1:
            raise ValueError("num_blocks must be >= 1")
        if block_size < 1:
            raise ValueError("block_size must be >= 1")
        self.block_size = block_size
        self._size = num_blocks
        self._store = store
        self._owners = array("i", bytes(4 * num_blocks))
        self._ring = array("i", range(num_blocks))
        if self._owners.itemsize != 4:  # pragma: no cover - every supported platform has 4-byte int
            raise RuntimeError("the block pool needs a 4-byte C int")
        self._owners_v = np.frombuffer(self._owners, dtype=np.int32)
        self._ring_v = np.frombuffer(self._ring, dtype=np.int32)
        self._head = 0
        self._nfree = num_blocks

    # --- sizes ---------------------------------------------------------------------------

    @property
    def num_blocks(self) -> int:
        return self._size

    @property
    def num_free_blocks(self) -> int:
        return self._nfree

    @property
    def num_used_blocks(self) -> int:
        return self._size - self._nfree

    @property
    def utilization(self) -> float:
        """Share of the pool held by at least one owner."""
        return (self._size - self._nfree) / self._size

    # --- queries -------------------------------------------------------------------------

    def ref_count(self, block_id: int) -> int:
        if not 0 <= block_id < self._size:
            raise InvariantError(f"block id {block_id} is outside the pool")
        return self._owners[block_id]

    def counts_of(self, block_ids) -> np.ndarray:
        """Owner counts of many blocks in one gather (int32, same order as ``block_ids``)."""
        ids = np.asarray(block_ids, dtype=np.int64)
        if ids.size and (ids.min() < 0 or ids.max() >= self._size):
            bad = int(ids[(ids < 0) | (ids >= self._size)][0])
            raise InvariantError(f"block id {bad} is outside the pool")
        return self._owners_v[ids]

    def shared_positions(self, table, lo: int, hi: int) -> list[int]:
        """Indices ``i`` in ``[lo, hi)`` whose block ``table[i]`` has more than one owner. A few
        entries (a decode step writes one block) are read one by one from the owner array; longer
        stretches take one NumPy gather (:meth:`counts_of`)."""
        if hi - lo > 8:
            owners = self.counts_of(table[lo:hi])
            return [lo + int(k) for k in (owners > 1).nonzero()[0]]
        size, counts = self._size, self._owners
        shared = []
        for index in range(lo, hi):
            block = table[index]
            if not 0 <= block < size:
                raise InvariantError(f"block id {block} is outside the pool")
            if counts[block] > 1:
                shared.append(index)
        return shared

    def free_order(self) -> list[int]:
        """The free ids, oldest first: the order in which they will be allocated."""
        return self._take_view(self._nfree).tolist()

    def snapshot(self) -> tuple[int, ...]:
        """Owner count of every block."""
        return tuple(self._owners)

    # --- the ring ------------------------------------------------------------------------

    def _take_view(self, count: int) -> np.ndarray:
        """The ``count`` oldest free ids (a copy), without removing them."""
        end = self._head + count
        if end <= self._size:
            return self._ring_v[self._head : end].copy()
        return np.concatenate((self._ring_v[self._head :], self._ring_v[: end - self._size]))

    def _push(self, block_id: int) -> None:
        tail = self._head + self._nfree
        self._ring[tail - self._size if tail >= self._size else tail] = block_id
        self._nfree += 1

    def _push_many(self, ids: np.ndarray) -> None:
        slots = (self._head + self._nfree + np.arange(ids.size)) % self._size
        self._ring_v[slots] = ids
        self._nfree += int(ids.size)

    # --- ownership -----------------------------------------------------------------------

    def allocate(self) -> int:
        """The oldest free block, now with one owner."""
        if self._nfree == 0:
            raise BlockAllocationError("the KV block pool is exhausted")
        block_id = self._ring[self._head]
        self._head = self._head + 1 if self._head + 1 < self._size else 0
        self._nfree -= 1
        self._owners[block_id] = 1
        return block_id

    def allocate_many(self, count: int) -> list[int]:
        """The ``count`` oldest free blocks, each with one owner; nothing if they do not all fit."""
        if count < 0:
            raise ValueError("count must be >= 0")
        if count > self._nfree:
            raise BlockAllocationError(
                f"need {count} blocks, {self._nfree} free in a pool of {self._size}"
            )
        head, size = self._head, self._size
        end = head + count
        self._head = end - size if end >= size else end
        self._nfree -= count
        if count >= _VECTOR_MIN:
            ids = self._ring_v[head:end].copy() if end <= size else np.concatenate(
                (self._ring_v[head:], self._ring_v[: end - size]))  # fmt: skip
            self._owners_v[ids] = 1
            return ids.tolist()
        ring = self._ring
        ids = ring[head:end].tolist() if end <= size else ring[head:].tolist() + ring[: end - size].tolist()
        owners = self._owners
        for block_id in ids:
            owners[block_id] = 1
        return ids

    def incref(self, block_id: int) -> int:
        """One more owner of a held block; returns its new count."""
        if not 0 <= block_id < self._size:
            raise InvariantError(f"block id {block_id} is outside the pool")
        owners = self._owners[block_id]
        if owners == 0:
            raise InvariantError(f"block {block_id} is free and cannot gain a reference")
        self._owners[block_id] = owners + 1
        return owners + 1

    def free(self, block_id: int) -> int:
        """One owner fewer; the block rejoins the ring, behind every free id, when none is left.
        Returns the remaining count."""
        if not 0 <= block_id < self._size:
            raise InvariantError(f"block id {block_id} is outside the pool")
        owners = self._owners[block_id]
        if owners == 0:
            raise InvariantError(f"block {block_id} was freed twice")
        owners -= 1
        self._owners[block_id] = owners
        if owners == 0:
            self._push(block_id)
        return owners

    def free_many(self, block_ids: Iterable[int]) -> None:
        """:meth:`free` of each id, in order. A table of distinct, held ids is released with one
        gather and one scatter; anything else (repeats, a free or foreign id) takes the one-by-one
        path, so an error is raised at the same id, after the same earlier releases."""
        ids = block_ids if isinstance(block_ids, (list, tuple)) else list(block_ids)
        if len(ids) < _VECTOR_MIN:
            owners, ring, size = self._owners, self._ring, self._size
            for block_id in ids:
                if not 0 <= block_id < size:
                    raise InvariantError(f"block id {block_id} is outside the pool")
                left = owners[block_id] - 1
                if left < 0:
                    raise InvariantError(f"block {block_id} was freed twice")
                owners[block_id] = left
                if left == 0:
                    tail = self._head + self._nfree
                    ring[tail - size if tail >= size else tail] = block_id
                    self._nfree += 1
            return
        arr = np.asarray(ids, dtype=np.int64)
        if (
            arr.min() < 0
            or arr.max() >= self._size
            or np.unique(arr).size != arr.size
            or not np.all(self._owners_v[arr] > 0)
        ):
            for block_id in ids:
                self.free(block_id)
            return
        left = self._owners_v[arr] - 1
        self._owners_v[arr] = left
        released = arr[left == 0]
        if released.size:
            self._push_many(released.astype(np.int32))

    def prepare_for_write(self, block_id: int) -> int:
        """The block the caller may write: ``block_id`` itself when the caller is its only owner,
        otherwise a fresh block that receives a copy of it (the caller's ownership moves there)."""
        if not 0 <= block_id < self._size:
            raise InvariantError(f"block id {block_id} is outside the pool")
        owners = self._owners[block_id]
        if owners == 0:
            raise InvariantError(f"block {block_id} is free and cannot be written")
        if owners == 1:
            return block_id
        private = self.allocate()
        self._store.copy_block(block_id, private)
        self.free(block_id)
        return private

    # --- consistency ---------------------------------------------------------------------

    def check_invariants(self) -> None:
        """Raise :class:`InvariantError` unless the ring holds exactly the ownerless blocks,
        each once, and no count is negative."""
        free = self._take_view(self._nfree).astype(np.int64)
        listed = np.zeros(self._size, dtype=np.int64)
        np.add.at(listed, free, 1)
        if np.any(listed > 1):
            raise InvariantError(f"block {int(np.flatnonzero(listed > 1)[0])} is on the free ring twice")
        owners = self._owners_v
        if np.any(owners < 0):
            raise InvariantError(f"block {int(np.flatnonzero(owners < 0)[0])} has a negative owner count")
        wrong = np.flatnonzero((owners == 0) != (listed == 1))
        if wrong.size:
            block = int(wrong[0])
            where = "is" if listed[block] else "is not"
            raise InvariantError(f"block {block} has {int(owners[block])} owners but {where} on the free ring")
        held = int(np.count_nonzero(owners))
        if held + self._nfree != self._size:
            raise InvariantError(f"{held} held + {self._nfree} free != {self._size} blocks")
