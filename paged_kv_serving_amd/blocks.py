"""Reference-counted block allocator with copy-on-write, with the reference's API and semantics.

Mirrors src/paged_kv_serving/engine/blocks.py:35-192. Block ids are handed out FIFO from a free
list that starts as ``0, 1, ..., num_blocks - 1`` and receives a block back at its tail when the
last owner frees it, so the sequence of ids (and therefore every block table built on top) is
identical to the reference's for the same sequence of calls. ``prepare_for_write`` of a shared
block allocates the destination, asks the store to copy, then drops the caller's reference on
the source -- the exact order of blocks.py:156-165, which fixes which ids copies land in.

The store behind copy-on-write is any object with ``copy_block(source, destination)``; the GPU
:class:`~paged_kv_serving_amd.runner.ModelRunner` is one.
"""

from __future__ import annotations

from collections import deque
from collections.abc import Iterable
from typing import Protocol, runtime_checkable

__all__ = [
    "BlockAllocationError",
    "BlockManager",
    "BlockStore",
    "InvariantError",
    "RecordingBlockStore",
]


class BlockAllocationError(RuntimeError):
    """No free block is available (blocks.py:35-36)."""


class InvariantError(AssertionError):
    """An allocator invariant is broken (blocks.py:39-40)."""


@runtime_checkable
class BlockStore(Protocol):
    """The bytes behind block ids (blocks.py:43-48)."""

    def copy_block(self, source: int, destination: int) -> None:
        """Copy every byte of block ``source`` over block ``destination``."""


class RecordingBlockStore:
    """Records copies instead of moving bytes (blocks.py:51-60)."""

    def __init__(self) -> None:
        self.copies: list[tuple[int, int]] = []

    def copy_block(self, source: int, destination: int) -> None:
        if source == destination:
            raise InvariantError("copy-on-write must not copy a block onto itself")
        self.copies.append((source, destination))


class BlockManager:
    """FIFO, reference-counted allocator over a fixed pool of KV blocks (blocks.py:63-192)."""

    def __init__(self, *, num_blocks: int, block_size: int, store: BlockStore) -> None:
        if num_blocks < 1:
            raise ValueError("num_blocks must be >= 1")
        if block_size < 1:
            raise ValueError("block_size must be >= 1")
        self._num_blocks = num_blocks
        self.block_size = block_size
        self._store = store
        self._refs = [0] * num_blocks
        self._free: deque[int] = deque(range(num_blocks))

    @property
    def num_blocks(self) -> int:
        return self._num_blocks

    @property
    def num_free_blocks(self) -> int:
        return len(self._free)

    @property
    def num_used_blocks(self) -> int:
        return self._num_blocks - len(self._free)

    @property
    def utilization(self) -> float:
        return self.num_used_blocks / self._num_blocks

    def _id(self, block_id: int) -> int:
        if block_id < 0 or block_id >= self._num_blocks:
            raise InvariantError(f"block id {block_id} is outside the pool")
        return block_id

    def ref_count(self, block_id: int) -> int:
        return self._refs[self._id(block_id)]

    def allocate(self) -> int:
        """Pop the oldest free block; it starts with one reference."""
        if not self._free:
            raise BlockAllocationError("the KV block pool is exhausted")
        block_id = self._free.popleft()
        self._refs[block_id] = 1
        return block_id

    def allocate_many(self, count: int) -> list[int]:
        """``count`` blocks, or none if the pool cannot cover all of them."""
        if count < 0:
            raise ValueError("count must be >= 0")
        available = len(self._free)
        if count > available:
            raise BlockAllocationError(
                f"need {count} blocks, {available} free in a pool of {self._num_blocks}"
            )
        return [self.allocate() for _ in range(count)]

    def incref(self, block_id: int) -> int:
        block_id = self._id(block_id)
        if self._refs[block_id] == 0:
            raise InvariantError(f"block {block_id} is free and cannot gain a reference")
        self._refs[block_id] += 1
        return self._refs[block_id]

    def free(self, block_id: int) -> int:
        """Drop one owner; the last one returns the block to the tail of the free list."""
        block_id = self._id(block_id)
        if self._refs[block_id] == 0:
            raise InvariantError(f"block {block_id} was freed twice")
        self._refs[block_id] -= 1
        if self._refs[block_id] == 0:
            self._free.append(block_id)
        return self._refs[block_id]

    def free_many(self, block_ids: Iterable[int]) -> None:
        for block_id in block_ids:
            self.free(block_id)

    def prepare_for_write(self, block_id: int) -> int:
        """The block the caller may write: itself if unshared, else a fresh private copy."""
        block_id = self._id(block_id)
        owners = self._refs[block_id]
        if owners == 0:
            raise InvariantError(f"block {block_id} is free and cannot be written")
        if owners == 1:
            return block_id
        private = self.allocate()
        self._store.copy_block(block_id, private)
        self.free(block_id)
        return private

    def check_invariants(self) -> None:
        """Raise :class:`InvariantError` on a leak, double free or corrupted free list."""
        on_free_list = set(self._free)
        if len(on_free_list) != len(self._free):
            raise InvariantError("the free list contains duplicate block ids")
        for block_id, count in enumerate(self._refs):
            if count < 0:
                raise InvariantError(f"block {block_id} has a negative reference count")
            listed = block_id in on_free_list
            if (count == 0) != listed:
                raise InvariantError(
                    f"block {block_id} has count {count} but "
                    f"{'is' if listed else 'is not'} on the free list"
                )
        referenced = sum(1 for count in self._refs if count > 0)
        if referenced + len(self._free) != self._num_blocks:
            raise InvariantError(
                f"{referenced} referenced + {len(self._free)} free != {self._num_blocks} blocks"
            )

    def snapshot(self) -> tuple[int, ...]:
        return tuple(self._refs)
