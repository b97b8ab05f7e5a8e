"""Prefix cache: full KV blocks found again by a hash chain over the tokens in front of them.

Interface (kept so callers and cached block identities stay compatible with the reference,
src/paged_kv_serving/engine/prefix_cache.py:47-202): ``chain_seed``, ``next_block_hash`` and
``block_hash_chain`` with the reference's byte format; ``PrefixCache`` with ``lookup / register /
evict / evict_until_free / flush / cached_block_ids / scope_bytes / record_lookup``, its ``stats``
counters and the ``enabled`` / ``scope`` switches.

Byte format of the chain (BLAKE2b, 16-byte digests):

    seed   = H("paged-kv-serving/prefix-v1" "|" scope)
    h_i    = H(h_{i-1} || u32le(block_size) || u32le(token) for each token of block i)

Behaviour: a lookup returns the blocks of the longest run of leading hashes that are cached,
each with one more owner, and marks them most recently used; a block is registered under its
hash once, with an owner held by the cache; eviction walks entries least recently used first and
releases only those whose sole owner is the cache.

Representation. One insertion-ordered ``dict`` from hash to block id, oldest use first; a hit
moves the entry to the end. Eviction gathers the owner counts of all cached blocks in one
:meth:`BlockManager.counts_of` call and releases the first ``count`` entries the cache holds
alone, in one :meth:`BlockManager.free_many`, instead of asking the pool about each entry in turn.
"""

from __future__ import annotations

import hashlib
import sys
from array import array
from collections.abc import Sequence
from dataclasses import dataclass
from typing import Literal

import numpy as np

from paged_kv_serving_amd.blocks import BlockManager

__all__ = [
    "CacheScope",
    "PrefixCache",
    "PrefixCacheStats",
    "block_hash_chain",
    "chain_seed",
    "next_block_hash",
]

CacheScope = Literal["per_key", "global"]

_SEED_PREFIX = b"paged-kv-serving/prefix-v1|"
_DIGEST = 16
_SWAP = sys.byteorder != "little"


def chain_seed(scope: bytes = b"") -> bytes:
    """The hash a chain starts from; different scopes never share a chain."""
    return hashlib.blake2b(_SEED_PREFIX + scope, digest_size=_DIGEST).digest()


def _u32le(values) -> bytes:
    """Little-endian uint32 bytes; a negative or too-large value raises OverflowError."""
    packed = array("I", values)
    if packed.itemsize != 4:  # pragma: no cover - every supported platform has 4-byte uint
        packed = array("L", values)
    if _SWAP:  # pragma: no cover - big-endian hosts
        packed.byteswap()
    return packed.tobytes()


def next_block_hash(parent: bytes, token_ids: Sequence[int], block_size: int) -> bytes:
    """The chain hash of one full block of ``block_size`` tokens that follows ``parent``."""
    if len(token_ids) != block_size:
        raise ValueError("only full blocks are hashed and cached")
    message = parent + _u32le((block_size,)) + _u32le(token_ids)
    return hashlib.blake2b(message, digest_size=_DIGEST).digest()


def block_hash_chain(
    token_ids: Sequence[int], *, block_size: int, num_blocks: int, scope: bytes = b""
) -> list[bytes]:
    """Chain hashes of the first ``num_blocks`` full blocks of ``token_ids``."""
    if block_size < 1:
        raise ValueError("block_size must be >= 1")
    if num_blocks < 0:
        raise ValueError("num_blocks must be >= 0")
    if num_blocks * block_size > len(token_ids):
        raise ValueError("not enough tokens for the requested number of full blocks")
    return list(_walk_chain(chain_seed(scope), token_ids, block_size, 0, num_blocks))


def _walk_chain(parent: bytes, token_ids: Sequence[int], block_size: int, first: int, stop: int):
    """Yield the chain hashes of blocks ``first .. stop - 1`` given the hash before ``first``."""
    for index in range(first, stop):
        parent = next_block_hash(parent, token_ids[index * block_size : (index + 1) * block_size], block_size)
        yield parent


@dataclass
class PrefixCacheStats:
    """Lifetime counters (field names are the reference's, read by its metrics)."""

    queried_blocks: int = 0
    hit_blocks: int = 0
    registered_blocks: int = 0
    evicted_blocks: int = 0

    @property
    def hit_ratio(self) -> float:
        return self.hit_blocks / self.queried_blocks if self.queried_blocks else 0.0

    def as_dict(self) -> dict[str, float]:
        counters = ("queried_blocks", "hit_blocks", "registered_blocks", "evicted_blocks")
        return {**{name: float(getattr(self, name)) for name in counters}, "hit_ratio": self.hit_ratio}


class PrefixCache:
    """Hash -> block id, least recently used first, one owner per entry; see the module docstring."""

    def __init__(self, manager: BlockManager, *, enabled: bool = True, scope: CacheScope = "per_key") -> None:
        self._pool = manager
        self._blocks: dict[bytes, int] = {}
        self.enabled = enabled
        self.scope = scope
        self.stats = PrefixCacheStats()

    def __len__(self) -> int:
        return len(self._blocks)

    def scope_bytes(self, key_id: str) -> bytes:
        """What a caller's chains start from: its key id, or one shared constant."""
        return key_id.encode("utf-8") if self.scope == "per_key" else b"shared"

    def _hit(self, block_hash: bytes) -> int | None:
        """The block cached under ``block_hash``, now most recently used and with one more owner."""
        block = self._blocks.pop(block_hash, None)
        if block is None:
            return None
        self._blocks[block_hash] = block
        self._pool.incref(block)
        return block

    def lookup(self, hashes: Sequence[bytes], *, record: bool = True) -> list[int]:
        """Blocks of the longest cached run of leading ``hashes``, each with a new owner that the
        caller now holds. ``record=False`` leaves the hit counters alone."""
        found: list[int] = []
        if self.enabled:
            for block_hash in hashes:
                block = self._hit(block_hash)
                if block is None:
                    break
                found.append(block)
        if record:
            self.record_lookup(len(hashes), len(found))
        return found

    def match(self, seed: bytes, token_ids: Sequence[int], block_size: int, count: int, *, record: bool = True):
        """:meth:`lookup` of the chain over the first ``count`` full blocks of ``token_ids``,
        hashing only as far as the first miss (nothing past it can match). Returns the matched
        blocks and their hashes; the counters see ``count`` queried blocks, as a lookup of the
        whole chain would."""
        blocks: list[int] = []
        hashes: list[bytes] = []
        if self.enabled:
            for block_hash in _walk_chain(seed, token_ids, block_size, 0, count):
                block = self._hit(block_hash)
                if block is None:
                    break
                blocks.append(block)
                hashes.append(block_hash)
        if record:
            self.record_lookup(count, len(blocks))
        return blocks, hashes

    def record_lookup(self, queried_blocks: int, hit_blocks: int) -> None:
        self.stats.queried_blocks += queried_blocks
        self.stats.hit_blocks += hit_blocks

    def register(self, block_hash: bytes, block_id: int) -> bool:
        """Cache a full block under its chain hash, taking an owner of it. False when the cache is
        off or already holds that hash."""
        if not self.enabled or block_hash in self._blocks:
            return False
        self._pool.incref(block_id)
        self._blocks[block_hash] = block_id
        self.stats.registered_blocks += 1
        return True

    def evict(self, count: int = 1) -> int:
        """Release up to ``count`` entries that only the cache holds, least recently used first.
        Entries a live sequence still reads stay. Returns how many were released."""
        if count <= 0 or not self._blocks:
            return 0
        keys = list(self._blocks)
        ids = np.fromiter(self._blocks.values(), dtype=np.int64, count=len(keys))
        owners = self._pool.counts_of(ids)
        if np.unique(ids).size != ids.size or np.any(owners < 1):
            released = self._evict_one_by_one(keys, count)
        else:
            chosen = np.flatnonzero(owners == 1)[:count]
            for k in chosen.tolist():
                del self._blocks[keys[k]]
            self._pool.free_many(ids[chosen].tolist())
            released = int(chosen.size)
        self.stats.evicted_blocks += released
        return released

    def _evict_one_by_one(self, keys: list[bytes], count: int) -> int:
        """Eviction when a block sits under two hashes or the counts are already inconsistent:
        each entry's owners are read just before it is considered."""
        released = 0
        for key in keys:
            if released >= count:
                break
            block = self._blocks[key]
            if self._pool.ref_count(block) > 1:
                continue
            del self._blocks[key]
            self._pool.free(block)
            released += 1
        return released

    def evict_until_free(self, needed: int) -> int:
        """Evict just enough for ``needed`` free blocks. Returns how many were released."""
        missing = needed - self._pool.num_free_blocks
        return self.evict(missing) if missing > 0 else 0

    def flush(self) -> int:
        """Release every entry only the cache holds."""
        return self.evict(len(self._blocks))

    def cached_block_ids(self) -> tuple[int, ...]:
        """Cached block ids, least recently used first."""
        return tuple(self._blocks.values())

    def sole_owner_count(self) -> int:
        """How many cached blocks only the cache holds (what eviction could release)."""
        if not self._blocks:
            return 0
        ids = np.fromiter(self._blocks.values(), dtype=np.int64, count=len(self._blocks))
        return int(np.count_nonzero(self._pool.counts_of(ids) == 1))
