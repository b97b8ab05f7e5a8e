"""Block-level prefix cache keyed by a BLAKE2b hash chain over full blocks.

Mirrors src/paged_kv_serving/engine/prefix_cache.py:41-202, byte for byte in the hash inputs so
cached-block identities agree with the reference's:

    h_0 = BLAKE2b-16(b"paged-kv-serving/prefix-v1" + b"|" + scope)
    h_i = BLAKE2b-16(h_{i-1} + block_size as u32 LE + each token as u32 LE)

The cache is an LRU map from chain hash to block id that holds one reference per entry and only
evicts entries whose block no live sequence is reading.
"""

from __future__ import annotations

import hashlib
from collections import OrderedDict
from collections.abc import Sequence
from dataclasses import dataclass
from typing import Literal

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

_DOMAIN = b"paged-kv-serving/prefix-v1"
_DIGEST = 16


def chain_seed(scope: bytes = b"") -> bytes:
    """Start of a chain; distinct scopes never share a prefix (prefix_cache.py:47-49)."""
    return hashlib.blake2b(_DOMAIN + b"|" + scope, digest_size=_DIGEST).digest()


def next_block_hash(parent: bytes, token_ids: Sequence[int], block_size: int) -> bytes:
    """Extend a chain by one full block (prefix_cache.py:52-59)."""
    if len(token_ids) != block_size:
        raise ValueError("only full blocks are hashed and cached")
    body = bytearray(parent)
    body += block_size.to_bytes(4, "little")
    for token in token_ids:
        body += int(token).to_bytes(4, "little", signed=False)
    return hashlib.blake2b(bytes(body), digest_size=_DIGEST).digest()


def block_hash_chain(
    token_ids: Sequence[int], *, block_size: int, num_blocks: int, scope: bytes = b""
) -> list[bytes]:
    """Chained hashes of the first ``num_blocks`` full blocks (prefix_cache.py:62-83)."""
    if block_size < 1:
        raise ValueError("block_size must be >= 1")
    if num_blocks < 0:
        raise ValueError("num_blocks must be >= 0")
    if num_blocks * block_size > len(token_ids):
        raise ValueError("not enough tokens for the requested number of full blocks")
    chain: list[bytes] = []
    parent = chain_seed(scope)
    for i in range(num_blocks):
        parent = next_block_hash(parent, token_ids[i * block_size : (i + 1) * block_size], block_size)
        chain.append(parent)
    return chain


@dataclass
class PrefixCacheStats:
    queried_blocks: int = 0
    hit_blocks: int = 0
    registered_blocks: int = 0
    evicted_blocks: int = 0

    @property
    def hit_ratio(self) -> float:
        return self.hit_blocks / self.queried_blocks if self.queried_blocks else 0.0

    def as_dict(self) -> dict[str, float]:
        return {
            "queried_blocks": float(self.queried_blocks),
            "hit_blocks": float(self.hit_blocks),
            "registered_blocks": float(self.registered_blocks),
            "evicted_blocks": float(self.evicted_blocks),
            "hit_ratio": self.hit_ratio,
        }


class PrefixCache:
    """LRU map from chained block hash to block id, one reference per entry."""

    def __init__(
        self, manager: BlockManager, *, enabled: bool = True, scope: CacheScope = "per_key"
    ) -> None:
        self._manager = manager
        self._entries: OrderedDict[bytes, int] = OrderedDict()
        self.enabled = enabled
        self.scope = scope
        self.stats = PrefixCacheStats()

    def __len__(self) -> int:
        return len(self._entries)

    def scope_bytes(self, key_id: str) -> bytes:
        return key_id.encode("utf-8") if self.scope == "per_key" else b"shared"

    def lookup(self, hashes: Sequence[bytes], *, record: bool = True) -> list[int]:
        """Block ids of the longest cached prefix of ``hashes``, each increfed for the caller."""
        matched: list[int] = []
        if self.enabled:
            for block_hash in hashes:
                block_id = self._entries.get(block_hash)
                if block_id is None:
                    break
                self._entries.move_to_end(block_hash)
                self._manager.incref(block_id)
                matched.append(block_id)
        if record:
            self.record_lookup(len(hashes), len(matched))
        return matched

    def record_lookup(self, queried_blocks: int, hit_blocks: int) -> None:
        self.stats.queried_blocks += queried_blocks
        self.stats.hit_blocks += hit_blocks

    def register(self, block_hash: bytes, block_id: int) -> bool:
        """Cache a newly filled block (taking a reference); False if already cached."""
        if not self.enabled or block_hash in self._entries:
            return False
        self._manager.incref(block_id)
        self._entries[block_hash] = block_id
        self.stats.registered_blocks += 1
        return True

    def evict(self, count: int = 1) -> int:
        """Evict up to ``count`` LRU entries the cache holds alone; returns blocks released."""
        if count <= 0:
            return 0
        released = 0
        for block_hash in list(self._entries):
            if released >= count:
                break
            block_id = self._entries[block_hash]
            if self._manager.ref_count(block_id) > 1:
                continue
            del self._entries[block_hash]
            self._manager.free(block_id)
            released += 1
        self.stats.evicted_blocks += released
        return released

    def evict_until_free(self, needed: int) -> int:
        shortfall = needed - self._manager.num_free_blocks
        return self.evict(shortfall) if shortfall > 0 else 0

    def flush(self) -> int:
        return self.evict(len(self._entries))

    def cached_block_ids(self) -> tuple[int, ...]:
        return tuple(self._entries.values())
