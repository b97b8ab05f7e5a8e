"""The sequence state the KV-cache manager reads and writes, for callers without the reference's.

``KVCacheManager`` duck-reads a sequence (src/paged_kv_serving/engine/sequence.py:129-241):
``token_ids`` (prompt, then sampled tokens), ``block_table``, ``block_hashes``,
``num_computed_tokens``, ``cached_prefix_blocks``, ``num_tokens`` and ``request.key_id``. The
reference's own ``Sequence`` objects work unchanged; these small types are for this package's
trace replay and tests. The bookkeeping rule is the reference's (sequence.py:3-13): an iteration
runs ``token_ids[num_computed_tokens : num_computed_tokens + chunk]`` at those positions and
produces logits when the chunk reaches the end of ``token_ids``.
"""

from __future__ import annotations

from dataclasses import dataclass, field

__all__ = ["Request", "Sequence", "new_sequence_id"]


def new_sequence_id(request_id: str, index: int) -> str:
    """The reference's sequence id of sample ``index`` of a request (sequence.py:44-45)."""
    return f"{request_id}#{index}"


@dataclass(frozen=True)
class Request:
    """The part of a request the KV path sees: its prompt, sample count and prefix-cache key."""

    request_id: str
    prompt_token_ids: tuple[int, ...]
    n: int = 1
    key_id: str = "anonymous"

    def __post_init__(self) -> None:
        if not self.prompt_token_ids:
            raise ValueError("the prompt must contain at least one token")
        if self.n < 1:
            raise ValueError("n must be >= 1")

    @property
    def prompt_len(self) -> int:
        return len(self.prompt_token_ids)


@dataclass
class Sequence:
    """One sample of a request, as the KV-cache manager sees it."""

    seq_id: str
    request: Request
    token_ids: list[int] = field(default_factory=list)
    block_table: list[int] = field(default_factory=list)
    block_hashes: list[bytes] = field(default_factory=list)
    num_computed_tokens: int = 0
    cached_prefix_blocks: int = 0

    @classmethod
    def from_request(cls, request: Request, sample_index: int = 0) -> Sequence:
        return cls(new_sequence_id(request.request_id, sample_index), request, list(request.prompt_token_ids))

    @property
    def num_tokens(self) -> int:
        return len(self.token_ids)

    @property
    def num_uncomputed_tokens(self) -> int:
        return len(self.token_ids) - self.num_computed_tokens
