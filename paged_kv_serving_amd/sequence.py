"""Requests and per-sample sequence state, with the fields the KV cache manager reads.

Mirrors the parts of src/paged_kv_serving/engine/sequence.py:45-241 that the data path touches:
``token_ids`` (prompt then sampled tokens), ``block_table``, ``block_hashes``,
``num_computed_tokens``, ``cached_prefix_blocks``, ``num_tokens`` and ``request.key_id``. The
bookkeeping rule is the reference's: an iteration runs
``token_ids[num_computed_tokens : num_computed_tokens + chunk]`` at those positions and
produces logits exactly when the chunk reaches the end of ``token_ids`` (sequence.py:3-13).
"""

from __future__ import annotations

import itertools
from dataclasses import dataclass, field
from enum import Enum

__all__ = [
    "FinishReason",
    "Request",
    "SamplingParams",
    "Sequence",
    "SequenceStatus",
    "finish_reason_for",
    "new_sequence_id",
]

_ORDER = itertools.count()


def new_sequence_id(request_id: str, index: int) -> str:
    return f"{request_id}#{index}"


class SequenceStatus(Enum):
    WAITING = "waiting"
    RUNNING = "running"
    PREEMPTED = "preempted"
    FINISHED = "finished"


class FinishReason(Enum):
    LENGTH = "length"
    STOP = "stop"
    CONTEXT_LIMIT = "context_limit"


@dataclass(frozen=True)
class SamplingParams:
    """Greedy decoding with a token cap (the only policy the data-path runs use)."""

    max_new_tokens: int = 32
    seed: int = 0

    def __post_init__(self) -> None:
        if self.max_new_tokens < 1:
            raise ValueError("max_new_tokens must be >= 1")


@dataclass(frozen=True)
class Request:
    request_id: str
    prompt_token_ids: tuple[int, ...]
    sampling: SamplingParams = SamplingParams()
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
    seq_id: str
    request: Request
    sample_index: int = 0
    token_ids: list[int] = field(default_factory=list)
    block_table: list[int] = field(default_factory=list)
    num_computed_tokens: int = 0
    status: SequenceStatus = SequenceStatus.WAITING
    cached_prefix_blocks: int = 0
    # Running slots held for the samples that fork from this one once its prompt is computed.
    fork_slots: int = 0
    block_hashes: list[bytes] = field(default_factory=list)
    preemption_count: int = 0
    finish_reason: FinishReason | None = None
    admission_order: int = field(default_factory=lambda: next(_ORDER))

    @classmethod
    def from_request(cls, request: Request, sample_index: int) -> Sequence:
        return cls(
            seq_id=new_sequence_id(request.request_id, sample_index),
            request=request,
            sample_index=sample_index,
            token_ids=list(request.prompt_token_ids),
        )

    @property
    def num_tokens(self) -> int:
        return len(self.token_ids)

    @property
    def num_output_tokens(self) -> int:
        return len(self.token_ids) - self.request.prompt_len

    @property
    def num_uncomputed_tokens(self) -> int:
        return self.num_tokens - self.num_computed_tokens

    @property
    def output_token_ids(self) -> list[int]:
        return self.token_ids[self.request.prompt_len :]

    @property
    def is_decoding(self) -> bool:
        return self.num_computed_tokens > 0 and self.num_uncomputed_tokens == 1

    @property
    def is_finished(self) -> bool:
        return self.status is SequenceStatus.FINISHED

    def append_token(self, token_id: int) -> None:
        self.token_ids.append(token_id)

    def reset_for_recompute(self) -> None:
        """Forget the cached KV; sampled tokens stay and are recomputed (sequence.py:210-221)."""
        self.num_computed_tokens = 0
        self.block_table.clear()
        self.block_hashes.clear()
        self.cached_prefix_blocks = 0
        self.status = SequenceStatus.PREEMPTED
        self.preemption_count += 1

    def finish(self, reason: FinishReason) -> None:
        self.status = SequenceStatus.FINISHED
        self.finish_reason = reason

    def priority_key(self) -> tuple[int, float, int]:
        """One service class, no deadlines: arrival order (sequence.py:230-241)."""
        return (0, float("inf"), self.admission_order)


def finish_reason_for(
    sequence: Sequence, token: int, *, eos_token_id: int | None, max_context_tokens: int
) -> FinishReason | None:
    """Stop token, then the output cap, then the context cap (sequence.py:244-262)."""
    if eos_token_id is not None and token == eos_token_id:
        return FinishReason.STOP
    if sequence.num_output_tokens >= sequence.request.sampling.max_new_tokens:
        return FinishReason.LENGTH
    if sequence.num_tokens >= max_context_tokens:
        return FinishReason.CONTEXT_LIMIT
    return None
