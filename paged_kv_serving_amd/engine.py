"""A continuous-batching loop that drives the GPU ModelRunner the way the reference engine does.

The scheduler and engine are callers of the data path, not part of it. This module restates
their behaviour for a single service class with no deadlines, so the path can run end to end
(the config-1 workload) without the reference's code:

* ``Scheduler.schedule`` follows src/paged_kv_serving/engine/scheduler.py:209-425:
  - decode rows first, one token per decoding sequence in priority order;
  - when the pool runs dry, the lowest-priority unscheduled sequence is preempted and
    recomputed later;
  - then one pass in priority order continues running prefills and admits waiting sequences
    with their first chunk, within the token budget, the running-slot cap and the admission
    watermark.
  The order of ``KVCacheManager.reserve`` calls, and so every block id, is the reference's.
* ``Engine.step`` follows engine.py:413-465: schedule, execute, advance
  ``num_computed_tokens``, publish full blocks to the prefix cache, sample greedily from the
  returned rows, fork the remaining samples of an n-way request, and free finished sequences.

Sampling is greedy (``argmax``, ties to the lowest id, sampling.py:28-30), the only policy the
data-path runs use. With the GPU runner it runs on the device (``ModelRunner.execute_greedy``,
one int32 per row back to the host); an executor with only ``execute`` (the NumPy runner, a
recording wrapper) is sampled on the host with the same rule.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

import numpy as np

from paged_kv_serving_amd.blocks import BlockAllocationError, BlockManager
from paged_kv_serving_amd.config import EngineConfig
from paged_kv_serving_amd.kvcache import KVCacheManager
from paged_kv_serving_amd.prefix_cache import PrefixCache
from paged_kv_serving_amd.runner import BatchEntry, ExecutionBatch, ModelRunner
from paged_kv_serving_amd.sequence import (
    Request,
    Sequence,
    SequenceStatus,
    finish_reason_for,
)

__all__ = ["Engine", "RecordingExecutor", "Scheduler", "ScheduledSequence", "SchedulerOutput", "greedy_token"]


@dataclass(frozen=True)
class ScheduledSequence:
    """A sequence, the tokens it computes this iteration, and whether it then samples."""

    sequence: Sequence
    num_tokens: int
    is_prefill: bool
    produces_token: bool


@dataclass(frozen=True)
class SchedulerOutput:
    batch: ExecutionBatch
    scheduled: tuple[ScheduledSequence, ...] = ()
    preempted: tuple[str, ...] = ()
    admitted: tuple[str, ...] = ()

    @property
    def is_empty(self) -> bool:
        return not self.scheduled


class Scheduler:
    """Waiting and running queues over one KV pool (scheduler.py:114-425, one service class)."""

    def __init__(self, config: EngineConfig, cache: KVCacheManager) -> None:
        self.config = config
        self.cache = cache
        self.waiting: list[Sequence] = []
        self.running: list[Sequence] = []
        self.preemptions = 0

    @property
    def has_work(self) -> bool:
        return bool(self.waiting or self.running)

    def slots_in_use(self) -> int:
        return sum(1 + seq.fork_slots for seq in self.running)

    def add(self, sequence: Sequence) -> None:
        sequence.status = SequenceStatus.WAITING
        self.waiting.append(sequence)

    def add_running(self, sequence: Sequence) -> None:
        sequence.status = SequenceStatus.RUNNING
        self.running.append(sequence)

    def drop_finished(self) -> list[Sequence]:
        finished = [seq for seq in self.running if seq.is_finished]
        for seq in finished:
            self.running.remove(seq)
            self.cache.free(seq)
        return finished

    def _preempt(self, victim: Sequence, preempted: list[str]) -> None:
        self.running.remove(victim)
        self.cache.free(victim)
        victim.reset_for_recompute()
        self.waiting.append(victim)
        self.preemptions += 1
        preempted.append(victim.seq_id)

    def _max_chunk_by_memory(self, seq: Sequence, reserve_blocks: int) -> int:
        available = self.cache.num_free_blocks + self.cache.evictable_blocks() - reserve_blocks
        capacity = (len(seq.block_table) + max(0, available)) * self.cache.block_size
        return capacity - seq.num_computed_tokens

    def schedule(self) -> SchedulerOutput:
        budget = self.config.max_batched_tokens
        scheduled: list[ScheduledSequence] = []
        preempted: list[str] = []
        admitted: list[str] = []
        budget = self._schedule_decodes(budget, scheduled, preempted)
        self._schedule_prefills(budget, scheduled, preempted, admitted)
        self.waiting.sort(key=lambda s: s.priority_key())
        entries = tuple(self._entry(item) for item in scheduled)
        return SchedulerOutput(ExecutionBatch(entries), tuple(scheduled), tuple(preempted), tuple(admitted))

    def _schedule_decodes(self, budget, scheduled, preempted) -> int:
        """One token per decoding sequence, preempting when the pool runs dry (:248-275)."""
        pending = deque(s for s in sorted(self.running, key=lambda s: s.priority_key()) if s.is_decoding)
        while pending and budget > 0:
            seq = pending[0]
            try:
                self.cache.reserve(seq, seq.num_tokens)
            except BlockAllocationError:
                prefilling = [s for s in self.running if not s.is_decoding]
                victim = max([*prefilling, pending[-1]], key=lambda s: s.priority_key())
                if victim is pending[-1]:
                    pending.pop()
                self._preempt(victim, preempted)
                continue
            pending.popleft()
            scheduled.append(ScheduledSequence(seq, 1, is_prefill=False, produces_token=True))
            budget -= 1
        return budget

    def _schedule_prefills(self, budget, scheduled, preempted, admitted) -> int:
        """Running prefills and waiting sequences in one priority-ordered pass (:277-321)."""
        self.waiting.sort(key=lambda s: s.priority_key())
        order = sorted(
            [*(s for s in self.running if not s.is_decoding), *self.waiting], key=lambda s: s.priority_key()
        )
        admitting = not preempted
        for position, seq in enumerate(order):
            if budget <= 0:
                break
            if seq.status is SequenceStatus.RUNNING:
                before = len(preempted)
                budget = self._continue_prefill(seq, budget, order[position + 1 :], scheduled, preempted)
                admitting = admitting and len(preempted) == before
            elif admitting:
                spent = self._admit(seq, budget, scheduled, admitted)
                admitting = spent > 0
                budget -= spent
        return budget

    def _continue_prefill(self, seq, budget, behind, scheduled, preempted) -> int:
        """Next chunk of a running prompt; preempt a running prefill behind it if needed (:323-369)."""
        wanted = min(budget, seq.num_uncomputed_tokens)
        if wanted <= 0:
            return budget
        chunk = min(wanted, self._max_chunk_by_memory(seq, 0))
        while chunk <= 0:
            victims = [o for o in behind if o.status is SequenceStatus.RUNNING and o.block_table]
            if not victims:
                return budget
            self._preempt(victims[-1], preempted)
            chunk = min(wanted, self._max_chunk_by_memory(seq, 0))
        try:
            self.cache.reserve(seq, seq.num_computed_tokens + chunk)
        except BlockAllocationError:
            return budget
        produces = seq.num_computed_tokens + chunk == seq.num_tokens
        scheduled.append(ScheduledSequence(seq, chunk, is_prefill=True, produces_token=produces))
        return budget - chunk

    def _admit(self, seq, budget, scheduled, admitted) -> int:
        """Admit a waiting sequence with its first chunk; 0 when it cannot start (:371-413)."""
        if self.slots_in_use() + 1 + seq.fork_slots > self.config.max_running_seqs:
            return 0
        reuse = self.cache.attach_prefix(seq, record=False)
        watermark = int(self.config.watermark * self.cache.blocks.num_blocks) if self.running else 0
        chunk = min(budget, seq.num_uncomputed_tokens)
        chunk = min(chunk, self._max_chunk_by_memory(seq, watermark))
        if chunk <= 0:
            self.cache.detach_prefix(seq)
            return 0
        try:
            self.cache.reserve(seq, seq.num_computed_tokens + chunk)
        except BlockAllocationError:
            self.cache.detach_prefix(seq)
            return 0
        self.cache.record_prefix(reuse)
        self.waiting.remove(seq)
        seq.status = SequenceStatus.RUNNING
        self.running.append(seq)
        produces = seq.num_computed_tokens + chunk == seq.num_tokens
        scheduled.append(ScheduledSequence(seq, chunk, is_prefill=True, produces_token=produces))
        admitted.append(seq.seq_id)
        return chunk

    @staticmethod
    def _entry(item: ScheduledSequence) -> BatchEntry:
        seq = item.sequence
        start = seq.num_computed_tokens
        stop = start + item.num_tokens
        return BatchEntry(
            seq_id=seq.seq_id,
            token_ids=tuple(seq.token_ids[start:stop]),
            positions=tuple(range(start, stop)),
            block_table=tuple(seq.block_table),
            logits_index=item.num_tokens - 1 if item.produces_token else None,
        )


def greedy_token(logits: np.ndarray) -> int:
    """Highest-scoring token id, ties to the lowest id (reference sampling.py:28-30, 62-65)."""
    if logits.ndim != 1:
        raise ValueError("logits must be a 1-D array over the vocabulary")
    return int(np.argmax(logits))


@dataclass
class RecordingExecutor:
    """Executes on a runner and keeps a copy of every logits row (equivalence.py:120-139)."""

    runner: object
    records: list[tuple[str, int, np.ndarray]] = field(default_factory=list)

    def execute(self, batch: ExecutionBatch) -> dict[str, np.ndarray]:
        result = self.runner.execute(batch)
        for entry in batch.entries:
            row = result.get(entry.seq_id)
            if row is not None:
                self.records.append((entry.seq_id, entry.context_len, row.copy()))
        return result


@dataclass
class _RequestState:
    request: Request
    sequences: dict[int, Sequence] = field(default_factory=dict)
    pending_forks: list[Sequence] = field(default_factory=list)
    finished: dict[int, tuple[int, ...]] = field(default_factory=dict)


class Engine:
    """Continuous batching over a paged KV cache on the GPU (engine.py:174-465, greedy)."""

    def __init__(
        self,
        model,
        config: EngineConfig | None = None,
        *,
        runner: ModelRunner | None = None,
        eos_token_id: int | None = None,
        **runner_options,
    ) -> None:
        self.config = config or EngineConfig()
        if self.config.max_context_tokens > model.config.max_seq_len:
            raise ValueError("max_context_tokens exceeds the model's max_seq_len")
        self.model = model
        self.eos_token_id = eos_token_id
        self.runner = runner or ModelRunner(
            model, num_blocks=self.config.num_blocks, block_size=self.config.block_size, **runner_options
        )
        self.executor = self.runner
        self.blocks = BlockManager(
            num_blocks=self.config.num_blocks, block_size=self.config.block_size, store=self.runner
        )
        self.prefix_cache = PrefixCache(self.blocks, enabled=self.config.enable_prefix_cache)
        self.cache = KVCacheManager(self.blocks, self.prefix_cache)
        self.scheduler = Scheduler(self.config, self.cache)
        self._requests: dict[str, _RequestState] = {}
        self.iterations = 0

    @property
    def has_work(self) -> bool:
        return self.scheduler.has_work or any(s.pending_forks for s in self._requests.values())

    def submit(self, request: Request) -> None:
        """Queue a request; its n - 1 extra samples fork once the prompt is computed."""
        if request.request_id in self._requests:
            raise ValueError(f"request {request.request_id} is already in flight")
        if request.prompt_len > self.config.max_prompt_tokens:
            raise ValueError("prompt longer than max_prompt_tokens")
        sampling = request.sampling
        if (
            sampling.max_new_tokens > self.config.max_new_tokens
            or request.prompt_len + sampling.max_new_tokens > self.config.max_context_tokens
        ):
            raise ValueError("request exceeds max_new_tokens or max_context_tokens")
        state = _RequestState(request)
        primary = Sequence.from_request(request, 0)
        primary.fork_slots = request.n - 1
        state.sequences[0] = primary
        for index in range(1, request.n):
            child = Sequence.from_request(request, index)
            state.sequences[index] = child
            state.pending_forks.append(child)
        self._requests[request.request_id] = state
        self.scheduler.add(primary)

    def step(self) -> SchedulerOutput:
        """One iteration (engine.py:413-465)."""
        output = self.scheduler.schedule()
        if output.is_empty:
            return output
        self.iterations += 1
        # An executor that samples on the device (ModelRunner.execute_greedy) returns token ids;
        # any other returns host logits rows, sampled here with the same argmax rule.
        device_greedy = getattr(self.executor, "execute_greedy", None)
        if device_greedy is not None:
            tokens = device_greedy(output.batch)
        else:
            tokens = {seq_id: greedy_token(row) for seq_id, row in self.executor.execute(output.batch).items()}
        for item in output.scheduled:
            seq = item.sequence
            seq.num_computed_tokens += item.num_tokens
            self.cache.publish_full_blocks(seq)
            if not item.produces_token:
                continue
            token = tokens[seq.seq_id]
            self._fork_pending(seq, token)
            self._emit(seq, token)
        for seq in self.scheduler.drop_finished():
            state = self._requests.get(seq.request.request_id)
            if state is not None:
                state.finished[seq.sample_index] = tuple(seq.output_token_ids)
        return output

    def _fork_pending(self, seq: Sequence, token: int) -> None:
        state = self._requests.get(seq.request.request_id)
        if state is None or seq.sample_index != 0 or seq.num_output_tokens:
            return
        for child in state.pending_forks:
            self.cache.fork(seq, child)
            self.scheduler.add_running(child)
            self._emit(child, token)
        state.pending_forks.clear()
        seq.fork_slots = 0

    def _emit(self, seq: Sequence, token: int) -> None:
        seq.append_token(token)
        reason = finish_reason_for(
            seq, token, eos_token_id=self.eos_token_id, max_context_tokens=self.config.max_context_tokens
        )
        if reason is not None:
            seq.finish(reason)

    def run_until_idle(self, max_iterations: int = 100_000) -> dict[str, list[tuple[int, ...]]]:
        """Step until nothing is left; returns each request's samples' output tokens."""
        for _ in range(max_iterations):
            if not self.has_work:
                break
            if self.step().is_empty and self.scheduler.has_work:
                raise RuntimeError(
                    f"the scheduler produced an empty batch with {len(self.scheduler.running)} "
                    f"running and {len(self.scheduler.waiting)} waiting sequences"
                )
        else:
            raise RuntimeError(f"engine did not drain within {max_iterations} iterations")
        outputs = {}
        for request_id, state in list(self._requests.items()):
            if len(state.finished) == state.request.n:
                outputs[request_id] = [state.finished[i] for i in range(state.request.n)]
                del self._requests[request_id]
        return outputs

    def generate(self, requests) -> dict[str, list[tuple[int, ...]]]:
        for request in requests:
            self.submit(request)
        return self.run_until_idle()

    def check_invariants(self) -> None:
        self.cache.check_invariants()
