"""Replay a recorded reference serving run through this package's KV-cache path.

The reference's Scheduler and Engine choose, every iteration, which sequences run how many
tokens, which are admitted, preempted, forked and finished. They call the data path and stay
the reference's (they are outside this build, and the reference does not exist on the GPU box).
A trace recorded from them (``tests/golden/make_reference_traces.py``) lists every call the
engine made into its ``KVCacheManager`` -- with the sequence state the call saw and what it
returned -- and every batch it executed, with its slot mapping and logits.

:class:`TraceReplay` issues the same calls in the same order to this package's
``KVCacheManager`` (over its ``BlockManager`` and ``PrefixCache``, with the runner as the block
store, so copy-on-write copies reach the pool exactly when the reference's did), builds every
batch from the block tables those calls produced, and executes it on a runner: the GPU
``ModelRunner``, or any object with ``execute(batch)`` and ``copy_block(source, destination)``.

With ``check=True`` each result is compared with the record when it happens: returned values,
block tables, copy-on-write pairs, prefix-hash chains, every batch's entries and slot mapping,
and after every iteration digests of the pool's owner counts, its free-list order, the cached
block ids in LRU order and the cache counters. The first difference raises
:class:`ReplayMismatch` naming the event. Sampled tokens come from the trace (the reference's
per-request samplers), so a run's batches are the reference's whatever the logits.
"""

from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from paged_kv_serving_amd.blocks import BlockAllocationError, BlockManager
from paged_kv_serving_amd.config import ModelConfig
from paged_kv_serving_amd.kvcache import KVCacheManager, PrefixReuse
from paged_kv_serving_amd.prefix_cache import PrefixCache
from paged_kv_serving_amd.sequence import Request, Sequence

__all__ = ["ReplayMismatch", "ReplayResult", "StaticReplay", "Trace", "TraceReplay", "digest_ints", "weights_sha256"]


class ReplayMismatch(AssertionError):
    """This package did something other than what the recorded reference run did."""


def digest_ints(values) -> str:
    """First 16 hex digits of SHA-256 over the values as little-endian int64."""
    return hashlib.sha256(np.asarray(list(values), dtype="<i8").tobytes()).hexdigest()[:16]


def _digest_hashes(hashes) -> str:
    return hashlib.sha256(b"".join(hashes)).hexdigest()[:16]


def weights_sha256(weights) -> str:
    """SHA-256 of every parameter as little-endian float32: the embedding, then per layer
    attn_norm, qkv_proj, out_proj, ffn_norm, gate_proj, up_proj, down_proj, then final_norm."""
    digest = hashlib.sha256()
    digest.update(np.ascontiguousarray(weights.token_embedding, dtype="<f4").tobytes())
    for layer in weights.layers:
        for name in ("attn_norm", "qkv_proj", "out_proj", "ffn_norm", "gate_proj", "up_proj", "down_proj"):
            digest.update(np.ascontiguousarray(getattr(layer, name), dtype="<f4").tobytes())
    digest.update(np.ascontiguousarray(weights.final_norm, dtype="<f4").tobytes())
    return digest.hexdigest()


@dataclass
class Trace:
    """A recorded reference run (the JSON written by the trace script, plus its logits rows)."""

    name: str
    model: dict
    engine: dict
    requests: list[dict]
    tokens: dict[str, list[int]]
    events: list[list]
    iterations: list[dict]
    summary: dict
    logits: np.ndarray | None = None
    kind: str = "engine"  # "engine": the continuous Engine; "static": the StaticBatchingEngine

    @classmethod
    def load(cls, path: str | Path) -> Trace:
        path = Path(path)
        data = json.loads(path.read_text())
        if data.get("format") != 1:
            raise ValueError(f"{path}: unknown trace format {data.get('format')}")
        rows = path.with_name(path.stem + "_logits.npy")
        logits = np.load(rows) if rows.exists() else None
        fields = ("name", "model", "engine", "requests", "tokens", "events", "iterations", "summary")
        return cls(**{k: data[k] for k in fields}, logits=logits, kind=data.get("kind", "engine"))

    def model_config(self) -> ModelConfig:
        m = self.model
        return ModelConfig(
            vocab_size=m["vocab_size"], d_model=m["d_model"], n_layers=m["n_layers"], n_heads=m["n_heads"],
            d_ff=m["d_ff"], max_seq_len=m["max_seq_len"], rope_theta=m["rope_theta"], norm_eps=m["norm_eps"],
        )  # fmt: skip

    def language_model(self):
        """The run's model: ``random_weights`` of its config and seed, checked against the
        SHA-256 of the reference's weights."""
        from paged_kv_serving_amd.model import LanguageModel, random_weights

        config = self.model_config()
        weights = random_weights(config, seed=self.model["seed"])
        if weights_sha256(weights) != self.model["weights_sha256"]:
            raise ReplayMismatch(f"{self.name}: random_weights(seed {self.model['seed']}) differs from the reference's")
        return LanguageModel(config, weights)

    @property
    def greedy_requests(self) -> set[str]:
        return {r["request_id"] for r in self.requests if r["temperature"] < 1e-5}


class _StoreTap:
    """The block store of the replayed pool: forwards copies to the runner and notes them."""

    def __init__(self, runner) -> None:
        self.runner = runner
        self.pairs: list[list[int]] = []

    def copy_block(self, source: int, destination: int) -> None:
        self.pairs.append([int(source), int(destination)])
        self.runner.copy_block(source, destination)


@dataclass
class ReplayResult:
    """What a replay produced: logits rows (or greedy token ids) in the trace's row order."""

    rows: list = field(default_factory=list)
    greedy: list[int] = field(default_factory=list)
    row_seqs: list[tuple[str, int]] = field(default_factory=list)  # (seq id, context length)
    iterations: int = 0
    copies: int = 0
    calls: int = 0


class TraceReplay:
    """Drives this package's KV-cache manager and a runner with a recorded reference run."""

    def __init__(self, trace: Trace, runner, *, check: bool = True, greedy: bool = False) -> None:
        engine = trace.engine
        self.trace = trace
        self.runner = runner
        self.check = check
        self.greedy = greedy
        self.block_size = engine["block_size"]
        self.store = _StoreTap(runner)
        self.blocks = BlockManager(num_blocks=engine["num_blocks"], block_size=self.block_size, store=self.store)
        self.prefix_cache = PrefixCache(
            self.blocks, enabled=engine["enable_prefix_cache"], scope=engine["prefix_cache_scope"]
        )
        self.cache = KVCacheManager(self.blocks, self.prefix_cache)
        self._requests = {
            r["request_id"]: Request(r["request_id"], tuple(r["prompt"]), n=r["n"], key_id=r["key_id"])
            for r in trace.requests
        }
        self.sequences: dict[str, Sequence] = {}
        self._event = 0

    # --- sequences -----------------------------------------------------------------------

    def _sequence(self, seq_id: str, num_tokens: int, num_computed: int | None = None) -> Sequence:
        """Our sequence ``seq_id``, with the token count (and computed count) the call saw."""
        seq = self.sequences.get(seq_id)
        if seq is None:
            request = self._requests[seq_id.rsplit("#", 1)[0]]
            seq = Sequence(seq_id, request)
            self.sequences[seq_id] = seq
        have = len(seq.token_ids)
        if have != num_tokens:
            tokens = self.trace.tokens[seq_id]
            if have + 1 == num_tokens:  # one token sampled since the last call
                seq.token_ids.append(tokens[have])
            else:
                seq.token_ids = tokens[:num_tokens]
        if num_computed is not None:
            seq.num_computed_tokens = num_computed
        return seq

    def _expect(self, what: str, got, want) -> None:
        if self.check and got != want:
            raise ReplayMismatch(f"{self.trace.name} event {self._event}: {what}: got {got!r}, reference {want!r}")

    # --- the run -------------------------------------------------------------------------

    def run(self) -> ReplayResult:
        result = ReplayResult()
        handlers = {
            "attach": self._attach, "record": self._record, "detach": self._detach, "reserve": self._reserve,
            "fork": self._fork, "free": self._free, "publish": self._publish, "evictable": self._evictable,
            "free_blocks": self._free_blocks, "sealed": self._sealed,
        }  # fmt: skip
        for index, event in enumerate(self.trace.events):
            self._event = index
            kind = event[0]
            if kind == "execute":
                self._execute(event[1], result)
            else:
                handlers[kind](*event[1:])
                result.calls += 1
        result.copies = len(self.store.pairs)
        if self.check:
            self.cache.check_invariants()
            if result.iterations != len(self.trace.iterations):
                raise ReplayMismatch(f"{self.trace.name}: {result.iterations} iterations replayed")
        return result

    def _attach(self, seq_id, record, num_tokens, num_computed, reuse, table_after, hashes_after) -> None:
        seq = self._sequence(seq_id, num_tokens, num_computed)
        got = self.cache.attach_prefix(seq, record=record)
        if self.check:
            self._expect(f"attach_prefix({seq_id})", [got.blocks, got.tokens, got.queried_blocks], reuse)
            self._expect(f"table of {seq_id} after attach", seq.block_table, table_after)
            self._expect(f"hash chain of {seq_id}", [len(seq.block_hashes), _digest_hashes(seq.block_hashes)],
                         hashes_after)  # fmt: skip

    def _record(self, queried, hits) -> None:
        self.cache.record_prefix(PrefixReuse(blocks=hits, tokens=hits * self.block_size, queried_blocks=queried))

    def _detach(self, seq_id, num_tokens, num_computed) -> None:
        self.cache.detach_prefix(self._sequence(seq_id, num_tokens, num_computed))

    def _reserve(self, seq_id, num_tokens, num_computed, up_to, ok, table_after, copies) -> None:
        seq = self._sequence(seq_id, num_tokens, num_computed)
        start = len(self.store.pairs)
        try:
            self.cache.reserve(seq, up_to)
            done = True
        except BlockAllocationError:
            done = False
        if self.check:
            self._expect(f"reserve({seq_id}, {up_to}) succeeded", done, ok)
            self._expect(f"table of {seq_id} after reserve", seq.block_table, table_after)
            self._expect(f"copy-on-write pairs of reserve({seq_id})", self.store.pairs[start:], copies)

    def _fork(self, parent_id, num_tokens, num_computed, child_id, child_tokens, table_after) -> None:
        parent = self._sequence(parent_id, num_tokens, num_computed)
        child = self._sequence(child_id, child_tokens)
        self.cache.fork(parent, child)
        self._expect(f"table of {child_id} after fork", child.block_table, table_after)

    def _free(self, seq_id, returned) -> None:
        seq = self.sequences[seq_id]
        self._expect(f"free({seq_id})", self.cache.free(seq), returned)

    def _publish(self, seq_id, num_tokens, num_computed, published, hashes_after) -> None:
        seq = self._sequence(seq_id, num_tokens, num_computed)
        got = self.cache.publish_full_blocks(seq)
        if self.check:
            self._expect(f"publish_full_blocks({seq_id})", got, published)
            self._expect(f"hash chain of {seq_id}", [len(seq.block_hashes), _digest_hashes(seq.block_hashes)],
                         hashes_after)  # fmt: skip

    def _evictable(self, value) -> None:
        self._expect("evictable_blocks()", self.cache.evictable_blocks(), value)

    def _free_blocks(self, value) -> None:
        self._expect("num_free_blocks", self.cache.num_free_blocks, value)

    def _sealed(self, iteration) -> None:
        if not self.check:
            return
        want = self.trace.iterations[iteration]["state"]
        stats = self.prefix_cache.stats
        got = {
            "refs": digest_ints(self.blocks.snapshot()),
            "free": digest_ints(self.blocks.free_order()),
            "free_count": self.blocks.num_free_blocks,
            "cached": digest_ints(self.prefix_cache.cached_block_ids()),
            "stats": [stats.queried_blocks, stats.hit_blocks, stats.registered_blocks, stats.evicted_blocks],
        }
        self._expect(f"allocator state after iteration {iteration}", got, want)

    def batch(self, iteration: int):
        """Iteration ``iteration``'s batch, built from this replay's own block tables."""
        from paged_kv_serving_amd.runner import BatchEntry, ExecutionBatch

        entries = []
        for seq_id, start, count, logits_index, table in self.trace.iterations[iteration]["entries"]:
            seq = self.sequences[seq_id]
            if self.check:
                self._expect(f"iteration {iteration} table of {seq_id}", seq.block_table, table)
            entries.append(
                BatchEntry(
                    seq_id=seq_id,
                    token_ids=tuple(self.trace.tokens[seq_id][start : start + count]),
                    positions=tuple(range(start, start + count)),
                    block_table=tuple(seq.block_table),
                    logits_index=None if logits_index < 0 else logits_index,
                )
            )
        return ExecutionBatch(tuple(entries))

    def _execute(self, iteration: int, result: ReplayResult) -> None:
        batch = self.batch(iteration)
        if self.check:
            from paged_kv_serving_amd.runner import compute_slots

            slots = compute_slots(batch.entries, self.block_size).tolist()
            self._expect(f"iteration {iteration} slot mapping", slots, self.trace.iterations[iteration]["slots"])
        wanted = [e for e in batch.entries if e.logits_index is not None]
        if self.greedy:
            tokens = self.runner.execute_greedy(batch)
            result.greedy.extend(tokens[e.seq_id] for e in wanted)
        else:
            logits = self.runner.execute(batch)
            result.rows.extend(logits[e.seq_id] for e in wanted)
        result.row_seqs.extend((e.seq_id, e.context_len) for e in wanted)
        result.iterations += 1


class StaticReplay:
    """Replays a recorded run of the reference's StaticBatchingEngine (static.py:183-226) on a
    runner. That engine owns no KV-cache manager: each of its ``batch_size`` slots is a fixed
    contiguous run of ``blocks_per_slot`` blocks (static.py:123-137), every group starts with a
    prefill padded to its longest prompt whose logits are read at each row's own last prompt
    token, and its decode rounds re-run finished rows at their last position. The batches are
    executed as recorded (token ids included, padding and re-runs too) on a runner made as the
    engine makes its own (static.py:124-126: ``batch_size * blocks_per_slot`` blocks).

    With ``check=True`` every block table must be one whole slot region and every slot mapping
    the reference's. A row's context in :attr:`ReplayResult.row_seqs` is the position its logits
    are read at, plus one."""

    def __init__(self, trace: Trace, runner, *, check: bool = True, greedy: bool = False) -> None:
        if trace.kind != "static":
            raise ValueError(f"{trace.name} is not a static-batching trace")
        self.trace = trace
        self.runner = runner
        self.check = check
        self.greedy = greedy
        self.block_size = trace.engine["block_size"]
        self.per_slot = trace.engine["blocks_per_slot"]

    def batch(self, iteration: int):
        from paged_kv_serving_amd.runner import BatchEntry, ExecutionBatch

        entries = []
        for seq_id, start, tokens, logits_index, table in self.trace.iterations[iteration]["entries"]:
            first = table[0] if table else -1
            if self.check and (first % self.per_slot or table != list(range(first, first + self.per_slot))):
                raise ReplayMismatch(f"{self.trace.name} iteration {iteration}: {seq_id}'s table is not a slot region")
            entries.append(
                BatchEntry(
                    seq_id=seq_id,
                    token_ids=tuple(tokens),
                    positions=tuple(range(start, start + len(tokens))),
                    block_table=tuple(table),
                    logits_index=None if logits_index < 0 else logits_index,
                )
            )
        return ExecutionBatch(tuple(entries))

    def run(self) -> ReplayResult:
        from paged_kv_serving_amd.runner import compute_slots

        result = ReplayResult()
        for iteration, record in enumerate(self.trace.iterations):
            batch = self.batch(iteration)
            if self.check:
                slots = compute_slots(batch.entries, self.block_size).tolist()
                if slots != record["slots"]:
                    raise ReplayMismatch(f"{self.trace.name} iteration {iteration}: slot mapping differs")
            wanted = [e for e in batch.entries if e.logits_index is not None]
            if self.greedy:
                tokens = self.runner.execute_greedy(batch)
                result.greedy.extend(tokens[e.seq_id] for e in wanted)
            else:
                logits = self.runner.execute(batch)
                result.rows.extend(logits[e.seq_id] for e in wanted)
            result.row_seqs.extend((e.seq_id, e.positions[e.logits_index] + 1) for e in wanted)
            result.iterations += 1
        return result
