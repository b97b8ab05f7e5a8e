"""Write golden traces of the reference engine: every KV-cache call, batch, slot mapping, COW pair
and logits row of a seeded run.

Runs only in the build container, where the reference sources are present
(``PKV_REFERENCE``, default ``/root/reference``); the traces it writes under
``tests/golden/traces/`` are plain data and are all the tests and the GPU box ever read.

Why an import: the block tables a serving run produces depend on the reference scheduler's
ordering (``scheduler.py:209-425``: decode first, one priority pass of prefills and admissions,
chunking, the watermark, preemption), on ``KVCacheManager`` (``kvcache.py:148-195``) and on the
prefix cache's LRU (``prefix_cache.py:109-202``). No closed form pins those, and neither does the
``random_weights`` draw order (``model.py:173-203``), so this script runs the reference itself
and records what it did. The scheduler is a caller of the data path and stays the reference's;
the traces let the tests drive this repository's ``KVCacheManager`` / ``BlockManager`` /
``PrefixCache`` and ``ModelRunner`` with exactly the calls the reference engine makes.

The reference needs Python 3.12; two standard-library names it uses are filled in for 3.10
(``typing.Self`` from ``typing_extensions``, ``datetime.UTC``), and the package ``__init__``
modules are replaced by empty namespace modules so that only the engine modules load.

Each trace is ``<name>.json`` plus ``<name>_logits.npy`` (float32 rows in the order the
iterations returned them). Event records (lists, in call order):

    ["attach", seq, record, num_tokens, num_computed, [blocks, tokens, queried], table_after, hashes_after]
    ["record", queried, hits]
    ["detach", seq, num_tokens, num_computed]
    ["reserve", seq, num_tokens, num_computed, up_to, ok, table_after, copies]
    ["fork", parent, num_tokens, num_computed, child, child_num_tokens, table_after]
    ["free", seq, returned]
    ["publish", seq, num_tokens, num_computed, published, hashes_after]
    ["evictable", value]      ["free_blocks", value]
    ["execute", iteration]    ["sealed", iteration]   (the end of that iteration's step)

``table_after`` is the sequence's block table after the call, ``copies`` the (source,
destination) block copies the call asked the store for, and ``hashes_after`` the number of
block hashes the sequence holds plus a digest of them. Each iteration records its batch entries
``[seq, first position, tokens, logits index or -1, block table]``, the slot mapping the
reference runner computes (``runner.py:149-159``) and digests of the allocator state after the
step (reference counts, free-list order, cached block ids in LRU order, cache counters).

Usage: python tests/golden/make_reference_traces.py [--check]
"""

from __future__ import annotations

import argparse
import dataclasses
import datetime
import hashlib
import importlib
import json
import os
import sys
import tempfile
import types
import typing
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
OUT = HERE / "traces"
REFERENCE = Path(os.environ.get("PKV_REFERENCE", "/root/reference"))


def _reference():
    """The reference's engine modules, loaded from its sources (no bytecode is written next to
    them: the reference tree stays as it is)."""
    import typing_extensions

    sys.dont_write_bytecode = True

    if not hasattr(typing, "Self"):
        typing.Self = typing_extensions.Self
    if not hasattr(datetime, "UTC"):
        datetime.UTC = datetime.timezone.utc
    src = REFERENCE / "src" / "paged_kv_serving"
    if not src.is_dir():
        raise SystemExit(f"reference sources not found under {REFERENCE}")
    for name, path in (("paged_kv_serving", src), ("paged_kv_serving.engine", src / "engine")):
        module = types.ModuleType(name)
        module.__path__ = [str(path)]
        sys.modules[name] = module
    names = ("config", "blocks", "kvcache", "model", "runner", "engine", "sequence", "equivalence", "weights",
             "static")  # fmt: skip
    return types.SimpleNamespace(**{n: importlib.import_module(f"paged_kv_serving.engine.{n}") for n in names})


def digest_ints(values) -> str:
    return hashlib.sha256(np.asarray(list(values), dtype="<i8").tobytes()).hexdigest()[:16]


def digest_hashes(hashes) -> str:
    return hashlib.sha256(b"".join(hashes)).hexdigest()[:16]


def weights_sha256(weights) -> str:
    """SHA-256 over every parameter in draw-independent order: embedding, then per layer the
    seven matrices/vectors, then the final norm (little-endian float32 bytes)."""
    digest = hashlib.sha256()
    digest.update(np.ascontiguousarray(weights.token_embedding, dtype="<f4").tobytes())
    for layer in weights.layers:
        for name in ("attn_norm", "qkv_proj", "out_proj", "ffn_norm", "gate_proj", "up_proj", "down_proj"):
            digest.update(np.ascontiguousarray(getattr(layer, name), dtype="<f4").tobytes())
    digest.update(np.ascontiguousarray(weights.final_norm, dtype="<f4").tobytes())
    return digest.hexdigest()


class CopyLog:
    """The block store behind the reference BlockManager: forwards to the runner, logs pairs."""

    def __init__(self, runner) -> None:
        self.runner = runner
        self.pairs: list[list[int]] = []

    def copy_block(self, source: int, destination: int) -> None:
        self.pairs.append([int(source), int(destination)])
        self.runner.copy_block(source, destination)


class CacheLog:
    """Stands in for the reference KVCacheManager in front of its Scheduler and Engine, logging
    every call with the state of the sequences it touches."""

    def __init__(self, cache, copies: CopyLog) -> None:
        self._cache = cache
        self._copies = copies
        self.events: list[list] = []

    def __getattr__(self, name):  # blocks, prefix_cache, block_size, utilization, ...
        return getattr(self._cache, name)

    @property
    def num_free_blocks(self) -> int:
        value = self._cache.num_free_blocks
        self.events.append(["free_blocks", value])
        return value

    def evictable_blocks(self) -> int:
        value = self._cache.evictable_blocks()
        self.events.append(["evictable", value])
        return value

    def attach_prefix(self, sequence, *, record: bool = True):
        num_tokens, num_computed = sequence.num_tokens, sequence.num_computed_tokens
        reuse = self._cache.attach_prefix(sequence, record=record)
        self.events.append([
            "attach", sequence.seq_id, record, num_tokens, num_computed,
            [reuse.blocks, reuse.tokens, reuse.queried_blocks],
            list(sequence.block_table), [len(sequence.block_hashes), digest_hashes(sequence.block_hashes)],
        ])  # fmt: skip
        return reuse

    def record_prefix(self, reuse) -> None:
        self.events.append(["record", reuse.queried_blocks, reuse.blocks])
        self._cache.record_prefix(reuse)

    def detach_prefix(self, sequence) -> None:
        self.events.append(["detach", sequence.seq_id, sequence.num_tokens, sequence.num_computed_tokens])
        self._cache.detach_prefix(sequence)

    def reserve(self, sequence, up_to_tokens: int) -> None:
        record = ["reserve", sequence.seq_id, sequence.num_tokens, sequence.num_computed_tokens, up_to_tokens]
        start = len(self._copies.pairs)
        try:
            self._cache.reserve(sequence, up_to_tokens)
        except Exception as error:
            if type(error).__name__ != "BlockAllocationError":
                raise
            self.events.append([*record, False, list(sequence.block_table), self._copies.pairs[start:]])
            raise
        self.events.append([*record, True, list(sequence.block_table), self._copies.pairs[start:]])

    def fork(self, parent, child) -> None:
        record = ["fork", parent.seq_id, parent.num_tokens, parent.num_computed_tokens, child.seq_id, child.num_tokens]
        self._cache.fork(parent, child)
        self.events.append([*record, list(child.block_table)])

    def free(self, sequence) -> int:
        returned = self._cache.free(sequence)
        self.events.append(["free", sequence.seq_id, returned])
        return returned

    def publish_full_blocks(self, sequence) -> int:
        record = ["publish", sequence.seq_id, sequence.num_tokens, sequence.num_computed_tokens]
        published = self._cache.publish_full_blocks(sequence)
        self.events.append([*record, published, [len(sequence.block_hashes), digest_hashes(sequence.block_hashes)]])
        return published


class ExecuteLog:
    """The engine's executor: runs the reference runner and records batches, slots and rows."""

    def __init__(self, ref, runner, cache_log: CacheLog, blocks, prefix_cache) -> None:
        self.ref = ref
        self.runner = runner
        self.cache_log = cache_log
        self.blocks = blocks
        self.prefix_cache = prefix_cache
        self.iterations: list[dict] = []
        self.rows: list[np.ndarray] = []
        self.records: list = []

    def execute(self, batch):
        self.cache_log.events.append(["execute", len(self.iterations)])
        result = self.runner.execute(batch)
        entries, slots = [], []
        for entry in batch.entries:
            index = -1 if entry.logits_index is None else entry.logits_index
            entries.append([entry.seq_id, entry.positions[0], entry.num_tokens, index, list(entry.block_table)])
            slots.extend(int(s) for s in self.runner._slots(entry))
            row = result.get(entry.seq_id)
            if row is not None:
                self.rows.append(np.asarray(row, dtype=np.float32).copy())
                self.records.append(self.ref.equivalence.LogitRecord(entry.seq_id, entry.context_len, row.copy()))
        self.iterations.append({"entries": entries, "slots": slots})
        return result

    def seal_state(self) -> None:
        """Allocator state at the end of the step that the last execute belongs to (after its
        publishes, forks and frees), marked by a ``["sealed", iteration]`` event."""
        self.cache_log.events.append(["sealed", len(self.iterations) - 1])
        stats = self.prefix_cache.stats
        self.iterations[-1]["state"] = {
            "refs": digest_ints(self.blocks.snapshot()),
            "free": digest_ints(self.blocks._free),
            "free_count": self.blocks.num_free_blocks,
            "cached": digest_ints(self.prefix_cache.cached_block_ids()),
            "stats": [stats.queried_blocks, stats.hit_blocks, stats.registered_blocks, stats.evicted_blocks],
        }


def run_trace(ref, name: str, model, model_seed: int, engine_config, requests, *, scope: str = "per_key") -> dict:
    engine = ref.engine.Engine(model, engine_config, prefix_cache_scope=scope)
    copies = CopyLog(engine.runner)
    engine.blocks._store = copies
    cache_log = CacheLog(engine.cache, copies)
    engine.cache = cache_log
    engine.scheduler.cache = cache_log
    executor = ExecuteLog(ref, engine.runner, cache_log, engine.blocks, engine.prefix_cache)
    engine.executor = executor

    admitted = [r.request_id for r in requests if engine.submit(r).admitted]
    outputs = []
    for _ in range(100_000):
        if not engine.has_work:
            break
        step = engine.step()
        outputs.extend(step.finished)
        if not step.is_empty:
            executor.seal_state()
        elif engine.scheduler.has_work:
            raise RuntimeError("the reference scheduler produced an empty batch with work queued")
    else:
        raise RuntimeError("the reference engine did not drain")
    engine.check_invariants()
    tokens = ref.equivalence.sequence_tokens(
        requests, {o.request_id: [s.token_ids for s in o.samples] for o in outputs}
    )
    gap, rows = ref.equivalence.engine_logit_gap(model, executor.records, tokens)
    cfg = model.config
    trace = {
        "format": 1,
        "name": name,
        "model": {
            "vocab_size": cfg.vocab_size, "d_model": cfg.d_model, "n_layers": cfg.n_layers,
            "n_heads": cfg.n_heads, "d_ff": cfg.d_ff, "max_seq_len": cfg.max_seq_len,
            "rope_theta": cfg.rope_theta, "norm_eps": cfg.norm_eps, "seed": model_seed,
            "weights_sha256": weights_sha256(model.weights),
        },
        "engine": {
            "block_size": engine_config.block_size, "num_blocks": engine_config.num_blocks,
            "max_batched_tokens": engine_config.max_batched_tokens,
            "max_running_seqs": engine_config.max_running_seqs,
            "enable_prefix_cache": engine_config.enable_prefix_cache, "watermark": engine_config.watermark,
            "prefix_cache_scope": scope,
        },
        "requests": [
            {"request_id": r.request_id, "prompt": list(r.prompt_token_ids), "n": r.n, "key_id": r.key_id,
             "max_new_tokens": r.sampling.max_new_tokens, "temperature": r.sampling.temperature,
             "seed": r.sampling.seed}
            for r in requests
        ],
        "admitted": admitted,
        "tokens": tokens,
        "events": cache_log.events,
        "iterations": executor.iterations,
        "summary": {
            "iterations": len(executor.iterations),
            "logits_rows": len(executor.rows),
            "preemptions": engine.scheduler.stats.preemptions,
            "prefix_hit_blocks": engine.prefix_cache.stats.hit_blocks,
            "copies": len(copies.pairs),
            "rows_checked": rows,
            "reference_max_abs_logit_gap": gap,
        },
    }  # fmt: skip
    logits = np.stack(executor.rows) if executor.rows else np.zeros((0, cfg.vocab_size), np.float32)
    return trace, logits


# --- the workloads ---------------------------------------------------------------------------


def config1(ref):
    """random_weights(seed 0) of a 2-layer, 4 x 32-head, vocab-256 decoder; 32
    requests with prompts of U[16, 128] random tokens (one default_rng(0) draws each length,
    then its tokens), 32 greedy tokens each, EngineConfig defaults."""
    config = ref.config.ModelConfig(vocab_size=256, d_model=128, n_layers=2, n_heads=4, d_ff=320, max_seq_len=1024)
    model = ref.model.LanguageModel(config, ref.model.random_weights(config, seed=0))
    rng = np.random.default_rng(0)
    requests = []
    for i in range(32):
        length = int(rng.integers(16, 129))
        prompt = tuple(int(t) for t in rng.integers(0, 256, length))
        requests.append(ref.sequence.Request(f"req{i}", prompt, ref.sequence.SamplingParams(max_new_tokens=32, seed=i)))
    return run_trace(ref, "config1", model, 0, ref.config.EngineConfig(), requests)


def engine_equivalence(ref):
    """bench_engine_equivalence (bench/bench_baseline.py:241-284) at its own shape: the
    build_random_checkpoint(seed 3, max_seq_len 512) model, a 20-block pool with a 48-token
    budget and no watermark, 16 requests (odd ones behind a shared 32-token prefix, n = 2 for
    every fifth, temperature 0.9 for every third), drawn from default_rng(6) as the benchmark does."""
    with tempfile.TemporaryDirectory() as tmp:
        checkpoint = ref.weights.build_random_checkpoint(Path(tmp) / "checkpoint", seed=3, max_seq_len=512)
    model = checkpoint.model
    base = ref.config.EngineConfig(
        block_size=16, num_blocks=192, max_batched_tokens=128, max_running_seqs=12,
        max_prompt_tokens=192, max_new_tokens=24, max_context_tokens=256,
    )  # fmt: skip
    config = dataclasses.replace(base, num_blocks=20, max_batched_tokens=48, watermark=0.0)
    rng = np.random.default_rng(6)
    vocab = min(model.config.vocab_size, 256)
    shared = [int(v) for v in rng.integers(1, vocab, 32)]
    requests = []
    for index in range(16):
        tail = [int(v) for v in rng.integers(1, vocab, int(rng.integers(8, 90)))]
        requests.append(
            ref.sequence.Request(
                request_id=f"eq-{index}",
                prompt_token_ids=tuple([*shared, *tail] if index % 2 else tail),
                sampling=ref.sequence.SamplingParams(
                    max_new_tokens=int(rng.integers(4, 24)), temperature=0.0 if index % 3 else 0.9, seed=index
                ),
                n=2 if index % 5 == 0 else 1,
            )
        )
    return run_trace(ref, "engine_equivalence", model, 3, config, requests)


def sharing(ref, name: str, seed: int, *, block_size: int, num_blocks: int, n_heads: int, d_model: int):
    """Small pools under prefix sharing: three shared prompt stems across two keys, n-way samples
    (fork, then copy-on-write of the shared partial block), preemption and cache eviction."""
    config = ref.config.ModelConfig(vocab_size=96, d_model=d_model, n_layers=2, n_heads=n_heads,
                                    d_ff=2 * d_model, max_seq_len=256)  # fmt: skip
    model = ref.model.LanguageModel(config, ref.model.random_weights(config, seed=seed))
    engine_config = ref.config.EngineConfig(
        block_size=block_size, num_blocks=num_blocks, max_batched_tokens=64, max_running_seqs=8,
        max_prompt_tokens=96, max_new_tokens=20, max_context_tokens=128, watermark=0.0,
    )  # fmt: skip
    rng = np.random.default_rng(seed)
    stems = [[int(t) for t in rng.integers(0, 96, int(rng.integers(12, 40)))] for _ in range(3)]
    requests = []
    for i in range(18):
        stem = stems[int(rng.integers(0, 3))] if i % 4 else []
        tail = [int(t) for t in rng.integers(0, 96, int(rng.integers(1, 30)))]
        requests.append(
            ref.sequence.Request(
                request_id=f"{name}-{i}",
                prompt_token_ids=tuple(stem + tail),
                sampling=ref.sequence.SamplingParams(
                    max_new_tokens=int(rng.integers(2, 20)), temperature=0.0 if i % 3 else 0.8, seed=seed + i
                ),
                n=int(rng.choice([1, 1, 2, 3])),
                key_id="alice" if i % 5 else "bob",
            )
        )
    return run_trace(ref, name, model, seed, engine_config, requests)


class StaticLog:
    """The StaticBatchingEngine's runner (static.py:124): runs the reference runner and records
    every batch as the engine built it (explicit token ids, so the padded prefill and the
    re-run rows of finished sequences are kept), its slot mapping and its logits rows."""

    def __init__(self, runner) -> None:
        self.runner = runner
        self.iterations: list[dict] = []
        self.rows: list[np.ndarray] = []

    def execute(self, batch):
        result = self.runner.execute(batch)
        entries, slots = [], []
        for entry in batch.entries:
            start = entry.positions[0]
            if list(entry.positions) != list(range(start, start + entry.num_tokens)):
                raise RuntimeError("the static engine ran non-consecutive positions")
            index = -1 if entry.logits_index is None else entry.logits_index
            entries.append([entry.seq_id, start, list(entry.token_ids), index, list(entry.block_table)])
            slots.extend(int(s) for s in self.runner._slots(entry))
            if entry.logits_index is not None:
                self.rows.append(np.asarray(result[entry.seq_id], dtype=np.float32).copy())
        self.iterations.append({"entries": entries, "slots": slots})
        return result


def static_batching(ref):
    """StaticBatchingEngine (static.py:79-257), the caller of ModelRunner.execute whose batches
    differ from the continuous engine's: fixed groups of batch_size requests, a prefill padded to
    the group's longest prompt with logits read at each row's own last prompt token
    (static.py:188-198), block tables of a whole contiguous slot region however short the
    context (static.py:135-137), and decode rounds to the group's longest request in which
    finished rows are re-run at their last position (static.py:204-226). Fourteen requests in
    groups of six over a block-8 pool; one request ends exactly at max_context_tokens and is then
    re-run at the region's last slot while a longer request of its group decodes on; two sample
    at temperature 0.8."""
    config = ref.config.ModelConfig(vocab_size=96, d_model=128, n_layers=2, n_heads=4, d_ff=256, max_seq_len=256)
    model = ref.model.LanguageModel(config, ref.model.random_weights(config, seed=21))
    engine = ref.static.StaticBatchingEngine(model, batch_size=6, max_context_tokens=96, block_size=8,
                                             clock=lambda: 0.0, sleep=lambda _: None)  # fmt: skip
    log = StaticLog(engine.runner)
    engine.runner = log
    rng = np.random.default_rng(21)
    requests = []
    for i in range(14):
        length = int(rng.integers(4, 41))
        new = int(rng.integers(2, 25))
        if i in (3, 4):  # st-3 fills its slot region; st-4 keeps the group running after it
            length, new = (40, 96 - 40) if i == 3 else (10, 60)
        requests.append(
            ref.sequence.Request(
                request_id=f"st-{i}",
                prompt_token_ids=tuple(int(t) for t in rng.integers(0, 96, length)),
                sampling=ref.sequence.SamplingParams(
                    max_new_tokens=new, temperature=0.8 if i in (5, 9) else 0.0, seed=100 + i
                ),
            )
        )
    outputs = engine.generate(requests)
    by_id = {r.request_id: r for r in requests}
    tokens = {}
    for out in outputs:
        seq_id = ref.sequence.new_sequence_id(out.request_id, 0)
        tokens[seq_id] = [*by_id[out.request_id].prompt_token_ids, *out.token_ids]
    trace = {
        "format": 1,
        "kind": "static",
        "name": "static_batching",
        "model": {
            "vocab_size": config.vocab_size, "d_model": config.d_model, "n_layers": config.n_layers,
            "n_heads": config.n_heads, "d_ff": config.d_ff, "max_seq_len": config.max_seq_len,
            "rope_theta": config.rope_theta, "norm_eps": config.norm_eps, "seed": 21,
            "weights_sha256": weights_sha256(model.weights),
        },
        "engine": {
            "batch_size": engine.batch_size, "max_context_tokens": engine.max_context_tokens,
            "block_size": engine.block_size, "blocks_per_slot": engine.blocks_per_slot,
            "num_blocks": engine.runner.runner.num_blocks,
        },
        "requests": [
            {"request_id": r.request_id, "prompt": list(r.prompt_token_ids), "n": r.n, "key_id": r.key_id,
             "max_new_tokens": r.sampling.max_new_tokens, "temperature": r.sampling.temperature,
             "seed": r.sampling.seed}
            for r in requests
        ],
        "tokens": tokens,
        "events": [],
        "iterations": log.iterations,
        "summary": {
            "iterations": len(log.iterations),
            "logits_rows": len(log.rows),
            "padding_tokens": engine.total_padding_tokens,
            "wasted_decode_tokens": engine.total_wasted_decode_tokens,
        },
    }  # fmt: skip
    return trace, np.stack(log.rows)


WORKLOADS = {
    "config1": config1,
    "engine_equivalence": engine_equivalence,
    "sharing_b8": lambda ref: sharing(ref, "sharing_b8", 11, block_size=8, num_blocks=40, n_heads=2, d_model=64),
    "sharing_b4": lambda ref: sharing(ref, "sharing_b4", 12, block_size=4, num_blocks=48, n_heads=4, d_model=64),
    "sharing_b16": lambda ref: sharing(ref, "sharing_b16", 13, block_size=16, num_blocks=16, n_heads=2, d_model=256),
    "static_batching": static_batching,
}


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--check", action="store_true", help="regenerate and compare, write nothing")
    parser.add_argument("names", nargs="*", help="workloads to write (default: all)")
    args = parser.parse_args()
    ref = _reference()
    ref.blocks  # noqa: B018 - loaded for the recorder's error type name
    OUT.mkdir(exist_ok=True)
    status = 0
    for name in args.names or list(WORKLOADS):
        trace, logits = WORKLOADS[name](ref)
        text = json.dumps(trace, separators=(",", ":")) + "\n"
        json_path, npy_path = OUT / f"{name}.json", OUT / f"{name}_logits.npy"
        if args.check:
            same = json_path.read_text() == text and np.array_equal(np.load(npy_path), logits)
            print(f"{name}: {'identical' if same else 'DIFFERS'}")
            status |= 0 if same else 1
            continue
        json_path.write_text(text)
        np.save(npy_path, logits)
        print(f"{name}: {trace['summary']} -> {json_path.name} ({len(text)} B), {npy_path.name}")
    return status


if __name__ == "__main__":
    sys.exit(main())
