"""The continuous-batching loop that drives the runner (config 1), on the CPU.

Scheduler known answers are ported from the reference's tests/unit/test_scheduler.py for one
service class (priority = arrival order). Engine runs use the oracle's NumPy runner as executor
and block store, so every logits row the engine samples from -- chunked prefill, mixed batches,
forks with copy-on-write, recomputation after preemption -- is compared with the cache-free
recompute at the reference's 1e-4 (its bench/thresholds.json:10-11). The same loop drives the
GPU runner in tests/test_gpu_engine.py.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest

from oracle.model import OracleModel, random_weights
from oracle.runner import OracleRunner
from paged_kv_serving_amd.blocks import BlockManager, RecordingBlockStore
from paged_kv_serving_amd.config import EngineConfig, ModelConfig
from paged_kv_serving_amd.engine import Engine, RecordingExecutor, Scheduler
from paged_kv_serving_amd.kvcache import KVCacheManager
from paged_kv_serving_amd.prefix_cache import PrefixCache
from paged_kv_serving_amd.sequence import FinishReason, Request, SamplingParams, Sequence, SequenceStatus

CONFIG = EngineConfig(
    block_size=4, num_blocks=16, max_batched_tokens=8, max_running_seqs=4,
    max_prompt_tokens=32, max_new_tokens=8, max_context_tokens=48,
)  # fmt: skip
TIGHT = EngineConfig(
    block_size=4, num_blocks=4, max_batched_tokens=16, max_running_seqs=4,
    max_prompt_tokens=8, max_new_tokens=8, max_context_tokens=16, watermark=0.0,
)  # fmt: skip


def build(config: EngineConfig = CONFIG) -> Scheduler:
    blocks = BlockManager(num_blocks=config.num_blocks, block_size=config.block_size, store=RecordingBlockStore())
    return Scheduler(config, KVCacheManager(blocks, PrefixCache(blocks, enabled=config.enable_prefix_cache)))


def make(index: int, prompt_len: int, max_new_tokens: int = 4) -> Sequence:
    request = Request(f"r{index}", tuple(range(1, prompt_len + 1)), SamplingParams(max_new_tokens, index))
    return Sequence.from_request(request, 0)


def advance(scheduler: Scheduler, output) -> None:
    for item in output.scheduled:
        item.sequence.num_computed_tokens += item.num_tokens
        scheduler.cache.publish_full_blocks(item.sequence)
        if item.produces_token:
            item.sequence.append_token(1)


def test_a_long_prompt_is_split_across_iterations() -> None:
    scheduler = build()
    scheduler.add(make(0, 20))
    sizes = []
    for _ in range(3):
        output = scheduler.schedule()
        sizes.append((output.batch.num_tokens, output.scheduled[0].produces_token))
        advance(scheduler, output)
    assert sizes == [(8, False), (8, False), (4, True)]


def test_decode_tokens_are_taken_before_prefill() -> None:
    scheduler = build()
    streaming = make(0, 4)
    scheduler.add(streaming)
    advance(scheduler, scheduler.schedule())
    scheduler.add(make(1, 24))
    output = scheduler.schedule()
    decode = [i for i in output.scheduled if not i.is_prefill]
    prefill = [i for i in output.scheduled if i.is_prefill]
    assert [i.sequence.seq_id for i in decode] == [streaming.seq_id]
    assert prefill[0].num_tokens == CONFIG.max_batched_tokens - 1
    assert output.batch.num_tokens == CONFIG.max_batched_tokens


def test_admission_follows_arrival_order_and_the_running_set_is_capped() -> None:
    scheduler = build(dataclasses.replace(CONFIG, max_running_seqs=2, max_batched_tokens=32))
    seqs = [make(i, 2) for i in range(4)]
    for seq in seqs:
        scheduler.add(seq)
    output = scheduler.schedule()
    assert list(output.admitted) == [seqs[0].seq_id, seqs[1].seq_id]
    assert len(scheduler.running) == 2 and len(scheduler.waiting) == 2


def test_memory_pressure_preempts_the_later_arrival_and_it_is_recomputed() -> None:
    scheduler = build(TIGHT)
    first, second = make(0, 8, max_new_tokens=8), make(1, 8, max_new_tokens=8)
    scheduler.add(first)
    scheduler.add(second)
    advance(scheduler, scheduler.schedule())
    assert scheduler.cache.num_free_blocks == 0
    seen = False
    for _ in range(60):
        output = scheduler.schedule()
        if output.preempted and not seen:
            assert output.preempted == (second.seq_id,), "the later arrival must pay"
            assert second.status is SequenceStatus.PREEMPTED and second.block_table == []
            assert second.num_computed_tokens == 0 and second.preemption_count == 1
            assert second.num_tokens > second.request.prompt_len, "produced tokens are kept"
            seen = True
        advance(scheduler, output)
        for item in output.scheduled:
            if item.sequence.num_output_tokens >= item.sequence.request.sampling.max_new_tokens:
                item.sequence.finish(FinishReason.LENGTH)
        scheduler.drop_finished()
        scheduler.cache.check_invariants()
        if not scheduler.has_work:
            break
    assert seen and not scheduler.has_work and scheduler.preemptions >= 1


def test_add_running_inserts_a_fork_without_readmission() -> None:
    scheduler = build()
    parent = make(0, 4)
    scheduler.add(parent)
    advance(scheduler, scheduler.schedule())
    child = Sequence.from_request(parent.request, 1)
    child.token_ids = list(parent.token_ids)
    scheduler.cache.fork(parent, child)
    scheduler.add_running(child)
    output = scheduler.schedule()
    assert {i.sequence.seq_id for i in output.scheduled} == {parent.seq_id, child.seq_id}


def test_an_empty_scheduler_produces_an_empty_batch() -> None:
    output = build().schedule()
    assert output.is_empty and output.batch.num_tokens == 0


# --- engine runs against the cache-free recompute -------------------------------------------

TINY = ModelConfig(vocab_size=64, d_model=32, n_layers=2, n_heads=2, d_ff=64, max_seq_len=192)
ENGINE = EngineConfig(
    block_size=8, num_blocks=64, max_batched_tokens=32, max_running_seqs=6,
    max_prompt_tokens=64, max_new_tokens=16, max_context_tokens=128,
)  # fmt: skip


@pytest.fixture(scope="module")
def model() -> OracleModel:
    return OracleModel(TINY, random_weights(TINY, seed=11))


def run_engine(model, config, requests):
    runner = OracleRunner(model, num_blocks=config.num_blocks, block_size=config.block_size)
    engine = Engine(model, config, runner=runner)
    recorder = RecordingExecutor(runner)
    engine.executor = recorder
    outputs = engine.generate(requests)
    engine.check_invariants()
    return engine, recorder, outputs


def worst_gap(model, requests, recorder, outputs) -> tuple[float, int]:
    full = {}
    for request in requests:
        for index, produced in enumerate(outputs[request.request_id]):
            full[f"{request.request_id}#{index}"] = [*request.prompt_token_ids, *produced]
    cache, worst, rows = {}, 0.0, 0
    for seq_id, context, row in recorder.records:
        if seq_id not in cache:
            cache[seq_id] = model.reference_forward(full[seq_id])
        worst = max(worst, float(np.max(np.abs(cache[seq_id][context - 1] - row))))
        rows += 1
    return worst, rows


def requests_for(seed: int, count: int, *, shared: int = 0, n_every: int = 0):
    rng = np.random.default_rng(seed)
    prefix = [int(t) for t in rng.integers(1, 64, shared)]
    out = []
    for i in range(count):
        tail = [int(t) for t in rng.integers(1, 64, int(rng.integers(3, 40)))]
        out.append(Request(
            f"q{i}", tuple(prefix + tail if i % 2 else tail),
            SamplingParams(max_new_tokens=int(rng.integers(2, 12)), seed=i),
            n=2 if n_every and i % n_every == 0 else 1,
        ))  # fmt: skip
    return out


def test_engine_logits_match_the_cache_free_recompute(model) -> None:
    requests = requests_for(0, 10, shared=16, n_every=4)
    engine, recorder, outputs = run_engine(model, ENGINE, requests)
    assert set(outputs) == {r.request_id for r in requests}
    for request in requests:
        samples = outputs[request.request_id]
        assert len(samples) == request.n
        assert all(len(s) == request.sampling.max_new_tokens for s in samples)
        if request.n == 2:  # greedy forks share the first token and agree afterwards
            assert samples[0] == samples[1]
    worst, rows = worst_gap(model, requests, recorder, outputs)
    assert rows >= sum(r.sampling.max_new_tokens * r.n for r in requests) - sum(r.n - 1 for r in requests)
    assert worst < 1e-4
    assert engine.prefix_cache.stats.hit_blocks > 0  # shared prompts reused cached blocks
    assert engine.blocks.num_free_blocks + len(engine.prefix_cache) == ENGINE.num_blocks


def test_a_cramped_pool_preempts_and_still_matches(model) -> None:
    config = dataclasses.replace(ENGINE, num_blocks=20, max_batched_tokens=48, watermark=0.0)
    requests = requests_for(1, 8)
    engine, recorder, outputs = run_engine(model, config, requests)
    assert engine.scheduler.preemptions > 0
    worst, _ = worst_gap(model, requests, recorder, outputs)
    assert worst < 1e-4


def test_an_n_way_request_forks_and_copies_only_the_partial_block(model) -> None:
    config = dataclasses.replace(ENGINE, enable_prefix_cache=False)
    request = Request("fork", tuple(range(1, 12)), SamplingParams(max_new_tokens=3), n=3)
    runner = OracleRunner(model, num_blocks=config.num_blocks, block_size=config.block_size)
    copies = []
    original = runner.copy_block

    def record(src, dst):
        copies.append((src, dst))
        original(src, dst)

    runner.copy_block = record
    engine = Engine(model, config, runner=runner)
    outputs = engine.generate([request])
    # 11 prompt tokens + 1 sampled = 12 -> block 1 (tokens 8..11) is partial and shared by 3;
    # the first decode write of two of the samples copies it, the last owner writes in place.
    assert len(copies) == 2 and len({src for src, _ in copies}) == 1
    assert len(outputs["fork"]) == 3
