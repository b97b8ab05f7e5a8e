"""Config 1 end to end on the GPU: the engine loop over the GPU ModelRunner.

Random-init fp32 decoder (vocab 256, d_model 128, 2 layers, 4 heads x 32, d_ff 320,
max_seq_len 1024, random_weights seed 0), 32 requests with prompt lengths uniform in [16, 128]
(seed 0), 32 greedy tokens each, EngineConfig defaults (block 16, 512 blocks, budget 256): chunked
prefill and continuous batching. Every logits row the engine samples from is compared with the
oracle's cache-free recompute of that sequence at the reference's bar of 1e-4.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.model import OracleModel
from oracle.runner import OracleRunner
from paged_kv_serving_amd.config import EngineConfig, ModelConfig
from paged_kv_serving_amd.engine import Engine, RecordingExecutor
from paged_kv_serving_amd.model import LanguageModel, random_weights
from paged_kv_serving_amd.sequence import Request, SamplingParams

pytestmark = pytest.mark.gpu

CONFIG1 = ModelConfig(vocab_size=256, d_model=128, n_layers=2, n_heads=4, d_ff=320, max_seq_len=1024)


def config1_requests(seed: int = 0, count: int = 32, new_tokens: int = 32) -> list[Request]:
    rng = np.random.default_rng(seed)
    requests = []
    for i in range(count):
        length = int(rng.integers(16, 129))
        tokens = tuple(int(t) for t in rng.integers(0, 256, length))
        requests.append(Request(f"req{i}", tokens, SamplingParams(max_new_tokens=new_tokens, seed=i)))
    return requests


def test_config1_engine_matches_the_cache_free_recompute(device) -> None:
    weights = random_weights(CONFIG1, seed=0)
    model = LanguageModel(CONFIG1, weights)
    oracle = OracleModel(CONFIG1, weights)
    engine = Engine(model, EngineConfig(), device=device)
    recorder = RecordingExecutor(engine.runner)
    engine.executor = recorder
    requests = config1_requests()
    outputs = engine.generate(requests)
    engine.check_invariants()
    assert all(len(outputs[r.request_id][0]) == 32 for r in requests)
    full = {f"{r.request_id}#0": [*r.prompt_token_ids, *outputs[r.request_id][0]] for r in requests}
    references, worst = {}, 0.0
    for seq_id, context, row in recorder.records:
        if seq_id not in references:
            references[seq_id] = oracle.reference_forward(full[seq_id])
        worst = max(worst, float(np.max(np.abs(references[seq_id][context - 1] - row))))
    print(f"config 1: {len(recorder.records)} rows, {engine.iterations} iterations, worst gap {worst:.3g}", flush=True)
    assert len(recorder.records) == 32 * 32
    assert worst < 1e-4

    # The same loop over the NumPy runner produces the same tokens (greedy, no near-ties here).
    cpu = Engine(oracle, EngineConfig(), runner=OracleRunner(oracle, num_blocks=512, block_size=16))
    cpu_outputs = cpu.generate(config1_requests())
    same = sum(cpu_outputs[r.request_id] == outputs[r.request_id] for r in requests)
    print(f"config 1: {same}/32 sequences token-identical between the GPU and NumPy runners", flush=True)
    assert same >= 30


def test_random_engine_runs_with_shared_prompts_and_small_pools(device) -> None:
    """Seeded engine runs whose prompts mostly share one of three prefixes, over pools of 48, 96
    or 512 blocks (the small ones force preemption and recompute), with the prefix cache on or
    off and varied token budgets. Every sampled logits row matches the cache-free recompute at
    1e-4 and the allocator's invariants hold; across the runs, sequences were preempted and
    prefix blocks were reused."""
    weights = random_weights(CONFIG1, seed=0)
    model, oracle = LanguageModel(CONFIG1, weights), OracleModel(CONFIG1, weights)
    preemptions = hits = 0
    for seed in range(16):
        rng = np.random.default_rng(900 + seed)
        prefixes = [tuple(int(t) for t in rng.integers(0, 256, int(rng.integers(16, 161)))) for _ in range(3)]
        requests = []
        for i in range(int(rng.integers(8, 25))):
            shared = prefixes[int(rng.integers(0, 3))] if rng.random() < 0.7 else ()
            tail = tuple(int(t) for t in rng.integers(0, 256, int(rng.integers(1, 61))))
            requests.append(Request(f"r{i}", shared + tail, SamplingParams(max_new_tokens=int(rng.integers(4, 25)), seed=i)))
        blocks = int(rng.choice([48, 96, 512]))
        config = EngineConfig(
            num_blocks=blocks, max_batched_tokens=int(rng.choice([64, 128, 256])),
            max_running_seqs=int(rng.choice([4, 8, 32])), max_prompt_tokens=512, max_new_tokens=32,
            max_context_tokens=min(1024, blocks * 16), enable_prefix_cache=bool(rng.random() < 0.8),
        )  # fmt: skip
        print("engine run", seed, len(requests), "requests,", blocks, "blocks", flush=True)
        engine = Engine(model, config, device=device)
        recorder = RecordingExecutor(engine.runner)
        engine.executor = recorder
        outputs = engine.generate(requests)
        engine.check_invariants()
        assert all(len(outputs[r.request_id][0]) == r.sampling.max_new_tokens for r in requests)
        full = {f"{r.request_id}#0": [*r.prompt_token_ids, *outputs[r.request_id][0]] for r in requests}
        references, worst = {}, 0.0
        for seq_id, context, row in recorder.records:
            if seq_id not in references:
                references[seq_id] = oracle.reference_forward(full[seq_id])
            worst = max(worst, float(np.max(np.abs(references[seq_id][context - 1] - row))))
        assert worst < 1e-4, (seed, worst)
        preemptions += engine.scheduler.preemptions
        hits += engine.prefix_cache.stats.hit_blocks
    assert preemptions > 0 and hits > 0, (preemptions, hits)
