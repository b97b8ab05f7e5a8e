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
