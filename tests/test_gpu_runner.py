"""The GPU ModelRunner against the cache-free recompute (the reference's central claim).

Ports the properties of the reference's tests/property/test_equivalence.py (chunk splits,
scattered block tables, tile size, batch composition, a shared prefix) with seeded cases
instead of hypothesis draws, at its tolerance of 1e-4 on logits and BLOCK_SIZE 8, plus the
runner surface: copy-on-write through BlockManager with real bytes, the block fingerprint,
reset, the weight-swap hazard and the reference's error messages.
"""

from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

from oracle.model import OracleModel
from oracle.runner import OracleRunner
from paged_kv_serving_amd.blocks import BlockManager
from paged_kv_serving_amd.config import ModelConfig
from paged_kv_serving_amd.kvcache import KVCacheManager
from paged_kv_serving_amd.model import LanguageModel, random_weights
from paged_kv_serving_amd.prefix_cache import PrefixCache
from paged_kv_serving_amd.runner import BatchEntry, ExecutionBatch, ModelRunner
from paged_kv_serving_amd.sequence import Request, Sequence

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-4
BLOCK_SIZE = 8
#: The reference's tiny test model (its tests/conftest.py:42-44).
TINY_MODEL = dict(vocab_size=64, d_model=32, n_layers=2, n_heads=2, d_ff=64, max_seq_len=192)


@pytest.fixture(scope="module")
def models():
    config = ModelConfig(**TINY_MODEL)
    weights = random_weights(config, seed=11)
    return LanguageModel(config, weights), OracleModel(config, weights)


def split_sizes(total: int, chunk: int) -> list[int]:
    sizes = [chunk] * (total // chunk)
    if total % chunk:
        sizes.append(total % chunk)
    return sizes


def chunked_logits(model, tokens, *, chunks=None, block_order=None, tile_blocks=8, device=None):
    """Last-position logits through the GPU runner, chunk by chunk (equivalence.py:49-92)."""
    sizes = chunks or [len(tokens)]
    needed = -(-len(tokens) // BLOCK_SIZE)
    table = tuple(block_order) if block_order is not None else tuple(range(needed))
    runner = ModelRunner(model, num_blocks=max(table) + 1, block_size=BLOCK_SIZE,
                         tile_blocks=tile_blocks, device=device)  # fmt: skip
    start, logits = 0, None
    for size in sizes:
        stop = start + size
        entry = BatchEntry("s", tuple(tokens[start:stop]), tuple(range(start, stop)), table,
                           size - 1 if stop == len(tokens) else None)  # fmt: skip
        result = runner.execute(ExecutionBatch((entry,)))
        logits = result.get("s", logits)
        start = stop
    return logits


def token_cases(count: int, seed: int, low: int = 1, high: int = 40):
    rng = np.random.default_rng(seed)
    return [[int(t) for t in rng.integers(0, 64, int(rng.integers(low, high + 1)))] for _ in range(count)]


@pytest.mark.parametrize("case", range(12))
def test_chunked_prefill_matches_a_cache_free_recompute(device, models, case) -> None:
    model, oracle = models
    tokens = token_cases(12, 1)[case]
    chunk = 1 + case % 13
    got = chunked_logits(model, tokens, chunks=split_sizes(len(tokens), chunk), device=device)
    want = oracle.reference_forward(tokens)[-1]
    gap = float(np.max(np.abs(got - want)))
    print("chunked", case, len(tokens), chunk, gap, flush=True)
    assert gap < TOLERANCE


@pytest.mark.parametrize("case", range(8))
def test_a_scattered_block_table_gives_the_same_logits(device, models, case) -> None:
    model, oracle = models
    tokens = token_cases(8, 2)[case]
    needed = -(-len(tokens) // BLOCK_SIZE)
    order = [int(v) for v in np.random.default_rng(case).permutation(needed * 2 + 3)[:needed]]
    got = chunked_logits(model, tokens, block_order=order, device=device)
    assert float(np.max(np.abs(got - oracle.reference_forward(tokens)[-1]))) < TOLERANCE


@pytest.mark.parametrize("tile", [1, 2, 6])
def test_tile_size_does_not_change_the_result(device, models, tile) -> None:
    model, oracle = models
    for tokens in token_cases(3, 3 + tile):
        got = chunked_logits(model, tokens, chunks=split_sizes(len(tokens), 5), tile_blocks=tile, device=device)
        assert float(np.max(np.abs(got - oracle.reference_forward(tokens)[-1]))) < TOLERANCE


@pytest.mark.parametrize("decode_first", [False, True])
def test_batch_composition_does_not_change_a_sequences_logits(device, models, decode_first) -> None:
    model, _ = models
    sequences = token_cases(4, 4)
    per_seq = [-(-len(t) // BLOCK_SIZE) for t in sequences]
    runner = ModelRunner(model, num_blocks=sum(per_seq), block_size=BLOCK_SIZE, device=device)
    order = list(range(len(sequences)))[:: -1 if decode_first else 1]
    entries = []
    for i in order:
        start = sum(per_seq[:i])
        entries.append(BatchEntry(f"s{i}", tuple(sequences[i]), tuple(range(len(sequences[i]))),
                                  tuple(range(start, start + per_seq[i])), len(sequences[i]) - 1))  # fmt: skip
    batched = runner.execute(ExecutionBatch(tuple(entries)))
    for i, tokens in enumerate(sequences):
        alone = chunked_logits(model, tokens, device=device)
        assert float(np.max(np.abs(batched[f"s{i}"] - alone))) < TOLERANCE


def test_mixed_decode_and_prefill_rows_match_the_numpy_runner(device, models) -> None:
    """One ragged batch of decode rows and chunk rows: GPU logits vs the NumPy runner's."""
    model, oracle = models
    gpu = ModelRunner(model, num_blocks=40, block_size=BLOCK_SIZE, device=device)
    cpu = OracleRunner(oracle, num_blocks=40, block_size=BLOCK_SIZE)
    rng = np.random.default_rng(7)
    prompts = [[int(t) for t in rng.integers(0, 64, n)] for n in (17, 9, 30)]
    tables = [tuple(range(0, 5)), tuple(range(10, 15)), tuple(range(20, 25))]
    first = ExecutionBatch(tuple(
        BatchEntry(f"s{i}", tuple(p), tuple(range(len(p))), tables[i], len(p) - 1)
        for i, p in enumerate(prompts)
    ))  # fmt: skip
    for runner in (gpu, cpu):
        runner.execute(first)
    entries = (
        BatchEntry("s0", (5,), (17,), tables[0], 0),  # decode
        BatchEntry("s1", (1, 2, 3, 4), (9, 10, 11, 12), tables[1], 3),  # chunk
        BatchEntry("s2", (8,), (30,), tables[2], 0),  # decode
    )
    got = gpu.execute(ExecutionBatch(entries))
    want = cpu.execute(ExecutionBatch(entries))
    for name in want:
        assert float(np.max(np.abs(got[name] - want[name]))) < TOLERANCE
    # and the pools hold the same keys/values (float32 rounding only)
    for layer in range(2):
        gk, gv = gpu.block_view(layer)
        assert float(np.max(np.abs(gk.cpu().numpy() - cpu.keys[layer]))) < 1e-5
        assert float(np.max(np.abs(gv.cpu().numpy() - cpu.values[layer]))) < 1e-5


def test_a_shared_prompt_decodes_through_prefix_tiles(device) -> None:
    """20 sequences share a 544-token prompt's blocks; their decode step reads the prompt as
    MFMA tiles over whole partitions (head_dim 32) and matches the NumPy runner."""
    config = ModelConfig(vocab_size=64, d_model=64, n_layers=1, n_heads=2, d_ff=64, max_seq_len=1024)
    weights = random_weights(config, seed=3)
    model, oracle = LanguageModel(config, weights), OracleModel(config, weights)
    block = 16
    gpu = ModelRunner(model, num_blocks=120, block_size=block, device=device)
    cpu = OracleRunner(oracle, num_blocks=120, block_size=block)
    rng = np.random.default_rng(11)
    prompt = [int(t) for t in rng.integers(0, 64, 544)]
    shared = tuple(range(34))
    fill = ExecutionBatch((BatchEntry("p", tuple(prompt), tuple(range(544)), shared, None),))
    suffixes = [int(n) for n in rng.integers(3, 20, 20)]
    tables = [shared + (34 + 2 * i, 35 + 2 * i) for i in range(20)]
    children = ExecutionBatch(tuple(
        BatchEntry(f"c{i}", tuple(int(t) for t in rng.integers(0, 64, n)), tuple(range(544, 544 + n)),
                   tables[i], n - 1)
        for i, n in enumerate(suffixes)
    ))  # fmt: skip
    decode = ExecutionBatch(tuple(
        BatchEntry(f"c{i}", (int(rng.integers(0, 64)),), (544 + n,), tables[i], 0)
        for i, n in enumerate(suffixes)
    ))  # fmt: skip
    for batch in (fill, children):
        gpu.execute(batch)
        cpu.execute(batch)
    got = gpu.execute(decode)
    plan = gpu.last_plan
    assert plan.tiles.shape[0] == 1 and plan.tiles[0, 1] == 20 and plan.tiles[0, 3] >= 1
    # every row's row-pass items start at the first partition after the prefix tile's
    firsts = {}
    for t, p in plan.rows.tolist():
        firsts[t] = min(p, firsts.get(t, p))
    assert set(firsts.values()) == {int(plan.tiles[0, 3])}
    want = cpu.execute(decode)
    assert set(got) == set(want)
    for name in want:
        assert float(np.max(np.abs(got[name] - want[name]))) < TOLERANCE, name


def test_interleaved_sharers_are_grouped_into_prefix_tiles(device) -> None:
    """The same 20 sharing sequences, interleaved in the batch with 8 unrelated ones: the runner
    orders the sharers next to each other, so their prompt is still read as prefix tiles, and
    every logits row (returned in batch order) matches the NumPy runner."""
    config = ModelConfig(vocab_size=64, d_model=64, n_layers=1, n_heads=2, d_ff=64, max_seq_len=1024)
    weights = random_weights(config, seed=5)
    model, oracle = LanguageModel(config, weights), OracleModel(config, weights)
    block = 16
    gpu = ModelRunner(model, num_blocks=160, block_size=block, device=device)
    cpu = OracleRunner(oracle, num_blocks=160, block_size=block)
    rng = np.random.default_rng(12)
    prompt = [int(t) for t in rng.integers(0, 64, 544)]
    shared = tuple(range(34))
    suffixes = [int(n) for n in rng.integers(3, 20, 20)]
    tables = [shared + (34 + 2 * i, 35 + 2 * i) for i in range(20)]
    others = [(f"o{i}", tuple(range(80 + 3 * i, 83 + 3 * i)), int(rng.integers(10, 40))) for i in range(8)]
    setup = [ExecutionBatch((BatchEntry("p", tuple(prompt), tuple(range(544)), shared, None),)),
             ExecutionBatch(tuple(
                 BatchEntry(f"c{i}", tuple(int(t) for t in rng.integers(0, 64, n)),
                            tuple(range(544, 544 + n)), tables[i], n - 1)
                 for i, n in enumerate(suffixes))),
             ExecutionBatch(tuple(
                 BatchEntry(name, tuple(int(t) for t in rng.integers(0, 64, n)), tuple(range(n)), table,
                            n - 1)
                 for name, table, n in others))]  # fmt: skip
    for batch in setup:
        gpu.execute(batch)
        cpu.execute(batch)
    children = [BatchEntry(f"c{i}", (int(rng.integers(0, 64)),), (544 + n,), tables[i], 0)
                for i, n in enumerate(suffixes)]  # fmt: skip
    strangers = [BatchEntry(name, (int(rng.integers(0, 64)),), (n,), table, 0) for name, table, n in others]
    mixed = []
    for i, child in enumerate(children):
        mixed.append(child)
        if i % 3 == 1 and strangers:
            mixed.append(strangers.pop())
    mixed += strangers
    decode = ExecutionBatch(tuple(mixed))
    got = gpu.execute(decode)
    plan = gpu.last_plan
    assert plan.tiles.shape[0] == 1 and plan.tiles[0, 1] == 20 and plan.tiles[0, 3] >= 1
    assert list(got) == [e.seq_id for e in mixed]  # batch order
    want = cpu.execute(decode)
    for name in want:
        assert float(np.max(np.abs(got[name] - want[name]))) < TOLERANCE, name


def test_sharing_a_prefix_block_does_not_change_either_continuation(device, models) -> None:
    model, oracle = models
    rng = np.random.default_rng(12)
    prefix = [int(t) for t in rng.integers(0, 64, 16)]
    a = [*prefix, *[int(t) for t in rng.integers(0, 64, 7)]]
    b = [*prefix, *[int(t) for t in rng.integers(0, 64, 11)]]
    runner = ModelRunner(model, num_blocks=8, block_size=BLOCK_SIZE, device=device)
    shared = (0, 1)
    runner.execute(ExecutionBatch((BatchEntry("p", tuple(prefix), tuple(range(16)), shared),)))
    for name, seq, own in (("a", a, (2,)), ("b", b, (4, 5))):
        result = runner.execute(ExecutionBatch((BatchEntry(
            name, tuple(seq[16:]), tuple(range(16, len(seq))), shared + own, len(seq) - 17),)))  # fmt: skip
        assert float(np.max(np.abs(result[name] - oracle.reference_forward(seq)[-1]))) < TOLERANCE


def test_copy_on_write_moves_real_bytes_and_keeps_the_original(device, models) -> None:
    """Fork, then the child's first write: BlockManager asks the runner for one copy."""
    model, oracle = models
    runner = ModelRunner(model, num_blocks=16, block_size=4, device=device)
    blocks = BlockManager(num_blocks=16, block_size=4, store=runner)
    cache = KVCacheManager(blocks, PrefixCache(blocks))
    parent = Sequence.from_request(Request("p", (1, 2, 3, 4, 5, 6)), 0)
    cache.reserve(parent, 6)
    runner.execute(ExecutionBatch((BatchEntry("p", (1, 2, 3, 4, 5, 6), tuple(range(6)),
                                              tuple(parent.block_table), 5),)))  # fmt: skip
    parent.num_computed_tokens = 6
    child = Sequence.from_request(Request("c", (1, 2, 3, 4, 5, 6)), 0)
    cache.fork(parent, child)
    shared = parent.block_table[1]
    before = runner.block_fingerprint(shared)
    child.token_ids.append(9)
    cache.reserve(child, 7)  # copy-on-write of the partial block, queued in the runner
    private = child.block_table[1]
    assert private != shared
    result = runner.execute(ExecutionBatch((BatchEntry("c", (9,), (6,), tuple(child.block_table), 0),)))
    assert runner.block_fingerprint(shared) == before, "the original block changed"
    k, v = runner.block_view(0)
    assert torch.equal(k[private, :2], k[shared, :2]) and torch.equal(v[private, :2], v[shared, :2])
    want = oracle.reference_forward([1, 2, 3, 4, 5, 6, 9])[-1]
    assert float(np.max(np.abs(result["c"] - want))) < TOLERANCE


def test_fingerprint_matches_the_reference_byte_layout(device, models) -> None:
    model, _ = models
    runner = ModelRunner(model, num_blocks=4, block_size=4, device=device)
    runner.execute(ExecutionBatch((BatchEntry("s", (3, 1, 4, 1, 5), tuple(range(5)), (2, 0)),)))
    keys = runner.key_cache.cpu().numpy()
    values = runner.value_cache.cpu().numpy()
    digest = hashlib.blake2b(digest_size=16)
    digest.update(np.ascontiguousarray(keys[:, 2]).tobytes())
    digest.update(np.ascontiguousarray(values[:, 2]).tobytes())
    assert runner.block_fingerprint(2) == digest.digest()
    runner.reset_cache()
    assert not runner.key_cache.any() and not runner.value_cache.any()


def test_a_weight_swap_is_picked_up(device, models) -> None:
    model, _ = models
    config = model.config
    swapped = LanguageModel(config, random_weights(config, seed=11))
    runner = ModelRunner(swapped, num_blocks=4, block_size=8, device=device)
    entry = BatchEntry("s", (1, 2, 3), (0, 1, 2), (0,), 2)
    first = runner.execute(ExecutionBatch((entry,)))["s"]
    swapped.weights = random_weights(config, seed=12)  # what the reference's admin swap does
    runner.reset_cache()
    second = runner.execute(ExecutionBatch((entry,)))["s"]
    oracle = OracleModel(config, swapped.weights)
    assert float(np.max(np.abs(second - oracle.reference_forward([1, 2, 3])[-1]))) < TOLERANCE
    assert not np.allclose(first, second)


def test_reference_error_messages(device, models) -> None:
    model, _ = models
    with pytest.raises(ValueError, match="num_blocks and block_size must be >= 1"):
        ModelRunner(model, num_blocks=0, block_size=4, device=device)
    with pytest.raises(ValueError, match="tile_blocks must be >= 1"):
        ModelRunner(model, num_blocks=4, block_size=4, tile_blocks=0, device=device)
    runner = ModelRunner(model, num_blocks=4, block_size=4, device=device)
    with pytest.raises(ValueError, match="token id outside the vocabulary"):
        runner.execute(ExecutionBatch((BatchEntry("s", (64,), (0,), (0,)),)))
    with pytest.raises(ValueError, match="position beyond max_seq_len"):
        runner.execute(ExecutionBatch((BatchEntry("s", (1,), (192,), (0,)),)))
    with pytest.raises(ValueError, match="sequence s: position 4 has no block in the table"):
        runner.execute(ExecutionBatch((BatchEntry("s", (1,), (4,), (0,)),)))
    with pytest.raises(ValueError, match="onto itself"):
        runner.copy_block(1, 1)
    assert runner.execute(ExecutionBatch(())) == {}
    # an entry ending at a negative position has context_len < 1 (attention.py:76-77)
    with pytest.raises(ValueError, match="context_len must be >= 1"):
        runner.execute(ExecutionBatch((BatchEntry("s", (1, 2), (-2, -1), (0, 1)),)))


def test_negative_positions_run_as_in_the_reference(device, models) -> None:
    """A chunk whose first positions are negative: their slots come from the end of the table,
    their rotary angle from the end of the tables, and all their keys are masked. The GPU runner
    must agree with the NumPy runner, which follows the reference's indexing."""
    model, oracle = models
    runner = ModelRunner(model, num_blocks=6, block_size=BLOCK_SIZE, device=device)
    cpu = OracleRunner(oracle, num_blocks=6, block_size=BLOCK_SIZE)
    table = (3, 0, 5)
    batch = ExecutionBatch((BatchEntry("s", (5, 9, 11, 2, 7), (-3, -2, -1, 0, 1), table, 4),))
    got, want = runner.execute(batch), cpu.execute(batch)
    assert float(np.max(np.abs(got["s"] - want["s"]))) < TOLERANCE
    later = ExecutionBatch((BatchEntry("s", (3,), (2,), table, 0),))
    got, want = runner.execute(later), cpu.execute(later)
    assert float(np.max(np.abs(got["s"] - want["s"]))) < TOLERANCE


def test_steps_from_changing_worker_threads_match_one_thread(device, models) -> None:
    """The reference's service calls execute() from asyncio.to_thread workers that change between
    steps (service.py:265-296). The same steps, each run on a fresh thread, give the same logits
    bit for bit as on the calling thread, and leave the same pool bytes."""
    import threading

    model, _ = models
    rng = np.random.default_rng(21)
    prompts = [[int(t) for t in rng.integers(0, 64, n)] for n in (23, 9, 17)]
    tables = [(0, 1, 2, 3), (4, 5), (6, 7, 8)]

    def steps():
        """A chunked prefill of three prompts, then four decode steps of all three."""
        out = [ExecutionBatch(tuple(
            BatchEntry(f"s{i}", tuple(p[:8]), tuple(range(8)), tables[i], 7) for i, p in enumerate(prompts)))]  # fmt: skip
        out.append(ExecutionBatch(tuple(
            BatchEntry(f"s{i}", tuple(p[8:]), tuple(range(8, len(p))), tables[i], len(p) - 9)
            for i, p in enumerate(prompts) if len(p) > 8)))  # fmt: skip
        for step in range(4):
            out.append(ExecutionBatch(tuple(
                BatchEntry(f"s{i}", (step + i,), (len(p) + step,), tables[i], 0) for i, p in enumerate(prompts))))  # fmt: skip
        return out

    def run(on_threads: bool):
        runner = ModelRunner(model, num_blocks=10, block_size=BLOCK_SIZE, device=device)
        results = []
        for batch in steps():
            if on_threads:
                box = {}
                worker = threading.Thread(target=lambda b=batch: box.update(r=runner.execute(b)))
                worker.start()
                worker.join()
                results.append(box["r"])
            else:
                results.append(runner.execute(batch))
        return results, [runner.block_fingerprint(b) for b in range(10)]

    main, main_prints = run(False)
    threaded, thread_prints = run(True)
    assert main_prints == thread_prints
    for a, b in zip(main, threaded):
        assert a.keys() == b.keys()
        assert all(np.array_equal(a[k], b[k]) for k in a)


def test_a_bfloat16_pool_matches_the_numpy_runner_on_rounded_kv(device, models, monkeypatch) -> None:
    """ModelRunner with bfloat16 K/V storage through chunked prefill and decode steps, against
    the NumPy runner whose append stores each key and value rounded to bfloat16 (nearest even):
    the north star's bar for bfloat16 KV, at the reference's logits tolerance."""
    import oracle.runner as oracle_runner
    from oracle.bf16 import bf16_round

    model, oracle = models
    plain_append = oracle_runner.append

    def rounded_append(key_pool, value_pool, slots, keys, values):
        plain_append(key_pool, value_pool, slots, bf16_round(np.asarray(keys, dtype=np.float32)),
                     bf16_round(np.asarray(values, dtype=np.float32)))  # fmt: skip

    monkeypatch.setattr(oracle_runner, "append", rounded_append)
    rng = np.random.default_rng(33)
    prompts = [[int(t) for t in rng.integers(0, 64, n)] for n in (29, 13)]
    tables = [(0, 1, 2, 3, 4), (5, 6, 7)]
    gpu = ModelRunner(model, num_blocks=8, block_size=BLOCK_SIZE, kv_dtype=torch.bfloat16, device=device)
    cpu = OracleRunner(oracle, num_blocks=8, block_size=BLOCK_SIZE)
    batches = [ExecutionBatch(tuple(BatchEntry(f"s{i}", tuple(p), tuple(range(len(p))), tables[i], len(p) - 1)
                                    for i, p in enumerate(prompts)))]  # fmt: skip
    for step in range(6):
        batches.append(ExecutionBatch(tuple(
            BatchEntry(f"s{i}", (step * 3 + i,), (len(p) + step,), tables[i], 0) for i, p in enumerate(prompts))))  # fmt: skip
    for batch in batches:
        want, got = cpu.execute(batch), gpu.execute(batch)
        assert want.keys() == got.keys()
        for name in want:
            assert float(np.max(np.abs(got[name] - want[name]))) < TOLERANCE, name
    assert gpu.kv_dtype == torch.bfloat16


def _attend_case(seed: int, *, sharers: int = 0, prefill: bool = True):
    """A batch over a random pool: decode entries (``sharers`` of them interleaved with the rest
    share 40 leading blocks), optionally one prefill chunk, with random q/k/v."""
    rng = np.random.default_rng(seed)
    config = ModelConfig(vocab_size=16, d_model=256, n_layers=2, n_heads=4, d_ff=32, max_seq_len=2048)
    model = LanguageModel(config, random_weights(config, seed=seed))
    block, num_blocks = 16, 4000
    perm = [int(b) for b in rng.permutation(num_blocks)]
    shared = perm[:40]
    used = 40
    entries = []
    for i in range(40):
        if sharers and i % 2 == 0 and i // 2 < sharers:
            ctx = 40 * block + int(rng.integers(1, 60))
            table = shared + perm[used : used + (-(-ctx // block)) - 40]
        else:
            ctx = int(rng.integers(1, 900))
            table = perm[used : used + (-(-ctx // block))]
        used += len(table) - (40 if table[:40] == shared else 0)
        entries.append(BatchEntry(f"d{i}", (1,), (ctx - 1,), tuple(table), 0))
    if prefill:
        table = perm[used : used + 6]
        entries.append(BatchEntry("p", tuple(i % 15 + 1 for i in range(40)), tuple(range(50, 90)), tuple(table), 39))
    batch = ExecutionBatch(tuple(entries))
    total = batch.num_tokens
    q, k, v = (rng.standard_normal((total, 4, 64)).astype(np.float32) for _ in range(3))
    return model, batch, q, k, v, num_blocks, block


@pytest.mark.parametrize(("seed", "sharers", "prefill"), [(0, 0, True), (1, 0, False), (2, 18, False), (3, 18, True)])
def test_attend_appends_and_attends_like_the_reference_runner(device, seed, sharers, prefill) -> None:
    """ModelRunner.attend: the caller's keys and values land at the batch's slots (bit for bit)
    and every query's output matches the oracle's paged attention (1e-5): prefill and decode rows
    together, a decode-only batch (the append fused into the attention call), and decode rows
    whose shared prefix makes the runner reorder them."""
    from oracle.attention import paged_attention
    from oracle.runner import append as oracle_append, slots_for

    model, batch, q, k, v, num_blocks, block = _attend_case(seed, sharers=sharers, prefill=prefill)
    runner = ModelRunner(model, num_blocks=num_blocks, block_size=block, device=device)
    rng = np.random.default_rng(100 + seed)
    keys0 = rng.standard_normal((num_blocks, block, 4, 64)).astype(np.float32)
    values0 = rng.standard_normal((num_blocks, block, 4, 64)).astype(np.float32)
    runner.key_cache[1].copy_(torch.from_numpy(keys0))
    runner.value_cache[1].copy_(torch.from_numpy(values0))
    for layer in (2, -1):  # a layer outside the pools is refused before anything is enqueued
        with pytest.raises(IndexError, match=f"layer {layer} is outside"):
            runner.attend(batch, *(torch.from_numpy(a).to(device) for a in (q, k, v)), layer=layer)
    out = runner.attend(batch, *(torch.from_numpy(a).to(device) for a in (q, k, v)), layer=1).cpu().numpy()
    if sharers:
        assert runner.last_plan is not None and runner.last_plan.tiles.shape[0] > 0, "prefix tiles"
    # a decode batch whose rows write private blocks appends inside the attention call, shared-
    # prefix tiles or not; a prefill chunk makes the runner append first
    assert runner.last_append_fused == (not prefill)
    slots = [s for e in batch.entries for s in slots_for(e.seq_id, e.positions, e.block_table, block)]
    oracle_append(keys0, values0, slots, k, v)
    assert np.array_equal(runner.key_cache[1].cpu().numpy(), keys0)
    assert np.array_equal(runner.value_cache[1].cpu().numpy(), values0)
    offset, worst = 0, 0.0
    for entry in batch.entries:
        n = len(entry.token_ids)
        want = paged_attention(q[offset : offset + n], np.asarray(entry.positions), keys0, values0,
                               np.asarray(entry.block_table), entry.context_len, 64**-0.5)  # fmt: skip
        worst = max(worst, float(np.max(np.abs(out[offset : offset + n] - want))))
        offset += n
    assert worst < 1e-5


def test_attend_metadata_of_growing_and_shrinking_batches(device) -> None:
    """One runner's calls whose metadata grows past the first staging buffer (64 KiB: a
    3,000-token prefill chunk sends 72 KiB of int64 sections alone) and shrinks again: every
    call's slots and outputs match the oracle, so each call read its own sections."""
    from oracle.attention import paged_attention
    from oracle.runner import append as oracle_append, slots_for

    rng = np.random.default_rng(11)
    config = ModelConfig(vocab_size=16, d_model=64, n_layers=1, n_heads=2, d_ff=32, max_seq_len=4096)
    model = LanguageModel(config, random_weights(config, seed=11))
    block, num_blocks = 16, 600
    runner = ModelRunner(model, num_blocks=num_blocks, block_size=block, device=device)
    keys = rng.standard_normal((num_blocks, block, 2, 32)).astype(np.float32)
    values = rng.standard_normal((num_blocks, block, 2, 32)).astype(np.float32)
    runner.key_cache[0].copy_(torch.from_numpy(keys))
    runner.value_cache[0].copy_(torch.from_numpy(values))
    perm = [int(b) for b in rng.permutation(num_blocks)]
    small = (BatchEntry("a", (1,), (40,), tuple(perm[:3]), 0), BatchEntry("b", (2,), (7,), tuple(perm[3:4]), 0))
    long_table = tuple(perm[4:4 + 3000 // block + 1])
    large = small + (BatchEntry("c", tuple(i % 15 + 1 for i in range(3000)), tuple(range(3000)), long_table, 2999),)
    for entries in (small, large, small, large):
        batch = ExecutionBatch(entries)
        total = batch.num_tokens
        q, k, v = (rng.standard_normal((total, 2, 32)).astype(np.float32) for _ in range(3))
        out = runner.attend(batch, *(torch.from_numpy(a).to(device) for a in (q, k, v))).cpu().numpy()
        slots = [s for e in entries for s in slots_for(e.seq_id, e.positions, e.block_table, block)]
        oracle_append(keys, values, slots, k, v)
        assert np.array_equal(runner.key_cache[0].cpu().numpy(), keys)
        assert np.array_equal(runner.value_cache[0].cpu().numpy(), values)
        offset = 0
        for entry in entries:
            n = len(entry.token_ids)
            want = paged_attention(q[offset : offset + n], np.asarray(entry.positions), keys, values,
                                   np.asarray(entry.block_table), entry.context_len, 32**-0.5)  # fmt: skip
            assert float(np.max(np.abs(out[offset : offset + n] - want))) < 1e-5, (total, entry.seq_id)
            offset += n
    assert runner._staging.host.numel() > 1 << 16


@pytest.mark.parametrize("flush", ["block_view", "execute"])
def test_queued_copies_with_dependencies_land_in_order(device, models, flush) -> None:
    """Copies queued by copy_block run as batched launches of independent groups: a chain
    (1 -> 2, 2 -> 3), a swap back (4 -> 5, 5 -> 4) and a copy over a block read earlier in the
    same group (6 -> 7, 0 -> 6) must leave the pool exactly as copying one block at a time in
    queue order (runner.py:128-133). Flushed by block_view, or by the next execute, which sends
    the pairs in its metadata copy and launches one copy per group before its kernels."""
    model, _ = models
    runner = ModelRunner(model, num_blocks=12, block_size=BLOCK_SIZE, device=device)
    keys, values = runner.key_cache, runner.value_cache  # [layers, blocks, B, H, D]
    keys.copy_(torch.randn(keys.shape, device=device))
    values.copy_(torch.randn(values.shape, device=device))
    want_k, want_v = keys.cpu().numpy().copy(), values.cpu().numpy().copy()
    pairs = [(1, 2), (2, 3), (4, 5), (5, 4), (6, 7), (0, 6), (9, 10)]
    for src, dst in pairs:
        runner.copy_block(src, dst)
        want_k[:, dst] = want_k[:, src]
        want_v[:, dst] = want_v[:, src]
    if flush == "block_view":
        runner.block_view(0)
    else:  # a batch writing only block 11, so the copied blocks keep their bytes
        runner.execute(ExecutionBatch((BatchEntry("x", (1,), (0,), (11,), 0),)))
        want_k[:, 11], want_v[:, 11] = keys[:, 11].cpu().numpy(), values[:, 11].cpu().numpy()
    assert np.array_equal(keys.cpu().numpy(), want_k)
    assert np.array_equal(values.cpu().numpy(), want_v)


@pytest.mark.parametrize("case", ["same_sequence_twice", "shared_written_block", "private"])
def test_decode_rows_reading_a_block_another_row_writes(device, case) -> None:
    """A decode batch whose rows read a slot another row of the same call writes: the reference
    writes every new key and value before any attention (runner.py:195-212), so each reader sees
    the new bytes. The runner then appends before attending instead of fusing the append into the
    attention call; a batch of private tables still takes the fused path. Outputs match the
    oracle (1e-5) and the pool matches its append bit for bit."""
    from oracle.attention import paged_attention
    from oracle.runner import append as oracle_append, slots_for

    rng = np.random.default_rng(7)
    config = ModelConfig(vocab_size=16, d_model=256, n_layers=1, n_heads=4, d_ff=32, max_seq_len=4096)
    model = LanguageModel(config, random_weights(config, seed=7))
    block, num_blocks = 16, 400
    perm = [int(b) for b in rng.permutation(num_blocks)]
    a, b, c = tuple(perm[:40]), tuple(perm[40:70]), tuple(perm[70:75])
    if case == "same_sequence_twice":  # one sequence at positions p and p + 1 (same block)
        entries = [BatchEntry("x", (1,), (600,), a, 0), BatchEntry("y", (1,), (300,), b, 0),
                   BatchEntry("x", (2,), (601,), a, 0)]  # fmt: skip
    elif case == "shared_written_block":  # y's table ends in the block x writes
        entries = [BatchEntry("x", (1,), (600,), a, 0), BatchEntry("y", (1,), (70,), c[:4] + (a[37],), 0)]
    else:
        entries = [BatchEntry("x", (1,), (600,), a, 0), BatchEntry("y", (1,), (70,), c, 0)]
    batch = ExecutionBatch(tuple(entries))
    runner = ModelRunner(model, num_blocks=num_blocks, block_size=block, device=device)
    keys = rng.standard_normal((num_blocks, block, 4, 64)).astype(np.float32)
    values = rng.standard_normal((num_blocks, block, 4, 64)).astype(np.float32)
    runner.key_cache[0].copy_(torch.from_numpy(keys))
    runner.value_cache[0].copy_(torch.from_numpy(values))
    q, k, v = (rng.standard_normal((len(entries), 4, 64)).astype(np.float32) for _ in range(3))
    step = runner._prepare(batch)
    assert step.decode_only == (case == "private")
    out = runner.attend(batch, *(torch.from_numpy(t).to(device) for t in (q, k, v))).cpu().numpy()
    slots = [s for e in entries for s in slots_for(e.seq_id, e.positions, e.block_table, block)]
    oracle_append(keys, values, slots, k, v)
    assert np.array_equal(runner.key_cache[0].cpu().numpy(), keys)
    assert np.array_equal(runner.value_cache[0].cpu().numpy(), values)
    for i, entry in enumerate(entries):
        want = paged_attention(q[i : i + 1], np.asarray(entry.positions), keys, values, np.asarray(entry.block_table),
                               entry.context_len, 64**-0.5)  # fmt: skip
        assert float(np.max(np.abs(out[i] - want[0]))) < 1e-5, (case, entry.seq_id)


def test_a_decode_loop_with_forks_and_copies_matches_the_oracle_step_by_step(device) -> None:
    """Thirty steps of a serving loop through ModelRunner.attend, driven by the KV-cache manager:
    two parents prefill their prompts, children fork from them at different steps (a first write
    into a shared block copies it through the runner's copy_block), some finish and free their
    blocks, and every step's batch is rebuilt from the sequences' block-table lists in a shuffled
    order (tuple(seq.block_table), as the reference's scheduler builds its entries,
    scheduler.py:423), so rows come and go in the arena and sharers of one prefix are interleaved
    with the other family's. After every step the pools equal a NumPy shadow that applies the same
    copies and appends in order, bit for bit, and every output row is within 1e-5 of the
    oracle's paged attention over the shadow."""
    from oracle.attention import paged_attention
    from oracle.runner import append as oracle_append
    from oracle.runner import copy_block as oracle_copy
    from oracle.runner import slots_for

    rng = np.random.default_rng(23)
    heads, dim, block, num_blocks = 4, 64, 16, 640
    config = ModelConfig(vocab_size=64, d_model=heads * dim, n_layers=1, n_heads=heads, d_ff=32, max_seq_len=2048)
    model = LanguageModel(config, random_weights(config, seed=23))
    runner = ModelRunner(model, num_blocks=num_blocks, block_size=block, device=device)
    keys = rng.standard_normal((1, num_blocks, block, heads, dim)).astype(np.float32)
    values = rng.standard_normal((1, num_blocks, block, heads, dim)).astype(np.float32)
    runner.key_cache.copy_(torch.from_numpy(keys))
    runner.value_cache.copy_(torch.from_numpy(values))
    copies: list[tuple[int, int]] = []

    class Store:  # the runner's copy_block, recorded for the shadow
        def copy_block(self, source: int, destination: int) -> None:
            runner.copy_block(source, destination)
            copies.append((source, destination))

    blocks = BlockManager(num_blocks=num_blocks, block_size=block, store=Store())
    cache = KVCacheManager(blocks, PrefixCache(blocks, enabled=False))
    scale = dim**-0.5
    worst, fused_steps, tiled = 0.0, 0, 0

    def run(steps):  # one attend call over [(sequence, new token count)], checked against the shadow
        nonlocal worst, fused_steps, tiled
        entries = []
        for seq, n in steps:
            start = seq.num_computed_tokens
            cache.reserve(seq, start + n)
            entries.append(BatchEntry(seq.seq_id, tuple(seq.token_ids[start : start + n]),
                                      tuple(range(start, start + n)), tuple(seq.block_table), n - 1))  # fmt: skip
        batch = ExecutionBatch(tuple(entries))
        total = batch.num_tokens
        q, k, v = (rng.standard_normal((total, heads, dim)).astype(np.float32) for _ in range(3))
        out = runner.attend(batch, *(torch.from_numpy(a).to(device) for a in (q, k, v))).cpu().numpy()
        for source, destination in copies:
            oracle_copy(keys, values, source, destination)
        copies.clear()
        slots = [s for e in entries for s in slots_for(e.seq_id, e.positions, e.block_table, block)]
        oracle_append(keys[0], values[0], slots, k, v)
        assert np.array_equal(runner.key_cache.cpu().numpy(), keys)
        assert np.array_equal(runner.value_cache.cpu().numpy(), values)
        offset = 0
        for entry in entries:
            n = len(entry.token_ids)
            want = paged_attention(q[offset : offset + n], np.asarray(entry.positions), keys[0], values[0],
                                   np.asarray(entry.block_table), entry.context_len, scale)  # fmt: skip
            worst = max(worst, float(np.max(np.abs(out[offset : offset + n] - want))))
            offset += n
        fused_steps += runner.last_append_fused
        tiled += runner.last_plan is not None and runner.last_plan.tiles.shape[0] > 0
        for seq, n in steps:
            seq.num_computed_tokens += n

    parents = []
    for name, length in (("pa", 600), ("pb", 530)):  # 37 blocks + 8 and 33 blocks + 2: partial last blocks
        parent = Sequence.from_request(Request(name, tuple(int(t) for t in rng.integers(0, 64, length))), 0)
        parents.append(parent)
    run([(p, p.num_tokens) for p in parents])
    live, made = list(parents), 0
    for step in range(30):
        if step in (0, 4, 11):  # new children of both parents
            for parent in parents:
                for _ in range(15 if step == 0 else 4):
                    child = Sequence.from_request(Request(f"c{made}", tuple(parent.token_ids)), 0)
                    made += 1
                    cache.fork(parent, child)
                    live.append(child)
        if step in (8, 19):  # a few children finish
            for seq in [s for s in live if s not in parents][:5]:
                cache.free(seq)
                live.remove(seq)
        for seq in live:
            seq.token_ids.append(int(rng.integers(0, 64)))
        order = rng.permutation(len(live))
        run([(live[i], 1) for i in order])
        cache.check_invariants()
    assert worst < 1e-5
    assert fused_steps >= 25, "decode steps append inside the attention call"
    assert tiled >= 25, "interleaved sharers regrouped and read through prefix tiles"


def test_attend_on_an_empty_batch_returns_no_rows(device) -> None:
    """An empty ExecutionBatch: attend returns a [0, heads, head_dim] float32 tensor on the
    device, launches nothing and leaves a queued copy-on-write copy queued; reading the pools
    (key_cache) lands it."""
    config = ModelConfig(vocab_size=16, d_model=64, n_layers=1, n_heads=2, d_ff=32, max_seq_len=64)
    model = LanguageModel(config, random_weights(config, seed=3))
    runner = ModelRunner(model, num_blocks=4, block_size=4, device=device)
    runner.key_cache.copy_(torch.randn_like(runner.key_cache))
    want = runner.key_cache.clone()
    want[:, 1] = want[:, 0]
    runner.copy_block(0, 1)
    none = torch.zeros((0, 2, 32), device=device)
    out = runner.attend(ExecutionBatch(()), none, none, none)
    assert out.shape == (0, 2, 32) and out.dtype == torch.float32 and out.device == none.device
    assert runner.pending_copies == [(0, 1)]
    assert torch.equal(runner.key_cache, want) and runner.pending_copies == []
