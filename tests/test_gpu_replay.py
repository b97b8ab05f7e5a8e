"""Recorded reference serving runs replayed through the GPU ModelRunner.

The traces (tests/golden/traces/, written from the reference engine by
tests/golden/make_reference_traces.py) are config 1, the reference's bench_engine_equivalence
shape, three small-pool runs with prefix sharing, n-way forks, copy-on-write, preemption and
eviction, and a run of the reference's StaticBatchingEngine (padded prefill, whole slot regions
as tables, finished rows re-run). The replay drives this package's KVCacheManager with the
reference engine's calls and the GPU ModelRunner with its batches, so copy-on-write copies,
slot-mapped appends and paged attention all run on the device in the reference's order. Checked: every block table, slot
mapping and copy-on-write pair bit for bit; every logits row within 1e-4 of the reference's
recorded NumPy row and of the cache-free recompute (the reference's bar,
tests/property/test_equivalence.py:34); greedy rows pick the reference's token unless the
reference's two best logits are within 1e-4 of each other.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle.model import OracleModel
from paged_kv_serving_amd.replay import Trace, TraceReplay

pytestmark = pytest.mark.gpu

TRACES = Path(__file__).resolve().parent / "golden" / "traces"
NAMES = ("config1", "engine_equivalence", "sharing_b8", "sharing_b4", "sharing_b16")


def _runner(trace, device, **kwargs):
    from paged_kv_serving_amd.runner import ModelRunner

    model = trace.language_model()
    engine = trace.engine
    return model, ModelRunner(model, num_blocks=engine["num_blocks"], block_size=engine["block_size"],
                              device=device, **kwargs)  # fmt: skip


def _tokens_agree(trace, result, rows) -> tuple[int, int]:
    """(greedy rows whose argmax is the reference's token, greedy rows checked) over rows whose
    reference top-2 margin exceeds 1e-4."""
    greedy = trace.greedy_requests
    agree = checked = 0
    for row, ref_row, (seq_id, context) in zip(rows, trace.logits, result.row_seqs):
        if seq_id.rsplit("#", 1)[0] not in greedy:
            continue
        top2 = np.sort(ref_row)[-2:]
        if top2[1] - top2[0] <= 1e-4:
            continue
        checked += 1
        agree += int(np.argmax(row)) == trace.tokens[seq_id][context]
    return agree, checked


@pytest.mark.parametrize("name", NAMES)
def test_the_reference_run_replays_on_the_gpu_runner(name, device) -> None:
    trace = Trace.load(TRACES / f"{name}.json")
    model, runner = _runner(trace, device)
    print(f"replay {name}: {len(trace.events)} events, {len(trace.iterations)} iterations", flush=True)
    result = TraceReplay(trace, runner).run()
    rows = np.stack(result.rows)
    gap_ref = float(np.max(np.abs(rows - trace.logits)))
    oracle = OracleModel(model.config, model.weights)
    dense, gap_dense = {}, 0.0
    for row, (seq_id, context) in zip(rows, result.row_seqs):
        if seq_id not in dense:
            dense[seq_id] = oracle.reference_forward(trace.tokens[seq_id])
        gap_dense = max(gap_dense, float(np.max(np.abs(dense[seq_id][context - 1] - row))))
    agree, checked = _tokens_agree(trace, result, rows)
    print(f"replay {name}: {rows.shape[0]} rows, {result.copies} COW copies, gap vs reference rows "
          f"{gap_ref:.3g}, vs recompute {gap_dense:.3g} (reference's own {trace.summary['reference_max_abs_logit_gap']:.3g}); "
          f"greedy tokens {agree}/{checked}", flush=True)  # fmt: skip
    assert gap_ref < 1e-4 and gap_dense < 1e-4
    assert agree == checked


def test_a_bfloat16_pool_replays_config1_within_tolerance(device) -> None:
    """Config 1 over a bfloat16 pool: tables and slots are unchanged (bit-exact checks pass);
    logits stay within 2e-2 of the fp32 reference rows (K/V rounded to 8 mantissa bits)."""
    import torch

    trace = Trace.load(TRACES / "config1.json")
    _, runner = _runner(trace, device, kv_dtype=torch.bfloat16)
    result = TraceReplay(trace, runner).run()
    gap = float(np.max(np.abs(np.stack(result.rows) - trace.logits)))
    print(f"config 1 on a bf16 pool: gap {gap:.3g}", flush=True)
    assert gap < 2e-2


def test_device_greedy_sampling_picks_the_host_argmax(device) -> None:
    """execute_greedy (argmax on the device, one int32 per row back) against np.argmax of the
    rows execute returns, over the whole config-1 run."""
    trace = Trace.load(TRACES / "config1.json")
    _, host_runner = _runner(trace, device)
    rows = np.stack(TraceReplay(trace, host_runner).run().rows)
    _, device_runner = _runner(trace, device)
    picked = TraceReplay(trace, device_runner, greedy=True).run().greedy
    assert picked == [int(np.argmax(row)) for row in rows]


@pytest.mark.parametrize("greedy", [False, True])
def test_the_static_batching_run_replays_on_the_gpu_runner(device, greedy) -> None:
    """The reference StaticBatchingEngine's recorded batches (static.py:183-226) through the GPU
    ModelRunner made as that engine makes its own (static.py:124-126): prefill rows padded to the
    group's longest prompt, logits read at each row's own last prompt token, block tables of a
    whole slot region, finished rows re-run at their last position. Slots bit for bit; every row
    within 1e-4 of the reference's recorded row and of the cache-free recompute; with greedy
    sampling on the device, every greedy row that the reference continued picks its token (rows
    whose reference top-2 margin is 1e-4 or less excepted)."""
    from paged_kv_serving_amd.replay import StaticReplay
    from paged_kv_serving_amd.runner import ModelRunner

    trace = Trace.load(TRACES / "static_batching.json")
    model = trace.language_model()
    engine = trace.engine
    runner = ModelRunner(model, num_blocks=engine["batch_size"] * engine["blocks_per_slot"],
                         block_size=engine["block_size"], device=device)  # fmt: skip
    print(f"static replay: {len(trace.iterations)} iterations, greedy={greedy}", flush=True)
    result = StaticReplay(trace, runner, greedy=greedy).run()
    greedy_ids = {f"{r['request_id']}#0" for r in trace.requests if r["temperature"] < 1e-5}
    if greedy:
        checked = 0
        for token, ref_row, (seq_id, context) in zip(result.greedy, trace.logits, result.row_seqs):
            top2 = np.sort(ref_row)[-2:]
            if seq_id in greedy_ids and context < len(trace.tokens[seq_id]) and top2[1] - top2[0] > 1e-4:
                assert token == trace.tokens[seq_id][context], (seq_id, context)
                checked += 1
        print(f"static replay: {checked} greedy rows pick the reference's token", flush=True)
        assert checked > 100
        return
    rows = np.stack(result.rows)
    gap_ref = float(np.max(np.abs(rows - trace.logits)))
    oracle = OracleModel(model.config, model.weights)
    dense, gap_dense = {}, 0.0
    for row, (seq_id, context) in zip(rows, result.row_seqs):
        if seq_id not in dense:
            dense[seq_id] = oracle.reference_forward(trace.tokens[seq_id])
        gap_dense = max(gap_dense, float(np.max(np.abs(dense[seq_id][context - 1] - row))))
    print(f"static replay: {rows.shape[0]} rows, gap vs reference rows {gap_ref:.3g}, vs recompute {gap_dense:.3g}",
          flush=True)  # fmt: skip
    assert gap_ref < 1e-4 and gap_dense < 1e-4
