"""Benchmark of the KV-cache data path on one MI355X (BASELINE.json ``metric``).

Workload ("config 2"): one decode step of one layer for 64 sequences
with contexts uniform in [512, 4096], 32 heads x head_dim 128 (MHA), block_size 16, float32 K/V,
block tables drawn from a shuffled 20,000-block pool; seeded N(0, 1) data resident in HBM.
A step is the data path of that iteration, in one call:

    pkv_paged_attention_append  the 64 new tokens' keys and values into their slots, appended by
                                the row pass itself, and 64 decode queries over their block
                                tables (row pass + reduce pass)

The standalone pkv_append on the same tokens is timed outside the steps and reported as
``append_us`` / ``append_gbps`` (4.2 MB: launch-bound), beside the attention call without the
fused append (``fused_append_cost_us`` is the difference). ``append_bulk`` times pkv_append of
every context token of the 64 sequences (the append of a 64 x 4k-context prefill, 9.8 GB) for
the append's HBM rate at that scale.

``value`` is decode tokens per second (64 tokens per step). The roofline object is for the
dominant kernel, the attention pass: achieved = algorithmic bytes per launch (each sequence's
K+V context read once, plus queries, outputs and block tables) / its mean duration, measured
with HIP events on the launching stream over the timed steps. The CPU baseline times the
oracle's NumPy restatement of the reference path (reference attention.py:42-121 per sequence,
tile_blocks 8, plus the runner.py:195-196 append) on a bounded sample of the same workload,
single-threaded BLAS as the reference pins it.

The default run then times the other BASELINE.json configurations in the same process (configs
1, 3, 4 and 5, up to 20 steps each) and adds their figures as ``other_configs``; the headline
``value`` and ``roofline`` stay config 2's.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--partition P] [--no-cpu] [--no-others]
       python bench.py --config {1,3,4,5}   (the other BASELINE.json configurations;
                                         --config 3 --kv bf16: its shape on bfloat16 pools)
       python bench.py --micro              (the reference's published micro-benchmarks)
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, published
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix, published
METRIC = "paged-attn decode tokens/s & HBM GB/s (% of peak) at 64 seq x 4k ctx; append GB/s"


def parse() -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--config", type=int, default=2, choices=(1, 2, 3, 4, 5),
                        help="BASELINE.json config to run (2 is the headline metric)")
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--partition", type=int, default=0, help="keys per partition (0: default)")
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--kv", choices=("f32", "bf16"), default="f32",
                        help="config 3's K/V pool type (the configuration itself is float32)")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    parser.add_argument("--no-others", action="store_true",
                        help="config 2 only: skip the other configurations of the default run")
    parser.add_argument("--cpu-seqs", type=int, default=64, help="sequences in the CPU sample")
    parser.add_argument("--cpu-repeats", type=int, default=5, help="timed CPU steps (median)")
    parser.add_argument("--micro", action="store_true",
                        help="the reference's published micro-benchmarks of the path instead")
    return parser.parse_args()


def traffic_from_profiles() -> float | None:
    """HBM bytes per attention launch measured with rocprofv3 FETCH_SIZE/WRITE_SIZE, if recorded."""
    path = ROOT / "profiles" / "attention_decode_config2_traffic.json"
    if not path.exists():
        return None
    try:
        return float(json.loads(path.read_text())["bytes_per_launch"])
    except (KeyError, ValueError, json.JSONDecodeError):
        return None


def copy_peak(device) -> dict:
    """Achievable HBM copy bandwidth on this box: pkv_copy_blocks over 2048 contiguous block
    pairs of a separate [1, 4096, 16, 32, 128] float32 pool pair (1 GiB read + 1 GiB written).
    The same dispatch is the known-size reference for the rocprofv3 FETCH_SIZE/WRITE_SIZE
    calibration."""
    import torch

    from paged_kv_serving_amd import ops

    keys = torch.zeros((1, 4096, 16, 32, 128), dtype=torch.float32, device=device)
    values = torch.zeros_like(keys)
    pairs = torch.stack([torch.arange(2048), torch.arange(2048, 4096)], dim=1).to(device)
    for _ in range(3):
        ops.copy_blocks(keys, values, pairs)
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(10)]
    for start, stop in marks:
        start.record()
        ops.copy_blocks(keys, values, pairs)
        stop.record()
    torch.cuda.synchronize()
    ms = float(np.median([a.elapsed_time(b) for a, b in marks]))
    moved = 2 * 2 * 2048 * 16 * 32 * 128 * 4  # K and V, read + write
    del keys, values
    return {"copy_peak_gbps": round(moved / (ms * 1e-3) / 1e9, 1), "copy_bytes": moved, "copy_ms": round(ms, 4)}


def cpu_baseline(args: argparse.Namespace) -> dict:
    """Oracle (NumPy restatement of the reference path) on a bounded sample of config 2."""
    from oracle.attention import paged_attention
    from oracle.runner import append

    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    rng = np.random.default_rng(args.seed)
    contexts = rng.integers(512, 4097, 64)[: args.cpu_seqs]  # the workload's first sequences
    heads, dim, block = 32, 128, 16
    need = [-(-int(c) // block) for c in contexts]
    pool = sum(need)
    data = np.random.default_rng(args.seed + 1)
    # Uniform fill: the timing depends on bytes moved, not on the distribution of the values.
    keys = data.random((pool, block, heads, dim), dtype=np.float32)
    values = data.random((pool, block, heads, dim), dtype=np.float32)
    perm = data.permutation(pool)
    tables, offset = [], 0
    for n in need:
        tables.append(perm[offset : offset + n])
        offset += n
    queries = data.standard_normal((len(contexts), 1, heads, dim), dtype=np.float32)
    new_k = data.standard_normal((len(contexts), 1, heads, dim), dtype=np.float32)
    new_v = data.standard_normal((len(contexts), 1, heads, dim), dtype=np.float32)
    scale = dim**-0.5

    def step() -> None:
        for s, ctx in enumerate(contexts):
            p = int(ctx) - 1
            slot = int(tables[s][p // block]) * block + p % block
            append(keys, values, [slot], new_k[s], new_v[s])
            paged_attention(queries[s], np.asarray([p]), keys, values, tables[s], int(ctx), scale, tile_blocks=8)

    from contextlib import nullcontext

    def median_seconds() -> float:
        step()  # warmup
        samples = []
        for _ in range(args.cpu_repeats):
            start = time.perf_counter_ns()
            step()
            samples.append((time.perf_counter_ns() - start) / 1e9)
        return float(np.median(samples))

    with threadpool_limits(1) if threadpool_limits else nullcontext():
        seconds = median_seconds()
    # The reference pins BLAS to one thread; a second run with the library's default pool.
    threads = None
    if threadpool_limits is not None:
        from threadpoolctl import threadpool_info

        threads = max((int(i.get("num_threads", 1)) for i in threadpool_info()), default=1)
    seconds_all = median_seconds()
    kv_bytes = int(contexts.sum()) * 2 * heads * dim * 4
    return {
        "value": round(len(contexts) / seconds, 2),
        "unit": "decode tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": (
            f"{len(contexts)} of the 64 config-2 sequences (contexts {int(contexts.min())}-"
            f"{int(contexts.max())}, {kv_bytes / 1e9:.2f} GB K+V), oracle NumPy paged attention "
            f"tile_blocks 8 + append, 1 BLAS thread, median of {args.cpu_repeats} after 1 warmup"
        ),
        "seconds_per_sample": round(seconds, 4),
        "gbps": round(kv_bytes / seconds / 1e9, 3),
        "all_cores": {
            "value": round(len(contexts) / seconds_all, 2),
            "blas_threads": threads,
            "gbps": round(kv_bytes / seconds_all / 1e9, 3),
        },
        "host_cpus": os.cpu_count(),
        "cpu_model": cpu_model(),
    }


def cpu_model() -> str | None:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def timed(fn, steps: int, stream) -> float:
    """Mean milliseconds of ``fn`` over ``steps`` calls, by HIP events on ``stream``."""
    import torch

    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for start, stop in marks:
        start.record(stream)
        fn()
        stop.record(stream)
    torch.cuda.synchronize()
    return float(np.mean([a.elapsed_time(b) for a, b in marks]))


def attention_call(batch, args, out, workspace, *, fused_append: bool = False):
    """One ragged attention call over the batch; with ``fused_append`` the decode append rides
    in the same call (pkv_paged_attention_append)."""
    from paged_kv_serving_amd import ops

    append = (batch.new_keys, batch.new_values, batch.slot_mapping) if fused_append else None

    def attend() -> None:
        ops.paged_attention_ragged(
            batch.queries, batch.query_positions, batch.query_seq, batch.key_cache,
            batch.value_cache, batch.block_tables, batch.context_lens, batch.scale,
            max_context_len=batch.max_context_len, out=out, workspace=workspace, plan=batch.plan,
            append=append,
        )  # fmt: skip

    return attend


def run_attention_config(args, batch, *, metric: str, workload: str, dtype: str, extra=None) -> dict:
    """Time ``args.steps`` steps of append + ragged attention on a resident batch."""
    import torch

    from paged_kv_serving_amd import ops

    if args.partition:
        batch.replan(args.partition)

    device = batch.queries.device
    heads, dim = batch.key_cache.shape[2], batch.key_cache.shape[3]
    need = ops.attention_workspace_bytes(
        batch.num_queries, heads, dim, batch.max_context_len, batch.plan.partition_size
    )
    workspace = torch.empty(max(need // 4, 1), dtype=torch.float32, device=device)
    out = torch.empty_like(batch.queries)

    def append() -> None:
        ops.append_kv(batch.key_cache, batch.value_cache, batch.new_keys, batch.new_values, batch.slot_mapping)

    # A decode batch (one row per sequence, at its last position) whose written blocks no other
    # row reads appends inside the attention call, as the runner does; any other batch appends
    # first with its own launch.
    fused = batch.fusable_append()
    attend = attention_call(batch, args, out, workspace, fused_append=fused)
    for _ in range(args.warmup):
        if not fused:
            append()
        attend()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(device)
    # Events bracket each attention call (and the separate append, when there is one); the fused
    # step records only the two around its single call.
    marks = [[torch.cuda.Event(enable_timing=True) for _ in range(2 if fused else 3)] for _ in range(args.steps)]
    start = time.perf_counter()
    for events in marks:
        if not fused:
            events[-3].record(stream)
            append()
        events[-2].record(stream)
        attend()
        events[-1].record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    attention_ms = float(np.mean([events[-2].elapsed_time(events[-1]) for events in marks]))
    if fused:
        # The standalone append kernel on the same tokens, outside the timed steps, for the
        # record (it rewrites the same rows with the same values). Each one is queued behind an
        # attention call, so the GPU does not wait for the host to submit it.
        # The same attention without the fused append is timed between them, so the fused
        # append's own cost is the difference of the two attention times.
        plain = attention_call(batch, args, out, workspace)
        standalone = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
        for p0, e0, e1 in standalone:
            p0.record(stream)
            plain()
            e0.record(stream)
            append()
            e1.record(stream)
        torch.cuda.synchronize()
        plain_ms = float(np.mean([p0.elapsed_time(e0) for p0, e0, _ in standalone]))
        append_ms = float(np.mean([e0.elapsed_time(e1) for _, e0, e1 in standalone]))
    else:
        append_ms = float(np.mean([events[0].elapsed_time(events[1]) for events in marks]))
    tokens = batch.num_queries
    esize = batch.key_cache.element_size()
    kv_bytes = batch.context_bytes()
    io_bytes = 2 * tokens * heads * dim * 4 + batch.block_tables.numel() * 4 + 3 * tokens * 4
    attention_bytes = kv_bytes + io_bytes
    append_bytes = 2 * tokens * heads * dim * (4 + esize) + tokens * 8  # read k, v + write k, v
    achieved = attention_bytes / (attention_ms * 1e-3) / 1e9
    result = {
        "metric": metric,
        "value": round(tokens * args.steps / elapsed, 1),
        "unit": "query tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic: seeded N(0,1) K/V pools, queries and new tokens resident in HBM",
        "config": {
            "workload": workload,
            "partition_size": batch.plan.partition_size or 512,
            "shared_prefix_tiles": int(batch.plan.tiles[:, 3].gt(0).sum()) if batch.plan.num_tiles else 0,
            "kv_loads": "cached" if batch.plan.shared_kv else "streaming",
            "context_tokens": int(kv_bytes // (2 * heads * dim * esize)),
        },
        "attention_ms": round(attention_ms, 4),
        "attention_gbps": round(achieved, 1),
        "attention_frac_of_peak": round(achieved / HBM_PEAK_GBPS, 4),
        "attention_tokens_per_s": round(tokens / (attention_ms * 1e-3), 1),
        "append_fused_into_attention": fused,
        **({"attention_without_append_ms": round(plain_ms, 4),
            "fused_append_cost_us": round((attention_ms - plain_ms) * 1e3, 2)} if fused else {}),
        "append_us": round(append_ms * 1e3, 2),
        "append_gbps": round(append_bytes / (append_ms * 1e-3) / 1e9, 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": None,
            "kernel": "pkv_paged_attention (row_partial + tile_partial + reduce)",
            "algorithmic_bytes_per_launch": attention_bytes,
        },
    }
    if extra:
        result.update(extra(result, attention_ms))
    return result


def config2(args) -> dict:
    from paged_kv_serving_amd.workloads import decode_batch

    import torch

    batch = decode_batch(seed=args.seed, device=torch.device("cuda", 0))
    result = run_attention_config(
        args, batch, metric=METRIC, dtype="f32",
        workload="config2 decode: 64 seqs, ctx U[512,4096] (seed 0), 32 heads x 128 MHA, "
        "block 16, fp32 KV, 20000-block shuffled pool, 1 layer; step = append 64 tokens + "
        "paged attention in one call (append fused into the row pass)",
    )  # fmt: skip
    result["unit"] = "decode tokens/s"
    result.update(bulk_append_timing(args, batch))
    result.update(runner_step_timing(args, batch))
    result["runner_step_over_kernel"] = round(result["runner_step_ms"] / result["attention_ms"], 4)
    result["roofline"]["traffic"] = traffic_from_profiles()
    result["roofline"]["kernel"] = (
        "row_partial_kernel<float,128> (append fused) + reduce_kernel<128>"
        if result["append_fused_into_attention"] else "row_partial_kernel<float,128> + reduce_kernel<128>"
    )
    return result


def runner_step_timing(args, batch, *, cow_pairs=None) -> dict:
    """The same step through ``ModelRunner.attend``, as a serving loop runs it: reference-style
    BatchEntry objects (one per sequence, its consecutive query rows as one chunk; block tables
    as tuples), host validation and slots, the block-table arena
    update, the host plan (pkv_plan_batch), one metadata copy from pinned memory, the queued
    copy-on-write flush (config 4), the append + attention call, and the synchronisation that
    ends a step. Wall time per step, median; the runner has its own pool of the batch's size and
    a model object with only the attention shape (attend reads no weights)."""
    from types import SimpleNamespace

    import torch

    from paged_kv_serving_amd.config import ModelConfig
    from paged_kv_serving_amd.runner import BatchEntry, ExecutionBatch, ModelRunner

    device = batch.queries.device
    num_blocks, block = batch.key_cache.shape[0], batch.key_cache.shape[1]
    heads, dim = batch.key_cache.shape[2], batch.key_cache.shape[3]
    config = ModelConfig(vocab_size=2, d_model=heads * dim, n_layers=1, n_heads=heads, d_ff=1,
                         max_seq_len=int(batch.max_context_len) + 1)  # fmt: skip
    model = SimpleNamespace(config=config, weights=None, rope=None, attention_scale=float(batch.scale))
    runner = ModelRunner(model, num_blocks=num_blocks, block_size=block, device=device, kv_dtype=batch.key_cache.dtype)
    entries = []
    seq, pos = batch.host_seq, batch.host_positions
    starts = np.flatnonzero(np.r_[True, seq[1:] != seq[:-1]])  # runs of one sequence's rows
    for first, end in zip(starts.tolist(), np.r_[starts[1:], seq.size].tolist()):
        s = int(seq[first])
        entries.append(BatchEntry(f"s{s}", (0,) * (end - first), tuple(int(p) for p in pos[first:end]),
                                  tuple(int(b) for b in batch.host_tables[s]), end - first - 1))  # fmt: skip
    step_batch = ExecutionBatch(tuple(entries))

    def step() -> None:
        for source, destination in cow_pairs or ():
            runner.copy_block(source, destination)
        runner.attend(step_batch, batch.queries, batch.new_keys, batch.new_values)
        torch.cuda.synchronize(device)

    for _ in range(max(args.warmup, 3)):
        step()
    seconds = []
    for _ in range(max(args.steps, 5)):
        start = time.perf_counter()
        step()
        seconds.append(time.perf_counter() - start)
    ms = float(np.median(seconds)) * 1e3
    del runner
    torch.cuda.empty_cache()
    return {"runner_step_ms": round(ms, 4)}


def config3(args) -> dict:
    import torch

    from paged_kv_serving_amd.workloads import mixed_batch

    kv = torch.bfloat16 if args.kv == "bf16" else torch.float32
    batch = mixed_batch(seed=args.seed, device=torch.device("cuda", 0), kv_dtype=kv)
    offsets = batch.host_positions[batch.host_seq < 8].reshape(8, -1)[:, 0]
    # causal prefill FLOPs: each chunk row i at offset o sees o + i + 1 keys; QK^T and PV, 2 each
    visible = sum(int((o + np.arange(1, 513)).sum()) for o in offsets)
    prefill_flops = 4 * 32 * 128 * visible

    rope = rope_append_timing(args, batch)
    tiles_ms = prefill_tiles_alone_ms(args, batch)
    tflops = prefill_flops / (tiles_ms * 1e-3) / 1e12

    def extra(result, attention_ms):
        return {
            "prefill_gflop": round(prefill_flops / 1e9, 2),
            # The chunks' MFMA tiles as their own call (no decode rows beside them).
            "prefill_tiles_alone_ms": round(tiles_ms, 4),
            "prefill_tiles_alone_tflops": round(tflops, 1),
            "prefill_tiles_alone_frac_of_fp32_mfma_peak": round(tflops / FP32_MFMA_PEAK_TFLOPS, 4),
            **rope,
        }

    pool = "bf16 K/V (fp32 arithmetic)" if args.kv == "bf16" else "fp32"
    def extra_with_runner(result, attention_ms):
        out = extra(result, attention_ms)
        out.update(runner_step_timing(args, batch))
        out["runner_step_over_kernel"] = round(out["runner_step_ms"] / (attention_ms + result["append_us"] * 1e-3), 4)
        return out

    return run_attention_config(
        args, batch, dtype="f32", extra=extra_with_runner,
        metric="mixed ragged batch: query tokens/s, attention GB/s and append GB/s (config 3)",
        workload="config3 mixed: 8 prefill chunks x 512 tokens at offsets U[0,2048] + 120 decode "
        f"rows ctx U[256,4096], 32x128 {pool}, block 16, 40000-block shuffled pool; step = append "
        "4216 tokens + one ragged attention call (MFMA tiles for chunks, row pass for decode)",
    )  # fmt: skip


def prefill_tiles_alone_ms(args, batch) -> float:
    """Mean HIP-event time of the batch's prefill chunks as their own attention call: the
    chunks' rows (the batch's first rows) planned without the decode rows, so the plan holds
    whole tiles only and the tile pass runs one workgroup per (tile, head) with nothing beside
    it (the decode rows' outputs are left unwritten). This is the MFMA-bound part of config 3
    measured alone."""
    import torch

    from paged_kv_serving_amd import ops

    device = batch.queries.device
    heads, dim = batch.key_cache.shape[2], batch.key_cache.shape[3]
    block = batch.key_cache.shape[1]
    mixed = ops.plan_batch(
        batch.host_seq, dim, heads, batch.host_tables, batch.host_context, block,
        partition_size=args.partition, query_positions=batch.host_positions, kv_dtype=batch.key_cache.dtype,
    )  # fmt: skip
    chunk_rows = int((mixed.tiles[:, 0] + mixed.tiles[:, 1]).max())
    host = ops.plan_batch(
        batch.host_seq[:chunk_rows], dim, heads, batch.host_tables, batch.host_context, block,
        partition_size=args.partition, query_positions=batch.host_positions[:chunk_rows],
        kv_dtype=batch.key_cache.dtype,
    )  # fmt: skip
    if host.rows.shape[0] != 0 or int(host.tiles[:, 1].sum()) != chunk_rows:
        raise RuntimeError("the prefill chunks are not the batch's first rows")
    plan = ops.upload_plan(np.zeros((0, 2), np.int32), host.tiles, device,
                           partition_size=host.partition_size, merge=np.zeros(0, np.int32))  # fmt: skip
    need = ops.attention_workspace_bytes(batch.num_queries, heads, dim, batch.max_context_len,
                                         host.partition_size)  # fmt: skip
    workspace = torch.empty(max(need // 4, 1), dtype=torch.float32, device=device)
    out = torch.empty_like(batch.queries)

    def run() -> None:
        ops.paged_attention_ragged(
            batch.queries, batch.query_positions, batch.query_seq, batch.key_cache,
            batch.value_cache, batch.block_tables, batch.context_lens, batch.scale,
            max_context_len=batch.max_context_len, out=out, workspace=workspace, plan=plan,
        )  # fmt: skip

    for _ in range(max(args.warmup, 1)):
        run()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(device)
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(max(args.steps, 1))]  # fmt: skip
    for e0, e1 in marks:
        e0.record(stream)
        run()
        e1.record(stream)
    torch.cuda.synchronize()
    return float(np.mean([e0.elapsed_time(e1) for e0, e1 in marks]))


def bulk_append_timing(args, batch) -> dict:
    """``pkv_append`` of every context token of the batch, into the batch's own slots: the append
    a prefill of all its sequences makes (149,713 tokens for config 2, 9.8 GB moved). Timed with
    HIP events on the launching stream after the attention steps; it overwrites the pool rows
    with fresh values, which nothing timed afterwards reads for its result."""
    import torch

    from paged_kv_serving_amd import ops

    device = batch.queries.device
    _, block_size, heads, dim = batch.key_cache.shape
    slots = np.concatenate([
        np.asarray(table, dtype=np.int64)[np.arange(c) // block_size] * block_size + np.arange(c) % block_size
        for table, c in zip(batch.host_tables, batch.host_context.tolist())
    ])  # fmt: skip
    tokens = slots.size
    gen = torch.Generator(device=device)
    gen.manual_seed(args.seed + 1)
    keys = torch.randn((tokens, heads, dim), generator=gen, device=device)
    values = torch.randn((tokens, heads, dim), generator=gen, device=device)
    slot_mapping = torch.from_numpy(slots).to(device)

    def run() -> None:
        ops.append_kv(batch.key_cache, batch.value_cache, keys, values, slot_mapping)

    for _ in range(max(args.warmup, 1)):
        run()
    torch.cuda.synchronize()
    ms = timed(run, max(5, min(args.steps, 20)), torch.cuda.current_stream(device))
    moved = 2 * tokens * heads * dim * (4 + batch.key_cache.element_size()) + tokens * 8
    del keys, values, slot_mapping
    gbps = moved / (ms * 1e-3) / 1e9
    return {
        "append_bulk": {
            "tokens": tokens, "us": round(ms * 1e3, 1), "gbps": round(gbps, 1),
            "frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4), "bytes": moved,
            "what": "pkv_append of all context tokens of the 64 sequences (a 64 x 4k-context "
            "prefill's append), read k, v + write k, v + slots",
        }
    }  # fmt: skip


def rope_append_timing(args, batch) -> dict:
    """The fused RoPE + append kernel on the batch's tokens (a [T, 3, H, D] projection output),
    timed on its own as ModelRunner.execute runs it: the rotated queries overwrite the query
    slice of the projection output in place, the rotated keys and the values go to the pool."""
    import torch

    from paged_kv_serving_amd import ops
    from paged_kv_serving_amd.model import rope_tables

    device = batch.queries.device
    tokens, heads, dim = batch.queries.shape
    gen = torch.Generator(device=device)
    gen.manual_seed(args.seed)
    fused = torch.randn((tokens, 3, heads, dim), generator=gen, device=device)
    cos, sin = (torch.from_numpy(t).to(device) for t in rope_tables(4096, dim, 10_000.0))
    positions = batch.slot_mapping.remainder(4096)

    def run() -> None:
        ops.rope_append(
            batch.key_cache, batch.value_cache, fused[:, 0], fused[:, 1], fused[:, 2],
            positions, cos, sin, batch.slot_mapping, out=fused[:, 0],
        )  # fmt: skip

    for _ in range(max(args.warmup, 1)):
        run()
    torch.cuda.synchronize()
    ms = timed(run, args.steps, torch.cuda.current_stream(device))
    esize = batch.key_cache.element_size()
    row = heads * dim
    # read q, k, v and the two table rows; write q', k' and v
    moved = tokens * (3 * row * 4 + dim * 4 + row * 4 + 2 * row * esize + 16)
    return {
        "rope_append_us": round(ms * 1e3, 2),
        "rope_append_gbps": round(moved / (ms * 1e-3) / 1e9, 1),
        "rope_append_bytes": moved,
    }


def config5(args) -> dict:
    import torch

    from paged_kv_serving_amd.workloads import long_context_batch

    batch = long_context_batch(seed=args.seed, device=torch.device("cuda", 0))
    return run_attention_config(
        args, batch, dtype="bf16 storage, f32 math",
        metric="long-context decode tokens/s and HBM GB/s, bf16 KV (config 5)",
        workload="config5 long context: 16 seqs x 32768 ctx, bf16 KV, fp32 accumulation, 32x128, "
        "block 16, 40000-block shuffled pool, split-context partitions + reduce",
    )  # fmt: skip


def config4(args) -> dict:
    import torch

    from paged_kv_serving_amd import ops
    from paged_kv_serving_amd.workloads import prefix_sharing_step

    device = torch.device("cuda", 0)
    step = prefix_sharing_step(seed=args.seed, device=device)
    batch = step.decode
    stream = torch.cuda.current_stream(device)

    def cow() -> None:
        ops.copy_blocks(step.key_cache, step.value_cache, step.cow_pairs)

    for _ in range(args.warmup):
        cow()
    torch.cuda.synchronize()
    cow_ms = timed(cow, args.steps, stream)
    result = run_attention_config(
        args, batch, dtype="f32",
        metric="prefix sharing: COW GB/s and decode tokens/s over 256 sequences (config 4)",
        workload="config4 prefix sharing: 256 seqs fork a 1016-token prefix (63 full + 1 partial "
        "block), suffixes U[32,256]; 256 COW copies of the partial block, then one decode step",
    )  # fmt: skip
    result.update(runner_step_timing(args, batch, cow_pairs=step.host_pairs))
    result["runner_step_over_kernel"] = round(result["runner_step_ms"] / (result["attention_ms"] + cow_ms), 4)
    unique = step.unique_context_bytes()
    # The roofline counts each distinct block once: the shared prefix is one HBM read, and the
    # logical rate (prefix counted per sequence) exceeds the HBM peak through cache hits.
    unique_rate = unique / (result["attention_ms"] * 1e-3) / 1e9
    result["roofline"].update({
        "achieved": round(unique_rate, 1),
        "frac": round(unique_rate / HBM_PEAK_GBPS, 4),
        "algorithmic_bytes_per_launch": unique,
        "bytes_counted": "distinct K+V blocks read once",
    })  # fmt: skip
    # The 256 COW pairs all copy the same partial block (every sequence forked it), so after its
    # first read the caches serve the source: cow_gbps is not an HBM rate. The same launch over
    # 256 distinct random sources (HBM-bound) gives the copy's HBM rate; run last, it overwrites
    # pool blocks the decode step used.
    rng = np.random.default_rng(args.seed + 1)
    picks = rng.permutation(step.key_cache.shape[1])[:512]
    distinct = torch.from_numpy(np.stack([picks[:256], picks[256:]], axis=1).astype(np.int64)).to(device)

    def cow_distinct() -> None:
        ops.copy_blocks(step.key_cache, step.value_cache, distinct)

    for _ in range(args.warmup):
        cow_distinct()
    torch.cuda.synchronize()
    distinct_ms = timed(cow_distinct, args.steps, stream)
    result.update({
        "cow_distinct_sources_us": round(distinct_ms * 1e3, 2),
        "cow_distinct_sources_gbps": round(step.cow_bytes() / (distinct_ms * 1e-3) / 1e9, 1),
        "cow_distinct_sources_frac_of_peak": round(step.cow_bytes() / (distinct_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
    })  # fmt: skip
    # Attention rates on the distinct blocks read (the roofline's bytes); the rate over the bytes
    # the tables name (the prefix once per sequence) is kept under its own name, for the record.
    logical_gbps = result.pop("attention_gbps")
    result.pop("attention_frac_of_peak")
    result.update({
        "cow_pairs": len(step.host_pairs),
        # the workload's copies all read one shared source block: a time, not an HBM rate
        "cow_shared_source_us": round(cow_ms * 1e3, 2),
        "unique_context_bytes": unique,
        "attention_gbps": round(unique_rate, 1),
        "attention_frac_of_peak": round(unique_rate / HBM_PEAK_GBPS, 4),
        "attention_table_bytes_gbps": logical_gbps,
        "note": "attention_gbps / attention_frac_of_peak count each distinct K/V block once "
        "(unique_context_bytes); attention_table_bytes_gbps counts the shared prefix once per "
        "sequence, which the caches serve, and is not an HBM rate. cow_shared_source_us times the "
        "workload's 256 copies of one shared source block (cache-served after its first read); "
        "cow_distinct_sources_* is the same launch over 256 distinct random sources, the copy's "
        "HBM rate",
    })  # fmt: skip
    return result


TRACES = ROOT / "tests" / "golden" / "traces"


def config1(args) -> dict:
    """Config 1 end to end: the reference engine's recorded run (scheduler decisions, KV-cache
    calls, batches; tests/golden/traces/config1.json) replayed through this package's
    KVCacheManager and the GPU ModelRunner, sampling greedily on the device. The timed run is
    the whole replay: allocator calls, 42 iterations of the 2-layer model, one int32 per sampled
    row back to the host."""
    import torch

    from paged_kv_serving_amd.replay import Trace, TraceReplay
    from paged_kv_serving_amd.runner import ModelRunner

    trace = Trace.load(TRACES / "config1.json")
    model = trace.language_model()
    device = torch.device("cuda", 0)

    def one_run(check: bool):
        runner = ModelRunner(model, num_blocks=trace.engine["num_blocks"], block_size=trace.engine["block_size"],
                             device=device)  # fmt: skip
        result = TraceReplay(trace, runner, check=check, greedy=True).run()
        torch.cuda.synchronize(device)
        return result

    checked = one_run(True)  # bit-exact tables, slots and allocator state; warms the kernels
    for _ in range(max(0, args.warmup // 5 - 1)):
        one_run(False)
    runs = max(1, args.steps // 10)
    seconds = []
    for _ in range(runs):
        start = time.perf_counter()
        result = one_run(False)
        seconds.append(time.perf_counter() - start)
    elapsed = float(np.median(seconds))
    generated = len(result.greedy)
    agree = sum(int(tok == trace.tokens[sid][ctx]) for tok, (sid, ctx) in zip(checked.greedy, checked.row_seqs))
    return {
        "metric": "engine output tokens/s, continuous batching + chunked prefill (config 1)",
        "value": round(generated / elapsed, 1),
        "unit": "output tokens/s",
        "n_gpus": 1,
        "steps": result.iterations,
        "warmup": max(1, args.warmup // 5),
        "ms_per_step": round(elapsed * 1e3 / result.iterations, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: random_weights(seed 0), 32 prompts U[16,128] random tokens (seed 0), "
        "the reference engine's recorded schedule",
        "config": {
            "workload": "config1: fp32 decoder vocab 256, d_model 128, 2 layers, 4 heads x 32, d_ff "
            "320; 32 requests, 32 greedy tokens each; EngineConfig defaults (block 16, 512 blocks, "
            "budget 256, 32 running)",
            "runs": runs,
        },
        "seconds_per_run": round(elapsed, 4),
        "generated_tokens": generated,
        "greedy_tokens_equal_reference": f"{agree}/{len(checked.greedy)}",
        "reference_published": "1453.36 output tok/s (engine_throughput_24_requests, i5-8500, "
        "bench/results/latest.json:46-53; a different workload, for orientation only)",
    }


#: What each other configuration contributes to the default run's ``other_configs`` object.
OTHER_FIELDS = {
    3: ("attention_ms", "attention_gbps", "attention_frac_of_peak", "prefill_gflop", "prefill_tiles_alone_ms",
        "prefill_tiles_alone_tflops", "prefill_tiles_alone_frac_of_fp32_mfma_peak", "append_us", "append_gbps",
        "rope_append_us", "rope_append_gbps", "runner_step_ms", "runner_step_over_kernel"),
    4: ("cow_shared_source_us", "cow_distinct_sources_us", "cow_distinct_sources_gbps",
        "cow_distinct_sources_frac_of_peak", "attention_ms", "attention_gbps", "attention_frac_of_peak",
        "unique_context_bytes", "runner_step_ms", "runner_step_over_kernel"),
    5: ("attention_ms", "attention_gbps", "attention_frac_of_peak", "attention_tokens_per_s"),
    1: ("value", "unit", "ms_per_step", "seconds_per_run", "generated_tokens", "greedy_tokens_equal_reference"),
}  # fmt: skip


def other_configs(args) -> dict:
    """BASELINE.json's other configurations (configs[0], [2], [3], [4]: config 1 end to end,
    configs 3, 4 and 5 of one layer), each timed in this process after the headline with up to
    20 steps, so the default run's line carries them: the fields of ``OTHER_FIELDS`` from each
    config's own line (``bench.py --config N`` prints all of it), its roofline fraction, and the
    wall time the config took here."""
    import torch

    sub = argparse.Namespace(**{**vars(args), "steps": min(args.steps, 20), "warmup": min(args.warmup, 5),
                                "partition": 0, "kv": "f32"})  # fmt: skip
    runners = {3: config3, 4: config4, 5: config5, 1: config1}
    out = {}
    for number, run in runners.items():
        start = time.perf_counter()
        line = run(sub)
        picked = {key: line[key] for key in OTHER_FIELDS[number] if key in line}
        if "roofline" in line:
            picked["roofline_frac"] = line["roofline"]["frac"]
        picked["workload"] = line["config"]["workload"]
        picked["wall_s"] = round(time.perf_counter() - start, 2)
        out[f"config{number}"] = picked
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return out


def _host_timed(function, runs: int, warmup: int = 5) -> dict:
    """p50/p95 microseconds of host wall time per call, ``perf_counter_ns`` around each call
    after ``warmup`` calls: the reference's timing method (bench/bench_baseline.py:70-83)."""
    for _ in range(warmup):
        function()
    samples = []
    for _ in range(runs):
        start = time.perf_counter_ns()
        function()
        samples.append(time.perf_counter_ns() - start)
    micros = np.asarray(samples, dtype=np.float64) / 1e3
    return {"runs": runs, "p50_us": round(float(np.percentile(micros, 50)), 1),
            "p95_us": round(float(np.percentile(micros, 95)), 1)}  # fmt: skip


def micro(args) -> dict:
    """The reference's published benchmarks of this path (bench/bench_baseline.py: the paged
    decode, the copy-on-write cycle, the two correctness gaps, and the 128-token iteration of the
    runner), at their own shapes and with their own timing method, run on this build. The
    published figures are bench/results/latest.json (an i5-8500, 1 BLAS thread). Calls that
    return a result the caller can read include the synchronisation that makes it readable."""
    import torch

    from paged_kv_serving_amd import ops
    from paged_kv_serving_amd.attention import paged_attention
    from paged_kv_serving_amd.blocks import BlockManager, RecordingBlockStore
    from paged_kv_serving_amd.equivalence import max_logit_gap, rows_logit_gap
    from paged_kv_serving_amd.replay import Trace, TraceReplay
    from paged_kv_serving_amd.runner import BatchEntry, ExecutionBatch, ModelRunner

    device = torch.device("cuda", 0)
    out: dict = {}

    # paged_attention_decode_256ctx (bench_baseline.py:122-136): 1 query, 4 heads x 32, 16 blocks.
    rng = np.random.default_rng(0)
    heads, dim, block_size, blocks = 4, 32, 16, 16
    keys = rng.standard_normal((blocks, block_size, heads, dim)).astype(np.float32)
    values = rng.standard_normal((blocks, block_size, heads, dim)).astype(np.float32)
    query = rng.standard_normal((1, heads, dim)).astype(np.float32)
    positions = np.asarray([blocks * block_size - 1], dtype=np.int64)
    table = np.arange(blocks, dtype=np.int64)
    context, scale = blocks * block_size, dim**-0.5
    host_call = lambda: paged_attention(query, positions, keys, values, table, context, scale)  # noqa: E731
    d_keys, d_values, d_query, d_pos, d_table = (
        torch.from_numpy(a).to(device) for a in (keys, values, query, positions, table)
    )

    def resident_call():
        paged_attention(d_query, d_pos, d_keys, d_values, d_table, context, scale)
        torch.cuda.synchronize(device)

    q32, seq32 = d_query.contiguous(), torch.zeros(1, dtype=torch.int32, device=device)
    pos32, table32 = d_pos.to(torch.int32), d_table.to(torch.int32).reshape(1, -1).contiguous()
    ctx32 = torch.tensor([context], dtype=torch.int32, device=device)
    result_buffer = torch.empty_like(q32)
    kernel_call = lambda: ops.paged_attention_ragged(  # noqa: E731
        q32, pos32, seq32, d_keys, d_values, table32, ctx32, scale, max_context_len=context,
        out=result_buffer)  # fmt: skip
    for _ in range(10):
        kernel_call()
    torch.cuda.synchronize(device)
    out["paged_attention_decode_256ctx"] = {
        "reference_p50_us": 129.4, "reference_p95_us": 171.9,
        "host_arrays": _host_timed(host_call, 2000),
        "device_resident": _host_timed(resident_call, 2000),
        "gpu_us_per_call": round(timed(kernel_call, 200, torch.cuda.current_stream(device)) * 1e3, 2),
        "what": "host_arrays: the drop-in call on NumPy arrays (K/V copied in, output copied "
        "back); device_resident: device tensors in and out, synchronised; gpu_us_per_call: HIP "
        "events around back-to-back ragged calls",
    }  # fmt: skip

    # copy_on_write_block (bench_baseline.py:97-110): host bookkeeping of one COW cycle.
    manager = BlockManager(num_blocks=4096, block_size=16, store=RecordingBlockStore())

    def cow_cycle(blocks_manager):
        block = blocks_manager.allocate()
        blocks_manager.incref(block)
        blocks_manager.incref(block)
        private = blocks_manager.prepare_for_write(block)
        blocks_manager.free(private)
        blocks_manager.free(block)
        blocks_manager.free(block)

    out["copy_on_write_block"] = {"reference_p50_us": 1.8, "reference_p95_us": 2.0,
                                  **_host_timed(lambda: cow_cycle(manager), 5000)}  # fmt: skip

    # The reference benchmarks' model: build_random_checkpoint(seed 3, max_seq_len 512), i.e.
    # random_weights(seed 3) of a 4-layer d_model-128 vocab-512 decoder; the engine-equivalence
    # trace holds the SHA-256 of the reference's weights, which language_model() checks.
    trace = Trace.load(TRACES / "engine_equivalence.json")
    model = trace.language_model()

    # The same COW cycle with the bytes moved: the block store is a ModelRunner (4 layers,
    # 4 heads x 32, block 16: 32 KiB per block and layer for K+V), flushed and synchronised.
    store = ModelRunner(model, num_blocks=4096, block_size=16, device=device)
    moving = BlockManager(num_blocks=4096, block_size=16, store=store)

    def cow_with_copy():
        cow_cycle(moving)
        store.flush_copies()
        torch.cuda.synchronize(device)

    out["copy_on_write_block"]["with_device_copy"] = _host_timed(cow_with_copy, 2000)

    # engine_iteration_128_tokens (bench_baseline.py:163-186): 16 decode rows + a 112-token
    # prefill through the 4-layer model: one ModelRunner.execute, logits back on the host.
    runner = ModelRunner(model, num_blocks=256, block_size=16, device=device)
    entries = [BatchEntry(seq_id=f"decode-{i}", token_ids=(1,), positions=(63,),
                          block_table=tuple(range(i * 4, i * 4 + 4)), logits_index=0)
               for i in range(16)]  # fmt: skip
    entries.append(BatchEntry(seq_id="prefill", token_ids=tuple(range(1, 113)),
                              positions=tuple(range(112)), block_table=tuple(range(128, 135)),
                              logits_index=111))  # fmt: skip
    batch = ExecutionBatch(tuple(entries))
    out["engine_iteration_128_tokens"] = {"reference_p50_us": 12330.9, "reference_p95_us": 13426.5,
                                          **_host_timed(lambda: runner.execute(batch), 20, warmup=3)}  # fmt: skip

    # paged_vs_reference_equivalence (bench_baseline.py:217-238): 4 prompts from default_rng(5),
    # each through the paged runner whole, token by token, in 7/5/13/rest chunks and over a
    # reversed block table, against one dense pass (float32 torch on the device).
    draw = np.random.default_rng(5)
    vocab = min(model.config.vocab_size, 256)
    worst = 0.0
    for _ in range(4):
        length = int(draw.integers(20, 120))
        tokens = [int(v) for v in draw.integers(1, vocab, length)]
        for chunks in ([length], [1] * length, [7, 5, 13, length - 25]):
            if any(size < 1 for size in chunks):
                continue
            worst = max(worst, max_logit_gap(model, tokens, device=device, block_size=16, chunks=chunks))
        blocks_needed = -(-length // 16)
        worst = max(worst, max_logit_gap(model, tokens, device=device, block_size=16,
                                         block_order=list(reversed(range(blocks_needed)))))  # fmt: skip
    out["paged_vs_reference_equivalence"] = {"runs": 4, "max_abs_logit_gap": float(f"{worst:.4g}"),
                                             "reference_max_abs_logit_gap": 2.444e-06}  # fmt: skip

    # engine_vs_reference_equivalence (bench_baseline.py:241-284): the reference engine's run
    # over a 20-block pool (preemption, prefix hits, forked samples), replayed through this
    # package's KV-cache manager and the GPU runner; every sampled row against the dense pass.
    replay_runner = ModelRunner(model, num_blocks=trace.engine["num_blocks"], block_size=16, device=device)
    replayed = TraceReplay(trace, replay_runner).run()
    gap, rows_checked = rows_logit_gap(model, replayed.rows, replayed.row_seqs, trace.tokens, device)
    out["engine_vs_reference_equivalence"] = {
        "runs": 1, "max_abs_logit_gap": float(f"{gap:.4g}"), "rows_checked": float(rows_checked),
        "preemptions": float(trace.summary["preemptions"]), "prefix_hit_blocks": float(trace.summary["prefix_hit_blocks"]),
        "cow_copies": replayed.copies,
        "max_abs_gap_to_reference_rows": float(f"{float(np.max(np.abs(np.stack(replayed.rows) - trace.logits))):.4g}"),
        "reference_max_abs_logit_gap": 3.248e-06,
    }  # fmt: skip

    latency = out["paged_attention_decode_256ctx"]["device_resident"]["p50_us"]
    return {
        "metric": "reference micro-benchmarks of the path (bench/bench_baseline.py) at their own "
        "shapes: paged_attention_decode_256ctx p50 latency, device-resident",
        "value": latency,
        "unit": "us",
        "n_gpus": 1,
        "steps": 2000,
        "warmup": 5,
        "ms_per_step": round(latency / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(latency / 129.4, 4),  # the published p50 of the same benchmark
        "dtype": "f32",
        "data": "synthetic: the reference benchmarks' own seeded inputs and random-init weights",
        "config": {"workload": "reference benchmarks of the path: decode 256 ctx (1 query, 4 heads "
                   "x 32, 16 blocks), COW cycle, 128-token iteration, paged-vs-dense and "
                   "engine-vs-dense logit gaps on a 4-layer d_model-128 vocab-512 model"},  # fmt: skip
        "micro": out,
    }


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU: --gpus {args.gpus} is not supported (this build has no "
            "multi-GPU path; the data path shards by heads with no exchange, which one GPU's "
            "share at its real shape already measures)",
            file=sys.stderr,
        )
        return 2
    import torch

    if args.micro:
        torch.cuda.set_device(0)
        print(json.dumps(micro(args)), flush=True)
        return 0
    torch.cuda.set_device(0)
    runners = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}
    result = runners[args.config](args)
    if args.config == 2:
        # The known-size dispatch that calibrates the rocprofv3 FETCH_SIZE/WRITE_SIZE counters.
        peak = copy_peak(torch.device("cuda", 0))
        result["copy_peak_gbps"] = peak["copy_peak_gbps"]
        if not args.no_others:
            result["other_configs"] = other_configs(args)
        if not args.no_cpu:
            result["cpu_baseline"] = cpu_baseline(args)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
