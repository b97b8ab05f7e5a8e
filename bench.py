"""Benchmark of the KV-cache data path on one MI355X (BASELINE.json ``metric``).

Workload ("config 2"): one decode step of one layer for 64 sequences
with contexts uniform in [512, 4096], 32 heads x head_dim 128 (MHA), block_size 16, float32 K/V,
block tables drawn from a shuffled 20,000-block pool; seeded N(0, 1) data resident in HBM.
A step is the data path of that iteration:

    pkv_append           the 64 new tokens' keys and values into their slots
    pkv_paged_attention  64 decode queries over their block tables (partial + reduce passes)

``value`` is decode tokens per second (64 tokens per step). The roofline object is for the
dominant kernel, the attention pass: achieved = algorithmic bytes per launch (each sequence's
K+V context read once, plus queries, outputs and block tables) / its mean duration, measured
with HIP events on the launching stream over the timed steps. The CPU baseline times the
oracle's NumPy restatement of the reference path (reference attention.py:42-121 per sequence,
tile_blocks 8, plus the runner.py:195-196 append) on a bounded sample of the same workload,
single-threaded BLAS as the reference pins it.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--partition P] [--no-cpu]
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
METRIC = "paged-attn decode tokens/s & HBM GB/s (% of peak) at 64 seq x 4k ctx; append GB/s"


def parse() -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--partition", type=int, default=0, help="keys per partition (0: default)")
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    parser.add_argument("--cpu-seqs", type=int, default=64, help="sequences in the CPU sample")
    parser.add_argument("--cpu-repeats", type=int, default=5, help="timed CPU steps (median)")
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

    with threadpool_limits(1) if threadpool_limits else nullcontext():
        step()  # warmup
        samples = []
        for _ in range(args.cpu_repeats):
            start = time.perf_counter_ns()
            step()
            samples.append((time.perf_counter_ns() - start) / 1e9)
    seconds = float(np.median(samples))
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
        "host_cpus": os.cpu_count(),
    }


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU: --gpus {args.gpus} is not supported (this build has no "
            "multi-GPU path; see DESIGN.md for how the data path would shard)",
            file=sys.stderr,
        )
        return 2
    import torch

    from paged_kv_serving_amd import ops
    from paged_kv_serving_amd.workloads import decode_batch

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    batch = decode_batch(seed=args.seed, device=device)
    workspace_bytes = ops.attention_workspace_bytes(
        batch.num_queries, 32, 128, batch.max_context_len, args.partition
    )
    workspace = torch.empty(max(workspace_bytes // 4, 1), dtype=torch.float32, device=device)
    out = torch.empty_like(batch.queries)

    def append() -> None:
        ops.append_kv(batch.key_cache, batch.value_cache, batch.new_keys, batch.new_values, batch.slot_mapping)

    def attend() -> None:
        ops.paged_attention_ragged(
            batch.queries, batch.query_positions, batch.query_seq, batch.key_cache,
            batch.value_cache, batch.block_tables, batch.context_lens, batch.scale,
            max_context_len=batch.max_context_len, partition_size=args.partition,
            out=out, workspace=workspace,
        )  # fmt: skip

    for _ in range(args.warmup):
        append()
        attend()
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(device)
    marks = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    start = time.perf_counter()
    for e0, e1, e2 in marks:
        e0.record(stream)
        append()
        e1.record(stream)
        attend()
        e2.record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start

    append_ms = float(np.mean([e0.elapsed_time(e1) for e0, e1, _ in marks]))
    attention_ms = float(np.mean([e1.elapsed_time(e2) for _, e1, e2 in marks]))
    tokens = batch.num_queries
    heads, dim = 32, 128
    kv_bytes = batch.context_bytes()
    io_bytes = 2 * tokens * heads * dim * 4 + batch.block_tables.numel() * 4 + 3 * tokens * 4
    attention_bytes = kv_bytes + io_bytes
    append_bytes = 2 * tokens * heads * dim * 4 * 2 + tokens * 8  # read k, v + write k, v + slots
    achieved = attention_bytes / (attention_ms * 1e-3) / 1e9
    append_gbps = append_bytes / (append_ms * 1e-3) / 1e9
    ms_per_step = elapsed * 1e3 / args.steps
    result = {
        "metric": METRIC,
        "value": round(tokens * args.steps / elapsed, 1),
        "unit": "decode tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded N(0,1) K/V pools, queries and new tokens resident in HBM",
        "config": {
            "workload": "config2 decode: 64 seqs, ctx U[512,4096] (seed 0), 32 heads x 128 MHA, "
            "block 16, fp32 KV, 20000-block shuffled pool, 1 layer; step = append 64 tokens + "
            "paged attention",
            "partition_size": args.partition or 512,
            "context_tokens": int(batch.host_context.sum()),
        },
        "attention_ms": round(attention_ms, 4),
        "attention_gbps": round(achieved, 1),
        "attention_frac_of_peak": round(achieved / HBM_PEAK_GBPS, 4),
        "attention_tokens_per_s": round(tokens / (attention_ms * 1e-3), 1),
        "append_us": round(append_ms * 1e3, 2),
        "append_gbps": round(append_gbps, 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic_from_profiles(),
            "kernel": "attention_partial_kernel<float,128> + attention_reduce_kernel<128>",
            "algorithmic_bytes_per_launch": attention_bytes,
        },
    }
    peak = copy_peak(device)
    result["copy_peak_gbps"] = peak["copy_peak_gbps"]
    result["attention_frac_of_copy_peak"] = round(achieved / peak["copy_peak_gbps"], 4)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(args)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
