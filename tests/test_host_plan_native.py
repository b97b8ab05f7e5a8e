"""The library's host planner (pkv_plan_batch, C++) against the Python planner it replaces in the
runner (ops.plan_batch), on the CPU: the same rows, tiles, merge list, partition size and flags,
bit for bit, over seeded random batches that mix decode rows, prefill runs of every length,
shared prefixes (with members whose tables end inside the prefix), positions that hide part of
the context, block sizes 1-32, head dims with and without a tile kernel, given or chosen
partition sizes, and float32 or bfloat16 pools."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from paged_kv_serving_amd import _native, ops


def _same(a: ops.BatchPlan, b: ops.BatchPlan) -> None:
    assert np.array_equal(np.asarray(a.rows, np.int32).reshape(-1, 2), b.rows), "rows"
    assert np.array_equal(np.asarray(a.tiles, np.int32).reshape(-1, 4), b.tiles), "tiles"
    assert np.array_equal(np.asarray(a.merge, np.int32), b.merge), "merge"
    assert (a.partition_size, a.shared_kv, a.short_rows, a.dominant_tiles) == (
        b.partition_size, b.shared_kv, b.short_rows, b.dominant_tiles
    )


def random_batch(seed: int):
    rng = np.random.default_rng(seed)
    block = int(rng.choice([1, 2, 4, 8, 16, 32]))
    heads = int(rng.choice([1, 2, 8, 32]))
    dim = int(rng.choice([8, 32, 64, 128, 256]))
    pool = rng.permutation(1 << 20)
    used = 0
    tables, contexts, seq, positions = [], [], [], []
    stems = []
    for _ in range(int(rng.integers(0, 3))):
        n = int(rng.integers(1, 2048 // block + 2))
        stems.append(pool[used : used + n].tolist())
        used += n
    num_seqs = int(rng.integers(1, 160))
    # Sometimes a run of consecutive decode sequences shares one long stem (a prefix group),
    # with a few members whose whole table ends inside it.
    run_start, run_stem = -1, None
    if rng.random() < 0.4:
        run_stem = pool[used : used + int(rng.integers(600, 2500)) // block + 1].tolist()
        used += len(run_stem)
        run_start = int(rng.integers(0, num_seqs))
        num_seqs = max(num_seqs, run_start + int(rng.integers(16, 140)))
    for s in range(num_seqs):
        kind = rng.random()
        ctx = int(rng.integers(1, 3000))
        need = -(-ctx // block)
        table = []
        in_run = run_stem is not None and s >= run_start
        if in_run:
            kind = 1.0
            ctx = len(run_stem) * block + int(rng.integers(1, 400)) if rng.random() > 0.05 else int(rng.integers(1, 200))
            need = -(-ctx // block)
            table = run_stem[: min(len(run_stem), need)]
        elif stems and rng.random() < 0.6:
            stem = stems[int(rng.integers(0, len(stems)))]
            table = stem[: min(len(stem), need)]
        table = table + pool[used : used + need - len(table)].tolist()
        used += need
        tables.append(table)
        contexts.append(ctx)
        if kind < 0.2 and not in_run:  # a prefill run ending at the context
            run = int(rng.integers(1, min(ctx, 300) + 1))
            rows_pos = list(range(ctx - run, ctx))
        else:  # a decode row (sometimes at an earlier position)
            rows_pos = [ctx - 1 if rng.random() < 0.9 else int(rng.integers(-1, ctx))]
        seq += [s] * len(rows_pos)
        positions += rows_pos
    width = max(len(t) for t in tables) + int(rng.integers(0, 4))
    arena = np.full((num_seqs, width), -7, np.int32)
    for i, t in enumerate(tables):
        arena[i, : len(t)] = t
    partition = int(rng.choice([0, 0, 0, 64, 256, 512, 1024]))
    return dict(query_seq=np.asarray(seq, np.int64), head_dim=dim, num_heads=heads, tables=arena,
                context_lens=np.asarray(contexts, np.int64), block_size=block, partition_size=partition,
                query_positions=np.asarray(positions, np.int64))  # fmt: skip


@pytest.mark.parametrize("seed", range(300))
def test_the_native_planner_matches_the_python_planner(seed) -> None:
    case = random_batch(seed)
    kv = torch.bfloat16 if seed % 2 else torch.float32
    want = ops.plan_batch(
        case["query_seq"], case["head_dim"], case["num_heads"], case["tables"], case["context_lens"],
        case["block_size"], partition_size=case["partition_size"], query_positions=case["query_positions"],
        kv_dtype=kv,
    )  # fmt: skip
    got = ops.plan_batch_native(
        case["query_seq"], case["head_dim"], case["num_heads"], case["tables"], case["context_lens"],
        case["block_size"], partition_size=case["partition_size"], query_positions=case["query_positions"],
        kv_dtype=kv,
    )  # fmt: skip
    _same(want, got)


def _tables(contexts, block, rng, shared=0):
    pool = rng.permutation(200_000)
    prefix = pool[:shared].tolist()
    out, used = [], shared
    for c in contexts:
        need = -(-int(c) // block) - shared
        out.append(np.asarray(prefix + pool[used : used + need].tolist()))
        used += need
    return out


@pytest.mark.parametrize("rows", [16, 63, 64, 65, 200, 256])
def test_shared_prefix_batches_plan_the_same(rows) -> None:
    rng = np.random.default_rng(rows)
    contexts = 1016 + rng.integers(32, 257, rows) + 1
    tables = _tables(contexts, 16, rng, shared=63)
    contexts[rows // 2] = 16  # a member whose table ends inside the prefix
    tables[rows // 2] = tables[rows // 2][:1]
    seq = np.arange(rows)
    args = (seq, 128, 32, tables, contexts, 16)
    _same(ops.plan_batch(*args, query_positions=contexts - 1), ops.plan_batch_native(*args, query_positions=contexts - 1))
    _same(ops.plan_batch(*args), ops.plan_batch_native(*args))


def test_whole_tile_batches_plan_the_same() -> None:
    """Config 3's shape: 8 x 512-token prefill chunks and 120 decode rows."""
    rng = np.random.default_rng(3)
    offsets = rng.integers(0, 2049, 8)
    decode = rng.integers(256, 4097, 120)
    contexts = np.concatenate([offsets + 512, decode])
    tables = _tables(contexts, 16, rng)
    positions = np.concatenate([np.arange(o, o + 512) for o in offsets] + [decode - 1])
    seq = np.concatenate([np.full(512, i) for i in range(8)] + [np.arange(8, 128)])
    want = ops.plan_batch(seq, 128, 32, tables, contexts, 16, query_positions=positions)
    assert np.any(want.tiles[:, 3] == ops.TILE_WHOLE)
    _same(want, ops.plan_batch_native(seq, 128, 32, tables, contexts, 16, query_positions=positions))
    # the chunks alone (no row-pass rows: longest tile first)
    alone = ops.plan_batch(seq[:4096], 128, 32, tables, contexts, 16, query_positions=positions[:4096])
    assert alone.rows.shape[0] == 0 and np.all(alone.tiles[:, 3] == ops.TILE_WHOLE)
    _same(alone, ops.plan_batch_native(seq[:4096], 128, 32, tables, contexts, 16,
                                       query_positions=positions[:4096]))  # fmt: skip


def test_small_buffers_grow_and_bad_arguments_are_refused() -> None:
    planner = ops.NativePlanner()
    planner._rows = np.zeros((1, 2), np.int32)  # far too small: the planner must grow it
    rng = np.random.default_rng(1)
    contexts = rng.integers(512, 4097, 64)
    tables = ops.plan_batch_native.__globals__["np"].zeros((64, 256), np.int32)
    for i, t in enumerate(_tables(contexts, 16, rng)):
        tables[i, : len(t)] = t
    plan = planner.plan(np.arange(64), 128, 32, tables, contexts, 16)
    _same(ops.plan_batch(np.arange(64), 128, 32, tables, contexts, 16), plan)
    lib = _native.library()
    counts, launch = np.zeros(3, np.int64), np.zeros(2, np.int32)
    seq = np.asarray([0, 5], np.int32)  # sequence 5 does not exist
    ctx = np.asarray([10], np.int32)
    assert lib.pkv_plan_batch(seq.ctypes.data, None, 2, tables.ctypes.data, 256, ctx.ctypes.data, 1, 16, 32, 128,
                              0, 0, 8, None, 0, None, 0, None, 0, counts.ctypes.data, launch.ctypes.data) == -1  # fmt: skip
    seq = np.asarray([0], np.int32)
    assert lib.pkv_plan_batch(seq.ctypes.data, None, 1, tables.ctypes.data, 256, ctx.ctypes.data, 1, 16, 32, 128,
                              7, 0, 8, None, 0, None, 0, None, 0, counts.ctypes.data, launch.ctypes.data) == -1  # fmt: skip
