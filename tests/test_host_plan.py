"""Host-side batch planning: the row/tile split and the per-batch partition and load hints.

Both run on the CPU before a ragged attention call (the library only needs to load for
``pkv_tile_head_dim_supported``). The split must put every query row in exactly one pass; the
hints only pick launch parameters, so the GPU tests check that every choice gives the same rows.
"""

from __future__ import annotations

import numpy as np
import pytest

from paged_kv_serving_amd import ops


def _check_split(seq: np.ndarray, rows: np.ndarray, tiles: np.ndarray, min_rows: int) -> None:
    covered = list(rows.tolist())
    for first, count in tiles.tolist():
        assert 1 <= count <= ops.TILE_ROWS
        assert len(set(seq[first : first + count].tolist())) == 1, "a tile spans one sequence"
        covered += range(first, first + count)
    assert sorted(covered) == list(range(seq.size)), "every row in exactly one pass"
    # a row left to the row pass belongs to a run shorter than min_rows
    starts = np.flatnonzero(np.concatenate([[True], seq[1:] != seq[:-1]]))
    lengths = np.diff(np.concatenate([starts, [seq.size]]))
    run_len = np.repeat(lengths, lengths)
    assert np.all(run_len[rows] < min_rows)


@pytest.mark.parametrize("seed", range(6))
def test_every_row_goes_to_exactly_one_pass(seed) -> None:
    rng = np.random.default_rng(seed)
    runs = rng.integers(1, 150, int(rng.integers(1, 30)))
    seq = np.repeat(np.arange(runs.size), runs).astype(np.int32)
    for min_rows in (2, ops.MIN_TILE_ROWS, 65):
        rows, tiles = ops.plan_rows(seq, 128, min_tile_rows=min_rows)
        _check_split(seq, rows, tiles, min_rows)


def test_known_splits() -> None:
    seq = np.array([0] * 130 + [1] + [2] * 8 + [3] * 7, np.int32)
    rows, tiles = ops.plan_rows(seq, 64)
    assert tiles.tolist() == [[0, 64], [64, 64], [128, 2], [131, 8]]
    assert rows.tolist() == [130, *range(139, 146)]
    # head dims without a tile kernel keep everything in the row pass
    rows, tiles = ops.plan_rows(seq, 8)
    assert tiles.shape == (0, 2) and rows.tolist() == list(range(146))
    rows, tiles = ops.plan_rows(np.zeros(0, np.int32), 128)
    assert rows.size == 0 and tiles.shape == (0, 2)


def _tables(contexts, block_size, rng, shared_prefix=0):
    pool = rng.permutation(200_000)
    prefix = pool[:shared_prefix].tolist()
    out, used = [], shared_prefix
    for c in contexts:
        need = -(-int(c) // block_size) - shared_prefix
        out.append(np.asarray(prefix + pool[used : used + need].tolist()))
        used += need
    return out


def test_partition_hint_follows_the_work_per_partition() -> None:
    rng = np.random.default_rng(0)
    decode = rng.integers(512, 4097, 64)  # 64 x U[512, 4096] decode, 32 heads
    assert ops.batch_hints(_tables(decode, 16, rng), decode, 32, 16) == (512, False)
    long = np.full(16, 32768)  # 16 x 32k decode, 32 heads: 16 x 32 x 32 work items
    assert ops.batch_hints(_tables(long, 16, rng), long, 32, 16) == (1024, False)
    # the same contexts with 8 query rows per sequence cross the threshold
    assert ops.batch_hints(_tables(decode, 16, rng), decode, 8, 16, num_rows=8 * 64)[0] == 1024
    assert ops.batch_hints([], np.zeros(0), 32, 16) == (0, False)


def test_shared_hint_counts_repeated_block_ids() -> None:
    rng = np.random.default_rng(1)
    contexts = np.full(256, 1116)  # 64 shared prefix blocks + 6 private ones each
    assert ops.batch_hints(_tables(contexts, 16, rng, shared_prefix=64), contexts, 32, 16)[1]
    small = np.full(256, 16 * 70)
    # one shared block out of 70 per table is below the threshold
    assert not ops.batch_hints(_tables(small, 16, rng, shared_prefix=1), small, 32, 16)[1]
    # entries past a sequence's context are padding and never count
    tables = [np.concatenate([[i], np.full(10, 5)]) for i in range(100)]
    assert not ops.batch_hints(tables, np.full(100, 16), 32, 16)[1]
