"""Host-side batch planning: the row/tile split and the per-batch partition and load hints.

Both run on the CPU before a ragged attention call (the library only needs to load for
``pkv_tile_head_dim_supported``). The split must put every query row in exactly one pass; the
hints only pick launch parameters, so the GPU tests check that every choice gives the same rows.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from paged_kv_serving_amd import ops


def _check_split(seq: np.ndarray, rows: np.ndarray, tiles: np.ndarray, min_rows: int) -> None:
    assert rows.shape[1] == 2 and tiles.shape[1] == 4
    assert np.all(rows[:, 1] == 0) and np.all(tiles[:, 2:] == 0), "no shared-prefix split here"
    covered = list(rows[:, 0].tolist())
    for first, count, _, _ in tiles.tolist():
        assert 1 <= count <= ops.TILE_ROWS
        assert len(set(seq[first : first + count].tolist())) == 1, "a tile spans one sequence"
        covered += range(first, first + count)
    assert sorted(covered) == list(range(seq.size)), "every row in exactly one pass"
    # a row left to the row pass belongs to a run shorter than min_rows
    starts = np.flatnonzero(np.concatenate([[True], seq[1:] != seq[:-1]]))
    lengths = np.diff(np.concatenate([starts, [seq.size]]))
    run_len = np.repeat(lengths, lengths)
    assert np.all(run_len[rows[:, 0]] < min_rows)


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
    assert tiles.tolist() == [[0, 64, 0, 0], [64, 64, 0, 0], [128, 2, 0, 0], [131, 8, 0, 0]]
    assert rows[:, 0].tolist() == [130, *range(139, 146)]
    # head dims without a tile kernel keep everything in the row pass
    rows, tiles = ops.plan_rows(seq, 8)
    assert tiles.shape == (0, 4) and rows[:, 0].tolist() == list(range(146))
    rows, tiles = ops.plan_rows(np.zeros(0, np.int32), 128)
    assert rows.shape == (0, 2) and tiles.shape == (0, 4)


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


# --- shared prefixes -----------------------------------------------------------------------------


def _covered(plan, seq, contexts, block_size):
    """(row, partition) pairs each pass computes; every visible partition exactly once."""
    P = plan.partition_size
    seen = {}
    for first, count, pb, pe in plan.tiles.tolist():
        for t in range(first, first + count):
            parts = max(1, -(-int(contexts[seq[t]]) // P))
            for p in range(pb, pe if pe > pb else parts):
                if p < parts:
                    seen[(t, p)] = seen.get((t, p), 0) + 1
    for t, p in plan.rows.tolist():  # row-pass work items
        seen[(t, p)] = seen.get((t, p), 0) + 1
    want = {(t, p) for t in range(seq.size) for p in range(max(1, -(-int(contexts[seq[t]]) // P)))}
    assert set(seen) == want and all(v == 1 for v in seen.values())


def test_a_shared_prefix_becomes_tiles_over_whole_partitions() -> None:
    """256 decode rows sharing 63 leading blocks (1008 tokens, the prefix-sharing workload's
    shape): the prefix goes to four 64-row tiles over three 336-key partitions."""
    rng = np.random.default_rng(3)
    contexts = 1016 + rng.integers(32, 257, 256) + 1
    tables = _tables(contexts, 16, rng, shared_prefix=63)
    seq = np.arange(256)
    plan = ops.plan_batch(seq, 128, 32, tables, contexts, 16)
    assert plan.partition_size == 336
    assert plan.tiles.tolist() == [[64 * i, 64, 0, 3] for i in range(4)]
    assert plan.rows.shape == (256, 2) and np.all(plan.rows[:, 1] == 3), "one suffix item per row"
    assert plan.short_rows, "suffixes of 32-256 keys: the lighter row-pass workgroup"
    assert not plan.shared_kv, "what the row pass still reads is private"
    _covered(plan, seq, contexts, 16)


def test_prefix_groups_split_where_tables_diverge_and_skip_small_groups() -> None:
    rng = np.random.default_rng(4)
    a = _tables(np.full(40, 2000), 16, rng, shared_prefix=100)  # 40 rows share 100 blocks
    b = _tables(np.full(10, 2000), 16, rng, shared_prefix=100)  # only 10: too few to tile
    c = _tables(np.full(30, 900), 16, rng, shared_prefix=40)  # 30 rows share 40 blocks (640 tokens)
    tables = a + b + c
    contexts = np.asarray([2000] * 50 + [900] * 30)
    seq = np.arange(80)
    plan = ops.plan_batch(seq, 128, 8, tables, contexts, 16)
    P = plan.partition_size
    groups = {(f, n, pb, pe) for f, n, pb, pe in plan.tiles.tolist()}
    assert {f for f, _, _, _ in groups} == {0, 50}
    assert all(pe * P <= 100 * 16 for f, _, _, pe in groups if f == 0)
    assert all(pe * P <= 40 * 16 for f, _, _, pe in groups if f == 50)
    starts = {t for t, p in plan.rows.tolist() if p == 0}
    assert set(range(40, 50)) <= starts, "the small group stays in the row pass"
    _covered(plan, seq, contexts, 16)


def test_a_member_whose_table_ends_inside_the_prefix_still_joins() -> None:
    rng = np.random.default_rng(5)
    tables = _tables(np.full(20, 3000), 16, rng, shared_prefix=150)
    contexts = np.full(20, 3000)
    contexts[7] = 700  # its visible keys end inside the shared prefix
    tables[7] = tables[7][:44]
    seq = np.arange(20)
    plan = ops.plan_batch(seq, 64, 4, tables, contexts, 16)
    assert plan.tiles.shape[0] == 1 and plan.tiles[0, 0] == 0 and plan.tiles[0, 1] == 20
    _covered(plan, seq, contexts, 16)


def test_no_tile_starts_at_a_member_whose_table_ends_inside_the_prefix() -> None:
    """80 decode rows share 39 blocks, but row 64 holds only block 0 (context 16). A tile reads
    keys through its first row's table, so row 64 must not start the second 64-row tile: every
    tile's first row has to cover the tile's parts * partition keys."""
    rng = np.random.default_rng(8)
    contexts = np.full(80, 39 * 16 + 40)
    tables = _tables(contexts, 16, rng, shared_prefix=39)
    contexts[64] = 16
    tables[64] = tables[64][:1]
    seq = np.arange(80)
    plan = ops.plan_batch(seq, 128, 32, tables, contexts, 16)
    P = plan.partition_size
    assert plan.tiles.shape[0] >= 1
    for first, count, _, end in plan.tiles.tolist():
        assert end != ops.TILE_WHOLE
        assert len(tables[first]) * 16 >= end * P, f"tile at row {first} reads past its table"
    _covered(plan, seq, contexts, 16)


def test_no_sharing_keeps_the_plain_plan() -> None:
    rng = np.random.default_rng(6)
    contexts = rng.integers(512, 4097, 64)
    tables = _tables(contexts, 16, rng)
    plan = ops.plan_batch(np.arange(64), 128, 32, tables, contexts, 16)
    assert plan.tiles.shape == (0, 4)
    assert (plan.partition_size, plan.shared_kv) == ops.batch_hints(tables, contexts, 32, 16)
    assert not plan.short_rows, "512-key partitions of 512-4096-key contexts are long items"
    _covered(plan, np.arange(64), contexts, 16)


def test_plan_hint_sees_shared_blocks_in_list_and_arena_tables() -> None:
    """A batch of forks (every sequence reads the same 40 blocks, then 5 of its own) keeps the
    cached-load hint in both table forms; distinct first blocks, zero contexts and an empty
    arena give the streaming hint and no prefix tiles."""
    rng = np.random.default_rng(8)
    contexts = np.full(24, 45 * 16)
    tables = _tables(contexts, 16, rng, shared_prefix=40)
    arena = np.zeros((24, 50), np.int32)
    for i, t in enumerate(tables):
        arena[i, : len(t)] = t
    for form in (tables, arena):
        plan = ops.plan_batch(np.arange(24), 128, 8, form, contexts, 16, partition_size=1024)
        assert plan.tiles.shape == (0, 4), "a 640-key prefix fills no 1024-key partition"
        assert plan.shared_kv == ops.batch_hints(tables, contexts, 8, 16)[1] is True
    private = _tables(contexts, 16, rng)
    plan = ops.plan_batch(np.arange(24), 128, 8, private, contexts, 16)
    assert not plan.shared_kv and plan.tiles.shape == (0, 4)
    zero = np.zeros(24, np.int64)
    for form in (private, np.zeros((24, 0), np.int32)):
        plan = ops.plan_batch(np.arange(24), 128, 8, form, zero, 16)
        assert not plan.shared_kv and plan.tiles.shape == (0, 4)


def test_every_public_name_of_ops_exists_and_the_workspace_helper_answers() -> None:
    missing = [name for name in ops.__all__ if not hasattr(ops, name)]
    assert not missing
    assert ops.attention_workspace_bytes(64, 32, 128, 4096, 512) == 64 * 32 * 8 * 130 * 4
    assert ops.attention_workspace_bytes(64, 32, 128, 512, 512) == 0


# --- whole prefill tiles and the merge list ------------------------------------------------------


def _mixed(rng, heads):
    """The mixed workload's shape: 8 chunks of 512 rows at offsets U[0, 2048], then 120 decode
    rows with contexts U[256, 4096]."""
    offsets = rng.integers(0, 2049, 8)
    decode = rng.integers(256, 4097, 120)
    contexts = np.concatenate([offsets + 512, decode])
    positions = np.concatenate([np.arange(o, o + 512) for o in offsets] + [decode - 1])
    seq = np.concatenate([np.full(512, i) for i in range(8)] + [np.arange(8, 128)])
    return seq, positions, contexts, _tables(contexts, 16, rng)


def test_prefill_tiles_become_whole_when_they_fill_the_gpu() -> None:
    rng = np.random.default_rng(7)
    seq, positions, contexts, tables = _mixed(rng, 32)
    plan = ops.plan_batch(seq, 128, 32, tables, contexts, 16, query_positions=positions)
    assert plan.tiles.shape == (64, 4) and 64 * 32 >= ops.WHOLE_TILE_GROUPS
    assert np.all(plan.tiles[:, 2] == 0) and np.all(plan.tiles[:, 3] == ops.TILE_WHOLE)
    # chunk by chunk, longest chunk first; an even-ranked chunk's 8 tiles from its last rows to
    # its first, an odd-ranked chunk's from its first rows to its last
    chunks = [int(seq[f]) for f in plan.tiles[:, 0].tolist()]
    assert [chunks[8 * r] for r in range(8)] == np.argsort(-contexts[:8], kind="stable").tolist()
    for r in range(8):
        firsts = plan.tiles[8 * r : 8 * r + 8, 0].tolist()
        assert len({int(seq[f]) for f in firsts}) == 1
        base = 512 * chunks[8 * r]
        rows_order = [base + 64 * i for i in range(8)]
        assert firsts == (rows_order[::-1] if r % 2 == 0 else rows_order)
    _covered(plan, seq, contexts, 16)
    # only decode rows are merged, and only those spanning more than one partition
    visible = np.minimum(contexts[seq], positions + 1)
    want = [t for t in range(4096, 4216) if visible[t] > plan.partition_size]
    assert plan.merge.tolist() == want
    # with 8 heads the 64 tiles would leave the GPU half empty: they stay split by partition
    plan8 = ops.plan_batch(seq, 128, 8, tables, contexts, 16, query_positions=positions)
    assert np.all(plan8.tiles[:, 3] == 0)
    assert set(range(4096)) <= set(plan8.merge.tolist()) | {
        t for t in range(4096) if visible[t] <= plan8.partition_size
    }


def test_prefill_tiles_without_row_pass_rows_run_longest_first() -> None:
    """The 8 chunks on their own: one workgroup per item, so the longest tile comes first."""
    rng = np.random.default_rng(7)
    seq, positions, contexts, tables = _mixed(rng, 32)
    seq, positions = seq[:4096], positions[:4096]
    plan = ops.plan_batch(seq, 128, 32, tables, contexts, 16, query_positions=positions)
    assert plan.tiles.shape == (64, 4) and plan.rows.shape[0] == 0
    assert np.all(plan.tiles[:, 2] == 0) and np.all(plan.tiles[:, 3] == ops.TILE_WHOLE)
    # tile i of chunk c holds positions o_c + 64 i .. o_c + 64 i + 63: its last row sees
    # o_c + 64 (i + 1) keys; ties keep row order (chunk, then tile)
    offsets = contexts[:8] - 512
    keyed = sorted((-(int(offsets[c]) + 64 * (i + 1)), c, i) for c in range(8) for i in range(8))
    assert plan.tiles[:, 0].tolist() == [512 * c + 64 * i for _, c, i in keyed]
    assert plan.tiles[:, 1].tolist() == [64] * 64
    _covered(plan, seq, contexts, 16)
    assert plan.merge.size == 0


@pytest.mark.parametrize(
    ("decode", "kv", "dominant"),
    [(120, torch.float32, False), (60, torch.float32, True), (120, torch.bfloat16, True),
     (240, torch.bfloat16, False)],
)  # fmt: skip
def test_dominant_tiles_when_the_tile_pass_outweighs_the_rows(decode, kv, dominant) -> None:
    """The 8 chunks beside 60-240 decode rows: the hint turns on past the measured crossover
    (the tile pass's estimated time 1.1 times the row pass's; here 0.87 and 1.79 in float32 at
    120 and 60 rows), and a bfloat16 pool's rows weigh half as much (1.75 at 120 rows, 0.87 at
    240); never without rows or without tiles."""
    rng = np.random.default_rng(7)
    seq, positions, contexts, tables = _mixed(rng, 32)
    seq, positions = seq[: 4096 + decode], positions[: 4096 + decode]
    if decode > 120:  # more decode rows than _mixed draws: repeat them
        extra = np.arange(8, 8 + decode - 120) % 120 + 8
        seq = np.concatenate([seq, extra])
        positions = np.concatenate([positions, contexts[extra] - 1])
    plan = ops.plan_batch(seq, 128, 32, tables, contexts, 16, query_positions=positions, kv_dtype=kv)
    assert plan.tiles.shape[0] == 64 and plan.rows.shape[0] > 0
    assert plan.dominant_tiles == dominant
    alone = ops.plan_batch(seq[:4096], 128, 32, tables, contexts, 16, query_positions=positions[:4096], kv_dtype=kv)
    rows = ops.plan_batch(seq[4096:], 128, 32, tables, contexts, 16, query_positions=positions[4096:], kv_dtype=kv)
    assert not alone.dominant_tiles and not rows.dominant_tiles


def test_merge_list_without_positions_is_every_row_outside_whole_tiles() -> None:
    tiles = np.array([[0, 64, 0, ops.TILE_WHOLE], [64, 10, 0, 0], [80, 3, 0, ops.TILE_WHOLE]])
    assert ops.merge_rows_for(90, tiles).tolist() == [*range(64, 80), *range(83, 90)]
    visible = np.arange(90) * 10
    assert ops.merge_rows_for(90, tiles, visible, 700).tolist() == [*range(71, 80), *range(83, 90)]
    assert ops.merge_rows_for(0, np.zeros((0, 4), np.int32)).tolist() == []


def test_upload_derives_a_merge_list_for_whole_tiles() -> None:
    import torch

    rows = np.array([[5, 0], [6, 0]], np.int32)
    tiles = np.array([[0, 5, 0, ops.TILE_WHOLE]], np.int32)
    plan = ops.upload_plan(rows, tiles, torch.device("cpu"))
    assert plan.merge.tolist() == [5, 6]
    plan = ops.upload_plan(rows, np.array([[0, 5, 0, 0]], np.int32), torch.device("cpu"))
    assert plan.merge is None, "without whole tiles every row may be merged"
    plan = ops.upload_plan(rows, tiles, torch.device("cpu"), merge=np.array([6]))
    assert plan.rows.tolist() == rows.tolist() and plan.tiles.tolist() == tiles.tolist()
    assert plan.merge.tolist() == [6]


def test_row_items_list_each_partition_full_ones_first() -> None:
    rows = np.array([[0, 0], [1, 0], [2, 2], [3, 0]], np.int32)
    visible = np.array([1030, 512, 3000, 0])
    items = ops.expand_rows(rows, visible, 512)
    # full partitions in row order, then the partial last ones, longest first
    assert items.tolist() == [[0, 0], [0, 1], [1, 0], [2, 2], [2, 3], [2, 4], [2, 5], [0, 2], [3, 0]]
    assert ops.expand_rows(rows, visible, 0).tolist() == items.tolist(), "0 is the 512 default"
    # a row whose first partition is past its visible keys has nothing left for the row pass
    assert ops.expand_rows(np.array([[5, 3]]), np.full(6, 1000), 512).tolist() == []
    assert ops.expand_rows(np.zeros((0, 2), np.int32), visible, 512).shape == (0, 2)


def _entry(seq_id, table, tokens=1):
    from paged_kv_serving_amd.runner import BatchEntry

    start = len(table) * 16 - tokens
    return BatchEntry(seq_id, tuple([1] * tokens), tuple(range(start, start + tokens)), tuple(table), tokens - 1)


def test_shared_prefix_order_groups_decode_rows_that_share_leading_blocks() -> None:
    from paged_kv_serving_amd.runner import shared_prefix_order

    prefix = list(range(40))  # 640 tokens at block size 16: past the 512-token threshold
    children = [_entry(f"c{i}", prefix + [100 + i]) for i in range(20)]
    strangers = [_entry(f"s{i}", list(range(200 + 50 * i, 241 + 50 * i))) for i in range(20)]
    prefill = _entry("p", list(range(2000, 2050)), tokens=30)
    interleaved = [e for pair in zip(children, strangers) for e in pair] + [prefill]
    order = shared_prefix_order(interleaved, 16)
    assert order is not None and sorted(order) == list(range(len(interleaved)))
    names = [interleaved[i].seq_id for i in order]
    first = names.index("c0")
    assert names[first : first + 20] == [f"c{i}" for i in range(20)]  # stable within the group
    assert names[-1] == "p"  # non-decode entries keep their place after the decode rows
    # Already grouped, no sharing, or too few decode rows: the batch order is kept.
    assert shared_prefix_order(children + strangers + [prefill], 16) is None
    assert shared_prefix_order(strangers, 16) is None
    assert shared_prefix_order(interleaved[:10], 16) is None


def _groups_scalar(rows, seq, tables, used_blocks, min_blocks):
    """Row-by-row restatement of the shared-prefix run search (the vectorised planner must
    find exactly these runs)."""
    def common(a, b):
        n = min(len(a), len(b))
        for k in range(n):
            if a[k] != b[k]:
                return k
        return n

    groups, count, i = [], rows.shape[0], 0
    while i < count:
        s0 = int(seq[int(rows[i, 0])])
        first = list(tables[s0][: used_blocks[s0]])
        shared_len, j = len(first), i + 1
        while j < count and int(rows[j, 0]) == int(rows[j - 1, 0]) + 1:
            sj = int(seq[int(rows[j, 0])])
            mine = list(tables[sj][: used_blocks[sj]])
            c = common(first, mine)
            limit = shared_len if c == len(mine) else min(shared_len, c)
            if limit < min_blocks:
                break
            shared_len = limit
            j += 1
        if j - i >= ops.MIN_SHARED_ROWS and shared_len >= min_blocks:
            groups.append((i, j - i, shared_len))
            i = j
        else:
            i += 1
    return groups


@pytest.mark.parametrize("seed", range(40))
def test_vectorised_prefix_groups_match_the_row_by_row_search(seed) -> None:
    rng = np.random.default_rng(seed)
    min_blocks = int(rng.integers(2, 12))
    trunks = [list(rng.integers(0, 10**6, 40)) for _ in range(3)]
    tables = []
    while len(tables) < 40 + seed * 3:  # runs of rows that branch off one trunk, or private rows
        length = int(rng.integers(1, 30))
        trunk = trunks[int(rng.integers(0, len(trunks)))] if rng.random() < 0.7 else None
        for _ in range(length):
            if trunk is None:
                t = list(rng.integers(2 * 10**6, 3 * 10**6, int(rng.integers(0, 50))))
            else:
                r = rng.random()  # mostly long branches; some end inside the trunk or diverge early
                keep = int(rng.integers(min_blocks, 41)) if r < 0.8 else int(rng.integers(0, min_blocks + 2))
                tail = 0 if r > 0.9 else int(rng.integers(0, 20))
                t = trunk[:keep] + list(rng.integers(10**6, 2 * 10**6, tail))
            tables.append(np.asarray(t, dtype=np.int64))
    n = len(tables)
    used = np.asarray([t.size for t in tables])
    seq = np.arange(n)
    rows = np.zeros((n, 2), np.int32)
    gaps = np.cumsum(rng.random(n) < 0.05)  # now and then a query row the row pass does not hold
    rows[:, 0] = np.arange(n) + gaps
    seq_full = np.zeros(int(rows[:, 0].max()) + 1, dtype=np.int64)
    seq_full[rows[:, 0]] = seq
    want = _groups_scalar(rows, seq_full, tables, used, min_blocks)
    assert ops._prefix_groups(rows, seq_full, tables, used, min_blocks) == want
    # the 2-D arena form of the same tables gives the same runs
    width = max(1, int(used.max()))
    arena = np.full((n, width + 3), -5, dtype=np.int64)
    for s, t in enumerate(tables):
        arena[s, : t.size] = t
    assert ops._prefix_groups(rows, seq_full, arena, used, min_blocks) == want
