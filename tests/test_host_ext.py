"""The _pkvhost extension (csrc/pkv_host.cpp) against the Python it replaces in the runner, on
the CPU: the flattened batch, every slot (the reference's rule, runner.py:149-159, including
Python's floor division and negative indices), the first slot problem and the validation
statistics; the row order that groups decode entries sharing their leading blocks
(runner.shared_prefix_order); and the copy-on-write grouping (ops.independent_groups)."""

from __future__ import annotations

import numpy as np
import pytest

from paged_kv_serving_amd import _native, ops
from paged_kv_serving_amd.runner import BatchEntry, compute_slots, shared_prefix_order

ext = _native.host()


def gather(entries, block_size):
    count = len(entries)
    lengths, contexts, logits = np.zeros(count, np.int64), np.zeros(count, np.int32), np.zeros(count, np.int64)
    tokens, positions, slots = (np.zeros(1, np.int64) for _ in range(3))
    while True:
        total, problem, entry, position = ext.gather(entries, block_size, tokens, positions, slots, lengths, contexts, logits)
        if total >= 0:
            return tokens[:total], positions[:total], slots[:total], lengths, contexts, logits, (problem, entry, position)
        tokens, positions, slots = (np.zeros(-total, np.int64) for _ in range(3))


def random_entries(rng, block_size, count, *, negative=False):
    entries = []
    for i in range(count):
        n = int(rng.integers(1, 40)) if rng.random() < 0.3 else 1
        start = int(rng.integers(-3 if negative else 0, 500))
        positions = tuple(range(start, start + n))
        # long enough for the last position and for the negative ones (they index from the end)
        need = max(1, -(-(start + n) // block_size), -(-max(-start, 0) // block_size) + 1)
        table = tuple(int(b) for b in rng.integers(0, 10_000, need + int(rng.integers(0, 3))))
        index = None if rng.random() < 0.3 else int(rng.integers(0, n))
        entries.append(BatchEntry(f"s{i}", tuple(int(t) for t in rng.integers(0, 50, n)), positions, table, index))
    return tuple(entries)


@pytest.mark.parametrize("seed", range(40))
def test_gather_matches_the_python_batch_walk(seed) -> None:
    rng = np.random.default_rng(seed)
    block = int(rng.choice([1, 4, 16]))
    entries = random_entries(rng, block, int(rng.integers(1, 80)), negative=seed % 3 == 0)
    tokens, positions, slots, lengths, contexts, logits, problem = gather(entries, block)
    assert problem == (0, 0, 0)
    assert tokens.tolist() == [t for e in entries for t in e.token_ids]
    assert positions.tolist() == [p for e in entries for p in e.positions]
    assert slots.tolist() == compute_slots(entries, block).tolist()
    assert lengths.tolist() == [len(e.token_ids) for e in entries]
    assert contexts.tolist() == [e.positions[-1] + 1 for e in entries]
    starts = np.cumsum(lengths) - lengths
    assert logits.tolist() == [-1 if e.logits_index is None else int(s) + e.logits_index for e, s in zip(entries, starts)]


def test_gather_reports_the_first_slot_problem() -> None:
    entries = (
        BatchEntry("a", (1,), (3,), (7,)),
        BatchEntry("b", (1, 2), (15, 16), (4,)),  # position 16 has no block (block size 16)
        BatchEntry("c", (1,), (40,), (1,)),
    )
    *_, problem = gather(entries, 16)
    assert problem == (1, 1, 16)
    with pytest.raises(ValueError, match="sequence b: position 16 has no block in the table"):
        compute_slots(entries, 16)
    *_, problem = gather((BatchEntry("z", (1,), (-40,), (3, 4)),), 16)  # index -3 of a 2-block table
    assert problem == (2, 0, -40)


def test_gather_reads_entries_of_any_class_as_getattr_does() -> None:
    """BatchEntry keeps its fields in __slots__, which gather reads at their offsets; objects of
    other classes (a plain dataclass, a namespace) and a subclass that overrides a field with a
    property go through getattr, so each gives what its attributes say."""
    from dataclasses import dataclass
    from types import SimpleNamespace

    @dataclass(frozen=True)
    class PlainEntry:
        seq_id: str
        token_ids: tuple
        positions: tuple
        block_table: tuple
        logits_index: int | None = None

    class Remapped(BatchEntry):
        @property
        def block_table(self):  # shadows the slot of the same name, which keeps the given table
            return (99, 98, 97)

        @block_table.setter
        def block_table(self, value):
            BatchEntry.block_table.__set__(self, value)

    assert not hasattr(BatchEntry("a", (1,), (3,), (7,)), "__dict__")
    fields = [("a", (1, 2), (3, 4), (7,), 1), ("b", (5,), (20,), (4, 6), None), ("c", (2,), (0,), (11,), 0)]
    plain = tuple(BatchEntry(*f) for f in fields)
    expected = gather(plain, 16)
    for kind in (lambda *f: PlainEntry(*f), lambda *f: SimpleNamespace(
            seq_id=f[0], token_ids=f[1], positions=f[2], block_table=f[3], logits_index=f[4])):  # fmt: skip
        got = gather(tuple(kind(*f) for f in fields), 16)
        for a, b in zip(got[:6], expected[:6]):
            assert a.tolist() == b.tolist()
        assert got[6] == expected[6]
    mixed = (plain[0], Remapped(*fields[1]), plain[2])  # classes change along the walk
    *_, problem = gather(mixed, 16)
    assert problem == (0, 0, 0)
    slots = gather(mixed, 16)[2]
    assert slots.tolist() == compute_slots(mixed, 16).tolist()
    assert slots[2] == 98 * 16 + 4  # position 20 of the property's table


def test_gather_converts_ints_of_every_size_and_kind() -> None:
    """Small exact ints are read from the object; zero, negatives, ints past one 30-bit digit,
    bools and NumPy integers take the general conversion and give the same values."""
    big = 1 << 40
    entries = (
        BatchEntry("a", (0, True, np.int64(7)), (0, 1, 2), (3,)),
        BatchEntry("b", (big,), (-1,), (5, 6)),  # negative: from the end of the table
        BatchEntry("c", ((1 << 30) + 3,), ((1 << 30) + 5,), (1, 2, 9)),  # block (2**30 + 5) // 2**29 = 2
        BatchEntry("d", (2,), (np.int32(17),), (4, big)),
    )
    tokens = gather(entries[:1], 16)[0]
    assert tokens.tolist() == [0, 1, 7]
    tokens, positions, slots, *_ = gather(entries[1:2], 16)
    assert tokens.tolist() == [big] and positions.tolist() == [-1] and slots.tolist() == [6 * 16 + 15]
    tokens, positions, slots, *_ = gather(entries[2:3], 1 << 29)
    assert positions.tolist() == [(1 << 30) + 5]
    assert slots.tolist() == [9 * (1 << 29) + 5]
    slots = gather(entries[3:], 16)[2]
    assert slots.tolist() == [big * 16 + 1]
    with pytest.raises(TypeError):
        gather((BatchEntry("e", (1,), (2.0,), (3,)),), 16)


def _prefix_case(rng, block):
    stems = [tuple(int(b) for b in rng.integers(0, 1000, 40)) for _ in range(3)]
    entries = []
    for i in range(int(rng.integers(1, 120))):
        if rng.random() < 0.6:
            stem = stems[int(rng.integers(0, 3))] if rng.random() < 0.8 else tuple(int(b) for b in rng.integers(1000, 2000, 40))
            table = stem + tuple(int(b) for b in rng.integers(5000, 9000, int(rng.integers(1, 5))))
            entries.append(BatchEntry(f"d{i}", (1,), (len(table) * block - 1,), table, 0))
        else:
            n = int(rng.integers(1, 30))
            entries.append(BatchEntry(f"p{i}", tuple(range(n)), tuple(range(n)), tuple(range(3)), None))
    return tuple(entries)


@pytest.mark.parametrize("seed", range(40))
def test_prefix_order_from_the_arena_matches_the_python_grouping(seed) -> None:
    from paged_kv_serving_amd.tables import BlockTableArena

    rng = np.random.default_rng(seed)
    block = 16
    entries = _prefix_case(rng, block)
    if seed % 5 == 0:  # already grouped: sharers adjacent, nothing to move
        entries = tuple(sorted(entries, key=lambda e: (len(e.token_ids) != 1, e.block_table[:32])))
    arena = BlockTableArena("cpu", rows=4, width=8)  # grows to fit
    for _ in range(2):  # a fresh arena, then the same tables again (rows reused, nothing uploaded)
        update = arena.update(entries)
        arena.apply_nothing()
        lengths = np.asarray([len(e.token_ids) for e in entries], np.int64)
        out = np.full(len(entries) + 3, -5, np.int64)
        moved = ext.prefix_order_rows(update.rows, lengths, arena.host, arena.held_lengths, -(-512 // block), 16, out)
        want = shared_prefix_order(entries, block)
        assert (out[: len(entries)].tolist() if moved else None) == want
        assert np.all(out[len(entries) :] == -5) and (moved or np.all(out == -5))


@pytest.mark.parametrize("seed", range(40))
def test_gather_statistics_are_the_reductions_the_runner_validates(seed) -> None:
    rng = np.random.default_rng(seed)
    block = int(rng.choice([1, 4, 16]))
    entries = random_entries(rng, block, int(rng.integers(1, 80)), negative=seed % 3 == 0)
    if seed % 4 == 1:  # two decode rows starting in the same block
        first = entries[0]
        entries = entries + (BatchEntry("twin", (1,), (first.positions[-1],), first.block_table, 0),
                             BatchEntry("twin2", (2,), (first.positions[-1],), first.block_table, 0))
    count = len(entries)
    total = sum(len(e.token_ids) for e in entries)
    tokens, positions, slots = (np.zeros(total, np.int64) for _ in range(3))
    lengths, contexts, logits = np.zeros(count, np.int64), np.zeros(count, np.int32), np.zeros(count, np.int64)
    stats = np.zeros(9, np.int64)
    got = ext.gather(entries, block, tokens, positions, slots, lengths, contexts, logits, stats)
    assert got[0] == total
    decode_firsts = [e.block_table[0] for e in entries if len(e.token_ids) == 1]
    want = [tokens.min(), tokens.max(), positions.min(), positions.max(), slots.min(), slots.max(), contexts.min(),
            int(len(set(decode_firsts)) < len(decode_firsts)), contexts.max()]  # fmt: skip
    assert stats.tolist() == [int(v) for v in want]
    assert stats[7] == (1 if seed % 4 == 1 else stats[7])


def test_gather_statistics_count_unformed_slots_as_minus_one() -> None:
    entries = (BatchEntry("a", (3,), (5,), (7,)), BatchEntry("b", (4,), (40,), (1,)))
    stats = np.zeros(9, np.int64)
    buffers = [np.zeros(2, np.int64) for _ in range(3)] + [np.zeros(2, np.int64), np.zeros(2, np.int32), np.zeros(2, np.int64)]
    total, problem, entry, position = ext.gather(entries, 16, *buffers, stats)
    assert (total, problem, entry, position) == (2, 1, 1, 40)
    assert stats.tolist() == [3, 4, 5, 40, -1, 7 * 16 + 5, 6, 0, 41]
    with pytest.raises(ValueError, match="stats must hold 9 entries"):
        ext.gather(entries, 16, *buffers, np.zeros(8, np.int64))


def _python_groups(pairs):
    return [len(g) for g in ops.independent_groups(pairs)]


@pytest.mark.parametrize("seed", range(60))
def test_copy_queue_groups_match_the_python_grouping(seed) -> None:
    rng = np.random.default_rng(seed)
    n = int(rng.integers(0, 300))
    ids = int(rng.choice([4, 20, 1000, 100_000]))
    pairs = [(int(a), int(b)) for a, b in rng.integers(0, ids, (n, 2)) if a != b]
    queue = ext.CopyQueue(ids)
    for source, destination in pairs:
        queue.push(source, destination)
    assert len(queue) == len(pairs) and queue.items() == pairs
    assert queue.groups() == _python_groups(pairs)
    assert queue.groups() == _python_groups(pairs)  # the per-block marks were left all zero
    queue.clear()
    assert len(queue) == 0 and queue.groups() == []


def test_copy_queue_flush_checks_its_buffers_before_any_device_work() -> None:
    """CopyQueue.flush: an empty queue does nothing; a pinned buffer too small for the pairs is
    reported as the bytes needed (the runner grows it and calls again); a missing device buffer
    is refused. None of these reaches the device, so they run on any machine."""
    bound = _native.bound_host()
    queue = bound.CopyQueue(64)
    assert queue.flush(0, 0, 0, 1, 16, np.zeros(0, np.uint8), 0, 0, 0) == (0, 0)
    for source, destination in [(1, 2), (3, 4), (5, 6)]:
        queue.push(source, destination)
    assert queue.flush(0, 0, 0, 1, 16, np.zeros(47, np.uint8), 4096, 0, 0) == (0, -48)  # 16 bytes a pair
    with pytest.raises(ValueError, match="device buffer"):
        queue.flush(0, 0, 0, 1, 16, np.zeros(48, np.uint8), 0, 0, 0)
    with pytest.raises(TypeError):  # the pinned buffer must be bytes
        queue.flush(0, 0, 0, 1, 16, np.zeros(48, np.int32), 4096, 0, 0)
    assert queue.items() == [(1, 2), (3, 4), (5, 6)]  # nothing was dequeued


def test_copy_queue_groups_of_forks_are_one_group_and_bad_pairs_are_refused() -> None:
    queue = ext.CopyQueue(400)
    for i in range(256):  # every child copies the same shared block
        queue.push(7, 100 + i)
    assert queue.groups() == [256]
    queue.clear()
    for source, destination in [(1, 2), (2, 3), (3, 1)]:
        queue.push(source, destination)
    assert queue.groups() == [1, 1, 1]
    # the reference's checks (runner.py:128-133), NumPy integers accepted as ids
    queue.push(np.int64(5), np.int32(6))
    assert queue.items()[-1] == (5, 6)
    with pytest.raises(ValueError, match="onto itself"):
        queue.push(4, 4)
    for bad in [(1, 400), (-1, 2), (2**70, 1)]:
        with pytest.raises(IndexError, match=f"block id {bad[0] if not 0 <= bad[0] < 400 else bad[1]} is outside"):
            queue.push(*bad)
    with pytest.raises(TypeError):
        queue.push(1)
    with pytest.raises(TypeError):
        queue.push("1", 2)
    assert len(queue) == 4  # nothing refused was queued
    with pytest.raises(ValueError):
        ext.CopyQueue(0)


def test_the_bound_planner_matches_the_ctypes_planner() -> None:
    from test_host_plan_native import random_batch

    for seed in range(60):
        case = random_batch(seed)
        planner = ops.NativePlanner()
        want = planner.plan(case["query_seq"], case["head_dim"], case["num_heads"], case["tables"],
                            case["context_lens"], case["block_size"], partition_size=case["partition_size"],
                            query_positions=case["query_positions"])  # fmt: skip
        fast = ops.NativePlanner()
        fast._rows = np.zeros((1, 2), np.int32)  # grows on the first call
        rows, tiles, merge, partition, flags = fast.plan_views(
            case["query_seq"].astype(np.int32), case["query_positions"].astype(np.int32), case["tables"],
            case["context_lens"].astype(np.int32), case["block_size"], case["num_heads"], case["head_dim"],
            case["partition_size"],
        )  # fmt: skip
        assert np.array_equal(rows, want.rows) and np.array_equal(tiles, want.tiles)
        assert np.array_equal(merge, want.merge) and partition == want.partition_size
        assert bool(flags & _native.PKV_ATTN_SHARED_KV) == want.shared_kv
        assert bool(flags & _native.PKV_ATTN_SHORT_ROWS) == want.short_rows


def test_the_bound_model_ops_reach_the_library_and_check_their_arguments() -> None:
    """_pkvhost.rms_norm / silu_mul / rope_append pass their arguments to pkv_rms_norm /
    pkv_silu_mul / pkv_rope_append unchanged: empty calls succeed and malformed ones are refused,
    both before any device work (so this runs without a GPU)."""
    host = _native.bound_host()
    ok, einval = _native.PKV_OK, _native.PKV_EINVAL
    one = 16  # an address never dereferenced: every call below returns first
    assert host.rms_norm(0, 4, 0, 4, 0, 0, 0, 0, 4, 1e-5, 0, 0) == ok  # no rows
    assert host.rms_norm(one, 4, one, 4, 0, 0, one, 1, 0, 1e-5, 0, 0) == einval  # dim 0
    assert host.rms_norm(one, 3, one, 4, 0, 0, one, 1, 4, 1e-5, 0, 0) == einval  # out stride < dim
    assert host.rms_norm(one, 4, one, 4, 0, 0, one, 1, 4, -1.0, 0, 0) == einval  # eps < 0
    assert host.silu_mul(0, 4, 0, 0, 8, 0, 4, 0, 0) == ok
    assert host.silu_mul(one, 4, one, one, 3, 1, 4, 0, 0) == einval  # input stride < width
    rope = [one, 64, one, one, one, 64, 64, 64, one, one, one, 16, one, one, 0, 100, one, 2, 2, 32, 0, 0]
    assert host.rope_append(*rope[:17], 0, *rope[18:]) == ok  # no tokens
    assert host.rope_append(*rope[:19], 31, *rope[20:]) == einval  # odd head_dim
    assert host.rope_append(*rope[:14], 7, *rope[15:]) == einval  # unknown pool dtype


def test_stage_packs_the_parts_and_issues_one_host_to_device_copy() -> None:
    """_pkvhost.stage packs the int64 parts, then the int32 parts, back to back into the pinned
    buffer and hands the packed bytes to one hipMemcpyAsync (host to device, on the given stream).
    hipMemcpyAsync is replaced here by a recording stand-in, so this runs without a GPU; the
    real one is bound again afterwards."""
    import ctypes

    lib = _native.library()
    host = _native.bound_host()
    address = lambda fn: ctypes.cast(fn, ctypes.c_void_p).value  # noqa: E731
    entry_points = [address(getattr(lib, name)) for name in (
        "pkv_plan_batch", "pkv_paged_attention", "pkv_paged_attention_append", "pkv_copy_blocks",
        "pkv_rms_norm", "pkv_silu_mul", "pkv_rope_append")]  # fmt: skip
    calls = []

    def record(dst, src, size, kind, stream):
        calls.append((dst, ctypes.string_at(src, size), kind, stream))
        return 0

    fake = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                            ctypes.c_void_p)(record)  # fmt: skip
    host.bind(*entry_points, address(fake))
    try:
        p64 = [np.arange(3, dtype=np.int64) - 5, np.zeros(0, np.int64), np.array([1 << 40], np.int64)]
        p32 = [np.array([7, -8, 9], np.int32), np.zeros(0, np.int32), np.array([2**31 - 1], np.int32)]
        buf = np.full(64, 0xAB, dtype=np.uint8)
        offsets = host.stage(p64, p32, buf, 4096, 77)
        want = np.concatenate(p64).tobytes() + np.concatenate(p32).tobytes()
        assert offsets == [0, 24, 24, 32, 44, 44]
        assert buf[: len(want)].tobytes() == want and np.all(buf[len(want) :] == 0xAB)
        assert calls == [(4096, want, 1, 77)]
        # Too small a buffer: nothing written, nothing copied, None so the caller can grow it.
        small = np.zeros(len(want) - 1, np.uint8)
        assert host.stage(p64, p32, small, 4096, 77) is None and not small.any() and len(calls) == 1
        # Nothing to send: offsets only, no copy.
        assert host.stage([np.zeros(0, np.int64)], [], np.zeros(0, np.uint8), 0, 0) == [0]
        assert len(calls) == 1
        with pytest.raises(TypeError):  # a part of the wrong width
            host.stage([np.zeros(2, np.int32)], [], buf, 4096, 77)
        with pytest.raises(ValueError, match="contiguous"):  # a part that is not contiguous
            host.stage([np.arange(8, dtype=np.int64)[::2]], [], buf, 4096, 77)
        with pytest.raises(ValueError):  # no device buffer for a non-empty copy
            host.stage(p64, p32, buf, 0, 77)
        # With an event: the copy that last read the buffer is waited for before the packing,
        # and the event is recorded on the same stream right after the new copy.
        events = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)
        record_event = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p)(
            lambda event, stream: calls.append(("record", event, stream)) or 0)
        synchronize = events(lambda event: calls.append(("synchronize", event)) or 0)
        host.bind(*entry_points, address(fake), 0, 0, 0, 0, 0, address(record_event), address(synchronize), 0)
        del calls[:]
        assert host.stage(p64, p32, buf, 4096, 77, 555) == offsets
        assert calls == [("synchronize", 555), (4096, want, 1, 77), ("record", 555, 77)]
        fail = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                ctypes.c_void_p)(lambda *args: 1)  # fmt: skip
        host.bind(*entry_points, address(fail))
        with pytest.raises(RuntimeError, match="hipMemcpyAsync"):
            host.stage(p64, p32, buf, 4096, 77)
        with pytest.raises(RuntimeError, match="event entry points"):  # unbound event functions
            host.stage(p64, p32, buf, 4096, 77, 555)
    finally:
        _native._BOUND = False  # bind every entry point again, the optional ones included
        _native.bound_host()


def exclusive_by_brute_force(tables, contexts, block_size, num_blocks) -> bool:
    """Each written block (that of position context - 1) occurs once among all visible blocks."""
    visible = [b for t, c in zip(tables, contexts) for b in t[: -(-c // block_size)]]
    for table, ctx in zip(tables, contexts):
        written = table[(ctx - 1) // block_size]
        if 0 <= written < num_blocks and visible.count(written) != 1:
            return False
    return True


def exclusive(tables, contexts, block_size, num_blocks) -> bool:
    width = max(len(t) for t in tables)
    host = np.zeros((len(tables) + 3, width + 2), np.int32)  # arena rows in scrambled order
    rows = np.random.default_rng(len(tables)).permutation(host.shape[0])[: len(tables)].astype(np.int32)
    for row, table in zip(rows, tables):
        host[row, : len(table)] = table
    marks = np.zeros(num_blocks, np.uint8)
    got = ext.exclusive_writes(rows, np.asarray(contexts, np.int32), host, block_size, marks)
    assert not marks.any(), "the marks buffer is left all zero"
    return got


def test_exclusive_writes_decides_when_the_decode_append_may_be_fused() -> None:
    """ModelRunner fuses a decode batch's append into attention only when no row reads a block
    another row writes (the reference writes every slot first, runner.py:195-212)."""
    private = [(0, 1, 2), (3, 4), (5,)]
    assert exclusive(private, [40, 20, 3], 16, 8)
    # the same sequence twice (positions p and p + 1): the first row's block is read by the second
    assert not exclusive([(0, 1, 2), (0, 1, 2)], [40, 41], 16, 8)
    # two tables share the block being written (a partially filled shared block without COW)
    assert not exclusive([(0, 1, 2), (3, 2)], [40, 20], 16, 8)
    # a shared *earlier* block is read by both, but nobody writes it: still exclusive
    assert exclusive([(0, 1, 2), (0, 4)], [40, 20], 16, 8)
    # a table naming its written block twice reads the written slot at another position too
    assert not exclusive([(2, 1, 2)], [40], 16, 8)
    # two rows writing one block
    assert not exclusive([(0, 7), (1, 7)], [20, 25], 16, 8)
    # blocks past the visible ones do not count
    assert exclusive([(0, 1, 5), (5, 6)], [20, 20], 16, 8)


def test_exclusive_writes_refuses_tiles_over_a_new_position() -> None:
    """Only the row pass appends, so a fused call's tiles must cover no row's own position
    (context - 1): tile records (first row, count, first partition, end partition) over the
    entries in the order given; end <= first partition runs through the last, -1 is whole."""
    tables = [tuple(range(10 * i, 10 * i + 5)) for i in range(4)]  # private blocks
    rows = np.arange(4, dtype=np.int32)
    host = np.zeros((4, 5), np.int32)
    for i, t in enumerate(tables):
        host[i] = t
    contexts = np.asarray([70, 65, 80, 33], np.int32)  # own positions 69, 64, 79, 32
    marks = np.zeros(64, np.uint8)

    def fused(tiles, partition=32):
        return ext.exclusive_writes(rows, contexts, host, 16, marks, np.asarray(tiles, np.int32).reshape(-1, 4),
                                    partition)  # fmt: skip

    assert ext.exclusive_writes(rows, contexts, host, 16, marks)
    assert fused(np.zeros((0, 4)))
    assert fused([[0, 3, 0, 2]])  # keys [0, 64) of rows 0-2: no own position
    assert not fused([[0, 3, 0, 3]])  # keys [0, 96) hold row 1's position 64
    assert fused([[3, 1, 2, 3]])  # keys [64, 96) of row 3 (position 32)
    assert not fused([[2, 2, 1, 1]])  # from key 32 through the last: row 3's position 32
    assert not fused([[1, 1, 0, -1]])  # a whole tile covers everything
    assert not fused([[2, 5, 0, 1]])  # rows past the batch
    with pytest.raises(ValueError):
        fused([[0, 3, 0, 2]], partition=0)
    assert not marks.any()


@pytest.mark.parametrize("seed", range(60))
def test_exclusive_writes_matches_the_brute_force_rule(seed) -> None:
    rng = np.random.default_rng(seed)
    block = int(rng.choice([1, 4, 16]))
    num_blocks = int(rng.integers(8, 200))
    tables, contexts = [], []
    for _ in range(int(rng.integers(1, 30))):
        ctx = int(rng.integers(1, 6 * block + 1))
        need = -(-ctx // block) + int(rng.integers(0, 3))
        # a few ids past the pool, which no pass reads
        tables.append(tuple(int(b) for b in rng.integers(0, num_blocks + 3, need)))
        contexts.append(ctx)
    assert exclusive(tables, contexts, block, num_blocks) == exclusive_by_brute_force(tables, contexts, block, num_blocks)


@pytest.mark.parametrize("seed", range(60))
def test_exclusive_writes_on_forked_tables_matches_the_brute_force_rule(seed) -> None:
    """Tables that share leading blocks (forks of one or two parents), the case whose repeated
    prefixes the check skips: rows ending inside a shared prefix, rows writing a block another
    row reads past the prefix, prefixes of different lengths next to each other."""
    rng = np.random.default_rng(1000 + seed)
    block = int(rng.choice([1, 4, 16]))
    ids = iter(rng.permutation(5000).tolist())
    parents = [[next(ids) for _ in range(int(rng.integers(1, 12)))] for _ in range(2)]
    tables, contexts = [], []
    for _ in range(int(rng.integers(2, 25))):
        parent = parents[int(rng.integers(2))]
        keep = int(rng.integers(0, len(parent) + 1))
        private = int(rng.integers(0, 4)) if rng.random() < 0.1 else int(rng.integers(1, 4))
        table = parent[:keep] + [next(ids) for _ in range(private)]
        if not table:
            table = [next(ids)]
        ctx = int(rng.integers((len(table) - 1) * block + 1, len(table) * block + 1))
        if rng.random() < 0.05 and tables:  # write into a block some other row holds
            other = tables[int(rng.integers(len(tables)))]
            table = list(other[: max(1, len(other) - 1)])
            ctx = len(table) * block
        tables.append(tuple(table))
        contexts.append(ctx)
    assert exclusive(tables, contexts, block, 5000) == exclusive_by_brute_force(tables, contexts, block, 5000)


def test_forward_refuses_bad_arguments_before_any_device_work() -> None:
    """_pkvhost.forward (the runner's whole forward pass as one call) checks its field count and
    sizes before it touches a device, so these run on any machine."""
    bound = _native.bound_host()
    with pytest.raises(ValueError, match="integers"):
        bound.forward((0,) * 5, [], 1e-5, 0.1)
    fields = [0] * 52
    fields[2], fields[3], fields[4], fields[5], fields[6], fields[7], fields[8] = 4, 1, 64, 2, 16, 32, 10
    with pytest.raises(ValueError, match="out of range"):  # d_model != heads * head_dim
        bound.forward(tuple(fields), [], 1e-5, 0.1)
    fields[6] = 32
    fields[2] = 0  # no tokens
    with pytest.raises(ValueError, match="out of range"):
        bound.forward(tuple(fields), [], 1e-5, 0.1)
    fields[2] = 4
    with pytest.raises(ValueError, match="six weight addresses"):
        bound.forward(tuple(fields), [(1, 2, 3)], 1e-5, 0.1)
