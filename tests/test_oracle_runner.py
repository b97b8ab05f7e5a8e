"""Pin slots, append, copy-on-write and copy batching (integer and byte work: bit-exact).

The slot of a position is ``block_table[p // B] * B + p % B`` (reference runner.py:158). The
oracle's loop and the package's vectorised ``compute_slots`` are checked against a brute force
that walks the table token by token, and against a shadow read-back: after scattering token ids
into a pool by slot, reading every sequence back through its table in logical order returns its
own tokens. Copy batching (``independent_groups``) must equal one-at-a-time copies in list order.
"""

from __future__ import annotations

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle.runner import append, copy_block, slots_for
from paged_kv_serving_amd.ops import independent_groups
from paged_kv_serving_amd.runner import BatchEntry, compute_slots


def brute_slots(positions, table, block):
    """Walk the table one token at a time: logical token i lives at (table[i // B], i % B)."""
    layout = {}
    for i in range(len(table) * block):
        layout[i] = table[i // block] * block + (i - (i // block) * block)
    return [layout[p] for p in positions]


@settings(max_examples=60, deadline=None)
@given(
    block=st.integers(1, 17),
    data=st.data(),
)
def test_slots_agree_with_brute_force(block, data) -> None:
    blocks = data.draw(st.integers(1, 12))
    table = data.draw(st.permutations(range(blocks * 3)))[:blocks]
    positions = data.draw(st.lists(st.integers(0, blocks * block - 1), min_size=1, max_size=30))
    want = brute_slots(positions, table, block)
    assert slots_for("s", positions, table, block) == want
    entry = BatchEntry("s", tuple([0] * len(positions)), tuple(positions), tuple(table))
    got = compute_slots([entry, entry], block)
    assert got.dtype == np.int64 and got.tolist() == want + want


def test_a_position_without_a_block_is_refused_with_the_reference_message() -> None:
    entry = BatchEntry("seq-7", (1, 2), (3, 4), (5,))
    with pytest.raises(ValueError, match="sequence seq-7: position 4 has no block in the table"):
        compute_slots([entry], 4)
    with pytest.raises(ValueError, match="sequence seq-7: position 4 has no block in the table"):
        slots_for("seq-7", (3, 4), (5,), 4)


def test_shadow_read_back_through_the_tables() -> None:
    rng = np.random.default_rng(0)
    block, heads, dim, pool = 4, 2, 3, 40
    keys = np.zeros((pool, block, heads, dim), dtype=np.float32)
    values = np.zeros_like(keys)
    perm = rng.permutation(pool)
    lengths, tables, offset = [7, 13, 1, 9], [], 0
    for n in lengths:
        used = -(-n // block)
        tables.append(perm[offset : offset + used].tolist())
        offset += used
    entries, rows_k, rows_v = [], [], []
    for s, n in enumerate(lengths):
        entries.append(BatchEntry(f"s{s}", tuple([0] * n), tuple(range(n)), tuple(tables[s])))
        rows_k.append(np.full((n, heads, dim), s + 1, dtype=np.float32) + np.arange(n)[:, None, None])
        rows_v.append(-rows_k[-1])
    append(keys, values, compute_slots(entries, block), np.concatenate(rows_k), np.concatenate(rows_v))
    for s, n in enumerate(lengths):
        logical = keys[tables[s]].reshape(-1, heads, dim)[:n]
        assert np.array_equal(logical, rows_k[s])
        assert np.array_equal(values[tables[s]].reshape(-1, heads, dim)[:n], rows_v[s])
    used_blocks = {b for t in tables for b in t}
    assert not keys[[b for b in range(pool) if b not in used_blocks]].any()


def test_copy_block_copies_every_layer_and_refuses_a_self_copy() -> None:
    rng = np.random.default_rng(1)
    keys = rng.standard_normal((3, 5, 2, 1, 4)).astype(np.float32)
    values = rng.standard_normal((3, 5, 2, 1, 4)).astype(np.float32)
    before_k, before_v = keys.copy(), values.copy()
    copy_block(keys, values, 4, 1)
    assert np.array_equal(keys[:, 1], before_k[:, 4]) and np.array_equal(values[:, 1], before_v[:, 4])
    assert np.array_equal(np.delete(keys, 1, axis=1), np.delete(before_k, 1, axis=1))
    with pytest.raises(ValueError, match="onto itself"):
        copy_block(keys, values, 2, 2)


@settings(max_examples=200, deadline=None)
@given(st.lists(st.tuples(st.integers(0, 7), st.integers(0, 7)).filter(lambda p: p[0] != p[1]), max_size=12))
def test_batched_copy_groups_equal_copies_in_order(pairs) -> None:
    start = list(range(100, 108))
    sequential = list(start)
    for src, dst in pairs:
        sequential[dst] = sequential[src]
    batched = list(start)
    groups = independent_groups(pairs)
    assert [p for g in groups for p in g] == pairs
    for group in groups:
        reads = [batched[src] for src, _ in group]  # all reads of a group happen concurrently
        dsts = [dst for _, dst in group]
        assert len(set(dsts)) == len(dsts)
        assert not set(dsts) & {src for src, _ in group}
        for dst, value in zip(dsts, reads):
            batched[dst] = value
    assert batched == sequential
