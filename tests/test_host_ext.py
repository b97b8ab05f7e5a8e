"""The _pkvhost extension (csrc/pkv_host.cpp) against the Python it replaces in the runner, on
the CPU: the flattened batch, every slot (the reference's rule, runner.py:149-159, including
Python's floor division and negative indices) and the first slot problem; and the row order
that groups decode entries sharing their leading blocks (runner.shared_prefix_order)."""

from __future__ import annotations

import numpy as np
import pytest

from paged_kv_serving_amd import _native
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


@pytest.mark.parametrize("seed", range(30))
def test_prefix_order_matches_the_python_grouping(seed) -> None:
    rng = np.random.default_rng(seed)
    block = 16
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
    entries = tuple(entries)
    lead = -(-512 // block)
    assert ext.prefix_order(entries, lead, 16) == shared_prefix_order(entries, block)
