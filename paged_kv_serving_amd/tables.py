"""Block tables kept on the device between iterations, refreshed where they changed.

The reference converts every entry's ``block_table`` tuple to an array on every call
(runner.py:187) and, per sequence, hands it to ``paged_attention``. A continuing sequence's
table changes little from one iteration to the next: a decode step appends a block every
``block_size`` tokens, and a copy-on-write swaps the one shared block being written. The arena
below keeps one padded int32 row per recently seen sequence, in host memory and on the device,
and each iteration uploads only the entries from the first one that differs from what that row
already holds. Attention then reads the arena directly: a query's sequence index is its
sequence's arena row, so no per-call table tensor is built at all.

Rows are keyed by sequence id. A sequence not seen in the current iteration may lose its row to
a newcomer (least recently used first); the arena grows when one iteration needs more rows, or
a longer table, than it has.
"""

from __future__ import annotations

import numpy as np
import torch

__all__ = ["BlockTableArena", "TableUpdate"]


class TableUpdate:
    """What one iteration changes: the arena row of every entry, and the flat (row * width +
    column) indices and values of the table entries to write on the device."""

    __slots__ = ("rows", "index", "values")

    def __init__(self, rows: np.ndarray, index: np.ndarray, values: np.ndarray) -> None:
        self.rows = rows
        self.index = index
        self.values = values


class BlockTableArena:
    """Padded int32 block-table rows, mirrored on ``device``; see the module docstring."""

    def __init__(self, device: torch.device | str, *, rows: int = 64, width: int = 64) -> None:
        if rows < 1 or width < 1:
            raise ValueError("rows and width must be >= 1")
        self.device = torch.device(device)
        self.host = np.zeros((rows, width), dtype=np.int32)
        self.tables = torch.zeros((rows, width), dtype=torch.int32, device=self.device)
        self._row_of: dict[object, int] = {}
        self._key_of: list[object | None] = [None] * rows
        self._held: list[tuple[int, ...]] = [()] * rows
        self._last_use = np.zeros(rows, dtype=np.int64)
        self._step = 0
        # Rows whose recorded content an update changed and no apply() has written to the device
        # yet. If the caller fails between the two, the next update forgets what they hold.
        self._unapplied: list[int] = []

    @property
    def num_rows(self) -> int:
        return self.host.shape[0]

    @property
    def width(self) -> int:
        return self.host.shape[1]

    def held(self, row: int) -> tuple[int, ...]:
        """The table arena row ``row`` currently holds."""
        return self._held[row]

    def update(self, entries) -> TableUpdate:
        """Assign a row to every entry (by ``seq_id``) and record the table entries that differ
        from what the row holds. The host mirror is updated at once; the device rows change when
        the returned indices and values are applied with :meth:`apply`. If the previous update
        was never applied (its caller raised in between), the rows it changed are treated as
        holding nothing, so their whole tables are uploaded again."""
        for row in self._unapplied:
            self._held[row] = ()
        self._unapplied = []
        self._step += 1
        step = self._step
        count = len(entries)
        longest = max((len(e.block_table) for e in entries), default=0)
        if count > self.num_rows or longest > self.width:
            self._grow(max(count, self.num_rows), longest)
        rows = np.empty(count, dtype=np.int32)
        index_parts: list[np.ndarray] = []
        value_parts: list[tuple[int, ...]] = []
        seen: dict[object, int] = {}
        width = self.width
        for i, entry in enumerate(entries):
            key: object = entry.seq_id
            repeat = seen.get(key, 0)
            seen[key] = repeat + 1
            if repeat:  # the same sequence twice in one batch gets a row per occurrence
                key = (entry.seq_id, repeat)
            row = self._row_of.get(key)
            if row is None:
                row = self._claim(key, step)
            self._last_use[row] = step
            rows[i] = row
            new = tuple(entry.block_table)
            old = self._held[row]
            if new == old:
                continue
            start = _common_prefix(old, new)
            if start < len(new):
                segment = new[start:]
                self.host[row, start : len(new)] = segment
                index_parts.append(np.arange(row * width + start, row * width + len(new), dtype=np.int64))
                value_parts.append(segment)
            self._held[row] = new
            self._unapplied.append(row)
        if index_parts:
            index = np.concatenate(index_parts)
            values = np.fromiter((v for part in value_parts for v in part), dtype=np.int32, count=index.size)
        else:
            index = np.zeros(0, dtype=np.int64)
            values = np.zeros(0, dtype=np.int32)
        return TableUpdate(rows, index, values)

    def apply(self, index: torch.Tensor, values: torch.Tensor) -> None:
        """Write an update's values (device int32) at its flat indices (device int64)."""
        if index.numel():
            self.tables.view(-1).index_copy_(0, index, values)
        self._unapplied = []

    def used_blocks(self, rows: np.ndarray, block_counts: np.ndarray) -> np.ndarray:
        """The first ``block_counts[i]`` table entries of arena row ``rows[i]``, concatenated."""
        if rows.size == 0:
            return np.zeros(0, dtype=np.int32)
        counts = np.minimum(np.asarray(block_counts, dtype=np.int64), self.width)
        mask = np.arange(self.width)[None, :] < counts[:, None]
        return self.host[rows][mask]

    # --- rows ----------------------------------------------------------------------------

    def _claim(self, key: object, step: int) -> int:
        """A free row, or the least recently used row not used in this iteration."""
        candidates = np.flatnonzero(self._last_use < step)
        if candidates.size == 0:  # every row is in use by this iteration: add rows
            self._grow(self.num_rows + 1, self.width)
            candidates = np.flatnonzero(self._last_use < step)
        row = int(candidates[np.argmin(self._last_use[candidates])])
        previous = self._key_of[row]
        if previous is not None:
            del self._row_of[previous]
        self._key_of[row] = key
        self._row_of[key] = row
        self._held[row] = ()  # nothing the row holds may be trusted for the new key
        return row

    def _grow(self, rows: int, width: int) -> None:
        new_rows = max(rows, self.num_rows)
        if new_rows > self.num_rows:
            new_rows = max(new_rows, 2 * self.num_rows)
        new_width = max(width, self.width)
        if new_width > self.width:
            new_width = max(new_width, 2 * self.width)
        host = np.zeros((new_rows, new_width), dtype=np.int32)
        host[: self.num_rows, : self.width] = self.host
        tables = torch.zeros((new_rows, new_width), dtype=torch.int32, device=self.device)
        tables[: self.num_rows, : self.width] = self.tables
        extra = new_rows - self.num_rows
        self._key_of.extend([None] * extra)
        self._held.extend([()] * extra)
        self._last_use = np.concatenate([self._last_use, np.zeros(extra, dtype=np.int64)])
        self.host = host
        self.tables = tables


def _common_prefix(old: tuple[int, ...], new: tuple[int, ...]) -> int:
    """Length of the longest common prefix of two tables."""
    n = min(len(old), len(new))
    if old[:n] == new[:n]:
        return n
    # Usually only the last block or two differ (copy-on-write of the block being written).
    lo, hi = 0, n
    while hi - lo > 1:  # invariant: old[:lo] == new[:lo], old[:hi] != new[:hi]
        mid = (lo + hi) // 2
        if old[:mid] == new[:mid]:
            lo = mid
        else:
            hi = mid
    return lo
