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

from paged_kv_serving_amd import _native

__all__ = ["BlockTableArena", "TableUpdate"]


class TableUpdate:
    """What one iteration changes: the arena row of every entry, and the flat (row * width +
    column) indices and values of the table entries to write on the device. The arrays are views
    of the arena's buffers, valid until its next update."""

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
        # How many leading entries of each host row the device row is known to hold, and the
        # tuple each row was last filled from (None: compare by value).
        self._held_len = np.zeros(rows, dtype=np.int32)
        self._held_obj: list[object] = [None] * rows
        self._last_use = np.zeros(rows, dtype=np.int64)
        self._step = 0
        # Rows an update touched whose device copy no apply() has written yet. If the caller
        # fails between the two, the next update forgets what they hold.
        self._none = np.zeros(0, dtype=np.int32)
        self._unapplied = self._none
        self._index = np.zeros(1024, dtype=np.int64)
        self._values = np.zeros(1024, dtype=np.int32)
        self._rows = np.zeros(64, dtype=np.int32)
        self._host_ext = _native.host()

    @property
    def num_rows(self) -> int:
        return self.host.shape[0]

    @property
    def width(self) -> int:
        return self.host.shape[1]

    @property
    def held_lengths(self) -> np.ndarray:
        """int32 per row: how many leading entries of the host row are the row's table."""
        return self._held_len

    def held(self, row: int) -> tuple[int, ...]:
        """The table arena row ``row`` currently holds."""
        return tuple(self.host[row, : self._held_len[row]].tolist())

    def update(self, entries) -> TableUpdate:
        """Assign a row to every entry (by ``seq_id``) and record the table entries that differ
        from what the row holds. The host mirror is updated at once; the device rows change when
        the returned indices and values are applied with :meth:`apply`. If the previous update
        was never applied (its caller raised in between), the rows it touched are treated as
        holding nothing, so their whole tables are uploaded again.

        The walk over the entries runs in C++ (``_pkvhost.arena_update``): a sequence not seen
        before claims the least recently used row not used in this iteration, the same sequence
        twice in one batch gets a row per occurrence, and only the entries from the first one
        that differs from the row's content travel."""
        if self._unapplied.size:
            self._held_len[self._unapplied] = 0
            for row in self._unapplied.tolist():
                self._held_obj[row] = None
            self._unapplied = self._none
        self._step += 1
        count = len(entries)
        if self._rows.size < count:
            self._rows = np.zeros(max(count, 2 * self._rows.size), dtype=np.int32)
        while True:
            changed, extra = self._host_ext.arena_update(
                entries, self._row_of, self._key_of, self._held_len, self._held_obj, self._last_use, self.host,
                self._step, self._rows, self._index, self._values,
            )  # fmt: skip
            if changed == -1:  # more rows or a wider table than the arena has
                self._grow(max(count, self.num_rows), extra)
            elif changed == -2:  # the index/values buffers may be too small
                self._index = np.zeros(max(extra, 2 * self._index.size), dtype=np.int64)
                self._values = np.zeros(max(extra, 2 * self._values.size), dtype=np.int32)
            else:
                break
        # Views of the reused buffers: the caller consumes them before its next update (which
        # reads _unapplied before rewriting them).
        rows = self._rows[:count]
        self._unapplied = rows
        return TableUpdate(rows, self._index[:changed], self._values[:changed])

    def apply(self, index: torch.Tensor, values: torch.Tensor) -> None:
        """Write an update's values (device int32) at its flat indices (device int64)."""
        if index.numel():
            self.tables.view(-1).index_copy_(0, index, values)
        self._unapplied = self._none

    def apply_nothing(self) -> None:
        """Record that an update with no changed entries has been applied."""
        self._unapplied = self._none

    def used_blocks(self, rows: np.ndarray, block_counts: np.ndarray) -> np.ndarray:
        """The first ``block_counts[i]`` table entries of arena row ``rows[i]``, concatenated."""
        if rows.size == 0:
            return np.zeros(0, dtype=np.int32)
        counts = np.minimum(np.asarray(block_counts, dtype=np.int64), self.width)
        mask = np.arange(self.width)[None, :] < counts[:, None]
        return self.host[rows][mask]

    # --- rows ----------------------------------------------------------------------------

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
        self._held_len = np.concatenate([self._held_len, np.zeros(extra, dtype=np.int32)])
        self._held_obj.extend([None] * extra)
        self._last_use = np.concatenate([self._last_use, np.zeros(extra, dtype=np.int64)])
        self.host = host
        self.tables = tables
