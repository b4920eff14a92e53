"""Block tables resident on the device, one row per running sequence.

The reference rebuilds every sequence's -1 padded table on the host each
decode step and copies it row by row (minivllm/model_runner.py:176-201). A
sequence's table only changes when it gains a block (every S steps) or when it
is preempted and later recomputed into new blocks, so here each step sends
only the entries that changed:

* the device tensor ``table [rows, cols]`` holds one row per sequence; row 0
  is never assigned and stays all -1 (padding rows of a batch gather it);
* ``_shadow[r]`` is a host copy of the entries row r holds; entries past it
  are -1. Every upload keeps that invariant, and the comparison of a
  sequence's live table with its shadow is an exact list comparison, so a
  table rewritten in place (preemption, recompute, external edits) is
  re-uploaded in full;
* ``stage`` returns the batch's row ids and the (row, col, value) updates,
  which the caller packs into its one host-to-device copy; ``apply`` writes
  the updates with one index_put_ and ``gather`` / ``gather_into`` build the
  batch's [B, M] table with one index_select.

Rows of sequences that left the batch stay cached until their row is needed
(least recently used first); the table grows when a batch needs more rows or
a table more columns than it has.
"""
from __future__ import annotations

import torch


class DeviceBlockTables:
    def __init__(self, device, rows: int = 256, cols: int = 64):
        self.device = torch.device(device)
        self.table = torch.full((rows + 1, max(1, cols)), -1, dtype=torch.int64, device=self.device)
        self._row: dict[str, int] = {}        # seq_id -> row
        self._owner: dict[int, str] = {}      # row -> seq_id
        self._shadow: dict[int, list[int]] = {}
        self._used: dict[int, int] = {}       # row -> step it was last staged in
        self._free = list(range(rows, 0, -1))
        self._step = 0

    @property
    def rows(self) -> int:
        return self.table.shape[0] - 1

    @property
    def cols(self) -> int:
        return self.table.shape[1]

    def _grow(self, rows: int, cols: int) -> None:
        R, C = self.table.shape
        new = torch.full((max(rows + 1, R), max(cols, C)), -1, dtype=torch.int64, device=self.device)
        new[:R, :C] = self.table
        self._free = list(range(new.shape[0] - 1, R - 1, -1)) + self._free
        self.table = new

    def _assign(self, seq_id: str) -> int:
        if not self._free:
            stale = [r for r, s in self._used.items() if s < self._step]
            if stale:
                r = min(stale, key=self._used.__getitem__)
                del self._row[self._owner.pop(r)]
                del self._used[r]
                self._free.append(r)          # its shadow still describes the device row
            else:
                self._grow(2 * self.rows, self.cols)
        r = self._free.pop()
        self._row[seq_id] = r
        self._owner[r] = seq_id
        self._shadow.setdefault(r, [])
        return r

    def stage(self, seq_ids, tables) -> tuple[list[int], list[int]]:
        """Row ids of this batch and the flat [row, col, value, ...] updates
        that make each row equal its table. Updates are applied with
        ``apply`` before the next ``gather``."""
        self._step += 1
        widest = max((len(t) for t in tables), default=0)
        if widest > self.cols:
            self._grow(self.rows, max(widest, 2 * self.cols))
        rows: list[int] = []
        upd: list[int] = []
        for sid, t in zip(seq_ids, tables):
            r = self._row.get(sid)
            if r is None:
                r = self._assign(sid)
            self._used[r] = self._step
            rows.append(r)
            prev = self._shadow[r]
            if t == prev:
                continue
            n = len(prev)
            if len(t) >= n and t[:n] == prev:
                first = n
            else:
                first = 0
                for c in range(len(t), n):
                    upd += (r, c, -1)
            for c in range(first, len(t)):
                upd += (r, c, t[c])
            self._shadow[r] = list(t)
        return rows, upd

    def apply(self, upd: torch.Tensor) -> None:
        """Writes flat (row, col, value) triples, an int64 device tensor."""
        if upd.numel():
            u = upd.view(-1, 3)
            self.table.index_put_((u[:, 0], u[:, 1]), u[:, 2])

    def gather(self, rows: torch.Tensor, M: int) -> torch.Tensor:
        """The batch's -1 padded tables, a new contiguous [len(rows), M] tensor."""
        if M > self.cols:
            self._grow(self.rows, M)
        return self.table[:, :M].index_select(0, rows)

    def gather_into(self, rows: torch.Tensor, out: torch.Tensor) -> None:
        """gather(rows, out.shape[1]) written into ``out`` (contiguous)."""
        if out.shape[1] > self.cols:
            self._grow(self.rows, out.shape[1])
        torch.index_select(self.table[:, :out.shape[1]], 0, rows, out=out)
