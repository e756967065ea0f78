"""One sequence's block table: logical block i of its context -> physical pool block.

Contract with the kernels and the reference (inference_server/core/block_table.py:
70-76, 110-159): token position p lives at flat slot `ids[p // bs] * bs + p % bs` of
the pool viewed as [num_blocks * bs, Hkv, D]; a table grows by whole blocks
(`ensure_capacity` takes ceil(tokens / bs) - held, all or nothing, MemoryError when
the pool is short); `ensure_private` is the copy-on-write guard that moves a shared
block to a private copy through the `copy(src, dst)` hook before it is written.

Representation: the ids live in a growable int64 numpy row, which is what the
executor copies into its per-step block-table tensors (a slice copy, no per-block
Python work), and every change of the ids takes a new `version` stamp. A holder of a
device copy of the row (the decode-step graphs' persistent metadata) compares stamps
and rewrites only the rows that changed since its last upload.
"""

from __future__ import annotations

import itertools
from typing import Callable

import numpy as np

from inference_server.config import CONFIG
from inference_server.core.block_allocator import BlockAllocator

_INITIAL = 8
#: Version stamps are drawn from one process-wide counter, so a stamp names one state
#: of one table: a cache keyed by stamps cannot confuse a new table with a dead one.
_STAMPS = itertools.count(1)


class BlockTable:
    def __init__(self, allocator: BlockAllocator, block_size: int = CONFIG.block_size) -> None:
        self.allocator = allocator
        self.block_size = int(block_size)
        self._ids = np.zeros(_INITIAL, dtype=np.int64)
        self._n = 0
        #: A fresh stamp on every change of the block ids (growth, adoption, remap, free).
        self.version = next(_STAMPS)
        #: Full blocks already offered to the prefix cache (its cursor; reset by free()).
        self.registered = 0

    # ------------------------------------------------------------------ views
    @property
    def ids(self) -> np.ndarray:
        """The held block ids in logical order (a view; do not modify)."""
        return self._ids[:self._n]

    @property
    def blocks(self) -> list[int]:
        return self._ids[:self._n].tolist()

    @property
    def num_blocks(self) -> int:
        return self._n

    def __len__(self) -> int:
        return self._n

    @property
    def capacity(self) -> int:
        """Token slots held, used or not."""
        return self._n * self.block_size

    def blocks_for(self, num_tokens: int) -> int:
        """Blocks that hold num_tokens tokens: ceiling division in integers (16 tokens
        of 16 per block need 1 block, 17 need 2)."""
        return (num_tokens + self.block_size - 1) // self.block_size

    def waste(self, num_tokens: int) -> int:
        """Held slots past num_tokens (at most block_size - 1 while the table is
        sized by ensure_capacity)."""
        return self.capacity - num_tokens

    # ------------------------------------------------------------------ growth
    def _append(self, new: list[int]) -> None:
        need = self._n + len(new)
        if need > self._ids.size:
            grown = np.zeros(max(need, 2 * self._ids.size), dtype=np.int64)
            grown[:self._n] = self._ids[:self._n]
            self._ids = grown
        self._ids[self._n:need] = new
        self._n = need
        self.version = next(_STAMPS)

    def ensure_capacity(self, num_tokens: int) -> list[int]:
        """Hold at least num_tokens slots; returns the newly taken blocks (empty when
        the table is already big enough). MemoryError, with nothing taken, when the
        pool cannot supply them."""
        short = self.blocks_for(num_tokens) - self._n
        if short <= 0:
            return []
        fresh = self.allocator.allocate_many(short)
        self._append(fresh)
        return fresh

    def adopt(self, blocks: list[int]) -> None:
        """Start an empty table on blocks another holder already holds (a prefix-cache
        match), taking one reference on each."""
        if self._n:
            raise ValueError("adopt() onto a non-empty table; prefix sharing is prefix-only")
        for b in blocks:
            self.allocator.incref(b)
        self._append(list(blocks))

    # ------------------------------------------------------------------ copy-on-write
    def ensure_private(self, logical: int, copy: Callable[[int, int], None] | None = None) -> tuple[int, int] | None:
        """Make logical block `logical` this table's alone before it is written: if the
        block has other holders, take a fresh block, let copy(src, dst) move the bytes,
        drop this table's reference on src and point the entry at dst. Returns (src,
        dst) when a copy was made, None when the block was already private."""
        if not 0 <= logical < self._n:
            raise IndexError(f"logical block {logical} outside [0, {self._n})")
        src = int(self._ids[logical])
        if self.allocator.refcount(src) <= 1:
            return None
        dst = self.allocator.allocate()
        if copy is not None:
            copy(src, dst)
        self.allocator.free(src)
        self._ids[logical] = dst
        self.version = next(_STAMPS)
        return src, dst

    def make_writable(self, start: int, stop: int, copy: Callable[[int, int], None]) -> None:
        """ensure_private for every block holding positions start..stop-1, with one
        bulk reference-count read to find the shared ones (usually none)."""
        if stop <= start:
            return
        lo, hi = start // self.block_size, (stop - 1) // self.block_size + 1
        if hi - lo == 1:                                  # one block (every decode pass)
            if self.allocator.refcount(int(self._ids[lo])) > 1:
                self.ensure_private(lo, copy)
            return
        shared = np.nonzero(self.allocator.refcounts(self._ids[lo:hi]) > 1)[0]
        for i in shared.tolist():
            self.ensure_private(lo + i, copy)

    # ------------------------------------------------------------------ addressing
    def slot(self, position: int) -> tuple[int, int]:
        """(physical block, offset) of a token position."""
        if not 0 <= position < self.capacity:
            raise IndexError(f"position {position} outside [0, {self.capacity})")
        return int(self._ids[position // self.block_size]), position % self.block_size

    def slot_of(self, position: int) -> int:
        """Flat pool slot of one held position (no bounds check; callers pass
        positions below `capacity`)."""
        bs = self.block_size
        return int(self._ids[position // bs]) * bs + position % bs

    def slot_range(self, start: int, stop: int) -> np.ndarray:
        """Flat pool slots of positions start..stop-1 (int64; O(stop - start))."""
        if stop > self.capacity:
            raise IndexError(f"{stop} tokens requested, capacity is {self.capacity}")
        bs = self.block_size
        if stop - start == 1:
            return np.array([self._ids[start // bs] * bs + start % bs], dtype=np.int64)
        pos = np.arange(start, stop, dtype=np.int64)
        return self._ids[pos // bs] * bs + pos % bs

    def slots(self, num_tokens: int) -> np.ndarray:
        """Flat slots of the first num_tokens positions."""
        return self.slot_range(0, num_tokens)

    # ------------------------------------------------------------------ release
    def free(self) -> None:
        """Return every held block (a no-op on an empty table)."""
        if not self._n:
            return
        held = self._ids[:self._n].copy()
        self._n = 0
        self.registered = 0
        self.version = next(_STAMPS)
        self.allocator.free_many(held)

    def __repr__(self) -> str:
        return f"BlockTable({self._n} blocks, {self.capacity} slots)"
