"""Physical KV blocks of the pool: who holds them and which are free.

Behaviour the rest of the engine relies on (reference contract:
inference_server/core/block_allocator.py:38-130): a block is handed out with one
reference; `incref` adds a holder (prefix sharing); a block returns to the free set
when its last holder lets go, and `on_release(block)` is told before it can be handed
out again (the prefix cache drops its index entry there). Asking for more blocks than
are free raises MemoryError and takes nothing (the scheduler preempts on it); a
double free, an incref of a free block, or an index outside the pool raise.

Representation: the reference keeps Python lists; here the reference counts are one
int32 numpy array and the free set is a stack in an int64 numpy array with a top index.
Taking n blocks is one slice, returning a table's blocks is one vectorised update, and
the counts can be read in bulk (`refcounts`), which is how the executor finds the
shared blocks a step is about to write without a per-block Python call. The stack
hands out low indices first on a fresh pool and reuses the most recently freed block
first.
"""

from __future__ import annotations

from typing import Callable, Iterable

import numpy as np


class BlockAllocator:
    def __init__(self, num_blocks: int) -> None:
        if num_blocks <= 0:
            raise ValueError(f"num_blocks must be positive, got {num_blocks}")
        self.num_blocks = int(num_blocks)
        self._refs = np.zeros(self.num_blocks, dtype=np.int32)
        # Free stack: entries [0, _top) are free, the top of the stack is handed out next.
        self._stack = np.arange(self.num_blocks - 1, -1, -1, dtype=np.int64)
        self._top = self.num_blocks
        #: Called with a block id when its count reaches zero, before it can be reused.
        self.on_release: Callable[[int], None] | None = None

    # ------------------------------------------------------------------ queries
    @property
    def num_free(self) -> int:
        return self._top

    @property
    def num_allocated(self) -> int:
        return self.num_blocks - self._top

    def refcount(self, block: int) -> int:
        return int(self._refs[self._index(block)])

    def refcounts(self, blocks: np.ndarray) -> np.ndarray:
        """Reference counts of many blocks at once (no bounds check: callers pass ids
        they hold)."""
        return self._refs[blocks]

    # ------------------------------------------------------------------ taking
    def allocate(self) -> int:
        """One block, held once. MemoryError when none is free (the scheduler's
        preemption trigger; nothing is taken)."""
        if self._top == 0:
            raise MemoryError(f"block pool exhausted ({self.num_blocks} blocks, all held)")
        self._top -= 1
        block = int(self._stack[self._top])
        self._refs[block] = 1
        return block

    def allocate_many(self, count: int) -> list[int]:
        """`count` blocks or none: capacity is checked before anything is taken."""
        if count < 0:
            raise ValueError(f"count must be non-negative, got {count}")
        if count > self._top:
            raise MemoryError(f"need {count} blocks, {self._top} free")
        if count == 0:
            return []
        taken = self._stack[self._top - count:self._top][::-1].copy()
        self._top -= count
        self._refs[taken] = 1
        return taken.tolist()

    def incref(self, block: int) -> int:
        """Another holder of a held block (prefix sharing)."""
        b = self._index(block)
        if self._refs[b] == 0:
            raise ValueError(f"incref on free block {b} — use-after-free")
        self._refs[b] += 1
        return int(self._refs[b])

    # ------------------------------------------------------------------ returning
    def free(self, block: int) -> int:
        """Drop one holder; at zero the block is released. Returns the new count."""
        b = self._index(block)
        if self._refs[b] == 0:
            raise ValueError(f"double free of block {b}")
        self._refs[b] -= 1
        if self._refs[b] == 0:
            self._release(b)
        return int(self._refs[b])

    def free_many(self, blocks: Iterable[int]) -> None:
        """Drop one holder of each listed block (a block listed twice loses two), in
        one vectorised check-and-update; released blocks go back in list order."""
        ids = np.asarray(list(blocks) if not isinstance(blocks, np.ndarray) else blocks, dtype=np.int64)
        if ids.size == 0:
            return
        if ids.min() < 0 or ids.max() >= self.num_blocks:
            bad = ids[(ids < 0) | (ids >= self.num_blocks)][0]
            raise IndexError(f"block {int(bad)!r} outside [0, {self.num_blocks})")
        uniq, counts = np.unique(ids, return_counts=True)
        short = self._refs[uniq] < counts
        if short.any():
            raise ValueError(f"double free of block {int(uniq[short][0])}")
        np.subtract.at(self._refs, ids, 1)
        if (self._refs[uniq] == 0).any():
            seen = set()
            for b in ids.tolist():
                if self._refs[b] == 0 and b not in seen:
                    seen.add(b)
                    self._release(b)

    # ------------------------------------------------------------------ internals
    def _release(self, block: int) -> None:
        if self.on_release is not None:
            self.on_release(block)
        self._stack[self._top] = block
        self._top += 1

    def _index(self, block) -> int:
        if isinstance(block, (bool, np.bool_)) or not isinstance(block, (int, np.integer)) \
                or not 0 <= block < self.num_blocks:
            raise IndexError(f"block {block!r} outside [0, {self.num_blocks})")
        return int(block)

    def __repr__(self) -> str:
        return f"BlockAllocator({self.num_allocated}/{self.num_blocks} held)"
