"""Physical block indices: a LIFO free list with per-block reference counts.

Same API and invariants as the reference allocator
(inference_server/core/block_allocator.py:65-117): a block is on the free list iff
its refcount is 0; `allocate_many` is all-or-nothing; a double free or an incref of a
free block raises; `on_release(block)` fires when a refcount reaches 0, before the
block is reusable (the prefix cache drops its entry there). Integers only.
"""

from __future__ import annotations

from typing import Callable


class BlockAllocator:
    def __init__(self, num_blocks: int) -> None:
        if num_blocks <= 0:
            raise ValueError(f"num_blocks must be positive, got {num_blocks}")
        self.num_blocks = num_blocks
        # Popped from the end: block 0 is handed out first, and the most recently
        # freed block is the next one reused.
        self._free: list[int] = list(range(num_blocks - 1, -1, -1))
        self._refs: list[int] = [0] * num_blocks
        self.on_release: Callable[[int], None] | None = None

    @property
    def num_free(self) -> int:
        return len(self._free)

    @property
    def num_allocated(self) -> int:
        return self.num_blocks - len(self._free)

    def refcount(self, block: int) -> int:
        return self._refs[self._valid(block)]

    def allocate(self) -> int:
        """One block with refcount 1; MemoryError when none is free (the preemption
        trigger, never a crash)."""
        if not self._free:
            raise MemoryError(f"block pool exhausted ({self.num_blocks} blocks, all held)")
        block = self._free.pop()
        self._refs[block] = 1
        return block

    def allocate_many(self, count: int) -> list[int]:
        if count < 0:
            raise ValueError(f"count must be non-negative, got {count}")
        if count > len(self._free):
            raise MemoryError(f"need {count} blocks, {len(self._free)} free")
        return [self.allocate() for _ in range(count)]

    def incref(self, block: int) -> int:
        self._valid(block)
        if self._refs[block] == 0:
            raise ValueError(f"incref on free block {block} — use-after-free")
        self._refs[block] += 1
        return self._refs[block]

    def free(self, block: int) -> int:
        self._valid(block)
        if self._refs[block] == 0:
            raise ValueError(f"double free of block {block}")
        self._refs[block] -= 1
        if self._refs[block] == 0:
            if self.on_release is not None:
                self.on_release(block)
            self._free.append(block)
        return self._refs[block]

    def free_many(self, blocks: list[int]) -> None:
        for block in blocks:
            self.free(block)

    def _valid(self, block: int) -> int:
        if not isinstance(block, int) or not 0 <= block < self.num_blocks:
            raise IndexError(f"block {block!r} outside [0, {self.num_blocks})")
        return block

    def __repr__(self) -> str:
        return f"BlockAllocator({self.num_allocated}/{self.num_blocks} held)"
