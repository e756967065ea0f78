"""One sequence's logical -> physical block map.

API of the reference's BlockTable (inference_server/core/block_table.py:38-186).
Logical position p lives in block blocks[p // bs] at offset p % bs; its flat slot is
blocks[p // bs] * bs + p % bs, the row index of the pool viewed as [NB * bs, Hkv, D].
`ensure_private` is the copy-on-write guard; the byte copy itself is the pool's
(PagedKVPool.copy_block, one launch over every layer on the hip backend).
"""

from __future__ import annotations

from typing import Callable

from inference_server.config import CONFIG
from inference_server.core.block_allocator import BlockAllocator


class BlockTable:
    def __init__(self, allocator: BlockAllocator, block_size: int = CONFIG.block_size) -> None:
        self.allocator = allocator
        self.block_size = block_size
        self.blocks: list[int] = []
        #: Chained content hashes of the FULL blocks, in order (prefix cache).
        self.hashes: list[bytes] = []
        #: Blocks below this index are known to be in the prefix cache.
        self.published: int = 0

    @property
    def capacity(self) -> int:
        return len(self.blocks) * self.block_size

    @property
    def num_blocks(self) -> int:
        return len(self.blocks)

    def blocks_for(self, num_tokens: int) -> int:
        """ceil(num_tokens / block_size) without floats: 17 -> 2, 16 -> 1."""
        return -(-num_tokens // self.block_size)

    def ensure_capacity(self, num_tokens: int) -> list[int]:
        """Grow to hold num_tokens slots; returns the new blocks. MemoryError if the
        pool cannot supply them (nothing is taken in that case)."""
        missing = self.blocks_for(num_tokens) - len(self.blocks)
        if missing <= 0:
            return []
        fresh = self.allocator.allocate_many(missing)
        self.blocks.extend(fresh)
        return fresh

    def adopt(self, blocks: list[int], hashes: list[bytes]) -> None:
        """Point an EMPTY table at shared full blocks, one reference each."""
        if self.blocks:
            raise ValueError("adopt() onto a non-empty table; prefix sharing is prefix-only")
        if len(hashes) != len(blocks):
            raise ValueError(f"{len(blocks)} blocks with {len(hashes)} hashes")
        for block in blocks:
            self.allocator.incref(block)
        self.blocks.extend(blocks)
        self.hashes.extend(hashes)

    def ensure_private(self, logical: int, copy: Callable[[int, int], None] | None = None) -> tuple[int, int] | None:
        """Copy-on-write before a write into logical block `logical`: if another
        sequence also references it, move to a fresh copy. Returns (src, dst) when a
        copy happened, None when the block was already private."""
        if not 0 <= logical < len(self.blocks):
            raise IndexError(f"logical block {logical} outside [0, {len(self.blocks)})")
        src = self.blocks[logical]
        if self.allocator.refcount(src) <= 1:
            return None
        dst = self.allocator.allocate()
        if copy is not None:
            copy(src, dst)
        self.allocator.free(src)
        self.blocks[logical] = dst
        return src, dst

    def slot(self, position: int) -> tuple[int, int]:
        if not 0 <= position < self.capacity:
            raise IndexError(f"position {position} outside [0, {self.capacity})")
        return self.blocks[position // self.block_size], position % self.block_size

    def slots(self, num_tokens: int) -> list[int]:
        """Flat slots of the first num_tokens positions."""
        return self.slot_range(0, num_tokens)

    def slot_range(self, start: int, stop: int) -> list[int]:
        """Flat slots of positions start..stop-1 (only those — O(stop - start))."""
        if stop > self.capacity:
            raise IndexError(f"{stop} tokens requested, capacity is {self.capacity}")
        bs = self.block_size
        return [self.blocks[p // bs] * bs + p % bs for p in range(start, stop)]

    def free(self) -> None:
        """Return every block (idempotent)."""
        if not self.blocks:
            return
        self.allocator.free_many(self.blocks)
        self.blocks = []
        self.hashes = []
        self.published = 0

    def waste(self, num_tokens: int) -> int:
        return self.capacity - num_tokens

    def __len__(self) -> int:
        return len(self.blocks)

    def __repr__(self) -> str:
        return f"BlockTable({len(self.blocks)} blocks, {self.capacity} slots)"
