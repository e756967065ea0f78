"""Prefix cache: chained content hash of each FULL block -> physical block.

Same scheme and API as the reference (inference_server/core/prefix_cache.py:57-193):
block i's key is blake2b-128(key of block i-1 or 16 zero bytes, the block's token ids
as little-endian int64), so equal keys mean equal full prefixes. Only full blocks are
shared, so a sequence adopting n blocks starts writing at a block boundary in a
private block and copy-on-write never triggers under this policy. Entries die with
their block (allocator on_release).
"""

from __future__ import annotations

import hashlib

import numpy as np

from inference_server.core.block_allocator import BlockAllocator
from inference_server.core.block_table import BlockTable

_DIGEST = 16
_ROOT = b"\x00" * _DIGEST


def block_hash(prev: bytes | None, tokens: list[int]) -> bytes:
    h = hashlib.blake2b(prev if prev is not None else _ROOT, digest_size=_DIGEST)
    h.update(np.asarray(tokens, dtype="<i8").tobytes())
    return h.digest()


def hash_chain(tokens: list[int], block_size: int, prefix: list[bytes] = ()) -> list[bytes]:
    """Keys of every full block of `tokens`, continuing from known keys `prefix`."""
    chain = list(prefix)
    prev = chain[-1] if chain else None
    for i in range(len(chain), len(tokens) // block_size):
        prev = block_hash(prev, tokens[i * block_size:(i + 1) * block_size])
        chain.append(prev)
    return chain


class PrefixCache:
    def __init__(self, allocator: BlockAllocator, block_size: int) -> None:
        self.allocator = allocator
        self.block_size = block_size
        self._block_of: dict[bytes, int] = {}
        self._key_of: dict[int, bytes] = {}
        self.hits = 0
        self.misses = 0
        self.blocks_shared = 0
        allocator.on_release = self._forget

    @property
    def entries(self) -> int:
        return len(self._block_of)

    def match(self, tokens: list[int]) -> tuple[list[int], list[bytes]]:
        """Longest cached run of full blocks at the start of `tokens`, capped so at
        least the last token is still fed through the model. No side effects."""
        limit = max(0, (len(tokens) - 1) // self.block_size)
        blocks: list[int] = []
        keys: list[bytes] = []
        prev = None
        for i in range(limit):
            prev = block_hash(prev, tokens[i * self.block_size:(i + 1) * self.block_size])
            block = self._block_of.get(prev)
            if block is None:
                break
            blocks.append(block)
            keys.append(prev)
        return blocks, keys

    def claim(self, table: BlockTable, blocks: list[int], hashes: list[bytes], full_blocks: int) -> int:
        """Adopt matched blocks into an empty table; returns tokens now covered."""
        assert not table.blocks, "prefix match applies to an empty table only"
        table.adopt(blocks, hashes)
        self.hits += len(blocks)
        self.blocks_shared += len(blocks)
        self.misses += max(0, full_blocks - len(blocks))
        return len(blocks) * self.block_size

    def register(self, table: BlockTable, tokens: list[int], num_cached: int) -> int:
        """Publish the table's newly completed full blocks; returns how many were new.
        `table.published` is the first block not known to be cached as ours."""
        full = min(num_cached, len(tokens)) // self.block_size
        if full <= table.published:
            return 0
        if full > len(table.hashes):
            table.hashes = hash_chain(tokens[:full * self.block_size], self.block_size, table.hashes)
        published = 0
        advancing = True
        for i in range(table.published, full):
            key, block = table.hashes[i], table.blocks[i]
            if key not in self._block_of:
                if block in self._key_of:
                    raise RuntimeError(f"block {block} registered under two hashes")
                self._block_of[key] = block
                self._key_of[block] = key
                published += 1
            if advancing and self._block_of[key] == block:
                table.published = i + 1
            else:
                # Someone else's copy of this content is the cached one: recheck this
                # block on a later step (it is ours to publish once theirs is gone).
                advancing = False
        return published

    def _forget(self, block: int) -> None:
        key = self._key_of.pop(block, None)
        if key is not None:
            del self._block_of[key]

    def stats(self) -> dict:
        return {
            "prefix_hits": self.hits,
            "prefix_misses": self.misses,
            "prefix_blocks_shared": self.blocks_shared,
            "prefix_entries": self.entries,
            "prefix_tokens_saved": self.blocks_shared * self.block_size,
        }

    def __repr__(self) -> str:
        return f"PrefixCache({self.entries} entries, {self.hits} hits, {self.misses} misses)"
