"""Prefix cache: pool blocks whose K/V were computed over a known full-block prefix,
found by content key so that a new request can start on them instead of prefilling.

Key (the reference's, inference_server/core/prefix_cache.py:53-82, kept so that equal
histories share the same blocks): block i of a history has key
blake2b-128(key of block i-1, or 16 zero bytes for block 0 || the block's token ids as
little-endian int64). A key therefore covers every token from position 0 to the end
of the block, and equal keys mean interchangeable K/V. Only full blocks get keys, so a
sequence that starts on n cached blocks writes its first token at a block boundary,
into a block of its own.

Rules (reference prefix_cache.py:86-193): a match never covers a request's last token
(the model must see it to produce a logit); an entry lives exactly as long as its
block is held (the allocator's on_release removes it before the block can be reused).

Design here:
* Keys are computed once per block of a history and kept on the Sequence
  (`Sequence.prefix_keys`), extended as the history grows; matching a queued request
  again on a later step costs dictionary lookups, not hashing.
* When two held blocks carry the same key (two requests prefilled the same prefix in
  one pass), one is indexed and the others are kept as spares of that key; when the
  indexed block is released a spare takes its place at once, so the entry survives as
  long as any holder of that content does.
* `register` walks each table's newly completed full blocks once: the table's
  `registered` cursor only moves forward (reset when the table is freed).
"""

from __future__ import annotations

import hashlib

import numpy as np

from inference_server.core.block_allocator import BlockAllocator
from inference_server.core.block_table import BlockTable

KEY_BYTES = 16
_ROOT = bytes(KEY_BYTES)


def block_key(prev: bytes | None, tokens) -> bytes:
    """The key of one full block given its predecessor's key (None for block 0)."""
    h = hashlib.blake2b(prev if prev is not None else _ROOT, digest_size=KEY_BYTES)
    h.update(np.asarray(tokens, dtype="<i8").tobytes())
    return h.digest()


def chain_keys(tokens: list[int], block_size: int, keys: list[bytes] | None = None,
               upto: int | None = None) -> list[bytes]:
    """Extend `keys` (the keys of the first len(keys) blocks of `tokens`, extended in
    place; a new list if None) to cover the first `upto` full blocks (every full block
    if None). Returns the list."""
    keys = [] if keys is None else keys
    full = len(tokens) // block_size
    stop = full if upto is None else min(upto, full)
    prev = keys[-1] if keys else None
    for i in range(len(keys), stop):
        prev = block_key(prev, tokens[i * block_size:(i + 1) * block_size])
        keys.append(prev)
    return keys


class PrefixCache:
    def __init__(self, allocator: BlockAllocator, block_size: int) -> None:
        self.allocator = allocator
        self.block_size = int(block_size)
        self._index: dict[bytes, int] = {}                # key -> the block that serves it
        self._spares: dict[bytes, list[int]] = {}         # key -> other held blocks with that content
        self._key_of: list[bytes | None] = [None] * allocator.num_blocks
        # Cumulative counters, in full prompt blocks seen by `claim`: an admission that
        # matched nothing is not counted (reference prefix_cache.py:121-129 counts misses
        # only when a match is claimed).
        self.hits = 0
        self.misses = 0
        self.blocks_shared = 0
        allocator.on_release = self._released

    @property
    def entries(self) -> int:
        return len(self._index)

    # ------------------------------------------------------------------ admission
    def _keys(self, seq, upto: int) -> list[bytes]:
        return chain_keys(seq.tokens, self.block_size, seq.prefix_keys, upto)

    def match(self, seq) -> list[int]:
        """Blocks serving the longest cached run of full blocks at the start of the
        sequence's history, stopping before the block holding its last token. No side
        effects (admission may still decline)."""
        limit = (seq.total_len - 1) // self.block_size
        found: list[int] = []
        if limit <= 0:
            return found
        keys = self._keys(seq, limit)
        for key in keys[:limit]:
            block = self._index.get(key)
            if block is None:
                break
            found.append(block)
        return found

    def claim(self, seq, blocks: list[int]) -> int:
        """Start the sequence's (empty) table on the matched blocks and count the
        admission; returns the number of tokens now cached."""
        table = seq.block_table
        table.adopt(blocks)
        table.registered = len(blocks)
        full = (seq.total_len - 1) // self.block_size
        self.hits += len(blocks)
        self.blocks_shared += len(blocks)
        self.misses += max(0, full - len(blocks))
        return len(blocks) * self.block_size

    # ------------------------------------------------------------------ publication
    def register(self, seq) -> int:
        """Offer the table's newly completed full blocks (those entirely below
        num_cached) to the cache; returns how many became index entries."""
        table: BlockTable | None = seq.block_table
        if table is None:
            return 0
        full = min(seq.num_cached, seq.total_len) // self.block_size
        if full <= table.registered:
            return 0
        keys = self._keys(seq, full)
        ids = table.ids
        added = 0
        for i in range(table.registered, full):
            key, block = keys[i], int(ids[i])
            held = self._key_of[block]
            if held is not None:
                if held != key:
                    raise RuntimeError(f"block {block} registered under two keys")
                continue                                  # already indexed or a spare
            self._key_of[block] = key
            if key in self._index:
                self._spares.setdefault(key, []).append(block)
            else:
                self._index[key] = block
                added += 1
        table.registered = full
        return added

    def _released(self, block: int) -> None:
        """Allocator callback: the block's last holder let go."""
        key = self._key_of[block]
        if key is None:
            return
        self._key_of[block] = None
        spares = self._spares.get(key)
        if self._index.get(key) == block:
            if spares:
                self._index[key] = spares.pop()
            else:
                del self._index[key]
        elif spares is not None:
            spares.remove(block)
        if spares is not None and not spares:
            del self._spares[key]

    # ------------------------------------------------------------------ metrics
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
