"""Oracle: slot arithmetic and the KV byte movers, restated in numpy.

Test infrastructure only (see oracle/__init__.py). Every function works on numpy
arrays of any dtype (bf16 data is handled as its raw uint16 words, so results are
compared bit for bit) and returns new arrays rather than mutating its inputs.
"""

from __future__ import annotations

import numpy as np


def slots_for(blocks: list[int], block_size: int, num_tokens: int) -> np.ndarray:
    """Flat slots of a sequence's first num_tokens positions: blocks[p // bs] * bs +
    p % bs (reference core/block_table.py:143-159)."""
    p = np.arange(num_tokens, dtype=np.int64)
    return np.asarray(blocks, dtype=np.int64)[p // block_size] * block_size + p % block_size


def kv_append(pool: np.ndarray, new_rows: np.ndarray, slots: np.ndarray) -> np.ndarray:
    """pool [NB, bs, Hkv, D] with row t of new_rows [T, Hkv, D] written at flat slot
    slots[t] — `pool.view(-1, H, D).index_copy_(0, slots, rows)` of reference
    core/paged_executor.py:116-125. Slots are distinct."""
    nb, bs = pool.shape[:2]
    out = pool.copy()
    flat = out.reshape(nb * bs, *pool.shape[2:])
    flat[np.asarray(slots, dtype=np.int64)] = new_rows
    return out


def copy_blocks(pool: np.ndarray, pairs: list[tuple[int, int]]) -> np.ndarray:
    """pool with block dst replaced by block src for every pair — the per-layer
    `layer[dst].copy_(layer[src])` of reference core/paged_executor.py:265-270. Sources
    are read before any destination is written (no dst is another pair's src)."""
    out = pool.copy()
    src = np.array([s for s, _ in pairs], dtype=np.int64)
    dst = np.array([d for _, d in pairs], dtype=np.int64)
    if len(pairs):
        out[dst] = pool[src]
    return out


def swap_out(layers: list[np.ndarray], blocks: list[int]) -> list[np.ndarray]:
    """Host copies [n, bs, Hkv, D] of the named blocks of every layer tensor — the
    per-layer index_select of reference core/kv_pool.py:157-166."""
    idx = np.asarray(blocks, dtype=np.int64)
    return [t[idx].copy() for t in layers]


def swap_in(layers: list[np.ndarray], host: list[np.ndarray], blocks: list[int]) -> list[np.ndarray]:
    """Layer tensors with host[l][i] written to block blocks[i] — the per-layer
    index_copy_ of reference core/kv_pool.py:175-182, including its count check."""
    if len(blocks) != (host[0].shape[0] if host else 0):
        raise ValueError(f"swap_in: {host[0].shape[0] if host else 0} host blocks into {len(blocks)} device blocks")
    idx = np.asarray(blocks, dtype=np.int64)
    out = []
    for t, h in zip(layers, host):
        t2 = t.copy()
        t2[idx] = h
        out.append(t2)
    return out
