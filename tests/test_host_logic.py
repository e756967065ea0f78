"""Host logic of the paged path's callers, on the CPU: allocator invariants, block
table slot arithmetic and copy-on-write, prefix-cache sharing, pool sizing, and the
scheduler's swap / recompute preemption driving PagedKVPool (torch backend).

Mirrors the reference's tests/test_block_allocator.py, test_block_table.py,
test_kv_pool.py, test_swap.py and the COW part of test_prefix_cache.py.
"""

from __future__ import annotations

import pytest
import torch

from inference_server.config import CONFIG, DEFAULT_NUM_BLOCKS
from inference_server.core.block_allocator import BlockAllocator
from inference_server.core.block_table import BlockTable
from inference_server.core.kv_pool import HostBlocks, ModelDims, PagedKVPool
from inference_server.core.prefix_cache import PrefixCache, block_hash, hash_chain
from inference_server.core.scheduler import QueueFull, Scheduler, SequenceTooLong
from inference_server.core.sequence import Sequence, Status

GPT2 = ModelDims(num_layers=12, num_kv_heads=12, head_dim=64, dtype=torch.float32)


# ------------------------------------------------------------------ allocator
def test_allocator_invariants():
    a = BlockAllocator(4)
    got = a.allocate_many(3)
    assert sorted(got) == [0, 1, 2] and a.num_free == 1
    with pytest.raises(MemoryError):
        a.allocate_many(2)
    assert a.num_free == 1                            # all-or-nothing
    a.incref(got[0])
    assert a.free(got[0]) == 1 and a.num_free == 1
    assert a.free(got[0]) == 0 and a.num_free == 2
    with pytest.raises(ValueError, match="double free"):
        a.free(got[0])
    with pytest.raises(ValueError, match="use-after-free"):
        a.incref(got[0])
    with pytest.raises(IndexError):
        a.refcount(4)
    released = []
    a.on_release = released.append
    a.free(got[1])
    assert released == [got[1]]


# ------------------------------------------------------------------ block table
def test_slots_and_capacity():
    a = BlockAllocator(8)
    t = BlockTable(a, block_size=4)
    assert t.ensure_capacity(5) == [0, 1] and t.capacity == 8
    assert t.ensure_capacity(8) == []
    assert t.slots(6) == [0, 1, 2, 3, 4, 5]
    t.blocks = [7, 2]
    assert t.slots(6) == [28, 29, 30, 31, 8, 9]
    assert t.slot_range(3, 6) == [31, 8, 9]
    assert t.slot(5) == (2, 1)
    with pytest.raises(IndexError):
        t.slots(9)
    assert t.blocks_for(17) == 5 and t.blocks_for(16) == 4


def test_ensure_private_copies_shared_block_only():
    """Reference tests/test_prefix_cache.py:242-266: COW fires only when shared."""
    a = BlockAllocator(8)
    owner = BlockTable(a, 4)
    owner.ensure_capacity(8)
    sharer = BlockTable(a, 4)
    sharer.adopt(owner.blocks[:1], [b"h" * 16])
    assert a.refcount(owner.blocks[0]) == 2
    copies = []
    assert owner.ensure_private(1, lambda s, d: copies.append((s, d))) is None
    src = owner.blocks[0]
    moved = sharer.ensure_private(0, lambda s, d: copies.append((s, d)))
    assert moved == (src, sharer.blocks[0]) and copies == [moved]
    assert a.refcount(src) == 1 and a.refcount(sharer.blocks[0]) == 1


def test_cow_copies_bytes_through_the_pool():
    pool = PagedKVPool(ModelDims(2, 2, 4, torch.float32), num_blocks=8, block_size=4, device="cpu")
    for t in pool.k + pool.v:
        t.copy_(torch.randn_like(t))
    before = [t.clone() for t in pool.k + pool.v]
    a = BlockAllocator(8)
    owner = BlockTable(a, 4)
    owner.ensure_capacity(4)
    sharer = BlockTable(a, 4)
    sharer.adopt(list(owner.blocks), [b"x" * 16])
    src, dst = sharer.ensure_private(0, pool.copy_block)
    for t, b in zip(pool.k + pool.v, before):
        assert torch.equal(t[dst], b[src])


# ------------------------------------------------------------------ prefix cache
def test_hash_chain_covers_the_whole_prefix():
    toks = list(range(40))
    chain = hash_chain(toks, 16)
    assert len(chain) == 2 and chain[1] == block_hash(chain[0], toks[16:32])
    other = [999] + toks[1:]
    assert hash_chain(other, 16)[1] != chain[1]       # block 1 same tokens, different prefix


def test_prefix_cache_shares_full_blocks_and_forgets_on_release():
    a = BlockAllocator(16)
    cache = PrefixCache(a, 4)
    first = BlockTable(a, 4)
    first.ensure_capacity(10)
    toks = list(range(10))
    assert cache.register(first, toks, 10) == 2
    blocks, hashes = cache.match(toks + [50, 51])
    assert blocks == first.blocks[:2]
    second = BlockTable(a, 4)
    assert cache.claim(second, blocks, hashes, 2) == 8
    assert a.refcount(blocks[0]) == 2
    # match never covers the last token: a fully cached prompt still feeds a block
    assert cache.match(toks[:8])[0] == first.blocks[:1]
    first.free()
    second.free()
    assert cache.entries == 0 and a.num_free == 16


# ------------------------------------------------------------------ pool sizing
def test_pool_dims_and_sizes():
    assert GPT2.bytes_per_token() == 2 * 12 * 12 * 64 * 4
    per_block = GPT2.bytes_per_block(16)
    assert GPT2.blocks_for_budget(per_block * 10 - 1, 16) == 9
    pool = PagedKVPool(GPT2, num_blocks=8, block_size=16, device="cpu")
    assert len(pool.k) == len(pool.v) == 12 and pool.k[0].shape == (8, 16, 12, 64)
    assert pool.nbytes == sum(t.numel() * t.element_size() for t in pool.k + pool.v)
    assert pool.num_slots == 128
    assert DEFAULT_NUM_BLOCKS * CONFIG.block_size == CONFIG.max_running * CONFIG.max_seq_len


def test_swap_round_trip_cpu():
    pool = PagedKVPool(ModelDims(2, 2, 4, torch.float32), num_blocks=8, block_size=4, device="cpu")
    for t in pool.k + pool.v:
        t.copy_(torch.randn_like(t))
    k0 = [t.clone() for t in pool.k]
    host = pool.swap_out([1, 5, 2])
    assert isinstance(host, HostBlocks) and len(host) == 3
    for t in pool.k + pool.v:
        t[[1, 5, 2]] = 0
    pool.swap_in(host, [6, 0, 3])
    for layer in range(2):
        assert torch.equal(pool.k[layer][[6, 0, 3]], k0[layer][[1, 5, 2]])
    with pytest.raises(ValueError, match="swap_in"):
        pool.swap_in(host, [2])


# ------------------------------------------------------------------ scheduler
class PoolExecutor:
    """Fake forward pass whose only state is the pool (reference tests/test_swap.py:
    153-180): each fed token is written to layer 0's K at its slot; the next token is
    a function of every cached slot, read back through the CURRENT block table."""

    def __init__(self, pool: PagedKVPool) -> None:
        self.flat_k = pool.k[0].view(-1, pool.dims.num_kv_heads, pool.dims.head_dim)

    def execute(self, seqs):
        out = []
        for s in seqs:
            fed = s.next_input_ids
            start = s.num_cached
            for slot, tok in zip(s.block_table.slot_range(start, start + len(fed)), fed):
                self.flat_k[slot] = float(tok)
            s.num_cached = start + len(fed)
            total = self.flat_k[s.block_table.slots(s.num_cached)][:, 0, 0].sum().item()
            out.append(1 + (int(total) * 7) % 49)
        return out


def _workload(n=6):
    return [Sequence(seq_id=f"s{i}", prompt_token_ids=[10 + (i * 3 + j) % 17 for j in range(5 + i % 5)],
                     max_tokens=6 + (i * 5) % 5) for i in range(n)]


def _run(seqs, num_blocks, monkeypatch, mode):
    monkeypatch.setattr(CONFIG, "block_size", 4)
    monkeypatch.setattr(CONFIG, "preemption", mode)
    pool = PagedKVPool(ModelDims(2, 2, 4, torch.float32), num_blocks=num_blocks, block_size=4, device="cpu")
    alloc = BlockAllocator(num_blocks)
    sched = Scheduler(PoolExecutor(pool), eos_token_id=0, allocator=alloc, pool=pool)
    for s in seqs:
        sched.add(s)
    for _ in range(10_000):
        if not sched.has_work:
            return sched, alloc
        sched.step()
        for s in sched.preempted:
            if s.status is Status.SWAPPED:
                assert s.block_table.num_blocks == 0 and s.num_cached > 0
    raise AssertionError("scheduler did not drain")


@pytest.mark.parametrize("mode", ["swap", "recompute"])
def test_preemption_is_invisible_to_outputs(monkeypatch, mode):
    ref = _workload()
    _run(ref, 512, monkeypatch, mode)
    seqs = _workload()
    sched, alloc = _run(seqs, 8, monkeypatch, mode)
    stats = sched.stats()
    assert stats["preemptions"] > 0
    assert (stats["swaps"] > 0) == (mode == "swap")
    for got, want in zip(seqs, ref):
        assert got.is_finished and got.output_token_ids == want.output_token_ids
    assert alloc.num_free == 8
    assert all(s.host_kv is None for s in seqs)


def test_door_refusals(monkeypatch):
    monkeypatch.setattr(CONFIG, "block_size", 4)
    sched = Scheduler(None, 0, allocator=BlockAllocator(2))
    with pytest.raises(SequenceTooLong):
        sched.add(Sequence("long", list(range(8)), max_tokens=4))
    monkeypatch.setattr(CONFIG, "max_queue_depth", 1)
    sched.add(Sequence("a", [1], max_tokens=1))
    with pytest.raises(QueueFull):
        sched.add(Sequence("b", [1], max_tokens=1))
