"""Host logic of the paged path's callers, on the CPU: allocator, block table (slot
arithmetic, growth, copy-on-write), sequence lifecycle, prefix cache, pool sizing and
swap, and the scheduler's policy driving PagedKVPool (torch backend).

Covers the behaviours the reference's own tests pin (tests/test_block_allocator.py,
test_block_table.py, test_sequence.py, test_prefix_cache.py, test_preemption.py,
test_admission.py, test_kv_pool.py, test_swap.py), checked here against this build's
implementation.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from inference_server.config import CONFIG, DEFAULT_NUM_BLOCKS
from inference_server.core.block_allocator import BlockAllocator
from inference_server.core.block_table import BlockTable
from inference_server.core.kv_pool import HostBlocks, ModelDims, PagedKVPool
from inference_server.core.prefix_cache import PrefixCache, block_key, chain_keys
from inference_server.core.scheduler import QueueFull, Scheduler, SequenceTooLong
from inference_server.core.sequence import Sequence, Status

GPT2 = ModelDims(num_layers=12, num_kv_heads=12, head_dim=64, dtype=torch.float32)


def _consistent(a: BlockAllocator) -> None:
    """Free set and reference counts agree, and nothing is lost."""
    free = a._stack[:a.num_free]
    assert len(set(free.tolist())) == a.num_free
    assert (a._refs[free] == 0).all()
    assert (a._refs > 0).sum() + a.num_free == a.num_blocks


# ------------------------------------------------------------------ allocator
def test_allocator_hands_out_low_ids_first_and_reuses_the_last_freed():
    a = BlockAllocator(6)
    assert a.allocate_many(3) == [0, 1, 2] and a.allocate() == 3
    a.free(1)
    assert a.allocate() == 1                        # most recently freed first
    _consistent(a)


def test_allocate_many_is_all_or_nothing():
    a = BlockAllocator(4)
    a.allocate_many(3)
    with pytest.raises(MemoryError):
        a.allocate_many(2)
    assert a.num_free == 1
    assert a.allocate_many(0) == []
    with pytest.raises(ValueError):
        a.allocate_many(-1)
    a.allocate()
    with pytest.raises(MemoryError, match="exhausted"):
        a.allocate()
    _consistent(a)


def test_refcounts_defer_the_release_and_guard_misuse():
    a = BlockAllocator(4)
    released = []
    a.on_release = released.append
    b = a.allocate()
    assert a.incref(b) == 2 and a.refcount(b) == 2
    assert a.free(b) == 1 and released == [] and a.num_free == 3
    assert a.free(b) == 0 and released == [b] and a.num_free == 4
    with pytest.raises(ValueError, match="double free"):
        a.free(b)
    with pytest.raises(ValueError, match="use-after-free"):
        a.incref(b)
    for bad in (4, -1, 1.0, True):
        with pytest.raises(IndexError):
            a.refcount(bad)
    _consistent(a)


def test_free_many_is_checked_before_anything_changes():
    a = BlockAllocator(8)
    got = a.allocate_many(4)
    a.incref(got[0])
    with pytest.raises(ValueError, match="double free"):
        a.free_many([got[1], got[1]])               # held once, listed twice
    assert a.num_free == 4 and a.refcount(got[1]) == 1
    with pytest.raises(IndexError):
        a.free_many([got[2], 99])
    released = []
    a.on_release = released.append
    a.free_many(np.array(got))
    assert released == got[1:] and a.refcount(got[0]) == 1
    _consistent(a)


def test_no_leak_after_churn():
    rng = np.random.default_rng(0)
    a = BlockAllocator(64)
    held: list[int] = []
    for _ in range(2000):
        if held and rng.random() < 0.5:
            a.free(held.pop(int(rng.integers(len(held)))))
        else:
            try:
                held.extend(a.allocate_many(int(rng.integers(1, 5))))
            except MemoryError:
                pass
    a.free_many(held)
    assert a.num_free == 64
    _consistent(a)


# ------------------------------------------------------------------ block table
@pytest.mark.parametrize("tokens,blocks", [(0, 0), (1, 1), (15, 1), (16, 1), (17, 2), (32, 2), (33, 3)])
def test_block_count_is_a_ceiling(tokens, blocks):
    assert BlockTable(BlockAllocator(4), 16).blocks_for(tokens) == blocks


def test_slots_follow_the_physical_layout():
    a = BlockAllocator(8)
    t = BlockTable(a, block_size=4)
    assert t.ensure_capacity(5) == [0, 1] and t.capacity == 8
    assert t.ensure_capacity(8) == [] and t.num_blocks == 2
    assert t.slots(6).tolist() == [0, 1, 2, 3, 4, 5]
    t._ids[:2] = [7, 2]
    assert t.slots(6).tolist() == [28, 29, 30, 31, 8, 9]
    assert t.slot_range(3, 6).tolist() == [31, 8, 9]
    assert t.slot_range(4, 5).tolist() == [8] and t.slot_of(5) == 9
    assert t.slot(5) == (2, 1)
    with pytest.raises(IndexError):
        t.slots(9)
    with pytest.raises(IndexError):
        t.slot(8)


def test_distinct_tables_never_share_a_slot_and_waste_stays_under_a_block():
    a = BlockAllocator(64)
    tables = [BlockTable(a, 16) for _ in range(5)]
    lens = [1, 16, 17, 100, 255]
    for t, n in zip(tables, lens):
        t.ensure_capacity(n)
        assert 0 <= t.waste(n) < 16
    slots = np.concatenate([t.slots(n) for t, n in zip(tables, lens)])
    assert len(set(slots.tolist())) == sum(lens)


def test_growth_fails_whole_and_free_is_idempotent():
    a = BlockAllocator(3)
    t = BlockTable(a, 4)
    t.ensure_capacity(8)
    with pytest.raises(MemoryError):
        t.ensure_capacity(16)                       # needs 2 more, 1 free
    assert t.num_blocks == 2 and a.num_free == 1
    t.free()
    t.free()
    assert a.num_free == 3 and t.num_blocks == 0


def test_every_change_of_the_ids_takes_a_new_unique_stamp():
    a = BlockAllocator(16)
    t, u = BlockTable(a, 4), BlockTable(a, 4)
    seen = {t.version, u.version}
    assert len(seen) == 2
    for change in (lambda: t.ensure_capacity(5), lambda: u.adopt(t.blocks[:1]),
                   lambda: u.ensure_private(0, None), lambda: t.free()):
        before = (t.version, u.version)
        change()
        after = (t.version, u.version)
        assert after != before and not (set(after) - set(before)) & seen
        seen |= set(after)
    v = t.version
    t.ensure_capacity(0)                             # no change, no new stamp
    assert t.version == v


def test_copy_on_write_moves_only_shared_blocks():
    a = BlockAllocator(8)
    owner = BlockTable(a, 4)
    owner.ensure_capacity(8)
    sharer = BlockTable(a, 4)
    sharer.adopt(owner.blocks[:1])
    assert a.refcount(owner.blocks[0]) == 2
    copies = []
    assert owner.ensure_private(1, lambda s, d: copies.append((s, d))) is None
    src = owner.blocks[0]
    moved = sharer.ensure_private(0, lambda s, d: copies.append((s, d)))
    assert moved == (src, sharer.blocks[0]) and copies == [moved]
    assert a.refcount(src) == 1 and a.refcount(sharer.blocks[0]) == 1
    with pytest.raises(ValueError, match="non-empty"):
        sharer.adopt([src])


def test_make_writable_copies_each_shared_block_of_the_write_once():
    a = BlockAllocator(16)
    parent = BlockTable(a, 4)
    parent.ensure_capacity(12)
    child = BlockTable(a, 4)
    child.adopt(parent.blocks)
    pairs = []
    child.make_writable(3, 9, lambda s, d: pairs.append((s, d)))  # blocks 0, 1, 2
    assert [s for s, _ in pairs] == parent.blocks and child.blocks == [d for _, d in pairs]
    child.make_writable(3, 9, lambda s, d: pairs.append((s, d)))
    assert len(pairs) == 3                          # already private


def test_cow_copies_bytes_through_the_pool():
    pool = PagedKVPool(ModelDims(2, 2, 4, torch.float32), num_blocks=8, block_size=4, device="cpu")
    for t in pool.k + pool.v:
        t.copy_(torch.randn_like(t))
    before = [t.clone() for t in pool.k + pool.v]
    a = BlockAllocator(8)
    owner = BlockTable(a, 4)
    owner.ensure_capacity(4)
    sharer = BlockTable(a, 4)
    sharer.adopt(owner.blocks)
    src, dst = sharer.ensure_private(0, pool.copy_block)
    for t, b in zip(pool.k + pool.v, before):
        assert torch.equal(t[dst], b[src])


@pytest.mark.parametrize("pairs", [[(1, 2), (3, 2)], [(1, 2), (2, 5)], [(4, 4)]])
def test_copy_blocks_refuses_pairs_that_would_race(pairs):
    """The hip backend copies every pair at once: a repeated destination, or a block
    that is both a source and a destination, would race, so both backends refuse them
    before copying anything."""
    pool = PagedKVPool(ModelDims(2, 2, 4, torch.float32), num_blocks=8, block_size=4, device="cpu")
    for t in pool.k + pool.v:
        t.copy_(torch.randn_like(t))
    before = [t.clone() for t in pool.k + pool.v]
    with pytest.raises(ValueError, match="copy_blocks"):
        pool.copy_blocks(pairs)
    assert all(torch.equal(t, b) for t, b in zip(pool.k + pool.v, before))
    pool.copy_blocks([(1, 2), (1, 3), (0, 7)])          # a source may feed several copies
    for t, b in zip(pool.k + pool.v, before):
        assert torch.equal(t[2], b[1]) and torch.equal(t[3], b[1]) and torch.equal(t[7], b[0])


# ------------------------------------------------------------------ sequence
def test_sequence_lifecycle():
    s = Sequence("a", [5, 6, 7], max_tokens=3)
    assert s.status is Status.WAITING and s.needs_prefill and s.is_prefilling
    assert s.next_input_ids == [5, 6, 7] and s.cached_after_next_pass == 3
    s.admit()
    s.num_cached = 3
    s.append_token(8, eos_id=0)
    assert not s.is_prefilling and s.next_input_ids == [8] and s.next_position == 3
    assert s.prompt_token_ids == [5, 6, 7] and s.output_token_ids == [8]
    s.preempt(step=4)                                # recompute: history re-fed
    assert s.status is Status.WAITING and s.num_cached == 0 and s.next_input_ids == [5, 6, 7, 8]
    with pytest.raises(RuntimeError, match="preempted while waiting"):
        s.preempt(step=5)
    s.admit()
    s.num_cached = 4
    s.preempt(step=6, host_kv="host")                # swap: cache kept
    assert s.status is Status.SWAPPED and s.num_cached == 4 and s.host_kv == "host"
    s.admit()
    assert s.host_kv is None and s.preemptions == 2
    s.append_token(9, eos_id=0)
    s.append_token(10, eos_id=0)
    assert s.is_finished and s.finish_reason == "length" and s.output_token_ids == [8, 9, 10]
    with pytest.raises(RuntimeError, match="sampled again"):
        s.append_token(1, eos_id=0)
    with pytest.raises(RuntimeError, match="admitted while finished"):
        s.admit()


def test_eos_stops_early_and_a_request_override_wins():
    s = Sequence("a", [1], max_tokens=10)
    s.append_token(0, eos_id=0)
    assert s.is_finished and s.finish_reason == "eos"
    t = Sequence("b", [1], max_tokens=10, eos_token_id=7)
    t.append_token(0, eos_id=0)
    assert not t.is_finished
    t.append_token(7, eos_id=0)
    assert t.finish_reason == "eos" and t.ttft_s >= 0 and t.latency_s >= t.ttft_s


# ------------------------------------------------------------------ prefix cache
def test_keys_chain_over_the_whole_prefix():
    toks = list(range(40))
    keys = chain_keys(toks, 16)
    assert len(keys) == 2 and keys[1] == block_key(keys[0], toks[16:32])
    assert keys[0] == block_key(None, toks[:16])
    assert chain_keys([999] + toks[1:], 16)[1] != keys[1]   # same block tokens, other prefix
    part = chain_keys(toks, 16, upto=1)
    assert part == keys[:1] and chain_keys(toks, 16, part) == keys   # extends in place


def _seq_with_table(alloc, tokens, cached, bs=4):
    s = Sequence("s", tokens, max_tokens=4)
    s.block_table = BlockTable(alloc, bs)
    s.block_table.ensure_capacity(cached)
    s.num_cached = cached
    return s


def test_prefix_cache_shares_full_blocks_and_forgets_on_release():
    a = BlockAllocator(16)
    cache = PrefixCache(a, 4)
    toks = list(range(10))
    first = _seq_with_table(a, toks, 10)
    assert cache.register(first) == 2 and cache.register(first) == 0
    second = Sequence("t", toks + [50, 51], max_tokens=4)
    blocks = cache.match(second)
    assert blocks == first.block_table.blocks[:2]
    second.block_table = BlockTable(a, 4)
    assert cache.claim(second, blocks) == 8 and a.refcount(blocks[0]) == 2
    # a match never covers the last token: a fully cached 8-token prompt feeds its last block
    assert cache.match(Sequence("u", toks[:8], max_tokens=1)) == first.block_table.blocks[:1]
    assert cache.match(Sequence("v", toks[:4], max_tokens=1)) == []
    first.block_table.free()
    assert cache.entries == 2                        # `second` still holds both
    second.block_table.free()
    assert cache.entries == 0 and a.num_free == 16
    assert cache.stats()["prefix_hits"] == 2 and cache.stats()["prefix_tokens_saved"] == 8


def test_a_held_duplicate_takes_over_when_the_indexed_block_goes():
    """Two sequences prefill the same prefix in one pass: one block is indexed, the
    other is a spare; when the indexed one is released the spare serves the key."""
    a = BlockAllocator(16)
    cache = PrefixCache(a, 4)
    toks = list(range(9))
    x = _seq_with_table(a, toks, 9)
    y = _seq_with_table(a, toks, 9)
    assert cache.register(x) == 2 and cache.register(y) == 0
    assert cache.entries == 2
    x.block_table.free()
    probe = Sequence("p", toks + [1], max_tokens=1)
    assert cache.match(probe) == y.block_table.blocks[:2]
    y.block_table.free()
    assert cache.match(probe) == [] and cache.entries == 0 and not cache._spares


def test_prefix_keys_are_computed_once_per_block():
    a = BlockAllocator(16)
    cache = PrefixCache(a, 4)
    s = Sequence("s", list(range(13)), max_tokens=4)
    cache.match(s)
    keys = list(s.prefix_keys)
    assert len(keys) == 3
    cache.match(s)
    assert s.prefix_keys == keys and all(k1 is k2 for k1, k2 in zip(s.prefix_keys, keys))


# ------------------------------------------------------------------ pool sizing and swap
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
    """A forward pass whose only state is the pool: each fed token is written into
    layer 0's K at its slot, and the next token is a function of every cached slot
    read back through the sequence's CURRENT block table — so a lost, stale or
    misplaced block after preemption, swap or sharing changes the outputs."""

    def __init__(self, pool: PagedKVPool) -> None:
        self.flat_k = pool.k[0].view(-1, pool.dims.num_kv_heads, pool.dims.head_dim)
        self.batches: list[list[str]] = []
        self.fed: dict[str, int] = {}

    def execute(self, seqs):
        self.batches.append([s.seq_id for s in seqs])
        out = []
        for s in seqs:
            fed = s.next_input_ids
            self.fed[s.seq_id] = self.fed.get(s.seq_id, 0) + len(fed)
            start = s.num_cached
            slots = s.block_table.slot_range(start, start + len(fed))
            self.flat_k[torch.from_numpy(slots), 0, 0] = torch.tensor(fed, dtype=torch.float32)
            s.num_cached = start + len(fed)
            cached = self.flat_k[torch.from_numpy(s.block_table.slots(s.num_cached)), 0, 0]
            weights = torch.arange(1, s.num_cached + 1, dtype=torch.float32)
            out.append(1 + int((cached * weights).sum().item()) % 97)
        return out


def _workload(n=6, prefix=()):
    return [Sequence(seq_id=f"s{i}", prompt_token_ids=list(prefix) + [10 + (i * 3 + j) % 17 for j in range(5 + i % 5)],
                     max_tokens=6 + (i * 5) % 5) for i in range(n)]


def _scheduler(num_blocks, monkeypatch, mode="recompute", prefix=False, max_running=32):
    monkeypatch.setattr(CONFIG, "block_size", 4)
    monkeypatch.setattr(CONFIG, "preemption", mode)
    monkeypatch.setattr(CONFIG, "max_running", max_running)
    pool = PagedKVPool(ModelDims(2, 2, 4, torch.float32), num_blocks=num_blocks, block_size=4, device="cpu")
    alloc = BlockAllocator(num_blocks)
    cache = PrefixCache(alloc, 4) if prefix else None
    return Scheduler(PoolExecutor(pool), eos_token_id=0, allocator=alloc, pool=pool, prefix_cache=cache), alloc


def _drain(sched, seqs):
    for s in seqs:
        sched.add(s)
    for _ in range(10_000):
        if not sched.has_work:
            return
        sched.step()
        for s in sched.returning:
            assert s.block_table is None or s.block_table.num_blocks == 0   # no block held while off the device
    raise AssertionError("scheduler did not drain")


@pytest.mark.parametrize("mode", ["swap", "recompute"])
@pytest.mark.parametrize("prefix", [False, True])
def test_preemption_and_sharing_are_invisible_to_outputs(monkeypatch, mode, prefix):
    shared = list(range(30, 39)) if prefix else []
    ref = _workload(prefix=shared)
    sched, _ = _scheduler(512, monkeypatch, mode)
    _drain(sched, ref)
    seqs = _workload(prefix=shared)
    sched, alloc = _scheduler(9, monkeypatch, mode, prefix=prefix)
    _drain(sched, seqs)
    stats = sched.stats()
    assert stats["preemptions"] > 0
    assert (stats["swaps"] > 0) == (mode == "swap")
    for got, want in zip(seqs, ref):
        assert got.is_finished and got.output_token_ids == want.output_token_ids
    assert alloc.num_free == 9 and all(s.host_kv is None for s in seqs)
    if prefix:
        assert stats["prefix_hits"] > 0 and stats["prefix_entries"] == 0


def test_prefix_hits_skip_the_shared_blocks(monkeypatch):
    shared = list(range(100, 112))                   # three full blocks of 4
    seqs = _workload(n=4, prefix=shared)
    sched, alloc = _scheduler(64, monkeypatch, prefix=True, max_running=4)
    sched.add(seqs[0])
    sched.step()                                     # prefills and publishes the prefix
    _drain(sched, seqs[1:])
    st = sched.stats()
    # Each later request starts on the 3 prefix blocks the first one still holds.
    assert st["prefix_hits"] == 9 and st["prefix_blocks_shared"] == 9
    assert sched.executor.batches[1] == ["s1", "s2", "s3"]
    assert alloc.num_free == 64


def test_two_sequences_share_exactly_the_common_full_blocks(monkeypatch):
    """The reference's sharing scenario (tests/test_prefix_cache.py:111-137): two
    prompts with a common two-block head; the second is admitted onto the first's two
    blocks, is fed only its tail, and the admission that matched nothing counts no
    misses."""
    head = [10, 11, 12, 13, 14, 15, 16, 17]          # two full blocks of 4
    sched, alloc = _scheduler(512, monkeypatch, prefix=True)
    cache = sched.prefix_cache
    s1 = Sequence(seq_id="a", prompt_token_ids=head + [1, 2, 3], max_tokens=4)
    s2 = Sequence(seq_id="b", prompt_token_ids=head + [7, 8], max_tokens=8)
    sched.add(s1)
    sched.step()                                     # s1 prefills alone and publishes
    assert cache.entries == 2 and cache.hits == 0 and cache.misses == 0
    sched.add(s2)
    sched.step()                                     # s2 matches the 2 head blocks
    b1, b2 = list(s1.block_table.blocks), list(s2.block_table.blocks)
    assert b2[:2] == b1[:2] and b2[2:] and not set(b2[2:]) & set(b1)
    assert all(alloc.refcount(b) == 2 for b in b1[:2])
    assert all(alloc.refcount(b) == 1 for b in b1[2:] + b2[2:])
    assert cache.hits == 2 and cache.blocks_shared == 2 and cache.misses == 0
    assert sched.executor.fed["b"] == 2, "only the tail past the shared prefix is fed"
    assert sched.stats()["prefix_hits"] == 2 and sched.stats()["prefix_misses"] == 0
    while not s1.is_finished:
        sched.step()
    sched.step()                                     # s1's blocks are released
    assert all(alloc.refcount(b) == 1 for b in s2.block_table.blocks[:2])
    assert cache.entries >= 2
    for _ in range(100):
        if not sched.has_work:
            break
        sched.step()
    assert alloc.num_free == 512 and cache.entries == 0


def test_prefix_entries_die_with_their_last_holder(monkeypatch):
    shared = list(range(100, 112))
    seqs = _workload(n=2, prefix=shared)
    sched, _ = _scheduler(64, monkeypatch, prefix=True, max_running=1)
    _drain(sched, seqs)                              # one at a time: nothing to share
    assert sched.stats()["prefix_hits"] == 0 and sched.stats()["prefix_entries"] == 0


def test_victim_is_the_most_recently_admitted_and_comes_back_first(monkeypatch):
    sched, alloc = _scheduler(6, monkeypatch, max_running=3)
    seqs = [Sequence(f"q{i}", [1 + i] * 7, max_tokens=8) for i in range(3)]   # 2 blocks each at prefill
    for s in seqs:
        sched.add(s)
    sched.step()                                     # all three prefill: 6 blocks used
    assert [s.seq_id for s in sched.active] == ["q0", "q1", "q2"]
    sched.step()                                     # decode to position 7: fits
    sched.step()                                     # position 8 needs a 3rd block for each
    assert sched.num_preemptions >= 1 and sched.returning[0].seq_id == "q2"
    assert sched.returning[0].preempted_step == sched.tick
    # Not re-admitted on its own preemption step, and ahead of new arrivals after.
    late = Sequence("late", [9] * 3, max_tokens=2)
    sched.add(late)
    _drain(sched, [])
    assert all(s.is_finished for s in seqs + [late])
    order = [b for b in sched.executor.batches if "q2" in b or "late" in b]
    first_q2 = next(i for i, b in enumerate(sched.executor.batches) if "q2" in b and i > 2)
    first_late = next(i for i, b in enumerate(sched.executor.batches) if "late" in b)
    assert order and first_q2 <= first_late
    assert alloc.num_free == 6


def test_admission_reserves_the_running_sets_growth(monkeypatch):
    """A newcomer that would take the block a running sequence needs next waits."""
    sched, alloc = _scheduler(3, monkeypatch, max_running=4)
    a = Sequence("a", [1, 2, 3, 4], max_tokens=3)    # 1 block now, a 2nd at its first decode
    sched.add(a)
    sched.step()
    b = Sequence("b", [5, 6, 7, 8, 9, 10, 11, 12], max_tokens=1)   # needs 2 blocks
    sched.add(b)
    sched.step()                                     # free 2, a reserves 1: b does not fit
    assert [s.seq_id for s in sched.active] == ["a"] and sched.queue_depth == 1
    _drain(sched, [])
    assert a.is_finished and b.is_finished and sched.num_preemptions == 0


def test_head_of_line_blocking_keeps_fifo(monkeypatch):
    sched, _ = _scheduler(4, monkeypatch, max_running=4)
    big = Sequence("big", list(range(1, 14)), max_tokens=2)        # 4 blocks
    small = Sequence("small", [1], max_tokens=2)
    hold = Sequence("hold", [1, 2], max_tokens=3)
    sched.add(hold)
    sched.step()
    sched.add(big)
    sched.add(small)
    sched.step()
    assert [s.seq_id for s in sched.active] == ["hold"]          # small waits behind big
    _drain(sched, [])
    batches = sched.executor.batches
    assert min(i for i, b in enumerate(batches) if "big" in b) < min(i for i, b in enumerate(batches) if "small" in b)


def test_prefills_run_before_decodes(monkeypatch):
    sched, _ = _scheduler(32, monkeypatch, max_running=4)
    a = Sequence("a", [1, 2], max_tokens=4)
    sched.add(a)
    sched.step()
    sched.add(Sequence("b", [3, 4, 5], max_tokens=2))
    sched.step()
    assert sched.executor.batches[-1] == ["b"]                    # a's decode waits a pass
    sched.step()
    assert sorted(sched.executor.batches[-1]) == ["a", "b"]


def test_door_refusals(monkeypatch):
    monkeypatch.setattr(CONFIG, "block_size", 4)
    sched = Scheduler(None, 0, allocator=BlockAllocator(2))
    with pytest.raises(SequenceTooLong, match="needs up to 3 blocks"):
        sched.add(Sequence("long", list(range(8)), max_tokens=4))
    sched.add(Sequence("fits", list(range(4)), max_tokens=5))      # 8 cached tokens at most
    monkeypatch.setattr(CONFIG, "max_queue_depth", 1)
    with pytest.raises(QueueFull) as info:
        sched.add(Sequence("b", [1], max_tokens=1))
    assert info.value.depth == 1 and info.value.bound == 1 and sched.queue_depth == 1


def test_stats_fields(monkeypatch):
    sched, _ = _scheduler(8, monkeypatch, prefix=True)
    assert set(sched.stats()) == {"queue_depth", "num_running", "num_waiting", "num_swapped", "free_blocks",
                                  "num_blocks", "preemptions", "swaps", "completed", "prefix_hits",
                                  "prefix_misses", "prefix_blocks_shared", "prefix_entries", "prefix_tokens_saved"}


def test_graph_metadata_rows_follow_the_tables_incrementally():
    """TableRows (the decode/prefill graphs' pinned block-table segment) under random
    growth, copy-on-write remaps, frees and batch reorderings: after every write the
    first len(batch) rows equal the batch's tables, zero-padded; rows of unchanged
    tables are not rewritten."""
    from inference_server.core.decode_graphs import TableRows

    rng = np.random.default_rng(3)
    a = BlockAllocator(256)
    tables = [BlockTable(a, 4) for _ in range(6)]
    rows = np.zeros((4, 40), dtype=np.int64)
    tr = TableRows(rows)
    for _ in range(400):
        t = tables[int(rng.integers(len(tables)))]
        op = rng.random()
        if op < 0.5:
            t.ensure_capacity(min(t.capacity + int(rng.integers(1, 9)), 160))
        elif op < 0.6:
            t.free()
        elif op < 0.8 and t.num_blocks:
            other = tables[int(rng.integers(len(tables)))]
            if other is not t and not other.num_blocks:
                other.adopt(t.blocks[:1])
                other.ensure_private(0, None)
        batch = [tables[i] for i in rng.permutation(len(tables))[:int(rng.integers(1, 5))]]
        before = tr.rewrites
        tr.write(batch)
        tr.write(batch)
        assert tr.rewrites - before <= len(batch)
        for i, tb in enumerate(batch):
            assert (rows[i, :tb.num_blocks] == tb.ids).all() and not rows[i, tb.num_blocks:].any()
