"""End-to-end paged engine: the executor's transformers hooks, the scheduler and the
pool together.

CPU (gather backend, a 2-layer random GPT-2): greedy tokens equal a full-recompute
greedy loop over HuggingFace's own eager attention; preemption (recompute and swap)
and prefix sharing leave the tokens unchanged (reference tests/test_preemption.py,
test_swap.py:147-171, test_prefix_cache.py:316-365, whose pretrained-GPT-2 goldens
are not available offline).

GPU: BASELINE config 1's workload on GPT-2 124M fp32 with ATTENTION=hip gives
token ids identical to ATTENTION=gather on the same device and weights; the hip
path also survives swap and recompute preemption with identical tokens.
"""

from __future__ import annotations

import pytest
import torch

from inference_server.bench import workload
from inference_server.config import CONFIG
from inference_server.core.block_allocator import BlockAllocator
from inference_server.core.block_table import BlockTable
from inference_server.core.kv_pool import ModelDims, PagedKVPool
from inference_server.core.paged_executor import PagedExecutor
from inference_server.core.sequence import Sequence
from inference_server.engine.paged import PagedEngine, Request
from inference_server.model import load


def _requests(n=5, vocab=1000, max_tokens=12, prefix=None, seed=0):
    g = torch.Generator().manual_seed(seed)
    reqs = []
    for i in range(n):
        tail = torch.randint(0, vocab, (int(torch.randint(5, 60, (1,), generator=g)),), generator=g).tolist()
        reqs.append(Request(f"r{i}", (prefix or []) + tail, max_tokens))
    return reqs


def _recompute_greedy(model, req):
    ids = list(req.prompt_token_ids)
    out = []
    with torch.no_grad():
        for _ in range(req.max_tokens):
            t = int(model(torch.tensor([ids], device=next(model.parameters()).device)).logits[0, -1].argmax())
            out.append(t)
            ids.append(t)
    return out


@pytest.fixture
def small_model(monkeypatch):
    monkeypatch.setattr(CONFIG, "attention", "gather")
    return load(small=True)


def test_paged_engine_matches_full_recompute(small_model):
    model, tok = small_model
    reqs = _requests()
    res = PagedEngine(model, tok, num_blocks=64, block_size=16, device="cpu").run(reqs)
    for r in reqs:
        assert res.outputs[r.request_id] == _recompute_greedy(model, r), r.request_id
    assert res.generated_tokens == sum(r.max_tokens for r in reqs)


@pytest.mark.parametrize("mode", ["recompute", "swap"])
def test_preemption_does_not_change_tokens(small_model, monkeypatch, mode):
    model, tok = small_model
    reqs = _requests(n=6, max_tokens=20)
    ref = PagedEngine(model, tok, num_blocks=128, block_size=16, device="cpu").run(reqs)
    monkeypatch.setattr(CONFIG, "preemption", mode)
    tight = PagedEngine(model, tok, num_blocks=9, block_size=16, device="cpu").run(reqs)
    assert tight.stats["preemptions"] > 0
    assert (tight.stats["swaps"] > 0) == (mode == "swap")
    assert tight.outputs == ref.outputs


def test_prefix_sharing_does_not_change_tokens(small_model):
    model, tok = small_model
    prefix = list(range(100, 148))                     # three full 16-token blocks
    reqs = _requests(n=4, prefix=prefix)
    # The first request prefills alone and publishes the prefix; the rest arrive
    # while it still holds those blocks (entries live only as long as a holder).
    arrivals = [0, 2, 2, 3]
    off = PagedEngine(model, tok, num_blocks=64, block_size=16, device="cpu",
                      prefix_caching=False).run(reqs, arrival_steps=arrivals)
    on = PagedEngine(model, tok, num_blocks=64, block_size=16, device="cpu",
                     prefix_caching=True).run(reqs, arrival_steps=arrivals)
    assert on.stats["prefix_hits"] > 0
    assert on.outputs == off.outputs


def _forked_decode(model, tok, device, forks=3, steps=3):
    """A parent prefills 20 tokens (its second block holds 4 rows); `forks - 1` forks
    adopt both of its blocks, the partly written one included, and every sequence
    continues with a different token. The first decode step writes row 20 of that
    shared block in every sequence, so the executor must give all but one of them a
    private copy first — all of the step's copies in one copy_blocks call. Returns
    the sequences, the non-empty copy_blocks calls, and whether every sequence's
    second block still holds the parent's rows 16-19 bit for bit afterwards."""
    dims = ModelDims.from_model(model, dtype=next(model.parameters()).dtype)
    pool = PagedKVPool(dims, num_blocks=16, block_size=16, device=device)
    ex = PagedExecutor(model, tok, pool)
    alloc = BlockAllocator(16)
    prompt = list(range(200, 220))
    parent = Sequence("s0", prompt, 16)
    parent.block_table = BlockTable(alloc, 16)
    parent.block_table.ensure_capacity(len(prompt))
    ex.execute([parent])
    seqs = [parent]
    for i in range(1, forks):
        fork = Sequence(f"s{i}", prompt, 16)
        fork.num_cached = len(prompt)
        fork.block_table = BlockTable(alloc, 16)
        fork.block_table.adopt(parent.block_table.blocks)
        seqs.append(fork)
    for i, seq in enumerate(seqs):
        seq.tokens.append(300 + i)
    shared = parent.block_table.blocks[1]
    rows = [t[shared, :4].clone() for t in pool.k + pool.v]
    calls = []
    batched = pool.copy_blocks

    def spy(pairs):
        if pairs:
            calls.append(list(pairs))
        batched(pairs)

    pool.copy_blocks = spy
    for _ in range(steps):
        for seq in seqs:
            seq.block_table.ensure_capacity(seq.total_len)
        for seq, t in zip(seqs, ex.execute(seqs)):
            seq.tokens.append(t)
    kept = all(torch.equal(t[seq.block_table.blocks[1], :4], r)
               for seq in seqs for t, r in zip(pool.k + pool.v, rows))
    pool.release()
    return seqs, calls, kept


def test_forks_copy_a_shared_partial_block_once_per_step(small_model):
    """Copy-on-write through the executor (reference core/paged_executor.py:227-231,
    block_table.py:110-134): every fork's private block holds the parent's rows, its
    tokens equal a full-recompute greedy loop over its own history, and the two
    copies of the first step went out as one call."""
    model, tok = small_model
    seqs, calls, kept = _forked_decode(model, tok, "cpu")
    assert len(calls) == 1 and len(calls[0]) == 2
    assert kept
    assert len({seq.block_table.blocks[1] for seq in seqs}) == 3
    for seq in seqs:
        history = seq.prompt_token_ids + seq.output_token_ids[:1]
        want = _recompute_greedy(model, Request(seq.seq_id, history, len(seq.output_token_ids) - 1))
        assert seq.output_token_ids[1:] == want, seq.seq_id


def test_workloads_are_seeded_and_shaped():
    a, b = workload.config1(), workload.config1()
    assert [r.prompt_token_ids for r in a] == [r.prompt_token_ids for r in b]
    assert len(a) == 8 and all(16 <= len(r.prompt_token_ids) <= 256 and r.max_tokens == 32 for r in a)
    c5 = workload.config5()
    assert len(c5) == 200 and all(8 <= r.max_tokens <= 512 for r in c5)
    shared = sum(r.prompt_token_ids[:128] == c5[0].prompt_token_ids[:128] for r in c5 if len(r.prompt_token_ids) > 128)
    assert 60 <= shared <= 140


# ------------------------------------------------------------------ GPU
def _gpt2_run(monkeypatch, backend, reqs, num_blocks=2048, mode="recompute", dtype=torch.float32):
    monkeypatch.setattr(CONFIG, "attention", backend)
    monkeypatch.setattr(CONFIG, "preemption", mode)
    model, tok = load(dtype=dtype, device="cuda")
    engine = PagedEngine(model, tok, num_blocks=num_blocks, block_size=16, device="cuda")
    try:
        return engine.run(reqs)
    finally:
        engine.shutdown()


@pytest.mark.gpu
def test_config1_gpt2_fp32_hip_tokens_identical_to_gather(monkeypatch):
    reqs = workload.config1()
    gather = _gpt2_run(monkeypatch, "gather", reqs)
    hip = _gpt2_run(monkeypatch, "hip", reqs)
    assert hip.generated_tokens == 8 * 32
    assert hip.outputs == gather.outputs


@pytest.mark.gpu
def test_config5_subset_fp16_runs_on_hip(monkeypatch):
    """GPT-2 fp16 with a shared prefix and an undersized pool (BASELINE config 5 shape,
    24 requests): every request completes with its requested length on ATTENTION=hip.
    (fp16 greedy streams are not required to match gather token for token.)"""
    reqs = workload.config5(n=24)
    for r in reqs:
        r.max_tokens = min(r.max_tokens, 40)
    res = _gpt2_run(monkeypatch, "hip", reqs, num_blocks=160, mode="swap", dtype=torch.float16)
    assert res.generated_tokens == sum(r.max_tokens for r in reqs)
    assert all(len(res.outputs[r.request_id]) == r.max_tokens for r in reqs)
    assert res.stats["prefix_hits"] > 0 or res.stats["preemptions"] > 0


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["recompute", "swap"])
def test_hip_engine_under_preemption(monkeypatch, mode):
    """A pool too small for the batch forces preemption on the hip path (swap moves
    blocks through libpagedkv's gather/DMA/scatter); tokens equal a roomy run."""
    reqs = workload.config1(n=8, max_tokens=24)
    roomy = _gpt2_run(monkeypatch, "hip", reqs)
    tight = _gpt2_run(monkeypatch, "hip", reqs, num_blocks=40, mode=mode)
    assert tight.stats["preemptions"] > 0
    assert (tight.stats["swaps"] > 0) == (mode == "swap")
    assert tight.outputs == roomy.outputs


@pytest.mark.gpu
def test_hip_forks_copy_on_write_tokens_identical_to_gather(monkeypatch):
    """The fork scenario on GPT-2 fp32: the batched copy (one pkv_copy_blocks launch
    on hip) leaves every fork's tokens identical to the gather path's."""
    model, tok = load(dtype=torch.float32, device="cuda")
    outs = {}
    for backend in ("gather", "hip"):
        monkeypatch.setattr(CONFIG, "attention", backend)
        seqs, calls, kept = _forked_decode(model, tok, "cuda", forks=4, steps=4)
        assert len(calls) == 1 and len(calls[0]) == 3
        assert kept
        outs[backend] = [seq.output_token_ids for seq in seqs]
    assert outs["hip"] == outs["gather"]


def _engine_result(model, tok, reqs, num_blocks, graphs, capture=False, mode="recompute", keep_pool=False,
                   prefill_graphs=None):
    CONFIG.decode_graphs = graphs
    CONFIG.prefill_graphs = graphs if prefill_graphs is None else prefill_graphs
    CONFIG.preemption = mode
    engine = PagedEngine(model, tok, num_blocks=num_blocks, block_size=16, device="cuda", capture_graphs=capture)
    try:
        res = engine.run(reqs)
        dg, pg = engine.executor.graphs, engine.executor.prefill_graphs
        info = {"replays": dg.replays if dg else 0, "census": dict(dg.census) if dg else {},
                "prefill_replays": pg.replays if pg else 0, "prefill_census": dict(pg.census) if pg else {}}
        pool = [t.clone() for t in engine.pool.k + engine.pool.v] if keep_pool else None
        return res, info, pool
    finally:
        engine.shutdown()


@pytest.mark.gpu
def test_step_graph_replays_are_bit_identical_to_eager_steps(monkeypatch):
    """BASELINE config 1 (GPT-2 fp32) on ATTENTION=hip with the prefill step (padded to
    its token bucket) and every decode step replayed from HIP graphs captured on first
    use vs issued eagerly: identical tokens and a bit-identical KV pool afterwards. The
    replays run between the program's own eager work and host syncs (each step reads
    its tokens back); no graph holds a memset."""
    monkeypatch.setattr(CONFIG, "attention", "hip")
    monkeypatch.setattr(CONFIG, "decode_graphs", CONFIG.decode_graphs)
    monkeypatch.setattr(CONFIG, "prefill_graphs", CONFIG.prefill_graphs)
    monkeypatch.setattr(CONFIG, "preemption", CONFIG.preemption)
    model, tok = load(dtype=torch.float32, device="cuda")
    reqs = workload.config1()
    eager, e_info, e_pool = _engine_result(model, tok, reqs, 2048, graphs=False, keep_pool=True)
    graph, g_info, g_pool = _engine_result(model, tok, reqs, 2048, graphs=True, keep_pool=True)
    assert e_info["replays"] == 0 and g_info["replays"] >= 30 and g_info["prefill_replays"] >= 1
    assert graph.outputs == eager.outputs
    for a, b in zip(g_pool, e_pool):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    for census in list(g_info["census"].values()) + list(g_info["prefill_census"].values()):
        assert census.get("kernel", 0) > 12 and not census.get("memset")


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["recompute", "swap"])
def test_precaptured_decode_graphs_under_preemption_fp16(monkeypatch, mode):
    """Config 5's shape (GPT-2 fp16, shared prefix, 24 requests) on a 96-block pool:
    every batch size captured at engine start, then preemption (recompute or swap)
    and prefix sharing while decode steps replay. Tokens equal the eager run's."""
    monkeypatch.setattr(CONFIG, "attention", "hip")
    monkeypatch.setattr(CONFIG, "decode_graphs", CONFIG.decode_graphs)
    monkeypatch.setattr(CONFIG, "preemption", CONFIG.preemption)
    model, tok = load(dtype=torch.float16, device="cuda")
    reqs = workload.config5(n=24)
    for r in reqs:
        r.max_tokens = min(r.max_tokens, 40)
    eager, _, _ = _engine_result(model, tok, reqs, 96, graphs=False, mode=mode)
    graph, info, _ = _engine_result(model, tok, reqs, 96, graphs=True, capture=True, mode=mode, prefill_graphs=False)
    assert eager.stats["preemptions"] > 0
    assert len(info["census"]) == CONFIG.max_running and info["replays"] > 0
    assert graph.outputs == eager.outputs
    assert graph.stats["preemptions"] == eager.stats["preemptions"]


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["recompute", "swap"])
def test_precaptured_prefill_graphs_under_preemption_fp16(monkeypatch, mode):
    """The same workload with every prefill bucket and decode batch size captured at
    engine start. A padded prefill's GEMMs see M = the bucket, so fp16 results may
    differ from the eager step's in the last bit: every request completes with its
    length, every first token (the prefill graph's own output) equals the eager run's,
    and at least 90% of the streams are identical (fp16 greedy streams diverge after a
    near-tie, as hip and gather do)."""
    monkeypatch.setattr(CONFIG, "attention", "hip")
    monkeypatch.setattr(CONFIG, "decode_graphs", CONFIG.decode_graphs)
    monkeypatch.setattr(CONFIG, "prefill_graphs", CONFIG.prefill_graphs)
    monkeypatch.setattr(CONFIG, "preemption", CONFIG.preemption)
    model, tok = load(dtype=torch.float16, device="cuda")
    reqs = workload.config5(n=24)
    for r in reqs:
        r.max_tokens = min(r.max_tokens, 40)
    eager, _, _ = _engine_result(model, tok, reqs, 96, graphs=False, mode=mode)
    graph, info, _ = _engine_result(model, tok, reqs, 96, graphs=True, capture=True, mode=mode)
    assert info["prefill_replays"] > 0 and len(info["prefill_census"]) >= 8
    assert all(len(graph.outputs[r.request_id]) == r.max_tokens for r in reqs)
    assert all(graph.outputs[r.request_id][0] == eager.outputs[r.request_id][0] for r in reqs)
    assert sum(graph.outputs[r.request_id] == eager.outputs[r.request_id] for r in reqs) >= 0.9 * len(reqs)

