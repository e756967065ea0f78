"""Attention with the step's KV append fused in (`pkv_paged_attention_decode_append`
on decode batches, `pkv_paged_attention_prefill_append` on any other batch).

GPU (`-m gpu`): the pool after the fused call must equal oracle.kvops.kv_append bit for
bit and the output must match oracle.gather over that pool (2e-2 fp16/bf16, 1e-5
fp32); as a regression guard the two calls it replaces — the append
(`PagedKVPool.append`'s kernel) followed by attention — must also give bit-identical
pool and output. Decode cases cover both partition lengths the launch picks, head_dim
64 / 128, GQA 1 / 4, the new token at the first position, at wave-slice and partition
boundaries. Prefill cases cover fresh prompts, chunks onto a cached prefix that ends
inside a block, mixed prefill + decode batches, GQA groups that split a KV head over
several workgroups, and new slots that hold NaN before the call (a read of a slot this
launch is still writing would show). fp32, odd-stride sources and GQA groups with no
tuned instance (3, 6) take the separate append launch inside the call. The executor's steps are checked eager and replayed
from graphs.
"""

from __future__ import annotations

import pytest
import torch

from inference_server.core.attention_hip import paged_attention_hip_launch


def _case(n_seqs, n_kv, group, d, max_ctx, dtype, seed, fixed=()):
    g = torch.Generator().manual_seed(seed)
    bs = 16
    ctx = torch.randint(1, max_ctx + 1, (n_seqs,), generator=g)
    for i, c in enumerate(fixed):
        ctx[i] = c
    width = int((ctx.max() + bs - 1) // bs)
    n_blocks = n_seqs * width + 3
    perm = torch.randperm(n_blocks, generator=g)
    tables = perm[: n_seqs * width].view(n_seqs, width).clone()
    k_pool = torch.randn(n_blocks, bs, n_kv, d, generator=g).to(dtype)
    v_pool = torch.randn(n_blocks, bs, n_kv, d, generator=g).to(dtype)
    q = torch.randn(n_seqs, n_kv * group, d, generator=g).to(dtype)
    # New rows as HF hands them over: [1, Hkv, B, D] transposed to [B, Hkv, D] views.
    k_new = torch.randn(n_kv, n_seqs, d, generator=g).to(dtype).transpose(0, 1)
    v_new = torch.randn(n_kv, n_seqs, d, generator=g).to(dtype).transpose(0, 1)
    last = ctx - 1
    slots = tables[torch.arange(n_seqs), last // bs] * bs + last % bs
    return q, k_pool, v_pool, tables, ctx, k_new, v_new, slots


def _run_both(q, k_pool, v_pool, tables, ctx, k_new, v_new, slots):
    dev = "cuda"
    qd, td, cd, sd = q.to(dev), tables.to(dev), ctx.to(dev), slots.to(dev)
    ql = torch.ones_like(cd)

    def on_device(t):  # device tensors pass as they are; host ones keep HF's transposed layout
        if t.is_cuda:
            return t
        return t.transpose(0, 1).contiguous().to(dev).transpose(0, 1) if t.stride(0) < t.stride(1) else t.to(dev)

    kn, vn = on_device(k_new), on_device(v_new)
    ka, va = k_pool.to(dev), v_pool.to(dev)
    ka.view(-1, *ka.shape[2:])[sd] = kn
    va.view(-1, *va.shape[2:])[sd] = vn
    scale = q.shape[-1] ** -0.5
    ref = paged_attention_hip_launch(qd, ka, va, td, cd, ql, scale)
    kb, vb = k_pool.to(dev), v_pool.to(dev)
    out = paged_attention_hip_launch(qd, kb, vb, td, cd, ql, scale, append=(kn, vn, sd))
    torch.cuda.synchronize()
    return ref, out, (ka, va), (kb, vb)


CASES = [
    # (n_seqs, n_kv, group, d, max_ctx, dtype, fixed contexts)
    (4, 2, 4, 128, 2000, torch.bfloat16, (1, 256, 257, 768)),       # short partitions
    (6, 12, 1, 64, 1100, torch.float16, (1, 64, 65, 256, 1024)),    # GPT-2 decode shape
    (64, 8, 4, 128, 3000, torch.bfloat16, (1, 192, 193, 768, 769)), # long partitions
    (40, 4, 1, 64, 5000, torch.float16, (2, 191, 192, 1536, 1537)),
    (8, 2, 2, 64, 700, torch.bfloat16, ()),
    (5, 2, 4, 128, 600, torch.float32, (1, 100)),                    # fp32: append launch first
    (6, 2, 3, 128, 900, torch.bfloat16, (1, 300)),                   # group 3: no tuned instance
    (5, 2, 6, 64, 700, torch.float16, (2, 257)),                     # group 6: no tuned instance
]


def _raw(t: torch.Tensor):
    """Raw bits as numpy (bf16 has no numpy dtype)."""
    t = t.detach().cpu().contiguous()
    return t.view({2: torch.int16, 4: torch.int32}[t.element_size()]).numpy()


def _check_against_oracle(args, out, kb, vb):
    """The fused call's pool against oracle.kvops.kv_append (bit-exact) and its output
    against oracle.gather over the appended pool (2e-2 fp16/bf16, 1e-5 fp32)."""
    from oracle.gather import paged_attention_gather
    from oracle.kvops import kv_append

    q, k_pool, v_pool, tables, ctx, k_new, v_new, slots = args
    k_want = kv_append(_raw(k_pool), _raw(k_new), slots.numpy())
    v_want = kv_append(_raw(v_pool), _raw(v_new), slots.numpy())
    assert (_raw(kb) == k_want).all() and (_raw(vb) == v_want).all()
    ref = paged_attention_gather(q, kb.cpu(), vb.cpu(), tables, ctx, torch.ones_like(ctx), q.shape[-1] ** -0.5)
    tol = 1e-5 if q.dtype == torch.float32 else 2e-2
    torch.testing.assert_close(out.cpu(), ref, atol=tol, rtol=tol)


@pytest.mark.gpu
@pytest.mark.parametrize("n_seqs,n_kv,group,d,max_ctx,dtype,fixed", CASES)
def test_fused_append_is_bit_identical_to_append_then_decode(n_seqs, n_kv, group, d, max_ctx, dtype, fixed):
    args = _case(n_seqs, n_kv, group, d, max_ctx, dtype, seed=n_seqs * 31 + d, fixed=fixed)
    ref, out, (ka, va), (kb, vb) = _run_both(*args)
    _check_against_oracle(args, out, kb, vb)
    # Regression guard beside the oracle check: the unfused pair gives the same bytes.
    assert torch.equal(ka, kb) and torch.equal(va, vb)
    assert torch.equal(ref, out)


@pytest.mark.gpu
def test_fused_append_with_odd_strided_rows_takes_the_append_launch():
    q, k_pool, v_pool, tables, ctx, k_new, v_new, slots = _case(6, 3, 2, 64, 900, torch.float16, seed=5)
    wide_k = torch.zeros(6, 3, 65, dtype=torch.float16)
    wide_v = torch.zeros(6, 3, 65, dtype=torch.float16)
    wide_k[..., :64], wide_v[..., :64] = k_new, v_new
    kn, vn = wide_k.cuda()[..., :64], wide_v.cuda()[..., :64]  # row stride 195, head stride 65 (odd)
    ref, out, (ka, va), (kb, vb) = _run_both(q, k_pool, v_pool, tables, ctx, kn, vn, slots)
    _check_against_oracle((q, k_pool, v_pool, tables, ctx, k_new, v_new, slots), out, kb, vb)
    assert torch.equal(ka, kb) and torch.equal(va, vb)
    assert torch.equal(ref, out)


@pytest.mark.gpu
def test_fused_append_refuses_a_strided_pool_and_writes_nothing():
    """A pool view whose head_dim is not unit-stride cannot take the rows in place (a
    contiguous copy would swallow them): the call raises before any launch."""
    q, k_pool, v_pool, tables, ctx, k_new, v_new, slots = _case(3, 2, 1, 64, 100, torch.float16, seed=9)
    wide = torch.zeros(2, *k_pool.shape[:3], 128, dtype=torch.float16, device="cuda")
    wide[0, ..., ::2], wide[1, ..., ::2] = k_pool.cuda(), v_pool.cuda()
    kp, vp = wide[0, ..., ::2], wide[1, ..., ::2]                   # head_dim stride 2
    before = wide.clone()
    with pytest.raises(ValueError, match="fused append needs k_pool and v_pool"):
        paged_attention_hip_launch(q.cuda(), kp, vp, tables.cuda(), ctx.cuda(), torch.ones_like(ctx).cuda(),
                                   0.125, append=(k_new.cuda(), v_new.cuda(), slots.cuda()))
    torch.cuda.synchronize()
    assert torch.equal(wide, before)
    # Without the append the same strided pool is read correctly (through a copy).
    out = paged_attention_hip_launch(q.cuda(), kp, vp, tables.cuda(), ctx.cuda(), torch.ones_like(ctx).cuda(), 0.125)
    from oracle.gather import paged_attention_gather

    ref = paged_attention_gather(q, k_pool, v_pool, tables, ctx, torch.ones_like(ctx), 0.125)
    torch.testing.assert_close(out.cpu(), ref, atol=2e-2, rtol=2e-2)


@pytest.mark.gpu
def test_fused_append_rejects_rows_that_do_not_match_the_tokens():
    q, k_pool, v_pool, tables, ctx, k_new, v_new, slots = _case(3, 2, 1, 64, 100, torch.float16, seed=7)
    ql = torch.tensor([1, 2, 1])
    qd = torch.randn(4, 2, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError, match="one new row"):
        paged_attention_hip_launch(qd, k_pool.cuda(), v_pool.cuda(), tables.cuda(), (ctx + 1).cuda(), ql.cuda(),
                                   0.125, append=(k_new.cuda(), v_new.cuda(), slots.cuda()))


def _prefill_case(spans, n_kv, group, d, dtype, seed, spare=5):
    """spans: (cached, new) per sequence. Each sequence owns ceil((cached + new) / 16)
    random blocks; the pool holds random values below each context's new rows and NaN
    from the first new position on (new slots and the unused tail of each last block)."""
    g = torch.Generator().manual_seed(seed)
    bs = 16
    ctx = torch.tensor([c + n for c, n in spans])
    ql = torch.tensor([n for _, n in spans])
    width = int((ctx.max() + bs - 1) // bs)
    n_blocks = len(spans) * width + spare
    perm = torch.randperm(n_blocks, generator=g)
    tables = perm[: len(spans) * width].view(len(spans), width).clone()
    k_pool = torch.randn(n_blocks, bs, n_kv, d, generator=g).to(dtype)
    v_pool = torch.randn(n_blocks, bs, n_kv, d, generator=g).to(dtype)
    slots = []
    for i, (c, n) in enumerate(spans):
        pos = torch.arange(c, width * bs)
        tail = tables[i, pos // bs] * bs + pos % bs
        k_pool.view(-1, n_kv, d)[tail] = float("nan")
        v_pool.view(-1, n_kv, d)[tail] = float("nan")
        slots.append(tail[:n])
    slots = torch.cat(slots)
    n_tok = int(ql.sum())
    q = torch.randn(n_tok, n_kv * group, d, generator=g).to(dtype)
    k_new = torch.randn(n_kv, n_tok, d, generator=g).to(dtype).transpose(0, 1)
    v_new = torch.randn(n_kv, n_tok, d, generator=g).to(dtype).transpose(0, 1)
    return q, k_pool, v_pool, tables, ctx, ql, k_new, v_new, slots


PREFILL_CASES = [
    # (spans, n_kv, group, d, dtype)
    ([(0, 37), (0, 128), (0, 200)], 2, 4, 128, torch.bfloat16),            # fresh prompts
    ([(100, 61), (16, 300), (255, 1), (0, 5)], 12, 1, 64, torch.float16),  # GPT-2 chunks + a decode row
    ([(512, 512), (7, 130)], 2, 8, 128, torch.bfloat16),                   # group 8: KV head over workgroups
    ([(1, 1), (33, 1), (0, 64), (64, 64), (70, 129)], 4, 2, 64, torch.float16),
    ([(40, 50), (0, 19)], 2, 2, 64, torch.float32),                        # fp32: append launch first
    # GQA groups with no MFMA instance (3, 6): the generic kernel reads the pool, so the
    # rows must be appended by the separate launch first.
    ([(0, 40), (17, 90), (200, 1)], 2, 3, 128, torch.bfloat16),
    ([(30, 33), (0, 70)], 2, 6, 64, torch.float16),
]


def _run_prefill_both(q, k_pool, v_pool, tables, ctx, ql, k_new, v_new, slots):
    dev = "cuda"
    qd, td, cd, qld, sd = q.to(dev), tables.to(dev), ctx.to(dev), ql.to(dev), slots.to(dev)
    kn = k_new.transpose(0, 1).contiguous().to(dev).transpose(0, 1)
    vn = v_new.transpose(0, 1).contiguous().to(dev).transpose(0, 1)
    ka, va = k_pool.to(dev), v_pool.to(dev)
    ka.view(-1, *ka.shape[2:])[sd] = kn
    va.view(-1, *va.shape[2:])[sd] = vn
    scale = q.shape[-1] ** -0.5
    ref = paged_attention_hip_launch(qd, ka, va, td, cd, qld, scale)
    kb, vb = k_pool.to(dev), v_pool.to(dev)
    out = paged_attention_hip_launch(qd, kb, vb, td, cd, qld, scale, append=(kn, vn, sd))
    torch.cuda.synchronize()
    return ref, out, (ka, va), (kb, vb)


@pytest.mark.gpu
@pytest.mark.parametrize("spans,n_kv,group,d,dtype", PREFILL_CASES)
def test_fused_prefill_append_matches_oracle_and_append_then_prefill(spans, n_kv, group, d, dtype):
    from oracle.gather import paged_attention_gather
    from oracle.kvops import kv_append

    args = _prefill_case(spans, n_kv, group, d, dtype, seed=len(spans) * 17 + d)
    q, k_pool, v_pool, tables, ctx, ql, k_new, v_new, slots = args
    ref, out, (ka, va), (kb, vb) = _run_prefill_both(*args)
    assert (_raw(kb) == kv_append(_raw(k_pool), _raw(k_new), slots.numpy())).all()
    assert (_raw(vb) == kv_append(_raw(v_pool), _raw(v_new), slots.numpy())).all()
    want = paged_attention_gather(q, kb.cpu(), vb.cpu(), tables, ctx, ql, d ** -0.5)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert not out.isnan().any()
    torch.testing.assert_close(out.cpu(), want, atol=tol, rtol=tol)
    # NaN never equals itself: compare the pools' bits.
    assert (_raw(ka) == _raw(kb)).all() and (_raw(va) == _raw(vb)).all()
    assert torch.equal(ref, out)


@pytest.mark.gpu
def test_fused_prefill_append_with_odd_strided_rows_takes_the_append_launch():
    args = _prefill_case([(20, 45), (0, 70)], 3, 2, 64, torch.float16, seed=11)
    q, k_pool, v_pool, tables, ctx, ql, k_new, v_new, slots = args
    n_tok = int(ql.sum())
    wide_k = torch.zeros(n_tok, 3, 65, dtype=torch.float16)
    wide_v = torch.zeros(n_tok, 3, 65, dtype=torch.float16)
    wide_k[..., :64], wide_v[..., :64] = k_new, v_new
    kn, vn = wide_k.cuda()[..., :64], wide_v.cuda()[..., :64]          # head stride 65 (odd)
    kb, vb = k_pool.cuda(), v_pool.cuda()
    out = paged_attention_hip_launch(q.cuda(), kb, vb, tables.cuda(), ctx.cuda(), ql.cuda(), 0.125,
                                     append=(kn, vn, slots.cuda()))
    ref, _, (ka, va), _ = _run_prefill_both(*args)
    assert (_raw(ka) == _raw(kb)).all() and (_raw(va) == _raw(vb)).all()
    torch.testing.assert_close(out, paged_attention_hip_launch(q.cuda(), ka, va, tables.cuda(), ctx.cuda(),
                                                               ql.cuda(), 0.125), atol=0, rtol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("graphs", [True, False])
def test_decode_steps_with_fused_append_match_separate_append(monkeypatch, graphs):
    """GPT-2 fp16, config 5's shape (24 requests), prefill and decode steps replayed
    from graphs or issued eagerly: fused append vs the per-layer append launch give
    identical token streams."""
    from inference_server.bench import workload
    from inference_server.config import CONFIG
    from inference_server.engine.paged import PagedEngine
    from inference_server.model import load

    monkeypatch.setattr(CONFIG, "attention", "hip")
    monkeypatch.setattr(CONFIG, "decode_graphs", graphs)
    monkeypatch.setattr(CONFIG, "prefill_graphs", graphs)
    # The QKV-epilogue projection rounds in its own order; this test isolates the
    # attention-side append, so both runs keep the model's own projection.
    monkeypatch.setattr(CONFIG, "qkv_epilogue", False)
    model, tok = load(dtype=torch.float16, device="cuda")
    reqs = workload.config5(n=24)
    for r in reqs:
        r.max_tokens = min(r.max_tokens, 40)
    outs = []
    for fused in (True, False):
        monkeypatch.setattr(CONFIG, "fused_append", fused)
        engine = PagedEngine(model, tok, num_blocks=1024, block_size=16, device="cuda")
        try:
            assert engine.executor.fuse_append == fused
            outs.append(engine.run(reqs))
        finally:
            engine.shutdown()
    assert outs[0].generated_tokens == sum(r.max_tokens for r in reqs)
    assert outs[0].outputs == outs[1].outputs
