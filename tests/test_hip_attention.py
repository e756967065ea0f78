"""HIP paged attention vs the oracle gather path, through libpagedkv's C ABI.

Mirrors the reference's kernel tier (tests/test_paged_attention_triton.py:164-230):
every batch shape in CASES, production block size / head dim, GQA, non-power-of-two
sizes, 0-padded tables that point at live blocks, a strided query, the empty batch —
plus the BASELINE shapes: config 2 (fp16 decode, 64 x 12 heads x d64, lognormal
contexts) at full size, config 4 (Llama-3-8B-shaped bf16 GQA decode, contexts up to
8192, and chunked prefill) at full size on the bench's own workloads, every output row
checked.

Tolerances are the north-star bars: rtol = atol = 1e-5 in fp32 and 2e-2 in fp16/bf16
against the gather path (the kernels accumulate P·V in fp32 and round their
probabilities against a running max, the gather path rounds normalised ones), and
2.5e-6 in fp32 against the block-order online oracle (oracle/online.py).
"""

from __future__ import annotations

import inspect
import math

import numpy as np
import pytest
import torch

from cases import CASES, build, dense_causal_f64
from inference_server.config import CONFIG
from inference_server.core import attention
from inference_server.core.attention import paged_attention, paged_attention_hip
from inference_server.core.attention_hip import attach_host
from oracle.gather import paged_attention_gather as oracle_gather

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _compare(lengths, *, dtype=torch.float32, **kw):
    q, kp, vp, tables, ctx, ql = build(lengths, dtype=dtype, device="cuda", **kw)
    scale = q.shape[-1] ** -0.5
    out = paged_attention_hip(q, kp, vp, tables, ctx, ql, scale)
    torch.cuda.synchronize()
    ref = oracle_gather(q, kp, vp, tables, ctx, ql, scale)
    assert out.shape == ref.shape and out.dtype == q.dtype and out.device == q.device
    tol = TOL[dtype]
    torch.testing.assert_close(out.cpu(), ref, atol=tol, rtol=tol)
    return out


@pytest.mark.parametrize("case", list(CASES))
def test_cases_fp32(case):
    _compare(CASES[case])


@pytest.mark.parametrize("case", list(CASES))
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_cases_half(case, dtype):
    _compare(CASES[case], dtype=dtype)


#: fp32 kernels against the block-order online oracle (oracle/online.py, the restated
#: mirror of the reference kernel, core/attention_triton.py:309-384): a bar 4x tighter
#: than the gather path's 1e-5. Both fold keys into a running (max, sum, numerator) in
#: fp32; they differ only in summation order inside a block, the partition split and
#: exp2 on pre-multiplied scores against exp.
ONLINE_TOL = 2.5e-6

ONLINE_SHAPES = {
    **{name: (lengths, {}) for name, lengths in CASES.items()},
    "bs16_d64_decode": ([(300, 1), (16, 1), (129, 1), (1, 1), (17, 1)], dict(bs=16, d=64, num_blocks=128)),
    "bs16_d64_mixed": ([(300, 1), (16, 16), (129, 1), (64, 40)], dict(bs=16, d=64, num_blocks=128)),
    "bs16_d128_gqa4_decode": ([(700, 1), (33, 1), (257, 1), (512, 1)],
                              dict(bs=16, d=128, heads=8, kv_heads=2, num_blocks=128)),
    "bs16_d128_gqa4_prefill": ([(90, 90), (200, 31)], dict(bs=16, d=128, heads=8, kv_heads=2, num_blocks=128)),
}


@pytest.mark.parametrize("name", list(ONLINE_SHAPES))
def test_fp32_kernels_match_the_online_order_oracle(name):
    from oracle.online import paged_attention_online

    lengths, kw = ONLINE_SHAPES[name]
    q, kp, vp, tables, ctx, ql = build(lengths, dtype=torch.float32, device="cuda", **kw)
    scale = q.shape[-1] ** -0.5
    out = paged_attention_hip(q, kp, vp, tables, ctx, ql, scale).cpu().numpy()
    want = paged_attention_online(*(t.cpu().numpy() for t in (q, kp, vp, tables, ctx, ql)), scale)
    err = np.abs(out - want).max()
    np.testing.assert_allclose(out, want, rtol=ONLINE_TOL, atol=ONLINE_TOL, err_msg=f"max abs err {err:.3g}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_production_block_size_and_head_dim(dtype):
    """bs 16, d 64 (gpt2) — the tuned decode kernel's shape — with multi-block contexts."""
    _compare([(300, 1), (16, 16), (129, 1), (64, 40)], bs=16, d=64, dtype=dtype, num_blocks=128)
    _compare([(300, 1), (16, 1), (129, 1), (1, 1), (17, 1)], bs=16, d=64, dtype=dtype, num_blocks=128)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_tuned_decode_gqa_groups(dtype, d, group):
    """Every (head_dim, GQA group) the tuned decode kernel instantiates, with contexts
    on both sides of the 256-token split-KV partition boundaries (1 to 5 partitions)."""
    lengths = [(1, 1), (255, 1), (256, 1), (257, 1), (513, 1), (1100, 1), (37, 1)]
    _compare(lengths, bs=16, d=d, heads=2 * group, kv_heads=2, dtype=dtype, num_blocks=256)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_tuned_prefill_gqa_groups(dtype, d, group):
    """Every shape the MFMA prefill kernel instantiates: full prefills, chunks onto a
    cached prefix, partial 32-query tiles, a 1-token decode row in the same batch, and
    contexts crossing several 64-key tiles."""
    lengths = [(70, 70), (300, 45), (33, 33), (129, 1), (200, 200), (1, 1), (97, 64)]
    _compare(lengths, bs=16, d=d, heads=2 * group, kv_heads=2, dtype=dtype, num_blocks=256)


#: fp32 pools at block size 16 and head_dim 64/128: prefill, chunks and mixed batches
#: run on the fp32 MFMA kernel (csrc/attn_prefill_f32.hip), decode at head_dim 128 on
#: the tiled fp32 kernel (csrc/attn_f32.hip). These shapes were written for the tiled
#: kernel's lane shapes and now also cover the MFMA kernel's prefill tiles.
F32_SMALL = [(70, 70), (300, 45), (33, 33), (129, 1), (1, 1), (97, 64), (17, 17), (16, 16)]


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_fp32_tiled_kernel_small_batches(d, group):
    from oracle.online import paged_attention_online

    out = _compare(F32_SMALL, bs=16, d=d, heads=2 * group, kv_heads=2, num_blocks=256)
    q, kp, vp, tables, ctx, ql = build(F32_SMALL, bs=16, d=d, heads=2 * group, kv_heads=2, num_blocks=256)
    want = paged_attention_online(*(t.numpy() for t in (q, kp, vp, tables, ctx, ql)), d ** -0.5)
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=ONLINE_TOL, atol=ONLINE_TOL)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("group", [1, 8])
def test_fp32_tiled_kernel_large_batches(d, group):
    """16 kv heads x 20 sequences of 96-160 new tokens onto 0-200 cached ones: enough
    waves for the widest lane shape."""
    rng = np.random.default_rng(d + group)
    lengths = [(int(c) + int(n), int(n)) for c, n in zip(rng.integers(0, 200, 20), rng.integers(96, 161, 20))]
    _compare(lengths, bs=16, d=d, heads=16 * group, kv_heads=16, num_blocks=512)


#: fp32 prefill / chunked-prefill batches run on the fp32 MFMA kernel
#: (csrc/attn_prefill_f32.hip): 32-key tiles, 32-query tiles, every GQA group and head
#: dim it instantiates; contexts crossing many tiles, tiles cut by the context end and
#: by the causal bound, 1-token rows in the same batch, and a query block starting past
#: a 32-query tile boundary. Against the gather path at 1e-5 and the block-order online
#: oracle at 2.5e-6.
F32_MFMA = [(1000, 1000), (777, 130), (33, 33), (64, 64), (65, 1), (2049, 300), (5, 5), (96, 33)]


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_fp32_mfma_prefill(d, group):
    from oracle.online import paged_attention_online

    kw = dict(bs=16, d=d, heads=2 * group, kv_heads=2, num_blocks=512)
    out = _compare(F32_MFMA, **kw)
    q, kp, vp, tables, ctx, ql = build(F32_MFMA, **kw)
    want = paged_attention_online(*(t.numpy() for t in (q, kp, vp, tables, ctx, ql)), d ** -0.5)
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=ONLINE_TOL, atol=ONLINE_TOL)


@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_fp32_decode_head_dim_128(group):
    """fp32 decode at head_dim 128 (no register decode kernel at that size): the tiled
    fp32 kernel with the GQA group's heads in the lanes."""
    lengths = [(1, 1), (255, 1), (256, 1), (257, 1), (513, 1), (1100, 1), (37, 1)]
    _compare(lengths, bs=16, d=128, heads=2 * group, kv_heads=2, num_blocks=256)


def test_in_kernel_merge_returns_its_counters_to_zero():
    """Ragged 16-bit decode batches merge their split-KV partials inside the partition
    kernel, counting partitions in per (sequence, KV head) in the workspace's first
    256 KiB. After every call those counters are zero again (the next call depends on
    it), and repeated calls give the same bits; checked against the oracle too."""
    from inference_server.core.attention_hip import _WORKSPACES

    rng = np.random.default_rng(11)
    # Up to 3 partitions of 768 tokens: the in-kernel merge for any number of pairs.
    lengths = [(int(c), 1) for c in rng.integers(1, 2300, size=64)]
    for dtype, d, kvh, heads in ((torch.float16, 64, 12, 12), (torch.bfloat16, 128, 2, 8)):
        first = _compare(lengths, bs=16, d=d, heads=heads, kv_heads=kvh, dtype=dtype, num_blocks=8192)
        q, kp, vp, tables, ctx, ql = build(lengths, bs=16, d=d, heads=heads, kv_heads=kvh, dtype=dtype,
                                           device="cuda", num_blocks=8192)
        dev = torch.device("cuda")
        ws = _WORKSPACES.partials(dev, torch.cuda.current_stream().cuda_stream, 0)
        for _ in range(5):
            out = paged_attention_hip(q, kp, vp, tables, ctx, ql, d ** -0.5)
            torch.cuda.synchronize()
            assert torch.equal(out, first)
            assert int(ws[: 256 * 1024].count_nonzero()) == 0


def test_grouped_query_heads():
    _compare([(9, 9), (5, 1), (12, 3)], kv_heads=1)


def test_non_power_of_two_sizes():
    _compare([(13, 13), (7, 1), (18, 4)], bs=6, d=12)


def test_block_table_padding_is_never_read():
    """0-padded rows point at block 0, which another sequence owns; poison every
    block beyond each sequence's context and the result must not change."""
    for seed in range(3):
        q, kp, vp, tables, ctx, ql = build(CASES["padding_hits_block0"], seed=seed, device="cuda")
        scale = q.shape[-1] ** -0.5
        ref = paged_attention_hip(q, kp, vp, tables, ctx, ql, scale)
        used = set()
        for i, c in enumerate(ctx.tolist()):
            used.update(tables[i, : -(-c // kp.shape[1])].tolist())
        unused = [b for b in range(kp.shape[0]) if b not in used]
        kp2, vp2 = kp.clone(), vp.clone()
        kp2[unused] = float("nan")
        vp2[unused] = float("nan")
        out = paged_attention_hip(q, kp2, vp2, tables, ctx, ql, scale)
        assert torch.equal(out, ref)


def test_tail_of_last_block_is_never_read():
    """Slots past context_len inside a sequence's last block hold garbage (a previous
    tenant's KV, or NaN); they must not contribute."""
    q, kp, vp, tables, ctx, ql = build([(21, 1), (300, 1), (5, 5)], bs=16, d=64, device="cuda", num_blocks=64)
    scale = 0.125
    ref = paged_attention_hip(q, kp, vp, tables, ctx, ql, scale)
    kp2, vp2 = kp.clone(), vp.clone()
    for i, c in enumerate(ctx.tolist()):
        last = int(tables[i, (c - 1) // 16])
        kp2[last, c % 16 or 16:] = float("nan")
        vp2[last, c % 16 or 16:] = float("nan")
    out = paged_attention_hip(q, kp2, vp2, tables, ctx, ql, scale)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128])
def test_tuned_prefill_reads_only_live_rows_and_takes_strided_queries(dtype, d):
    """The MFMA prefill kernels (fp32 and 16-bit) at block size 16: NaN in every block no
    sequence uses and in every slot past a context's end changes no output bit, and a
    query tensor with the executor's transposed strides gives the same bits as a
    contiguous one."""
    lengths = [(70, 70), (300, 45), (33, 33), (129, 1), (21, 21), (16, 16)]
    q, kp, vp, tables, ctx, ql = build(lengths, bs=16, d=d, heads=8, kv_heads=2, dtype=dtype, device="cuda",
                                       num_blocks=128)
    scale = d ** -0.5
    ref = paged_attention_hip(q, kp, vp, tables, ctx, ql, scale)
    torch.testing.assert_close(ref.cpu(), oracle_gather(q, kp, vp, tables, ctx, ql, scale), atol=TOL[dtype],
                               rtol=TOL[dtype])
    used = set()
    kp2, vp2 = kp.clone(), vp.clone()
    for i, c in enumerate(ctx.tolist()):
        used.update(tables[i, : -(-c // 16)].tolist())
        last = int(tables[i, (c - 1) // 16])
        kp2[last, c % 16 or 16:] = float("nan")
        vp2[last, c % 16 or 16:] = float("nan")
    unused = [b for b in range(kp.shape[0]) if b not in used]
    kp2[unused] = float("nan")
    vp2[unused] = float("nan")
    assert torch.equal(paged_attention_hip(q, kp2, vp2, tables, ctx, ql, scale), ref)
    strided = q.transpose(0, 1).contiguous().transpose(0, 1)
    assert not strided.is_contiguous()
    assert torch.equal(paged_attention_hip(strided, kp, vp, tables, ctx, ql, scale), ref)


def test_accepts_non_contiguous_query():
    """The executor hands over `query[0].transpose(0, 1)` (reference
    core/paged_executor.py:146); the strides pass through without a copy."""
    for lengths in (CASES["mixed"], CASES["decode_ragged"]):
        q, kp, vp, tables, ctx, ql = build(lengths, device="cuda")
        scale = q.shape[-1] ** -0.5
        strided = q.transpose(0, 1).contiguous().transpose(0, 1)
        assert not strided.is_contiguous()
        out = paged_attention_hip(strided, kp, vp, tables, ctx, ql, scale)
        ref = oracle_gather(q, kp, vp, tables, ctx, ql, scale)
        torch.testing.assert_close(out.cpu(), ref, atol=1e-5, rtol=1e-5)


def test_empty_batch():
    q = torch.empty(0, 3, 8, device="cuda")
    pool = torch.zeros(4, 4, 3, 8, device="cuda")
    zero = torch.zeros(0, dtype=torch.long, device="cuda")
    out = paged_attention_hip(q, pool, pool, torch.zeros(0, 1, dtype=torch.long, device="cuda"), zero, zero, 0.5)
    assert out.shape == (0, 3, 8)


def test_host_metadata_gives_the_same_answer():
    """Attached host copies of the lengths skip the device round trip; same result."""
    q, kp, vp, tables, ctx, ql = build(CASES["mixed"], device="cuda")
    scale = q.shape[-1] ** -0.5
    a = paged_attention_hip(q, kp, vp, tables, ctx, ql, scale)
    attach_host(ctx, ctx.cpu())
    attach_host(ql, ql.cpu())
    b = paged_attention_hip(q, kp, vp, tables, ctx, ql, scale)
    assert torch.equal(a, b)


def test_contract_errors_match_the_reference():
    q, kp, vp, tables, ctx, ql = build([(4, 4), (2, 2)], device="cuda")
    with pytest.raises(ValueError, match="query_len exceeds context_len"):
        paged_attention_hip(q, kp, vp, tables, ctx - 1, ql, 0.5)
    with pytest.raises(ValueError, match="query_lens sum"):
        paged_attention_hip(q[:-1], kp, vp, tables, ctx, ql, 0.5)
    with pytest.raises(ValueError, match="more blocks than its block_tables row holds"):
        paged_attention_hip(q, kp, vp, tables[:, :0], ctx, ql, 0.5)


def test_dispatcher_routes_hip(monkeypatch):
    q, kp, vp, tables, ctx, ql = build(CASES["mixed"], device="cuda")
    scale = q.shape[-1] ** -0.5
    monkeypatch.setattr(CONFIG, "attention", "hip")
    out = paged_attention(q, kp, vp, tables, ctx, ql, scale)
    torch.testing.assert_close(out.cpu(), oracle_gather(q, kp, vp, tables, ctx, ql, scale), atol=1e-5, rtol=1e-5)
    sig = list(inspect.signature(paged_attention).parameters)
    assert list(inspect.signature(attention.paged_attention_hip).parameters) == sig


def test_repeated_calls_reuse_the_workspace():
    """Many calls on one cached split-KV workspace give the same bits."""
    q, kp, vp, tables, ctx, ql = build([(2000, 1), (700, 1), (513, 1)], bs=16, d=128, heads=8, kv_heads=2,
                                       dtype=torch.bfloat16, device="cuda", num_blocks=256)
    first = paged_attention_hip(q, kp, vp, tables, ctx, ql, 0.1)
    for _ in range(20):
        assert torch.equal(paged_attention_hip(q, kp, vp, tables, ctx, ql, 0.1), first)


@pytest.mark.parametrize("dtype,d,group", [(torch.bfloat16, 64, 4), (torch.float16, 128, 1)])
def test_streaming_decode_repeats_bit_identical(dtype, d, group):
    """The streaming decode kernel is deterministic: 30 calls on a batch of 128
    sequences with contexts of 1-2400 tokens (single- and multi-partition sequences,
    partition and merge kernels, the first round of workgroups included) give the same
    bits every time."""
    rng = np.random.default_rng(3)
    batch, kv = 128, 8
    ctx = rng.integers(1, 2400, size=batch)
    nb = int(((ctx + 15) // 16).sum()) + 8
    q, tables, ctx_t = _random_decode(batch, kv * group, kv, d, ctx, nb, dtype, seed=3)
    kp, vp = _fill_pool(nb, kv, d, dtype, 3)
    ql = torch.ones(batch, dtype=torch.long).cuda()
    q, tables, ctx_t = q.cuda(), tables.cuda(), ctx_t.cuda()
    first = paged_attention_hip(q, kp, vp, tables, ctx_t, ql, d ** -0.5)
    for i in range(30):
        again = paged_attention_hip(q, kp, vp, tables, ctx_t, ql, d ** -0.5)
        assert torch.equal(again, first), f"call {i + 1}: {int((again != first).sum())} elements differ"


def test_chunked_prefill_repeats_bit_identical():
    """The MFMA prefill kernel is deterministic: 10 chunked-prefill calls (8 sequences,
    256-token chunks onto contexts of 0-1500 tokens, GQA 4, d128, bf16) give the same bits."""
    rng = np.random.default_rng(4)
    c0 = rng.integers(0, 1501, size=8)
    ctx = c0 + 256
    q, tables, ctx_t = _random_decode(8, 32, 8, 128, ctx, int(((ctx + 15) // 16).sum()) + 8, torch.bfloat16, seed=4)
    kp, vp = _fill_pool(tables.shape[0] * tables.shape[1] + 8, 8, 128, torch.bfloat16, 4)
    g = torch.Generator().manual_seed(4)
    qp = torch.randn(8 * 256, 32, 128, generator=g).to(torch.bfloat16).cuda()
    ql = torch.full((8,), 256, dtype=torch.long).cuda()
    tables, ctx_t = tables.cuda(), ctx_t.cuda()
    first = paged_attention_hip(qp, kp, vp, tables, ctx_t, ql, 128 ** -0.5)
    for i in range(10):
        assert torch.equal(paged_attention_hip(qp, kp, vp, tables, ctx_t, ql, 128 ** -0.5), first), f"call {i + 1}"


# --------------------------------------------------------------------- BASELINE configs
def _random_decode(batch, heads, kv_heads, d, ctx_lens, num_blocks, dtype, seed=1337):
    """Seeded decode batch: block tables are slices of one permutation of the pool."""
    g = torch.Generator().manual_seed(seed)
    bs = 16
    ctx = torch.as_tensor(ctx_lens, dtype=torch.long)
    nblk = (ctx + bs - 1) // bs
    width = int(nblk.max())
    perm = torch.randperm(num_blocks, generator=g)
    tables = torch.zeros(batch, width, dtype=torch.long)
    off = 0
    for i in range(batch):
        n = int(nblk[i])
        tables[i, :n] = perm[off:off + n]
        off += n
    q = torch.randn(batch, heads, d, generator=g).to(dtype)
    return q, tables, ctx


def _fill_pool(num_blocks, kv_heads, d, dtype, seed):
    torch.cuda.manual_seed(seed)
    kp = torch.randn(num_blocks, 16, kv_heads, d, device="cuda", dtype=dtype)
    vp = torch.randn(num_blocks, 16, kv_heads, d, device="cuda", dtype=dtype)
    return kp, vp


def test_config2_fp16_decode_full_size():
    """BASELINE config 2 at full size: 64 sequences, 12 heads, d64, fp16, lognormal
    contexts (median 300, sigma 0.9, clipped to [16, 2048]), 8192-block pool."""
    rng = np.random.default_rng(1337)
    ctx = np.clip(np.round(np.exp(rng.normal(math.log(300), 0.9, 64))), 16, 2048).astype(np.int64)
    q, tables, ctx_t = _random_decode(64, 12, 12, 64, ctx, 8192, torch.float16)
    kp, vp = _fill_pool(8192, 12, 64, torch.float16, 2)
    ql = torch.ones(64, dtype=torch.long)
    out = paged_attention_hip(q.cuda(), kp, vp, tables.cuda(), ctx_t.cuda(), ql.cuda(), 1 / 8)
    ref = oracle_gather(q, kp, vp, tables, ctx_t, ql, 1 / 8)
    torch.testing.assert_close(out.cpu(), ref, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("dtype,d,heads,kv", [(torch.bfloat16, 128, 32, 8), (torch.float32, 64, 12, 12)])
@pytest.mark.parametrize("n_seqs,tied", [(200, True), (257, False), (300, False)])
def test_prefill_dispatch_order_large_and_tied_batches(dtype, d, heads, kv, n_seqs, tied):
    """The MFMA prefill kernels (bf16 and fp32) run a batch's sequences longest context
    first when it has at most 256 of them (each workgroup ranks the contexts, ties by
    index) and in index order beyond: 200 sequences that all share one context length
    (every rank decided by the tie-break), and 257 / 300 sequences of ragged chunks (the
    index-order path). Every row against oracle.gather."""
    rng = np.random.default_rng(n_seqs + d)
    if tied:
        lengths = [(96, int(q)) for q in rng.integers(1, 97, size=n_seqs)]
    else:
        ctx = rng.integers(2, 161, size=n_seqs)
        lengths = [(int(c), int(rng.integers(2, min(int(c), 40) + 1))) for c in ctx]
    _compare(lengths, dtype=dtype, bs=16, d=d, heads=heads, kv_heads=kv, num_blocks=4096, seed=n_seqs)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_large_batch_of_short_contexts(dtype):
    """A large batch of short contexts: 4100 sequences of 1 to 700 tokens (1 to 3
    partitions, so most workgroups of the partition grid are empty), GQA group 2, d64;
    40 seeded rows re-derived by the CPU oracle."""
    rng = np.random.default_rng(7)
    batch = 4100
    ctx = rng.integers(1, 701, size=batch)
    nb = int(((ctx + 15) // 16).sum()) + 8
    q, tables, ctx_t = _random_decode(batch, 4, 2, 64, ctx, nb, dtype, seed=11)
    kp, vp = _fill_pool(nb, 2, 64, dtype, 5)
    ql = torch.ones(batch, dtype=torch.long)
    out = paged_attention_hip(q.cuda(), kp, vp, tables.cuda(), ctx_t.cuda(), ql.cuda(), 0.125).cpu()
    pick = sorted(set(rng.choice(batch, size=36, replace=False).tolist() + [0, batch - 1, int(np.argmax(ctx)),
                                                                            int(np.argmin(ctx))]))
    for i in pick:
        c = int(ctx_t[i])
        used = tables[i, : -(-c // 16)]
        ref = oracle_gather(q[i:i + 1], kp[used.cuda()].cpu(), vp[used.cuda()].cpu(),
                            torch.arange(len(used))[None], ctx_t[i:i + 1], ql[:1], 0.125)
        torch.testing.assert_close(out[i:i + 1], ref, atol=2e-2, rtol=2e-2, msg=lambda m: f"seq {i}: {m}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d,kv,batch,top", [(128, 2, 40, 3000), (128, 2, 16, 1100), (64, 4, 24, 2000)])
@pytest.mark.parametrize("group", [1, 4, 8])
def test_short_partition_decode_wave_counts(dtype, d, kv, batch, top, group):
    """Launches too small for 768-token partitions take 256-token ones, with 8 waves x
    32 tokens where the workgroups fit one round (head_dim 64, or at most 512
    workgroups at 128) and 4 waves x 64 tokens otherwise: the first case here (40
    sequences x 2 KV heads, up to 12 partitions = 960 workgroups, d128) takes 4 waves,
    the other two take 8. Sampled rows against the CPU oracle, and 10 repeated calls
    bit-identical."""
    rng = np.random.default_rng(group * 10 + d + batch)
    ctx = rng.integers(1, top, size=batch)
    ctx[:4] = [255, 256, 257, top - 1]
    nb = int(((ctx + 15) // 16).sum()) + 8
    q, tables, ctx_t = _random_decode(batch, kv * group, kv, d, ctx, nb, dtype, seed=group + d)
    kp, vp = _fill_pool(nb, kv, d, dtype, d + group)
    ql = torch.ones(batch, dtype=torch.long)
    qd, td, cd, qld = q.cuda(), tables.cuda(), ctx_t.cuda(), ql.cuda()
    out = paged_attention_hip(qd, kp, vp, td, cd, qld, d ** -0.5)
    for _ in range(10):
        assert torch.equal(paged_attention_hip(qd, kp, vp, td, cd, qld, d ** -0.5), out)
    out = out.cpu()
    pick = sorted(set(rng.choice(batch, size=6, replace=False).tolist() + [0, 1, 2, 3]))
    for i in pick:
        c = int(ctx_t[i])
        used = tables[i, : -(-c // 16)]
        ref = oracle_gather(q[i:i + 1], kp[used.cuda()].cpu(), vp[used.cuda()].cpu(),
                            torch.arange(len(used))[None], ctx_t[i:i + 1], ql[:1], d ** -0.5)
        torch.testing.assert_close(out[i:i + 1], ref, atol=2e-2, rtol=2e-2, msg=lambda m: f"seq {i}: {m}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_long_partition_decode_every_group(dtype, d, group):
    """128 sequences x 8 KV heads: enough workgroups for the 768-token stream
    partitions (small batches, as in test_tuned_decode_gqa_groups, take the 256-token
    ones). Contexts straddle partition edges (767, 768, 769, 1536, 1537) and run to four
    partitions; 14 rows re-derived by the CPU oracle."""
    rng = np.random.default_rng(group * 100 + d)
    batch, kv = 128, 8
    ctx = rng.integers(1, 2400, size=batch)
    ctx[:5] = [767, 768, 769, 1536, 1537]
    nb = int(((ctx + 15) // 16).sum()) + 8
    q, tables, ctx_t = _random_decode(batch, kv * group, kv, d, ctx, nb, dtype, seed=group)
    kp, vp = _fill_pool(nb, kv, d, dtype, d)
    ql = torch.ones(batch, dtype=torch.long)
    out = paged_attention_hip(q.cuda(), kp, vp, tables.cuda(), ctx_t.cuda(), ql.cuda(), d ** -0.5).cpu()
    pick = sorted(set(rng.choice(batch, size=9, replace=False).tolist() + [0, 1, 2, 3, 4]))
    for i in pick:
        c = int(ctx_t[i])
        used = tables[i, : -(-c // 16)]
        ref = oracle_gather(q[i:i + 1], kp[used.cuda()].cpu(), vp[used.cuda()].cpu(),
                            torch.arange(len(used))[None], ctx_t[i:i + 1], ql[:1], d ** -0.5)
        torch.testing.assert_close(out[i:i + 1], ref, atol=2e-2, rtol=2e-2, msg=lambda m: f"seq {i}: {m}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_long_partition_separate_merge_every_group(dtype, d, group):
    """32 sequences x 8 KV heads of 2,400-3,500 tokens (four or five 768-token
    partitions, at most 512 (sequence, KV head) pairs): the 4-wave 768-token kernel with
    the separate merge kernel, which grouped heads take only in this regime (with the
    in-kernel merge they run 8 waves per partition). 10 rows re-derived by the CPU
    oracle."""
    rng = np.random.default_rng(group * 10 + d + 7)
    batch, kv = 32, 8
    ctx = rng.integers(2400, 3501, size=batch)
    ctx[:3] = [2305, 3072, 3073]
    nb = int(((ctx + 15) // 16).sum()) + 8
    q, tables, ctx_t = _random_decode(batch, kv * group, kv, d, ctx, nb, dtype, seed=group + 40)
    kp, vp = _fill_pool(nb, kv, d, dtype, d + 1)
    ql = torch.ones(batch, dtype=torch.long)
    out = paged_attention_hip(q.cuda(), kp, vp, tables.cuda(), ctx_t.cuda(), ql.cuda(), d ** -0.5).cpu()
    rows = sorted(set(rng.choice(batch, size=7, replace=False).tolist() + [0, 1, 2]))
    _check_rows(out, q, kp, vp, tables, ctx_t, rows, d ** -0.5)


def _check_rows(out, q, kp, vp, tables, ctx_t, rows, scale):
    ql = torch.ones(1, dtype=torch.long)
    for i in rows:
        c = int(ctx_t[i])
        used = tables[i, : -(-c // 16)]
        ref = oracle_gather(q[i:i + 1], kp[used.cuda()].cpu(), vp[used.cuda()].cpu(),
                            torch.arange(len(used))[None], ctx_t[i:i + 1], ql, scale)
        torch.testing.assert_close(out[i:i + 1], ref, atol=2e-2, rtol=2e-2, msg=lambda m: f"seq {i}: {m}")


def test_decode_many_tiny_contexts_around_long_ones():
    """1000 sequences of 1-40 tokens (chunk and block edges 8, 16, 24, 32 included:
    one partial chunk, whole chunks, whole blocks) around ten long ones (3000-6000
    tokens, 4-8 partitions merged); fp16, d64, GQA 4. 40 rows re-derived by the CPU
    oracle, short and long."""
    rng = np.random.default_rng(21)
    batch, kv, group, d = 1000, 2, 4, 64
    ctx = rng.integers(1, 41, size=batch)
    ctx[:4] = [8, 16, 24, 32]
    long_rows = rng.choice(np.arange(4, batch), size=10, replace=False)
    ctx[long_rows] = rng.integers(3000, 6001, size=10)
    nb = int(((ctx + 15) // 16).sum()) + 8
    q, tables, ctx_t = _random_decode(batch, kv * group, kv, d, ctx, nb, torch.float16, seed=21)
    kp, vp = _fill_pool(nb, kv, d, torch.float16, 21)
    ql = torch.ones(batch, dtype=torch.long)
    out = paged_attention_hip(q.cuda(), kp, vp, tables.cuda(), ctx_t.cuda(), ql.cuda(), d ** -0.5).cpu()
    rows = sorted(set(rng.choice(batch, size=26, replace=False).tolist() + [0, 1, 2, 3, batch - 1]
                      + long_rows[:9].tolist()))
    _check_rows(out, q, kp, vp, tables, ctx_t, rows, d ** -0.5)


def test_decode_contexts_of_16k_to_24k_tokens():
    """48 sequences of 16-24k tokens, 8 KV heads, GQA 4, d128, bf16: 21-32 partitions
    per sequence, so the merge takes more than one 16-partition batch of loads. 6 rows
    re-derived by the CPU oracle."""
    rng = np.random.default_rng(22)
    batch, kv, group, d = 48, 8, 4, 128
    ctx = rng.integers(16000, 24001, size=batch)
    nb = int(((ctx + 15) // 16).sum()) + 8
    q, tables, ctx_t = _random_decode(batch, kv * group, kv, d, ctx, nb, torch.bfloat16, seed=22)
    kp, vp = _fill_pool(nb, kv, d, torch.bfloat16, 22)
    ql = torch.ones(batch, dtype=torch.long)
    out = paged_attention_hip(q.cuda(), kp, vp, tables.cuda(), ctx_t.cuda(), ql.cuda(), d ** -0.5).cpu()
    rows = sorted(set(rng.choice(batch, size=4, replace=False).tolist() + [0, batch - 1]))
    _check_rows(out, q, kp, vp, tables, ctx_t, rows, d ** -0.5)


def test_config4_bf16_gqa_decode_whole_batch():
    """BASELINE config 4 decode at full size, on the bench's own workload
    (bench.config4_decode: 128 sequences, 32/8 heads, d128, bf16, contexts U[512, 8192]
    seeded 1337, a 65536-block pool): the exact C-ABI call the bench times, then every
    one of the 128 output rows against the CPU oracle (each row depends only on its own
    sequence, so it is re-derived from that sequence's blocks). The product entry point
    paged_attention_hip gives the same bytes."""
    import bench

    w = bench.config4_decode()
    call = w.make_call()
    call()
    call()                      # a second call on the same workspace (merge counters reused)
    torch.cuda.synchronize()
    worst = bench.check_decode_whole(w, w.out)
    assert worst < 2e-2
    kp, vp = w.pools[0]
    out = paged_attention_hip(w.q, kp, vp, w.tables, w.ctx_dev, w.ql_dev, w.scale)
    assert torch.equal(out, w.out)


def test_config4_bf16_chunked_prefill_whole_batch():
    """BASELINE config 4 chunked prefill on the bench's own workload
    (bench.PrefillWorkload: 16 sequences x 512-token chunks onto cached contexts
    U[0, 4096], 65536-block pool, seed 1337): the exact C-ABI call the bench times,
    then all 16 chunks against the CPU oracle at 2e-2; paged_attention_hip gives the
    same bytes."""
    import bench

    wp = bench.PrefillWorkload()
    wp.make_call()()
    torch.cuda.synchronize()
    worst = bench.check_prefill_whole(wp, wp.out)
    assert worst < 2e-2
    out = paged_attention_hip(wp.q, wp.kp, wp.vp, wp.tables, wp.ctx_dev, wp.ql.cuda(), wp.d ** -0.5)
    assert torch.equal(out, wp.out)


def test_textbook_dense_agrees_on_gpu_output():
    """Closes the loop without the gather restatement: HIP fp32 vs float64 dense."""
    q, kp, vp, tables, ctx, ql = build(CASES["mixed"], bs=16, d=64, device="cuda", num_blocks=32)
    out = paged_attention_hip(q, kp, vp, tables, ctx, ql, 0.125).cpu().double().numpy()
    ref = dense_causal_f64(q, kp, vp, tables, ctx, ql, 0.125)
    np.testing.assert_allclose(out, ref, atol=1e-5, rtol=1e-5)
