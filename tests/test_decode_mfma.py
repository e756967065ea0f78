"""The persistent MFMA decode kernel (csrc/attn_decode_mfma.hip) against the oracle.

The library routes a decode batch to this kernel when its pools are fp16/bf16 with
block size 16, head_dim 64/128, GQA 1/2/4/8, a multiple of 4 KV heads, at most 1024
sequences and batch x KV heads x longest context x head_dim x 4 bytes >= 512 MiB (the
K/V the launch may read). Every case below meets that, and each
exercises a different part of the kernel's work split (equal runs of 16-key blocks
over the flattened batch, cut anywhere): waves per workgroup 8 (KV heads a multiple
of 8) and 4 (KV-head groups walked one after another), partial last blocks (contexts
of 1, 15, 16, 17 tokens), many short sequences inside one run, sequences cut into
several pieces whose partials are merged, and a fused append. Every output row is
checked against oracle.gather at 2e-2, the reference gather path's tolerance for 16-bit
pools (reference tests/test_paged_attention_triton.py:168-178). Two calls in a row on
one workspace must give the same bytes (the kernel's partials and prefix table are
rewritten by every call; the merge combines pieces in a fixed order).
"""

from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

from inference_server.core.attention import paged_attention_hip
from oracle.gather import paged_attention_gather as oracle_gather

pytestmark = pytest.mark.gpu

BS = 16


def _batch(batch, kv_heads, group, d, ctx, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.as_tensor(np.asarray(ctx), dtype=torch.long)
    nblk = (ctx + BS - 1) // BS
    num_blocks = int(nblk.sum()) + 7
    perm = torch.randperm(num_blocks, generator=g)
    tables = torch.zeros(batch, int(nblk.max()), dtype=torch.long)
    off = 0
    for i in range(batch):
        n = int(nblk[i])
        tables[i, :n] = perm[off:off + n]
        off += n
    q = torch.randn(batch, kv_heads * group, d, generator=g).to(dtype)
    torch.cuda.manual_seed(seed)
    kp = torch.randn(num_blocks, BS, kv_heads, d, device="cuda", dtype=dtype)
    vp = torch.randn(num_blocks, BS, kv_heads, d, device="cuda", dtype=dtype)
    return q, kp, vp, tables, ctx


def _check_all_rows(out, q, kp, vp, tables, ctx):
    one = torch.ones(1, dtype=torch.long)
    scale = q.shape[-1] ** -0.5
    out = out.cpu()
    for i in range(q.shape[0]):
        c = int(ctx[i])
        used = tables[i, : -(-c // BS)]
        idx = used.cuda()
        ref = oracle_gather(q[i:i + 1], kp[idx].cpu(), vp[idx].cpu(), torch.arange(len(used))[None],
                            ctx[i:i + 1], one, scale)
        torch.testing.assert_close(out[i:i + 1], ref, atol=2e-2, rtol=2e-2, msg=lambda m: f"row {i}: {m}")


CASES = {
    # name: (batch, kv_heads, group, head_dim, dtype, context lengths from rng)
    "bf16_kv8_g4_d128_ragged": (64, 8, 4, 128, torch.bfloat16, lambda r: r.integers(1, 8193, size=64)),
    "fp16_kv12_g1_d64": (128, 12, 1, 64, torch.float16, lambda r: r.integers(1, 4097, size=128)),
    "bf16_kv8_g8_d128_long": (32, 8, 8, 128, torch.bfloat16, lambda r: r.integers(4000, 16385, size=32)),
    "fp16_kv4_g2_d64_many_short": (512, 4, 2, 64, torch.float16, lambda r: r.integers(1, 2101, size=512)),
    "bf16_kv16_g1_d128_equal": (16, 16, 1, 128, torch.bfloat16, lambda r: np.full(16, 16384)),
    "fp16_kv8_g2_d128": (96, 8, 2, 128, torch.float16, lambda r: r.integers(512, 6001, size=96)),
}


@pytest.mark.parametrize("name", list(CASES))
def test_mfma_decode_matches_oracle_on_every_row(name):
    batch, kv, group, d, dtype, ctx_fn = CASES[name]
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    ctx = np.asarray(ctx_fn(rng), dtype=np.int64)
    if name != "bf16_kv16_g1_d128_equal":
        ctx[:4] = [1, 15, 16, 17]                      # partial, whole and just-over blocks
    # The launch qualifies by its longest context (the K/V bound reaches 512 MiB).
    ctx[-1] = max(int(ctx.max()), -(-(512 << 20) // (batch * kv * d * 4)))
    q, kp, vp, tables, ctx_t = _batch(batch, kv, group, d, ctx, dtype, seed=batch + d)
    ql = torch.ones(batch, dtype=torch.long).cuda()
    out = paged_attention_hip(q.cuda(), kp, vp, tables.cuda(), ctx_t.cuda(), ql, d ** -0.5)
    again = paged_attention_hip(q.cuda(), kp, vp, tables.cuda(), ctx_t.cuda(), ql, d ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(out, again), "a second call on the same workspace differs"
    _check_all_rows(out, q, kp, vp, tables, ctx_t)


def test_mfma_decode_with_fused_append():
    """The new token's K/V row of every sequence goes to its pool slot inside the call
    (the wave that reads the sequence's last block writes it first): the pool equals
    oracle.kvops.kv_append bit for bit and every row matches the oracle over it."""
    from inference_server.core.attention_hip import paged_attention_hip_launch
    from oracle.kvops import kv_append

    batch, kv, group, d, dtype = 64, 8, 4, 128, torch.bfloat16
    rng = np.random.default_rng(5)
    ctx = rng.integers(1, 8193, size=batch)
    ctx[:3] = [1, 16, 17]
    ctx[-1] = 8192
    q, kp, vp, tables, ctx_t = _batch(batch, kv, group, d, ctx, dtype, seed=77)
    g = torch.Generator().manual_seed(78)
    k_new = torch.randn(batch, kv, d, generator=g).to(dtype)
    v_new = torch.randn(batch, kv, d, generator=g).to(dtype)
    last = ctx_t - 1
    slots = tables[torch.arange(batch), last // BS] * BS + last % BS
    k_before = kp.view(torch.int16).cpu().numpy()
    v_before = vp.view(torch.int16).cpu().numpy()
    out = paged_attention_hip_launch(q.cuda(), kp, vp, tables.cuda(), ctx_t.cuda(),
                                     torch.ones(batch, dtype=torch.long).cuda(), d ** -0.5,
                                     append=(k_new.cuda(), v_new.cuda(), slots.cuda()))
    torch.cuda.synchronize()
    assert (kp.view(torch.int16).cpu().numpy() == kv_append(k_before, k_new.view(torch.int16).numpy(),
                                                            slots.numpy())).all()
    assert (vp.view(torch.int16).cpu().numpy() == kv_append(v_before, v_new.view(torch.int16).numpy(),
                                                            slots.numpy())).all()
    _check_all_rows(out, q, kp, vp, tables, ctx_t)


@pytest.mark.parametrize("seed", list(range(16)))
def test_mfma_decode_random_batches(seed):
    """Seeded random batches routed to the MFMA kernel: KV heads 4-24 (both wave counts
    per workgroup and several head groups), GQA 1/2/4/8, head_dim 64/128, fp16/bf16,
    contexts drawn from a mix of tiny (1-40 tokens), medium and long ranges so that runs
    hold many whole sequences as well as cut ones; leading blocks shared between
    sequences (a prefix-cache hit) and table rows padded with live block ids. One
    sequence is lengthened so the K/V bound reaches the 512 MiB the route needs. Every
    row against the oracle; a second call on the same workspace gives the same bytes."""
    rng = np.random.default_rng(4242 + seed)
    kv = int(rng.choice([4, 8, 12, 16, 20, 24]))
    group = int(rng.choice([1, 2, 4, 8] if kv <= 8 else [1, 2]))
    d = int(rng.choice([64, 128]))
    dtype = [torch.float16, torch.bfloat16][rng.integers(2)]
    batch = int(rng.integers(8, 257))
    kinds = rng.integers(0, 3, size=batch)
    ctx = np.where(kinds == 0, rng.integers(1, 41, size=batch),
                   np.where(kinds == 1, rng.integers(41, 1025, size=batch), rng.integers(1025, 6001, size=batch)))
    ctx = ctx.astype(np.int64)
    ctx[-1] = max(int(ctx.max()), -(-(512 << 20) // (batch * kv * d * 4)))
    # Keep the oracle's work bounded: shorten the longest contexts (the last one stays).
    while int(ctx.sum()) * kv * d > 6e8:
        i = int(np.argmax(ctx[:-1]))
        ctx[i] = max(1, ctx[i] // 2)
    nblk = -(-ctx // BS)
    shared = int(rng.integers(0, int(nblk.min()) + 1)) if rng.random() < 0.5 else 0
    num_blocks = shared + int((nblk - shared).sum()) + 5
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed))
    width = int(nblk.max()) + int(rng.integers(0, 3))
    tables = torch.zeros(batch, width, dtype=torch.long)
    off = shared
    for i in range(batch):
        n = int(nblk[i])
        tables[i, :shared] = perm[:shared]
        tables[i, shared:n] = perm[off:off + n - shared]
        off += n - shared
        tables[i, n:] = perm[torch.randint(0, num_blocks, (width - n,))]
    g = torch.Generator().manual_seed(seed + 1)
    q = torch.randn(batch, kv * group, d, generator=g).to(dtype)
    torch.cuda.manual_seed(seed + 2)
    kp = torch.randn(num_blocks, BS, kv, d, device="cuda", dtype=dtype)
    vp = torch.randn(num_blocks, BS, kv, d, device="cuda", dtype=dtype)
    ctx_t = torch.as_tensor(ctx)
    print(f"seed {seed}: batch {batch} kv {kv} g{group} d{d} {dtype} ctx sum {int(ctx.sum())} max {int(ctx.max())} "
          f"shared {shared}", flush=True)
    ql = torch.ones(batch, dtype=torch.long).cuda()
    out = paged_attention_hip(q.cuda(), kp, vp, tables.cuda(), ctx_t.cuda(), ql, d ** -0.5)
    again = paged_attention_hip(q.cuda(), kp, vp, tables.cuda(), ctx_t.cuda(), ql, d ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(out, again), "a second call on the same workspace differs"
    _check_all_rows(out, q, kp, vp, tables, ctx_t)
