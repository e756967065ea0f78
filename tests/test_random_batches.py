"""Seeded random batches through ATTENTION=hip against the oracle gather path.

The fixed cases (the reference's CASES and the BASELINE shapes) pin each kernel on the
shapes it was tuned for; these draw the combinations in between. Each seed builds one
batch with an independent choice of:

* pool dtype (fp32 / fp16 / bf16), head_dim (64 / 128 on the tuned kernels, 32 / 80 on
  the generic one), block size (16, or 8 / 32 on the generic kernel), KV heads and GQA
  group (1, 2, 3, 4, 8: group 3 has no tuned instance);
* batch kind: decode (every query length 1), prefill (query length = context),
  chunked prefill (query length <= context) or a mix of all three;
* contexts of 1 to ~2,000 tokens;
* block tables whose sequences share their leading blocks (a prefix-cache hit
  maps several sequences onto the same physical blocks: the kernels only read them),
  padded past each sequence's last block with live block ids, so a kernel that reads
  past the context reads real, finite data and is caught by the comparison rather
  than by luck;
* a query tensor that is a head slice of a wider one (non-unit head stride).

The second test draws the same batches with the step's new K/V rows appended inside the
attention call (`append=`: fused into the decode / prefill kernel where one covers the
shape, a separate append launch first otherwise). Shared blocks then end before every
sequence's first new position, as copy-on-write guarantees in the engine. The pool
after the call must equal oracle.kvops.kv_append bit for bit, and the output must match
oracle.gather over that pool.

Every output row is compared with oracle.gather (the reference gather path,
core/attention.py:92-199) at the north-star tolerances: 1e-5 in fp32, 2e-2 in 16-bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from inference_server.core.attention import paged_attention_hip
from oracle.gather import paged_attention_gather as oracle_gather

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}
SEEDS = list(range(64))


def _draw(seed):
    rng = np.random.default_rng(1000 + seed)
    dtype = [torch.float32, torch.float16, torch.bfloat16][rng.integers(3)]
    d = int(rng.choice([64, 128, 64, 128, 32, 80]))
    bs = int(rng.choice([16, 16, 16, 8, 32]))
    group = int(rng.choice([1, 2, 3, 4, 8]))
    kv_heads = int(rng.integers(1, 5 if group < 8 else 3))
    batch = int(rng.integers(1, 13))
    kind = ["decode", "prefill", "chunked", "mixed"][rng.integers(4)]
    long_ctx = rng.random() < 0.3
    ctx = rng.integers(1, 2049 if long_ctx else 400, size=batch)
    if kind == "decode":
        ql = np.ones(batch, dtype=np.int64)
    elif kind == "prefill":
        ctx = np.minimum(ctx, 300)
        ql = ctx.copy()
    elif kind == "chunked":
        ql = np.array([rng.integers(1, min(int(c), 160) + 1) for c in ctx])
    else:
        ql = np.array([[1, int(c) if c <= 200 else 1, rng.integers(1, min(int(c), 96) + 1)][rng.integers(3)]
                       for c in ctx])
    return rng, dict(dtype=dtype, d=d, bs=bs, group=group, kv_heads=kv_heads, kind=kind,
                     ctx=ctx.astype(np.int64), ql=ql.astype(np.int64))


def _tables(rng, ctx, bs, max_shared=None):
    """Tables with shared leading blocks (at most max_shared) and live-id padding;
    returns (tables, num_blocks)."""
    nblk = [-(-int(c) // bs) for c in ctx]
    cap = min(nblk) if max_shared is None else min(min(nblk), max_shared)
    shared = int(rng.integers(0, cap + 1)) if rng.random() < 0.4 else 0
    own = sum(n - shared for n in nblk)
    num_blocks = shared + own + 3
    perm = rng.permutation(num_blocks)
    prefix = perm[:shared].tolist()
    rest = perm[shared:].tolist()
    width = max(nblk) + int(rng.integers(0, 4))
    rows = []
    for n in nblk:
        row = prefix + rest[: n - shared]
        rest = rest[n - shared:]
        # Padding past the sequence's blocks: live ids, never read by a correct kernel.
        row += rng.integers(0, num_blocks, size=width - len(row)).tolist()
        rows.append(row)
    return torch.tensor(rows, dtype=torch.long), num_blocks


@pytest.mark.parametrize("seed", SEEDS)
def test_random_batch_matches_gather(seed):
    rng, c = _draw(seed)
    dtype, d, bs, group, kv = c["dtype"], c["d"], c["bs"], c["group"], c["kv_heads"]
    heads = kv * group
    tables, num_blocks = _tables(rng, c["ctx"], bs)
    g = torch.Generator().manual_seed(seed)
    kp = torch.randn(num_blocks, bs, kv, d, generator=g).to(dtype)
    vp = torch.randn(num_blocks, bs, kv, d, generator=g).to(dtype)
    n_tok = int(c["ql"].sum())
    strided = rng.random() < 0.3
    wide = torch.randn(n_tok, heads + (3 if strided else 0), d, generator=g).to(dtype)
    q = wide[:, :heads] if strided else wide
    ctx = torch.as_tensor(c["ctx"])
    ql = torch.as_tensor(c["ql"])
    scale = d ** -0.5
    print(f"seed {seed}: {c['kind']} {dtype} d{d} bs{bs} kv{kv} g{group} batch {len(ctx)} "
          f"ctx max {int(ctx.max())} tokens {n_tok} strided {strided}", flush=True)

    qd = q.cuda() if not strided else wide.cuda()[:, :heads]
    out = paged_attention_hip(qd, kp.cuda(), vp.cuda(), tables.cuda(), ctx.cuda(), ql.cuda(), scale)
    torch.cuda.synchronize()
    ref = oracle_gather(q, kp, vp, tables, ctx, ql, scale)
    assert out.shape == ref.shape and out.dtype == dtype
    tol = TOL[dtype]
    torch.testing.assert_close(out.cpu(), ref, atol=tol, rtol=tol)


@pytest.mark.parametrize("seed", SEEDS[:40])
def test_random_batch_with_fused_append(seed):
    from inference_server.core.attention_hip import paged_attention_hip_launch
    from oracle.kvops import kv_append

    rng, c = _draw(seed)
    dtype, d, bs, group, kv = c["dtype"], c["d"], c["bs"], c["group"], c["kv_heads"]
    heads = kv * group
    first_new = c["ctx"] - c["ql"]
    tables, num_blocks = _tables(rng, c["ctx"], bs, max_shared=int(first_new.min()) // bs)
    g = torch.Generator().manual_seed(seed)
    kp = torch.randn(num_blocks, bs, kv, d, generator=g).to(dtype)
    vp = torch.randn(num_blocks, bs, kv, d, generator=g).to(dtype)
    n_tok = int(c["ql"].sum())
    q = torch.randn(n_tok, heads, d, generator=g).to(dtype)
    k_new = torch.randn(n_tok, kv, d, generator=g).to(dtype)
    v_new = torch.randn(n_tok, kv, d, generator=g).to(dtype)
    # The slot of every new position ctx - q_len + i of every sequence.
    slots = torch.cat([tables[i, torch.arange(int(f), int(f + n)) // bs] * bs + torch.arange(int(f), int(f + n)) % bs
                       for i, (f, n) in enumerate(zip(first_new, c["ql"]))])
    assert len(set(slots.tolist())) == n_tok
    ctx = torch.as_tensor(c["ctx"])
    ql = torch.as_tensor(c["ql"])
    scale = d ** -0.5
    print(f"seed {seed}: {c['kind']} {dtype} d{d} bs{bs} kv{kv} g{group} batch {len(ctx)} "
          f"ctx max {int(ctx.max())} tokens {n_tok} (fused append)", flush=True)

    kd, vd = kp.cuda(), vp.cuda()
    out = paged_attention_hip_launch(q.cuda(), kd, vd, tables.cuda(), ctx.cuda(), ql.cuda(), scale,
                                     append=(k_new.cuda(), v_new.cuda(), slots.cuda()))
    torch.cuda.synchronize()
    raw = {2: torch.int16, 4: torch.int32}[kp.element_size()]
    k_want = kv_append(kp.view(raw).numpy(), k_new.view(raw).numpy(), slots.numpy())
    v_want = kv_append(vp.view(raw).numpy(), v_new.view(raw).numpy(), slots.numpy())
    assert (kd.cpu().view(raw).numpy() == k_want).all() and (vd.cpu().view(raw).numpy() == v_want).all()
    ref = oracle_gather(q, kd.cpu(), vd.cpu(), tables, ctx, ql, scale)
    tol = TOL[dtype]
    torch.testing.assert_close(out.cpu(), ref, atol=tol, rtol=tol)
