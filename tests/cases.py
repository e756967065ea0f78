"""Seeded input builders shared by the oracle, contract and HIP parity tests.

`build(lengths, ...)` follows the reference tests' builder
(tests/test_paged_attention_triton.py:46-70): random K/V pools, blocks drawn without
replacement from a seeded permutation (so a contiguity assumption is caught), one
(context_len, query_len) pair per sequence, tables 0-padded to the widest row.

`dense_causal_f64` is the textbook oracle of tests/test_paged_attention.py:30-37 —
for each sequence, copy its context out of the pool slot by slot and run plain causal
attention — recomputed in float64 numpy with an explicit per-query softmax, so it
shares no code or op order with either gather implementation.
"""

from __future__ import annotations

import numpy as np
import torch

# The reference's batch shapes (tests/test_paged_attention_triton.py:74-84).
CASES = {
    "prefill_on_boundary": [(4, 4), (8, 8), (16, 16)],
    "prefill_spilling": [(5, 5), (9, 9), (17, 17)],
    "prefill_partial": [(1, 1), (3, 3), (15, 15)],
    "prefill_ragged": [(7, 7), (4, 4), (13, 13), (1, 1), (16, 16)],
    "decode_singles": [(1, 1), (4, 1), (5, 1), (8, 1), (9, 1), (16, 1), (17, 1)],
    "decode_ragged": [(9, 1), (4, 1), (17, 1), (1, 1), (12, 1), (5, 1)],
    "mixed": [(6, 1), (10, 10), (4, 1), (9, 5), (16, 16), (13, 1)],
    "partial_query": [(11, 3), (8, 4), (20, 7)],
    "padding_hits_block0": [(3, 3), (19, 1), (4, 1)],
}

NUM_BLOCKS = 64


def build(lengths, *, bs=4, d=8, heads=3, kv_heads=3, seed=0, dtype=torch.float32, device="cpu",
          num_blocks=NUM_BLOCKS):
    g = torch.Generator().manual_seed(seed)
    k_pool = torch.randn(num_blocks, bs, kv_heads, d, generator=g)
    v_pool = torch.randn(num_blocks, bs, kv_heads, d, generator=g)
    perm = torch.randperm(num_blocks, generator=g).tolist()
    queries, tables = [], []
    for ctx, q_len in lengths:
        nblocks = -(-ctx // bs)
        blocks, perm = perm[:nblocks], perm[nblocks:]
        queries.append(torch.randn(q_len, heads, d, generator=g))
        tables.append(blocks)
    width = max(len(t) for t in tables)
    block_tables = torch.tensor([t + [0] * (width - len(t)) for t in tables], dtype=torch.long)
    to = dict(dtype=dtype, device=device)
    return (
        torch.cat(queries).to(**to),
        k_pool.to(**to),
        v_pool.to(**to),
        block_tables.to(device),
        torch.tensor([c for c, _ in lengths], dtype=torch.long, device=device),
        torch.tensor([q for _, q in lengths], dtype=torch.long, device=device),
    )


def dense_causal_f64(query, k_pool, v_pool, block_tables, context_lens, query_lens, scale) -> np.ndarray:
    q_all = query.detach().cpu().double().numpy()
    kp = k_pool.detach().cpu().double().numpy()
    vp = v_pool.detach().cpu().double().numpy()
    tables = block_tables.cpu().numpy()
    ctx = context_lens.cpu().numpy()
    ql = query_lens.cpu().numpy()
    n_tok, n_heads, d = q_all.shape
    bs, n_kv = kp.shape[1], kp.shape[2]
    group = n_heads // n_kv
    out = np.zeros((n_tok, n_heads, d))
    tok = 0
    for i in range(len(ctx)):
        c = int(ctx[i])
        # Slot by slot: logical position p lives in block tables[i, p // bs], row p % bs.
        k = np.stack([kp[tables[i, p // bs], p % bs] for p in range(c)]) if c else np.zeros((0, n_kv, d))
        v = np.stack([vp[tables[i, p // bs], p % bs] for p in range(c)]) if c else np.zeros((0, n_kv, d))
        for t in range(int(ql[i])):
            pos = c - int(ql[i]) + t
            for h in range(n_heads):
                kh = k[: pos + 1, h // group]
                s = kh @ q_all[tok, h] * scale
                w = np.exp(s - s.max())
                out[tok, h] = (w / w.sum()) @ v[: pos + 1, h // group]
            tok += 1
    return out
