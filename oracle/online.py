"""Oracle: the reference kernel's block-order online softmax, restated in numpy.

Test infrastructure only (see oracle/__init__.py). Restates the PyTorch mirror of
the reference's Triton kernel, `paged_attention_reference`
(core/attention_triton.py:309-384): per query token, walk the sequence's block table
one block at a time and fold each [block_size, head_dim] tile into a running
(max, denominator, numerator) in float32. Vectorised over heads; the loop over
tokens and blocks is plain Python, so keep inputs small (unit-test sizes).

It is the second checker of the fp32 kernels: tests/test_hip_attention.py compares
them with it at 2.5e-6 (4x tighter than the 1e-5 gather bar), since both fold keys
block by block into a running fp32 (max, denominator, numerator), where the gather
path materialises dense scores.
"""

from __future__ import annotations

import numpy as np


def paged_attention_online(query, k_pool, v_pool, block_tables, context_lens, query_lens, scale):
    """All array arguments are numpy (any float dtype is widened to float32);
    returns float32 [T, Hq, D]."""
    q_all = np.asarray(query, dtype=np.float32)
    kp = np.asarray(k_pool, dtype=np.float32)
    vp = np.asarray(v_pool, dtype=np.float32)
    tables = np.asarray(block_tables, dtype=np.int64)
    ctx = np.asarray(context_lens, dtype=np.int64)
    ql = np.asarray(query_lens, dtype=np.int64)
    n_tok, n_heads, head_dim = q_all.shape
    bs, n_kv = kp.shape[1], kp.shape[2]
    group = n_heads // n_kv
    kv_of_head = np.arange(n_heads) // group                  # attention_triton.py:181
    out = np.empty((n_tok, n_heads, head_dim), dtype=np.float32)

    cu = np.concatenate([[0], np.cumsum(ql)])
    for seq in range(len(ql)):
        for t in range(int(ql[seq])):
            tok = int(cu[seq]) + t
            n_keys = int(ctx[seq] - ql[seq] + t) + 1           # :185 causal bound
            q = q_all[tok] * np.float32(scale)                  # [H, D], pre-scaled (:191-194)
            m = np.full(n_heads, -np.inf, dtype=np.float32)
            l = np.zeros(n_heads, dtype=np.float32)
            acc = np.zeros((n_heads, head_dim), dtype=np.float32)
            for blk in range(-(-n_keys // bs)):                 # :203
                phys = int(tables[seq, blk])
                live = (blk * bs + np.arange(bs)) < n_keys       # :207-208
                k = kp[phys][:, kv_of_head, :]                   # [bs, H, D]
                v = vp[phys][:, kv_of_head, :]
                s = np.einsum("bhd,hd->hb", k, q).astype(np.float32)
                s = np.where(live[None, :], s, -np.inf)          # :216
                m_new = np.maximum(m, s.max(axis=1))             # :219
                alpha = np.exp(m - m_new)                        # :220
                p = np.exp(s - m_new[:, None])                   # :221
                l = alpha * l + p.sum(axis=1)                    # :226
                v = np.where(live[:, None, None], v, 0.0)
                acc = alpha[:, None] * acc + np.einsum("hb,bhd->hd", p, v)   # :227
                m = m_new
            out[tok] = acc / l[:, None]                          # :230
    return out
