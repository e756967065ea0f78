"""Oracle: the reference's PyTorch gather attention path, restated on the CPU.

Test infrastructure only (see oracle/__init__.py). The op sequence is the reference's
because its numerics are the target: gather blocks -> repeat KV heads -> matmul in the
pool dtype -> * scale -> masked_fill(-inf) -> softmax(dtype=float32) -> cast to the V
dtype -> matmul. In half precision the cast of the probabilities before P·V is part
of what the HIP kernels are compared against (within 2e-2).
"""

from __future__ import annotations

import torch


def token_map(context_lens: torch.Tensor, query_lens: torch.Tensor):
    """(seq_idx, q_pos, cu) per packed token — reference core/attention_triton.py:129-150.

    cu[i] = sum(query_lens[:i]); token tok of the packed row belongs to the sequence
    s with cu[s] <= tok < cu[s+1] and sits at position ctx_s - q_s + (tok - cu[s]).
    """
    ctx = context_lens.long().cpu()
    ql = query_lens.long().cpu()
    cu = torch.zeros(ql.numel() + 1, dtype=torch.long)
    cu[1:] = torch.cumsum(ql, 0)
    seq_idx = torch.repeat_interleave(torch.arange(ql.numel()), ql)
    tok = torch.arange(int(cu[-1]))
    q_pos = ctx[seq_idx] - ql[seq_idx] + (tok - cu[seq_idx])
    return seq_idx, q_pos, cu


def _kv_heads_for(kv: torch.Tensor, n_heads: int) -> torch.Tensor:
    """GQA expansion — reference core/attention.py:190-199 (head h reads KV head
    h // group; repeat_interleave produces exactly that order)."""
    group = n_heads // kv.shape[-2]
    return kv if group == 1 else kv.repeat_interleave(group, dim=-2)


def _sequence_kv(pool: torch.Tensor, table_row: torch.Tensor, ctx: int) -> torch.Tensor:
    """[ctx, Hkv, D]: the sequence's first ctx slots, block by block in logical order
    (reference core/attention.py:166-171)."""
    bs = pool.shape[1]
    n_blocks = -(-ctx // bs)
    return pool[table_row[:n_blocks]].reshape(n_blocks * bs, *pool.shape[2:])[:ctx]


def paged_attention_gather(query, k_pool, v_pool, block_tables, context_lens, query_lens, scale):
    """Reference core/attention.py:92-127 (dispatch), :130-153 (decode), :156-187 (ragged).
    Inputs may be on any device; everything is computed on the CPU."""
    q_all = query.detach().cpu()
    kp, vp = k_pool.detach().cpu(), v_pool.detach().cpu()
    tables = block_tables.detach().cpu().long()
    ctx = context_lens.detach().cpu().long()
    ql = query_lens.detach().cpu().long()
    n_tok, n_heads, head_dim = q_all.shape
    if n_tok == 0:
        return q_all.new_empty((0, n_heads, head_dim))

    if bool((ql == 1).all()):
        # Batched decode: pad every context to the longest, mask the tail (:130-153).
        longest = int(ctx.max())
        bs = kp.shape[1]
        width = -(-longest // bs)
        k = kp[tables[:, :width]].flatten(1, 2)[:, :longest]
        v = vp[tables[:, :width]].flatten(1, 2)[:, :longest]
        k = _kv_heads_for(k, n_heads).transpose(1, 2)             # [B, H, ctx, D]
        v = _kv_heads_for(v, n_heads).transpose(1, 2)
        scores = torch.matmul(q_all.unsqueeze(2), k.transpose(-1, -2)) * scale
        valid = torch.arange(longest)[None, :] < ctx[:, None]
        scores = scores.masked_fill(~valid[:, None, None, :], float("-inf"))
        probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(v.dtype)
        return torch.matmul(probs, v).squeeze(2)

    out = torch.empty_like(q_all)
    start = 0
    for i in range(tables.shape[0]):                              # (:156-187)
        n_q, c = int(ql[i]), int(ctx[i])
        if n_q == 0:
            continue
        k = _kv_heads_for(_sequence_kv(kp, tables[i], c), n_heads).transpose(0, 1)
        v = _kv_heads_for(_sequence_kv(vp, tables[i], c), n_heads).transpose(0, 1)
        q = q_all[start:start + n_q].transpose(0, 1)
        scores = torch.matmul(q, k.transpose(-1, -2)) * scale
        causal = torch.arange(c)[None, :] <= torch.arange(c - n_q, c)[:, None]
        scores = scores.masked_fill(~causal[None], float("-inf"))
        probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(v.dtype)
        out[start:start + n_q] = torch.matmul(probs, v).transpose(0, 1)
        start += n_q
    return out
