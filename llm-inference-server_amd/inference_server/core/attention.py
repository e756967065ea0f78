"""Paged attention: the contract, the dispatcher, and the PyTorch gather backend.

Contract (the reference's, inference_server/core/attention.py:19-58)::

    paged_attention(query [T, Hq, D], k_pool, v_pool [NB, bs, Hkv, D],
                    block_tables int64 [B, W] (0-padded), context_lens int64 [B]
                    (tokens cached AFTER this pass), query_lens int64 [B] (sum = T),
                    scale) -> [T, Hq, D] in query.dtype

Sequence i's query tokens are its last query_lens[i] positions: token t sits at
logical position context_lens[i] - query_lens[i] + t and attends to keys 0..that.
Query head h reads KV head h // (Hq // Hkv).

Backends, chosen by CONFIG.attention on every call (attention.py:84-88):

  gather  PyTorch ops, any device. The reference's shipping path, kept op-for-op so a
          CPU run and a GPU "gather" run reproduce the reference's numerics.
  triton  Named for interface parity only; this build ships no Triton and raises.
  hip     libpagedkv's CDNA4 kernels (core/attention_hip.py). Raises
          NotImplementedError if the library or a ROCm device is missing; never
          falls back to gather.
"""

from __future__ import annotations

import torch

from inference_server.config import CONFIG


def paged_attention(
    query: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    query_lens: torch.Tensor,
    scale: float,
) -> torch.Tensor:
    """Dispatch on CONFIG.attention (reference: core/attention.py:73-88)."""
    backend = CONFIG.attention
    if backend == "gather":
        return paged_attention_gather(query, k_pool, v_pool, block_tables, context_lens, query_lens, scale)
    if backend == "hip":
        return paged_attention_hip(query, k_pool, v_pool, block_tables, context_lens, query_lens, scale)
    if backend == "triton":
        return paged_attention_triton(query, k_pool, v_pool, block_tables, context_lens, query_lens, scale)
    raise ValueError(f"unknown ATTENTION={backend!r}; expected 'gather', 'triton' or 'hip'")


# ----------------------------------------------------------------------- gather
def paged_attention_gather(
    query: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    query_lens: torch.Tensor,
    scale: float,
) -> torch.Tensor:
    """Gather each sequence's blocks, then dense masked attention (reference:
    core/attention.py:92-127). All-decode batches run as one batched op; anything
    else loops over sequences so the score matrix stays one sequence wide."""
    _check(query, k_pool, block_tables, context_lens, query_lens)
    if query.shape[0] == 0:
        return query.new_empty((0, query.shape[1], query.shape[2]))
    if bool((query_lens == 1).all()):
        return _gather_decode(query, k_pool, v_pool, block_tables, context_lens, scale)
    return _gather_ragged(query, k_pool, v_pool, block_tables, context_lens, query_lens, scale)


def _gather_decode(query, k_pool, v_pool, block_tables, context_lens, scale):
    """One token per sequence (reference: core/attention.py:130-153)."""
    n_heads = query.shape[1]
    bs = k_pool.shape[1]
    longest = int(context_lens.max())
    tables = block_tables[:, : -(-longest // bs)]
    keys = _repeat_kv(k_pool[tables].flatten(1, 2)[:, :longest], n_heads).transpose(1, 2)
    vals = _repeat_kv(v_pool[tables].flatten(1, 2)[:, :longest], n_heads).transpose(1, 2)
    scores = torch.matmul(query.unsqueeze(2), keys.transpose(-1, -2)) * scale      # [B, H, 1, ctx]
    in_ctx = torch.arange(longest, device=query.device)[None, :] < context_lens[:, None]
    scores = scores.masked_fill(~in_ctx[:, None, None, :], float("-inf"))
    probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(vals.dtype)
    return torch.matmul(probs, vals).squeeze(2)


def _gather_ragged(query, k_pool, v_pool, block_tables, context_lens, query_lens, scale):
    """Per-sequence causal attention (reference: core/attention.py:156-187)."""
    n_heads = query.shape[1]
    bs = k_pool.shape[1]
    out = torch.empty_like(query)
    start = 0
    for i in range(block_tables.shape[0]):
        n_q = int(query_lens[i])
        ctx = int(context_lens[i])
        if n_q == 0:
            continue
        blocks = block_tables[i, : -(-ctx // bs)]
        keys = _repeat_kv(k_pool[blocks].flatten(0, 1)[:ctx], n_heads).transpose(0, 1)   # [H, ctx, D]
        vals = _repeat_kv(v_pool[blocks].flatten(0, 1)[:ctx], n_heads).transpose(0, 1)
        q = query[start : start + n_q].transpose(0, 1)                                     # [H, n_q, D]
        scores = torch.matmul(q, keys.transpose(-1, -2)) * scale
        q_pos = torch.arange(ctx - n_q, ctx, device=query.device)
        k_pos = torch.arange(ctx, device=query.device)
        scores = scores.masked_fill(~(k_pos[None, :] <= q_pos[:, None])[None], float("-inf"))
        probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(vals.dtype)
        out[start : start + n_q] = torch.matmul(probs, vals).transpose(0, 1)
        start += n_q
    return out


def _repeat_kv(kv: torch.Tensor, n_heads: int) -> torch.Tensor:
    """GQA: repeat each KV head for its query-head group (reference:
    core/attention.py:190-199)."""
    n_kv = kv.shape[-2]
    if n_kv == n_heads:
        return kv
    if n_heads % n_kv:
        raise ValueError(f"{n_heads} query heads not divisible by {n_kv} kv heads")
    return kv.repeat_interleave(n_heads // n_kv, dim=-2)


def _check(query, k_pool, block_tables, context_lens, query_lens) -> None:
    """The reference's contract checks and messages (core/attention.py:202-219).
    Reads lengths with host syncs; the hip backend runs the same checks on host
    copies instead (core/attention_hip.py)."""
    check_contract(
        query.dim(), tuple(query.shape), k_pool.dim(), tuple(k_pool.shape), block_tables.shape,
        context_lens.shape, query_lens.shape,
        lambda: (int(query_lens.sum()), bool((query_lens > context_lens).any()),
                 bool(((-(-context_lens // k_pool.shape[1])) > block_tables.shape[1]).any())),
    )


def check_contract(q_dim, q_shape, pool_dim, pool_shape, tables_shape, ctx_shape, qlens_shape, values) -> None:
    """Shape checks first, then `values()` -> (sum of query_lens, any query_len >
    context_len, any sequence needing more blocks than the table width)."""
    if q_dim != 3:
        raise ValueError(f"query must be [num_tokens, heads, dim], got {q_shape}")
    if pool_dim != 4:
        raise ValueError(f"k_pool must be [blocks, block_size, kv_heads, dim], got {pool_shape}")
    batch = tables_shape[0]
    if tuple(ctx_shape) != (batch,) or tuple(qlens_shape) != (batch,):
        raise ValueError("context_lens and query_lens must be [batch] to match block_tables")
    total, too_long, too_wide = values()
    if total != q_shape[0]:
        raise ValueError(f"query_lens sum to {total} but query has {q_shape[0]} tokens")
    if too_long:
        raise ValueError("query_len exceeds context_len — the query tokens must be counted in the context")
    if too_wide:
        raise ValueError("a sequence's context needs more blocks than its block_tables row holds")


# ----------------------------------------------------------------------- triton / hip
def paged_attention_triton(
    query: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    query_lens: torch.Tensor,
    scale: float,
) -> torch.Tensor:
    """The reference's Triton seam (core/attention.py:223-249). This build ships no
    Triton: selecting it raises, naming the backend that replaces it."""
    raise NotImplementedError(
        "ATTENTION=triton: this MI355X build ships no Triton kernel; use ATTENTION=hip "
        "(libpagedkv CDNA4 kernels) or ATTENTION=gather"
    )


def paged_attention_hip(
    query: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    query_lens: torch.Tensor,
    scale: float,
) -> torch.Tensor:
    """libpagedkv's decode / prefill kernels (see core/attention_hip.py)."""
    from inference_server.core.attention_hip import paged_attention_hip_launch

    return paged_attention_hip_launch(query, k_pool, v_pool, block_tables, context_lens, query_lens, scale)
