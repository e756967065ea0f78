"""ATTENTION=hip: paged attention on libpagedkv's CDNA4 kernels.

Same signature, contract checks and exception texts as the gather path
(core/attention.py). Differences are in where the checks read the lengths and in
what runs afterwards:

* Lengths. The reference's `_check` reads context_lens/query_lens back from the
  device with three to four host syncs per call (reference core/attention.py:212-218).
  Here a caller that already holds the lengths on the host (the paged executor
  builds them from Python lists) attaches them with `attach_host`; the checks then
  run with no device round trip. Without an attached copy one combined D2H copy is
  made, and CPU tensors are used as they are.
* Kernels. An all-decode batch (every query_len == 1) goes to
  pkv_paged_attention_decode (split-KV, GQA-shared K/V reads); any other batch goes
  to pkv_paged_attention_prefill. Both accept the strided query view the executor
  hands over (`query[0].transpose(0, 1)`, reference core/paged_executor.py:146)
  without a copy.
* No fallback. Without the library or a ROCm device this raises
  NotImplementedError, like the reference's Triton launcher
  (core/attention_triton.py:254-264).
"""

from __future__ import annotations

import threading

import torch

from inference_server import native
from inference_server.core.attention import check_contract

_HOST_ATTR = "_pkv_host"


def attach_host(device_tensor: torch.Tensor, host_tensor: torch.Tensor) -> torch.Tensor:
    """Record a host (CPU) copy of `device_tensor`'s values for host-side checks.
    The caller guarantees the two hold the same values. Returns device_tensor."""
    setattr(device_tensor, _HOST_ATTR, host_tensor)
    return device_tensor


_QSL_ATTR = "_pkv_qsl"


def attach_query_start(query_lens: torch.Tensor, query_start: torch.Tensor) -> torch.Tensor:
    """Record the device query_start_loc [B+1] (0, then the running sum of query_lens)
    that a prefill launch should use instead of building one from the host lengths
    (a caller that keeps its metadata in persistent device buffers, such as a captured
    graph, supplies it). The caller guarantees the values match. Returns query_lens."""
    setattr(query_lens, _QSL_ATTR, query_start)
    return query_lens


def host_copy(t: torch.Tensor) -> torch.Tensor | None:
    if t.device.type == "cpu":
        return t
    return getattr(t, _HOST_ATTR, None)


def _host_lengths(context_lens: torch.Tensor, query_lens: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    hc, hq = host_copy(context_lens), host_copy(query_lens)
    if hc is None or hq is None:
        both = torch.stack([context_lens.reshape(-1).long(), query_lens.reshape(-1).long()]).cpu()
        hc, hq = both[0], both[1]
    return hc.long(), hq.long()


class _Workspaces:
    """One split-KV decode workspace per (device, stream), grown on demand and reused
    across calls. It is zero-filled when allocated: the merge counters at its front
    must read zero when a call starts, and every completed call leaves them zero
    again (the partials behind them need no initialisation). Calls on one stream are
    ordered; a different stream gets its own buffer. After a call that did not
    complete (a launch error, a reset device), `reset()` drops the buffers so the
    next call gets a zero-filled one."""

    def __init__(self) -> None:
        self._lock = threading.Lock()
        self._bufs: dict[tuple[int, int], torch.Tensor] = {}

    def partials(self, device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        key = (idx, stream)
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                # Zero-filled once: the merge counters at its front must start at zero (every
                # call leaves them zero again); the partials need no initialisation.
                buf = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
                self._bufs[key] = buf
            return buf

    def reset(self) -> None:
        """Forget every buffer (the next call on each stream allocates a zeroed one)."""
        with self._lock:
            self._bufs.clear()


_WORKSPACES = _Workspaces()

_META_ATTR = "_pkv_step_meta"


def _batch_facts(context_lens: torch.Tensor, query_lens: torch.Tensor, block_size: int, width: int) -> dict:
    """Host-side facts about one batch's lengths: the contract checks' inputs, the
    decode/prefill choice, the maxima that size the grids. The paged executor hands
    the same length tensors, with host copies attached, to every layer of a step, so
    for attached tensors the facts are computed once and kept on context_lens, keyed
    by the identity of both host copies (re-attaching new values invalidates them).
    Tensors without attached copies are read afresh on every call."""
    hc_att, hq_att = host_copy(context_lens), host_copy(query_lens)
    cacheable = context_lens.device.type != "cpu" and hc_att is not None and hq_att is not None
    key = (id(hc_att), id(hq_att), block_size, width)
    if cacheable:
        hit = getattr(context_lens, _META_ATTR, None)
        if hit is not None and hit[0] == key:
            return hit[1]
    hctx, hql = _host_lengths(context_lens, query_lens)
    n = int(hctx.numel())
    facts = {
        "hctx": hctx,
        "hql": hql,
        "total": int(hql.sum()),
        "q_gt_c": bool((hql > hctx).any()),
        "too_few_blocks": bool(((-(-hctx // block_size)) > width).any()),
        "all_decode": bool((hql == 1).all()),
        "max_ctx": int(hctx.max()) if n else 0,
        "max_q": int(hql.max()) if n else 0,
        "qsl": None,  # device query_start_loc, built on first prefill use
    }
    if cacheable:
        setattr(context_lens, _META_ATTR, (key, facts))
    return facts


def paged_attention_hip_launch(
    query: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    query_lens: torch.Tensor,
    scale: float,
    append: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
) -> torch.Tensor:
    """The hip backend of `paged_attention`. With `append` = (k_new, v_new, slots) — the
    batch's new rows [T, Hkv, D] (one per query token) and their flat slots, already
    range-checked — the rows are written into the pool inside the attention call: on a
    decode batch `pkv_paged_attention_decode_append` (the decode kernel stores each row
    from the wave that reads it), on any other batch `pkv_paged_attention_prefill_append`
    (the MFMA kernel stages new positions from the rows themselves and each workgroup
    writes its own tokens' rows), so the step has no separate append launch."""
    native.require_gpu(query, "paged_attention")
    bs = k_pool.shape[1] if k_pool.dim() == 4 else 1
    width = block_tables.shape[1] if block_tables.dim() == 2 else 0
    facts: dict = {}

    def values():
        facts.update(_batch_facts(context_lens, query_lens, bs, width))
        return facts["total"], facts["q_gt_c"], facts["too_few_blocks"]

    check_contract(
        query.dim(), tuple(query.shape), k_pool.dim(), tuple(k_pool.shape), block_tables.shape,
        context_lens.shape, query_lens.shape, values,
    )
    if not facts:
        facts.update(_batch_facts(context_lens, query_lens, bs, width))
    hql = facts["hql"]
    if k_pool.shape != v_pool.shape:
        raise ValueError(f"k_pool {tuple(k_pool.shape)} and v_pool {tuple(v_pool.shape)} differ")
    dev = query.device
    for name, t in (("k_pool", k_pool), ("v_pool", v_pool)):
        if t.device != dev:
            raise ValueError(f"{name} is on {t.device}, query is on {dev}")
        if t.dtype != query.dtype:
            raise ValueError(f"{name} dtype {t.dtype} differs from query dtype {query.dtype}")
    n_tok, n_heads, head_dim = query.shape
    n_blocks, block_size, n_kv, pool_dim = k_pool.shape
    if pool_dim != head_dim:
        raise ValueError(f"query head_dim {head_dim} != pool head_dim {pool_dim}")
    if n_heads % n_kv:
        raise ValueError(f"{n_heads} query heads not divisible by {n_kv} kv heads")
    dt = native.dtype_code(query.dtype)

    out = torch.empty((n_tok, n_heads, head_dim), dtype=query.dtype, device=dev)
    n_seqs = block_tables.shape[0]
    if n_tok == 0 or n_seqs == 0:
        return out

    if query.stride(2) != 1:
        query = query.contiguous()
    if k_pool.stride(3) != 1 or v_pool.stride() != k_pool.stride():
        if append is not None:
            # A fused append writes the new rows into the pool in place; a contiguous
            # copy of the pool would take the rows and be thrown away.
            raise ValueError("a fused append needs k_pool and v_pool with unit head_dim stride and equal strides; "
                             f"got {tuple(k_pool.stride())} and {tuple(v_pool.stride())}")
        k_pool, v_pool = k_pool.contiguous(), v_pool.contiguous()
    tables = block_tables.to(device=dev, dtype=torch.long)
    if tables.stride(1) != 1:
        tables = tables.contiguous()
    ctx_dev = context_lens.to(device=dev, dtype=torch.long).contiguous()

    L = native.lib()
    stream = native.stream_handle(dev)
    common_pool = (k_pool.data_ptr(), v_pool.data_ptr(), k_pool.stride(0), k_pool.stride(1), k_pool.stride(2),
                   n_blocks, block_size, n_kv, head_dim,
                   tables.data_ptr(), tables.stride(0), tables.shape[1])
    if append is not None:
        k_new, v_new, slots = append
        if k_new.shape != (n_tok, n_kv, head_dim) or v_new.shape != k_new.shape:
            raise ValueError(f"a fused append needs one new row [{n_kv}, {head_dim}] per query token; "
                             f"got {tuple(k_new.shape)} and {tuple(v_new.shape)} for {n_tok} tokens")
        if k_new.stride(2) != 1 or v_new.stride() != k_new.stride():
            k_new, v_new = k_new.contiguous(), v_new.contiguous()
        slots = slots.to(device=dev, dtype=torch.long)
    if facts["all_decode"] and append is not None:
        max_ctx = facts["max_ctx"]
        ws_bytes = L.pkv_paged_attention_decode_workspace_bytes(n_seqs, n_heads, n_kv, head_dim, max_ctx)
        ws = _WORKSPACES.partials(dev, stream, ws_bytes)
        rc = L.pkv_paged_attention_decode_append(
            out.data_ptr(), out.stride(0), out.stride(1),
            query.data_ptr(), query.stride(0), query.stride(1),
            *common_pool[:9],
            k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), k_new.stride(1), slots.data_ptr(),
            *common_pool[9:],
            ctx_dev.data_ptr(),
            n_seqs, n_heads, max_ctx,
            float(scale), dt,
            ws.data_ptr(), ws.numel(),
            stream,
        )
        native.check(rc, "pkv_paged_attention_decode_append")
        return out
    if facts["all_decode"]:
        max_ctx = facts["max_ctx"]
        ws_bytes = L.pkv_paged_attention_decode_workspace_bytes(n_seqs, n_heads, n_kv, head_dim, max_ctx)
        ws = _WORKSPACES.partials(dev, stream, ws_bytes)
        rc = L.pkv_paged_attention_decode(
            out.data_ptr(), out.stride(0), out.stride(1),
            query.data_ptr(), query.stride(0), query.stride(1),
            *common_pool,
            ctx_dev.data_ptr(),
            n_seqs, n_heads, max_ctx,
            float(scale), dt,
            ws.data_ptr(), ws.numel(),
            stream,
        )
        native.check(rc, "pkv_paged_attention_decode")
        return out

    qsl = getattr(query_lens, _QSL_ATTR, None)
    if qsl is None:
        qsl = facts["qsl"]
        if qsl is None or qsl.device != dev:
            qsl_host = torch.zeros(n_seqs + 1, dtype=torch.long)
            torch.cumsum(hql, 0, out=qsl_host[1:])
            qsl = facts["qsl"] = qsl_host.to(dev)
    if append is not None:
        rc = L.pkv_paged_attention_prefill_append(
            out.data_ptr(), out.stride(0), out.stride(1),
            query.data_ptr(), query.stride(0), query.stride(1),
            *common_pool[:9],
            k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), k_new.stride(1), slots.data_ptr(),
            *common_pool[9:],
            ctx_dev.data_ptr(), qsl.data_ptr(),
            n_seqs, n_heads, n_tok, facts["max_q"],
            float(scale), dt,
            stream,
        )
        native.check(rc, "pkv_paged_attention_prefill_append")
        return out
    rc = L.pkv_paged_attention_prefill(
        out.data_ptr(), out.stride(0), out.stride(1),
        query.data_ptr(), query.stride(0), query.stride(1),
        *common_pool,
        ctx_dev.data_ptr(), qsl.data_ptr(),
        n_seqs, n_heads, n_tok, facts["max_q"],
        float(scale), dt,
        stream,
    )
    native.check(rc, "pkv_paged_attention_prefill")
    return out
