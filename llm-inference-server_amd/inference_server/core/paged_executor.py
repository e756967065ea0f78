"""One forward pass of a HuggingFace causal LM whose KV cache is the paged pool.

The boundary where the KV hot path is called, with the reference's hooks
(inference_server/core/paged_executor.py:83-295):

* Packing: every sequence's new tokens go into ONE row, input_ids [1, T], with
  per-token position_ids; block tables (0-padded), context_lens (cached AFTER the
  pass), query_lens and the flat write slots describe the batch to the kernels.
* `_PagedCache.update` (transformers calls it per layer with the new K/V) scatters
  them into the pool — PagedKVPool.append, one HIP launch for K and V on the hip
  backend — and returns them untouched.
* `_paged_attention_forward` is registered in transformers' AttentionInterface; it
  ignores the K/V it is handed and reads everything back out of the pool through the
  block tables via core.attention.paged_attention.
* Copy-on-write: before a block is written, BlockTable.ensure_private moves the
  sequence onto a fresh block; the step's copies are collected and issued as ONE
  PagedKVPool.copy_blocks call (one launch over every pair and layer on hip) before
  the forward, where the reference copies one block per hook call.

* Decode steps on ATTENTION=hip (every sequence feeds one token, at most
  CONFIG.max_running of them) replay a HIP graph captured once per batch size
  (core/decode_graphs.py): the same kernels as the eager step, over one persistent
  device metadata buffer rewritten by one copy per step. Prefill steps replay a graph
  captured per packed-token bucket, padded to it (PREFILL_GRAPHS=0 turns that off).

Differences from the reference, none visible in the outputs: write slots are
computed only for the new positions (the reference materialises every slot of the
sequence, O(context) per step), and on a GPU the metadata tensors carry host copies
of their values so the hip path validates without device->host syncs.
"""

from __future__ import annotations

import contextlib
from dataclasses import dataclass

import numpy as np
import torch
from transformers import AttentionInterface, Cache

from inference_server.config import CONFIG
from inference_server.core.attention import paged_attention
from inference_server.core.attention_hip import attach_host, paged_attention_hip_launch
from inference_server.core.decode_graphs import DecodeGraphs, PrefillGraphs
from inference_server.core.kv_pool import PagedKVPool
from inference_server.core.qkv_epilogue import QkvEpilogue
from inference_server.core.sampling import fused_greedy_supported, fused_max_rows, lm_head_argmax, lm_head_weight
from inference_server.core.sequence import Sequence

#: The name the model's config points at while a paged forward runs.
ATTN_IMPL = "inference_server_paged"


@dataclass
class HostStep:
    """One pass as the host sees it: packed new token ids and their positions, the
    flat pool slot each is written to, per-sequence query and context lengths, and
    the sequences' block tables (widest = `width` blocks)."""
    ids: list[int]
    pos: list[int]
    slots: np.ndarray             # int64 [T]
    qlens: list[int]
    ctxs: list[int]
    tables: list                  # BlockTable per sequence
    width: int


@dataclass(frozen=True)
class _StepContext:
    write_slots: torch.Tensor     # int64 [T]: flat pool slot of each new token
    block_tables: torch.Tensor    # int64 [B, W], 0-padded
    context_lens: torch.Tensor    # int64 [B]: cached tokens after this pass
    query_lens: torch.Tensor      # int64 [B]: new tokens per sequence
    pool: PagedKVPool
    host_slots: torch.Tensor | None = None  # CPU copy of write_slots (hip range checks)
    # hip with a 16-bit pool: the attention call writes each layer's new K/V rows
    # (pkv_paged_attention_decode_append on decode steps, pkv_paged_attention_prefill_append
    # otherwise) and `update` only checks the slots.
    fuse_append: bool = False
    # Decode step with a QKV epilogue (implies fuse_append): every layer's c_attn runs
    # as pkv_qkv_append, which already stored K/V at their slots; attention only reads.
    epilogue: bool = False


class _PagedCache(Cache):
    """A Cache whose only job is to catch `update` and write into the pool."""

    def __init__(self, ctx: _StepContext) -> None:
        super().__init__(layers=[])
        self.ctx = ctx

    def update(self, key_states, value_states, layer_idx: int, *args, **kwargs):
        # [1, Hkv, T, D] -> [T, Hkv, D] views; the append takes the strides as they are.
        if self.ctx.fuse_append:
            self.ctx.pool.check_slots(self.ctx.write_slots, self.ctx.host_slots)
            return key_states, value_states
        k = key_states[0].transpose(0, 1)
        v = value_states[0].transpose(0, 1)
        self.ctx.pool.append(layer_idx, k, v, self.ctx.write_slots, host_slots=self.ctx.host_slots)
        return key_states, value_states

    def get_seq_length(self, layer_idx: int = 0) -> int:
        raise RuntimeError("PagedExecutor must pass explicit position_ids; the pool has no single length")

    def get_mask_sizes(self, query_length: int, layer_idx: int = 0):
        raise RuntimeError("no mask is built for the paged kernel; create_causal_mask should have early-exited")


def _paged_attention_forward(module, query, key, value, attention_mask, scaling=None, **kwargs):
    """AttentionInterface hook: [1, H, T, D] in, ([1, T, H, D], None) out."""
    ctx: _StepContext = kwargs["paged_ctx"]
    if scaling is None:
        scaling = query.shape[-1] ** -0.5
    q = query[0].transpose(0, 1)                                  # [T, H, D], strided
    if ctx.fuse_append and not ctx.epilogue:
        # `key` / `value` are the step's new rows, as `update` returned them unwritten.
        new = (key[0].transpose(0, 1), value[0].transpose(0, 1), ctx.write_slots)
        out = paged_attention_hip_launch(q, ctx.pool.k[module.layer_idx], ctx.pool.v[module.layer_idx],
                                         ctx.block_tables, ctx.context_lens, ctx.query_lens, scaling, append=new)
    else:
        out = paged_attention(q, ctx.pool.k[module.layer_idx], ctx.pool.v[module.layer_idx], ctx.block_tables,
                              ctx.context_lens, ctx.query_lens, scaling)
    return out.unsqueeze(0), None


AttentionInterface.register(ATTN_IMPL, _paged_attention_forward)


class PagedExecutor:
    """One forward pass over the pool, no policy (reference: core/paged_executor.py:162-295)."""

    def __init__(self, model, tokenizer, pool: PagedKVPool, decode_graphs: bool | None = None,
                 max_batch: int | None = None) -> None:
        self.model = model
        self.tokenizer = tokenizer
        self.pool = pool
        self.device = pool.device
        self.graphs: DecodeGraphs | None = None
        self.prefill_graphs: PrefillGraphs | None = None
        # LM head weight for greedy sampling fused into the head (hip backend only:
        # `gather` keeps the reference's logits + argmax).
        # Every step (eager or replayed from graphs) writes each layer's new K/V inside
        # the attention call (16-bit pools on hip; FUSED_APPEND=0 turns it off).
        self.fuse_append = (CONFIG.attention == "hip" and CONFIG.fused_append
                            and pool.k[0].dtype in (torch.float16, torch.bfloat16))
        # Decode steps of a GPT-2-shaped 16-bit model project Q/K/V with the K/V append in
        # the projection's epilogue (pkv_qkv_append), unless QKV_EPILOGUE=0.
        self.qkv: QkvEpilogue | None = (QkvEpilogue.make(model, pool)
                                        if self.fuse_append and CONFIG.qkv_epilogue else None)
        head = lm_head_weight(model) if CONFIG.attention == "hip" and CONFIG.fused_greedy else None
        self.fused_head: torch.Tensor | None = head if fused_greedy_supported(head) else None
        #: Debug hook: called as logit_probe(seqs, logits) with the [B, vocab] logits of
        #: each step's sampled rows, on steps that compute logits (eager steps without
        #: the fused LM head). Parity tests record top-1/top-2 margins through it.
        self.logit_probe = None
        if decode_graphs is None:
            decode_graphs = CONFIG.decode_graphs
        if decode_graphs and CONFIG.attention == "hip" and torch.device(self.device).type == "cuda":
            cfg = model.config
            positions = getattr(cfg, "max_position_embeddings", None) or getattr(cfg, "n_positions", None) \
                or CONFIG.max_seq_len
            width = -(-positions // pool.block_size)
            self.graphs = DecodeGraphs(self, max_batch or CONFIG.max_running, width)
            if CONFIG.prefill_graphs:
                self.prefill_graphs = PrefillGraphs(self, max_batch or CONFIG.max_running, width)

    def release(self) -> None:
        """Drop the captured graphs (they point into the pool; call before freeing it)."""
        if self.graphs is not None or self.prefill_graphs is not None:
            torch.cuda.synchronize(torch.device(self.device))
            self.graphs = None
            self.prefill_graphs = None

    def capture_graphs(self) -> None:
        """Capture every decode batch size and prefill bucket up front (largest first, so
        each graph pool grows once). Call it while no sequence owns any pool block."""
        with torch.inference_mode():
            if self.graphs is not None:
                for b in range(self.graphs.max_batch, 0, -1):
                    self.graphs.capture(b)
            if self.prefill_graphs is not None:
                for t in reversed(self.prefill_graphs.buckets):
                    self.prefill_graphs.capture(t)

    @torch.inference_mode()
    def execute(self, seqs: list[Sequence]) -> list[int]:
        """Advance every sequence by one token; returns the greedy token ids."""
        if not seqs:
            return []
        phase = seqs[0].is_prefilling
        assert all(s.is_prefilling is phase for s in seqs), "mixed prefill/decode batch — the scheduler must split these"
        step = self._host_step(seqs)
        graphs = self.prefill_graphs if phase else self.graphs
        if (graphs is not None and len(seqs) <= graphs.max_batch and step.width <= graphs.width
                and (not phase or graphs.bucket(len(step.ids)))):
            if step.slots.size and (int(step.slots.min()) < 0 or int(step.slots.max()) >= self.pool.num_slots):
                raise IndexError(f"slot index outside [0, {self.pool.num_slots})")
            tokens = graphs.run(step)
        else:
            input_ids, position_ids, ctx, ends = self._pack(step)
            # Only each sequence's last position is sampled, so only those rows go
            # through the LM head (HF's logits_to_keep): [B, vocab] logits instead of
            # the reference's [T, vocab]; the greedy argmax runs on the device (fused
            # into the LM head where supported) and B ids come back.
            tokens = self._greedy(input_ids, position_ids, ctx, ends - 1, seqs).tolist()
        for s in seqs:
            s.num_cached += s.num_next_tokens
        return tokens

    def reset(self) -> None:
        """Nothing survives between passes."""

    # ------------------------------------------------------------------ packing
    def _tensor(self, values, shape=None) -> torch.Tensor:
        host = torch.as_tensor(values, dtype=torch.long)
        if shape is not None:
            host = host.view(shape)
        if torch.device(self.device).type == "cpu":
            return host
        return attach_host(host.to(self.device), host)

    def _host_step(self, seqs: list[Sequence]) -> "HostStep":
        """The pass on the host (new token ids, positions, write slots, lengths, the
        sequences' block tables), after giving every block the pass writes a private
        copy. Copy-on-write pairs of the whole step go out as ONE copy_blocks call
        before anything writes the pool: a deferred source keeps a reference, so no
        allocation later in this loop can hand it out as a destination, and
        destinations are fresh blocks nothing reads yet."""
        cow: list[tuple[int, int]] = []
        record = lambda src, dst: cow.append((src, dst))  # noqa: E731
        ids: list[int] = []
        pos: list[int] = []
        qlens: list[int] = []
        ctxs: list[int] = []
        tables = []
        slot_parts = []
        width = 0
        for s in seqs:
            table = s.block_table
            assert table is not None, f"{s.seq_id} reached the paged executor without a block table"
            start, after = s.num_cached, s.total_len
            assert table.capacity >= after, (
                f"{s.seq_id}: block table holds {table.capacity} slots, pass needs {after} — "
                "the scheduler must call ensure_capacity before execute")
            table.make_writable(start, after, record)
            ids.extend(s.next_input_ids)
            qlens.append(after - start)
            ctxs.append(after)
            tables.append(table)
            width = max(width, table.num_blocks)
            if after - start == 1:
                pos.append(start)
                slot_parts.append(table.slot_of(start))
            else:
                pos.extend(range(start, after))
                slot_parts.extend(table.slot_range(start, after).tolist())
        self.pool.copy_blocks(cow)
        return HostStep(ids, pos, np.asarray(slot_parts, dtype=np.int64), qlens, ctxs, tables, width)

    def _pack(self, step: "HostStep"):
        """Device tensors of an eagerly issued pass (host copies attached for the hip
        path's checks)."""
        rows = np.zeros((len(step.tables), max(step.width, 1)), dtype=np.int64)
        for i, t in enumerate(step.tables):
            rows[i, :t.num_blocks] = t.ids
        slot_t = self._tensor(step.slots)
        ctx = _StepContext(
            write_slots=slot_t,
            block_tables=self._tensor(rows),
            context_lens=self._tensor(step.ctxs),
            query_lens=self._tensor(step.qlens),
            pool=self.pool,
            host_slots=getattr(slot_t, "_pkv_host", slot_t),
            fuse_append=self.fuse_append,
            epilogue=self.qkv is not None and all(q == 1 for q in step.qlens),
        )
        ends = torch.tensor(step.qlens, dtype=torch.long).cumsum(0).to(self.device)
        input_ids = torch.tensor([step.ids], dtype=torch.long).to(self.device)
        position_ids = torch.tensor([step.pos], dtype=torch.long).to(self.device)
        return input_ids, position_ids, ctx, ends

    def _copy_block(self, src: int, dst: int) -> None:
        """COW hook for BlockTable.ensure_private: block src -> dst, every layer."""
        self.pool.copy_block(src, dst)

    # ------------------------------------------------------------------ forward
    def _forward(self, input_ids: torch.Tensor, position_ids: torch.Tensor, ctx: _StepContext,
                 keep: torch.Tensor | None = None, hidden_only: bool = False) -> torch.Tensor:
        """The model's logits for the rows `keep` (all rows if None), or with
        hidden_only its final hidden states [1, T, hidden] (the LM head not applied)."""
        config = self.model.config
        previous = config._attn_implementation
        config._attn_implementation = ATTN_IMPL
        extra = {} if keep is None or hidden_only else {"logits_to_keep": keep}
        module = self.model.base_model if hidden_only else self.model
        try:
            with self.qkv.installed(ctx) if ctx.epilogue else contextlib.nullcontext():
                out = module(input_ids=input_ids, position_ids=position_ids, past_key_values=_PagedCache(ctx),
                             use_cache=True, paged_ctx=ctx, **extra)
        finally:
            config._attn_implementation = previous
        return out.last_hidden_state if hidden_only else out.logits

    def _greedy(self, input_ids: torch.Tensor, position_ids: torch.Tensor, ctx: _StepContext,
                keep: torch.Tensor, seqs: list[Sequence] | None = None) -> torch.Tensor:
        """int64 [B] greedy ids of the rows `keep`: the reference's
        `logits[0, ends - 1, :].argmax(-1)` (core/paged_executor.py:194-203). With a
        fused-capable LM head (hip backend, fp16/bf16) the final hidden states of those
        rows go straight to core.sampling.lm_head_argmax and no logits are written (up
        to fused_max_rows(hidden size) rows; the GEMM + argmax is faster for more)."""
        if self.fused_head is None or keep.numel() > fused_max_rows(self.fused_head.shape[1]):
            logits = self._forward(input_ids, position_ids, ctx, keep=keep)[0]
            if self.logit_probe is not None and seqs is not None:
                self.logit_probe(seqs, logits)
            return logits.argmax(-1)
        hidden = self._forward(input_ids, position_ids, ctx, hidden_only=True)
        return lm_head_argmax(hidden[0].index_select(0, keep), self.fused_head)
