"""HIP-graph replay of the paged engine's decode steps.

A decode step (every sequence feeds one token) launches the same kernels every time
for a given batch size B: per layer the QKV projection, the KV append, paged decode
attention, the output projection and the MLP; then the LM head on the B sampled rows
and the greedy argmax. Issued eagerly from transformers' Python modules that is a few
milliseconds of host work per step for well under one millisecond of GPU work.
Captured once per B and replayed, a step is one host->device copy, one graph launch
and one device->host read of B token ids.

Step metadata lives in ONE persistent device buffer of int64, rewritten by one copy
from a pinned host mirror before each replay:

    ids[N] | pos[N] | slots[N] | ctx[N] | qlen[N] (= 1) | keep[N] (= 0..N-1) | tables[N, W]

(N = the largest batch, W = the block-table width every graph is captured with). The
graph for batch size B reads the first B entries of each segment and the first B
table rows, so every graph shares the one buffer and the one copy.

Attention is captured with the widest context a W-block table allows
(max_context_len = W * block_size): the grid covers every partition a sequence can
have, workgroups past a sequence's own context exit at once, and the split-KV
workspace is sized for it. A sequence's output depends only on its own context and
the GEMMs see the same M = B as the eager step, so a replay computes bit for bit what
the eager step computes.

Every capture is checked before it is instantiated: its nodes are counted by type
through libpagedkv (pkv_graph_node_counts) and a graph holding a memset node is
refused — such nodes have given wrong results on replays after the first on these
GPUs, so anything that needs clearing inside a step is cleared by a kernel.

No memory is allocated or freed while graphs are live except inside their private
pool: the split-KV workspace of the capture stream is sized for (N, W * block_size)
before the first capture, so no later capture can grow (and free) a buffer an earlier
graph points at.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from inference_server import native
from inference_server.core.attention_hip import _WORKSPACES, attach_host

#: hipGraphNodeType values (hip_runtime_api.h) the census reports by name.
NODE_KINDS = {0: "kernel", 1: "memcpy", 2: "memset", 3: "host", 4: "graph", 5: "empty",
              6: "wait_event", 7: "event_record"}
_NUM_TYPES = 16


def node_census(graph: torch.cuda.CUDAGraph) -> dict[str, int]:
    """Nodes of a captured graph (captured with keep_graph=True, not yet instantiated
    or still kept) by type name; types without a name are reported as `type<N>`."""
    counts = (ctypes.c_int64 * _NUM_TYPES)()
    native.check(native.lib().pkv_graph_node_counts(graph.raw_cuda_graph(), counts, _NUM_TYPES),
                 "pkv_graph_node_counts")
    return {NODE_KINDS.get(t, f"type{t}"): int(c) for t, c in enumerate(counts) if c}


class DecodeGraphs:
    """Captured decode steps of one executor, keyed by batch size."""

    def __init__(self, executor, max_batch: int, width: int) -> None:
        if max_batch < 1 or width < 1:
            raise ValueError(f"decode graphs need max_batch >= 1 and width >= 1, got {max_batch}, {width}")
        self.ex = executor
        self.max_batch = max_batch
        self.width = width
        self.device = torch.device(executor.device)
        n = max_batch
        self._off = {"ids": 0, "pos": n, "slots": 2 * n, "ctx": 3 * n, "qlen": 4 * n, "keep": 5 * n, "tables": 6 * n}
        total = 6 * n + n * width
        self.host = torch.zeros(total, dtype=torch.long, pin_memory=True)
        self._hn = self.host.numpy()
        self._hn[4 * n:5 * n] = 1
        self._hn[5 * n:6 * n] = np.arange(n)
        self.meta = self.host.to(self.device)
        self.stream = torch.cuda.Stream(device=self.device)
        self.mempool = torch.cuda.graph_pool_handle()
        self.graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor]] = {}
        self.census: dict[int, dict[str, int]] = {}
        self.replays = 0
        pool = executor.pool
        self.max_context = width * pool.block_size
        heads = executor.model.config.num_attention_heads
        ws = native.lib().pkv_paged_attention_decode_workspace_bytes(
            n, heads, pool.dims.num_kv_heads, pool.dims.head_dim, self.max_context)
        _WORKSPACES.partials(self.device, self.stream.cuda_stream, ws)

    # ------------------------------------------------------------------ views
    def _views(self, b: int):
        m, o = self.meta, self._off
        return (
            m[o["ids"]:o["ids"] + b].view(1, b),
            m[o["pos"]:o["pos"] + b].view(1, b),
            m[o["slots"]:o["slots"] + b],
            m[o["ctx"]:o["ctx"] + b],
            m[o["qlen"]:o["qlen"] + b],
            m[o["keep"]:o["keep"] + b],
            m[o["tables"]:o["tables"] + b * self.width].view(b, self.width),
        )

    def _body(self, b: int) -> torch.Tensor:
        """One decode step over the static views; returns the [b] greedy token ids.
        The host copies attached for the contract checks describe the widest batch a
        graph must serve (every context at W * block_size), which is what sizes the
        attention grid; the kernels read the real lengths from the device buffer."""
        from inference_server.core.paged_executor import _StepContext

        ids, pos, slots, ctx, qlen, keep, tables = self._views(b)
        attach_host(ctx, torch.full((b,), self.max_context, dtype=torch.long))
        attach_host(qlen, torch.ones(b, dtype=torch.long))
        step = _StepContext(write_slots=slots, block_tables=tables, context_lens=ctx, query_lens=qlen,
                            pool=self.ex.pool, host_slots=torch.zeros(b, dtype=torch.long))
        logits = self.ex._forward(ids, pos, step, keep=keep)
        return logits[0].argmax(-1)

    # ------------------------------------------------------------------ capture
    def capture(self, b: int) -> None:
        """Capture the step for batch size b. The eager warm-up pass before the capture
        runs on whatever the buffer holds: call this only when the buffer's first b
        rows describe a real step (`run` does) or while no sequence owns any block
        (the warm-up's dummy rows, context 0, then only write slot 0 of block 0)."""
        if not 1 <= b <= self.max_batch:
            raise ValueError(f"batch {b} outside [1, {self.max_batch}]")
        if b in self.graphs:
            return
        cur = torch.cuda.current_stream(self.device)
        self.stream.wait_stream(cur)
        with torch.cuda.stream(self.stream):
            self._body(b)
        cur.wait_stream(self.stream)
        graph = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(graph, pool=self.mempool, stream=self.stream):
            tokens = self._body(b)
        census = node_census(graph)
        if census.get("memset") or census.get("graph"):
            raise RuntimeError(f"decode graph for batch {b} holds memset or child-graph nodes ({census}); "
                               "set DECODE_GRAPHS=0 to run decode steps eagerly")
        graph.instantiate()
        self.census[b] = census
        self.graphs[b] = (graph, tokens)

    # ------------------------------------------------------------------ replay
    def run(self, ids: list[int], pos: list[int], slots: list[int], ctx: list[int],
            tables: list[list[int]]) -> list[int]:
        """One decode step for len(ids) sequences, from host lists the caller has
        validated (slots inside the pool, every table at most `width` blocks)."""
        b = len(ids)
        o, hn, w = self._off, self._hn, self.width
        hn[o["ids"]:o["ids"] + b] = ids
        hn[o["pos"]:o["pos"] + b] = pos
        hn[o["slots"]:o["slots"] + b] = slots
        hn[o["ctx"]:o["ctx"] + b] = ctx
        rows = hn[o["tables"]:o["tables"] + b * w].reshape(b, w)
        rows[:] = 0
        for i, t in enumerate(tables):
            rows[i, :len(t)] = t
        used = o["tables"] + b * w
        self.meta[:used].copy_(self.host[:used], non_blocking=True)
        if b not in self.graphs:
            self.capture(b)
        graph, tokens = self.graphs[b]
        graph.replay()
        self.replays += 1
        return tokens.tolist()
