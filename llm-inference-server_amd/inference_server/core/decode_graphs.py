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

Prefill steps (every sequence of the batch is prefilling, the scheduler never mixes the
phases) are captured too, keyed by the packed token count rounded up to a bucket
(PREFILL_BUCKETS) rather than by batch size: the step's ids, positions and write slots
are padded to the bucket (padding rows write slot -1, which the append kernel skips, and
belong to no sequence), the sequences to `max_running` (padding sequences have no query
tokens, so no attention workgroup touches them), and the LM head reads only each real
sequence's last row. The GEMMs then see M = the bucket, not the real token count, so
the library may pick other kernels than the eager step: replays are compared with eager
steps token for token by tests, not assumed identical.

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
from inference_server.core.attention_hip import _WORKSPACES, attach_host, attach_query_start

#: hipGraphNodeType values (hip_runtime_api.h) the census reports by name.
NODE_KINDS = {0: "kernel", 1: "memcpy", 2: "memset", 3: "host", 4: "graph", 5: "empty",
              6: "wait_event", 7: "event_record"}
_NUM_TYPES = 16


#: Packed-token buckets of the prefill graphs (at most 1.5x padding between neighbours).
PREFILL_BUCKETS = (32, 64, 128, 256, 384, 512, 768, 1024, 1536, 2048, 3072, 4096, 6144, 8192)


class TableRows:
    """The block-table segment [N, W] of a pinned host metadata buffer, kept in step
    with the sequences' BlockTables incrementally: row i is rewritten only when the
    table now in slot i carries another version stamp than the one last written there
    (stamps are unique per table state, so a new table in the slot always differs).
    A decode step usually rewrites no row: a table changes once every block_size
    tokens."""

    def __init__(self, rows: np.ndarray) -> None:
        self.rows = rows
        self._stamp = [0] * rows.shape[0]
        self._len = [0] * rows.shape[0]
        self.rewrites = 0

    def write(self, tables) -> None:
        rows, stamp, length = self.rows, self._stamp, self._len
        for i, t in enumerate(tables):
            if stamp[i] == t.version:
                continue
            n = t.num_blocks
            rows[i, :n] = t.ids
            if length[i] > n:
                rows[i, n:length[i]] = 0
            stamp[i], length[i] = t.version, n
            self.rewrites += 1


def node_census(graph: torch.cuda.CUDAGraph) -> dict[str, int]:
    """Nodes of a captured graph (captured with keep_graph=True, not yet instantiated
    or still kept) by type name; types without a name are reported as `type<N>`."""
    counts = (ctypes.c_int64 * _NUM_TYPES)()
    native.check(native.lib().pkv_graph_node_counts(graph.raw_cuda_graph(), counts, _NUM_TYPES),
                 "pkv_graph_node_counts")
    return {NODE_KINDS.get(t, f"type{t}"): int(c) for t, c in enumerate(counts) if c}


def capture_step(body, device: torch.device, stream: torch.cuda.Stream, mempool, what: str):
    """Run `body` once eagerly on `stream` (lazy library set-up, the step's own work when
    the buffers hold a real step), then capture it into a graph from `mempool`, census
    its nodes, refuse memset and child-graph nodes, instantiate it. Returns (graph,
    body's output tensor, census)."""
    cur = torch.cuda.current_stream(device)
    stream.wait_stream(cur)
    with torch.cuda.stream(stream):
        body()
    cur.wait_stream(stream)
    graph = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(graph, pool=mempool, stream=stream):
        out = body()
    census = node_census(graph)
    if census.get("memset") or census.get("graph"):
        raise RuntimeError(f"{what} holds memset or child-graph nodes ({census}); "
                           "set DECODE_GRAPHS=0 to run steps eagerly")
    graph.instantiate()
    return graph, out, census


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
        self.rows = TableRows(self._hn[6 * n:].reshape(n, width))
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
                            pool=self.ex.pool, host_slots=torch.zeros(b, dtype=torch.long),
                            fuse_append=self.ex.fuse_append, epilogue=self.ex.qkv is not None)
        return self.ex._greedy(ids, pos, step, keep)

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
        graph, tokens, census = capture_step(lambda: self._body(b), self.device, self.stream, self.mempool,
                                             f"decode graph for batch {b}")
        self.census[b] = census
        self.graphs[b] = (graph, tokens)

    # ------------------------------------------------------------------ replay
    def run(self, step) -> list[int]:
        """One decode step (a HostStep of len(step.ids) sequences) the caller has
        validated: slots inside the pool, every table at most `width` blocks."""
        b = len(step.ids)
        o, hn = self._off, self._hn
        hn[o["ids"]:o["ids"] + b] = step.ids
        hn[o["pos"]:o["pos"] + b] = step.pos
        hn[o["slots"]:o["slots"] + b] = step.slots
        hn[o["ctx"]:o["ctx"] + b] = step.ctxs
        self.rows.write(step.tables)
        used = o["tables"] + b * self.width
        self.meta[:used].copy_(self.host[:used], non_blocking=True)
        if b not in self.graphs:
            self.capture(b)
        graph, tokens = self.graphs[b]
        graph.replay()
        self.replays += 1
        return tokens.tolist()


class PrefillGraphs:
    """Captured prefill steps of one executor, keyed by a bucket of the packed token
    count. Each bucket has its own persistent int64 device buffer, rewritten by one
    pinned host->device copy per step:

        ids[T] | pos[T] | slots[T] | ctx[N] | qlen[N] | qsl[N+1] | keep[N] | tables[N, W]

    (T = the bucket, N = the largest batch, W = the table width)."""

    def __init__(self, executor, max_batch: int, width: int) -> None:
        self.ex = executor
        self.max_batch = max_batch
        self.width = width
        self.device = torch.device(executor.device)
        self.max_context = width * executor.pool.block_size
        # A bucket's capture describes its widest step: sequences of at most
        # max_context tokens each, summing to the bucket.
        self.buckets = tuple(t for t in PREFILL_BUCKETS if t <= max_batch * self.max_context)
        self.stream = torch.cuda.Stream(device=self.device)
        self.mempool = torch.cuda.graph_pool_handle()
        self.bufs: dict[int, tuple[torch.Tensor, np.ndarray, torch.Tensor]] = {}
        self.rows: dict[int, TableRows] = {}
        self.graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor]] = {}
        self.census: dict[int, dict[str, int]] = {}
        self.replays = 0

    def bucket(self, num_tokens: int) -> int | None:
        for t in self.buckets:
            if num_tokens <= t:
                return t
        return None

    def _buffer(self, t: int):
        if t not in self.bufs:
            n, w = self.max_batch, self.width
            host = torch.zeros(3 * t + 4 * n + 1 + n * w, dtype=torch.long, pin_memory=True)
            hn = host.numpy()
            self.bufs[t] = (host, hn, host.to(self.device))
            self.rows[t] = TableRows(hn[3 * t + 4 * n + 1:].reshape(n, w))
        return self.bufs[t]

    def _split(self, buf, t: int):
        n, w = self.max_batch, self.width
        o = [0, t, 2 * t, 3 * t, 3 * t + n, 3 * t + 2 * n, 3 * t + 3 * n + 1, 3 * t + 4 * n + 1]
        return (buf[o[0]:o[1]], buf[o[1]:o[2]], buf[o[2]:o[3]], buf[o[3]:o[4]], buf[o[4]:o[5]],
                buf[o[5]:o[6]], buf[o[6]:o[7]], buf[o[7]:o[7] + n * w])

    def _body(self, t: int) -> torch.Tensor:
        from inference_server.core.paged_executor import _StepContext

        _, _, dev = self._buffer(t)
        ids, pos, slots, ctx, qlen, qsl, keep, tables = self._split(dev, t)
        n, cap = self.max_batch, self.max_context
        hq = torch.zeros(n, dtype=torch.long)
        full, rem = divmod(t, cap)
        hq[:full] = cap
        if rem:
            hq[full] = rem
        attach_host(ctx, hq.clone())
        attach_host(qlen, hq)
        attach_query_start(qlen, qsl)
        step = _StepContext(write_slots=slots, block_tables=tables.view(n, self.width), context_lens=ctx,
                            query_lens=qlen, pool=self.ex.pool, host_slots=torch.zeros(t, dtype=torch.long),
                            fuse_append=self.ex.fuse_append)
        return self.ex._greedy(ids.view(1, t), pos.view(1, t), step, keep)

    def capture(self, t: int) -> None:
        """Capture bucket t. As for decode: the eager pass before the capture runs on the
        buffer's contents — a real step (`run`) or, before any sequence owns a block,
        zeros (its rows then write slot 0 of block 0 and no sequence has query tokens)."""
        if t in self.graphs:
            return
        self._buffer(t)
        graph, tokens, census = capture_step(lambda: self._body(t), self.device, self.stream, self.mempool,
                                             f"prefill graph for {t} tokens")
        self.census[t] = census
        self.graphs[t] = (graph, tokens)

    def run(self, step) -> list[int]:
        """One prefill step (a HostStep) the caller has validated: slots inside the
        pool, at most max_batch sequences, every table at most `width` blocks, the
        token count within the largest bucket."""
        t_real, b = len(step.ids), len(step.qlens)
        t = self.bucket(t_real)
        host, hn, dev = self._buffer(t)
        h_ids, h_pos, h_slots, h_ctx, h_q, h_qsl, h_keep, _ = self._split(hn, t)
        h_ids[:t_real] = step.ids
        h_ids[t_real:] = 0
        h_pos[:t_real] = step.pos
        h_pos[t_real:] = 0
        h_slots[:t_real] = step.slots
        h_slots[t_real:] = -1
        h_ctx[:b] = step.ctxs
        h_ctx[b:] = 0
        h_q[:b] = step.qlens
        h_q[b:] = 0
        h_qsl[0] = 0
        np.cumsum(h_q, out=h_qsl[1:])
        h_keep[:b] = h_qsl[1:b + 1] - 1
        h_keep[b:] = 0
        self.rows[t].write(step.tables)
        dev.copy_(host, non_blocking=True)
        if t not in self.graphs:
            self.capture(t)
        graph, tokens = self.graphs[t]
        graph.replay()
        self.replays += 1
        return tokens[:b].tolist()
