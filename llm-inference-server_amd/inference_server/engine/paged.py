"""A synchronous paged engine: model + pool + allocator + prefix cache + executor +
scheduler, driven step by step until every request finishes.

Wires the same components as the reference PagedEngine (inference_server/engine/
paged.py:52-82). The reference drives them from a background step thread behind an
asyncio/HTTP front end (engine/continuous.py); that front end is out of scope here,
so `run()` is the in-process closed loop: submit every request, step until the
scheduler drains, and report output tok/s = generated tokens / wall time from first
submit to last completion (the reference's metric, bench/metrics.py:73, :87).
"""

from __future__ import annotations

import time
from dataclasses import dataclass

import torch

from inference_server.config import CONFIG
from inference_server.core.block_allocator import BlockAllocator
from inference_server.core.kv_pool import ModelDims, PagedKVPool
from inference_server.core.paged_executor import PagedExecutor
from inference_server.core.prefix_cache import PrefixCache
from inference_server.core.scheduler import Scheduler
from inference_server.core.sequence import Sequence
from inference_server.model import sync


@dataclass
class Request:
    request_id: str
    prompt_token_ids: list[int]
    max_tokens: int


@dataclass
class RunResult:
    outputs: dict[str, list[int]]
    generated_tokens: int
    wall_s: float
    steps: int
    stats: dict

    @property
    def tok_per_s(self) -> float:
        return self.generated_tokens / self.wall_s if self.wall_s else 0.0


class PagedEngine:
    def __init__(self, model, tokenizer, *, num_blocks: int = CONFIG.num_blocks, block_size: int = CONFIG.block_size,
                 device: str | None = None, prefix_caching: bool | None = None,
                 capture_graphs: bool = False) -> None:
        self.model = model
        self.tokenizer = tokenizer
        self.device = device or str(next(model.parameters()).device)
        # The pool stores K/V in the model's own dtype (the reference takes it from the
        # DTYPE setting, which must then match the loaded model).
        dims = ModelDims.from_model(model, dtype=next(model.parameters()).dtype)
        self.pool = PagedKVPool(dims, num_blocks=num_blocks, block_size=block_size, device=self.device)
        self.allocator = BlockAllocator(self.pool.num_blocks)
        use_prefix = CONFIG.prefix_caching if prefix_caching is None else prefix_caching
        self.prefix_cache = PrefixCache(self.allocator, block_size) if use_prefix else None
        self.executor = PagedExecutor(model, tokenizer, self.pool)
        # Step graphs are captured on first use of each batch size / token bucket; a
        # server captures them all at start-up instead (the pool is still empty here).
        self.graph_capture_s = 0.0
        if capture_graphs:
            t0 = time.perf_counter()
            self.executor.capture_graphs()
            sync(self.device)
            self.graph_capture_s = time.perf_counter() - t0
        self.scheduler = Scheduler(self.executor, tokenizer.eos_token_id, allocator=self.allocator, pool=self.pool,
                                   prefix_cache=self.prefix_cache)

    def run(self, requests: list[Request], arrival_steps: list[int] | None = None,
            max_steps: int = 1_000_000) -> RunResult:
        """Submit every request (request i before step arrival_steps[i], default 0)
        and step until everything finished."""
        seqs = [Sequence(seq_id=r.request_id, prompt_token_ids=list(r.prompt_token_ids), max_tokens=r.max_tokens)
                for r in requests]
        arrivals = sorted(zip(arrival_steps or [0] * len(seqs), range(len(seqs))))
        t0 = time.perf_counter()
        steps = 0
        nxt = 0
        while nxt < len(arrivals) or self.scheduler.has_work:
            while nxt < len(arrivals) and arrivals[nxt][0] <= steps:
                self.scheduler.add(seqs[arrivals[nxt][1]])
                nxt += 1
            if steps >= max_steps:
                raise RuntimeError(f"scheduler did not drain in {max_steps} steps")
            self.scheduler.step()
            steps += 1
        sync(self.device)
        wall = time.perf_counter() - t0
        return RunResult(
            outputs={s.seq_id: list(s.output_token_ids) for s in seqs},
            generated_tokens=sum(s.num_generated for s in seqs),
            wall_s=wall,
            steps=steps,
            stats=self.scheduler.stats(),
        )

    def shutdown(self) -> None:
        self.executor.release()
        self.pool.release()
        if torch.device(self.device).type == "cuda":
            torch.cuda.empty_cache()
