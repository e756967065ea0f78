"""Seeded request lists for the end-to-end configs (token ids drawn directly; the
reference slices a text corpus through the pretrained tokenizer, which is not
available offline — bench/workload.py:86-118 there).

config1: 8 requests, prompt lengths U[16, 256], ids U[0, vocab), 32 greedy tokens.
config5: 200 requests, prompt lengths U[16, 256], output lengths
         clip(exp(N(3.4, 0.9)), 8, 512) (reference bench/workload.py:30-32, 97-98);
         50% of requests start with one shared 128-token prefix.
"""

from __future__ import annotations

import numpy as np

from inference_server.config import SEED
from inference_server.engine.paged import Request


def config1(vocab: int = 50257, n: int = 8, max_tokens: int = 32, seed: int = SEED) -> list[Request]:
    rng = np.random.default_rng(seed)
    lens = rng.integers(16, 257, size=n)
    return [Request(f"c1-{i:03d}", rng.integers(0, vocab, size=int(lens[i])).tolist(), max_tokens) for i in range(n)]


def config5(vocab: int = 50257, n: int = 200, shared_prefix: int = 128, seed: int = SEED) -> list[Request]:
    rng = np.random.default_rng(seed)
    out_lens = np.clip(np.exp(rng.normal(3.4, 0.9, n)), 8, 512).astype(int)
    prompt_lens = rng.integers(16, 257, size=n)
    prefix = rng.integers(0, vocab, size=shared_prefix).tolist()
    share = rng.random(n) < 0.5
    reqs = []
    for i in range(n):
        tail = rng.integers(0, vocab, size=int(prompt_lens[i])).tolist()
        prompt = (prefix + tail) if share[i] else tail
        reqs.append(Request(f"c5-{i:03d}", prompt, int(out_lens[i])))
    return reqs
