"""Writes the golden vectors under tests/golden/ (seeded inputs + oracle outputs).

    python tests/golden/make_goldens.py

attention_cases.npz  every reference batch shape (tests/test_paged_attention_triton.py
                     :74-84) plus GQA, bs16/d64 and bs6/d12 cases: inputs and the
                     oracle gather output in float32. Each output is also checked
                     against the float64 textbook dense attention before it is saved.
kvops.npz            a small pool with append / copy-on-write / swap-out results.

The reference's own golden file (tests/goldens/gpt2_greedy.json) needs pretrained
GPT-2 weights that are not available offline, so it is not reproduced here.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, str(HERE.parent))

from cases import CASES, build, dense_causal_f64  # noqa: E402
from oracle import gather, kvops  # noqa: E402

EXTRA = {
    "gqa_kv1": ([(9, 9), (5, 1), (12, 3)], dict(kv_heads=1)),
    "bs16_d64": ([(33, 1), (16, 16), (40, 9)], dict(bs=16, d=64, num_blocks=8)),
    "bs6_d12": ([(13, 13), (7, 1), (18, 4)], dict(bs=6, d=12)),
}


def attention_cases() -> dict:
    arrays: dict[str, np.ndarray] = {}
    names = []
    items = [(n, (lens, {})) for n, lens in CASES.items()] + list(EXTRA.items())
    for name, (lengths, kw) in items:
        q, kp, vp, tables, ctx, ql = build(lengths, **kw)
        scale = q.shape[-1] ** -0.5
        out = gather.paged_attention_gather(q, kp, vp, tables, ctx, ql, scale)
        ref = dense_causal_f64(q, kp, vp, tables, ctx, ql, scale)
        np.testing.assert_allclose(out.numpy(), ref, atol=1e-5, rtol=1e-5)
        for key, t in (("q", q), ("k", kp), ("v", vp), ("tables", tables), ("ctx", ctx), ("ql", ql), ("out", out)):
            arrays[f"{name}/{key}"] = t.numpy()
        arrays[f"{name}/scale"] = np.float64(scale)
        names.append(name)
    arrays["names"] = np.array(names)
    return arrays


def kvops_case() -> dict:
    rng = np.random.default_rng(1337)
    pool = rng.integers(0, 2**16, size=(8, 4, 2, 8), dtype=np.uint16)
    rows = rng.integers(0, 2**16, size=(5, 2, 8), dtype=np.uint16)
    slots = rng.permutation(32)[:5].astype(np.int64)
    pairs = np.array([[1, 6], [3, 0], [7, 2]], dtype=np.int64)
    blocks = np.array([5, 1, 4], dtype=np.int64)
    return dict(
        pool=pool, rows=rows, slots=slots, pairs=pairs, swap_blocks=blocks,
        append_out=kvops.kv_append(pool, rows, slots),
        copy_out=kvops.copy_blocks(pool, [tuple(p) for p in pairs.tolist()]),
        swap_host=kvops.swap_out([pool], blocks.tolist())[0],
    )


def main() -> None:
    torch.set_num_threads(1)
    np.savez_compressed(HERE / "attention_cases.npz", **attention_cases())
    np.savez_compressed(HERE / "kvops.npz", **kvops_case())
    for f in sorted(HERE.glob("*.npz")):
        print(f"{f.name}: {f.stat().st_size} bytes")


if __name__ == "__main__":
    main()
