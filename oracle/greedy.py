"""Oracle: greedy sampling over the LM head, restated in numpy.

Test infrastructure only (see oracle/__init__.py). The reference samples with
`logits[0, ends - 1, :].argmax(-1)` (inference_server/core/paged_executor.py:194-203):
logits are the bias-free LM head in the model dtype, and argmax returns the first
maximum of each row.
"""

from __future__ import annotations

import numpy as np


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values rounded to `dtype` ("float16", "bfloat16" or "float32") and widened
    back to float32; bf16 rounds to nearest, ties to even, on the float32 bits."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "float32":
        return x.copy()
    if dtype == "float16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        u = x.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
        nan = np.isnan(x)
        out = r.astype(np.uint32).view(np.float32).copy()
        out[nan] = np.nan
        return out
    raise ValueError(dtype)


def logits(hidden: np.ndarray, weight: np.ndarray, dtype: str) -> np.ndarray:
    """The LM head's [rows, vocab] output as the model dtype holds it: exact (float64)
    dot products rounded once to float32, then to `dtype`."""
    exact = np.asarray(hidden, dtype=np.float64) @ np.asarray(weight, dtype=np.float64).T
    return round_to(exact.astype(np.float32), dtype)


def greedy_ids(hidden: np.ndarray, weight: np.ndarray, dtype: str) -> np.ndarray:
    """int64 [rows]: first index of each row's maximum logit (torch.argmax's rule)."""
    return np.argmax(logits(hidden, weight, dtype), axis=-1).astype(np.int64)
