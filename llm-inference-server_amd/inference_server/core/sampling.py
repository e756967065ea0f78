"""Greedy sampling fused into the LM head (HIP backend).

The reference samples every step with `logits[0, ends - 1, :].argmax(-1)`
(inference_server/core/paged_executor.py:194-203): the model's LM head writes
[rows, vocab] logits in the model dtype and argmax picks the first maximum of each
row. `lm_head_argmax` returns the same ids from the final hidden states and the LM
head weight in one library call (`pkv_lm_head_argmax`): each logit is accumulated in
fp32 and rounded to the model dtype before ranking, ties go to the lowest index, and
the logits are never materialised.

fp16 and bf16 only; `fused_greedy_supported` says whether a model's LM head qualifies
(bias-free Linear over the hidden size, a dtype with a kernel). Callers keep the
matmul + argmax for everything else, and for more rows than `fused_max_rows` allows.
"""

from __future__ import annotations

import threading

import torch

from inference_server import native

_FUSED_DTYPES = (torch.float16, torch.bfloat16)

#: Most sampled rows the executor sends through the fused kernel at hidden sizes up to
#: 1200. Its time grows with the row count (each 16 rows add a column tile of MFMAs and
#: LDS reads per weight byte): GPT-2 fp16 on MI355X, 16.4 / 17.7 / 19.6 us at 1 / 32 / 64
#: rows vs ~35 us for the LM-head GEMM + argmax.
FUSED_MAX_ROWS = 64

#: Hidden-row bytes one workgroup of the streaming kernel stages in LDS
#: (csrc/greedy.hip kLdsBudget).
_LDS_BUDGET = 150 * 1024


class _Workspaces:
    """One greedy-sampling workspace per (device, stream), zero-filled when allocated and
    reused by every later call: the kernel merges the rows' keys inside its launch and
    keeps that merge's state (an arrival counter, the keys) in the workspace, which must
    read zero when a call starts; every completed call leaves it zero. Calls on one
    stream are ordered; another stream gets its own buffer. A buffer that had to grow is
    kept alive, not freed: a graph captured on that stream earlier replays into it. After
    a call that did not complete, `reset_workspaces()` drops every buffer."""

    _MIN_BYTES = 64 << 10   # the counter and 8 keys per row for up to ~1000 rows

    def __init__(self) -> None:
        self._lock = threading.Lock()
        self._bufs: dict[tuple[int, int], torch.Tensor] = {}
        self._kept: list[torch.Tensor] = []

    def get(self, device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        key = (idx, stream)
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                if buf is not None:
                    self._kept.append(buf)
                buf = torch.zeros(max(nbytes, self._MIN_BYTES), dtype=torch.uint8, device=device)
                self._bufs[key] = buf
            return buf

    def drop(self, device: torch.device, stream: int) -> None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        with self._lock:
            buf = self._bufs.pop((idx, stream), None)
            if buf is not None:
                self._kept.append(buf)

    def reset(self) -> None:
        with self._lock:
            self._bufs.clear()
            self._kept.clear()


_WORKSPACES = _Workspaces()


def reset_workspaces() -> None:
    """Forget every greedy workspace (the next call on each stream allocates a zeroed one)."""
    _WORKSPACES.reset()


def fused_max_rows(hidden_size: int) -> int:
    """Most sampled rows for which the fused kernel beats the GEMM + argmax: the rows
    its streaming kernel takes in one pass over the weight (16-row column tiles, at most
    4, that fit the LDS budget). Past one pass the weight is streamed again per pass:
    Llama-sized [32000, 4096] fp16 head on MI355X, fused 47.6 us vs 55.3 us for the GEMM
    + argmax at 16 rows (one pass), 86.7 vs 54.0 us at 32 rows (two)."""
    tiles = 4
    while tiles and 16 * tiles * hidden_size * 2 > _LDS_BUDGET:
        tiles //= 2
    return min(FUSED_MAX_ROWS, 16 * tiles)


def lm_head_weight(model) -> torch.Tensor | None:
    """The [vocab, hidden] weight of a model's bias-free LM head, or None if it has no
    plain one (a bias, or an output layer that is not a Linear)."""
    head = model.get_output_embeddings() if hasattr(model, "get_output_embeddings") else None
    if not isinstance(head, torch.nn.Linear) or head.bias is not None:
        return None
    return head.weight


def fused_greedy_supported(weight: torch.Tensor | None) -> bool:
    """True when `lm_head_argmax` has a kernel for this LM head weight."""
    return (
        weight is not None
        and weight.device.type == "cuda"
        and weight.dtype in _FUSED_DTYPES
        and weight.dim() == 2
        and weight.stride(1) == 1
        and weight.shape[1] % 16 == 0
        and weight.stride(0) % 8 == 0
        and weight.data_ptr() % 16 == 0
    )


def lm_head_argmax(hidden: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """int64 [rows] = (hidden @ weight.T).to(dtype).argmax(-1), fused.

    hidden: [rows, hidden_size]; weight: [vocab, hidden_size]; same fp16/bf16 dtype and
    device. Raises ValueError on a shape or dtype mismatch and NotImplementedError when
    the library is missing or has no kernel for the layout (never a fallback)."""
    if hidden.dim() != 2 or weight.dim() != 2:
        raise ValueError(f"lm_head_argmax: hidden must be [rows, hidden] and weight [vocab, hidden], got "
                         f"{tuple(hidden.shape)} and {tuple(weight.shape)}")
    if hidden.shape[1] != weight.shape[1]:
        raise ValueError(f"lm_head_argmax: hidden size {hidden.shape[1]} != weight's {weight.shape[1]}")
    if hidden.dtype != weight.dtype:
        raise ValueError(f"lm_head_argmax: hidden is {hidden.dtype}, weight is {weight.dtype}")
    if hidden.device != weight.device:
        raise ValueError(f"lm_head_argmax: hidden on {hidden.device}, weight on {weight.device}")
    native.require_gpu(hidden, "lm_head_argmax")
    if hidden.dtype not in _FUSED_DTYPES:
        raise NotImplementedError(f"lm_head_argmax: no fused kernel for {hidden.dtype} (fp16 and bf16 only)")
    rows, dim = hidden.shape
    # The kernel reads whole 16-byte pieces of each row: unit inner stride, row stride a
    # multiple of 8 elements and no smaller than a row, 16-byte aligned base.
    if hidden.stride(1) != 1 or hidden.stride(0) < dim or hidden.stride(0) % 8 or hidden.data_ptr() % 16:
        hidden = hidden.clone(memory_format=torch.contiguous_format)
    vocab = weight.shape[0]
    ids = torch.empty(rows, dtype=torch.long, device=hidden.device)
    if rows == 0:
        return ids
    L = native.lib()
    nbytes = L.pkv_lm_head_argmax_workspace_bytes(rows, vocab)
    stream = native.stream_handle(hidden.device)
    workspace = _WORKSPACES.get(hidden.device, stream, nbytes)
    rc = L.pkv_lm_head_argmax(hidden.data_ptr(), hidden.stride(0), weight.data_ptr(), weight.stride(0),
                              rows, dim, vocab, native.dtype_code(hidden.dtype), ids.data_ptr(),
                              workspace.data_ptr(), workspace.numel(), stream)
    if rc == native.PKV_EUNSUPPORTED:
        raise NotImplementedError(L.pkv_last_error().decode(errors="replace"))
    if rc:
        _WORKSPACES.drop(hidden.device, stream)   # its merge state may be incomplete
    native.check(rc, "pkv_lm_head_argmax")
    return ids
