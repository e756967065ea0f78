"""QKV projection with the KV append in its epilogue, for decode steps (ATTENTION=hip).

Per layer of a step the reference's model projects the hidden rows with GPT-2's fused
QKV Conv1D (`c_attn`, addmm(bias, x, W) with W [hidden, 3 * hidden]), splits Q/K/V, and
`_PagedCache.update` scatters K and V into the pool (reference
core/paged_executor.py:116-125). `QkvEpilogue` replaces the `c_attn` call of every
layer, for the duration of one forward, with `pkv_qkv_append`: the same projection
(fp32 accumulation, the bias added, one rounding to the model dtype) whose epilogue
also stores each K and V element at its row's pool slot. The layer's `update` then only
checks the slots, and attention reads the pool as it stands.

Used for decode steps of fp16/bf16 models whose attention blocks carry a bias-carrying
Conv1D `c_attn` over [Q | K | V] (GPT-2); prefill steps keep the model's own GEMM and
the append inside the attention call. Each layer's weight is kept once more, transposed
([3 * hidden, hidden], hidden contiguous), so both operands of the kernel's MFMA tiles
are contiguous loads.
"""

from __future__ import annotations

import contextlib

import torch

from inference_server import native

_DTYPES = (torch.float16, torch.bfloat16)


def _attention_blocks(model) -> list | None:
    base = getattr(model, "transformer", None)
    blocks = getattr(base, "h", None)
    if blocks is None:
        return None
    attns = [getattr(b, "attn", None) for b in blocks]
    if not attns or any(a is None or not hasattr(a, "c_attn") for a in attns):
        return None
    return attns


class QkvEpilogue:
    """Per-layer transposed QKV weights and the hook that routes `c_attn` to
    `pkv_qkv_append`. `make(model, pool)` returns None when the model or pool does not
    qualify (not GPT-2-shaped, not fp16/bf16, or a layout the kernel refuses)."""

    def __init__(self, attns, pool) -> None:
        self.attns = attns
        self.pool = pool
        cfg0 = attns[0]
        self.heads = int(cfg0.num_heads)
        self.head_dim = int(cfg0.head_dim)
        self.hidden = self.heads * self.head_dim
        self.weights_t = [a.c_attn.weight.detach().t().contiguous() for a in attns]
        self.biases = [a.c_attn.bias.detach().contiguous() if a.c_attn.bias is not None else None for a in attns]
        self.dtype = self.weights_t[0].dtype
        self.ctx = None

    @classmethod
    def make(cls, model, pool) -> "QkvEpilogue | None":
        attns = _attention_blocks(model)
        if attns is None:
            return None
        for a in attns:
            c = a.c_attn
            w = getattr(c, "weight", None)
            if type(c).__name__ != "Conv1D" or w is None or w.dim() != 2 or w.dtype not in _DTYPES:
                return None
            if getattr(a, "is_cross_attention", False) or not hasattr(a, "layer_idx"):
                return None
            hidden = int(a.num_heads) * int(a.head_dim)
            if w.shape != (hidden, 3 * hidden) or w.device.type != "cuda" or hidden % 16:
                return None
        dims = pool.dims
        if pool.k[0].dtype != attns[0].c_attn.weight.dtype or dims.num_kv_heads != int(attns[0].num_heads):
            return None
        if dims.head_dim != int(attns[0].head_dim) or len(pool.k) != len(attns):
            return None
        return cls(attns, pool)

    @contextlib.contextmanager
    def installed(self, ctx):
        """Route every layer's `c_attn` through the kernel for one forward over `ctx`
        (the step context: write_slots holds each row's flat pool slot)."""
        self.ctx = ctx
        for a in self.attns:
            a.c_attn.forward = self._hook(a)
        try:
            yield
        finally:
            for a in self.attns:
                del a.c_attn.forward
            self.ctx = None

    def _hook(self, attn):
        layer = int(attn.layer_idx)

        def forward(hidden_states: torch.Tensor) -> torch.Tensor:
            return self.project(layer, hidden_states, self.ctx.write_slots)

        return forward

    def project(self, layer: int, hidden_states: torch.Tensor, slots: torch.Tensor) -> torch.Tensor:
        """[..., hidden] -> [..., 3 * hidden]; K and V also go to pool slot slots[row]."""
        lead = hidden_states.shape[:-1]
        x = hidden_states.reshape(-1, self.hidden)
        if x.stride(-1) != 1:
            x = x.contiguous()
        rows = x.shape[0]
        out = torch.empty(rows, 3 * self.hidden, dtype=x.dtype, device=x.device)
        wt, b = self.weights_t[layer], self.biases[layer]
        kp, vp = self.pool.k[layer], self.pool.v[layer]
        rc = native.lib().pkv_qkv_append(
            x.data_ptr(), x.stride(0), wt.data_ptr(), wt.stride(0), b.data_ptr() if b is not None else None,
            rows, self.hidden, self.hidden, kp.shape[2], kp.shape[3],
            out.data_ptr(), out.stride(0),
            kp.data_ptr(), vp.data_ptr(), kp.stride(0), kp.stride(1), kp.stride(2),
            kp.shape[0], kp.shape[1], slots.data_ptr(), native.dtype_code(x.dtype),
            native.stream_handle(x.device),
        )
        native.check(rc, "pkv_qkv_append")
        return out.view(*lead, 3 * self.hidden)
