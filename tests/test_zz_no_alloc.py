"""pkv_paged_attention_decode_noalloc: decode attention whose split-KV partials live in
the library's static device scratch instead of a caller workspace (for callers that
cannot allocate). Called through the C ABI and compared bit for bit with
pkv_paged_attention_decode on the same inputs (same kernels, same partitions), on two
calls in a row where the second is smaller (the scratch keeps the first call's
partials; the second must read only its own), plus the oracle on one case, and the
refusal of a batch larger than the scratch.
"""

from __future__ import annotations

import re
from pathlib import Path

import pytest
import torch

from inference_server import native

HEADER = Path(__file__).resolve().parents[1] / "include" / "pagedkv.h"


def test_scratch_size_matches_the_header():
    m = re.search(r"#define PKV_DECODE_SCRATCH_BYTES \((\d+)ll \* 1024 \* 1024\)", HEADER.read_text())
    assert m and int(m.group(1)) * 1024 * 1024 == native.DECODE_SCRATCH_BYTES


def _case(n_seqs, n_kv, group, d, max_ctx, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    bs = 16
    ctx = torch.randint(1, max_ctx + 1, (n_seqs,), generator=g)
    ctx[0] = max_ctx
    width = -(-max_ctx // bs)
    n_blocks = n_seqs * width + 5
    tables = torch.randperm(n_blocks, generator=g)[: n_seqs * width].view(n_seqs, width).clone()
    k = torch.randn(n_blocks, bs, n_kv, d, generator=g).to(dtype)
    v = torch.randn(n_blocks, bs, n_kv, d, generator=g).to(dtype)
    q = torch.randn(n_seqs, n_kv * group, d, generator=g).to(dtype)
    return q, k, v, tables, ctx


def _args(out, q, k, v, tables, ctx, max_ctx):
    return (out.data_ptr(), out.stride(0), out.stride(1), q.data_ptr(), q.stride(0), q.stride(1),
            k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
            k.shape[0], k.shape[1], k.shape[2], k.shape[3],
            tables.data_ptr(), tables.stride(0), tables.shape[1], ctx.data_ptr(),
            q.shape[0], q.shape[1], max_ctx, q.shape[2] ** -0.5, native.dtype_code(q.dtype))


def _both(case, max_ctx):
    L = native.lib()
    q, k, v, tables, ctx = (t.cuda() for t in case)
    stream = native.stream_handle(q.device)
    ws_bytes = L.pkv_paged_attention_decode_workspace_bytes(q.shape[0], q.shape[1], k.shape[2], k.shape[3], max_ctx)
    assert 0 < ws_bytes <= native.DECODE_SCRATCH_BYTES
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device="cuda")  # zero-filled before first use
    ref = torch.empty_like(q)
    got = torch.full_like(q, float("nan"))
    native.check(L.pkv_paged_attention_decode(*_args(ref, q, k, v, tables, ctx, max_ctx), ws.data_ptr(), ws_bytes,
                                              stream), "pkv_paged_attention_decode")
    native.check(L.pkv_paged_attention_decode_noalloc(*_args(got, q, k, v, tables, ctx, max_ctx), stream),
                 "pkv_paged_attention_decode_noalloc")
    torch.cuda.synchronize()
    return ref, got


@pytest.mark.gpu
def test_noalloc_decode_matches_the_workspace_entry_point_on_two_calls_in_a_row():
    from oracle.gather import paged_attention_gather

    big = _case(96, 8, 4, 128, 6000, torch.bfloat16, seed=41)      # 24 partitions of 256
    small = _case(7, 12, 1, 64, 1500, torch.float16, seed=42)      # fewer, other shape
    for case, max_ctx in ((big, 6000), (small, 1500)):
        ref, got = _both(case, max_ctx)
        assert torch.equal(ref, got)
    q, k, v, tables, ctx = small
    want = paged_attention_gather(q, k, v, tables, ctx, torch.ones_like(ctx), q.shape[-1] ** -0.5)
    torch.testing.assert_close(got.cpu(), want, atol=2e-2, rtol=2e-2)


@pytest.mark.gpu
def test_noalloc_decode_refuses_a_batch_beyond_the_scratch():
    L = native.lib()
    q, k, v, tables, ctx = (t.cuda() for t in _case(4, 2, 4, 128, 64, torch.bfloat16, seed=43))
    out = torch.zeros_like(q)
    # Claim 600 sequences x 64 heads x 8192 tokens: 32 partitions of partials each,
    # far beyond the scratch; refused on the host before any launch.
    args = list(_args(out, q, k, v, tables, ctx, 8192))
    args[19], args[20] = 600, 64                       # num_seqs, num_heads
    args[17] = 8192 // 16                              # table_width
    rc = L.pkv_paged_attention_decode_noalloc(*args, native.stream_handle(q.device))
    assert rc == native.PKV_EWORKSPACE
    assert b"static scratch" in L.pkv_last_error()
    torch.cuda.synchronize()
    assert not out.any()
