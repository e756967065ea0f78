"""The product's attention surface on the CPU: the gather backend against the
textbook oracle (the reference's tests/test_paged_attention.py, case for case), the
contract errors with the reference's texts, dispatcher semantics, signature parity,
and the hip backend failing loudly where it cannot run."""

from __future__ import annotations

import inspect

import numpy as np
import pytest
import torch

from cases import CASES, build, dense_causal_f64
from inference_server.config import CONFIG
from inference_server.core import attention
from inference_server.core.attention import (paged_attention, paged_attention_gather, paged_attention_hip,
                                             paged_attention_triton)
from oracle.gather import paged_attention_gather as oracle_gather


@pytest.mark.parametrize("case", list(CASES))
def test_gather_backend_matches_dense(case):
    q, kp, vp, tables, ctx, ql = build(CASES[case])
    scale = q.shape[-1] ** -0.5
    out = paged_attention_gather(q, kp, vp, tables, ctx, ql, scale)
    np.testing.assert_allclose(out.double().numpy(), dense_causal_f64(q, kp, vp, tables, ctx, ql, scale),
                               atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_gather_backend_is_the_oracle_bit_for_bit(dtype):
    """Same op sequence as the oracle restatement, so identical bits on the CPU."""
    for lengths in (CASES["mixed"], CASES["decode_ragged"]):
        q, kp, vp, tables, ctx, ql = build(lengths, bs=16, d=64, dtype=dtype)
        a = paged_attention_gather(q, kp, vp, tables, ctx, ql, 0.125)
        assert torch.equal(a, oracle_gather(q, kp, vp, tables, ctx, ql, 0.125))


def test_grouped_query_heads_are_expanded():
    q, kp, vp, tables, ctx, ql = build([(9, 9), (5, 1)], kv_heads=1)
    out = paged_attention_gather(q, kp, vp, tables, ctx, ql, 8 ** -0.5)
    np.testing.assert_allclose(out.double().numpy(), dense_causal_f64(q, kp, vp, tables, ctx, ql, 8 ** -0.5),
                               atol=1e-5, rtol=1e-5)


def test_empty_batch_returns_empty():
    q = torch.empty(0, 3, 8)
    pool = torch.zeros(4, 4, 3, 8)
    out = paged_attention_gather(q, pool, pool, torch.zeros(0, 1, dtype=torch.long),
                                 torch.zeros(0, dtype=torch.long), torch.zeros(0, dtype=torch.long), 0.5)
    assert out.shape == (0, 3, 8)


def test_query_must_be_counted_in_context():
    q, kp, vp, tables, ctx, ql = build([(4, 4)])
    with pytest.raises(ValueError, match="query_len exceeds context_len"):
        paged_attention_gather(q, kp, vp, tables, ctx - 1, ql, 0.5)


def test_query_lens_must_sum_to_num_tokens():
    q, kp, vp, tables, ctx, ql = build([(4, 4), (2, 2)])
    with pytest.raises(ValueError, match="query_lens sum"):
        paged_attention_gather(q[:-1], kp, vp, tables, ctx, ql, 0.5)


def test_table_must_hold_the_context():
    q, kp, vp, tables, ctx, ql = build([(9, 1)])
    with pytest.raises(ValueError, match="more blocks than its block_tables row holds"):
        paged_attention_gather(q, kp, vp, tables[:, :2], ctx, ql, 0.5)


def test_shape_errors():
    q, kp, vp, tables, ctx, ql = build([(4, 4)])
    with pytest.raises(ValueError, match="query must be"):
        paged_attention_gather(q[0], kp, vp, tables, ctx, ql, 0.5)
    with pytest.raises(ValueError, match="k_pool must be"):
        paged_attention_gather(q, kp[0], vp, tables, ctx, ql, 0.5)
    with pytest.raises(ValueError, match="must be \\[batch\\]"):
        paged_attention_gather(q, kp, vp, tables, ctx[None], ql, 0.5)


def test_dispatcher(monkeypatch):
    q, kp, vp, tables, ctx, ql = build([(5, 5)])
    monkeypatch.setattr(CONFIG, "attention", "gather")
    ref = dense_causal_f64(q, kp, vp, tables, ctx, ql, 0.5)
    np.testing.assert_allclose(paged_attention(q, kp, vp, tables, ctx, ql, 0.5).double().numpy(), ref,
                               atol=1e-5, rtol=1e-5)
    monkeypatch.setattr(CONFIG, "attention", "triton")
    with pytest.raises(NotImplementedError, match="ATTENTION=triton"):
        paged_attention(q, kp, vp, tables, ctx, ql, 0.5)
    monkeypatch.setattr(CONFIG, "attention", "cuda-graphs")
    with pytest.raises(ValueError, match="ATTENTION"):
        paged_attention(q, kp, vp, tables, ctx, ql, 0.5)


def test_every_backend_shares_the_signature():
    sig = list(inspect.signature(paged_attention).parameters)
    for fn in (attention.paged_attention_gather, attention.paged_attention_triton, attention.paged_attention_hip):
        assert list(inspect.signature(fn).parameters) == sig


def test_hip_backend_fails_loudly_on_cpu_tensors(monkeypatch):
    """ATTENTION=hip never falls back to gather: CPU tensors raise, naming the reason."""
    q, kp, vp, tables, ctx, ql = build([(5, 5)])
    with pytest.raises(NotImplementedError, match="ATTENTION=hip"):
        paged_attention_hip(q, kp, vp, tables, ctx, ql, 0.5)
    monkeypatch.setattr(CONFIG, "attention", "hip")
    with pytest.raises(NotImplementedError, match="ATTENTION=hip"):
        paged_attention(q, kp, vp, tables, ctx, ql, 0.5)
    with pytest.raises(NotImplementedError, match="triton"):
        paged_attention_triton(q, kp, vp, tables, ctx, ql, 0.5)
