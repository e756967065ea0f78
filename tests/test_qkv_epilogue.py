"""QKV projection with the KV append in its epilogue (`pkv_qkv_append`, core/qkv_epilogue.py).

GPU (`-m gpu`). The projection is a floating-point GEMM, so it is checked against a
plain torch fp32 reference of the same op (x.float() @ W.float() + b.float()): every
element within half an ulp of the model dtype plus the fp32 summation-order bound of a
K-term dot product (2K eps32 |x| @ |W|; near-zero sums cancel, so a plain ulp count is
the wrong measure), and at least 99% equal to the reference rounded, bit for bit. The
epilogue's scatter is byte work and is checked bit for bit: the pool after the call must equal oracle.kvops.kv_append applied
to the pool before it with the kernel's own K and V columns, slots outside the pool
skipped. The host module is checked on GPT-2's own `c_attn` (Conv1D) weights against
the module's forward.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from inference_server import native

pytestmark = pytest.mark.gpu


def _bound_scale(dtype) -> float:
    return {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}[dtype]


def _check_close(out: torch.Tensor, x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None):
    """out against the fp32 reference x @ w + b: within half an ulp of the model dtype at
    out's magnitude (the one rounding) plus the fp32 summation-order error of a length-K
    dot product, bounded by 2K eps32 |x| @ |w| (a K-term sum reordered). At least 99% of
    the elements are the fp32 reference rounded, bit for bit."""
    xf, wf = x.float(), w.float()
    ref = xf @ wf + (b.float() if b is not None else 0.0)
    mag = xf.abs() @ wf.abs() + (b.float().abs() if b is not None else 0.0)
    eps = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}[out.dtype]
    bound = out.float().abs() * eps + 2 * x.shape[-1] * 2.0 ** -24 * mag + 1e-30
    err = (out.float() - ref).abs()
    assert bool((err <= bound).all()), f"worst excess {float((err / bound).max()):.3g}x the bound"
    assert float((out == ref.to(out.dtype)).float().mean()) >= 0.99


def _raw(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


def _call(x, wt, b, q_features, kv_heads, head_dim, kp, vp, slots):
    rows = x.shape[0]
    n = q_features + 2 * kv_heads * head_dim
    out = torch.empty(rows, n, dtype=x.dtype, device=x.device)
    rc = native.lib().pkv_qkv_append(
        x.data_ptr(), x.stride(0), wt.data_ptr(), wt.stride(0), b.data_ptr() if b is not None else None,
        rows, x.shape[1], q_features, kv_heads, head_dim, out.data_ptr(), out.stride(0),
        kp.data_ptr(), vp.data_ptr(), kp.stride(0), kp.stride(1), kp.stride(2), kp.shape[0], kp.shape[1],
        slots.data_ptr(), native.dtype_code(x.dtype), native.stream_handle(x.device))
    native.check(rc, "pkv_qkv_append")
    torch.cuda.synchronize()
    return out


SHAPES = [
    # (rows, in_features, q_features, kv_heads, head_dim)
    (1, 768, 768, 12, 64),      # GPT-2, one sequence
    (32, 768, 768, 12, 64),     # GPT-2, config 5's decode batch
    (33, 768, 768, 12, 64),     # a second row group
    (64, 256, 512, 2, 64),      # Q wider than K/V (GQA-shaped)
    (7, 1024, 1024, 8, 128),    # head_dim 128
    (20, 272, 256, 4, 32),      # in_features a multiple of 16 but not 32: 32-column tiles
    (100, 768, 768, 12, 64),    # beyond 64 rows: several row-tile passes
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,in_f,q_f,kvh,d", SHAPES)
def test_qkv_append_matches_fp32_reference_and_scatters_k_v(dtype, rows, in_f, q_f, kvh, d):
    from oracle.kvops import kv_append

    g = torch.Generator().manual_seed(rows * 131 + in_f + d)
    n = q_f + 2 * kvh * d
    x = torch.randn(rows, in_f, generator=g).to(dtype).cuda()
    w = (torch.randn(in_f, n, generator=g) / in_f ** 0.5).to(dtype).cuda()
    b = (torch.randn(n, generator=g) * 0.1).to(dtype).cuda()
    num_blocks, bs = 3 * rows + 5, 16
    kp = torch.randn(num_blocks, bs, kvh, d, generator=g).to(dtype).cuda()
    vp = torch.randn(num_blocks, bs, kvh, d, generator=g).to(dtype).cuda()
    slots = torch.randperm(num_blocks * bs, generator=g)[:rows].cuda()
    k_before, v_before = _raw(kp), _raw(vp)

    out = _call(x, w.t().contiguous(), b, q_f, kvh, d, kp, vp, slots)

    _check_close(out, x, w, b)
    k_new = out[:, q_f:q_f + kvh * d].reshape(rows, kvh, d)
    v_new = out[:, q_f + kvh * d:].reshape(rows, kvh, d)
    s = slots.cpu().numpy()
    assert (_raw(kp) == kv_append(k_before, _raw(k_new), s)).all()
    assert (_raw(vp) == kv_append(v_before, _raw(v_new), s)).all()


def test_qkv_append_skips_slots_outside_the_pool_and_takes_no_bias():
    dtype = torch.float16
    g = torch.Generator().manual_seed(3)
    rows, in_f, q_f, kvh, d = 5, 256, 256, 4, 64
    n = q_f + 2 * kvh * d
    x = torch.randn(rows, in_f, generator=g).to(dtype).cuda()
    w = (torch.randn(in_f, n, generator=g) / 16).to(dtype).cuda()
    kp = torch.randn(8, 16, kvh, d, generator=g).to(dtype).cuda()
    vp = torch.randn(8, 16, kvh, d, generator=g).to(dtype).cuda()
    slots = torch.tensor([3, -1, 127, 128, 40]).cuda()       # -1 and 128 (= 8 * 16) are outside
    k_before, v_before = kp.clone(), vp.clone()
    out = _call(x, w.t().contiguous(), None, q_f, kvh, d, kp, vp, slots)
    _check_close(out, x, w, None)
    flat_k, flat_v = kp.view(-1, kvh, d), vp.view(-1, kvh, d)
    for r, sl in enumerate(slots.tolist()):
        if 0 <= sl < 128:
            assert torch.equal(flat_k[sl], out[r, q_f:q_f + kvh * d].view(kvh, d))
            assert torch.equal(flat_v[sl], out[r, q_f + kvh * d:].view(kvh, d))
    written = {3, 127, 40}
    keep = [i for i in range(128) if i not in written]
    assert torch.equal(flat_k[keep], k_before.view(-1, kvh, d)[keep])
    assert torch.equal(flat_v[keep], v_before.view(-1, kvh, d)[keep])


def test_qkv_append_refuses_fp32_and_misaligned_rows():
    x = torch.randn(2, 64, device="cuda")
    wt = torch.randn(192, 64, device="cuda")
    kp = torch.zeros(4, 16, 1, 64, device="cuda")
    slots = torch.tensor([0, 1], device="cuda")
    out = torch.empty(2, 192, device="cuda")
    L = native.lib()
    rc = L.pkv_qkv_append(x.data_ptr(), 64, wt.data_ptr(), 64, None, 2, 64, 64, 1, 64, out.data_ptr(), 192,
                          kp.data_ptr(), kp.data_ptr(), 1024, 64, 64, 4, 16, slots.data_ptr(), native.PKV_FLOAT32,
                          native.stream_handle(x.device))
    assert rc == native.PKV_EUNSUPPORTED and b"fp16 and bf16" in L.pkv_last_error()
    xh = torch.randn(2, 72, device="cuda").half()
    rc = L.pkv_qkv_append(xh.data_ptr(), 72, wt.half().data_ptr(), 64, None, 2, 72, 64, 1, 64, out.data_ptr(), 192,
                          kp.half().data_ptr(), kp.half().data_ptr(), 1024, 64, 64, 4, 16, slots.data_ptr(),
                          native.PKV_FLOAT16, native.stream_handle(x.device))
    assert rc == native.PKV_EUNSUPPORTED


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_epilogue_module_matches_gpt2_c_attn(dtype):
    """QkvEpilogue.project on GPT-2's own layers against each layer's c_attn forward
    (HF's Conv1D: addmm(bias, x, W)), and the pool rows it wrote."""
    from inference_server.core.kv_pool import ModelDims, PagedKVPool
    from inference_server.core.qkv_epilogue import QkvEpilogue
    from inference_server.model import load

    model, _ = load(dtype=dtype, device="cuda")
    pool = PagedKVPool(ModelDims.from_model(model, dtype=dtype), num_blocks=64, block_size=16, device="cuda")
    qkv = QkvEpilogue.make(model, pool)
    assert qkv is not None
    g = torch.Generator().manual_seed(7)
    slots = torch.randperm(64 * 16, generator=g)[:24].cuda()
    for layer in (0, 5, 11):
        x = torch.randn(1, 24, 768, generator=g).to(dtype).cuda()
        attn = model.transformer.h[layer].attn
        with torch.no_grad():
            want = attn.c_attn(x)
            got = qkv.project(layer, x, slots)
        torch.cuda.synchronize()
        assert got.shape == want.shape == (1, 24, 2304)
        _check_close(got[0], x[0], attn.c_attn.weight, attn.c_attn.bias)
        # and against HF's own forward: both round one fp32 sum of the same terms
        diff = (got.float() - want.float()).abs()
        assert float(diff.max()) <= float((2 * _bound_scale(dtype)) * want.float().abs().max() + 1e-2)
        k = pool.k[layer].view(-1, 12, 64)[slots]
        v = pool.v[layer].view(-1, 12, 64)[slots]
        assert torch.equal(k, got[0, :, 768:1536].reshape(24, 12, 64))
        assert torch.equal(v, got[0, :, 1536:].reshape(24, 12, 64))
    del model, pool
    torch.cuda.empty_cache()


def test_engine_with_the_epilogue_gives_the_same_tokens_from_graphs_and_eager_steps(monkeypatch):
    """GPT-2 fp16, config 5's shape (24 requests, up to 40 tokens), QKV_EPILOGUE=1: decode
    steps replayed from HIP graphs and issued eagerly both project through
    pkv_qkv_append, and give identical token streams (the kernel is deterministic and
    the graph captures the same launches). Parity with the gather path at full size is
    tests/test_config5_parity.py's epilogue case."""
    from inference_server.bench import workload
    from inference_server.config import CONFIG
    from inference_server.engine.paged import PagedEngine
    from inference_server.model import load

    monkeypatch.setattr(CONFIG, "attention", "hip")
    monkeypatch.setattr(CONFIG, "qkv_epilogue", True)
    model, tok = load(dtype=torch.float16, device="cuda")
    reqs = workload.config5(n=24)
    for r in reqs:
        r.max_tokens = min(r.max_tokens, 40)
    outs = []
    for graphs in (True, False):
        monkeypatch.setattr(CONFIG, "decode_graphs", graphs)
        monkeypatch.setattr(CONFIG, "prefill_graphs", graphs)
        engine = PagedEngine(model, tok, num_blocks=1024, block_size=16, device="cuda")
        try:
            assert engine.executor.qkv is not None
            outs.append(engine.run(reqs))
        finally:
            engine.shutdown()
    assert outs[0].generated_tokens == sum(r.max_tokens for r in reqs)
    assert outs[0].outputs == outs[1].outputs
