"""Greedy sampling fused into the LM head.

CPU: the oracle (oracle/greedy.py) pinned against brute force, torch's own bf16
rounding and argmax's first-maximum rule, and the host contract checks. GPU
(`-m gpu`): `pkv_lm_head_argmax` through the C ABI against the oracle on seeded
inputs, planted ties, a tie that only exists after rounding to fp16, graph replays,
and the executor's fused path against the reference's logits + argmax.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from inference_server import native
from inference_server.core.sampling import fused_greedy_supported, fused_max_rows, lm_head_argmax, lm_head_weight
from oracle import greedy

NP_DTYPE = {torch.float16: "float16", torch.bfloat16: "bfloat16"}


# ------------------------------------------------------------------ oracle pins (CPU)
def test_oracle_one_hot_hidden_picks_the_column_maximum():
    rng = np.random.default_rng(0)
    w = rng.standard_normal((300, 16)).astype(np.float32)
    for k in range(16):
        h = np.zeros((1, 16), np.float32)
        h[0, k] = 1.0
        col = [float(v) for v in greedy.round_to(w[:, k], "float16")]
        best = 0
        for v in range(1, len(col)):  # brute force: first maximum
            if col[v] > col[best]:
                best = v
        assert greedy.greedy_ids(h, w, "float16")[0] == best


def test_oracle_ties_go_to_the_lowest_index():
    w = np.zeros((10, 4), np.float32)
    w[:, 0] = np.linspace(-1, 0.5, 10)
    w[3, 0] = w[7, 0] = 2.0
    assert greedy.greedy_ids(np.array([[1, 0, 0, 0]], np.float32), w, "float32")[0] == 3


def test_oracle_ranks_rounded_logits():
    """Exact logits 1.0 (index 2) and 1 + 2^-13 (index 9) both round to fp16 1.0, so the
    reference's fp16 logits tie and argmax returns 2; ranked in fp32 it would be 9."""
    w = np.zeros((12, 2), np.float32)
    w[:, 0] = 0.5
    w[2] = [1.0, 0.0]
    w[9] = [1.0, 2.0 ** -6]
    h = np.array([[1.0, 2.0 ** -7]], np.float32)
    assert greedy.greedy_ids(h, w, "float16")[0] == 2
    assert greedy.greedy_ids(h, w, "float32")[0] == 9


def test_oracle_bf16_rounding_is_torchs():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(20000).astype(np.float32) * 100
    # exact halfway cases (ties to even both ways) and the neighbours of 1.0
    x[:4] = [1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, -(1 + 2.0 ** -8), 1 + 2.0 ** -9]
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(greedy.round_to(x, "bfloat16"), want)


# ------------------------------------------------------------------ host contract (CPU)
def test_contract_errors_come_before_any_gpu_work():
    h = torch.zeros(2, 16, dtype=torch.float16)
    with pytest.raises(ValueError, match="hidden size"):
        lm_head_argmax(h, torch.zeros(5, 32, dtype=torch.float16))
    with pytest.raises(ValueError, match="float16"):
        lm_head_argmax(h, torch.zeros(5, 16, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="rows"):
        lm_head_argmax(h[0], torch.zeros(5, 16, dtype=torch.float16))
    with pytest.raises(NotImplementedError, match="ROCm GPU"):
        lm_head_argmax(h, torch.zeros(5, 16, dtype=torch.float16))


def test_supported_only_for_a_gpu_half_precision_head():
    head = torch.nn.Linear(16, 40, bias=False).half()
    assert lm_head_weight(type("M", (), {"get_output_embeddings": lambda self: head})()) is head.weight
    assert not fused_greedy_supported(head.weight)          # on the CPU
    assert not fused_greedy_supported(None)
    with_bias = torch.nn.Linear(16, 40)
    assert lm_head_weight(type("M", (), {"get_output_embeddings": lambda self: with_bias})()) is None


def test_workspace_size_is_host_arithmetic():
    L = native.load_library()
    # the arrival counter's 256 bytes, then 8 copies of one 64-bit key per row (rows
    # rounded up to 16), rounded up to 256 bytes; the vocabulary size does not matter
    assert L.pkv_lm_head_argmax_workspace_bytes(128, 50257) == 256 + 8 * 128 * 8
    assert L.pkv_lm_head_argmax_workspace_bytes(3, 1) == 256 + 8 * 16 * 8
    assert L.pkv_lm_head_argmax_workspace_bytes(17, 900) == 256 + 8 * 32 * 8
    assert L.pkv_lm_head_argmax_workspace_bytes(0, 50257) == 0


# ------------------------------------------------------------------ GPU parity
def _problem(rows, dim, vocab, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(rows, dim, generator=g)
    w = torch.randn(vocab, dim, generator=g) / dim ** 0.5 * 4
    return h.to(dtype), w.to(dtype)


def _check(ids, h, w, dtype):
    """Every id's logit is within one rounding step of the row maximum (the kernel and
    the oracle sum in different orders, so a rounded logit may differ by one ulp), and
    ids are exact wherever the oracle's top two logits are more than 2 ulps apart."""
    hn, wn = h.float().numpy(), w.float().numpy()
    lg = greedy.logits(hn, wn, NP_DTYPE[dtype])
    want = greedy.greedy_ids(hn, wn, NP_DTYPE[dtype])
    got = ids.cpu().numpy()
    rows = np.arange(len(got))
    top = lg[rows, want]
    ulp = np.abs(top) * (2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7) + 1e-6
    assert np.all(lg[rows, got] >= top - 2 * ulp), np.nonzero(lg[rows, got] < top - 2 * ulp)
    second = np.sort(lg, axis=1)[:, -2] if lg.shape[1] > 1 else np.full(len(got), -np.inf)
    clear = top - second > 2 * ulp
    np.testing.assert_array_equal(got[clear], want[clear])
    return clear.mean()


def test_fused_rows_stop_where_one_streaming_pass_ends():
    """The executor sends a batch through the fused kernel only while its streaming
    kernel covers the rows in one pass over the weight (16-row column tiles, at most 4,
    within a 150 KiB LDS budget of hidden rows); beyond, the GEMM + argmax is faster."""
    assert fused_max_rows(768) == 64           # GPT-2: 4 tiles of 16 rows
    assert fused_max_rows(1200) == 64 and fused_max_rows(1280) == 32
    assert fused_max_rows(2400) == 32 and fused_max_rows(2560) == 16
    assert fused_max_rows(4096) == 16          # Llama-sized hidden rows: one tile
    assert fused_max_rows(5120) == 0 and fused_max_rows(8192) == 0


CASES = [
    (torch.float16, 1, 768, 50257), (torch.float16, 32, 768, 50257), (torch.float16, 33, 768, 1000),
    (torch.bfloat16, 64, 768, 50257), (torch.bfloat16, 65, 128, 33), (torch.float16, 128, 768, 50257),
    (torch.float16, 200, 64, 4096), (torch.bfloat16, 300, 4096, 3000), (torch.float16, 5, 16, 31),
    (torch.bfloat16, 7, 144, 1), (torch.float16, 129, 32, 50257),
    # weight-streaming kernel: more than 256 workgroups (vocab > 65536), a 12-chunk ring
    (torch.float16, 24, 256, 70001), (torch.float16, 40, 1536, 5000), (torch.bfloat16, 16, 768, 17),
    # Llama-sized hidden rows: one 16-row pass of the streaming kernel; 33 rows, which would
    # take several passes, go to the tile kernel
    (torch.float16, 16, 4096, 5000), (torch.bfloat16, 33, 4096, 32000),
]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,rows,dim,vocab", CASES)
def test_fused_argmax_matches_oracle(dtype, rows, dim, vocab):
    h, w = _problem(rows, dim, vocab, dtype, seed=rows * 7 + dim)
    ids = lm_head_argmax(h.cuda(), w.cuda())
    torch.cuda.synchronize()
    assert ids.dtype == torch.int64 and ids.shape == (rows,)
    # Share of rows whose top two oracle logits are more than 2 ulps apart (checked
    # exactly): bf16's ulp is 8x fp16's, so near-ties are common over 50257 entries;
    # with a handful of rows one near-tie moves the share by a lot.
    clear = _check(ids, h, w, dtype)
    # Measured shares for these seeds: fp16 >= 0.95, bf16 0.80-0.95.
    assert rows < 16 or clear > (0.9 if dtype == torch.float16 else 0.75)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_argmax_strided_rows_and_empty(dtype):
    h, w = _problem(40, 256, 5000, dtype, seed=3)
    wide = torch.zeros(40, 512, dtype=dtype)
    wide[:, :256] = h
    ids = lm_head_argmax(wide.cuda()[:, :256], w.cuda())
    _check(ids, h, w, dtype)
    assert lm_head_argmax(h.cuda()[:0], w.cuda()).shape == (0,)
    # one row broadcast to every sampled row (row stride 0) is copied before the call
    one = h[:1].cuda().expand(6, 256)
    assert lm_head_argmax(one, w.cuda()).tolist() == [int(lm_head_argmax(h[:1].cuda(), w.cuda()))] * 6


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_argmax_ties_go_to_the_lowest_index(dtype):
    """Each row's winner copied to half its index (another vocabulary tile, usually
    another workgroup): identical weight rows give identical logits, and the lower
    index must win, as torch's argmax returns the first maximum."""
    h, w = _problem(96, 768, 50257, dtype, seed=11)
    want = greedy.greedy_ids(h.float().numpy(), w.float().numpy(), NP_DTYPE[dtype])
    w2 = w.clone()
    for v in want.tolist():
        w2[v // 2] = w[v]
    w2[-1] = w[int(want[0])]  # and one copy at the very end (a higher index)
    ids = lm_head_argmax(h.cuda(), w2.cuda()).cpu().numpy()
    lg = greedy.logits(h.float().numpy(), w2.float().numpy(), NP_DTYPE[dtype])
    first = np.argmax(lg, axis=1)
    checked = 0
    for r in range(len(ids)):
        top = lg[r, first[r]]
        below = lg[r][lg[r] < top]
        ulp = abs(top) * (2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7)
        if (lg[r] == top).sum() >= 2 and (below.size == 0 or top - below.max() > 2 * ulp):
            assert ids[r] == first[r], (r, ids[r], first[r])
            checked += 1
    assert checked >= 48


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("first_sign,second_sign", [(1.0, -1.0), (-1.0, 1.0), (-1.0, -1.0)])
def test_fused_argmax_nan_of_either_sign_wins_at_its_first_index(dtype, first_sign, second_sign):
    """A NaN logit outranks every number and the first NaN wins, whatever the sign bit
    of the NaN (torch's argmax treats NaN as the maximum and returns its first index).
    Weight rows 3 and 9 of a 64-entry vocabulary are NaN with the given signs; hidden
    rows of both signs also flip the sign of the products."""
    h, w = _problem(6, 32, 64, dtype, seed=21)
    w[3] = first_sign * float("nan")
    w[9] = second_sign * float("nan")
    h[1] = -h[1]
    ids = lm_head_argmax(h.cuda(), w.cuda()).tolist()
    assert ids == [3] * 6
    assert (h.float() @ w.float().T).argmax(-1).tolist() == [3] * 6
    want = greedy.greedy_ids(h.float().numpy(), w.float().numpy(), NP_DTYPE[dtype])
    assert want.tolist() == [3] * 6


@pytest.mark.gpu
def test_fused_argmax_ranks_the_fp16_rounded_logits():
    """1.0 (index 2) and 1 + 2^-13 (index 9) are both 1.0 in fp16: the tie goes to 2,
    as the reference's fp16 logits + argmax give."""
    w = torch.zeros(40, 16, dtype=torch.float16)
    w[:, 0] = 0.5
    w[2, 0] = 1.0
    w[9, 0], w[9, 1] = 1.0, 2.0 ** -6
    h = torch.zeros(3, 16, dtype=torch.float16)
    h[:, 0], h[:, 1] = 1.0, 2.0 ** -7
    assert lm_head_argmax(h.cuda(), w.cuda()).tolist() == [2, 2, 2]
    ref = (h.cuda() @ w.cuda().T).argmax(-1)
    assert ref.tolist() == [2, 2, 2]


@pytest.mark.gpu
def test_fused_argmax_rejects_a_short_workspace_and_fp32():
    h, w = _problem(4, 64, 100, torch.float16, seed=5)
    h, w = h.cuda(), w.cuda()
    L = native.lib()
    ids = torch.empty(4, dtype=torch.long, device="cuda")
    ws = torch.empty(64, dtype=torch.uint8, device="cuda")
    rc = L.pkv_lm_head_argmax(h.data_ptr(), 64, w.data_ptr(), 64, 4, 64, 100, native.PKV_FLOAT16,
                              ids.data_ptr(), ws.data_ptr(), 64, native.stream_handle(h.device))
    assert rc == native.PKV_EWORKSPACE and b"workspace" in L.pkv_last_error()
    with pytest.raises(NotImplementedError, match="fp16 and bf16"):
        lm_head_argmax(h.float(), w.float())


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,rows,dim,vocab", [(torch.float16, 32, 768, 50257), (torch.bfloat16, 64, 768, 50257),
                                                  (torch.float16, 3, 256, 70001), (torch.float16, 5, 64, 900)])
def test_fused_argmax_calls_in_a_row_on_one_workspace(dtype, rows, dim, vocab):
    """Through the C-ABI on one workspace, zero-filled once: calls in a row (different
    hidden rows, then fewer of them, then more) each match the oracle, and each leaves
    the workspace (the in-launch merge's arrival counter and keys) all zero again."""
    _, w = _problem(rows, dim, vocab, dtype, seed=rows)
    wd = w.cuda()
    L = native.lib()
    nbytes = L.pkv_lm_head_argmax_workspace_bytes(rows, vocab)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    stream = native.stream_handle(wd.device)
    for i, n in enumerate((rows, rows, max(1, rows // 2), rows)):
        h, _ = _problem(n, dim, 1, dtype, seed=100 + i)
        hd = h.cuda()
        ids = torch.full((n,), -7, dtype=torch.long, device="cuda")
        rc = L.pkv_lm_head_argmax(hd.data_ptr(), dim, wd.data_ptr(), dim, n, dim, vocab, native.dtype_code(dtype),
                                  ids.data_ptr(), ws.data_ptr(), nbytes, stream)
        assert rc == 0, L.pkv_last_error()
        torch.cuda.synchronize()
        _check(ids, h, w, dtype)
        assert int(ws.count_nonzero()) == 0, f"call {i} left merge state in the workspace"


@pytest.mark.gpu
def test_fused_argmax_replays_in_a_graph():
    """The call captured once: one kernel node and nothing else (no memset, no second
    launch), replayed one to three times in a row between eager calls, each replay's ids
    equal to the eager call's and the oracle's (the in-launch merge leaves its workspace
    zero for the next replay)."""
    from inference_server.core.decode_graphs import node_census

    dtype = torch.float16
    h, w = _problem(48, 768, 50257, dtype, seed=9)
    hd, wd = h.cuda(), w.cuda()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        lm_head_argmax(hd, wd)  # warm-up outside the capture: the stream's workspace
        graph = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(graph, stream=s):
            out = lm_head_argmax(hd, wd)
    torch.cuda.current_stream().wait_stream(s)
    assert node_census(graph) == {"kernel": 1}
    graph.instantiate()
    for reps, seed in ((1, 21), (2, 22), (3, 23)):
        h2, _ = _problem(48, 768, 1, dtype, seed=seed)
        hd.copy_(h2.cuda())
        for _ in range(reps):
            graph.replay()
        torch.cuda.synchronize()
        eager = lm_head_argmax(hd, wd)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        _check(out, h2, w, dtype)


@pytest.mark.gpu
def test_fused_argmax_on_two_streams_at_once():
    """Calls in flight on two streams together each get their stream's own zero-filled
    workspace (the in-launch merge's state is per workspace): both streams' ids match the
    oracle on every round, and each stream's workspace reads zero afterwards."""
    from inference_server.core import sampling

    dtype = torch.float16
    _, w = _problem(1, 768, 50257, dtype, seed=31)
    wd = w.cuda()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rnd in range(3):
        hs = [_problem(n, 768, 1, dtype, seed=40 + 2 * rnd + i)[0] for i, n in enumerate((32, 7))]
        hds = [h.cuda() for h in hs]
        torch.cuda.synchronize()
        outs = []
        for st, hd in zip(streams, hds):
            with torch.cuda.stream(st):
                outs.append(lm_head_argmax(hd, wd))
        torch.cuda.synchronize()
        for out, h in zip(outs, hs):
            _check(out, h, w, dtype)
    bufs = [sampling._WORKSPACES.get(wd.device, st.cuda_stream, 1) for st in streams]
    assert bufs[0].data_ptr() != bufs[1].data_ptr()
    assert all(int(b.count_nonzero()) == 0 for b in bufs)


# ------------------------------------------------------------------ executor (GPU)
def _config5_run(monkeypatch, fused):
    from inference_server.bench import workload
    from inference_server.config import CONFIG
    from inference_server.engine.paged import PagedEngine
    from inference_server.model import load

    monkeypatch.setattr(CONFIG, "attention", "hip")
    monkeypatch.setattr(CONFIG, "fused_greedy", fused)
    reqs = workload.config5(n=24)
    for r in reqs:
        r.max_tokens = min(r.max_tokens, 40)
    model, tok = load(dtype=torch.float16, device="cuda")
    engine = PagedEngine(model, tok, num_blocks=1024, block_size=16, device="cuda")
    try:
        assert (engine.executor.fused_head is not None) == fused
        return engine.run(reqs), reqs
    finally:
        engine.shutdown()


@pytest.mark.gpu
def test_executor_fused_greedy_matches_logits_argmax(monkeypatch):
    """GPT-2 fp16 (BASELINE config 5's shape, 24 requests) on ATTENTION=hip, decode and
    prefill step graphs on: greedy ids fused into the LM head vs the reference's
    logits + argmax over the same model. Both rank fp16-rounded logits, so streams only
    part where a rounded logit lands one ulp apart at a near-tie; at least 90% of the
    streams are identical and every request completes."""
    fused, reqs = _config5_run(monkeypatch, True)
    plain, _ = _config5_run(monkeypatch, False)
    assert fused.generated_tokens == plain.generated_tokens == sum(r.max_tokens for r in reqs)
    same = sum(fused.outputs[r.request_id] == plain.outputs[r.request_id] for r in reqs)
    assert same >= 0.9 * len(reqs), same
