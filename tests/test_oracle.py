"""Pins the CPU oracle before anything is compared against it.

Each oracle function is checked against something it does not share code with:

* gather / online attention vs the textbook dense causal attention of the
  reference's own test (tests/test_paged_attention.py:30-37), recomputed in float64
  slot by slot, on every reference batch shape, GQA, bs16/d64 and bs6/d12;
* the token map vs the reference's known answer (test_paged_attention_triton.py:141-147);
* slot arithmetic vs the reference block-table examples (block_table.py:70-76, 137-159);
* append / copy / swap vs brute-force element loops and the reference's swap round
  trip (tests/test_swap.py:35-56, :60-69);
* everything vs the committed golden vectors (tests/golden/).

The last tests plant mistakes IN THE ORACLE (a dropped scale, a wrong GQA mapping, an
off-by-one causal bound, a transposed append) and show that the pins catch each.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from cases import CASES, build, dense_causal_f64
from oracle import gather, kvops, online

GOLDEN = Path(__file__).resolve().parent / "golden"


def _np(t):
    return t.detach().cpu().double().numpy()


@pytest.mark.parametrize("case", list(CASES))
def test_gather_matches_textbook_dense(case):
    q, kp, vp, tables, ctx, ql = build(CASES[case])
    scale = q.shape[-1] ** -0.5
    got = gather.paged_attention_gather(q, kp, vp, tables, ctx, ql, scale)
    np.testing.assert_allclose(_np(got), dense_causal_f64(q, kp, vp, tables, ctx, ql, scale), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("case", list(CASES))
def test_online_mirror_matches_textbook_dense(case):
    q, kp, vp, tables, ctx, ql = build(CASES[case])
    scale = q.shape[-1] ** -0.5
    got = online.paged_attention_online(q.numpy(), kp.numpy(), vp.numpy(), tables.numpy(), ctx.numpy(),
                                        ql.numpy(), scale)
    np.testing.assert_allclose(got, dense_causal_f64(q, kp, vp, tables, ctx, ql, scale), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize(
    "lengths,kw",
    [
        ([(9, 9), (5, 1), (12, 3)], dict(kv_heads=1)),
        ([(33, 1), (16, 16), (40, 9)], dict(bs=16, d=64)),
        ([(13, 13), (7, 1), (18, 4)], dict(bs=6, d=12)),
        ([(30, 1), (17, 5)], dict(bs=16, d=128, heads=8, kv_heads=2)),
    ],
)
def test_shapes_gqa_and_non_power_of_two(lengths, kw):
    q, kp, vp, tables, ctx, ql = build(lengths, **kw)
    scale = q.shape[-1] ** -0.5
    ref = dense_causal_f64(q, kp, vp, tables, ctx, ql, scale)
    np.testing.assert_allclose(_np(gather.paged_attention_gather(q, kp, vp, tables, ctx, ql, scale)), ref,
                               atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(
        online.paged_attention_online(q.numpy(), kp.numpy(), vp.numpy(), tables.numpy(), ctx.numpy(), ql.numpy(),
                                      scale), ref, atol=1e-5, rtol=1e-5)


def test_half_precision_gather_is_close_to_dense():
    """In fp16/bf16 the gather path rounds scores and probabilities to the pool
    dtype; it stays within the 2e-2 bar of the exact answer on its own inputs."""
    for dtype in (torch.float16, torch.bfloat16):
        q, kp, vp, tables, ctx, ql = build(CASES["mixed"], bs=16, d=64, dtype=dtype)
        got = gather.paged_attention_gather(q, kp, vp, tables, ctx, ql, 0.125)
        assert got.dtype == dtype
        np.testing.assert_allclose(_np(got), dense_causal_f64(q, kp, vp, tables, ctx, ql, 0.125), atol=2e-2,
                                   rtol=2e-2)


def test_padding_entries_do_not_matter():
    """Reference tests/test_paged_attention.py:139-145: a 0-padded table entry is
    never used — changing what block 0 holds changes no output of a sequence that
    does not own block 0."""
    for seed in range(3):
        q, kp, vp, tables, ctx, ql = build(CASES["padding_hits_block0"], seed=seed)
        owner = [i for i in range(3) if 0 in tables[i, : -(-int(ctx[i]) // 4)].tolist()]
        a = gather.paged_attention_gather(q, kp, vp, tables, ctx, ql, 0.3)
        kp2 = kp.clone()
        kp2[0] += 100.0
        b = gather.paged_attention_gather(q, kp2, vp, tables, ctx, ql, 0.3)
        tok = 0
        for i, n in enumerate(ql.tolist()):
            if i not in owner:
                assert torch.equal(a[tok:tok + n], b[tok:tok + n])
            tok += n


def test_empty_batch():
    q = torch.empty(0, 3, 8)
    pool = torch.zeros(4, 4, 3, 8)
    zero = torch.zeros(0, dtype=torch.long)
    assert gather.paged_attention_gather(q, pool, pool, torch.zeros(0, 1, dtype=torch.long), zero, zero,
                                         0.5).shape == (0, 3, 8)


def test_token_map_known_answer():
    """Reference tests/test_paged_attention_triton.py:141-147."""
    seq_idx, q_pos, cu = gather.token_map(torch.tensor([6, 10, 4]), torch.tensor([1, 3, 4]))
    assert seq_idx.tolist() == [0, 1, 1, 1, 2, 2, 2, 2]
    assert q_pos.tolist() == [5, 7, 8, 9, 0, 1, 2, 3]
    assert cu.tolist() == [0, 1, 4, 8]


def test_slot_arithmetic_known_answers():
    """blocks [7, 2], bs 4: positions 0..5 -> 28 29 30 31 8 9 (block_table.py:143-159);
    17 tokens need 2 blocks of 16 and 16 need exactly 1 (block_table.py:70-76)."""
    assert kvops.slots_for([7, 2], 4, 6).tolist() == [28, 29, 30, 31, 8, 9]
    assert kvops.slots_for([3], 16, 16).tolist() == list(range(48, 64))
    assert -(-17 // 16) == 2 and -(-16 // 16) == 1


def test_append_matches_brute_force():
    rng = np.random.default_rng(0)
    pool = rng.standard_normal((6, 4, 3, 5)).astype(np.float32)
    rows = rng.standard_normal((7, 3, 5)).astype(np.float32)
    slots = rng.permutation(24)[:7]
    got = kvops.kv_append(pool, rows, slots)
    want = pool.copy()
    for t, s in enumerate(slots):
        for h in range(3):
            for d in range(5):
                want[s // 4, s % 4, h, d] = rows[t, h, d]
    assert np.array_equal(got, want)
    assert np.array_equal(pool, pool.copy())  # input untouched


def test_copy_and_swap_match_brute_force_and_round_trip():
    rng = np.random.default_rng(1)
    layers = [rng.integers(0, 2**16, size=(8, 4, 2, 4), dtype=np.uint16) for _ in range(4)]
    pairs = [(1, 6), (3, 0)]
    for t in layers:
        got = kvops.copy_blocks(t, pairs)
        for b in range(8):
            src = {6: 1, 0: 3}.get(b, b)
            assert np.array_equal(got[b], t[src])
    host = kvops.swap_out(layers, [1, 5, 2])
    assert all(h.shape == (3, 4, 2, 4) for h in host)
    cleared = [t.copy() for t in layers]
    for t in cleared:
        t[[1, 5, 2]] = 0
    back = kvops.swap_in(cleared, host, [6, 0, 3])
    for t0, t1 in zip(layers, back):
        assert np.array_equal(t1[[6, 0, 3]], t0[[1, 5, 2]])
        assert np.array_equal(t1[4], t0[4]) and np.array_equal(t1[7], t0[7])
    with pytest.raises(ValueError, match="swap_in"):
        kvops.swap_in(cleared, host, [2])


# ------------------------------------------------------------------ golden vectors
def _golden(name):
    path = GOLDEN / name
    if not path.exists():
        pytest.fail(f"missing golden fixture {path}; run tests/golden/make_goldens.py")
    return np.load(path, allow_pickle=False)


def test_attention_goldens():
    z = _golden("attention_cases.npz")
    names = [str(n) for n in z["names"]]
    for name in names:
        args = [torch.from_numpy(z[f"{name}/{k}"]) for k in ("q", "k", "v", "tables", "ctx", "ql")]
        scale = float(z[f"{name}/scale"])
        want = z[f"{name}/out"]
        got = gather.paged_attention_gather(*args, scale).numpy()
        np.testing.assert_allclose(got, want, atol=1e-6, rtol=1e-6, err_msg=name)
        np.testing.assert_allclose(dense_causal_f64(*args, scale), want, atol=1e-5, rtol=1e-5, err_msg=name)


def test_kvops_goldens():
    z = _golden("kvops.npz")
    assert np.array_equal(kvops.kv_append(z["pool"], z["rows"], z["slots"]), z["append_out"])
    pairs = [tuple(p) for p in z["pairs"].tolist()]
    assert np.array_equal(kvops.copy_blocks(z["pool"], pairs), z["copy_out"])
    assert np.array_equal(kvops.swap_out([z["pool"]], z["swap_blocks"].tolist())[0], z["swap_host"])


# ------------------------------------------------------------------ planted mistakes
def test_pins_catch_a_wrong_gqa_mapping(monkeypatch):
    """Planted in the oracle: tile KV heads (h % Hkv) instead of repeat (h // group)."""
    monkeypatch.setattr(gather, "_kv_heads_for",
                        lambda kv, n: kv.repeat(*([1] * (kv.dim() - 2)), n // kv.shape[-2], 1))
    q, kp, vp, tables, ctx, ql = build([(9, 9), (5, 1)], heads=4, kv_heads=2)
    got = gather.paged_attention_gather(q, kp, vp, tables, ctx, ql, 0.3)
    assert not np.allclose(_np(got), dense_causal_f64(q, kp, vp, tables, ctx, ql, 0.3), atol=1e-3)


def test_pins_catch_a_dropped_scale():
    q, kp, vp, tables, ctx, ql = build(CASES["mixed"])
    got = gather.paged_attention_gather(q, kp, vp, tables, ctx, ql, 1.0)      # "forgot" the scale
    assert not np.allclose(_np(got), dense_causal_f64(q, kp, vp, tables, ctx, ql, 8 ** -0.5), atol=1e-3)


def test_pins_catch_an_off_by_one_context_len():
    """Planted: the online oracle fed the PRE-pass context length (ctx - 1), the
    off-by-one the reference contract warns about (core/attention.py:35-38): every
    query then sits one position early and misses its own key."""
    q, kp, vp, tables, ctx, ql = build(CASES["partial_query"])
    ref = dense_causal_f64(q, kp, vp, tables, ctx, ql, 8 ** -0.5)
    got = online.paged_attention_online(q.numpy(), kp.numpy(), vp.numpy(), tables.numpy(), (ctx - 1).numpy(),
                                        ql.numpy(), 8 ** -0.5)
    assert not np.allclose(got, ref, atol=1e-3)


def test_pins_catch_a_transposed_append():
    """Planted: rows written as [H, T, D] reinterpreted, i.e. heads and tokens swapped."""
    rng = np.random.default_rng(2)
    pool = np.zeros((4, 4, 3, 5), dtype=np.float32)
    rows = rng.standard_normal((3, 3, 5)).astype(np.float32)
    slots = np.array([5, 0, 9])
    good = kvops.kv_append(pool, rows, slots)
    bad = kvops.kv_append(pool, rows.transpose(1, 0, 2), slots)
    assert not np.array_equal(good, bad)
    assert np.array_equal(good.reshape(16, 3, 5)[slots], rows)
