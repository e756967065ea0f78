"""HIP KV append, block copy and swap vs the numpy oracle — bit-exact.

Covers the reference's swap tests (tests/test_swap.py:35-79: round trip into
DIFFERENT blocks with untouched neighbours, count mismatch refused, free list not
touched) and COW copy (tests/test_prefix_cache.py:242-266), for fp32/fp16/bf16, and
BASELINE config 3 at full size (32 layers x [16384, 16, 8, 128] bf16): 256-row
appends, 512 copy-on-write pairs and a 1024-block swap out and back in.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from inference_server.config import CONFIG
from inference_server.core.kv_pool import ModelDims, PagedKVPool
from oracle import kvops

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


@pytest.fixture(autouse=True)
def hip_backend(monkeypatch):
    monkeypatch.setattr(CONFIG, "attention", "hip")


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw element bits (so NaN payloads and -0.0 compare exactly)."""
    t = t.detach().cpu().contiguous()
    view = {4: torch.int32, 2: torch.int16}[t.element_size()]
    return t.view(view).numpy()


def make_pool(layers=2, kv_heads=3, d=8, blocks=16, bs=4, dtype=torch.float32, seed=0):
    pool = PagedKVPool(ModelDims(layers, kv_heads, d, dtype), num_blocks=blocks, block_size=bs, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(seed)
    for t in pool.k + pool.v:
        t.copy_(torch.randn(t.shape, generator=g, device="cuda").to(dtype))
    return pool


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [8, 12, 64, 128])
def test_append_matches_oracle(dtype, d):
    pool = make_pool(kv_heads=3, d=d, blocks=16, bs=4, dtype=dtype)
    before_k, before_v = bits(pool.k[1]), bits(pool.v[1])
    g = torch.Generator().manual_seed(3)
    T = 11
    slots = torch.randperm(16 * 4, generator=g)[:T]
    # The executor's source is key_states[0].transpose(0, 1): strided [T, H, D].
    ks = torch.randn(1, 3, T, d, generator=g).to(dtype).cuda()
    vs = torch.randn(1, 3, T, d, generator=g).to(dtype).cuda()
    k, v = ks[0].transpose(0, 1), vs[0].transpose(0, 1)
    assert not k.is_contiguous()
    pool.append(1, k, v, slots.cuda(), host_slots=slots)
    want_k = kvops.kv_append(before_k, bits(k), slots.numpy())
    want_v = kvops.kv_append(before_v, bits(v), slots.numpy())
    assert np.array_equal(bits(pool.k[1]), want_k)
    assert np.array_equal(bits(pool.v[1]), want_v)


def test_append_rejects_out_of_range_slots():
    pool = make_pool()
    k = torch.zeros(2, 3, 8, device="cuda")
    with pytest.raises(IndexError):
        pool.append(0, k, k, torch.tensor([0, 64], device="cuda"))


def test_append_all_layers_one_launch():
    from inference_server import native

    L, nb, bs, H, D = 4, 32, 16, 2, 64
    pool = make_pool(layers=L, kv_heads=H, d=D, blocks=nb, bs=bs, dtype=torch.bfloat16)
    before = [bits(t) for t in pool.k + pool.v]
    g = torch.Generator().manual_seed(9)
    T = 40
    slots = torch.randperm(nb * bs, generator=g)[:T]
    k_new = torch.randn(L, T, H, D, generator=g).to(torch.bfloat16).cuda()
    v_new = torch.randn(L, T, H, D, generator=g).to(torch.bfloat16).cuda()
    tab = pool.pointer_table()
    rc = native.lib().pkv_kv_append_layers(
        tab.data_ptr(), tab.data_ptr() + 8 * L, L, nb, bs, H, D,
        k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), k_new.stride(1), k_new.stride(2),
        slots.cuda().data_ptr(), T, native.PKV_BFLOAT16, native.stream_handle(torch.device("cuda")),
    )
    native.check(rc, "pkv_kv_append_layers")
    for l in range(L):
        assert np.array_equal(bits(pool.k[l]), kvops.kv_append(before[l], bits(k_new[l]), slots.numpy()))
        assert np.array_equal(bits(pool.v[l]), kvops.kv_append(before[L + l], bits(v_new[l]), slots.numpy()))


@pytest.mark.parametrize("dtype", DTYPES)
def test_copy_blocks_matches_oracle(dtype):
    pool = make_pool(layers=3, dtype=dtype, blocks=16)
    before = [bits(t) for t in pool.k + pool.v]
    pairs = [(1, 9), (4, 0), (7, 12), (2, 3)]
    pool.copy_blocks(pairs)
    for t, b in zip(pool.k + pool.v, before):
        assert np.array_equal(bits(t), kvops.copy_blocks(b, pairs))


def test_copy_block_hook_single_pair():
    """The COW hook `copy(src, dst)` of BlockTable.ensure_private."""
    pool = make_pool(layers=2)
    before = [bits(t) for t in pool.k + pool.v]
    pool.copy_block(5, 11)
    for t, b in zip(pool.k + pool.v, before):
        assert np.array_equal(bits(t), kvops.copy_blocks(b, [(5, 11)]))


@pytest.mark.parametrize("dtype", DTYPES)
def test_swap_round_trip_lands_the_same_bytes_in_different_blocks(dtype):
    """Reference tests/test_swap.py:35-56 on the hip path."""
    pool = make_pool(layers=2, kv_heads=2, d=4, blocks=8, bs=4, dtype=dtype)
    k0 = [bits(t) for t in pool.k]
    v0 = [bits(t) for t in pool.v]
    host = pool.swap_out([1, 5, 2])
    assert len(host) == 3 and all(t.device.type == "cpu" and t.is_pinned() for t in host.k + host.v)
    assert host.nbytes == 3 * pool.dims.bytes_per_block(4)
    want_host = kvops.swap_out([*k0, *v0], [1, 5, 2])
    for got, want in zip(host.k + host.v, want_host):
        assert np.array_equal(bits(got), want)
    for t in pool.k + pool.v:
        t[[1, 5, 2]] = 0
    mid = [bits(t) for t in pool.k + pool.v]
    pool.swap_in(host, [6, 0, 3])
    torch.cuda.synchronize()
    want = kvops.swap_in(mid, want_host, [6, 0, 3])
    for t, w in zip(pool.k + pool.v, want):
        assert np.array_equal(bits(t), w)
    for layer in range(2):
        assert np.array_equal(bits(pool.k[layer])[[6, 0, 3]], k0[layer][[1, 5, 2]])
        assert np.array_equal(bits(pool.k[layer])[4], k0[layer][4])       # untouched
        assert np.array_equal(bits(pool.v[layer])[7], v0[layer][7])


def test_swap_in_refuses_a_mismatched_block_count():
    pool = make_pool(blocks=8)
    host = pool.swap_out([0, 1])
    with pytest.raises(ValueError):
        pool.swap_in(host, [2])
    with pytest.raises(ValueError):
        pool.swap_in(host, [2, 3, 4])


# --------------------------------------------------------------------- async swap
def test_swap_out_snapshot_is_taken_before_later_writes_to_the_freed_blocks():
    """swap_out returns while its PCIe copy is still queued on the copy stream. The
    freed blocks' next owner writes them on the current stream straight away (no host
    sync in between): the host copy must still be the blocks as they were."""
    pool = make_pool(layers=3, kv_heads=2, d=8, blocks=16, bs=4, dtype=torch.bfloat16)
    out = [3, 9, 4, 15]
    out_dev = torch.tensor(out, device="cuda")
    before = [bits(t) for t in pool.k + pool.v]
    torch.cuda.synchronize()
    host = pool.swap_out(out)
    assert host.ready is not None
    for t in pool.k + pool.v:
        t.index_fill_(0, out_dev, 7.0)
    want = kvops.swap_out(before, out)
    for got, w in zip(host.k + host.v, want):           # .k / .v wait for the copy
        assert np.array_equal(bits(got), w)
    assert host.ready is None
    for t in pool.k:
        assert bool((t[out_dev] == 7.0).all())


@pytest.mark.parametrize("dtype", DTYPES)
def test_swap_in_straight_after_swap_out_needs_no_host_wait(dtype):
    """Out of [1, 5, 2, 11], into [6, 0, 3, 12], then a read on the current stream —
    no synchronisation anywhere until the result is fetched. The restored blocks equal
    the originals bit for bit; the rest of the pool equals the oracle's swap_in."""
    pool = make_pool(layers=2, kv_heads=3, d=12, blocks=16, bs=4, dtype=dtype, seed=4)
    out, back = [1, 5, 2, 11], [6, 0, 3, 12]
    before = [bits(t) for t in pool.k + pool.v]
    torch.cuda.synchronize()
    host = pool.swap_out(out)
    pool.swap_in(host, back)
    assert host.ready is not None                       # swap_in did not wait on the CPU
    snap = [t.clone() for t in pool.k + pool.v]          # queued after the scatter
    want = kvops.swap_in(before, kvops.swap_out(before, out), back)
    for got, w in zip(snap, want):
        assert np.array_equal(bits(got), w)


def test_swap_round_trips_back_to_back_reuse_the_copy_stream():
    """Several victims swapped out, then in, in an interleaved order with no waits —
    the shape of a scheduler that preempts and re-admits in the same step."""
    pool = make_pool(layers=2, kv_heads=2, d=8, blocks=24, bs=4, dtype=torch.float16, seed=9)
    before = [bits(t) for t in pool.k + pool.v]
    torch.cuda.synchronize()
    a = pool.swap_out([0, 1, 2])
    b = pool.swap_out([10, 11])
    pool.swap_in(b, [20, 21])
    c = pool.swap_out([5])
    pool.swap_in(a, [17, 18, 19])
    pool.swap_in(c, [23])
    state = before
    for out, back in (([10, 11], [20, 21]), ([0, 1, 2], [17, 18, 19]), ([5], [23])):
        state = kvops.swap_in(state, kvops.swap_out(before, out), back)
    for t, w in zip(pool.k + pool.v, state):
        assert np.array_equal(bits(t), w)


def test_gather_and_scatter_blocks_skip_ids_outside_the_pool():
    """The two device halves of a swap through the C-ABI: ids outside [0, num_blocks)
    leave their staging slot (gather) or no block (scatter) written."""
    from inference_server import native

    pool = make_pool(layers=2, kv_heads=2, d=8, blocks=8, bs=4, dtype=torch.float16, seed=2)
    lib, stream = native.lib(), native.stream_handle(torch.device("cuda"))
    nt, nb = 4, pool.num_blocks
    before = [bits(t) for t in pool.k + pool.v]
    ids = torch.tensor([2, -1, 7, 8], dtype=torch.int64, device="cuda")
    staging = torch.full((nt, 4, 4, 2, 8), 3.0, dtype=torch.float16, device="cuda")
    native.check(lib.pkv_gather_blocks(pool.pointer_table().data_ptr(), nt, nb, pool.block_bytes,
                                       ids.data_ptr(), 4, staging.data_ptr(), stream), "pkv_gather_blocks")
    got = bits(staging)
    sentinel = bits(torch.full((4, 2, 8), 3.0, dtype=torch.float16))
    for i, b in enumerate(before):
        assert np.array_equal(got[i, 0], b[2]) and np.array_equal(got[i, 2], b[7])
        assert np.array_equal(got[i, 1], sentinel) and np.array_equal(got[i, 3], sentinel)

    back = torch.tensor([5, -3, 0, 1 << 40], dtype=torch.int64, device="cuda")
    native.check(lib.pkv_scatter_blocks(pool.pointer_table().data_ptr(), nt, nb, pool.block_bytes,
                                        back.data_ptr(), 4, staging.data_ptr(), stream), "pkv_scatter_blocks")
    for i, (t, b) in enumerate(zip(pool.k + pool.v, before)):
        want = b.copy()
        want[5], want[0] = got[i, 0], got[i, 2]
        assert np.array_equal(bits(t), want)


# --------------------------------------------------------------------- BASELINE config 3
def test_config3_full_size_round_trips():
    """BASELINE config 3 at full size, through the entry points bench.py times: 32
    layers x [16384, 16, 8, 128] bf16 (32 GiB of pool); (a) pkv_kv_append_layers of
    256 rows into random distinct slots of every layer, (b) one pkv_copy_blocks of 512
    (src, dst) pairs over every layer, (c) swap-out of 1024 blocks (pkv_gather_blocks +
    one DMA) and swap-in into a different set (DMA + pkv_scatter_blocks). Then ALL 64
    pool tensors are compared with torch.equal against torch's own index_copy_ /
    index_select applied in the same order to the same initial contents (regenerated
    per tensor from its seed), and every layer's host copy against the blocks it came
    from."""
    from inference_server import native

    L, NB, H, D = 32, 16384, 8, 128
    dev = torch.device("cuda")
    pool = PagedKVPool(ModelDims(L, H, D, torch.bfloat16), num_blocks=NB, block_size=16, device="cuda")
    tensors = pool.k + pool.v

    def initial(i):
        gen = torch.Generator(device="cuda").manual_seed(5000 + i)
        return torch.randn(tensors[i].shape, generator=gen, device="cuda", dtype=torch.bfloat16)

    for i, t in enumerate(tensors):
        t.copy_(initial(i))
    g = torch.Generator().manual_seed(1337)
    slots = torch.randperm(NB * 16, generator=g)[:256].to(dev)
    k_new = torch.randn(L, 256, H, D, generator=g).to(torch.bfloat16).to(dev)
    v_new = torch.randn(L, 256, H, D, generator=g).to(torch.bfloat16).to(dev)
    perm = torch.randperm(NB, generator=g)
    pairs = list(zip(perm[:512].tolist(), perm[512:1024].tolist()))
    out_blocks, in_blocks = perm[1024:2048].tolist(), perm[2048:3072].tolist()

    lib = native.lib()
    tab = pool.pointer_table()
    native.check(lib.pkv_kv_append_layers(tab.data_ptr(), tab.data_ptr() + 8 * L, L, NB, 16, H, D,
                                          k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), k_new.stride(1),
                                          k_new.stride(2), slots.data_ptr(), 256, native.PKV_BFLOAT16,
                                          native.stream_handle(dev)), "pkv_kv_append_layers")
    pool.copy_blocks(pairs)
    host = pool.swap_out(out_blocks)
    assert host.nbytes == 1024 * pool.dims.bytes_per_block(16)
    pool.swap_in(host, in_blocks)
    torch.cuda.synchronize()

    src = torch.tensor([a for a, _ in pairs], device=dev)
    dst = torch.tensor([b for _, b in pairs], device=dev)
    idx_out, idx_in = torch.tensor(out_blocks, device=dev), torch.tensor(in_blocks, device=dev)
    for i, t in enumerate(tensors):
        layer, rows = i % L, (k_new if i < L else v_new)
        ref = initial(i)
        ref.view(-1, H, D).index_copy_(0, slots, rows[layer])
        ref.index_copy_(0, dst, ref.index_select(0, src))
        swapped = ref.index_select(0, idx_out)
        ref.index_copy_(0, idx_in, swapped)
        assert torch.equal(t, ref), f"pool tensor {i} (layer {layer}, {'K' if i < L else 'V'})"
        parked = (host.k if i < L else host.v)[layer]
        assert torch.equal(parked.to(dev), swapped), f"host copy of tensor {i}"
    pool.release()
