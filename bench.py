"""Benchmark of the paged-KV hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra] [--no-e2e]
                    [--calibrate-copy]

Headline (`value`): paged decode attention on BASELINE config 4, the
Llama-3-8B-shaped batch the north-star target is quoted on — 128 sequences, 32 query
/ 8 KV heads, head_dim 128, bf16, block size 16, contexts U[512, 8192], block tables
a seeded permutation of a 65536-block pool. One step = one pkv_paged_attention_decode
call over the whole batch (one launch of the persistent MFMA decode kernel, then one of
its small merge kernel for the sequences whose blocks two or more workgroups' runs
share), inputs resident in HBM.
value = algorithmic bytes / mean step time, in GB/s.

Algorithmic bytes per launch: K and V once per KV head (sum(ctx) * 2 * Hkv * D * 2 B),
Q in and O out (2 * B * Hq * D * 2 B), the int64 block-table entries actually walked
(8 * sum(ceil(ctx / 16))) and context_lens (8 * B). The 2.3 GB touched per launch is
9x the 256 MB MALL, so the figure is an HBM figure.

Also reported (one JSON line, extra keys): roofline of the decode kernel, the CPU
oracle gather path timed on a bounded sample of the same workload on this host, and
secondary lines: config 2 (fp16 decode, MALL defeated by rotating 4 pool copies),
config 4 chunked prefill on MFMA (TFLOP/s), config 3 append / copy-on-write / swap
(GB/s, with the pinned-memcpy link ceiling), and the second half of the metric,
`paged_engine_output_tok_s`: config 5 end to end (GPT-2 fp16, 200 requests) with
ATTENTION=hip and ATTENTION=gather on the same GPU (plus a smaller pool that forces
recompute and swap preemption), and config 1 (GPT-2 fp32) on the host CPU with the
gather path beside ATTENTION=hip on the GPU. `--no-extra` / `--no-e2e` skip those.
"""

from __future__ import annotations

import argparse
import gc
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (str(REPO), str(REPO / "llm-inference-server_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402
import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
BS = 16


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def spread(ev_ms) -> dict:
    """Median and p10/p90 of per-step HIP-event times (ms)."""
    a = np.asarray(ev_ms, dtype=np.float64)
    return {"median": round(float(np.median(a)), 4), "p10": round(float(np.percentile(a, 10)), 4),
            "p90": round(float(np.percentile(a, 90)), 4)}


def pmc_traffic(kernel: str) -> dict | None:
    """HBM bytes per launch of `kernel` from the committed counter summary
    profiles/pmc_traffic.json: two rocprofv3 --pmc passes (FETCH_SIZE, then
    WRITE_SIZE) over this script with --calibrate-copy, each scaled by what the same
    counter reads for a 1 GiB device copy in the same process. None if absent."""
    path = REPO / "profiles" / "pmc_traffic.json"
    if not path.exists():
        return None
    data = json.loads(path.read_text())
    hit = data.get("kernels", {}).get(kernel)
    if hit is None:
        return None
    return {"hbm_bytes": hit["hbm_bytes"], "fetch_bytes": hit["fetch_bytes"], "write_bytes": hit["write_bytes"],
            "fetch_scale": data["calibration"]["fetch_scale"], "write_scale": data["calibration"]["write_scale"]}


# ------------------------------------------------------------------ workloads
class DecodeWorkload:
    """Seeded paged-decode batch with block tables over a permuted pool."""

    def __init__(self, batch, hq, hkv, d, ctx, num_blocks, dtype, seed=1337, pools=1):
        self.batch, self.hq, self.hkv, self.d, self.dtype = batch, hq, hkv, d, dtype
        self.ctx = torch.as_tensor(np.asarray(ctx), dtype=torch.long)
        g = torch.Generator().manual_seed(seed)
        nblk = (self.ctx + BS - 1) // BS
        width = int(nblk.max())
        perm = torch.randperm(num_blocks, generator=g)
        tables = torch.zeros(batch, width, dtype=torch.long)
        off = 0
        for i in range(batch):
            n = int(nblk[i])
            tables[i, :n] = perm[off:off + n]
            off += n
        self.tables_cpu = tables
        self.q_cpu = torch.randn(batch, hq, d, generator=g).to(dtype)
        dev = torch.device("cuda")
        torch.cuda.manual_seed(seed)
        self.pools = [(torch.randn(num_blocks, BS, hkv, d, device=dev, dtype=dtype),
                       torch.randn(num_blocks, BS, hkv, d, device=dev, dtype=dtype)) for _ in range(pools)]
        self.q = self.q_cpu.to(dev)
        self.tables = tables.to(dev)
        self.ctx_dev = self.ctx.to(dev)
        self.ql = torch.ones(batch, dtype=torch.long)
        self.ql_dev = self.ql.to(dev)
        self.scale = d ** -0.5
        self.out = torch.empty(batch, hq, d, device=dev, dtype=dtype)
        self.sum_ctx = int(self.ctx.sum())
        self.table_entries = int(nblk.sum())

    @property
    def algorithmic_bytes(self) -> int:
        s = torch.empty(0, dtype=self.dtype).element_size()
        kv = self.sum_ctx * 2 * self.hkv * self.d * s
        qo = 2 * self.batch * self.hq * self.d * s
        return kv + qo + 8 * self.table_entries + 8 * self.batch

    def make_call(self, pool_idx=0):
        """A zero-argument closure issuing exactly one pkv_paged_attention_decode."""
        from inference_server import native
        from inference_server.core.attention_hip import _WORKSPACES

        L = native.lib()
        kp, vp = self.pools[pool_idx]
        max_ctx = int(self.ctx.max())
        dev = torch.device("cuda")
        stream = native.stream_handle(dev)
        ws_bytes = L.pkv_paged_attention_decode_workspace_bytes(self.batch, self.hq, self.hkv, self.d, max_ctx)
        ws = _WORKSPACES.partials(dev, stream, ws_bytes)
        args = (self.out.data_ptr(), self.out.stride(0), self.out.stride(1),
                self.q.data_ptr(), self.q.stride(0), self.q.stride(1),
                kp.data_ptr(), vp.data_ptr(), kp.stride(0), kp.stride(1), kp.stride(2),
                kp.shape[0], BS, self.hkv, self.d,
                self.tables.data_ptr(), self.tables.stride(0), self.tables.shape[1],
                self.ctx_dev.data_ptr(), self.batch, self.hq, max_ctx,
                float(self.scale), native.dtype_code(self.dtype), ws.data_ptr(), ws.numel(), stream)
        fn = L.pkv_paged_attention_decode

        def call():
            rc = fn(*args)
            if rc:
                native.check(rc, "pkv_paged_attention_decode")
        return call


def check_decode_whole(w: DecodeWorkload, out: torch.Tensor, pool_idx: int = 0) -> float:
    """Every row of a decode output against oracle.gather at 2e-2 (bf16/fp16). A row
    depends only on its own sequence, so each is re-derived from just the blocks its
    table row names (copied back from the device). Returns the largest |difference|;
    raises AssertionError naming the first row outside the tolerance."""
    from oracle.gather import paged_attention_gather

    kp, vp = w.pools[pool_idx]
    out = out.cpu()
    one = torch.ones(1, dtype=torch.long)
    worst = 0.0
    for i in range(w.batch):
        c = int(w.ctx[i])
        used = w.tables_cpu[i, : -(-c // BS)]
        idx = used.to(kp.device)
        ref = paged_attention_gather(w.q_cpu[i:i + 1], kp[idx].cpu(), vp[idx].cpu(), torch.arange(len(used))[None],
                                     w.ctx[i:i + 1], one, w.scale)
        torch.testing.assert_close(out[i:i + 1], ref, atol=2e-2, rtol=2e-2, msg=lambda m: f"decode row {i}: {m}")
        worst = max(worst, float((out[i:i + 1].float() - ref.float()).abs().max()))
    return worst


def config4_decode():
    rng = np.random.default_rng(1337)
    ctx = rng.integers(512, 8193, size=128)
    return DecodeWorkload(128, 32, 8, 128, ctx, 65536, torch.bfloat16)


class PrefillWorkload:
    """BASELINE config 4 chunked prefill: 16 sequences x 512-token chunks appended to
    cached contexts of U[0, 4096] tokens; bf16, 32/8 heads, d128, 65536-block pool."""

    def __init__(self, seqs=16, chunk=512, hq=32, hkv=8, d=128, num_blocks=65536, seed=1337):
        rng = np.random.default_rng(seed)
        self.c0 = rng.integers(0, 4097, size=seqs)
        self.ctx = torch.as_tensor(self.c0 + chunk, dtype=torch.long)
        self.ql = torch.full((seqs,), chunk, dtype=torch.long)
        g = torch.Generator().manual_seed(seed)
        nblk = (self.ctx + BS - 1) // BS
        perm = torch.randperm(num_blocks, generator=g)
        tables = torch.zeros(seqs, int(nblk.max()), dtype=torch.long)
        off = 0
        for i in range(seqs):
            tables[i, : nblk[i]] = perm[off:off + int(nblk[i])]
            off += int(nblk[i])
        dev = torch.device("cuda")
        torch.cuda.manual_seed(seed)
        self.kp = torch.randn(num_blocks, BS, hkv, d, device=dev, dtype=torch.bfloat16)
        self.vp = torch.randn(num_blocks, BS, hkv, d, device=dev, dtype=torch.bfloat16)
        self.q_cpu = torch.randn(seqs * chunk, hq, d, generator=g).to(torch.bfloat16)
        self.q = self.q_cpu.to(dev)
        self.tables_cpu = tables
        self.tables = tables.to(dev)
        self.ctx_dev = self.ctx.to(dev)
        self.qsl = torch.cat([torch.zeros(1, dtype=torch.long), torch.cumsum(self.ql, 0)]).to(dev)
        self.out = torch.empty_like(self.q)
        self.seqs, self.chunk, self.hq, self.hkv, self.d = seqs, chunk, hq, hkv, d
        # causal flops: 4*D per (query, key, head): QK^T and P.V, 2 flops per MAC
        q = chunk
        self.flops = int(hq * 4 * d * sum(q * int(c) + q * (q + 1) // 2 for c in self.c0))

    def make_call(self):
        from inference_server import native

        L = native.lib()
        stream = native.stream_handle(torch.device("cuda"))
        args = (self.out.data_ptr(), self.out.stride(0), self.out.stride(1),
                self.q.data_ptr(), self.q.stride(0), self.q.stride(1),
                self.kp.data_ptr(), self.vp.data_ptr(), self.kp.stride(0), self.kp.stride(1), self.kp.stride(2),
                self.kp.shape[0], BS, self.hkv, self.d,
                self.tables.data_ptr(), self.tables.stride(0), self.tables.shape[1],
                self.ctx_dev.data_ptr(), self.qsl.data_ptr(), self.seqs, self.hq, self.seqs * self.chunk, self.chunk,
                float(self.d ** -0.5), native.PKV_BFLOAT16, stream)
        fn = L.pkv_paged_attention_prefill

        def call():
            rc = fn(*args)
            if rc:
                native.check(rc, "pkv_paged_attention_prefill")
        return call


def check_prefill_whole(wp: PrefillWorkload, out: torch.Tensor) -> float:
    """Every chunk of a prefill output against oracle.gather at 2e-2, one sequence at a
    time over the blocks its table row names. Returns the largest |difference|; raises
    AssertionError naming the first sequence outside the tolerance."""
    from oracle.gather import paged_attention_gather

    out = out.cpu()
    worst = 0.0
    for i in range(wp.seqs):
        c = int(wp.ctx[i])
        used = wp.tables_cpu[i, : -(-c // BS)]
        idx = used.to(wp.kp.device)
        rows = slice(i * wp.chunk, (i + 1) * wp.chunk)
        ref = paged_attention_gather(wp.q_cpu[rows], wp.kp[idx].cpu(), wp.vp[idx].cpu(),
                                     torch.arange(len(used))[None], wp.ctx[i:i + 1], wp.ql[i:i + 1], wp.d ** -0.5)
        torch.testing.assert_close(out[rows], ref, atol=2e-2, rtol=2e-2, msg=lambda m: f"prefill seq {i}: {m}")
        worst = max(worst, float((out[rows].float() - ref.float()).abs().max()))
    return worst


class Config1Fp32:
    """BASELINE config 1's attention at GPT-2 shape in fp32 (12 heads, d64, block 16):
    the prefill of its 8 prompts (lengths from workload.config1) in one call, and a
    decode step over the same 8 sequences 16 tokens later; seeded N(0,1) pool."""

    def __init__(self, num_blocks=2048, seed=1337):
        from inference_server.bench import workload

        self.ql = np.array([len(r.prompt_token_ids) for r in workload.config1()])
        self.hq = self.hkv = 12
        self.d = 64
        g = torch.Generator().manual_seed(seed)
        nblk = (self.ql + 16 + BS - 1) // BS
        perm = torch.randperm(num_blocks, generator=g)
        tables = torch.zeros(len(self.ql), int(nblk.max()), dtype=torch.long)
        off = 0
        for i, n in enumerate(nblk):
            tables[i, :n] = perm[off:off + int(n)]
            off += int(n)
        dev = torch.device("cuda")
        self.kp = torch.randn(num_blocks, BS, self.hkv, self.d, generator=g).to(dev)
        self.vp = torch.randn(num_blocks, BS, self.hkv, self.d, generator=g).to(dev)
        self.tables = tables.to(dev)
        self.q = torch.randn(int(self.ql.sum()), self.hq, self.d, generator=g).to(dev)
        self.out = torch.empty_like(self.q)
        self.ctx_p = torch.as_tensor(self.ql, dtype=torch.long).to(dev)
        self.qsl = torch.as_tensor(np.concatenate([[0], np.cumsum(self.ql)]), dtype=torch.long).to(dev)
        self.ctx_d = (self.ctx_p + 16).contiguous()
        self.qd = torch.randn(len(self.ql), self.hq, self.d, generator=g).to(dev)
        self.outd = torch.empty_like(self.qd)
        self.flops = int(self.hq * 4 * self.d * sum(int(n) * (int(n) + 1) // 2 for n in self.ql))
        s = 4
        self.decode_bytes = int((self.ql + 16).sum()) * 2 * self.hkv * self.d * s + 2 * len(self.ql) * self.hq * self.d * s \
            + 8 * int(((self.ql + 16 + BS - 1) // BS).sum()) + 8 * len(self.ql)

    def prefill_call(self):
        from inference_server import native

        L = native.lib()
        stream = native.stream_handle(torch.device("cuda"))
        kp, vp = self.kp, self.vp
        args = (self.out.data_ptr(), self.out.stride(0), self.out.stride(1),
                self.q.data_ptr(), self.q.stride(0), self.q.stride(1),
                kp.data_ptr(), vp.data_ptr(), kp.stride(0), kp.stride(1), kp.stride(2), kp.shape[0], BS, self.hkv,
                self.d, self.tables.data_ptr(), self.tables.stride(0), self.tables.shape[1],
                self.ctx_p.data_ptr(), self.qsl.data_ptr(), len(self.ql), self.hq, int(self.ql.sum()),
                int(self.ql.max()), float(self.d ** -0.5), native.PKV_FLOAT32, stream)
        fn = L.pkv_paged_attention_prefill

        def call():
            rc = fn(*args)
            if rc:
                native.check(rc, "pkv_paged_attention_prefill")
        return call

    def decode_call(self):
        from inference_server import native
        from inference_server.core.attention_hip import _WORKSPACES

        L = native.lib()
        dev = torch.device("cuda")
        stream = native.stream_handle(dev)
        kp, vp = self.kp, self.vp
        max_ctx = int(self.ql.max()) + 16
        ws_bytes = L.pkv_paged_attention_decode_workspace_bytes(len(self.ql), self.hq, self.hkv, self.d, max_ctx)
        ws = _WORKSPACES.partials(dev, stream, ws_bytes)
        args = (self.outd.data_ptr(), self.outd.stride(0), self.outd.stride(1),
                self.qd.data_ptr(), self.qd.stride(0), self.qd.stride(1),
                kp.data_ptr(), vp.data_ptr(), kp.stride(0), kp.stride(1), kp.stride(2), kp.shape[0], BS, self.hkv,
                self.d, self.tables.data_ptr(), self.tables.stride(0), self.tables.shape[1],
                self.ctx_d.data_ptr(), len(self.ql), self.hq, max_ctx,
                float(self.d ** -0.5), native.PKV_FLOAT32, ws.data_ptr(), ws.numel(), stream)
        fn = L.pkv_paged_attention_decode

        def call():
            rc = fn(*args)
            if rc:
                native.check(rc, "pkv_paged_attention_decode")
        return call


def config1_fp32(steps: int, warmup: int) -> dict:
    w = Config1Fp32()
    _, pf_ms = time_region([w.prefill_call()], steps, warmup)
    _, dec_ms = time_region([w.decode_call()], steps, warmup)
    return {
        "prefill_us": round(pf_ms * 1e3, 2),
        "prefill_TFLOP/s": round(w.flops / (pf_ms / 1e3) / 1e12, 2),
        "decode_us": round(dec_ms * 1e3, 2),
        "decode_GB/s": round(w.decode_bytes / (dec_ms / 1e3) / 1e9, 1),
        "causal_flops": w.flops,
        "decode_algorithmic_bytes": w.decode_bytes,
        "note": "GPT-2 shape fp32 (12 heads, d64, block 16): config 1's 8 prompts prefilled in one call "
                "(fp32 MFMA kernel), then one decode step over them 16 tokens later (fp32 register kernel)",
    }


def config3_kvops(steps: int) -> dict:
    """bf16, 32 layers x [16384, 16, 8, 128] (32 GiB of pool).
    (a) append 256 rows per layer into random distinct slots (one all-layer launch),
    (b) copy-on-write of 512 random (src, dst) pairs across all layers (one launch),
    (c) swap-out / swap-in of 1024 blocks through pinned host memory."""
    import inference_server.config as cfg
    from inference_server import native
    from inference_server.core.kv_pool import ModelDims, PagedKVPool

    old = cfg.CONFIG.attention
    cfg.CONFIG.attention = "hip"
    try:
        L, NB, H, D = 32, 16384, 8, 128
        pool = PagedKVPool(ModelDims(L, H, D, torch.bfloat16), num_blocks=NB, block_size=BS, device="cuda")
        g = torch.Generator().manual_seed(1337)
        dev = torch.device("cuda")
        stream = native.stream_handle(dev)
        lib = native.lib()
        out = {}

        # (a) append, all layers in one launch
        slots = torch.randperm(NB * BS, generator=g)[:256].to(dev)
        k_new = torch.randn(L, 256, H, D, device=dev, dtype=torch.bfloat16)
        v_new = torch.randn(L, 256, H, D, device=dev, dtype=torch.bfloat16)
        tab = pool.pointer_table()

        def append_all():
            native.check(lib.pkv_kv_append_layers(tab.data_ptr(), tab.data_ptr() + 8 * L, L, NB, BS, H, D,
                                                  k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0),
                                                  k_new.stride(1), k_new.stride(2), slots.data_ptr(), 256,
                                                  native.PKV_BFLOAT16, stream), "append")
        _, ms = time_region([append_all], steps, 3)
        nbytes = 2 * (2 * L * 256 * H * D * 2) + 8 * 256
        out["append_256_rows_x32_layers"] = {"GB/s": round(nbytes / (ms / 1e3) / 1e9, 1), "us": round(ms * 1e3, 2),
                                             "algorithmic_bytes": nbytes}

        # (b) copy-on-write, 512 pairs x 32 layers x K,V
        perm = torch.randperm(NB, generator=g)
        pairs = list(zip(perm[:512].tolist(), perm[512:1024].tolist()))
        flat = torch.tensor([b for pr in pairs for b in pr], device=dev)

        def cow():
            native.check(lib.pkv_copy_blocks(tab.data_ptr(), 2 * L, NB, pool.block_bytes, flat.data_ptr(), 512,
                                             stream), "copy")
        _, ms = time_region([cow], max(5, steps // 3), 2)
        nbytes = 2 * 512 * 2 * L * pool.block_bytes
        out["cow_512_pairs_x32_layers"] = {"GB/s": round(nbytes / (ms / 1e3) / 1e9, 1), "us": round(ms * 1e3, 2),
                                           "algorithmic_bytes": nbytes}

        # (c) swap: 1024 blocks out (gather + one D2H DMA), then in (H2D DMA + scatter)
        out_blocks = perm[1024:2048].tolist()
        in_blocks = perm[2048:3072].tolist()
        host = pool.swap_out(out_blocks)           # warm (allocates the pinned buffer once)
        pool.swap_in(host, in_blocks)
        torch.cuda.synchronize()
        reps = 3
        t_out, t_ret, t_in, t_in_ret = [], [], [], []
        for _ in range(reps):
            t0 = time.perf_counter()
            host = pool.swap_out(out_blocks)       # returns once the gather and DMA are queued
            t_ret.append(time.perf_counter() - t0)
            host.wait()                            # ... timed until the host copy has landed
            t_out.append(time.perf_counter() - t0)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            pool.swap_in(host, in_blocks)
            t_in_ret.append(time.perf_counter() - t0)
            torch.cuda.synchronize()
            t_in.append(time.perf_counter() - t0)
        nbytes = host.nbytes
        # Link ceiling on the same box: one pinned<->device copy of the same size.
        pinned = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
        devbuf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        devbuf.copy_(pinned)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        devbuf.copy_(pinned, non_blocking=True)
        torch.cuda.synchronize()
        h2d = nbytes / (time.perf_counter() - t0) / 1e9
        t0 = time.perf_counter()
        pinned.copy_(devbuf, non_blocking=True)
        torch.cuda.synchronize()
        d2h = nbytes / (time.perf_counter() - t0) / 1e9
        out["swap_1024_blocks"] = {
            "out_GB/s": round(nbytes / min(t_out) / 1e9, 2), "in_GB/s": round(nbytes / min(t_in) / 1e9, 2),
            "call_returns_after_ms": {"out": round(1e3 * min(t_ret), 3), "in": round(1e3 * min(t_in_ret), 3)},
            "bytes_each_way": nbytes, "pinned_memcpy_ceiling_GB/s": {"h2d": round(h2d, 2), "d2h": round(d2h, 2)},
        }
        # Bit check of what was timed, on all 2 x 32 pool tensors: torch's own
        # index_copy_ / index_select applied in the same order to the same (zero)
        # initial pool. Every timed operation is idempotent (distinct slots; COW and swap
        # over disjoint block sets), so one application of each is the expected state.
        del pinned, devbuf
        src = torch.tensor([a for a, _ in pairs], device=dev)
        dst = torch.tensor([b for _, b in pairs], device=dev)
        i_out, i_in = torch.tensor(out_blocks, device=dev), torch.tensor(in_blocks, device=dev)
        bad = []
        for i, t in enumerate(pool.k + pool.v):
            layer, rows = i % L, (k_new if i < L else v_new)
            ref = torch.zeros_like(t)
            ref.view(-1, H, D).index_copy_(0, slots, rows[layer])
            ref.index_copy_(0, dst, ref.index_select(0, src))
            parked = ref.index_select(0, i_out)
            ref.index_copy_(0, i_in, parked)
            host_copy = (host.k if i < L else host.v)[layer].to(dev)
            if not (torch.equal(t, ref) and torch.equal(host_copy, parked)):
                bad.append(i)
            del ref, parked, host_copy
        if bad:
            raise AssertionError(f"config 3: pool tensors {bad} differ from torch index ops after timing")
        out["bit_exact_after_timing"] = "all 64 pool tensors and host copies equal torch index_copy_/index_select"
        pool.release()
        del host, k_new, v_new
        torch.cuda.empty_cache()
        return out
    finally:
        cfg.CONFIG.attention = old


def _engine_run(model, tok, reqs, backend, mode, num_blocks, device, graphs=True, probe=None):
    """One engine run. On ATTENTION=hip decode and prefill steps replay HIP graphs
    (unless graphs=False), every batch size and token bucket captured when the engine
    starts — the start-up cost is reported as graph_capture_s, off the clock like model
    loading. `probe` (a MarginProbe) watches the logits of the timed run."""
    import inference_server.config as cfg
    from inference_server.engine.paged import PagedEngine

    saved = (cfg.CONFIG.attention, cfg.CONFIG.preemption, cfg.CONFIG.decode_graphs, cfg.CONFIG.prefill_graphs)
    cfg.CONFIG.attention, cfg.CONFIG.preemption = backend, mode
    cfg.CONFIG.decode_graphs = cfg.CONFIG.prefill_graphs = graphs
    try:
        warm = PagedEngine(model, tok, num_blocks=num_blocks, block_size=BS, device=device, prefix_caching=True)
        warm.run(reqs[:4])                               # one-time costs off the clock
        warm.shutdown()
        engine = PagedEngine(model, tok, num_blocks=num_blocks, block_size=BS, device=device, prefix_caching=True,
                             capture_graphs=graphs and backend == "hip" and device == "cuda")
        engine.executor.logit_probe = probe
        r = engine.run(reqs)
        dg, pg = engine.executor.graphs, engine.executor.prefill_graphs
        if dg is not None:
            r.graph_info = {"decode_graph_replays": dg.replays, "graph_capture_s": round(engine.graph_capture_s, 3),
                            "graph_nodes_b32": dg.census.get(max(dg.census), {}) if dg.census else {},
                            "decode_table_row_rewrites": dg.rows.rewrites}
        if pg is not None:
            r.graph_info["prefill_graph_replays"] = pg.replays
        engine.shutdown()
        return r
    finally:
        cfg.CONFIG.attention, cfg.CONFIG.preemption, cfg.CONFIG.decode_graphs, cfg.CONFIG.prefill_graphs = saved


def _summary(r, ref=None, probe=None, name=None) -> dict:
    out = {"tok/s": round(r.tok_per_s, 1), "generated": r.generated_tokens, "wall_s": round(r.wall_s, 2),
           "steps": r.steps, "preemptions": r.stats["preemptions"], "swaps": r.stats["swaps"],
           "prefix_hits": r.stats.get("prefix_hits", 0)}
    if ref is not None:
        from inference_server.bench.parity import first_divergences

        divs = first_divergences(ref.outputs, r.outputs, probe, name)
        out["requests_identical_to_gather"] = f"{len(ref.outputs) - len(divs)}/{len(ref.outputs)}"
        if probe is not None:
            # Each stream that differs: (request, first differing token index, how far
            # the hip token's fp16 logit sits below gather's maximum there, in ulps).
            out["divergences"] = [[d["seq"], d["index"], d["ulps_below_max"]] for d in divs]
            ulps = [d["ulps_below_max"] for d in divs if d["ulps_below_max"] is not None]
            out["max_divergence_ulps"] = max(ulps) if ulps else None
    out.update(getattr(r, "graph_info", {}))
    return out


def e2e_engine() -> dict:
    """The paged engine end to end (output tok/s = generated tokens / wall time).

    config 5 (GPU): GPT-2 124M fp16 (seeded random init), 200 requests, 50% sharing a
      128-token prefix, max 32 running, the specified 1024-block pool, with
      ATTENTION=hip and with ATTENTION=gather (the reference path) on the same GPU; the
      1024-block pool does not run out on this workload, so the same requests also run
      on a 256-block pool under recompute and swap preemption. hip runs replay decode
      and prefill steps from HIP graphs; one hip run issues steps eagerly for
      comparison. Each hip run is compared token by token with a gather run of the same
      pool and mode, whose logits a MarginProbe watches: every differing stream is
      reported with the ulp distance of its first differing token below gather's
      maximum logit (the streams may part only at near-ties).
    config 1: GPT-2 fp32, 8 requests x 32 greedy tokens: ATTENTION=gather on the host
      CPU (the reference's own CPU case) and ATTENTION=hip on the GPU, token ids
      compared."""
    from inference_server.bench import workload
    from inference_server.bench.parity import MarginProbe
    from inference_server.model import load

    res = {}
    reqs = workload.config5()
    model, tok = load(dtype=torch.float16, device="cuda")
    hip = {
        "hip_1024": _engine_run(model, tok, reqs, "hip", "recompute", 1024, "cuda"),
        "hip_1024_eager_steps": _engine_run(model, tok, reqs, "hip", "recompute", 1024, "cuda", graphs=False),
        "hip_256_recompute": _engine_run(model, tok, reqs, "hip", "recompute", 256, "cuda"),
        "hip_256_swap": _engine_run(model, tok, reqs, "hip", "swap", 256, "cuda"),
    }
    gather = _engine_run(model, tok, reqs, "gather", "recompute", 1024, "cuda")     # timed, unprobed
    res["config5_gather_1024"] = _summary(gather)
    for blocks, mode, names in ((1024, "recompute", ("hip_1024", "hip_1024_eager_steps")),
                                (256, "recompute", ("hip_256_recompute",)), (256, "swap", ("hip_256_swap",))):
        probe = MarginProbe({n: hip[n].outputs for n in names})
        ref = _engine_run(model, tok, reqs, "gather", mode, blocks, "cuda", probe=probe)
        for n in names:
            res[f"config5_{n}"] = _summary(hip[n], ref, probe, n)
    del model
    torch.cuda.empty_cache()

    reqs1 = workload.config1()
    model, tok = load(dtype=torch.float32, device="cuda")
    hip1 = _engine_run(model, tok, reqs1, "hip", "recompute", 2048, "cuda")
    del model
    torch.cuda.empty_cache()
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    model, tok = load(dtype=torch.float32, device="cpu")
    cpu1 = _engine_run(model, tok, reqs1, "gather", "recompute", 2048, "cpu")
    res["config1_cpu_gather_fp32"] = _summary(cpu1)
    res["config1_cpu_gather_fp32"]["threads"] = torch.get_num_threads()
    res["config1_gpu_hip_fp32"] = _summary(hip1, cpu1)
    return res


def config2_decode(pools=4):
    rng = np.random.default_rng(1337)
    ctx = np.clip(np.round(np.exp(rng.normal(math.log(300), 0.9, 64))), 16, 2048).astype(np.int64)
    return DecodeWorkload(64, 12, 12, 64, ctx, 8192, torch.float16, pools=pools)


def greedy_lm_head(steps, warmup, rows=32, vocab=50257, dim=768, per_graph=20):
    """pkv_lm_head_argmax on GPT-2's LM-head shape (config 5's model; `rows` = its
    decode batch, MAX_RUNNING) against the GEMM + argmax it replaces, same inputs. Each
    is captured `per_graph` times into one HIP graph (as the engine's step graphs run
    it) and the graph is replayed back to back, one event pair per timed region: GPU
    time per call without the host's launch cost, which at ~20 us per call would
    otherwise be what a Python loop measures. Algorithmic bytes: the fp16 weight and
    hidden rows read once, the int64 ids written."""
    from inference_server.core.sampling import lm_head_argmax

    g = torch.Generator(device="cuda").manual_seed(1337)
    w = (torch.randn(vocab, dim, device="cuda", generator=g) / 7).half()
    h = torch.randn(rows, dim, device="cuda", generator=g).half()
    fused = lm_head_argmax(h, w)
    same = bool(torch.equal(fused, (h @ w.T).argmax(-1)))

    def graphed(fn):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()  # outside the capture: the fused call's workspace for this stream
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=s):
                for _ in range(per_graph):
                    fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        return graph

    fg = graphed(lambda: lm_head_argmax(h, w))
    tg = graphed(lambda: (h @ w.T).argmax(-1))
    reps = max(1, steps // per_graph)
    _, f_ms = time_region([fg.replay], reps, max(1, warmup // per_graph))
    _, t_ms = time_region([tg.replay], reps, max(1, warmup // per_graph))
    f_ms, t_ms = f_ms / per_graph, t_ms / per_graph
    replayed = lm_head_argmax(h, w)
    nbytes = vocab * dim * 2 + rows * dim * 2 + rows * 8
    return {"GB/s": round(nbytes / (f_ms / 1e3) / 1e9, 1), "frac_of_hbm_peak": round(nbytes / (f_ms / 1e3) / 8e12, 4),
            "fused_ms_mean": round(f_ms, 4), "gemm_argmax_ms_mean": round(t_ms, 4),
            "speedup": round(t_ms / f_ms, 3), "ids_identical": same and bool(torch.equal(replayed, fused)),
            "algorithmic_bytes": nbytes,
            "note": f"{rows} rows x [{vocab}, {dim}] fp16 LM head; {reps * per_graph} calls each, "
                    f"timed as replays of a {per_graph}-call HIP graph (GPU time, no host launch cost)"}


# ------------------------------------------------------------------ timing
def time_region(calls, steps, warmup):
    """Run `warmup` untimed steps, then exactly `steps` timed ones back to back, the
    timed region bracketed by one pair of HIP events on the launch stream (and by
    synchronisations for the wall clock). Returns (total_seconds, event milliseconds per
    step): the average launch duration over the region, consecutive launches included
    as a serving loop issues them."""
    for i in range(warmup):
        calls[i % len(calls)]()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # No cyclic-garbage collection inside the region: a collection pass stalls the host
    # for milliseconds, and a launch-bound loop (config 2's 27 us calls) then measures
    # the stall instead of the GPU.
    gc.collect()
    gc.disable()
    try:
        t0 = time.perf_counter()
        a.record()
        for i in range(steps):
            calls[i % len(calls)]()
        b.record()
        torch.cuda.synchronize()
        total = time.perf_counter() - t0
    finally:
        gc.enable()
    return total, a.elapsed_time(b) / steps


def time_steps(calls, steps, warmup):
    """Run `warmup` untimed steps, then exactly `steps` timed ones. Each step issues
    calls[i % len(calls)] once, bracketed by HIP events on the launch stream (the
    events' markers add ~10 us between launches, so these are for the spread, not the
    mean). Returns (total_seconds, per-step event milliseconds)."""
    for i in range(warmup):
        calls[i % len(calls)]()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record()
        calls[i % len(calls)]()
        ev[i][1].record()
    torch.cuda.synchronize()
    total = time.perf_counter() - t0
    return total, [a.elapsed_time(b) for a, b in ev]


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(w: DecodeWorkload, n_seq=16, reps=3):
    """The oracle gather path (reference core/attention.py:130-153 restated, torch CPU
    ops) on `n_seq` sequences of the same workload, their real contexts and tables."""
    from oracle.gather import paged_attention_gather

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    idx = torch.arange(n_seq) * (w.batch // n_seq)
    ctx = w.ctx[idx]
    width = int(((ctx + BS - 1) // BS).max())
    used = w.tables_cpu[idx, :width]
    flat = used.flatten()
    uniq, inverse = torch.unique(flat, return_inverse=True)
    kp, vp = (t[uniq.to(t.device)].cpu() for t in w.pools[0])
    tables = inverse.view(n_seq, width)
    q = w.q_cpu[idx]
    ql = torch.ones(n_seq, dtype=torch.long)
    paged_attention_gather(q[:2], kp, vp, tables[:2], ctx[:2], ql[:2], w.scale)  # warm
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        paged_attention_gather(q, kp, vp, tables, ctx, ql, w.scale)
        times.append(time.perf_counter() - t)
    s = torch.empty(0, dtype=w.dtype).element_size()
    nbytes = int(ctx.sum()) * 2 * w.hkv * w.d * s + 2 * n_seq * w.hq * w.d * s + 8 * int(((ctx + 15) // 16).sum()) + 8 * n_seq
    med = float(np.median(times))
    return {
        "value": round(nbytes / med / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{n_seq} of the 128 config-4 sequences (every {w.batch // n_seq}th; sum ctx {int(ctx.sum())}), "
                   f"bf16 torch CPU ops, median of {reps} runs of {med:.2f} s; cpu {cpu_model()}, "
                   f"os.cpu_count()={os.cpu_count()}"),
    }


def cpu_legs() -> dict:
    """The CPU legs beside the secondary GPU lines, on this host's cores, same seeded
    shapes and the same algorithmic units: the oracle gather path (reference
    core/attention.py:92-199 restated as torch CPU ops) on config 2's fp16 decode batch
    (all 64 sequences) and on 8 of config 4's 16 prefill chunks (bf16); and the
    reference's KV byte movers as torch CPU ops on config 3's bf16 block shape over 2 of
    its 32 layers: the append's per-layer index_copy_ (core/paged_executor.py:116-125),
    copy-on-write's per-layer block copy_ (:265-270) and swap's per-layer index_select
    into a host tensor and index_copy_ back (core/kv_pool.py:142-182; on a CPU there is
    no host link, so this is the reference's memory traffic only). Reported baselines,
    not targets."""
    from oracle.gather import paged_attention_gather

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    out = {"cores": threads, "cpu": cpu_model(), "os.cpu_count()": os.cpu_count(), "kind": "port"}
    g = torch.Generator().manual_seed(1337)

    def med(fn, reps):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    # config 2: fp16 decode, 64 x 12 heads x d64, lognormal contexts, 8192-block pool
    rng = np.random.default_rng(1337)
    ctx = np.clip(np.round(np.exp(rng.normal(math.log(300), 0.9, 64))), 16, 2048).astype(np.int64)
    nblk = (ctx + BS - 1) // BS
    perm = torch.randperm(8192, generator=g)
    tables = torch.zeros(64, int(nblk.max()), dtype=torch.long)
    off = 0
    for i in range(64):
        tables[i, :nblk[i]] = perm[off:off + nblk[i]]
        off += int(nblk[i])
    kp = torch.randn(8192, BS, 12, 64, generator=g).half()
    vp = torch.randn(8192, BS, 12, 64, generator=g).half()
    q = torch.randn(64, 12, 64, generator=g).half()
    c, ql = torch.as_tensor(ctx), torch.ones(64, dtype=torch.long)
    sec = med(lambda: paged_attention_gather(q, kp, vp, tables, c, ql, 0.125), 3)
    nbytes = int(ctx.sum()) * 2 * 12 * 64 * 2 + 2 * 64 * 12 * 64 * 2 + 8 * int(nblk.sum()) + 8 * 64
    out["config2_decode_fp16"] = {"GB/s": round(nbytes / sec / 1e9, 4), "s": round(sec, 3),
                                  "sample": "all 64 sequences, median of 3"}
    del kp, vp

    # config 4 chunked prefill: 8 of the 16 chunks (every other one), bf16
    rng = np.random.default_rng(1337)
    c0 = rng.integers(0, 4097, size=16)[::2]
    hq, hkv, d, chunk = 32, 8, 128, 512
    ctxs = torch.as_tensor(c0 + chunk)
    nb = (ctxs + BS - 1) // BS
    kp = torch.randn(int(nb.sum()), BS, hkv, d, generator=g).bfloat16()
    vp = torch.randn(int(nb.sum()), BS, hkv, d, generator=g).bfloat16()
    tab = torch.zeros(len(c0), int(nb.max()), dtype=torch.long)
    off = 0
    for i in range(len(c0)):
        tab[i, :nb[i]] = torch.arange(off, off + int(nb[i]))
        off += int(nb[i])
    q = torch.randn(len(c0) * chunk, hq, d, generator=g).bfloat16()
    qls = torch.full((len(c0),), chunk, dtype=torch.long)
    sec = med(lambda: paged_attention_gather(q, kp, vp, tab, ctxs, qls, d ** -0.5), 1)
    flops = hq * 4 * d * sum(chunk * int(x) + chunk * (chunk + 1) // 2 for x in c0)
    out["config4_prefill_bf16"] = {"TFLOP/s": round(flops / sec / 1e12, 4), "s": round(sec, 3),
                                   "sample": "8 of the 16 chunks (contexts c0 of every other one), median of 1"}
    del kp, vp, q

    # config 3 on 2 of the 32 layers: [16384, 16, 8, 128] bf16 per K and V tensor
    layers, nbk, h, d = 2, 16384, 8, 128
    ks = [torch.zeros(nbk, BS, h, d, dtype=torch.bfloat16) for _ in range(layers)]
    vs = [torch.zeros(nbk, BS, h, d, dtype=torch.bfloat16) for _ in range(layers)]
    slots = torch.randperm(nbk * BS, generator=g)[:256]
    rows = torch.randn(256, h, d, generator=g).bfloat16()

    def append():
        for t in ks + vs:
            t.view(-1, h, d).index_copy_(0, slots, rows)
    sec = med(lambda: [append() for _ in range(50)], 3) / 50
    nb_app = 2 * (2 * layers * 256 * h * d * 2) + 8 * 256
    out["config3_append_bf16"] = {"GB/s": round(nb_app / sec / 1e9, 3), "us_per_2_layers": round(sec * 1e6, 1),
                                  "sample": "256 rows into K and V of 2 layers, 50 x median of 3"}
    bperm = torch.randperm(nbk, generator=g)
    pairs = list(zip(bperm[:512].tolist(), bperm[512:1024].tolist()))

    def cow():
        for src, dst in pairs:
            for t in ks + vs:
                t[dst].copy_(t[src])
    sec = med(cow, 3)
    block = BS * h * d * 2
    nb_cow = 2 * 512 * 2 * layers * block
    out["config3_cow_bf16"] = {"GB/s": round(nb_cow / sec / 1e9, 3), "ms_per_2_layers": round(sec * 1e3, 2),
                               "sample": "512 pairs over K and V of 2 layers, one copy_ per block per tensor"}
    out_b, in_b = bperm[1024:2048], bperm[2048:3072]

    def swap():
        parked = [t.index_select(0, out_b) for t in ks + vs]
        for t, hcopy in zip(ks + vs, parked):
            t.index_copy_(0, in_b, hcopy)
    sec = med(swap, 3)
    nb_swap = 1024 * 2 * layers * block
    out["config3_swap_out_and_in_bf16"] = {"GB/s_each_way": round(2 * nb_swap / sec / 1e9, 3),
                                           "ms_per_2_layers": round(sec * 1e3, 2),
                                           "sample": "1024 blocks of K and V of 2 layers out and back"}
    return out


# ------------------------------------------------------------------ main
def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 500 steps (~0.2 s of decode): after the synchronisation that opens the timed region
    # the GPU takes tens of milliseconds to return to its loaded clocks, so a short region
    # understates the steady rate (config 4 decode: 5,530-5,560 GB/s over 50 steps,
    # 5,590-5,600 over 500, 5,604 with no synchronisation at all).
    ap.add_argument("--steps", type=int, default=500)
    # ~40 ms of untimed decode calls: from an idle GPU the first tens of calls run ~1.5%
    # slower while clocks ramp up.
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary kernel configs (2, 3, 4-prefill)")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end paged-engine run (config 5)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run 3 plain 1 GiB device-to-device copies (for scaling rocprofv3 --pmc "
                         "FETCH_SIZE / WRITE_SIZE by a kernel of known traffic)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}). Run with --gpus 1.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2

    from inference_server import native

    native.lib()
    log(f"device {torch.cuda.get_device_name(0)}")

    if args.calibrate_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration: 3 x 1 GiB device-to-device copies done (1073741824 B read + written each)")
        del src, dst

    log("config 4 decode: building inputs")
    w4 = config4_decode()
    call = w4.make_call()
    torch.cuda.synchronize()
    log(f"config 4 decode: {args.warmup} warmup + {args.steps} timed steps")
    total, kern_ms = time_region([call], args.steps, args.warmup)
    ms_step = total / args.steps * 1e3
    nbytes = w4.algorithmic_bytes
    value = nbytes / (total / args.steps) / 1e9
    _, ev_ms = time_steps([call], max(10, args.steps // 2), 2)      # per-launch spread
    achieved = nbytes / (kern_ms / 1e3) / 1e9
    log(f"config 4 decode: {ms_step:.3f} ms/step, {value:.1f} GB/s, kernel {kern_ms:.3f} ms -> {achieved:.1f} GB/s")

    # Parity of the timed output against the oracle, every row (after timing).
    worst = check_decode_whole(w4, w4.out)
    log(f"config 4 decode: all {w4.batch} output rows match the oracle (max |diff| {worst:.3g}, tolerance 2e-2)")

    traffic = pmc_traffic("void pkv::paged_decode_mfma_kernel<pkv::bf16_t, 128, 4, 8>")
    result = {
        "metric": "paged decode-attn GB/s (% of HBM peak); paged-engine output tok/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) Q/K/V, seeded contexts and block tables)",
        "config": {
            "workload": "BASELINE config 4 paged decode (Llama-3-8B-shaped single layer)",
            "batch": 128, "num_heads": 32, "num_kv_heads": 8, "head_dim": 128, "block_size": BS,
            "context_lens": "U[512, 8192] seeded 1337", "sum_context": w4.sum_ctx, "pool_blocks": 65536,
            "algorithmic_bytes_per_step": nbytes,
        },
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic["hbm_bytes"] if traffic else None,
            "traffic_detail": (dict(traffic, source="profiles/pmc_traffic.json", algorithmic_bytes=nbytes)
                               if traffic else None),
            # One timed step = one pkv_paged_attention_decode call: the persistent MFMA
            # kernel (the traffic above is its launch's) and its split-KV merge kernel
            # (~5 us; the pieces of the sequences cut by run boundaries). kernel_ms_mean:
            # HIP events around the timed region / steps, both launches included;
            # kernel_ms: spread of a second loop with per-step events (whose markers add
            # ~10 us per step).
            "kernel": "paged_decode_mfma_kernel<bf16_t,128,4,8> (persistent: one workgroup of 8 waves per CU, equal runs of 16-key blocks) + paged_decode_mfma_merge_kernel (split-KV pieces cut by run boundaries)",
            "kernel_ms_mean": round(kern_ms, 4),
            "kernel_ms": spread(ev_ms),
        },
    }

    result["parity"] = {"config4_decode_rows_checked": w4.batch, "oracle_max_abs_diff": round(worst, 5),
                        "tolerance": 2e-2, "oracle": "oracle.gather (the reference gather path restated)"}

    if not args.no_extra:
        log("config 2 decode (fp16, 4 rotating pools): building inputs")
        w2 = config2_decode(pools=4)
        calls2 = [w2.make_call(i) for i in range(4)]
        _, k2 = time_region(calls2, max(args.steps, 40), args.warmup)
        _, ev2 = time_steps(calls2, 40, 4)
        result["secondary"] = {
            "config2_decode_fp16": {
                "GB/s": round(w2.algorithmic_bytes / (k2 / 1e3) / 1e9, 2),
                "kernel_ms_mean": round(k2, 4),
                "kernel_ms": spread(ev2),
                "algorithmic_bytes": w2.algorithmic_bytes,
                "note": "64 seqs x 12 heads x d64, lognormal ctx (median 300, sigma 0.9); 4 pool copies rotated",
            }
        }
        log(f"config 2 decode: {k2:.4f} ms -> {result['secondary']['config2_decode_fp16']['GB/s']} GB/s")
        del w2, calls2
        torch.cuda.empty_cache()

        log("config 4 chunked prefill (bf16, MFMA): building inputs")
        wp = PrefillWorkload()
        # The MFMA kernel is more clock-sensitive than decode: after the synchronisation
        # that opens a timed region it runs ~20% slower for the first ~30 ms (0.40 ms per
        # call over 30 calls, 0.366 over 100, 0.335 in a continuous stream), so the timed
        # region is 300 calls after 100 untimed ones.
        _, kp_ms = time_region([wp.make_call()], 300, 100)
        _, evp = time_steps([wp.make_call()], 10, 2)
        tflops = wp.flops / (kp_ms / 1e3) / 1e12
        result["secondary"]["config4_chunked_prefill_bf16"] = {
            "TFLOP/s": round(tflops, 1),
            "kernel_ms_mean": round(kp_ms, 4),
            "kernel_ms": spread(evp),
            "causal_flops": wp.flops,
            "frac_of_mfma_peak": round(tflops / 2500.0, 4),
            "note": "16 seqs x 512-token chunks onto cached contexts U[0,4096]; 32/8 heads, d128",
        }
        log(f"config 4 prefill: {kp_ms:.4f} ms -> {tflops:.1f} TFLOP/s ({100 * tflops / 2500:.1f}% of 2.5 PF)")
        worst = check_prefill_whole(wp, wp.out)
        result["secondary"]["config4_chunked_prefill_bf16"]["oracle_max_abs_diff"] = round(worst, 5)
        log(f"config 4 prefill: all {wp.seqs} timed chunks match the oracle (max |diff| {worst:.3g}, tolerance 2e-2)")
        del wp
        torch.cuda.empty_cache()

        log("config 1 attention in fp32 (GPT-2 shape): prefill of its 8 prompts, one decode step")
        result["secondary"]["config1_attention_fp32"] = config1_fp32(max(args.steps, 100), args.warmup)
        log(f"config 1 fp32: {json.dumps(result['secondary']['config1_attention_fp32'])}")

        log("greedy sampling fused into the LM head (GPT-2 fp16 shape, 32 rows)")
        result["secondary"]["greedy_lm_head_fp16"] = greedy_lm_head(max(args.steps, 100), args.warmup)
        log(f"greedy: {json.dumps(result['secondary']['greedy_lm_head_fp16'])}")

        log("config 3 append / copy-on-write / swap (bf16, 32 layers x 16384 blocks)")
        result["secondary"]["config3_kvops_bf16"] = config3_kvops(args.steps)
        log(f"config 3: {json.dumps(result['secondary']['config3_kvops_bf16'])}")

    if not args.no_e2e:
        log("config 5 end-to-end paged engine (GPT-2 fp16, 200 requests)")
        result["paged_engine_output_tok_s"] = e2e_engine()
        log(f"config 5: {json.dumps(result['paged_engine_output_tok_s'])}")

    if not args.no_cpu:
        log("cpu baseline: oracle gather on a bounded sample")
        result["cpu_baseline"] = cpu_baseline(w4)
        log(f"cpu baseline: {result['cpu_baseline']['value']} GB/s on {result['cpu_baseline']['cores']} threads")
        if not args.no_extra:
            log("cpu legs: config 2 decode, config 4 prefill, config 3 append / COW / swap")
            result["cpu_baseline_legs"] = cpu_legs()
            log(f"cpu legs: {json.dumps(result['cpu_baseline_legs'])}")
    else:
        result["cpu_baseline"] = None

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
