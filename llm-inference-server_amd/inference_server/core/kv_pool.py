"""The physical KV pool: per-layer block-major K and V tensors, allocated once, and
the byte movers that work on them (append, block copy, swap).

Layout and API follow the reference's PagedKVPool (inference_server/core/kv_pool.py:
38-199): per layer `k[l], v[l]` of shape [num_blocks, block_size, num_kv_heads,
head_dim], so a block is one contiguous slab of block_size * Hkv * D elements.

Who moves the bytes depends on CONFIG.kv_backend:

* "torch" (ATTENTION=gather): the reference's own tensor ops — index_copy_ for
  append, per-layer copy_ for copy-on-write, index_select + pinned copy for swap.
* "hip" (ATTENTION=hip): libpagedkv kernels over a device table of the 2L layer
  base pointers, so each operation is ONE launch across every layer of K and V
  (the reference issues 2L torch calls per operation), and swap moves the whole
  victim through one pinned host buffer with a single DMA each way, that DMA on a
  side copy stream so the CPU never waits for it.

Host buffers of a swap are one pinned allocation [2L, n, block_size, Hkv, D];
HostBlocks.k / .v are per-layer views into it, the reference's HostBlocks shape.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from inference_server import native
from inference_server.config import CONFIG


@dataclass(frozen=True)
class ModelDims:
    """Sizes that decide a block's footprint (reference: core/kv_pool.py:37-79)."""

    num_layers: int
    num_kv_heads: int
    head_dim: int
    dtype: torch.dtype

    @classmethod
    def from_model(cls, model, dtype: torch.dtype | None = None) -> "ModelDims":
        cfg = model.config
        heads = getattr(cfg, "num_attention_heads", None) or cfg.n_head
        hidden = getattr(cfg, "hidden_size", None) or cfg.n_embd
        return cls(
            num_layers=getattr(cfg, "num_hidden_layers", None) or cfg.n_layer,
            num_kv_heads=getattr(cfg, "num_key_value_heads", None) or heads,
            head_dim=getattr(cfg, "head_dim", None) or hidden // heads,
            dtype=dtype or CONFIG.torch_dtype,
        )

    @property
    def itemsize(self) -> int:
        return torch.empty(0, dtype=self.dtype).element_size()

    def bytes_per_token(self) -> int:
        """K and V, every layer: 2 * L * Hkv * D * itemsize."""
        return 2 * self.num_layers * self.num_kv_heads * self.head_dim * self.itemsize

    def bytes_per_block(self, block_size: int = CONFIG.block_size) -> int:
        return self.bytes_per_token() * block_size

    def blocks_for_budget(self, budget_bytes: int, block_size: int = CONFIG.block_size) -> int:
        """Blocks that fit in a byte budget, rounded down."""
        return max(0, budget_bytes // self.bytes_per_block(block_size))


class HostBlocks:
    """A swapped-out sequence's blocks in host memory (reference: core/kv_pool.py:82-103).
    k[l] / v[l] are [n, block_size, Hkv, D]. `packed`, when set, is the single pinned
    buffer [2L, n, ...] the views live in (what the hip swap-in DMAs back).

    `ready`, when set, is the event that completes the device->host copy. Reading
    .k / .v waits for it, so a host reader always sees the whole copy (the reference's
    swap_out returns only after its copies); swap_in never waits on the CPU — it
    orders its host->device copy after `ready` on the GPU."""

    def __init__(self, k: list[torch.Tensor], v: list[torch.Tensor],
                 packed: torch.Tensor | None = None, ready: torch.cuda.Event | None = None) -> None:
        self._k = k
        self._v = v
        self.packed = packed
        self.ready = ready

    def wait(self) -> "HostBlocks":
        """Block the calling thread until the device->host copy has landed."""
        if self.ready is not None:
            self.ready.synchronize()
            self.ready = None
        return self

    @property
    def k(self) -> list[torch.Tensor]:
        return self.wait()._k

    @property
    def v(self) -> list[torch.Tensor]:
        return self.wait()._v

    def __len__(self) -> int:
        return int(self._k[0].shape[0]) if self._k else 0

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self._k + self._v)

    def __repr__(self) -> str:
        state = "in flight" if self.ready is not None and not self.ready.query() else "landed"
        return f"HostBlocks({len(self)} blocks x {2 * len(self._k)} layer tensors, {self.nbytes} B, {state})"


class PagedKVPool:
    """The preallocated blocks (reference: core/kv_pool.py:106-199)."""

    def __init__(
        self,
        dims: ModelDims,
        num_blocks: int = CONFIG.num_blocks,
        block_size: int = CONFIG.block_size,
        device: str = CONFIG.device,
    ) -> None:
        self.dims = dims
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.device = device
        shape = (num_blocks, block_size, dims.num_kv_heads, dims.head_dim)
        self.k = [torch.zeros(shape, dtype=dims.dtype, device=device) for _ in range(dims.num_layers)]
        self.v = [torch.zeros(shape, dtype=dims.dtype, device=device) for _ in range(dims.num_layers)]
        self._ptr_table: torch.Tensor | None = None
        # Side stream for the PCIe halves of a swap (default priority, made on first use).
        self._copy: torch.cuda.Stream | None = None

    @classmethod
    def from_model(cls, model, **kwargs) -> "PagedKVPool":
        return cls(ModelDims.from_model(model), **kwargs)

    @property
    def num_slots(self) -> int:
        return self.num_blocks * self.block_size

    @property
    def nbytes(self) -> int:
        return self.num_blocks * self.dims.bytes_per_block(self.block_size)

    @property
    def block_bytes(self) -> int:
        """Bytes of one block of ONE layer's K (or V)."""
        return self.block_size * self.dims.num_kv_heads * self.dims.head_dim * self.dims.itemsize

    # ------------------------------------------------------------ hip plumbing
    def _use_hip(self) -> bool:
        if CONFIG.kv_backend != "hip":
            return False
        if torch.device(self.device).type != "cuda":
            raise NotImplementedError(f"ATTENTION=hip: the KV pool must live on a ROCm GPU, not {self.device}")
        native.lib()
        return True

    def pointer_table(self) -> torch.Tensor:
        """Device int64 [2L]: base addresses of k[0..L-1] then v[0..L-1]."""
        if self._ptr_table is None:
            ptrs = [t.data_ptr() for t in self.k + self.v]
            self._ptr_table = torch.tensor(ptrs, dtype=torch.int64, device=self.device)
        return self._ptr_table

    def _stream(self) -> int:
        return native.stream_handle(torch.device(self.device))

    def _copy_stream(self) -> torch.cuda.Stream:
        if self._copy is None:
            self._copy = torch.cuda.Stream(device=torch.device(self.device))
        return self._copy

    def _index(self, blocks: list[int]) -> torch.Tensor:
        idx = torch.as_tensor(blocks, dtype=torch.long)
        if idx.numel() and (int(idx.min()) < 0 or int(idx.max()) >= self.num_blocks):
            raise IndexError(f"block index outside [0, {self.num_blocks})")
        if torch.device(self.device).type == "cuda":
            # A pageable upload would drain the current stream first; a pinned one does not.
            return idx.pin_memory().to(self.device, non_blocking=True)
        return idx.to(self.device)

    # ------------------------------------------------------------ append
    def check_slots(self, slots: torch.Tensor, host_slots: torch.Tensor | None = None) -> None:
        """IndexError unless every slot is in [0, num_slots). The executor passes one
        slots tensor (with its host copy) to every layer of a step: the check runs once
        per host copy, not once per layer."""
        key = (id(host_slots), self.num_slots)
        if host_slots is None or getattr(slots, "_pkv_slots_checked", None) != key:
            hs = host_slots if host_slots is not None else slots.cpu()
            if hs.numel() and (int(hs.min()) < 0 or int(hs.max()) >= self.num_slots):
                raise IndexError(f"slot index outside [0, {self.num_slots})")
            if host_slots is not None:
                setattr(slots, "_pkv_slots_checked", key)

    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor, slots: torch.Tensor,
               host_slots: torch.Tensor | None = None) -> None:
        """Write rows k/v [T, Hkv, D] (any strides with a unit last stride) into flat
        slots (reference: core/paged_executor.py:116-125). `host_slots`, the same
        values on the CPU, lets the hip path range-check without a device sync."""
        if not self._use_hip():
            H, D = k.shape[1], k.shape[2]
            self.k[layer].view(-1, H, D).index_copy_(0, slots, k)
            self.v[layer].view(-1, H, D).index_copy_(0, slots, v)
            return
        n_tok = k.shape[0]
        if n_tok == 0:
            return
        if k.shape != v.shape or k.shape[1:] != self.k[layer].shape[2:]:
            raise ValueError(f"append rows {tuple(k.shape)} do not match pool rows {tuple(self.k[layer].shape[2:])}")
        if slots.shape != (n_tok,):
            raise ValueError(f"slots must be [{n_tok}], got {tuple(slots.shape)}")
        self.check_slots(slots, host_slots)
        # One stride pair describes both sources (the executor's K and V views share it).
        if k.stride(2) != 1 or v.stride() != k.stride():
            k, v = k.contiguous(), v.contiguous()
        kp, vp = self.k[layer], self.v[layer]
        slots = slots.to(device=self.device, dtype=torch.long)
        rc = native.lib().pkv_kv_append(
            kp.data_ptr(), vp.data_ptr(), kp.stride(0), kp.stride(1), kp.stride(2),
            self.num_blocks, self.block_size, kp.shape[2], kp.shape[3],
            k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
            slots.data_ptr(), n_tok, native.dtype_code(kp.dtype),
            self._stream(),
        )
        native.check(rc, "pkv_kv_append")

    # ------------------------------------------------------------ copy-on-write
    def copy_block(self, src: int, dst: int) -> None:
        """Copy one block, every layer of K and V (reference: core/paged_executor.py:265-270)."""
        self.copy_blocks([(src, dst)])

    def copy_blocks(self, pairs: list[tuple[int, int]]) -> None:
        """Copy many (src, dst) blocks in one launch. The pairs run concurrently, so a
        dst may not repeat and may not be any pair's src (ValueError, nothing copied):
        the torch backend's sequential copies would otherwise give another result."""
        if not pairs:
            return
        srcs = {src for src, _ in pairs}
        dsts = [dst for _, dst in pairs]
        if len(set(dsts)) != len(dsts):
            raise ValueError(f"copy_blocks: a destination block repeats in {pairs}")
        if srcs.intersection(dsts):
            raise ValueError(f"copy_blocks: block(s) {sorted(srcs.intersection(dsts))} are both a source and a "
                             "destination")
        if not self._use_hip():
            for src, dst in pairs:
                for layer in self.k:
                    layer[dst].copy_(layer[src])
                for layer in self.v:
                    layer[dst].copy_(layer[src])
            return
        flat = self._index([b for pair in pairs for b in pair])
        rc = native.lib().pkv_copy_blocks(
            self.pointer_table().data_ptr(), 2 * self.dims.num_layers, self.num_blocks, self.block_bytes,
            flat.data_ptr(), len(pairs), self._stream(),
        )
        native.check(rc, "pkv_copy_blocks")

    # ------------------------------------------------------------ swap
    def swap_out(self, blocks: list[int]) -> HostBlocks:
        """Copy the named blocks to host memory; the caller frees them afterwards
        (reference: core/kv_pool.py:142-166). Does not touch the allocator.

        torch backend: the host copy is complete when this returns. hip backend: the
        gather into a device staging buffer runs on the current stream, so any later
        write into the freed blocks is ordered after it; the PCIe copy runs on the
        pool's copy stream and overlaps whatever the current stream does next. The
        returned HostBlocks waits for it when its .k / .v are read."""
        if not self._use_hip():
            idx = torch.as_tensor(blocks, dtype=torch.long, device=self.device)
            pin = torch.device(self.device).type == "cuda"

            def to_host(layer: torch.Tensor) -> torch.Tensor:
                gathered = layer.index_select(0, idx)
                host = torch.empty(gathered.shape, dtype=gathered.dtype, device="cpu", pin_memory=pin)
                host.copy_(gathered)
                return host

            return HostBlocks(k=[to_host(t) for t in self.k], v=[to_host(t) for t in self.v])

        L, n = self.dims.num_layers, len(blocks)
        shape = (2 * L, n, self.block_size, self.dims.num_kv_heads, self.dims.head_dim)
        packed = torch.empty(shape, dtype=self.dims.dtype, pin_memory=True)
        if n == 0:
            return HostBlocks(k=list(packed[:L]), v=list(packed[L:]), packed=packed)
        idx = self._index(blocks)
        staging = torch.empty(shape, dtype=self.dims.dtype, device=self.device)
        rc = native.lib().pkv_gather_blocks(
            self.pointer_table().data_ptr(), 2 * L, self.num_blocks, self.block_bytes,
            idx.data_ptr(), n, staging.data_ptr(), self._stream(),
        )
        native.check(rc, "pkv_gather_blocks")
        compute = torch.cuda.current_stream(torch.device(self.device))
        copy = self._copy_stream()
        copy.wait_stream(compute)
        with torch.cuda.stream(copy):
            packed.copy_(staging, non_blocking=True)
        # staging belongs to the current stream's pool; keep it until the copy stream is done.
        staging.record_stream(copy)
        ready = torch.cuda.Event()
        ready.record(copy)
        return HostBlocks(k=list(packed[:L]), v=list(packed[L:]), packed=packed, ready=ready)

    def swap_in(self, host: HostBlocks, blocks: list[int]) -> None:
        """Copy a host copy back into `blocks`, which need not be the ones it left
        (reference: core/kv_pool.py:168-182). Lengths must match exactly.

        hip backend: the PCIe copy runs on the pool's copy stream (after the host
        copy's own `ready` event), and the scatter into `blocks` on the current stream
        after it, so work queued on the current stream sees the restored blocks and the
        CPU never waits."""
        if len(blocks) != len(host):
            raise ValueError(f"swap_in: {len(host)} host blocks into {len(blocks)} device blocks")
        if not self._use_hip():
            idx = torch.as_tensor(blocks, dtype=torch.long, device=self.device)
            non_blocking = torch.device(self.device).type == "cuda"
            for dst, src in zip(self.k, host.k):
                dst.index_copy_(0, idx, src.to(self.device, non_blocking=non_blocking))
            for dst, src in zip(self.v, host.v):
                dst.index_copy_(0, idx, src.to(self.device, non_blocking=non_blocking))
            return
        n = len(blocks)
        if n == 0:
            return
        packed = host.packed
        if packed is None or not packed.is_pinned() or not packed.is_contiguous():
            packed = torch.stack(host.k + host.v).contiguous().pin_memory()
        expect = (2 * self.dims.num_layers, n, self.block_size, self.dims.num_kv_heads, self.dims.head_dim)
        if tuple(packed.shape) != expect or packed.dtype != self.dims.dtype:
            raise ValueError(f"swap_in: host blocks {tuple(packed.shape)} {packed.dtype} do not fit pool {expect}")
        idx = self._index(blocks)
        # Allocated on the current stream: the copy stream first catches up with it, so
        # the staging memory is free by the time the PCIe copy writes it.
        staging = torch.empty(packed.shape, dtype=packed.dtype, device=self.device)
        compute = torch.cuda.current_stream(torch.device(self.device))
        copy = self._copy_stream()
        copy.wait_stream(compute)
        if host.ready is not None:
            copy.wait_event(host.ready)
        with torch.cuda.stream(copy):
            staging.copy_(packed, non_blocking=True)
        landed = torch.cuda.Event()
        landed.record(copy)
        compute.wait_event(landed)
        rc = native.lib().pkv_scatter_blocks(
            self.pointer_table().data_ptr(), 2 * self.dims.num_layers, self.num_blocks, self.block_bytes,
            idx.data_ptr(), n, staging.data_ptr(), self._stream(),
        )
        native.check(rc, "pkv_scatter_blocks")

    # ------------------------------------------------------------ lifetime
    def release(self) -> None:
        """Drop the tensors; sizes stay readable (reference: core/kv_pool.py:184-189)."""
        if self._copy is not None:
            self._copy.synchronize()
            self._copy = None
        self.k = []
        self.v = []
        self._ptr_table = None

    def describe(self) -> str:
        gib = self.nbytes / 1024**3
        return (
            f"{self.num_blocks} blocks x {self.block_size} tokens = {self.num_slots} slots, "
            f"{gib:.2f} GiB on {self.device} ({self.dims.num_layers}L "
            f"x {self.dims.num_kv_heads}H x {self.dims.head_dim}D, {self.dims.dtype})"
        )

    def __repr__(self) -> str:
        return f"PagedKVPool({self.describe()})"
