"""ctypes binding of libpagedkv.so (the C ABI declared in include/pagedkv.h).

`lib()` loads the in-tree library once and raises NotImplementedError when it is
missing or its ABI version differs: the HIP path never falls back to anything else.
`check(rc)` turns a non-zero return into RuntimeError carrying `pkv_last_error()`.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libpagedkv.so"
ABI_VERSION = 1

PKV_FLOAT32, PKV_FLOAT16, PKV_BFLOAT16 = 0, 1, 2
DTYPE_CODES = {torch.float32: PKV_FLOAT32, torch.float16: PKV_FLOAT16, torch.bfloat16: PKV_BFLOAT16}

PKV_OK, PKV_EINVAL, PKV_EUNSUPPORTED, PKV_EWORKSPACE, PKV_EHIP = 0, 1, 2, 3, 4
#: include/pagedkv.h PKV_DECODE_SCRATCH_BYTES: the no-alloc decode entry's static scratch.
DECODE_SCRATCH_BYTES = 96 * 1024 * 1024

_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p
_f32 = ctypes.c_float

# Every exported symbol with its (restype, argtypes); the loader binds all of them and
# the CPU test suite checks that each one exists.
SIGNATURES: dict[str, tuple] = {
    "pkv_abi_version": (_int, []),
    "pkv_last_error": (ctypes.c_char_p, []),
    "pkv_graph_node_counts": (_int, [_ptr, _ptr, _i64]),
    "pkv_paged_attention_decode_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "pkv_paged_attention_decode": (
        _int,
        [_ptr, _i64, _i64,                 # out, strides
         _ptr, _i64, _i64,                 # query, strides
         _ptr, _ptr, _i64, _i64, _i64,     # k_pool, v_pool, pool strides
         _i64, _i64, _i64, _i64,           # num_blocks, block_size, num_kv_heads, head_dim
         _ptr, _i64, _i64,                 # block_tables, table_stride, table_width
         _ptr,                             # context_lens
         _i64, _i64, _i64,                 # num_seqs, num_heads, max_context_len
         _f32, _int,                       # scale, dtype
         _ptr, _i64,                       # workspace, workspace_bytes
         _ptr],                            # stream
    ),
    "pkv_paged_attention_decode_append": (
        _int,
        [_ptr, _i64, _i64,                 # out, strides
         _ptr, _i64, _i64,                 # query, strides
         _ptr, _ptr, _i64, _i64, _i64,     # k_pool, v_pool, pool strides
         _i64, _i64, _i64, _i64,           # num_blocks, block_size, num_kv_heads, head_dim
         _ptr, _ptr, _i64, _i64, _ptr,     # k_new, v_new, new strides (t, h), slots
         _ptr, _i64, _i64,                 # block_tables, table_stride, table_width
         _ptr,                             # context_lens
         _i64, _i64, _i64,                 # num_seqs, num_heads, max_context_len
         _f32, _int,                       # scale, dtype
         _ptr, _i64,                       # workspace, workspace_bytes
         _ptr],                            # stream
    ),
    "pkv_paged_attention_decode_noalloc": (
        _int,
        [_ptr, _i64, _i64,                 # out, strides
         _ptr, _i64, _i64,                 # query, strides
         _ptr, _ptr, _i64, _i64, _i64,     # k_pool, v_pool, pool strides
         _i64, _i64, _i64, _i64,           # num_blocks, block_size, num_kv_heads, head_dim
         _ptr, _i64, _i64,                 # block_tables, table_stride, table_width
         _ptr,                             # context_lens
         _i64, _i64, _i64,                 # num_seqs, num_heads, max_context_len
         _f32, _int,                       # scale, dtype
         _ptr],                            # stream (no workspace: the library's static scratch)
    ),
    "pkv_paged_attention_prefill": (
        _int,
        [_ptr, _i64, _i64,
         _ptr, _i64, _i64,
         _ptr, _ptr, _i64, _i64, _i64,
         _i64, _i64, _i64, _i64,
         _ptr, _i64, _i64,
         _ptr, _ptr,                       # context_lens, query_start_loc
         _i64, _i64, _i64, _i64,           # num_seqs, num_heads, num_tokens, max_query_len
         _f32, _int,
         _ptr],
    ),
    "pkv_paged_attention_prefill_append": (
        _int,
        [_ptr, _i64, _i64,
         _ptr, _i64, _i64,
         _ptr, _ptr, _i64, _i64, _i64,
         _i64, _i64, _i64, _i64,
         _ptr, _ptr, _i64, _i64, _ptr,     # k_new, v_new, new strides (t, h), slots
         _ptr, _i64, _i64,
         _ptr, _ptr,                       # context_lens, query_start_loc
         _i64, _i64, _i64, _i64,           # num_seqs, num_heads, num_tokens, max_query_len
         _f32, _int,
         _ptr],
    ),
    "pkv_kv_append": (
        _int,
        [_ptr, _ptr, _i64, _i64, _i64,     # k_pool, v_pool, pool strides
         _i64, _i64, _i64, _i64,           # num_blocks, block_size, num_kv_heads, head_dim
         _ptr, _ptr, _i64, _i64,           # k_new, v_new, new strides (t, h)
         _ptr, _i64, _int,                 # slots, num_tokens, dtype
         _ptr],
    ),
    "pkv_qkv_append": (
        _int,
        [_ptr, _i64, _ptr, _i64, _ptr,     # x, x_stride, weight_t, weight_stride, bias
         _i64, _i64, _i64, _i64, _i64,     # num_rows, in_features, q_features, num_kv_heads, head_dim
         _ptr, _i64,                       # out, out_stride
         _ptr, _ptr, _i64, _i64, _i64,     # k_pool, v_pool, pool strides
         _i64, _i64, _ptr, _int,           # num_blocks, block_size, slots, dtype
         _ptr],
    ),
    "pkv_kv_append_layers": (
        _int,
        [_ptr, _ptr, _i64,                 # k_pools, v_pools (device tables), num_layers
         _i64, _i64, _i64, _i64,
         _ptr, _ptr, _i64, _i64, _i64,     # k_new, v_new, strides (layer, t, h)
         _ptr, _i64, _int,
         _ptr],
    ),
    "pkv_copy_blocks": (_int, [_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr]),
    "pkv_gather_blocks": (_int, [_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr, _ptr]),
    "pkv_scatter_blocks": (_int, [_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr, _ptr]),
    "pkv_swap_out": (_int, [_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr, _ptr, _ptr]),
    "pkv_swap_in": (_int, [_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr, _ptr, _ptr]),
    "pkv_lm_head_argmax_workspace_bytes": (_i64, [_i64, _i64]),
    "pkv_lm_head_argmax": (
        _int,
        [_ptr, _i64, _ptr, _i64,           # hidden, stride, weight, stride
         _i64, _i64, _i64, _int,           # num_rows, hidden_size, vocab_size, dtype
         _ptr, _ptr, _i64,                 # out_ids, workspace, workspace_bytes
         _ptr],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load_library(path: Path | str = LIB_PATH) -> ctypes.CDLL:
    """dlopen the library and bind every signature. No GPU is touched."""
    handle = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return handle


def lib() -> ctypes.CDLL:
    """The loaded library; NotImplementedError (never a fallback) if it cannot be."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NotImplementedError(
                    f"ATTENTION=hip: {LIB_PATH.name} is not built ({LIB_PATH}); "
                    "run `python -c 'import __graft_entry__ as g; g.build()'` on a ROCm box"
                )
            handle = load_library()
            version = handle.pkv_abi_version()
            if version != ABI_VERSION:
                raise NotImplementedError(f"{LIB_PATH.name} has ABI {version}, this binding expects {ABI_VERSION}")
            _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != PKV_OK:
        msg = lib().pkv_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (pkv status {rc}): {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise NotImplementedError(f"ATTENTION=hip: no kernel for dtype {dtype}") from None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The current HIP stream of `device` as an integer handle. Uses torch's raw-stream
    accessor when present (it skips building a Stream object, ~10 us per call on the
    per-layer path), else the public API; both return the same handle."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(t: torch.Tensor, what: str) -> None:
    """The HIP path runs on a ROCm device or not at all."""
    if t.device.type != "cuda":
        raise NotImplementedError(
            f"ATTENTION=hip: {what} needs a ROCm GPU tensor, got device {t.device}; use ATTENTION=gather on cpu"
        )
    lib()
