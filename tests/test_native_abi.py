"""libpagedkv.so loads on the CPU, exports every function include/pagedkv.h declares,
and its ctypes binding covers exactly that set. No kernel is launched here."""

from __future__ import annotations

import re
from pathlib import Path

import pytest

from inference_server import native

HEADER = Path(__file__).resolve().parents[1] / "include" / "pagedkv.h"


def declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(pkv_[a-z0-9_]+)\s*\(", text))


def test_header_declares_the_abi():
    names = declared_functions()
    assert {"pkv_abi_version", "pkv_last_error", "pkv_paged_attention_decode", "pkv_paged_attention_prefill",
            "pkv_kv_append", "pkv_kv_append_layers", "pkv_copy_blocks", "pkv_swap_out", "pkv_swap_in",
            "pkv_gather_blocks", "pkv_scatter_blocks"} <= names


def test_binding_matches_header():
    assert set(native.SIGNATURES) == declared_functions()


def test_library_loads_and_exports_every_symbol():
    if not native.LIB_PATH.exists():
        pytest.fail(f"{native.LIB_PATH} is not built; run __graft_entry__.build()")
    handle = native.load_library()
    for name in declared_functions():
        assert hasattr(handle, name), name
    assert handle.pkv_abi_version() == native.ABI_VERSION
    assert handle.pkv_last_error() == b""


def test_decode_workspace_size_is_host_arithmetic():
    """256 KiB of merge counters plus partials for ceil(ctx / 256) partitions per
    (seq, head); nothing when one partition covers every context."""
    handle = native.load_library()
    b, h, kv, d = 128, 32, 8, 128
    parts = -(-8192 // 256)  # 256-token split-KV partitions
    counters = 256 * 1024  # merge counters at the front, a fixed size
    want = counters + -(-(b * h * parts * 2 * 4) // 256) * 256 + -(-(b * h * parts * d * 4) // 256) * 256
    assert handle.pkv_paged_attention_decode_workspace_bytes(b, h, kv, d, 8192) == want
    assert handle.pkv_paged_attention_decode_workspace_bytes(4, 4, 4, 64, 100) == 0
    assert handle.pkv_paged_attention_decode_workspace_bytes(4, 0, 4, 64, 100) == 0
