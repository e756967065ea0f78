"""Build libpagedkv.so from the HIP sources with hipcc for gfx950.

Run as `python -m inference_server.native.build` (with llm-inference-server_amd on
sys.path) or through `__graft_entry__.build()`. Every call recompiles: object files go
to a temporary directory, the shared library is written next to this file and swapped
in atomically, so a process that already loaded the old one is unaffected.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG_ROOT = HERE.parents[1]                  # llm-inference-server_amd/
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
INCLUDE = REPO_ROOT / "include"
LIB_NAME = "libpagedkv.so"
LIB_PATH = HERE / LIB_NAME
ARCH = os.environ.get("PKV_OFFLOAD_ARCH", "gfx950")

# Packed-fp32 VALU ops are disabled for all device code (-packed-fp32-ops): the
# kernels must not depend on v_pk_{add,mul,fma}_f32. The host pass warns that it
# does not know the feature; that is expected.
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build libpagedkv")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip and link libpagedkv.so. Returns the library path."""
    cc = hipcc()
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with tempfile.TemporaryDirectory(prefix="pkv_build_") as tmp:
        tmpdir = Path(tmp)

        def compile_one(src: Path) -> Path:
            obj = tmpdir / (src.stem + ".o")
            cmd = [cc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
            res = subprocess.run(cmd, capture_output=True, text=True)
            if res.returncode != 0:
                raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr[-6000:]}")
            if verbose and res.stderr.strip():
                print(res.stderr)
            return obj

        workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
        with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
            objs = list(pool.map(compile_one, srcs))
        tmp_lib = tmpdir / LIB_NAME
        cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp_lib)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link of {LIB_NAME} failed:\n{res.stderr[-6000:]}")
        staged = HERE / (LIB_NAME + ".tmp")
        shutil.copyfile(tmp_lib, staged)
        os.replace(staged, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
