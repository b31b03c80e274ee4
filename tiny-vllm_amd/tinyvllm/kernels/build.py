"""Compile the HIP sources under ``csrc/`` into ``libtinyvllm_hip.so`` (gfx950).

This is the in-tree build step (the reference JIT-builds its CUDA sources
with ``torch.utils.cpp_extension.load``, tinyvllm/kernels/_extension.py:11-42;
here the library is a plain C-ABI shared object built ahead of time with
hipcc, so it travels with the source tree and needs no compiler at run time).

Usage: ``python -m tinyvllm.kernels.build`` or ``build_library()``.
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR.parents[1] / "csrc"
INCLUDE_DIR = PACKAGE_DIR.parents[2] / "include"
LIBRARY_NAME = "libtinyvllm_hip.so"
LIBRARY_PATH = PACKAGE_DIR / LIBRARY_NAME
OFFLOAD_ARCH = "gfx950"

HIPCC_FLAGS = (
    "-O3",
    f"--offload-arch={OFFLOAD_ARCH}",
    "-fPIC",
    "-std=c++20",
    # Every product and sum is rounded where the source says (the pointwise
    # kernels restate PyTorch expressions); explicit fmaf() is still fused.
    "-ffp-contract=off",
    "-mcode-object-version=5",
    # Packed FP32 VALU ops are disabled for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
)


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    if candidate.exists():
        return str(candidate)
    found = shutil.which("hipcc")
    if found is None:
        raise RuntimeError("hipcc not found: set ROCM_PATH to a ROCm install")
    return found


def sources() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.hip"))


def source_hash() -> str:
    """Digest of every input of the library (kernels, headers, flags); the
    loader compares it with the one compiled into the library."""
    h = hashlib.sha256()
    files = sorted(CSRC_DIR.glob("*.hip")) + sorted(CSRC_DIR.glob("*.h")) + \
        sorted(INCLUDE_DIR.glob("*.h"))
    for f in files:
        h.update(f.name.encode())
        h.update(f.read_bytes())
    h.update(" ".join(HIPCC_FLAGS).encode())
    return h.hexdigest()[:16]


def build_library(*, jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every ``csrc/*.hip`` and link the shared library; returns its path."""
    hipcc = _hipcc()
    build_dir = PACKAGE_DIR.parents[1] / "_build"
    build_dir.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")

    digest = source_hash()

    def compile_one(src: Path) -> Path:
        obj = build_dir / (src.stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE_DIR}",
               f'-DTVLLM_SOURCE_HASH="{digest}"', "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
        return obj

    workers = jobs or min(8, len(srcs), os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(compile_one, srcs))

    tmp = LIBRARY_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC",
           *map(str, objects), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY_PATH)
    return LIBRARY_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
