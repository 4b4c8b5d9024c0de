"""Builds liblsa_rocm.so (the HIP kernels + C ABI) for gfx950, in-tree.

    python latent-sparse-attention-rocm_amd/build_lib.py

Each source compiles to its own object under ``_build/`` (in parallel), then one
shared library lands at ``lsa_rocm_lab/_lib/liblsa_rocm.so`` next to the Python
package that loads it.
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "lsa_rocm_lab" / "_lib" / "liblsa_rocm.so"
SOURCES = ["lsa_abi.cpp", "select.hip", "beam.hip", "read.hip", "read_prefill.hip", "decode.hip", "decode_bf16.hip",
           "decode_f16.hip", "decode_f32.hip", "decode_noalloc.hip", "decode_shared.hip", "decode_tree_shared.hip",
           "build.hip"]
ARCH = os.environ.get("LSA_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise FileNotFoundError("hipcc not found (ROCm is required to build the HIP kernels)")


def flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        # packed fp32 VALU ops stay off: ordinary float code only
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{ROOT / 'include'}", f"-I{CSRC}",
    ]


def _compile(src: str) -> pathlib.Path:
    obj = BUILD / (src + ".o")
    cmd = [hipcc(), *flags(), "-c", str(CSRC / src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        noise = "is not a recognized feature for this target"
        err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj


def build(jobs: int | None = None) -> pathlib.Path:
    """Compiles every source and links the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    LIB.parent.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(int(sys.argv[1]) if len(sys.argv) > 1 else None))
