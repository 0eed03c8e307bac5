"""Build libglm_moe.so (the HIP kernels + C ABI) in-tree for gfx950.

    python glm-tpu_amd/build.py

Each ``csrc/*.hip`` is compiled to an object under ``glm-tpu_amd/_build`` and
linked with hipcc into ``glm-tpu_amd/glm_moe/libglm_moe.so``.  Packed-FP32
instruction selection is switched off (``-packed-fp32-ops``) for every HIP
file; hipcc's host pass warns that it does not know that feature, which is
harmless.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
BUILD = ROOT / "_build"
LIB = ROOT / "glm_moe" / "libglm_moe.so"
INCLUDE = ROOT.parent / "include"
ARCH = os.environ.get("GLM_MOE_ARCH", "gfx950")


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (ROCm is required to build libglm_moe.so)")


COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, f"-I{INCLUDE}", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)"
    messages = [line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line and line.strip()]
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n" + "\n".join(messages))
    if messages:
        print("\n".join(messages), file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, int(os.environ.get("MAX_JOBS", "8"))))
    with cf.ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    # roctx: each launch's shape-suffixed profiler name (rocprofv3 --kernel-rename)
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-lrocprofiler-sdk-roctx",
           "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("link failed:\n" + proc.stdout + proc.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB.relative_to(ROOT.parent)} from {len(sources)} sources for {ARCH}")
    return LIB


if __name__ == "__main__":
    build()
