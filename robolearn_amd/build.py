"""Build the MI355X learner library (librl_mi355x.so) with hipcc for gfx950.

The library is built in-tree so that it travels with the source snapshot.
``build()`` always recompiles; ``library_path()`` only locates the result.
"""

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE / "csrc"
BUILD_DIR = PACKAGE / "_build"
LIBRARY = PACKAGE / "librl_mi355x.so"
SOURCES = ("plan.hip", "gemm.hip", "gemm_bf16.hip", "gemm_bf16_big.hip", "optimizer.hip", "norm.hip", "categorical.hip", "policy.hip", "ppo.hip", "replay.hip")
ARCH = os.environ.get("ROBOLEARN_AMD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-result",
    # Packed fp32 VALU forms are disabled on this platform.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    path = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc was not found; set HIPCC or install ROCm.")
    return path


def library_path() -> Path:
    return LIBRARY


def _compile(source: str) -> Path:
    output = BUILD_DIR / (Path(source).stem + ".o")
    command = [hipcc(), *FLAGS, "-c", str(SOURCE_DIR / source), "-o", str(output)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source}:\n{result.stderr[-6000:]}")
    return output


def build(jobs: int | None = None) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    workers = jobs or min(len(SOURCES), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(_compile, SOURCES))
    temporary = LIBRARY.with_suffix(".so.tmp")
    command = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(temporary), *map(str, objects)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc link failed:\n{result.stderr[-6000:]}")
    os.replace(temporary, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
