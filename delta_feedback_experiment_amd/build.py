"""Build ``libpkda_gfx950.so`` from ``csrc/*.hip`` for gfx950, in-tree.

    python -m delta_feedback_experiment_amd.build

Each source compiles with ``hipcc --offload-arch=gfx950`` to an object; the
objects link with the host compiler into one shared library.  The library is
linked against the HIP runtime that PyTorch itself loads (``torch/lib``), so
a process that uses both sees one runtime, one device context and one set of
streams.  Packed FP32 instructions are disabled for every kernel.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = ROOT / "_build"
LIB_DIR = PKG / "lib"
LIB_NAME = "libpkda_gfx950.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-std=c++17",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the PKDA library needs ROCm's hipcc")
    return path


def _hip_runtime() -> Path:
    """The ``libamdhip64.so`` that ``import torch`` loads (falls back to ROCm's)."""
    try:
        import torch

        cand = Path(torch.__file__).resolve().parent / "lib" / "libamdhip64.so"
        if cand.exists():
            return cand
    except ImportError:
        pass
    for cand in (Path("/opt/rocm/lib/libamdhip64.so"),):
        if cand.exists():
            return cand
    raise RuntimeError("no libamdhip64.so found to link against")


def library_path() -> Path:
    return LIB_DIR / LIB_NAME


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every ``csrc/*.hip`` and link the shared library; return its path."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    BUILD.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    hipcc = _hipcc()
    headers = sorted(CSRC.glob("*.h")) + sorted(INCLUDE.glob("*.h"))

    def compile_one(src: Path) -> Path:
        obj = BUILD / (src.stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
        return obj

    del headers  # every call rebuilds; the dependency scan is not worth its bugs
    jobs = jobs or min(8, len(sources), os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(compile_one, sources))
    runtime = _hip_runtime()
    out = library_path()
    tmp = out.with_suffix(".so.tmp")
    cmd = ["g++", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects), str(runtime),
           f"-Wl,-rpath,{runtime.parent}", "-Wl,--no-undefined"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
