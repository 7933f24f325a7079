"""Builds liblsrm_hip.so (the gfx950 kernels and their C ABI) in-tree.

Each ``csrc/*.hip`` file is compiled with hipcc for gfx950 into ``_build/``
and the objects are linked into ``lsrm_hip/liblsrm_hip.so`` next to this
file.  Usage: ``python -m lsrm_hip.build`` from the package directory, or
``build()`` from Python.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent            # .../lsrm_hip
ROOT = PKG_DIR.parent                                # package root
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
BUILD_DIR = ROOT / "_build"
LIB_NAME = "liblsrm_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

# Packed fp32 VALU forms are disabled: the compiler would otherwise form
# v_pk_{add,mul,fma}_f32 from plain float code.  MFMA results are kept in
# ordinary VGPRs (gfx950 reads and writes MFMA operands from the unified
# register file); the AGPR form made the compiler copy every score and output
# accumulator between register files on each key tile.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build liblsrm_hip.so")


def _compile(src: Path, obj: Path, extra: list[str]) -> None:
    cmd = [hipcc(), *HIP_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")


def build(verbose: bool = False, jobs: int | None = None, extra: list[str] | None = None) -> Path:
    """Compiles every csrc/*.hip for gfx950 and links liblsrm_hip.so."""
    extra = list(extra or [])
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [BUILD_DIR / (s.stem + ".o") for s in sources]
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 4)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, s, o, extra) for s, o in zip(sources, objs)]
        for f in futs:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True, extra=sys.argv[1:])
