"""Builds the gfx950 HIP library ``sonic_sampler/_lib/libsonic_sampler.so`` with hipcc.

Usage: ``python sonic-sampler_amd/build_native.py`` (also called by ``__graft_entry__.build``).
The library exports the C-ABI declared in ``include/sonic_sampler.h``. Objects go to ``_build/``
next to this file; every call recompiles every source.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
OUT = HERE / "sonic_sampler" / "_lib" / "libsonic_sampler.so"

ARCH = os.environ.get("SS_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # no packed fp32 VALU instructions (v_pk_{add,mul,fma}_f32) anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # kernarg preload: the leading scalar arguments of a kernel (up to 16 dwords) arrive in SGPRs
    # at wave launch, so its first loads need not wait for a kernarg-segment read. Each kernel
    # takes the fields its first loads use as leading scalars ahead of the argument struct, which
    # is passed by reference in the kernarg segment and is never preloaded.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build sonic_sampler")


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"compiling {src.name} failed:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    OUT.parent.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"linking {OUT.name} failed:\n{proc.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT.relative_to(HERE.parent)} ({len(sources)} sources, {ARCH})")
    return OUT


if __name__ == "__main__":
    build()
