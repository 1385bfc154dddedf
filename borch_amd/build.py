"""Builds ``borch_amd/lib/libbq.so`` from ``borch_amd/csrc/*.hip`` for gfx950.

``python -m borch_amd.build`` (or ``__graft_entry__.build()``) compiles every source with
hipcc, in parallel, and links one shared library with a C ABI (``include/bq.h``). The
library's HIP runtime dependency is ``libamdhip64.so.7``; inside a process that imported
torch first, the dynamic loader binds it to the runtime torch already loaded (same
soname), so both share one HIP context and device pointers pass straight through.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libbq.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3", "-std=c++20", "-fPIC", f"--offload-arch={ARCH}",
    "-mcode-object-version=5",
    "-ffp-contract=off",
    # packed-fp32 instructions are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{ROOT / 'include'}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the int8 library cannot be built without ROCm")


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")
    noise = [ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")


def _link(objs, out: Path) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {out.name} failed:\n{r.stderr}")
    os.replace(tmp, out)


def build(verbose: bool = True) -> Path:
    """Compile every ``csrc/*.hip`` and link ``lib/libbq.so`` (returned)."""
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    objs = [objdir / (s.stem + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(_compile, srcs, objs))
    _link(objs, LIB)
    if verbose:
        print(f"built {LIB.relative_to(ROOT)} from {len(srcs)} sources")
    return LIB


def build_objects(srcs, objdir: Path, out: Path) -> Path:
    """Compile ``srcs`` with the library's flags into ``objdir`` and link the shared library
    ``out`` (bench.py's measurement probes use it)."""
    objdir.mkdir(parents=True, exist_ok=True)
    objs = [objdir / (Path(s).stem + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=max(1, min(8, len(srcs)))) as ex:
        list(ex.map(_compile, [Path(s) for s in srcs], objs))
    _link(objs, out)
    return out


if __name__ == "__main__":
    build()
