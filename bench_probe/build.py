"""Builds ``bench_probe/libbqprobe.so``: bench.py's measurement probes (``bq_probe.h``), not
part of the int8 library. ``python bench_probe/build.py`` (``__graft_entry__.build()`` runs it
after the library)."""
from __future__ import annotations

import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
PROBE_LIB = HERE / "libbqprobe.so"


def build(verbose: bool = True) -> Path:
    if str(ROOT) not in sys.path:
        sys.path.insert(0, str(ROOT))
    from borch_amd.build import build_objects
    srcs = sorted(HERE.glob("*.hip"))
    out = build_objects(srcs, HERE / "_build", PROBE_LIB)
    if verbose:
        print(f"built {out.relative_to(ROOT)} from {len(srcs)} sources")
    return out


if __name__ == "__main__":
    build()
