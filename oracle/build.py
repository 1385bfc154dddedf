"""Builds the CPU baseline library oracle/lib/libcpuref.so from oracle/cpu_ref.c (gcc).

Test and measurement infrastructure only. -ffp-contract=off keeps the multiply and the
add separate, as the reference's strict wasm module does (lib.rs `madd`); x86-64-v3
(AVX2) is the host ISA assumed for the GPU boxes' CPUs.
"""
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "lib" / "libcpuref.so"


def build() -> Path:
    OUT.parent.mkdir(exist_ok=True)
    cmd = ["gcc", "-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fPIC", "-shared", "-pthread",
           str(HERE / "cpu_ref.c"), "-o", str(OUT)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stderr)
        raise RuntimeError("gcc failed on oracle/cpu_ref.c")
    print(f"built {OUT.relative_to(HERE.parent)}")
    return OUT


if __name__ == "__main__":
    build()
