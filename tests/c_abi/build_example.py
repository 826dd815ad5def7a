"""Builds ``dk_c_example`` (this directory) from ``dk_c_example.c`` with gcc
against ``include/decodekernels_amd.h``, ``libdecodekernels_amd.so`` and the HIP
runtime (``libamdhip64``): a torch-free C caller of the C ABI. Run by
``__graft_entry__.build()`` after the library build; the binary finds the
library through an ``$ORIGIN``-relative rpath, so it runs from any copy of the
repository."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
SOURCE = HERE / "dk_c_example.c"
BINARY = HERE / "dk_c_example"


def command(out: Path) -> list[str]:
    return [
        os.environ.get("CC", "gcc"), "-std=c99", "-O2", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
        f"-I{ROCM}/include", f"-I{ROOT / 'include'}", str(SOURCE), "-o", str(out),
        f"-L{ROOT / 'decodekernels_amd'}", "-ldecodekernels_amd", f"-L{ROCM}/lib", "-lamdhip64", "-lm",
        "-Wl,-rpath,$ORIGIN/../../decodekernels_amd", f"-Wl,-rpath,{ROCM}/lib",
    ]


def build(out: Path = BINARY) -> Path:
    proc = subprocess.run(command(out), stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError("building the C-ABI example failed:\n" + proc.stdout)
    return out


if __name__ == "__main__":
    print(build())
    sys.exit(0)
