"""Builds the two shared libraries of the package, in place, for gfx950 only.

* ``libdecodekernels_amd.so`` -- every HIP kernel plus the C-ABI declared in
  ``include/decodekernels_amd.h``. Compiled with ``hipcc --offload-arch=gfx950``;
  it does not link against torch.
* ``_C.so`` -- the PyTorch binding: registers ``torch.ops.decode_kernels.*``
  (same schemas as DecodeKernels' ``csrc/ops.cu:270-286``) and forwards each op
  to the C-ABI. Host-only C++, compiled with the system C++ compiler against
  torch's headers; importing ``decodekernels_amd._C`` runs the registration.

The reference builds with ``torch.utils.cpp_extension.CUDAExtension``
(``setup.py:19-29``); on ROCm that path hipifies CUDA sources, which this
package has none of, so the commands are issued directly.

    python -m decodekernels_amd._build            # build both libraries
    python -m decodekernels_amd._build --resource-usage   # plus per-kernel VGPR/LDS/spill report

Every build keeps the compiler's per-kernel resource report (registers, spills,
scratch, LDS, occupancy; ``-Rpass-analysis=kernel-resource-usage``) of each
source in ``_build/<source>.resources.txt``; ``resource_table()`` parses it
(``tests/test_resource_usage.py`` gates on it, as the reference's
``tools/compile_check.sh`` reports registers and spills per kernel).
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = PKG / "_build"

HIP_SOURCES = ["capi.hip", "paged_attention.hip", "gemm.hip", "norm_act.hip", "rope_cache.hip", "noalloc_scratch.hip"]
LIB_NAME = "libdecodekernels_amd.so"
EXT_NAME = "_C.so"
ARCH = "gfx950"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

# Packed FP32 arithmetic is switched off for all device code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def _hipcc() -> str:
    return os.path.join(ROCM, "bin", "hipcc")


RESOURCE_REMARK = "-Rpass-analysis=kernel-resource-usage"


def _run(cmd: list[str], quiet_remarks: bool = False) -> str:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops' is not a recognized feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    shown = out
    if quiet_remarks:  # drop each resource remark and the source excerpt under it
        kept, skip = [], False
        for line in out.splitlines():
            if RESOURCE_REMARK in line:
                skip = True
            elif skip and "|" in line[:12]:
                pass
            else:
                skip = False
                kept.append(line)
        shown = "\n".join(kept)
    if shown.strip():
        print(shown)
    return out


def resource_report_path(src: str) -> Path:
    return BUILD / (Path(src).stem + ".resources.txt")


def _compile_hip(src: str, resource_usage: bool) -> Path:
    BUILD.mkdir(exist_ok=True)
    obj = BUILD / (Path(src).stem + ".o")
    cmd = [_hipcc(), RESOURCE_REMARK, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    out = _run(cmd, quiet_remarks=not resource_usage)
    resource_report_path(src).write_text(out)
    return obj


def parse_resource_report(text: str) -> list[dict]:
    """Per-kernel records of a ``-Rpass-analysis=kernel-resource-usage`` log:
    {"symbol", "name" (demangled), "SGPRs", "VGPRs", "AGPRs", "ScratchSize",
    "Occupancy", "SGPRs Spill", "VGPRs Spill", "LDS"} (integers)."""
    import re

    keys = {"TotalSGPRs": "SGPRs", "VGPRs": "VGPRs", "AGPRs": "AGPRs", "ScratchSize [bytes/lane]": "ScratchSize",
            "Occupancy [waves/SIMD]": "Occupancy", "SGPRs Spill": "SGPRs Spill", "VGPRs Spill": "VGPRs Spill",
            "LDS Size [bytes/block]": "LDS"}
    recs: list[dict] = []
    for line in text.splitlines():
        if RESOURCE_REMARK not in line:
            continue
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            recs.append({"symbol": m.group(1)})
            continue
        m = re.search(r"remark:\s+([^:]+): (\S+) \[", line)
        if m and recs and m.group(1).strip() in keys:
            recs[-1][keys[m.group(1).strip()]] = int(m.group(2))
    names = subprocess.run(["c++filt"], input="\n".join(r["symbol"] for r in recs), capture_output=True,
                           text=True).stdout.splitlines()
    for r, n in zip(recs, names):
        r["name"] = n
    return recs


def resource_table(sources: list[str] | None = None) -> list[dict]:
    """Resource records of every kernel of the sources, from the last build's
    reports; each record also names its "source"."""
    recs = []
    for src in sources or HIP_SOURCES:
        for r in parse_resource_report(resource_report_path(src).read_text()):
            r["source"] = src
            recs.append(r)
    return recs


def build_lib(resource_usage: bool = False, jobs: int = 4) -> Path:
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile_hip(s, resource_usage), HIP_SOURCES))
    out = PKG / LIB_NAME
    tmp = PKG / (LIB_NAME + ".tmp")
    _run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_ext() -> Path:
    import torch
    from torch.utils import cpp_extension

    torch_dir = Path(torch.__file__).resolve().parent
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    includes = [*cpp_extension.include_paths(), f"{ROCM}/include", sysconfig.get_paths()["include"], str(INCLUDE)]
    BUILD.mkdir(exist_ok=True)
    out = PKG / EXT_NAME
    tmp = PKG / (EXT_NAME + ".tmp")
    cmd = [
        os.environ.get("CXX", "g++"),
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-w",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *[f"-I{p}" for p in includes],
        str(CSRC / "torch_binding.cpp"),
        "-o",
        str(tmp),
        f"-L{PKG}",
        "-ldecodekernels_amd",
        f"-L{torch_dir / 'lib'}",
        "-ltorch",
        "-ltorch_cpu",
        "-ltorch_hip",
        "-lc10",
        "-lc10_hip",
        "-Wl,-rpath,$ORIGIN",
        f"-Wl,-rpath,{torch_dir / 'lib'}",
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build(resource_usage: bool = False) -> None:
    lib = build_lib(resource_usage)
    ext = build_ext()
    print(f"built {lib.relative_to(ROOT)} and {ext.relative_to(ROOT)} for {ARCH}")


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--resource-usage", action="store_true", help="print VGPR/SGPR/LDS/spill use per kernel")
    ap.add_argument("--lib-only", action="store_true", help="build only the C-ABI library")
    args = ap.parse_args(argv)
    if args.lib_only:
        build_lib(args.resource_usage)
    else:
        build(args.resource_usage)
    return 0


if __name__ == "__main__":
    sys.exit(main())
