"""Compile-only resource gate (CPU): registers, spills, scratch and occupancy of
every HIP kernel, as the compiler reports them for gfx950.

The reference compiles each kernel template in CI and prints registers and
spills per kernel (tools/compile_check.sh:17-42, tools/compile_check.cu:11-32),
and its README states that no kernel spills registers (README.md:107-119).
Here the same report comes from ``-Rpass-analysis=kernel-resource-usage``,
which every build keeps per source (``decodekernels_amd/_build.py``). When
that report is missing or older than a source, this test compiles the device
code itself.

Gates:
* every kernel (all ~400 instantiations): no scratch memory, no VGPR spills
  and no SGPR spills;
* the hot kernels keep the occupancy their designs are tuned for, so a change
  that costs a wave per SIMD fails here rather than as a slower bench.
"""

import concurrent.futures as cf
import os
import subprocess
import tempfile
from pathlib import Path

import pytest

from decodekernels_amd import _build

DEPS = [_build.CSRC / "dk_device.h", _build.CSRC / "dk_host.h", _build.INCLUDE / "decodekernels_amd.h"]
NO_KERNELS = {"capi.hip", "noalloc_scratch.hip"}  # host code and a device array only


def _fresh(src: str) -> bool:
    rep = _build.resource_report_path(src)
    if not rep.exists() or (rep.stat().st_size == 0 and src not in NO_KERNELS):
        return False
    newest = max(p.stat().st_mtime for p in [_build.CSRC / src, *DEPS])
    return rep.stat().st_mtime >= newest


def _compile_device_only(src: str, out_dir: str) -> str:
    cmd = [_build._hipcc(), _build.RESOURCE_REMARK, *_build.HIP_FLAGS, "--cuda-device-only", "-c",
           str(_build.CSRC / src), "-o", os.path.join(out_dir, Path(src).stem + ".o")]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert proc.returncode == 0, proc.stdout[-4000:]
    return proc.stdout


@pytest.fixture(scope="module")
def table():
    recs = []
    stale = [s for s in _build.HIP_SOURCES if not _fresh(s)]
    for src in _build.HIP_SOURCES:
        if src not in stale:
            recs += [dict(r, source=src) for r in _build.parse_resource_report(_build.resource_report_path(src).read_text())]
    if stale:
        with tempfile.TemporaryDirectory() as d, cf.ThreadPoolExecutor(max_workers=min(4, len(stale))) as ex:
            for src, text in zip(stale, ex.map(lambda s: _compile_device_only(s, d), stale)):
                recs += [dict(r, source=src) for r in _build.parse_resource_report(text)]
    assert len(recs) > 300, f"only {len(recs)} kernels reported"
    return recs


def test_no_kernel_spills_or_uses_scratch(table):
    bad = [(r["source"], r["name"], r["ScratchSize"], r["VGPRs Spill"], r["SGPRs Spill"]) for r in table
           if r["ScratchSize"] or r["VGPRs Spill"] or r["SGPRs Spill"]]
    assert not bad, "kernels with scratch / VGPR spills / SGPR spills:\n" + "\n".join(map(str, bad))


def test_every_source_reports_its_kernels(table):
    per_source = {s: sum(r["source"] == s for r in table) for s in _build.HIP_SOURCES}
    assert all(per_source[s] > 0 for s in _build.HIP_SOURCES if s not in NO_KERNELS), per_source


def _pick(table, *parts):
    got = [r for r in table if all(p in r["name"] for p in parts)]
    assert got, f"no kernel matches {parts}"
    return got


# (name fragments, waves per SIMD the design needs). Attention: the headline
# balanced kernel and its grid form hold two 4-wave workgroups per CU at
# head_dim 128 (16-bit cache), three with an fp8 cache, four at head_dim 64;
# the split-K reduce and norms are small. GEMM: one 8-wave LDS-DMA workgroup of
# the 256-row tiles per CU (two waves per SIMD), two 4-wave workgroups of the
# 64 x 64 decode tile, and the skinny M <= 64 tiles at least 6 waves per SIMD
# at M = 1.
OCCUPANCY = [
    (("paged_attention_balanced_kernel<dk::Bf16, 128, true, 16, 4, false>",), 2),
    (("paged_attention_balanced_kernel<dk::F16, 128, true, 16, 4, false>",), 2),
    (("paged_attention_kernel<dk::Bf16, 128, true, true, 16, 4, false>",), 2),
    (("paged_attention_balanced_kernel<dk::Bf16, 128, true, 16, 4, true>",), 3),
    (("paged_attention_balanced_kernel<dk::Bf16, 64, true, 16, 4, false>",), 4),
    (("paged_attention_balanced_kernel<dk::Bf16, 256, true, 16, 2, false>",), 1),
    (("paged_attention_reduce_kernel<dk::Bf16, 128",), 8),
    (("gemm_dma_kernel<dk::Bf16, 256, 256, 4, 2, 2>",), 2),
    (("gemm_dma_kernel<dk::Bf16, 256, 192, 4, 2, 2>",), 2),
    (("gemm_dma_kernel<dk::Bf16, 256, 224, 4, 2, 2>",), 2),
    (("gemm_dma_kernel<dk::Bf16, 192, 192, 4, 2, 3>",), 2),
    (("gemm_dma_kernel<dk::Bf16, 192, 224, 4, 2, 2>",), 2),
    (("gemm_dma_kernel<dk::Bf16, 64, 64, 2, 2, 4>",), 2),
    (("gemm_skinny_lds_kernel<dk::Bf16, 1,",), 6),
    (("rms_norm_vec_kernel<dk::Bf16, 8>",), 5),
    (("fused_add_rms_norm_vec_kernel<dk::Bf16, 8>",), 5),
    (("silu_and_mul_vec_kernel<dk::Bf16>",), 8),
]


@pytest.mark.parametrize("parts,waves", OCCUPANCY, ids=[p[0][0].split("<")[0] + "<" + p[0][0].split("<")[1][:24]
                                                        for p in OCCUPANCY])
def test_hot_kernel_occupancy(table, parts, waves):
    for r in _pick(table, *parts):
        assert r["Occupancy"] >= waves, (r["name"], r["Occupancy"], r["VGPRs"], r["AGPRs"], r["LDS"])
