"""CPU tests of the drop-in surface: the reference's import name and its vLLM
entry point.

* ``decode_kernels`` and its submodules (reference: decode_kernels/__init__.py:7-27)
  are this package's own modules, so callers written against the reference
  run unchanged;
* the ``vllm.general_plugins`` entry point (reference: pyproject.toml:22-27)
  is read back from the metadata that setup.py generates (``egg_info``, no
  build) and resolves to the plugin's ``register``.
"""

import importlib.metadata
import subprocess
import sys
from pathlib import Path

import pytest

import decodekernels_amd

ROOT = Path(__file__).resolve().parent.parent

# decode_kernels/__init__.py:7-27 of the reference
REFERENCE_EXPORTS = ["PARTITION_SIZE", "alloc_workspace", "fused_add_rms_norm", "gemm", "is_available",
                     "paged_attention_decode", "rms_norm", "silu_and_mul"]


def test_reference_import_names():
    import decode_kernels as dk
    from decode_kernels import ops, testing, vllm_patch, vllm_plugin

    for name in REFERENCE_EXPORTS:
        assert getattr(dk, name) is getattr(decodekernels_amd, name)
    assert ops is decodekernels_amd.ops and ops.PARTITION_SIZE == 512
    assert ops.MAX_GQA_GROUP >= 8 and {64, 128, 256} <= set(ops.SUPPORTED_HEAD_DIMS)
    assert testing.make_paged_kv is decodekernels_amd.testing.make_paged_kv
    assert vllm_patch is decodekernels_amd.vllm_patch  # one set of counters
    assert vllm_plugin.register is decodekernels_amd.vllm_plugin.register
    assert sys.modules["decode_kernels.ops"] is decodekernels_amd.ops


def test_reference_extension_name():
    if not decodekernels_amd.ops._AVAILABLE:
        pytest.skip("libraries not built")
    import torch

    import decode_kernels._C  # noqa: F401

    assert sys.modules["decode_kernels._C"] is decodekernels_amd._C
    assert hasattr(torch.ops.decode_kernels, "paged_attention_decode")


def test_vllm_entry_point_from_package_metadata(tmp_path):
    subprocess.run([sys.executable, "setup.py", "-q", "egg_info", "--egg-base", str(tmp_path)], cwd=ROOT, check=True,
                   capture_output=True)
    dists = [d for d in importlib.metadata.distributions(path=[str(tmp_path)])
             if d.metadata["Name"] == "decodekernels-amd"]
    assert len(dists) == 1
    eps = [e for e in dists[0].entry_points if e.group == "vllm.general_plugins"]
    assert [(e.name, e.value) for e in eps] == [("decode_kernels", "decode_kernels.vllm_plugin:register")]
    assert eps[0].load() is decodekernels_amd.vllm_plugin.register
    top = (Path(dists[0]._path) / "top_level.txt").read_text().split()
    assert set(top) == {"decode_kernels", "decodekernels_amd"}
    assert dists[0].metadata["Version"] == decodekernels_amd.__version__


def test_c_library_reports_the_package_version():
    from decodekernels_amd import capi

    assert capi.lib().dk_version().decode() == f"decodekernels_amd {decodekernels_amd.__version__} (gfx950)"


def test_plugin_docstring_names_the_registered_entry_point():
    text = decodekernels_amd.vllm_plugin.__doc__
    assert 'decode_kernels = "decode_kernels.vllm_plugin:register"' in text
