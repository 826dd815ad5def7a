"""Installs ``decodekernels_amd`` and its reference-named alias ``decode_kernels``.

    pip install --no-build-isolation .      # builds both libraries for gfx950, then installs
    pip install --no-build-isolation -e .   # editable: the libraries are built in place

The build step is ``decodekernels_amd._build`` (hipcc --offload-arch=gfx950 for
``libdecodekernels_amd.so``, the host compiler against torch's headers for
``_C.so``); the wheel ships both next to the Python modules. Metadata and the
vLLM entry point live in pyproject.toml (reference: setup.py:18-29,
pyproject.toml:22-27).
"""

import sys
from pathlib import Path

import setuptools
from setuptools import find_packages, setup
from setuptools.command.build_py import build_py

ROOT = Path(__file__).resolve().parent


class BuildHipThenPy(build_py):
    """Compiles the two shared libraries in place before the package files are collected."""

    def run(self):
        sys.path.insert(0, str(ROOT))
        from decodekernels_amd import _build

        _build.build()
        super().run()


def project_metadata() -> dict:
    """pyproject.toml's [project] table as setup() arguments, for setuptools < 61
    (which ignores the table); newer releases read it themselves."""
    if int(setuptools.__version__.split(".")[0]) >= 61:
        return {}
    try:
        import tomllib
    except ImportError:
        import tomli as tomllib
    with open(ROOT / "pyproject.toml", "rb") as f:
        proj = tomllib.load(f)["project"]
    entry_points = {group: [f"{name} = {target}" for name, target in eps.items()]
                    for group, eps in proj.get("entry-points", {}).items()}
    return dict(name=proj["name"], version=proj["version"], description=proj["description"],
                python_requires=proj["requires-python"], install_requires=proj["dependencies"],
                entry_points=entry_points)


setup(
    packages=find_packages(include=["decodekernels_amd", "decode_kernels"]),
    package_data={"decodekernels_amd": ["_C.so", "libdecodekernels_amd.so"]},
    cmdclass={"build_py": BuildHipThenPy},
    **project_metadata(),
)
