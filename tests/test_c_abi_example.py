"""The C ABI from a torch-free C program (``tests/c_abi/dk_c_example.c``):
gemm_tn with and without a workspace and paged decode attention on device
memory from the HIP runtime, each against a double-precision computation in
the program itself, plus two argument errors.

CPU: the program compiles (gcc, C99, -Wall -Wextra -Werror) against
``include/decodekernels_amd.h`` and links against the library. GPU: the binary
that ``__graft_entry__.build()`` builds next to the source runs and reports
every check passed."""

import subprocess

import pytest

from c_abi import build_example


def test_c_example_compiles_against_the_header(tmp_path):
    out = build_example.build(tmp_path / "dk_c_example")
    assert out.exists()


@pytest.mark.gpu
def test_c_example_runs():
    binary = build_example.BINARY
    assert binary.exists(), f"{binary} is not built (run __graft_entry__.build())"
    print("running the C-ABI example", flush=True)
    proc = subprocess.run([str(binary)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    print(proc.stdout, flush=True)
    assert proc.returncode == 0, proc.stdout
    assert "c abi example ok" in proc.stdout
    assert proc.stdout.count("\nok  ") >= 5
