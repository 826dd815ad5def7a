import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP libraries")


def pytest_collection_modifyitems(config, items):
    # A test marked gpu on a machine without a GPU is skipped, not failed, so
    # `pytest -m "not gpu"` and a bare `pytest` both work on the CPU.
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Achieved max abs error of the parity checks that ran: the full-size
    configurations one by one, and the checks closest to their bar."""
    try:
        from parity import ERRORS
    except ImportError:
        return
    if not ERRORS:
        return
    import json
    import os

    path = os.environ.get("DK_PARITY_REPORT")
    if path:
        with open(path, "w") as f:
            for rec in ERRORS:
                f.write(json.dumps(rec) + "\n")
    tr = terminalreporter
    tr.section("parity: achieved max abs error (bar: max(2e-2 bf16 / 5e-3 fp16, half an ulp + fp32 slack))")
    full = [r for r in ERRORS if "test_full_size" in r["test"]]
    for r in full:
        plain = r.get("worst_err_over_bar_without_slack")
        tr.write_line(f"  {r['what']:<48} {r['dtype']:<9} max err {r['max_abs_err']:.3e}  "
                      f"worst err/bar {r['worst_err_over_bar']:.3f}"
                      + ("" if plain is None else f" (without the slack {plain:.3f})"))
    tr.write_line(f"  {len(ERRORS)} checks; closest to the bar:")
    for r in sorted(ERRORS, key=lambda r: -r["worst_err_over_bar"])[:8]:
        tr.write_line(f"  {r['worst_err_over_bar']:.3f}  {r['max_abs_err']:.3e} {r['dtype']:<9} {r['what']}  [{r['test']}]")
