import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "mlx-turboquant_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs on the GPU box)")
    config.addinivalue_line("markers", "slow: long-running")


def _has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Code-parity accounting of the GPU codec tests: per call, the
    coordinates compared, the code mismatches against the oracle, how many of
    them lie inside the float32 boundary band (all must), and how many lie
    within 1 float32 ulp of a boundary. Printed under -q too."""
    helpers = sys.modules.get("gpu_helpers")
    log = getattr(helpers, "PARITY_LOG", None)
    if not log:
        return
    tr = terminalreporter
    tr.write_sep("=", "code parity against the oracle (mismatches: all / in band / within 1 ulp / outside band)")
    tot = [0, 0, 0, 0, 0]
    for test, bits, n, m, inb, ulp, out in log:
        tr.write_line(f"{test} bits={bits}: {n} coords, mismatches {m} / {inb} / {ulp} / {out}")
        for i, x in enumerate((n, m, inb, ulp, out)):
            tot[i] += x
    tr.write_line(f"TOTAL: {tot[0]} coords, mismatches {tot[1]} / in band {tot[2]} / within 1 ulp {tot[3]} / "
                  f"outside band {tot[4]} ({len(log)} comparisons)")
