"""pytest configuration: the ``gpu`` marker and the repo root on sys.path."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP path through the C-ABI")


def pytest_terminal_summary(terminalreporter):
    """How many n >= 2 outputs passed only by the accuracy clause of
    assert_parity (tests/test_gpu_q8.py): every check, summed, and each check
    that used it."""
    mod = sys.modules.get("test_gpu_q8")
    log = getattr(mod, "CLAUSE_LOG", None) if mod else None
    if not log:
        return
    used = [(w, c, s) for w, c, s in log if c]
    total = sum(s for _, _, s in log)
    terminalreporter.write_sep("-", "n>=2 parity: outputs that needed the accuracy clause")
    terminalreporter.write_line(f"{len(log)} checks, {sum(c for _, c, _ in log)} of {total} outputs "
                                f"({len(used)} checks used the clause)")
    for w, c, s in used:
        terminalreporter.write_line(f"  {w}: {c} of {s}")
