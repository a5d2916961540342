import os
import sys

import pytest

try:  # load torch's HIP runtime first, as bench.py does, so one runtime serves both
    import torch  # noqa: F401
except ImportError:
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); run with -m gpu")


def pytest_terminal_summary(terminalreporter):
    """Worst output errors per test module (every gpu_head.rel_err call), and
    the per-test ledger as JSON at $AQ_PARITY_LOG when that is set."""
    mod = sys.modules.get("gpu_head")
    ledger = getattr(mod, "ERROR_LEDGER", None) if mod else None
    if not ledger:
        return
    path = os.environ.get("AQ_PARITY_LOG")
    if path:
        import json
        with open(path, "w") as f:
            json.dump(ledger, f, indent=1, sort_keys=True)
    per_file = {}
    for node, e in ledger.items():
        f = per_file.setdefault(node.split("::")[0], {"calls": 0, "norm_max": 0.0,
                                                       "elem_rel_max": 0.0})
        f["calls"] += e["calls"]
        f["norm_max"] = max(f["norm_max"], e["norm_max"])
        f["elem_rel_max"] = max(f["elem_rel_max"], e["elem_rel_max"])
    tr = terminalreporter
    tr.write_sep("-", "worst output errors (norm-wise max|y-r|/max|r|; elementwise over |r| >= 1e-3 max|r|)")
    for name in sorted(per_file):
        f = per_file[name]
        tr.write_line(f"{name}: {f['calls']} comparisons, norm-wise {f['norm_max']:.2e}, "
                      f"elementwise {f['elem_rel_max']:.2e}")


@pytest.fixture(scope="session")
def oracle():
    from bind import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from bind import Ref
    if not Ref.available:
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    return Ref()


@pytest.fixture(scope="session")
def torch_dev():
    """torch with its HIP runtime (device buffers and streams for the
    device-form calls)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP GPU")
    return torch
