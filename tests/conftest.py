import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def rel_err(y, r) -> float:
    """Normwise max relative error max|y - r| / max|r|, computed in float64.

    This is the parity metric for every floating-point test (fp32 I/O bar
    1e-4, bf16 I/O bar 2e-2).  A tiny floor keeps all-zero references finite.
    """
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    den = max(float(np.max(np.abs(r))) if r.size else 0.0, 1e-30)
    return float(np.max(np.abs(y - r))) / den if r.size else 0.0


@pytest.fixture(scope="session")
def gpu():
    """The HIP library on cuda:0; GPU tests fail (not skip) if it cannot load."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import mogt_amd

    mogt_amd._lib.load()
    return torch.device("cuda:0")


def to_np(t):
    return t.detach().float().cpu().numpy()


# Tests may print the case they run before each GPU step (flushed), so a
# failure that ends the process still names it.
def announce(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


os.environ.setdefault("PYTHONUNBUFFERED", "1")
