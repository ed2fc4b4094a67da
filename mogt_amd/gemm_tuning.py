"""Tuned GEMM selection for the backbone's library GEMMs (hipBLASLt / rocBLAS).

The MOGT block's projections (phi_val + gate pre-logits, theta_read, the
SwiGLU projections) are plain GEMMs left to the BLAS libraries.  PyTorch's
TunableOp can time every hipBLASLt and rocBLAS solution for a GEMM shape and
keep the fastest; ``tuning/gemm_gfx950.csv`` is such a table for the shapes of
the backbone benchmarks (d_model 768, FFN 3072 and 2048, L = 8K / 16K / 32K,
forward and training), written on an MI355X by ``tuning/tune_gemms.py``.

``use_tuned_gemms()`` switches TunableOp on with tuning off and loads the
table: GEMMs whose shape is in it run the recorded solution, all others the
library default.  The table is valid only for the library versions and GPU
named in its header; TunableOp refuses it otherwise, and the default choice
is kept.  Results change only at the level of GEMM rounding (a different
summation order).
"""
from __future__ import annotations

from pathlib import Path

import torch

TABLE = Path(__file__).resolve().parent / "tuning" / "gemm_gfx950.csv"


def use_tuned_gemms(path: str | Path = TABLE) -> bool:
    """Enable TunableOp (tuning off) with the GEMM table at ``path``; returns
    whether the table was accepted."""
    path = Path(path)
    if not path.exists() or not torch.cuda.is_available():
        return False
    torch.cuda.tunable.enable(True)
    torch.cuda.tunable.tuning_enable(False)
    ok = bool(torch.cuda.tunable.read_file(str(path)))
    if not ok:
        torch.cuda.tunable.enable(False)
    return ok


def default_gemms() -> None:
    """Back to the libraries' own GEMM selection."""
    torch.cuda.tunable.enable(False)


def tuned_gemms_active() -> bool:
    return torch.cuda.tunable.is_enabled() and not torch.cuda.tunable.tuning_is_enabled()
