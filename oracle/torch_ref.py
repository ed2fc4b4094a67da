"""CPU PyTorch restatement of the reference's scans — TEST INFRASTRUCTURE ONLY.

Used by ``bench.py`` as the timed CPU baseline (``cpu_baseline.kind = "port"``)
and by tests as a second oracle.  Never imported by the product package.

``affine_scan_sequential_torch`` follows affine_scan.py:14-62: a Python loop
over L of ``torch.bmm`` with fp32 (or fp64) state; ``affine_scan_doubling_torch``
follows affine_scan.py:127-172 (Hillis-Steele, log2 L rounds).
"""
from __future__ import annotations

import torch


def affine_scan_sequential_torch(U: torch.Tensor, V: torch.Tensor, *,
                                 state_dtype: torch.dtype = torch.float32,
                                 output_dtype: torch.dtype | None = None) -> torch.Tensor:
    B, L, R, _ = U.shape
    C = V.shape[-1]
    output_dtype = output_dtype or V.dtype
    Uw = U.to(state_dtype)
    Vw = V.to(state_dtype)
    H = torch.zeros(B, R, C, dtype=state_dtype, device=U.device)
    out = []
    for t in range(L):
        H = torch.bmm(Uw[:, t], H) + Vw[:, t]
        out.append(H.to(output_dtype))
    return torch.stack(out, dim=1)


def affine_scan_doubling_torch(U: torch.Tensor, V: torch.Tensor, *,
                               state_dtype: torch.dtype = torch.float32,
                               output_dtype: torch.dtype | None = None) -> torch.Tensor:
    L = U.shape[1]
    output_dtype = output_dtype or V.dtype
    P = U.to(state_dtype).clone()
    H = V.to(state_dtype).clone()
    off = 1
    while off < L:
        Pp, Hp = P.clone(), H.clone()
        P[:, off:] = torch.matmul(Pp[:, off:], Pp[:, :-off])
        H[:, off:] = torch.matmul(Pp[:, off:], Hp[:, :-off]) + Hp[:, off:]
        off *= 2
    return H.to(output_dtype)


def diag_as_affine(a: torch.Tensor, b: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Fold [B, L, D] per-feature inputs into the reference API's R=C=1 layout
    U = a.transpose(1,2).reshape(B*D, L, 1, 1)."""
    B, L, D = a.shape
    U = a.transpose(1, 2).reshape(B * D, L, 1, 1)
    V = b.transpose(1, 2).reshape(B * D, L, 1, 1)
    return U, V


def unfold_affine(H: torch.Tensor, B: int, D: int) -> torch.Tensor:
    L = H.shape[1]
    return H.reshape(B, D, L).transpose(1, 2)
