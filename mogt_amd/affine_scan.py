"""Drop-in replacement of the reference's ``affine_scan`` module on MI355X.

The reference keeps three PyTorch scans (sequential, Hillis-Steele doubling,
block-structured) that differ only in how they evaluate the same recurrence
``H_t = U_t @ H_{t-1} + V_t`` (affine_scan.py:14-278).  Here every name keeps
its signature, argument validation and ``(U_prefix, H)`` return structure but
runs the HIP scan (one pipeline for all three: the results agree to fp32
rounding, which is what the reference's own sanity check asserts between them,
sanity_affine_scan.py:19-61).  The state is fp32 on the GPU: a ``state_dtype``
other than float32 raises ``ValueError`` instead of silently changing precision.
Tensors must live on the GPU.
"""
from __future__ import annotations

import torch

from . import ops, triton_scan


def _check_state_dtype(state_dtype: torch.dtype) -> None:
    if state_dtype != torch.float32:
        raise ValueError("the MI355X scan keeps its state in float32 (state_dtype=torch.float32)")


def affine_combine(U_next, V_next, U_prev, V_prev):
    """(U_n, V_n) (x) (U_p, V_p) = (U_n @ U_p, U_n @ V_p + V_n)  (affine_scan.py:4-11)."""
    return torch.matmul(U_next, U_prev), torch.matmul(U_next, V_prev) + V_next


def affine_scan_sequential(U, V, *, state_dtype=torch.float32, output_dtype=None,
                           return_prefix=False):
    """affine_scan.py:14-62 on the GPU."""
    ops.require_cuda("affine_scan_sequential", U, V)
    ops.check_affine_shapes(U, V)
    _check_state_dtype(state_dtype)
    return ops.affine_scan(U, V, output_dtype=output_dtype or V.dtype,
                           return_prefix=return_prefix)


def affine_scan_doubling(U, V, *, state_dtype=torch.float32, output_dtype=None,
                         return_prefix=False):
    """affine_scan.py:127-172 on the GPU (same recurrence, one pipeline)."""
    ops.require_cuda("affine_scan_doubling", U, V)
    ops.check_affine_shapes(U, V)
    _check_state_dtype(state_dtype)
    return ops.affine_scan(U, V, output_dtype=output_dtype or V.dtype,
                           return_prefix=return_prefix)


def affine_scan_block_reference(U, V, *, block_size=256, state_dtype=torch.float32,
                                output_dtype=None, carry_scan="sequential", return_prefix=False):
    """affine_scan.py:175-278 on the GPU; ``block_size``/``carry_scan`` are
    validated like the reference (:191-194) and only hint at the chunking."""
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    if carry_scan not in {"sequential", "doubling"}:
        raise ValueError("carry_scan must be 'sequential' or 'doubling'")
    ops.require_cuda("affine_scan_block_reference", U, V)
    ops.check_affine_shapes(U, V)
    _check_state_dtype(state_dtype)
    return ops.affine_scan(U, V, output_dtype=output_dtype or V.dtype,
                           return_prefix=return_prefix)


def affine_scan_sequential_backward(U, V, grad_H, *, state_dtype=torch.float32, need_grad_u=True,
                                    need_grad_v=True):
    """Gradients of the recurrence (affine_scan.py:65-124): reverse scan for
    dV, ``dU_t = G_t H_{t-1}^T``; cast back to the input dtypes."""
    if U.ndim != 4 or V.ndim != 4 or grad_H.ndim != 4:
        raise ValueError("U, V and grad_H must be rank-4 tensors")
    ops.require_cuda("affine_scan_sequential_backward", U, V, grad_H)
    B, L, R, C = ops.check_affine_shapes(U, V)
    if tuple(grad_H.shape) != (B, L, R, C):
        raise ValueError("grad_H must match V shape [B, L, R, C]")
    _check_state_dtype(state_dtype)
    return triton_scan._triton_affine_scan_hybrid_backward(
        U, V, grad_H, block_size=256, block_c=32, carry_scan="sequential",
        need_grad_u=need_grad_u, need_grad_v=need_grad_v)
