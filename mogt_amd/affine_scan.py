"""Drop-in replacement of the reference's ``affine_scan`` module on MI355X.

The reference keeps three PyTorch scans (sequential, Hillis-Steele doubling,
block-structured) that differ only in how they evaluate the same recurrence
``H_t = U_t @ H_{t-1} + V_t`` (affine_scan.py:14-278).  Here every name keeps
its signature, argument validation and ``(U_prefix, H)`` return structure and
runs one HIP scan for all three (the results agree to the state dtype's
rounding, which is what the reference's own sanity check asserts between them,
sanity_affine_scan.py:19-61):

- ``state_dtype`` float32 with R <= 32 runs on the matrix-core pipeline; a
  float64 state, R up to 1024 or fp16 / fp64 outputs run on the generic scan
  (``mogt_affine_scan_generic_fwd``).  Other state dtypes raise ``ValueError``.
- The outputs are differentiable in U and V, as the reference's PyTorch loops
  are (its backward check differentiates through them,
  sanity_affine_scan.py:102-135).
- Tensors on the host are copied to the current GPU, scanned there, and the
  results copied back to the host: the scan itself only runs on the GPU, and
  without one these functions raise ``RuntimeError``.
"""
from __future__ import annotations

import torch

from . import ops


def _check_state_dtype(state_dtype: torch.dtype) -> None:
    if state_dtype not in ops.STATE_DTYPES:
        raise ValueError(f"state_dtype {state_dtype} not supported by the MI355X scan "
                         "(torch.float32 or torch.float64)")


def _to_gpu(what: str, *tensors: torch.Tensor):
    """Return the tensors on a GPU and the device the results go back to."""
    home = tensors[0].device
    if all(t.device.type == "cuda" for t in tensors):
        return tensors, home
    if not torch.cuda.is_available():
        raise RuntimeError(f"{what}: the MOGT scan runs on the GPU (HIP) only and no GPU is available")
    gpu = torch.device("cuda", torch.cuda.current_device())
    return tuple(t.to(gpu) for t in tensors), home


def _home(x, device: torch.device):
    if x is None or x.device == device:
        return x
    return x.to(device)


def affine_combine(U_next, V_next, U_prev, V_prev):
    """(U_n, V_n) (x) (U_p, V_p) = (U_n @ U_p, U_n @ V_p + V_n)  (affine_scan.py:4-11)."""
    return torch.matmul(U_next, U_prev), torch.matmul(U_next, V_prev) + V_next


def _scan(what: str, U, V, state_dtype, output_dtype, return_prefix):
    ops.check_affine_shapes(U, V)
    _check_state_dtype(state_dtype)
    (Ug, Vg), home = _to_gpu(what, U, V)
    out = ops.affine_scan(Ug, Vg, output_dtype=output_dtype or V.dtype,
                          return_prefix=return_prefix, state_dtype=state_dtype)
    if return_prefix:
        return _home(out[0], home), _home(out[1], home)
    return _home(out, home)


def affine_scan_sequential(U, V, *, state_dtype=torch.float32, output_dtype=None,
                           return_prefix=False):
    """affine_scan.py:14-62 on the GPU."""
    return _scan("affine_scan_sequential", U, V, state_dtype, output_dtype, return_prefix)


def affine_scan_doubling(U, V, *, state_dtype=torch.float32, output_dtype=None,
                         return_prefix=False):
    """affine_scan.py:127-172 on the GPU (same recurrence, one pipeline)."""
    return _scan("affine_scan_doubling", U, V, state_dtype, output_dtype, return_prefix)


def affine_scan_block_reference(U, V, *, block_size=256, state_dtype=torch.float32,
                                output_dtype=None, carry_scan="sequential", return_prefix=False):
    """affine_scan.py:175-278 on the GPU; ``block_size``/``carry_scan`` are
    validated like the reference (:191-194) and only hint at the chunking."""
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    if carry_scan not in {"sequential", "doubling"}:
        raise ValueError("carry_scan must be 'sequential' or 'doubling'")
    return _scan("affine_scan_block_reference", U, V, state_dtype, output_dtype, return_prefix)


def affine_scan_sequential_backward(U, V, grad_H, *, state_dtype=torch.float32, need_grad_u=True,
                                    need_grad_v=True):
    """Gradients of the recurrence (affine_scan.py:65-124): reverse scan for
    dV, ``dU_t = G_t H_{t-1}^T``, computed in ``state_dtype`` and cast back to
    the input dtypes."""
    if U.ndim != 4 or V.ndim != 4 or grad_H.ndim != 4:
        raise ValueError("U, V and grad_H must be rank-4 tensors")
    B, L, R, C = ops.check_affine_shapes(U, V)
    if tuple(grad_H.shape) != (B, L, R, C):
        raise ValueError("grad_H must match V shape [B, L, R, C]")
    _check_state_dtype(state_dtype)
    (Ug, Vg, Gg), home = _to_gpu("affine_scan_sequential_backward", U, V, grad_H)
    grad_u, grad_v = ops.affine_scan_grad(Ug, Vg, Gg, None, state_dtype=state_dtype,
                                          need_grad_u=need_grad_u, need_grad_v=need_grad_v)
    return _home(grad_u, home), _home(grad_v, home)
