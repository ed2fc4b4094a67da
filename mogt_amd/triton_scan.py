"""Drop-in replacement of the reference's ``triton_scan`` module on MI355X.

Same public names, keyword arguments, return structure and ``ValueError``
conditions as lkcfqy/MOGT ``triton_scan.py``, backed by the HIP kernels of
``mogt_amd/csrc`` through ``torch.ops.mogt.*`` (no Triton).  Differences:
``block_size`` / ``block_c`` / ``carry_scan`` are validated exactly like the
reference but only hint at the internal chunking (results do not depend on
them beyond fp32 rounding), and the reference's ``R == 16`` restriction
(triton_scan.py:200-201) is lifted: ``R <= 32`` on the matrix-core pipeline,
up to 1024 on the generic scan.
"""
from __future__ import annotations

import torch

from . import ops


def _next_power_of_two(value: int) -> int:
    # triton_scan.py:8-11
    if value <= 0:
        raise ValueError("value must be positive")
    return 1 << (value - 1).bit_length()


def _check_cuda(what: str, *tensors: torch.Tensor) -> None:
    # triton_scan.py:191-192
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError(f"{what} requires CUDA tensors")


def triton_fused_scan(U: torch.Tensor) -> torch.Tensor:
    """Transport-only prefix product ``Y_t = U_t @ Y_{t-1}``, ``Y_0 = I``.

    Replaces triton_scan.py:151-175 (output dtype = ``U.dtype``).
    """
    _check_cuda("triton_fused_scan", U)
    B, L, R, R2 = U.shape
    if R != R2:
        raise ValueError("the last two dimensions must be square")
    return ops.fused_scan(U, output_dtype=U.dtype)


def triton_affine_local_scan(U: torch.Tensor, V: torch.Tensor, *, block_size: int = 256,
                             block_c: int = 32):
    """Block-local affine prefixes and per-block summaries (all fp32).

    Replaces triton_scan.py:178-229: returns ``(U_prefix, H_prefix, U_summary,
    H_summary)`` with the tail block padded by ``(I, 0)``.
    """
    _check_cuda("triton_affine_local_scan", U, V)
    ops.check_affine_shapes(U, V)
    _next_power_of_two(block_c)
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    return ops.affine_local_scan(U, V, block_size=block_size)


def _triton_affine_scan_hybrid_forward(U: torch.Tensor, V: torch.Tensor, *, block_size: int = 256,
                                       block_c: int = 32, carry_scan: str = "sequential",
                                       output_dtype: torch.dtype | None = None,
                                       return_prefix: bool = False):
    """Forward of the hybrid scan (triton_scan.py:232-311) as one HIP pipeline:
    chunk summaries, carries, output in registers -- no L-sized carry-apply
    pass.  ``output_dtype`` defaults to ``V.dtype`` (triton_scan.py:251)."""
    if carry_scan not in {"sequential", "doubling"}:
        raise ValueError("carry_scan must be 'sequential' or 'doubling'")
    _check_cuda("triton_affine_local_scan", U, V)
    ops.check_affine_shapes(U, V)
    _next_power_of_two(block_c)
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    output_dtype = output_dtype or V.dtype
    return ops.affine_scan(U, V, output_dtype=output_dtype, return_prefix=return_prefix)


def _triton_affine_scan_hybrid_backward(U: torch.Tensor, V: torch.Tensor, grad_H: torch.Tensor, *,
                                        block_size: int, block_c: int, carry_scan: str,
                                        need_grad_u: bool, need_grad_v: bool):
    """dV = G (reverse scan G_t = dH_t + U_{t+1}^T G_{t+1}), dU_t = G_t H_{t-1}^T
    (triton_scan.py:359-426) in fp32; H is recomputed with the forward scan,
    the outer products use a batched GEMM."""
    return ops.affine_scan_grad(U, V, grad_H, None, state_dtype=torch.float32,
                                need_grad_u=need_grad_u, need_grad_v=need_grad_v)


class _TritonAffineScanHybridAutograd(torch.autograd.Function):
    """Autograd contract of the reference (triton_scan.py:314-356)."""

    @staticmethod
    def forward(ctx, U, V, block_size, block_c, carry_scan, output_dtype):
        with torch.autograd.profiler.record_function("triton_hybrid.forward"):
            ctx.block_size = block_size
            ctx.block_c = block_c
            ctx.carry_scan = carry_scan
            ctx.output_dtype = output_dtype or V.dtype
            ctx.save_for_backward(U, V)
            return _triton_affine_scan_hybrid_forward(
                U, V, block_size=block_size, block_c=block_c, carry_scan=carry_scan,
                output_dtype=ctx.output_dtype, return_prefix=False)

    @staticmethod
    def backward(ctx, grad_output):
        U_saved, V_saved = ctx.saved_tensors
        with torch.autograd.profiler.record_function("triton_hybrid.backward_recompute"):
            grad_u, grad_v = _triton_affine_scan_hybrid_backward(
                U_saved, V_saved, grad_output, block_size=ctx.block_size, block_c=ctx.block_c,
                carry_scan=ctx.carry_scan, need_grad_u=ctx.needs_input_grad[0],
                need_grad_v=ctx.needs_input_grad[1])
        return grad_u, grad_v, None, None, None, None


def triton_affine_scan_hybrid(U: torch.Tensor, V: torch.Tensor, *, block_size: int = 256,
                              block_c: int = 32, carry_scan: str = "sequential",
                              output_dtype: torch.dtype | None = None,
                              return_prefix: bool = False):
    """Public entry, same dispatch as triton_scan.py:429-477: ``return_prefix``
    -> ``(U_prefix, H)`` without autograd; grad-enabled inputs -> the autograd
    Function; otherwise the plain forward."""
    if return_prefix:
        return _triton_affine_scan_hybrid_forward(
            U, V, block_size=block_size, block_c=block_c, carry_scan=carry_scan,
            output_dtype=output_dtype, return_prefix=True)
    needs_grad = torch.is_grad_enabled() and (U.requires_grad or V.requires_grad)
    if needs_grad:
        return _TritonAffineScanHybridAutograd.apply(U, V, block_size, block_c, carry_scan,
                                                     output_dtype)
    return _triton_affine_scan_hybrid_forward(
        U, V, block_size=block_size, block_c=block_c, carry_scan=carry_scan,
        output_dtype=output_dtype, return_prefix=False)
