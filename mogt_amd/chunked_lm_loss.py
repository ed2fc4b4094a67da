"""Chunked tied-head cross-entropy (chunked_lm_loss.py:5-84) on MI355X.

Same Function, entry point, arguments and ``ValueError`` conditions as the
reference.  The logits of each chunk come from the BLAS GEMM exactly as there
(``hidden.float() @ weight.float().t()``, so autocast applies the same way);
the loss and the softmax gradient of each logits block come from the HIP row
kernels of ``csrc/lm_loss.hip`` (one read of the block in the forward, one
read and an in-place write in the backward) instead of F.cross_entropy,
torch.softmax, the one-hot update and the scale pass.  The forward keeps the
per-token log-sum-exp (4 bytes per token) for the backward.

Labels equal to -100 (F.cross_entropy's default ``ignore_index``) contribute
zero loss, as in the reference's forward, and a zero gradient row; the
reference's backward instead subtracts 1 at column ``vocab - 100`` for them.
"""
from __future__ import annotations

import torch

from . import ops

IGNORE_INDEX = -100


class _ChunkedLinearCrossEntropy(torch.autograd.Function):
    """chunked_lm_loss.py:5-72: stores hidden states, weight and labels (plus the
    per-token log-sum-exp) and recomputes each chunk's logits in backward."""

    @staticmethod
    def forward(ctx, hidden_states, weight, labels, chunk_size: int):
        if hidden_states.ndim != 3:
            raise ValueError("hidden_states must be [B, L, D]")
        if labels.shape != hidden_states.shape[:2]:
            raise ValueError("labels must be [B, L]")
        if weight.ndim != 2 or weight.shape[1] != hidden_states.shape[-1]:
            raise ValueError("weight must be [V, D]")
        chunk_size = int(chunk_size)
        if chunk_size <= 0:
            raise ValueError("chunk_size must be positive")

        bsz, seq_len, d_model = hidden_states.shape
        total_tokens = bsz * seq_len
        hidden_flat = hidden_states.reshape(total_tokens, d_model)
        labels_flat = labels.reshape(total_tokens).to(torch.int64).contiguous()
        weight_float = weight.float()
        losses, lses = [], []
        with torch.no_grad():
            for start in range(0, total_tokens, chunk_size):
                end = min(start + chunk_size, total_tokens)
                logits = hidden_flat[start:end].float().matmul(weight_float.t())
                loss_rows, lse_rows = ops.lm_ce_forward(logits, labels_flat[start:end],
                                                        ignore_index=IGNORE_INDEX)
                losses.append(loss_rows)
                lses.append(lse_rows)
        if losses:
            loss_sum = torch.cat(losses).sum()
            lse = torch.cat(lses)
        else:
            loss_sum = hidden_states.new_zeros((), dtype=torch.float32)
            lse = hidden_states.new_zeros(0, dtype=torch.float32)
        ctx.save_for_backward(hidden_states, weight, labels_flat, lse)
        ctx.chunk_size = chunk_size
        ctx.total_tokens = total_tokens
        return loss_sum / total_tokens

    @staticmethod
    def backward(ctx, grad_output):
        hidden_states, weight, labels_flat, lse = ctx.saved_tensors
        chunk_size = ctx.chunk_size
        total_tokens = ctx.total_tokens
        bsz, seq_len, d_model = hidden_states.shape
        hidden_flat = hidden_states.reshape(total_tokens, d_model)

        grad_hidden_flat = torch.empty_like(hidden_flat)
        grad_weight = torch.zeros_like(weight, dtype=torch.float32)
        weight_float = weight.float()
        scale = (grad_output.float() / float(total_tokens)).reshape(1)

        for start in range(0, total_tokens, chunk_size):
            end = min(start + chunk_size, total_tokens)
            hidden_chunk = hidden_flat[start:end]
            logits = hidden_chunk.float().matmul(weight_float.t())
            probs = ops.lm_ce_backward_(logits, labels_flat[start:end], lse[start:end], scale,
                                        ignore_index=IGNORE_INDEX)
            grad_hidden_flat[start:end] = probs.matmul(weight_float).to(hidden_states.dtype)
            if probs.dtype == torch.float32:
                grad_weight.addmm_(probs.t(), hidden_chunk.float())
            else:   # reduced-precision logits (backward under autocast)
                grad_weight += probs.t().matmul(hidden_chunk.float())

        return grad_hidden_flat.view_as(hidden_states), grad_weight.to(weight.dtype), None, None


def chunked_linear_cross_entropy(hidden_states, weight, labels, *, chunk_size: int):
    """Memory-efficient CE for tied LM heads (chunked_lm_loss.py:75-84): only the
    hidden states, labels and LM weight are kept; logits are recomputed chunk by
    chunk in backward."""
    return _ChunkedLinearCrossEntropy.apply(hidden_states, weight, labels, int(chunk_size))
