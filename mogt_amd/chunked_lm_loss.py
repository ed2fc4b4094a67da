"""Tied-head cross-entropy without materialised logits (chunked_lm_loss.py:5-84).

``chunked_linear_cross_entropy(hidden_states, weight, labels, chunk_size=...)``
keeps the reference's contract: the mean over all B*L tokens of the
cross-entropy of ``hidden @ weight.T`` against ``labels``, computed over
``chunk_size`` token rows at a time, storing only the hidden states, labels and
weight (plus 4 bytes per token here) for a backward that recomputes the
logits.  The argument checks and their ``ValueError`` messages are the
reference's interface.

How it runs here:

* Each block of token rows is one GEMM (``rows.float() @ weight.float().T``,
  so autocast applies as in the reference's forward) followed by the HIP row
  kernels of ``csrc/lm_loss.hip``: the forward kernel reads the block once and
  writes per-row loss and log-sum-exp; the backward kernel reads the block
  once and writes ``scale * (softmax - onehot)`` as an fp32 block.
* The backward recomputes each block's logits under the autocast state the
  forward ran under (recorded at forward time), so they match the forward's
  logits, whose log-sum-exp it reuses.  The two gradient GEMMs run in fp32
  with autocast off, as the reference's backward does.
* Labels equal to -100 (F.cross_entropy's default ``ignore_index``) add zero
  loss, as in the reference's forward, and a zero gradient row; the
  reference's backward subtracts 1 at column ``vocab - 100`` for them.

``logits_cross_entropy(logits, labels)`` is the same loss for logits that are
kept anyway (MOGTForCausalLM's ``return_logits`` path, model_mogt.py:326-348):
the summed cross-entropy over the token count, on the same row kernels.
"""
from __future__ import annotations

import torch

from . import ops

IGNORE_INDEX = -100


def _token_blocks(total: int, size: int):
    """Consecutive row slices of at most ``size`` rows covering ``total``."""
    for lo in range(0, total, size):
        yield slice(lo, min(lo + size, total))


class _AutocastState:
    """The CUDA autocast setting of the forward, replayed in the backward."""

    def __init__(self):
        self.enabled = torch.is_autocast_enabled("cuda")
        self.dtype = torch.get_autocast_dtype("cuda")

    def __call__(self):
        return torch.autocast("cuda", dtype=self.dtype, enabled=self.enabled)


def _block_logits(rows: torch.Tensor, w32: torch.Tensor) -> torch.Tensor:
    """One block's logits exactly as the reference forms them (fp32 copies,
    matmul under the caller's autocast state)."""
    return rows.float().matmul(w32.t())


class _ChunkedLinearCrossEntropy(torch.autograd.Function):
    """chunked_lm_loss.py:5-72 on the HIP cross-entropy rows."""

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

        n_tok = labels.numel()
        rows = hidden_states.reshape(n_tok, hidden_states.shape[-1])
        targets = labels.reshape(n_tok).to(torch.int64).contiguous()
        w32 = weight.float()
        per_row = torch.empty(n_tok, dtype=torch.float32, device=hidden_states.device)
        lse = torch.empty(n_tok, dtype=torch.float32, device=hidden_states.device)
        with torch.no_grad():
            for sl in _token_blocks(n_tok, chunk_size):
                loss_rows, lse_rows = ops.lm_ce_forward(_block_logits(rows[sl], w32), targets[sl],
                                                        ignore_index=IGNORE_INDEX)
                per_row[sl] = loss_rows
                lse[sl] = lse_rows
        ctx.save_for_backward(hidden_states, weight, targets, lse)
        ctx.chunk_size = chunk_size
        ctx.autocast = _AutocastState()
        return per_row.sum() / n_tok

    @staticmethod
    def backward(ctx, grad_output):
        hidden_states, weight, targets, lse = ctx.saved_tensors
        n_tok = targets.numel()
        rows = hidden_states.reshape(n_tok, hidden_states.shape[-1])
        w32 = weight.float()
        scale = (grad_output.float() / n_tok).reshape(1)
        d_rows = torch.empty_like(rows)
        d_w32 = torch.zeros_like(w32)
        for sl in _token_blocks(n_tok, ctx.chunk_size):
            block = rows[sl]
            with ctx.autocast():
                logits = _block_logits(block, w32)
            # fp32 gradient block, whatever the logits' dtype
            g = ops.lm_ce_grad(logits, targets[sl], lse[sl], scale, ignore_index=IGNORE_INDEX)
            with torch.autocast("cuda", enabled=False):
                d_rows[sl] = g.matmul(w32).to(d_rows.dtype)
                d_w32.addmm_(g.t(), block.float())
        return d_rows.view_as(hidden_states), d_w32.to(weight.dtype), None, None


def chunked_linear_cross_entropy(hidden_states, weight, labels, *, chunk_size: int):
    """Memory-efficient CE for tied LM heads (chunked_lm_loss.py:75-84): only the
    hidden states, labels and LM weight are kept; logits are recomputed chunk by
    chunk in backward."""
    return _ChunkedLinearCrossEntropy.apply(hidden_states, weight, labels, int(chunk_size))


class _LogitsCrossEntropy(torch.autograd.Function):
    """sum of per-row cross-entropy / row count, for logits the caller keeps."""

    @staticmethod
    def forward(ctx, logits, labels):
        targets = labels.to(torch.int64).contiguous()
        block = logits if logits.stride(-1) == 1 else logits.contiguous()
        loss_rows, lse = ops.lm_ce_forward(block, targets, ignore_index=IGNORE_INDEX)
        ctx.save_for_backward(block, targets, lse)
        return loss_rows.sum() / max(targets.numel(), 1)

    @staticmethod
    def backward(ctx, grad_output):
        block, targets, lse = ctx.saved_tensors
        scale = (grad_output.float() / max(targets.numel(), 1)).reshape(1)
        grad = block.clone()
        ops.lm_ce_backward_(grad, targets, lse, scale, ignore_index=IGNORE_INDEX)
        return grad, None


def logits_cross_entropy(logits: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
    """Summed cross-entropy of ``logits [N, V]`` against ``labels [N]`` divided by
    N (the chunked loss of model_mogt.py:326-348 with the logits kept); labels
    of -100 add zero."""
    if logits.ndim != 2 or labels.shape != logits.shape[:1]:
        raise ValueError("logits must be [N, V] and labels [N]")
    return _LogitsCrossEntropy.apply(logits, labels)
