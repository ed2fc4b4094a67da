"""CPU oracle of the chunked tied-head cross-entropy — TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module.  A float64 numpy restatement of
chunked_lm_loss.py:5-72 (``_ChunkedLinearCrossEntropy``): per chunk, logits =
hidden @ weight^T, loss = sum of (logsumexp - logit[label]) over the chunk's
tokens divided by the total token count; backward: (softmax - onehot) * scale
times weight for the hidden states and its transpose times the hidden states
for the weight.  Labels equal to ``ignore_index`` contribute zero loss and a
zero gradient row (F.cross_entropy's forward; the GPU path's backward).

How each function is pinned (tests/test_oracle.py):
  ce_rows                 == torch.nn.functional.cross_entropy(reduction="none")
                             and torch.logsumexp in float64 (library routines),
                             incl. ignore_index rows and a shifted-logits
                             invariance (loss unchanged by adding a row constant)
  ce_rows_grad            == torch.autograd of F.cross_entropy in float64
  chunked_linear_ce       chunk-size invariance (1, 7, all) and loss / grads ==
                          torch.autograd of the unchunked F.cross_entropy(h W^T)
"""
from __future__ import annotations

import numpy as np


def ce_rows(logits: np.ndarray, labels: np.ndarray, ignore_index: int = -100):
    """Per-row (loss, lse) of a [rows, vocab] logits block (chunked_lm_loss.py:32-36
    with reduction="none"): lse = m + log(sum(exp(x - m))), loss = lse - x[label]."""
    x = np.asarray(logits, dtype=np.float64)
    m = x.max(axis=1, keepdims=True)
    lse = (m + np.log(np.exp(x - m).sum(axis=1, keepdims=True)))[:, 0]
    lab = np.asarray(labels, dtype=np.int64)
    keep = lab != ignore_index
    picked = np.zeros_like(lse)
    picked[keep] = x[np.nonzero(keep)[0], lab[keep]]
    loss = np.where(keep, lse - picked, 0.0)
    return loss, lse


def ce_rows_grad(logits: np.ndarray, labels: np.ndarray, scale: float, ignore_index: int = -100):
    """scale * (softmax(x) - onehot(label)) per row, zero rows for ignored labels
    (chunked_lm_loss.py:61-64)."""
    x = np.asarray(logits, dtype=np.float64)
    _, lse = ce_rows(x, labels, ignore_index)
    p = np.exp(x - lse[:, None])
    lab = np.asarray(labels, dtype=np.int64)
    keep = lab != ignore_index
    rows = np.nonzero(keep)[0]
    p[rows, lab[keep]] -= 1.0
    p[~keep] = 0.0
    return p * scale


def chunked_linear_ce(hidden: np.ndarray, weight: np.ndarray, labels: np.ndarray, chunk_size: int,
                      grad_output: float = 1.0, ignore_index: int = -100):
    """Loss and (d hidden, d weight) of chunked_linear_cross_entropy
    (chunked_lm_loss.py:7-72) in float64."""
    h = np.asarray(hidden, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    B, L, D = h.shape
    T = B * L
    hf = h.reshape(T, D)
    lab = np.asarray(labels, dtype=np.int64).reshape(T)
    loss_sum = 0.0
    gh = np.zeros_like(hf)
    gw = np.zeros_like(w)
    scale = grad_output / T
    for s in range(0, T, chunk_size):
        e = min(s + chunk_size, T)
        logits = hf[s:e] @ w.T
        loss, _ = ce_rows(logits, lab[s:e], ignore_index)
        loss_sum += loss.sum()
        g = ce_rows_grad(logits, lab[s:e], scale, ignore_index)
        gh[s:e] = g @ w
        gw += g.T @ hf[s:e]
    return loss_sum / T, gh.reshape(B, L, D), gw
