"""Seeded synthetic inputs for the benchmark configurations.

All draws use ``numpy.random.Generator(PCG64(seed))`` (version-stable across
numpy releases); ``N(mu, sigma)`` means mean and standard deviation.
Configurations (numbered as in the benchmark definition):
  1  diagonal scan, B=2, L=512, D=128, a=sigmoid(N(2,1)), b~N(0,1)
  2  diagonal scan, B=1, D=768, L in {8192,16384,32768}, a=sigmoid(N(3,1)), b~N(0,0.5)
  2' coupled per-rank gate: z~N(-2,1) [B,L,16], v~N(0,1) [B,L,768]
  3  rank-1 coupled write-forget: B=2, L=8192, H=12, d=64, f=sigmoid(N(2,1)),
     k,q L2-normalised N(0,1), v~N(0,1)
  4  dense per-head transition: B=1, H=8, d=32, L=16384, A_t = sigmoid(N(2,1)) *
     (I-W)^{-1}(I+W), W = T - T^T with T strictly upper-triangular N(0,0.05);
     B_t = v k^T, v~N(0,1), k L2-normalised N(0,1)
"""
from __future__ import annotations

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def _sigmoid(x: np.ndarray) -> np.ndarray:
    return (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)


def diag_inputs(B: int, L: int, D: int, *, a_mean: float = 3.0, b_std: float = 0.5,
                seed: int = 0) -> tuple[np.ndarray, np.ndarray]:
    g = rng(seed)
    x = g.standard_normal((B, L, D), dtype=np.float32) + np.float32(a_mean)
    a = _sigmoid(x)
    b = (g.standard_normal((B, L, D), dtype=np.float32) * np.float32(b_std)).astype(np.float32)
    return a, b


def cfg1_inputs(seed: int = 0):
    return diag_inputs(2, 512, 128, a_mean=2.0, b_std=1.0, seed=seed)


def cfg2_inputs(L: int, seed: int = 0):
    return diag_inputs(1, L, 768, a_mean=3.0, b_std=0.5, seed=seed)


def coupled_inputs(B: int, L: int, r: int, c: int, *, z_mean: float = -2.0, seed: int = 0):
    g = rng(seed)
    z = (g.standard_normal((B, L, r), dtype=np.float32) + np.float32(z_mean)).astype(np.float32)
    v = g.standard_normal((B, L, r * c), dtype=np.float32)
    return z, v


def _unit(x: np.ndarray) -> np.ndarray:
    n = np.linalg.norm(x.astype(np.float64), axis=-1, keepdims=True)
    return (x / np.maximum(n, 1e-12)).astype(np.float32)


def rank1_inputs(B: int, L: int, H: int, d: int, *, seed: int = 0):
    g = rng(seed)
    f = _sigmoid(g.standard_normal((B, L, H), dtype=np.float32) + np.float32(2.0))
    k = _unit(g.standard_normal((B, L, H, d), dtype=np.float32))
    q = _unit(g.standard_normal((B, L, H, d), dtype=np.float32))
    v = g.standard_normal((B, L, H, d), dtype=np.float32)
    return f, k, v, q


def skew_generators(n: int, d: int, *, std: float = 0.05, g: np.random.Generator) -> np.ndarray:
    T = np.triu(g.standard_normal((n, d, d), dtype=np.float32) * np.float32(std), k=1)
    return T - np.swapaxes(T, -1, -2)


def dense_cayley_inputs(B: int, L: int, H: int, d: int, *, seed: int = 0, chunk: int = 8192,
                        return_vk: bool = False):
    """U [B*H, L, d, d] (fp32) and V = v k^T [B*H, L, d, d] in the affine-scan API
    layout (sequence index = b*H + h); with ``return_vk`` also v and k
    [B*H, L, d] (V is their fp32 outer product)."""
    g = rng(seed)
    n = B * H * L
    U = np.empty((n, d, d), dtype=np.float32)
    eye = np.eye(d)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        W = skew_generators(e - s, d, g=g).astype(np.float64)
        U[s:e] = np.linalg.solve(eye - W, eye + W).astype(np.float32)
    gate = _sigmoid(g.standard_normal((n,), dtype=np.float32) + np.float32(2.0))
    U *= gate[:, None, None]
    v = g.standard_normal((n, d), dtype=np.float32)
    k = _unit(g.standard_normal((n, d), dtype=np.float32))
    V = (v[:, :, None] * k[:, None, :]).astype(np.float32)
    # [B, L, H, d, d] -> [B*H, L, d, d]
    U = U.reshape(B, L, H, d, d).transpose(0, 2, 1, 3, 4).reshape(B * H, L, d, d)
    V = V.reshape(B, L, H, d, d).transpose(0, 2, 1, 3, 4).reshape(B * H, L, d, d)
    if not return_vk:
        return np.ascontiguousarray(U), np.ascontiguousarray(V)
    v = v.reshape(B, L, H, d).transpose(0, 2, 1, 3).reshape(B * H, L, d)
    k = k.reshape(B, L, H, d).transpose(0, 2, 1, 3).reshape(B * H, L, d)
    return tuple(np.ascontiguousarray(x) for x in (U, V, v, k))


def reference_test_case(batch_size=2, seq_len=17, rank=4, channels=3):
    """The reference's own sanity inputs (sanity_affine_scan.py:11-16): torch seed 42,
    U = I + 0.05 N(0,1), V ~ N(0,1), float64."""
    import torch

    torch.manual_seed(42)
    U = torch.randn(batch_size, seq_len, rank, rank, dtype=torch.float64) * 0.05
    U = U + torch.eye(rank, dtype=torch.float64).view(1, 1, rank, rank)
    V = torch.randn(batch_size, seq_len, rank, channels, dtype=torch.float64)
    return U, V
