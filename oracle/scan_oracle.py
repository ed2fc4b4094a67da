"""CPU oracle for the MOGT scan operator — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this module, and only as the checker / the timed CPU baseline.
No product code path (``mogt_amd``) uses it.

A restatement in numpy of the reference's PyTorch scans (lkcfqy/MOGT
``affine_scan.py``) and of the scan specialisations the GPU kernels implement.
Arithmetic is done in ``state_dtype`` (float64 by default) with the
reference's semantics: ``H_0 = 0``, ``H_t = U_t @ H_{t-1} + V_t``, outputs cast
to ``output_dtype`` only at the end.

How each function is pinned (tests/test_oracle.py):
  affine_scan_sequential      closed-form sum, U=I -> cumsum, constant U ->
                              matrix_power, sequential == doubling == block (1e-10)
  affine_scan_doubling        == sequential (1e-10, the reference's own check)
  affine_scan_block_reference == sequential for several block sizes (1e-10)
  affine_scan_sequential_backward  == finite differences and == the adjoint
                              identity <dH, H(U,V)> linear in V (1e-8)
  diag_scan                   a=1 -> cumsum, a=0 -> b, b=0 -> 0, constant a ->
                              scipy.signal.lfilter, brute-force closed form,
                              == affine_scan_sequential with R=C=1
  coupled_rank_scan           == affine_scan_sequential with U=diag(1-g),
                              V=g*v (the reference's U/V construction)
  fused_scan                  constant U -> matrix_power, == return_prefix U
  rank1_coupled_scan          O(L^2) decayed-attention brute force
  cayley                      Q^T Q = I, == solve((I-W),(I+W))
"""
from __future__ import annotations

import numpy as np


def _check_rank4(U: np.ndarray, V: np.ndarray) -> tuple[int, int, int, int]:
    # affine_scan.py:26-32
    if U.ndim != 4 or V.ndim != 4:
        raise ValueError("U and V must be rank-4 tensors")
    B, L, R, R2 = U.shape
    Bv, Lv, Rv, C = V.shape
    if (B, L, R) != (Bv, Lv, Rv) or R != R2:
        raise ValueError("U must be [B, L, R, R] and V must be [B, L, R, C]")
    return B, L, R, C


def affine_combine(U_next, V_next, U_prev, V_prev):
    """(U_n, V_n) (x) (U_p, V_p) = (U_n U_p, U_n V_p + V_n)  (affine_scan.py:4-11)."""
    return U_next @ U_prev, U_next @ V_prev + V_next


def affine_scan_sequential(U, V, *, state_dtype=np.float64, output_dtype=None,
                           return_prefix=False):
    """H_t = U_t H_{t-1} + V_t, H_0 = 0 (affine_scan.py:14-62).

    Optional U_prefix_t = U_t ... U_1 (affine_scan.py:43-55).
    """
    B, L, R, C = _check_rank4(U, V)
    output_dtype = output_dtype or V.dtype
    Uw = np.asarray(U, dtype=state_dtype)
    Vw = np.asarray(V, dtype=state_dtype)
    H = np.zeros((B, R, C), dtype=state_dtype)
    Hs = np.empty((B, L, R, C), dtype=state_dtype)
    P = np.broadcast_to(np.eye(R, dtype=state_dtype), (B, R, R)).copy() if return_prefix else None
    Ps = np.empty((B, L, R, R), dtype=state_dtype) if return_prefix else None
    for t in range(L):
        H = Uw[:, t] @ H + Vw[:, t]
        Hs[:, t] = H
        if return_prefix:
            P = Uw[:, t] @ P
            Ps[:, t] = P
    if not return_prefix:
        return Hs.astype(output_dtype)
    return Ps.astype(output_dtype), Hs.astype(output_dtype)


def affine_scan_sequential_backward(U, V, grad_H, *, state_dtype=np.float64, need_grad_u=True,
                                    need_grad_v=True):
    """Reverse scan G_t = dH_t + U_{t+1}^T G_{t+1}; dV = G; dU_t = G_t H_{t-1}^T
    (affine_scan.py:65-124)."""
    B, L, R, C = _check_rank4(U, V)
    if grad_H.shape != (B, L, R, C):
        raise ValueError("grad_H must match V shape [B, L, R, C]")
    Uw = np.asarray(U, dtype=state_dtype)
    Vw = np.asarray(V, dtype=state_dtype)
    Gw = np.asarray(grad_H, dtype=state_dtype)
    Hprev = np.empty((B, L, R, C), dtype=state_dtype)
    H = np.zeros((B, R, C), dtype=state_dtype)
    for t in range(L):
        Hprev[:, t] = H
        H = Uw[:, t] @ H + Vw[:, t]
    gU = np.empty_like(Uw) if need_grad_u else None
    gV = np.empty_like(Vw) if need_grad_v else None
    carry = np.zeros((B, R, C), dtype=state_dtype)
    for t in range(L - 1, -1, -1):
        tot = Gw[:, t] + carry
        if need_grad_v:
            gV[:, t] = tot
        if need_grad_u:
            gU[:, t] = tot @ np.swapaxes(Hprev[:, t], -1, -2)
        carry = np.swapaxes(Uw[:, t], -1, -2) @ tot
    return (gU.astype(U.dtype) if gU is not None else None,
            gV.astype(V.dtype) if gV is not None else None)


def affine_scan_doubling(U, V, *, state_dtype=np.float64, output_dtype=None, return_prefix=False):
    """Hillis-Steele inclusive scan with doubling offsets (affine_scan.py:127-172)."""
    B, L, R, C = _check_rank4(U, V)
    output_dtype = output_dtype or V.dtype
    P = np.array(U, dtype=state_dtype)
    H = np.array(V, dtype=state_dtype)
    off = 1
    while off < L:
        Pp, Hp = P.copy(), H.copy()
        P[:, off:] = Pp[:, off:] @ Pp[:, :-off]
        H[:, off:] = Pp[:, off:] @ Hp[:, :-off] + Hp[:, off:]
        off *= 2
    if not return_prefix:
        return H.astype(output_dtype)
    return P.astype(output_dtype), H.astype(output_dtype)


def affine_scan_block_reference(U, V, *, block_size=256, state_dtype=np.float64, output_dtype=None,
                                carry_scan="sequential", return_prefix=False):
    """Three-phase chunked scan (affine_scan.py:175-278): local prefixes per block,
    scan of block summaries, carry for block k = inclusive prefix of block k-1
    ((I, 0) for block 0), apply U_loc @ H_carry + H_loc."""
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    if carry_scan not in {"sequential", "doubling"}:
        raise ValueError("carry_scan must be 'sequential' or 'doubling'")
    B, L, R, C = _check_rank4(U, V)
    output_dtype = output_dtype or V.dtype
    nb = (L + block_size - 1) // block_size
    locP, locH, sumP, sumH, ranges = [], [], [], [], []
    for k in range(nb):
        s, e = k * block_size, min((k + 1) * block_size, L)
        ranges.append((s, e))
        p_, h_ = affine_scan_sequential(U[:, s:e], V[:, s:e], state_dtype=state_dtype,
                                        output_dtype=state_dtype, return_prefix=True)
        locP.append(p_)
        locH.append(h_)
        sumP.append(p_[:, -1])
        sumH.append(h_[:, -1])
    bP = np.stack(sumP, axis=1)
    bH = np.stack(sumH, axis=1)
    scan = affine_scan_sequential if carry_scan == "sequential" else affine_scan_doubling
    incP, incH = scan(bP, bH, state_dtype=state_dtype, output_dtype=state_dtype, return_prefix=True)
    cP = np.broadcast_to(np.eye(R, dtype=state_dtype), (B, nb, R, R)).copy()
    cH = np.zeros((B, nb, R, C), dtype=state_dtype)
    if nb > 1:
        cP[:, 1:] = incP[:, :-1]
        cH[:, 1:] = incH[:, :-1]
    outP, outH = [], []
    for k in range(nb):
        outP.append(locP[k] @ cP[:, k:k + 1])
        outH.append(locP[k] @ cH[:, k:k + 1] + locH[k])
    Pout = np.concatenate(outP, axis=1).astype(output_dtype)
    Hout = np.concatenate(outH, axis=1).astype(output_dtype)
    return (Pout, Hout) if return_prefix else Hout


def local_scan(U, V, *, block_size=256, state_dtype=np.float64):
    """Block-local prefixes and per-block summaries, tail padded with (I, 0)
    (triton_scan.py:178-229 / :54-148): returns U_prefix, H_prefix [B,L,...]
    and U_summary, H_summary [B, nb, ...]."""
    B, L, R, C = _check_rank4(U, V)
    nb = (L + block_size - 1) // block_size
    Up = np.empty((B, L, R, R), dtype=state_dtype)
    Hp = np.empty((B, L, R, C), dtype=state_dtype)
    Us = np.empty((B, nb, R, R), dtype=state_dtype)
    Hs = np.empty((B, nb, R, C), dtype=state_dtype)
    for k in range(nb):
        s, e = k * block_size, min((k + 1) * block_size, L)
        p_, h_ = affine_scan_sequential(U[:, s:e], V[:, s:e], state_dtype=state_dtype,
                                        output_dtype=state_dtype, return_prefix=True)
        Up[:, s:e] = p_
        Hp[:, s:e] = h_
        Us[:, k] = p_[:, -1]   # identity padding leaves the last real prefix unchanged
        Hs[:, k] = h_[:, -1]
    return Up, Hp, Us, Hs


def fused_scan(U, *, state_dtype=np.float64):
    """Transport-only prefix product Y_t = U_t Y_{t-1}, Y_0 = I
    (triton_scan.py:13-51, :151-175)."""
    B, L, R, R2 = U.shape
    if R != R2:
        raise ValueError("U must be [B, L, R, R]")
    Uw = np.asarray(U, dtype=state_dtype)
    Y = np.broadcast_to(np.eye(R, dtype=state_dtype), (B, R, R)).copy()
    out = np.empty((B, L, R, R), dtype=state_dtype)
    for t in range(L):
        Y = Uw[:, t] @ Y
        out[:, t] = Y
    return out


def diag_scan(a, b, *, state_dtype=np.float64, return_prefix=False):
    """Per-feature h_t = a_t h_{t-1} + b_t over [B, L, D]: the R=C=1 case of
    affine_scan_sequential (affine_scan.py:48-55) with D folded into batch."""
    a = np.asarray(a, dtype=state_dtype)
    b = np.asarray(b, dtype=state_dtype)
    if a.shape != b.shape or a.ndim != 3:
        raise ValueError("a and b must both be [B, L, D]")
    B, L, D = a.shape
    h = np.empty_like(b)
    P = np.empty_like(a) if return_prefix else None
    hh = np.zeros((B, D), dtype=state_dtype)
    pp = np.ones((B, D), dtype=state_dtype)
    for t in range(L):
        hh = a[:, t] * hh + b[:, t]
        h[:, t] = hh
        if return_prefix:
            pp = a[:, t] * pp
            P[:, t] = pp
    return (P, h) if return_prefix else h


def sigmoid(x):
    x = np.asarray(x, dtype=np.float64)
    return 1.0 / (1.0 + np.exp(-x))


def round_bf16(x):
    """Round float32 values to bfloat16 (nearest-even) and back to float32."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    r = np.where(nan, ((u >> 16) | 0x40) << 16, r)
    return r.astype(np.uint32).view(np.float32)


def coupled_gate_inputs(gate_logits, v_raw, rank, *, damping=1.0, v_is_bf16=False):
    """The (a, b) pair the coupled MOGT mixer feeds its scan (model_mogt.py:166-182,
    identity connection _build_transport :91-102, damping :101-102):
    g = sigmoid(z) in fp32; U = damping*(1-g) on the rank diagonal;
    V = V_raw * g.to(V_raw.dtype), in bf16 when V_raw is bf16."""
    z = np.asarray(gate_logits, dtype=np.float32)
    v = np.asarray(v_raw, dtype=np.float32)
    B, L, D = v.shape
    c = D // rank
    g = (1.0 / (1.0 + np.exp(-z.astype(np.float64)))).astype(np.float32)
    a = (np.float32(damping) * (np.float32(1.0) - g)).astype(np.float32)
    if v_is_bf16:
        prod = v * round_bf16(np.repeat(g, c, axis=-1))
        b = round_bf16(prod)
    else:
        b = v * np.repeat(g, c, axis=-1)
    return np.repeat(a, c, axis=-1), b


def coupled_rank_scan(gate_logits, v_raw, rank, *, damping=1.0, v_is_bf16=False,
                      state_dtype=np.float64):
    """Scan of the coupled write-forget mixer, H flattened to [B, L, r*c]."""
    a, b = coupled_gate_inputs(gate_logits, v_raw, rank, damping=damping, v_is_bf16=v_is_bf16)
    return diag_scan(a, b, state_dtype=state_dtype)


def rank1_coupled_scan(f, k, v, q, *, state_dtype=np.float64):
    """S_t = f_t S_{t-1} + (1 - f_t) v_t k_t^T, y_t = S_t q_t per (batch, head).

    The affine recurrence of affine_scan.py:48-55 with U_t = f_t I and the
    rank-1 write V_t = (1-f_t) v_t k_t^T; shapes f [B,L,H], k/v/q [B,L,H,d]."""
    f = np.asarray(f, dtype=state_dtype)
    k = np.asarray(k, dtype=state_dtype)
    v = np.asarray(v, dtype=state_dtype)
    q = np.asarray(q, dtype=state_dtype)
    B, L, H, d = k.shape
    S = np.zeros((B, H, d, d), dtype=state_dtype)
    y = np.empty((B, L, H, d), dtype=state_dtype)
    for t in range(L):
        ft = f[:, t][:, :, None, None]
        S = ft * S + (1.0 - ft) * (v[:, t][:, :, :, None] * k[:, t][:, :, None, :])
        y[:, t] = np.einsum("bhij,bhj->bhi", S, q[:, t])
    return y


def cayley(W):
    """(I - W)^{-1} (I + W) for skew-symmetric W (batched over leading dims)."""
    W = np.asarray(W, dtype=np.float64)
    n = W.shape[-1]
    eye = np.eye(n)
    return np.linalg.solve(eye - W, eye + W)
