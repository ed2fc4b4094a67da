"""CPU oracle of the MOGT block and backbone forward — TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module.  A float64 CPU restatement of
model_mogt.py:9-30 (RMSNorm, SwiGLU), :79-258 (MOGTBlock.forward) and
:270-287 (MOGTModel.forward) that works on a plain dict of weights, with the
scan taken from the pinned numpy oracle (scan_oracle.affine_scan_sequential).
Everything else is composed from torch library routines (linear, sigmoid,
silu, matrix_exp, linalg.solve), so the only in-house arithmetic is the scan,
which tests/test_oracle.py pins independently.  The composition itself is
pinned by tests/test_golden_model.py against float64 outputs of the reference's
own classes (tests/golden/model_fixtures.npz).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import scan_oracle as so


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6, ref_casts: bool = False) -> torch.Tensor:
    # model_mogt.py:15-20; with ref_casts the statistics run in float32 and the
    # result is cast back (``self._norm(x.float()).type_as(x)``)
    xs = x.float() if ref_casts else x
    return (xs * torch.rsqrt(xs.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * w


def swiglu(x, w1, w2, w3):
    # model_mogt.py:29-30
    return F.linear(F.silu(F.linear(x, w1)) * F.linear(x, w2), w3)


def block_forward(p: dict, x: torch.Tensor, prefix: torch.Tensor | None, cfg: dict,
                  ref_casts: bool = False) -> torch.Tensor:
    """One MOGTBlock.forward (model_mogt.py:124-258) in float64.

    ``p`` holds the block's weights under the reference's parameter names;
    ``cfg`` the duck-typed attributes (connection_impl, connection_damping,
    value_gate_input_mode, couple_forget_to_value_gate, transport_gate_mode,
    transport_gate_scale, mogt_residual_scale, mogt_ffn_residual_scale, r, and
    residual_gate for mogt_residual_gate_enabled).

    ``scan_impl = "transport_triton"`` (or ``fast_throughput_mode``) selects the
    reference's transport-only mode; every other scan_impl is the affine scan.

    ``ref_casts=False`` keeps every intermediate in x's dtype (the oracle of
    the GPU paths).  ``ref_casts=True`` reproduces the reference's own float32
    steps for any input dtype: RMSNorm statistics (:19), the connection map
    (:80, float32 A and U), the transport and value gates (:143, :171, ``.float()``
    then cast back), and the scan state (:227-231, ``state_dtype=float32``, a
    torch.bmm loop as affine_scan.py:48-55)."""
    r = cfg["r"]
    B, L, D = x.shape
    c = D // r
    dt = x.dtype
    wd = torch.float32 if ref_casts else dt      # dtype of the reference's float32 steps
    residual = x
    xn = rmsnorm(x, p["norm_mogt.weight"], ref_casts=ref_casts)
    impl = cfg.get("connection_impl", "matrix_exp")
    damping = float(cfg.get("connection_damping", 0.999))
    if impl == "identity":
        U = torch.eye(r, dtype=wd).expand(B, L, r, r)
    else:
        A_raw = F.linear(xn, p["phi_conn.weight"]).view(B, L, r, r)
        A = ((A_raw - A_raw.transpose(-2, -1)) / r).to(wd)
        if impl == "matrix_exp":
            U = torch.matrix_exp(A)
        elif impl == "cayley":
            eye = torch.eye(r, dtype=wd)
            U = torch.linalg.solve(eye - 0.5 * A, eye + 0.5 * A)
        else:
            raise ValueError(impl)
    U = (U * damping).to(xn.dtype)
    if "phi_transport_gate.weight" in p:
        g = F.linear(xn, p["phi_transport_gate.weight"], p.get("phi_transport_gate.bias")).to(wd)
        g = g.view(B, L, 1, 1) if g.size(-1) == 1 else g.view(B, L, r, 1)
        mode = cfg.get("transport_gate_mode", "multiply")
        scale = float(cfg.get("transport_gate_scale", 1.0))
        if mode == "multiply":
            gate = torch.sigmoid(g)
        elif mode == "residual":
            gate = 1.0 + scale * torch.tanh(g)
        else:
            gate = 1.0 - scale * F.relu(torch.tanh(g))
        U = U * gate.to(U.dtype)
    V = F.linear(xn, p["phi_val.weight"]).view(B, L, r, c)
    if "phi_value_gate.weight" in p:
        mode = cfg.get("value_gate_input_mode", "current")
        parts = [xn]
        if "prev" in mode:
            prev = torch.zeros_like(xn)
            prev[:, 1:] = xn[:, :-1]
            parts.append(prev)
        if "prefix" in mode:
            pre = torch.zeros_like(xn[:, :1]) if prefix is None else prefix.to(xn.dtype).view(B, 1, D)
            parts.append(pre.expand(B, L, D))
        gl = F.linear(torch.cat(parts, dim=-1), p["phi_value_gate.weight"], p.get("phi_value_gate.bias")).to(wd)
        vg = torch.sigmoid(gl)
        vg = vg.view(B, L, 1, 1) if vg.size(-1) == 1 else vg.view(B, L, r, 1)
        V = V * vg.to(V.dtype)
        if cfg.get("couple_forget_to_value_gate", False):
            U = U * (1.0 - vg).to(U.dtype)
    if cfg.get("scan_impl") == "transport_triton" or cfg.get("fast_throughput_mode"):
        # transport-only mode (model_mogt.py:187-192): V_t = Y_t V_raw with the
        # prefix product Y_t = U_t Y_{t-1}, Y_0 = I (triton_scan.py:37-48), in
        # U's dtype as the Triton kernel keeps it
        Y = U.new_empty(U.shape)
        acc = torch.eye(r, dtype=U.dtype).expand(B, r, r)
        for t in range(L):
            acc = torch.matmul(U[:, t], acc)
            Y[:, t] = acc
        H = torch.matmul(Y, V.to(Y.dtype))
    elif ref_casts or (torch.is_grad_enabled() and (U.requires_grad or V.requires_grad)):
        # the reference's bmm loop: float32 state with ref_casts; otherwise a
        # float64 state, differentiable for autograd checks of the GPU backward
        from .torch_ref import affine_scan_sequential_torch

        H = affine_scan_sequential_torch(U, V, state_dtype=torch.float32 if ref_casts else torch.float64,
                                         output_dtype=U.dtype)
    else:
        H = torch.from_numpy(so.affine_scan_sequential(U.contiguous().numpy(), V.contiguous().numpy(),
                                                       state_dtype=np.float64, output_dtype=np.float64))
    H = H.reshape(B, L, D).to(dt)
    Z = F.linear(rmsnorm(H, p["norm_out.weight"], ref_casts=ref_casts), p["theta_read.weight"])
    scale = float(cfg.get("mogt_residual_scale", 1.0))
    if cfg.get("residual_gate") and "mogt_residual_gate_logit" in p:
        # model_mogt.py:243-247: learned gate on the mixer's residual term
        x = residual + (scale * torch.sigmoid(p["mogt_residual_gate_logit"]).to(Z.dtype)) * Z
    else:
        x = residual + scale * Z
    x = x + float(cfg.get("mogt_ffn_residual_scale", 1.0)) * swiglu(
        rmsnorm(x, p["norm_ffn.weight"], ref_casts=ref_casts), p["ffn.w1.weight"], p["ffn.w2.weight"],
        p["ffn.w3.weight"])
    return x


def model_forward(state: dict, input_ids: torch.Tensor, n_layers: int, cfg,
                  prefix_position: int | None = None, block_outputs: list | None = None,
                  ref_casts: bool = False) -> torch.Tensor:
    """MOGTModel.forward (model_mogt.py:270-287) in float64 on a state dict
    whose keys are the reference's (``embedding.weight``, ``blocks.{i}.*``,
    ``norm_f.weight``).  ``cfg`` is one block configuration for every layer or
    a list with one per layer; ``block_outputs`` (optional) collects each
    block's output; ``ref_casts`` as in block_forward."""
    x = F.embedding(input_ids, state["embedding.weight"])
    prefix = None
    if prefix_position is not None and -x.size(1) <= prefix_position < x.size(1):
        prefix = x[:, prefix_position, :]
    for i in range(n_layers):
        pre = f"blocks.{i}."
        p = {k[len(pre):]: v for k, v in state.items() if k.startswith(pre)}
        x = block_forward(p, x, prefix, cfg[i] if isinstance(cfg, (list, tuple)) else cfg,
                          ref_casts=ref_casts)
        if block_outputs is not None:
            block_outputs.append(x)
    return rmsnorm(x, state["norm_f.weight"], ref_casts=ref_casts)
