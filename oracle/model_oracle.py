"""CPU oracle of the MOGT block and backbone forward — TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module.  A float64 CPU restatement of
model_mogt.py:9-30 (RMSNorm, SwiGLU), :79-258 (MOGTBlock.forward) and
:270-287 (MOGTModel.forward) that works on a plain dict of weights, with the
scan taken from the pinned numpy oracle (scan_oracle.affine_scan_sequential).
Everything else is composed from torch library routines (linear, sigmoid,
silu, matrix_exp, linalg.solve), so the only in-house arithmetic is the scan,
which tests/test_oracle.py pins independently.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import scan_oracle as so


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    # model_mogt.py:15-20
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def swiglu(x, w1, w2, w3):
    # model_mogt.py:29-30
    return F.linear(F.silu(F.linear(x, w1)) * F.linear(x, w2), w3)


def block_forward(p: dict, x: torch.Tensor, prefix: torch.Tensor | None, cfg: dict) -> torch.Tensor:
    """One MOGTBlock.forward (model_mogt.py:124-258) in float64.

    ``p`` holds the block's weights under the reference's parameter names;
    ``cfg`` the duck-typed attributes (connection_impl, connection_damping,
    value_gate_input_mode, couple_forget_to_value_gate, transport_gate_mode,
    transport_gate_scale, mogt_residual_scale, mogt_ffn_residual_scale, r)."""
    r = cfg["r"]
    B, L, D = x.shape
    c = D // r
    residual = x
    xn = rmsnorm(x, p["norm_mogt.weight"])
    impl = cfg.get("connection_impl", "matrix_exp")
    damping = float(cfg.get("connection_damping", 0.999))
    if impl == "identity":
        U = torch.eye(r, dtype=x.dtype).expand(B, L, r, r)
    else:
        A_raw = F.linear(xn, p["phi_conn.weight"]).view(B, L, r, r)
        A = (A_raw - A_raw.transpose(-2, -1)) / r
        if impl == "matrix_exp":
            U = torch.matrix_exp(A)
        elif impl == "cayley":
            eye = torch.eye(r, dtype=x.dtype)
            U = torch.linalg.solve(eye - 0.5 * A, eye + 0.5 * A)
        else:
            raise ValueError(impl)
    U = U * damping
    if "phi_transport_gate.weight" in p:
        g = F.linear(xn, p["phi_transport_gate.weight"], p.get("phi_transport_gate.bias"))
        g = g.view(B, L, 1, 1) if g.size(-1) == 1 else g.view(B, L, r, 1)
        mode = cfg.get("transport_gate_mode", "multiply")
        scale = float(cfg.get("transport_gate_scale", 1.0))
        if mode == "multiply":
            gate = torch.sigmoid(g)
        elif mode == "residual":
            gate = 1.0 + scale * torch.tanh(g)
        else:
            gate = 1.0 - scale * F.relu(torch.tanh(g))
        U = U * gate
    V = F.linear(xn, p["phi_val.weight"]).view(B, L, r, c)
    if "phi_value_gate.weight" in p:
        mode = cfg.get("value_gate_input_mode", "current")
        parts = [xn]
        if "prev" in mode:
            prev = torch.zeros_like(xn)
            prev[:, 1:] = xn[:, :-1]
            parts.append(prev)
        if "prefix" in mode:
            pre = torch.zeros_like(xn[:, :1]) if prefix is None else prefix.view(B, 1, D)
            parts.append(pre.expand(B, L, D))
        gl = F.linear(torch.cat(parts, dim=-1), p["phi_value_gate.weight"], p.get("phi_value_gate.bias"))
        vg = torch.sigmoid(gl)
        vg = vg.view(B, L, 1, 1) if vg.size(-1) == 1 else vg.view(B, L, r, 1)
        V = V * vg
        if cfg.get("couple_forget_to_value_gate", False):
            U = U * (1.0 - vg)
    H = so.affine_scan_sequential(U.contiguous().numpy(), V.contiguous().numpy(),
                                  state_dtype=np.float64, output_dtype=np.float64)
    H = torch.from_numpy(H).reshape(B, L, D)
    Z = F.linear(rmsnorm(H, p["norm_out.weight"]), p["theta_read.weight"])
    x = residual + float(cfg.get("mogt_residual_scale", 1.0)) * Z
    x = x + float(cfg.get("mogt_ffn_residual_scale", 1.0)) * swiglu(
        rmsnorm(x, p["norm_ffn.weight"]), p["ffn.w1.weight"], p["ffn.w2.weight"], p["ffn.w3.weight"])
    return x


def model_forward(state: dict, input_ids: torch.Tensor, n_layers: int, cfg: dict,
                  prefix_position: int | None = None) -> torch.Tensor:
    """MOGTModel.forward (model_mogt.py:270-287) in float64 on a state dict
    whose keys are the reference's (``embedding.weight``, ``blocks.{i}.*``,
    ``norm_f.weight``)."""
    x = F.embedding(input_ids, state["embedding.weight"])
    prefix = None
    if prefix_position is not None and -x.size(1) <= prefix_position < x.size(1):
        prefix = x[:, prefix_position, :]
    for i in range(n_layers):
        pre = f"blocks.{i}."
        p = {k[len(pre):]: v for k, v in state.items() if k.startswith(pre)}
        x = block_forward(p, x, prefix, cfg)
    return rmsnorm(x, state["norm_f.weight"])
