"""MOGT layer and backbone on MI355X (drop-in for lkcfqy/MOGT ``model_mogt.py``).

Same classes, constructor arguments, parameter names and duck-typed
configuration attributes as the reference (model_mogt.py:9-380); configs and
state dicts carry over.  The scan always runs on the HIP kernels:

* generic path (any configuration, autograd): the reference's computation
  op for op on the GPU, with every ``scan_impl`` routed to the HIP affine scan
  (``sequential``, ``parallel_reference``, ``block_reference`` and
  ``triton_hybrid`` evaluate the same recurrence; ``transport_triton`` runs the
  HIP prefix product like the reference's transport-only mode);
* fused path (inference with an identity connection and a rank-wide value gate
  coupled to the forget gate -- the configuration of the reference's backbone
  benchmark, benchmark_backbone_throughput.py:40-57): ``U = damping*(1-g)`` is
  diagonal per rank, so gate + scan run as one HIP kernel (no [B,L,r,r] U, no
  [B,L,3d] concatenation, no phi_conn GEMM whose result the identity
  connection discards), RMSNorms and the SwiGLU gate are single-pass HIP
  kernels, and each block's residual add is folded into the next RMSNorm.

Tensors must be on the GPU; there is no CPU execution path.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

from . import ops, triton_scan
from .chunked_lm_loss import chunked_linear_cross_entropy


def _autocast_dtype() -> torch.dtype | None:
    if torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return None


def _gemm_weight(owner: nn.Module, name: str, params: tuple, build):
    """A GEMM operand built from parameters (a concatenation of weights, cast
    to the autocast dtype when autocast is on -- the cast F.linear would make).
    Without gradient recording it is cached on ``owner`` until a parameter
    changes (storage or version counter), the autocast dtype or the inference
    mode flag changes; with gradients it is rebuilt on every call so autograd
    reaches the parameters."""
    ad = _autocast_dtype()

    def make():
        w = build()
        return w.to(ad) if ad is not None and w.is_floating_point() else w

    if torch.is_grad_enabled():
        return make()
    key = (tuple((p.data_ptr(), p._version, p.dtype) for p in params), ad, torch.is_inference_mode_enabled())
    cache = owner.__dict__.setdefault("_gemm_weight_cache", {})
    hit = cache.get(name)
    if hit is None or hit[0] != key:
        hit = (key, make())
        cache[name] = hit
    return hit[1]


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps), computed in fp32, ``type_as(x)``, times
    ``weight`` (model_mogt.py:9-20)."""

    def __init__(self, d_model: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d_model))

    def _norm(self, x):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps)

    def forward(self, x):
        ops.require_cuda("RMSNorm", x)
        return ops.rmsnorm(x, self.weight, self.eps,
                           out_dtype=torch.promote_types(x.dtype, self.weight.dtype))


class SwiGLU(nn.Module):
    """w3(silu(w1 x) * w2 x) (model_mogt.py:22-30)."""

    def __init__(self, d_model: int, hidden_dim: int):
        super().__init__()
        self.w1 = nn.Linear(d_model, hidden_dim, bias=False)
        self.w2 = nn.Linear(d_model, hidden_dim, bias=False)
        self.w3 = nn.Linear(hidden_dim, d_model, bias=False)

    def forward(self, x):
        # one GEMM against [w1; w2], then the fused gate (autograd through the
        # silu_mul backward kernel and torch.cat back to w1, w2)
        w12 = _gemm_weight(self, "w12", (self.w1.weight, self.w2.weight),
                           lambda: torch.cat([self.w1.weight, self.w2.weight], dim=0))
        w3 = _gemm_weight(self, "w3", (self.w3.weight,), lambda: self.w3.weight)
        return F.linear(ops.silu_mul(F.linear(x, w12)), w3)


def reference_ffn_hidden(d_model: int) -> int:
    """256 * ceil((8 d / 3) / 256) -- model_mogt.py:66-68 (2048 at d = 768)."""
    return 256 * ((int(8 * d_model / 3) + 255) // 256)


class MOGTBlock(nn.Module):
    """One MOGT layer (model_mogt.py:32-258).  ``ffn_hidden`` defaults to the
    reference's formula; pass e.g. ``4 * d_model`` for a 4x gated MLP."""

    def __init__(self, d_model: int, r: int = 16, ffn_hidden: int | None = None):
        super().__init__()
        self.r = r
        self.d_model = d_model
        self.connection_impl = "matrix_exp"
        self.connection_damping = 0.999
        self.register_buffer("_identity_r", torch.eye(r, dtype=torch.float32), persistent=False)
        assert d_model % r == 0, "d_model must be divisible by the rank r"
        self.c = d_model // r
        self.norm_mogt = RMSNorm(d_model)
        self.phi_conn = nn.Linear(d_model, r * r, bias=False)
        self.phi_val = nn.Linear(d_model, r * self.c, bias=False)
        self.norm_out = RMSNorm(d_model)
        self.theta_read = nn.Linear(r * self.c, d_model, bias=False)
        self.norm_ffn = RMSNorm(d_model)
        self.ffn = SwiGLU(d_model, ffn_hidden or reference_ffn_hidden(d_model))

    # ---------------------------------------------------------------- config
    def _resolve_scan_impl(self):
        if getattr(self, "fast_throughput_mode", False):
            return "transport_triton"
        return getattr(self, "scan_impl", "sequential")

    def _resolve_connection_impl(self):
        return getattr(self, "connection_impl", "matrix_exp")

    def _residual_scale(self, like: torch.Tensor) -> float:
        scale = float(getattr(self, "mogt_residual_scale", 1.0))
        gate_logit = getattr(self, "mogt_residual_gate_logit", None)
        if getattr(self, "mogt_residual_gate_enabled", False) and gate_logit is not None:
            gate = torch.sigmoid(gate_logit).to(dtype=like.dtype, device=like.device)
            return float(scale * gate)
        return scale

    def fused_path_ok(self) -> bool:
        """Identity connection, no transport gate, rank-wide value gate coupled to
        the forget gate, an affine scan_impl; with autograd, no learned residual
        gate (its scale enters the fused residual update as a constant)."""
        gate = getattr(self, "phi_value_gate", None)
        if (torch.is_grad_enabled() and getattr(self, "mogt_residual_gate_enabled", False)
                and any(p.requires_grad for p in self.parameters())):
            return False
        return (self._resolve_connection_impl() == "identity"
                and getattr(self, "phi_transport_gate", None) is None
                and isinstance(gate, nn.Linear) and gate.out_features == self.r
                and bool(getattr(self, "couple_forget_to_value_gate", False))
                and self._resolve_scan_impl() in {"triton_hybrid", "sequential",
                                                  "parallel_reference", "block_reference"})

    # ------------------------------------------------------- reference pieces
    def _build_transport(self, A: torch.Tensor, output_dtype: torch.dtype):
        """model_mogt.py:79-102."""
        A_fp32 = (A / self.r).to(torch.float32)
        impl = self._resolve_connection_impl()
        if impl in ("matrix_exp", "cayley"):
            # HIP connection-map kernel (A is skew: A_raw - A_raw^T); damping and
            # the output cast are applied below exactly as in the reference
            name = "mogt.matrix_exp" if impl == "matrix_exp" else "mogt.cayley_solve"
            with torch.autograd.profiler.record_function(name):
                U_fp32 = ops.connection_map(A_fp32, impl)
        elif impl == "identity":
            U_fp32 = self._identity_r.view(1, 1, self.r, self.r).expand(
                A.shape[0], A.shape[1], self.r, self.r)
        else:
            raise ValueError(f"Unsupported connection_impl: {impl}")
        damping = float(getattr(self, "connection_damping", 0.999))
        return (U_fp32 * damping).to(output_dtype)

    def _build_value_gate_input(self, x_norm: torch.Tensor, prefix_condition: torch.Tensor | None):
        """model_mogt.py:104-122."""
        mode = getattr(self, "value_gate_input_mode", "current")
        if mode == "current":
            return x_norm
        parts = [x_norm]
        if "prev" in mode:
            prev = torch.zeros_like(x_norm)
            prev[:, 1:] = x_norm[:, :-1]
            parts.append(prev)
        if "prefix" in mode:
            if prefix_condition is None:
                prefix = torch.zeros_like(x_norm[:, :1])
            else:
                prefix = prefix_condition.to(dtype=x_norm.dtype).view(x_norm.size(0), 1, x_norm.size(-1))
            parts.append(prefix.expand(x_norm.size(0), x_norm.size(1), x_norm.size(-1)))
        return torch.cat(parts, dim=-1)

    # ---------------------------------------------------------------- forward
    def forward(self, x, prefix_condition=None):
        ops.require_cuda("MOGTBlock", x)
        if self.fused_path_ok() and x.dtype == torch.float32:
            x, (z, s) = self.forward_fused(x, prefix_condition, None)
            return x + s * z
        return self._forward_generic(x, prefix_condition)

    def _forward_generic(self, x, prefix_condition):
        """model_mogt.py:124-258 with the scan on the HIP kernels."""
        residual = x
        x_norm = self.norm_mogt(x)
        B, L, D = x_norm.shape
        impl = self._resolve_connection_impl()
        with torch.autograd.profiler.record_function("mogt.connection"):
            if impl == "identity":
                A = x_norm.new_zeros(B, L, self.r, self.r)   # identity ignores A
            else:
                A_raw = self.phi_conn(x_norm).view(B, L, self.r, self.r)
                A = A_raw - A_raw.transpose(-2, -1)
        with torch.autograd.profiler.record_function("mogt.connection_map"):
            U = self._build_transport(A, x_norm.dtype)
            phi_transport_gate = getattr(self, "phi_transport_gate", None)
            if phi_transport_gate is not None:
                gate_raw = phi_transport_gate(x_norm).float()
                if gate_raw.size(-1) == 1:
                    gate_raw = gate_raw.view(B, L, 1, 1)
                elif gate_raw.size(-1) == self.r:
                    gate_raw = gate_raw.view(B, L, self.r, 1)
                else:
                    raise ValueError("phi_transport_gate must output either 1 scalar or r rank gates")
                gate_mode = getattr(self, "transport_gate_mode", "multiply")
                if gate_mode == "multiply":
                    gate = torch.sigmoid(gate_raw)
                elif gate_mode == "residual":
                    gate = 1.0 + float(getattr(self, "transport_gate_scale", 1.0)) * torch.tanh(gate_raw)
                elif gate_mode == "forget_relu":
                    gate = 1.0 - float(getattr(self, "transport_gate_scale", 1.0)) * F.relu(torch.tanh(gate_raw))
                else:
                    raise ValueError(f"Unsupported transport_gate_mode: {gate_mode}")
                U = U * gate.to(U.dtype)
        with torch.autograd.profiler.record_function("mogt.value_projection"):
            V_t_raw = self.phi_val(x_norm).view(B, L, self.r, self.c)
            phi_value_gate = getattr(self, "phi_value_gate", None)
            if phi_value_gate is not None:
                value_gate_raw = phi_value_gate(self._build_value_gate_input(x_norm, prefix_condition)).float()
                if value_gate_raw.size(-1) == 1:
                    value_gate = torch.sigmoid(value_gate_raw).view(B, L, 1, 1)
                elif value_gate_raw.size(-1) == self.r:
                    value_gate = torch.sigmoid(value_gate_raw).view(B, L, self.r, 1)
                else:
                    raise ValueError("phi_value_gate must output either 1 scalar or r rank gates")
                V_t_raw = V_t_raw * value_gate.to(V_t_raw.dtype)
                if getattr(self, "couple_forget_to_value_gate", False):
                    U = U * (1.0 - value_gate).to(U.dtype)
        scan_impl = self._resolve_scan_impl()
        with torch.autograd.profiler.record_function("mogt.affine_scan"):
            if scan_impl == "transport_triton":
                Y = triton_scan.triton_fused_scan(U)
                V_t = torch.matmul(Y, V_t_raw.to(Y.dtype))
            elif scan_impl in {"triton_hybrid", "parallel_reference", "block_reference", "sequential"}:
                if scan_impl == "block_reference" or scan_impl == "triton_hybrid":
                    carry = getattr(self, "block_carry_scan", "sequential")
                else:
                    carry = "sequential"
                V_t = triton_scan.triton_affine_scan_hybrid(
                    U, V_t_raw, block_size=getattr(self, "scan_block_size", 256),
                    block_c=getattr(self, "scan_block_c", 32), carry_scan=carry,
                    output_dtype=U.dtype)
            else:
                raise ValueError(f"Unsupported scan_impl: {scan_impl}")
        V_t_flat = V_t.reshape(B, L, self.d_model)
        with torch.autograd.profiler.record_function("mogt.readout"):
            Z = self.theta_read(self.norm_out(V_t_flat))
        mogt_residual_scale = float(getattr(self, "mogt_residual_scale", 1.0))
        gate_logit = getattr(self, "mogt_residual_gate_logit", None)
        if getattr(self, "mogt_residual_gate_enabled", False) and gate_logit is not None:
            gate = torch.sigmoid(gate_logit).to(dtype=Z.dtype, device=Z.device)
            x = residual + ((mogt_residual_scale * gate) * Z)
        else:
            x = residual + (mogt_residual_scale * Z)
        residual = x
        with torch.autograd.profiler.record_function("mogt.ffn"):
            x_norm = self.norm_ffn(x)
            x = residual + (float(getattr(self, "mogt_ffn_residual_scale", 1.0)) * self.ffn(x_norm))
        return x

    def _gate_logits(self, xn: torch.Tensor, prefix_condition: torch.Tensor | None) -> torch.Tensor:
        """phi_value_gate over [x, x_{t-1}, prefix] without materialising the
        concatenation: W = [W_cur | W_prev | W_pref] (model_mogt.py:104-122)."""
        gate: nn.Linear = self.phi_value_gate
        mode = getattr(self, "value_gate_input_mode", "current")
        D = self.d_model
        W = gate.weight
        parts = [W[:, :D]]
        off = D
        if "prev" in mode:
            parts.append(W[:, off:off + D])
            off += D
        Wg = _gemm_weight(self, "gate", (W,), lambda: torch.cat(parts, dim=0))
        y = F.linear(xn, Wg).float()   # [B, L, r * n_parts]
        r = self.r
        z = y[..., :r]
        if "prev" in mode:
            z = z.clone()
            z[:, 1:] += y[:, :-1, r:2 * r]
        const = gate.bias.float() if gate.bias is not None else torch.zeros(r, device=xn.device)
        if "prefix" in mode and prefix_condition is not None:
            pref = prefix_condition.to(dtype=xn.dtype).view(xn.size(0), 1, D)
            const = const + F.linear(pref, W[:, off:off + D]).float()
        return (z + const).contiguous()

    def forward_fused(self, x: torch.Tensor, prefix_condition, pending):
        """Fused forward (differentiable: every kernel has its backward).  ``pending = (z, scale)`` is the previous
        block's last residual term (added here inside the first RMSNorm).
        Returns ``(x_after_mixer, (ffn_out, ffn_scale))``: the caller adds the
        FFN term (or hands it to the next block)."""
        ad = _autocast_dtype()
        gemm_dtype = ad or x.dtype
        eps = self.norm_mogt.eps
        if pending is None:
            xn = ops.rmsnorm(x, self.norm_mogt.weight, eps, out_dtype=gemm_dtype)
        else:
            x, xn = ops.add_rmsnorm(x, pending[0], pending[1], self.norm_mogt.weight, eps,
                                    out_dtype=gemm_dtype)
        with torch.autograd.profiler.record_function("mogt.value_projection"):
            v_raw = F.linear(xn, _gemm_weight(self, "phi_val", (self.phi_val.weight,), lambda: self.phi_val.weight))
            z = self._gate_logits(xn, prefix_condition)
        with torch.autograd.profiler.record_function("mogt.affine_scan"):
            h = ops.coupled_rank_scan(z, v_raw, damping=float(getattr(self, "connection_damping", 0.999)),
                                      out_dtype=torch.float32)
        with torch.autograd.profiler.record_function("mogt.readout"):
            hn = ops.rmsnorm(h, self.norm_out.weight, self.norm_out.eps, out_dtype=gemm_dtype)
            Z = F.linear(hn, _gemm_weight(self, "theta_read", (self.theta_read.weight,),
                                          lambda: self.theta_read.weight))
        with torch.autograd.profiler.record_function("mogt.ffn"):
            x, xn2 = ops.add_rmsnorm(x, Z, self._residual_scale(Z), self.norm_ffn.weight,
                                     self.norm_ffn.eps, out_dtype=gemm_dtype)
            f = self.ffn(xn2)
        return x, (f, float(getattr(self, "mogt_ffn_residual_scale", 1.0)))


class MOGTModel(nn.Module):
    """Embedding -> blocks -> norm_f (model_mogt.py:260-287)."""

    def __init__(self, vocab_size: int, d_model: int = 768, num_layers: int = 12, r: int = 16,
                 ffn_hidden: int | None = None):
        super().__init__()
        self.embedding = nn.Embedding(vocab_size, d_model)
        self.blocks = nn.ModuleList([MOGTBlock(d_model=d_model, r=r, ffn_hidden=ffn_hidden)
                                     for _ in range(num_layers)])
        self.norm_f = RMSNorm(d_model)
        self.gradient_checkpointing = False
        self.checkpoint_every_n = 1

    def forward(self, input_ids):
        x = self.embedding(input_ids)
        prefix_condition = None
        prefix_position = getattr(self, "prefix_condition_position", None)
        if prefix_position is not None:
            prefix_position = int(prefix_position)
            if -x.size(1) <= prefix_position < x.size(1):
                prefix_condition = x[:, prefix_position, :]
        use_checkpoint = self.training and getattr(self, "gradient_checkpointing", False)
        every = max(1, int(getattr(self, "checkpoint_every_n", 1)))
        if (not use_checkpoint and x.dtype == torch.float32 and len(self.blocks) > 0
                and all(b.fused_path_ok() for b in self.blocks)):
            pending = None
            for block in self.blocks:
                x, pending = block.forward_fused(x, prefix_condition, pending)
            _, out = ops.add_rmsnorm(x, pending[0], pending[1], self.norm_f.weight, self.norm_f.eps,
                                     out_dtype=torch.float32)
            return out
        for i, block in enumerate(self.blocks):
            if use_checkpoint and (i % every == 0):
                x = checkpoint(block, x, prefix_condition, use_reentrant=False)
            else:
                x = block(x, prefix_condition=prefix_condition)
        return self.norm_f(x)


class MOGTForCausalLM(nn.Module):
    """Backbone + weight-tied LM head (model_mogt.py:289-380); initialisation as
    the reference (N(0, 0.02), phi_conn N(0, 1e-4), theta_read and ffn.w3 zero)."""

    def __init__(self, vocab_size: int, d_model: int = 768, num_layers: int = 12, r: int = 16,
                 ffn_hidden: int | None = None):
        super().__init__()
        self.mogt = MOGTModel(vocab_size=vocab_size, d_model=d_model, num_layers=num_layers, r=r,
                              ffn_hidden=ffn_hidden)
        self.lm_head = nn.Linear(d_model, vocab_size, bias=False)
        self.lm_head.weight = self.mogt.embedding.weight
        self.apply(self._init_weights)
        for name, p in self.named_parameters():
            if "phi_conn" in name:
                torch.nn.init.normal_(p, mean=0.0, std=1e-4)
            elif "theta_read" in name or "ffn.w3" in name:
                torch.nn.init.zeros_(p)

    def _init_weights(self, module):
        if isinstance(module, nn.Linear):
            torch.nn.init.normal_(module.weight, mean=0.0, std=0.02)
            if module.bias is not None:
                torch.nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            torch.nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def _chunked_lm_loss(self, hidden_states, labels, loss_chunk_size: int, return_logits: bool):
        """Chunked loss that keeps the logits (model_mogt.py:326-348): per chunk of
        positions the LM head and a summed cross-entropy, divided by the token
        count."""
        vocab_size = self.lm_head.weight.size(0)
        total_loss = hidden_states.new_zeros(())
        total_tokens = 0
        logits_chunks = [] if return_logits else None
        for start in range(0, hidden_states.size(1), loss_chunk_size):
            end = min(start + loss_chunk_size, hidden_states.size(1))
            logits_chunk = self.lm_head(hidden_states[:, start:end, :])
            labels_chunk = labels[:, start:end]
            total_loss = total_loss + F.cross_entropy(logits_chunk.reshape(-1, vocab_size),
                                                      labels_chunk.reshape(-1), reduction="sum")
            total_tokens += labels_chunk.numel()
            if return_logits:
                logits_chunks.append(logits_chunk)
        loss = total_loss / total_tokens
        logits = torch.cat(logits_chunks, dim=1) if return_logits else None
        return logits, loss

    def forward(self, input_ids, labels=None, *, return_logits=True, loss_chunk_size=0):
        """model_mogt.py:350-380: with labels and ``loss_chunk_size > 0`` the loss
        is chunked -- keeping the logits through the LM head, or, without
        logits, through chunked_linear_cross_entropy (HIP cross-entropy rows)."""
        x = self.mogt(input_ids)
        logits = None
        loss = None
        loss_chunk_size = int(loss_chunk_size or 0)
        with torch.autograd.profiler.record_function("mogt.lm_head_loss"):
            if labels is not None and loss_chunk_size > 0:
                if return_logits:
                    logits, loss = self._chunked_lm_loss(x, labels, loss_chunk_size, True)
                else:
                    loss = chunked_linear_cross_entropy(x, self.lm_head.weight, labels,
                                                        chunk_size=loss_chunk_size)
            else:
                logits = self.lm_head(x)
                if labels is not None:
                    loss = F.cross_entropy(logits.reshape(-1, logits.size(-1)).float(), labels.reshape(-1))
                if not return_logits:
                    logits = None
        return logits, loss


def configure_coupled_gate(model: nn.Module, *, scan_impl: str = "triton_hybrid",
                           connection_impl: str = "identity", connection_damping: float = 1.0,
                           value_gate_input: str = "current_prev_prefix",
                           value_gate_bias: float = -2.0, prefix_condition_position: int = 1,
                           zero_gate_weight: bool = True) -> None:
    """The slot-addressed, identity-coupled block wiring of the reference's
    backbone benchmark (benchmark_backbone_throughput.py:33-59)."""
    backbone = model.mogt if hasattr(model, "mogt") else model
    D = backbone.embedding.embedding_dim
    n_in = {"current": 1, "current_prev": 2, "current_prev_prefix": 3}[value_gate_input]
    dev = backbone.embedding.weight.device
    for block in backbone.blocks:
        block.scan_impl = scan_impl
        block.connection_impl = connection_impl
        block.connection_damping = connection_damping
        block.phi_value_gate = nn.Linear(n_in * D, block.r, bias=True).to(dev)
        if zero_gate_weight:
            nn.init.zeros_(block.phi_value_gate.weight)
        nn.init.constant_(block.phi_value_gate.bias, value_gate_bias)
        block.value_gate_input_mode = value_gate_input
        block.couple_forget_to_value_gate = True
    backbone.prefix_condition_position = prefix_condition_position
