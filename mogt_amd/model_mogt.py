"""MOGT layer and backbone on MI355X (drop-in for lkcfqy/MOGT ``model_mogt.py``).

Same classes, constructor arguments, parameter names and duck-typed
configuration attributes as the reference (model_mogt.py:9-380); configs and
state dicts carry over.  The scan always runs on the HIP kernels.

A block's configuration is resolved once per call into a :class:`MixerSpec`
and the mixer is evaluated in one of three ways:

* fused (identity connection, rank-wide value gate coupled to the forget gate,
  no transport gate -- the wiring of the reference's backbone benchmark,
  benchmark_backbone_throughput.py:40-57): gate + scan in one HIP kernel (no
  ``[B,L,r,r]`` U, no ``[B,L,3d]`` gate input, no ``phi_conn`` GEMM whose result
  the identity connection discards), single-pass RMSNorm / SwiGLU kernels,
  residual adds folded into the next RMSNorm;
* diagonal (any other identity-connection configuration): the transport is a
  per-rank factor (damping x transport gate x (1 - value gate)), so the scan is
  the HIP diagonal scan over ``[B, L, d]`` instead of a dense scan of ``r x r``
  matrices;
* dense (matrix_exp / Cayley connections): the connection map and the affine
  scan on their HIP kernels.

Tensors must be on the GPU; there is no CPU execution path.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

from . import ops, triton_scan
from .chunked_lm_loss import chunked_linear_cross_entropy, logits_cross_entropy


def _autocast_dtype() -> torch.dtype | None:
    if torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return None


_CACHE_ATTR = "_gemm_weight_cache"


def _gemm_weight(owner: nn.Module, name: str, params: tuple, build):
    """A GEMM operand built from parameters (a concatenation of weights, cast
    to the autocast dtype when autocast is on -- the cast F.linear would make).
    Without gradient recording it is cached on ``owner`` until a parameter
    changes (storage or version counter), the autocast dtype or the inference
    mode flag changes; with gradients it is rebuilt on every call so autograd
    reaches the parameters.  Writes through ``p.data`` bypass the version
    counter: call ``invalidate_weight_cache()`` after them (train(), eval()
    and load_state_dict() do it)."""
    ad = _autocast_dtype()

    def make():
        w = build()
        return w.to(ad) if ad is not None and w.is_floating_point() else w

    if torch.is_grad_enabled():
        return make()
    key = (tuple((p.data_ptr(), p._version, p.dtype) for p in params), ad, torch.is_inference_mode_enabled())
    cache = owner.__dict__.setdefault(_CACHE_ATTR, {})
    hit = cache.get(name)
    if hit is None or hit[0] != key:
        hit = (key, make())
        cache[name] = hit
    return hit[1]


class _WeightCacheOwner(nn.Module):
    """Drops the cached GEMM operands of every submodule on train()/eval() and
    after load_state_dict()."""

    def __init__(self):
        super().__init__()
        self.register_load_state_dict_post_hook(lambda module, keys: module.invalidate_weight_cache())

    def invalidate_weight_cache(self) -> None:
        for m in self.modules():
            m.__dict__.pop(_CACHE_ATTR, None)

    def train(self, mode: bool = True):
        self.invalidate_weight_cache()
        return super().train(mode)


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps), computed in fp32, ``type_as(x)``, times
    ``weight`` (model_mogt.py:9-20)."""

    def __init__(self, d_model: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d_model))

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
        w3 = _gemm_weight(self, "w3", (self.w3.weight,), lambda: self.w3.weight)
        if not torch.is_grad_enabled() and x.is_cuda:
            # bf16 without gradients: silu(w1 x) * w2 x is one GEMM whose
            # epilogue applies the gate (csrc/swiglu_gemm.hip)
            w1 = _gemm_weight(self, "w1", (self.w1.weight,), lambda: self.w1.weight)
            w2 = _gemm_weight(self, "w2", (self.w2.weight,), lambda: self.w2.weight)
            xb = x.to(w1.dtype) if _autocast_dtype() is not None else x
            if ops.swiglu_gate_supported(xb, w1, w2):
                return F.linear(ops.swiglu_gate(xb, w1, w2), w3)
        # one GEMM against [w1; w2], then the fused gate (autograd through the
        # silu_mul backward kernel and torch.cat back to w1, w2)
        w12 = _gemm_weight(self, "w12", (self.w1.weight, self.w2.weight),
                           lambda: torch.cat([self.w1.weight, self.w2.weight], dim=0))
        return self.forward_with(x, w12, w3)

    def forward_with(self, x, w12, w3):
        """The differentiable path on operands the caller built: ``w12`` =
        [w1; w2] and ``w3`` in the GEMM dtype (bf16 weight gradients from the
        split-K kernel, ``ops.linear``)."""
        return ops.linear(ops.silu_mul(ops.linear(x, w12)), w3)


def reference_ffn_hidden(d_model: int) -> int:
    """256 * ceil((8 d / 3) / 256) -- model_mogt.py:66-68 (2048 at d = 768)."""
    return 256 * ((int(8 * d_model / 3) + 255) // 256)


# ---------------------------------------------------------------------------
# configuration
# ---------------------------------------------------------------------------
# transport-gate activations g(logit, scale) (model_mogt.py:152-162)
_TRANSPORT_GATE_FN = {
    "multiply": lambda g, s: torch.sigmoid(g),
    "residual": lambda g, s: 1.0 + s * torch.tanh(g),
    "forget_relu": lambda g, s: 1.0 - s * F.relu(torch.tanh(g)),
}
_CONNECTIONS = ("identity", "matrix_exp", "cayley")
# every scan_impl that evaluates the affine recurrence (model_mogt.py:193-232);
# "transport_triton" is the reference's transport-only mode (:187-192)
_AFFINE_SCAN_IMPLS = frozenset({"triton_hybrid", "parallel_reference", "block_reference", "sequential"})
_CARRY_HINT_IMPLS = frozenset({"triton_hybrid", "block_reference"})


def _gate_input_parts(mode: str) -> tuple[str, ...]:
    """Pieces of the value gate's input: the normalised token, then the
    previous token and the prefix condition when the mode names them
    (model_mogt.py:104-122)."""
    if mode == "current":
        return ("cur",)
    return ("cur",) + (("prev",) if "prev" in mode else ()) + (("prefix",) if "prefix" in mode else ())


@dataclass(frozen=True)
class MixerSpec:
    """A block's duck-typed configuration, resolved for one call."""
    connection: str
    damping: float
    transport_gate: nn.Module | None
    transport_mode: str
    transport_scale: float
    value_gate: nn.Module | None
    gate_parts: tuple[str, ...]
    coupled: bool
    scan: str
    residual_scale: float
    residual_gate_logit: torch.Tensor | None
    ffn_scale: float

    @staticmethod
    def of(block: "MOGTBlock") -> "MixerSpec":
        scan = "transport_triton" if getattr(block, "fast_throughput_mode", False) else \
            getattr(block, "scan_impl", "sequential")
        gate_logit = getattr(block, "mogt_residual_gate_logit", None)
        if not getattr(block, "mogt_residual_gate_enabled", False):
            gate_logit = None
        return MixerSpec(
            connection=getattr(block, "connection_impl", "matrix_exp"),
            damping=float(getattr(block, "connection_damping", 0.999)),
            transport_gate=getattr(block, "phi_transport_gate", None),
            transport_mode=getattr(block, "transport_gate_mode", "multiply"),
            transport_scale=float(getattr(block, "transport_gate_scale", 1.0)),
            value_gate=getattr(block, "phi_value_gate", None),
            gate_parts=_gate_input_parts(getattr(block, "value_gate_input_mode", "current")),
            coupled=bool(getattr(block, "couple_forget_to_value_gate", False)),
            scan=scan,
            residual_scale=float(getattr(block, "mogt_residual_scale", 1.0)),
            residual_gate_logit=gate_logit,
            ffn_scale=float(getattr(block, "mogt_ffn_residual_scale", 1.0)),
        )

    def validate(self) -> None:
        if self.connection not in _CONNECTIONS:
            raise ValueError(f"Unsupported connection_impl: {self.connection}")
        if self.transport_gate is not None and self.transport_mode not in _TRANSPORT_GATE_FN:
            raise ValueError(f"Unsupported transport_gate_mode: {self.transport_mode}")
        if self.scan != "transport_triton" and self.scan not in _AFFINE_SCAN_IMPLS:
            raise ValueError(f"Unsupported scan_impl: {self.scan}")

    def residual_factor(self, like: torch.Tensor):
        """Scale of the mixer's residual term: the constant scale, times the
        learned gate sigmoid(logit) when enabled (model_mogt.py:243-249)."""
        if self.residual_gate_logit is None:
            return self.residual_scale
        return self.residual_scale * torch.sigmoid(self.residual_gate_logit).to(dtype=like.dtype,
                                                                                device=like.device)


def _gate_input(xn: torch.Tensor, prefix_condition: torch.Tensor | None, parts: tuple[str, ...]):
    """The value gate's input pieces side by side (model_mogt.py:104-122): the
    normalised token, the previous one (zero at t = 0), the prefix condition
    broadcast over time (zero without one)."""
    pieces = []
    for name in parts:
        if name == "cur":
            pieces.append(xn)
        elif name == "prev":
            pieces.append(F.pad(xn[:, :-1], (0, 0, 1, 0)))
        else:
            row = (xn.new_zeros(xn.size(0), 1, xn.size(-1)) if prefix_condition is None
                   else prefix_condition.to(xn.dtype).view(xn.size(0), 1, xn.size(-1)))
            pieces.append(row.expand_as(xn))
    return pieces[0] if len(pieces) == 1 else torch.cat(pieces, dim=-1)


class MOGTBlock(_WeightCacheOwner):
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

    # ------------------------------------------------------------ dispatch
    def _resolve_scan_impl(self):
        return MixerSpec.of(self).scan

    def _resolve_connection_impl(self):
        return MixerSpec.of(self).connection

    def _residual_scale(self, like: torch.Tensor) -> float:
        return float(MixerSpec.of(self).residual_factor(like))

    def fused_path_ok(self) -> bool:
        """Identity connection, no transport gate, rank-wide value gate coupled to
        the forget gate, an affine scan_impl; with autograd, no learned residual
        gate (its scale enters the fused residual update as a constant)."""
        spec = MixerSpec.of(self)
        if (torch.is_grad_enabled() and spec.residual_gate_logit is not None
                and any(p.requires_grad for p in self.parameters())):
            return False
        return (spec.connection == "identity" and spec.transport_gate is None
                and isinstance(spec.value_gate, nn.Linear) and spec.value_gate.out_features == self.r
                and spec.coupled and spec.scan in _AFFINE_SCAN_IMPLS)

    def forward(self, x, prefix_condition=None):
        ops.require_cuda("MOGTBlock", x)
        if self.fused_path_ok() and x.dtype == torch.float32:
            x, (z, s) = self.forward_fused(x, prefix_condition, None)
            return x + s * z
        return self._forward_generic(x, prefix_condition)

    # ------------------------------------------------------------ generic path
    def _build_transport(self, A: torch.Tensor, output_dtype: torch.dtype):
        """``damping * map(A / r)`` as fp32 math cast to ``output_dtype``
        (model_mogt.py:79-102); the maps run on the HIP connection-map kernel."""
        spec = MixerSpec.of(self)
        if spec.connection == "identity":
            eye = self._identity_r.view(1, 1, self.r, self.r)
            return (eye * spec.damping).to(output_dtype).expand(A.shape[0], A.shape[1], self.r, self.r)
        if spec.connection not in _CONNECTIONS:
            raise ValueError(f"Unsupported connection_impl: {spec.connection}")
        label = "mogt.matrix_exp" if spec.connection == "matrix_exp" else "mogt.cayley_solve"
        with torch.autograd.profiler.record_function(label):
            mapped = ops.connection_map((A / self.r).to(torch.float32), spec.connection)
        return (mapped * spec.damping).to(output_dtype)

    def _value_gate_probs(self, spec: MixerSpec, xn, prefix_condition):
        """sigmoid of the value gate, fp32, shaped [B, L, w, 1] (w = 1 or r).
        A Linear gate never sees its concatenated input (``_gate_logits``);
        any other module is called on it."""
        if isinstance(spec.value_gate, nn.Linear):
            z = self._gate_logits(xn, prefix_condition)
        else:
            z = spec.value_gate(_gate_input(xn, prefix_condition, spec.gate_parts)).float()
        if z.size(-1) not in (1, self.r):
            raise ValueError("phi_value_gate must output either 1 scalar or r rank gates")
        return torch.sigmoid(z).unsqueeze(-1)

    def _transport_gate(self, spec: MixerSpec, xn):
        """The transport gate's factor, fp32, [B, L, w, 1] (w = 1 or r)."""
        logits = spec.transport_gate(xn).float()
        if logits.size(-1) not in (1, self.r):
            raise ValueError("phi_transport_gate must output either 1 scalar or r rank gates")
        return _TRANSPORT_GATE_FN[spec.transport_mode](logits.unsqueeze(-1), spec.transport_scale)

    def _forward_generic(self, x, prefix_condition):
        """MOGTBlock.forward (model_mogt.py:124-258), any configuration, with
        autograd; the scan on the HIP diagonal or dense kernels."""
        spec = MixerSpec.of(self)
        spec.validate()
        xn = self.norm_mogt(x)
        B, L, D = xn.shape
        r, c = self.r, self.c
        diagonal = spec.connection == "identity" and spec.scan != "transport_triton"
        with torch.autograd.profiler.record_function("mogt.connection_map"):
            if diagonal:
                # per-rank factor of U = factor * I: starts as the damping
                factor = torch.full((1, 1, 1, 1), spec.damping, dtype=torch.float32,
                                    device=xn.device).to(xn.dtype)
                U = None
            else:
                if spec.connection == "identity":
                    A = xn.new_zeros(B, L, r, r)   # the identity map ignores A
                else:
                    with torch.autograd.profiler.record_function("mogt.connection"):
                        A_raw = self.phi_conn(xn).view(B, L, r, r)
                        A = A_raw - A_raw.transpose(-2, -1)
                U = self._build_transport(A, xn.dtype)
            if spec.transport_gate is not None:
                tg = self._transport_gate(spec, xn)
                if diagonal:
                    factor = factor * tg.to(factor.dtype)
                else:
                    U = U * tg.to(U.dtype)
        with torch.autograd.profiler.record_function("mogt.value_projection"):
            values = self.phi_val(xn).view(B, L, r, c)
            if spec.value_gate is not None:
                vg = self._value_gate_probs(spec, xn, prefix_condition)
                values = values * vg.to(values.dtype)
                if spec.coupled:
                    keep = (1.0 - vg)
                    if diagonal:
                        factor = factor * keep.to(factor.dtype)
                    else:
                        U = U * keep.to(U.dtype)
        out_dtype = xn.dtype   # the scan's output dtype is U's (model_mogt.py:202)
        with torch.autograd.profiler.record_function("mogt.affine_scan"):
            if diagonal:
                decay = factor.float().expand(B, L, r, c).reshape(B, L, D)
                h = ops.diag_scan(decay, values.float().reshape(B, L, D), out_dtype=out_dtype)
            elif spec.scan == "transport_triton":
                Y = triton_scan.triton_fused_scan(U)
                h = torch.matmul(Y, values.to(Y.dtype)).reshape(B, L, D)
            else:
                carry = getattr(self, "block_carry_scan", "sequential") if spec.scan in _CARRY_HINT_IMPLS \
                    else "sequential"
                h = triton_scan.triton_affine_scan_hybrid(
                    U, values, block_size=getattr(self, "scan_block_size", 256),
                    block_c=getattr(self, "scan_block_c", 32), carry_scan=carry,
                    output_dtype=out_dtype).reshape(B, L, D)
        with torch.autograd.profiler.record_function("mogt.readout"):
            z = self.theta_read(self.norm_out(h))
        x = x + spec.residual_factor(z) * z
        with torch.autograd.profiler.record_function("mogt.ffn"):
            x = x + spec.ffn_scale * self.ffn(self.norm_ffn(x))
        return x

    # ------------------------------------------------------------ fused path
    def _gate_logits(self, xn: torch.Tensor, prefix_condition: torch.Tensor | None) -> torch.Tensor:
        """The value gate's logits, fp32 [B, L, w], over the input pieces of
        ``value_gate_input_mode`` without materialising their concatenation:
        with W = [W_cur | W_prev | W_pref], one GEMM of x against [W_cur; W_prev]
        gives the current term and the previous token's term (shifted by one
        step, zero at t = 0), and the prefix term is one row per sequence
        (zero without a prefix condition) -- model_mogt.py:104-122, :166-171."""
        gate: nn.Linear = self.phi_value_gate
        parts = _gate_input_parts(getattr(self, "value_gate_input_mode", "current"))
        D = self.d_model
        w = gate.out_features
        W = gate.weight
        if W.shape[1] != len(parts) * D:
            raise RuntimeError(f"phi_value_gate takes {W.shape[1]} inputs, the gate input mode builds "
                               f"{len(parts) * D}")
        cols = {name: W[:, i * D:(i + 1) * D] for i, name in enumerate(parts)}
        stacked = [cols["cur"]] + ([cols["prev"]] if "prev" in cols else [])
        Wg = _gemm_weight(self, "gate", (W,), lambda: torch.cat(stacked, dim=0))
        y = F.linear(xn, Wg).float()   # [B, L, w * (1 or 2)]
        z = y[..., :w]
        if "prev" in cols:
            z = torch.cat([z[:, :1], z[:, 1:] + y[:, :-1, w:2 * w]], dim=1)
        const = gate.bias.float() if gate.bias is not None else None
        if "prefix" in cols and prefix_condition is not None:
            pref = prefix_condition.to(dtype=xn.dtype).view(xn.size(0), 1, D)
            pt = F.linear(pref, cols["prefix"]).float()
            const = pt if const is None else const + pt
        return (z if const is None else z + const).contiguous()

    def _gate_const_weights(self):
        """(W_pref or None, bias or None) of the value gate: the weights of its
        per-sequence logit term."""
        gate: nn.Linear = self.phi_value_gate
        parts = _gate_input_parts(getattr(self, "value_gate_input_mode", "current"))
        D = self.d_model
        w_pref = gate.weight[:, parts.index("prefix") * D:(parts.index("prefix") + 1) * D] if "prefix" in parts \
            else None
        return w_pref, gate.bias

    def _value_and_gate_projection(self, xn: torch.Tensor, prefix_condition: torch.Tensor | None,
                                   const: torch.Tensor | None = None, const_given: bool = False,
                                   packed: dict | None = None):
        """One GEMM of x against [phi_val; W_cur; W_prev]: v and the value gate's
        pre-logits for the current and the previous token side by side, plus
        the per-sequence logit term (bias + prefix term, fp32 [B, r] or [r]),
        unless the caller passes it (``const_given``).  ``packed``: phi_val's
        and the gate's weights already in the GEMM dtype.  Returns (proj,
        has_prev, const)."""
        gate: nn.Linear = self.phi_value_gate
        parts = _gate_input_parts(getattr(self, "value_gate_input_mode", "current"))
        D = self.d_model
        W = packed["gate"] if packed is not None else gate.weight
        if W.shape[1] != len(parts) * D:
            raise RuntimeError(f"phi_value_gate takes {W.shape[1]} inputs, the gate input mode builds "
                               f"{len(parts) * D}")
        # column blocks as views whose backward is one stack (not one zero
        # fill and copy per sliced block)
        cols = dict(zip(parts, W.view(W.shape[0], len(parts), D).unbind(1)))
        if packed is not None:
            stacked = [packed["phi_val"], cols["cur"]] + ([cols["prev"]] if "prev" in cols else [])
            W_all = torch.cat(stacked, dim=0)
        else:
            stacked = [self.phi_val.weight, cols["cur"]] + ([cols["prev"]] if "prev" in cols else [])
            W_all = _gemm_weight(self, "value_and_gate", (self.phi_val.weight, W),
                                 lambda: torch.cat(stacked, dim=0))
        proj = ops.linear(xn, W_all)
        if const_given:
            return proj, "prev" in cols, const
        const = gate.bias.float() if gate.bias is not None else None
        if "prefix" in cols and prefix_condition is not None:
            pref = prefix_condition.to(dtype=xn.dtype).view(xn.size(0), D)
            pt = F.linear(pref, cols["prefix"]).float()
            const = pt if const is None else pt + const
        return proj, "prev" in cols, const

    def _mixer_inference(self, x, xn, prefix_condition, damping: float, gemm_dtype, gate_const=None):
        """Mixer of the fused path without autograd.  One GEMM gives phi_val's
        output and the gate's pre-logits, which the scan combines into the
        logits itself.  norm_out is folded around the read-out GEMM: the scan
        writes h in the GEMM's dtype plus per-row sums of squares, the GEMM runs
        against theta_read * norm_out.weight, and the next RMSNorm applies each
        row's factor rsqrt(mean(h^2) + eps) as it reads Z."""
        with torch.autograd.profiler.record_function("mogt.affine_scan"):
            proj, gate_prev, gconst = self._value_and_gate_projection(xn, prefix_condition, gate_const,
                                                                      const_given=gate_const is not None)
            h, stats = ops.coupled_rank_scan_proj(proj, self.d_model, rank=self.r, gate_prev=gate_prev,
                                                  gate_const=gconst, damping=damping)
        with torch.autograd.profiler.record_function("mogt.readout"):
            Zr = F.linear(h, _gemm_weight(self, "theta_read_folded", (self.theta_read.weight, self.norm_out.weight),
                                          lambda: self.theta_read.weight * self.norm_out.weight))
        return ops.add_rmsnorm_rowscale(x, Zr, stats, self._residual_scale(Zr), self.norm_ffn.weight,
                                        stat_eps=self.norm_out.eps, eps=self.norm_ffn.eps, out_dtype=gemm_dtype)

    def _mixer_training(self, x, xn, prefix_condition, damping: float, gemm_dtype, packed: dict | None = None):
        """Mixer of the fused path under autograd: every kernel has its backward.
        Where the row layout allows, the scan is fed by the one projection GEMM
        of the inference path, so the backward's epilogue writes the
        projection's gradient directly (one GEMM back to x and to the stacked
        weights); otherwise by separately computed gate logits."""
        parts = _gate_input_parts(getattr(self, "value_gate_input_mode", "current"))
        if ops.coupled_proj_scan_supported(self.d_model, self.r, "prev" in parts):
            with torch.autograd.profiler.record_function("mogt.affine_scan"):
                proj, gate_prev, gconst = self._value_and_gate_projection(xn, prefix_condition, packed=packed)
                if gconst is not None:
                    gconst = gconst.expand(xn.size(0), self.r).contiguous()
                h = ops.coupled_proj_scan(proj, self.d_model, rank=self.r, gate_prev=gate_prev, gate_const=gconst,
                                          damping=damping)
        else:
            with torch.autograd.profiler.record_function("mogt.value_projection"):
                v_raw = F.linear(xn, _gemm_weight(self, "phi_val", (self.phi_val.weight,),
                                                  lambda: self.phi_val.weight))
                z = self._gate_logits(xn, prefix_condition)
            with torch.autograd.profiler.record_function("mogt.affine_scan"):
                h = ops.coupled_rank_scan(z, v_raw, damping=damping, out_dtype=torch.float32)
        with torch.autograd.profiler.record_function("mogt.readout"):
            hn = ops.rmsnorm(h, self.norm_out.weight, self.norm_out.eps, out_dtype=gemm_dtype)
            Wr = packed["theta"] if packed is not None else _gemm_weight(self, "theta_read", (self.theta_read.weight,),
                                                                           lambda: self.theta_read.weight)
            Z = ops.linear(hn, Wr)
        return ops.add_rmsnorm(x, Z, self._residual_scale(Z), self.norm_ffn.weight, self.norm_ffn.eps,
                               out_dtype=gemm_dtype)

    def training_weight_groups(self) -> list | None:
        """The parameters behind this block's GEMM operands in the training
        path, as groups to concatenate and cast (``ops.cast_groups``): phi_val,
        the value gate, theta_read, [w1; w2], w3.  None where the block's
        training mixer does not take them so."""
        parts = _gate_input_parts(getattr(self, "value_gate_input_mode", "current"))
        ffn = self.ffn
        if not (isinstance(ffn, SwiGLU) and ops.coupled_proj_scan_supported(self.d_model, self.r, "prev" in parts)
                and self.phi_value_gate.weight.shape[1] == len(parts) * self.d_model):
            return None
        return [[self.phi_val.weight], [self.phi_value_gate.weight], [self.theta_read.weight],
                [ffn.w1.weight, ffn.w2.weight], [ffn.w3.weight]]

    @staticmethod
    def packed_weights(outs: list) -> dict:
        """The operands of ``training_weight_groups`` by name."""
        return dict(zip(("phi_val", "gate", "theta", "w12", "w3"), outs))

    def forward_fused(self, x: torch.Tensor, prefix_condition, pending, gate_const=None,
                      packed: dict | None = None):
        """Fused forward.  ``pending = (z, scale)`` is the previous block's last
        residual term (added here inside the first RMSNorm).  ``gate_const``
        (inference only): this block's per-sequence gate-logit term when the
        caller computed it.  ``packed`` (training only): the GEMM operands of
        ``training_weight_groups`` in the GEMM dtype.  Returns
        ``(x_after_mixer, (ffn_out, ffn_scale))``: the caller adds the FFN term
        (or hands it to the next block)."""
        gemm_dtype = _autocast_dtype() or x.dtype
        eps = self.norm_mogt.eps
        if pending is None:
            xn = ops.rmsnorm(x, self.norm_mogt.weight, eps, out_dtype=gemm_dtype)
        else:
            x, xn = ops.add_rmsnorm(x, pending[0], pending[1], self.norm_mogt.weight, eps, out_dtype=gemm_dtype)
        damping = float(getattr(self, "connection_damping", 0.999))
        if torch.is_grad_enabled():
            x, xn2 = self._mixer_training(x, xn, prefix_condition, damping, gemm_dtype, packed)
        else:
            x, xn2 = self._mixer_inference(x, xn, prefix_condition, damping, gemm_dtype, gate_const)
        with torch.autograd.profiler.record_function("mogt.ffn"):
            f = self.ffn(xn2) if packed is None else self.ffn.forward_with(xn2, packed["w12"], packed["w3"])
        return x, (f, float(getattr(self, "mogt_ffn_residual_scale", 1.0)))


class MOGTModel(_WeightCacheOwner):
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

    def _packed_training_weights(self) -> list:
        """Under autograd and autocast: every block's GEMM operands cast to the
        autocast dtype in one multi-tensor copy (and their gradients cast back
        in one), instead of a cast kernel per weight and the fp32
        concatenations; a list of None otherwise."""
        ad = _autocast_dtype()
        groups = [blk.training_weight_groups() for blk in self.blocks]
        if not torch.is_grad_enabled() or ad is None or any(g is None for g in groups):
            return [None] * len(self.blocks)
        outs = ops.cast_groups([grp for g in groups for grp in g], ad)
        packed, i = [], 0
        for g in groups:
            packed.append(MOGTBlock.packed_weights(outs[i:i + len(g)]))
            i += len(g)
        return packed

    def _prefix_condition(self, h: torch.Tensor) -> torch.Tensor | None:
        """The embedding row at ``prefix_condition_position`` (negative counts
        from the end), or None when unset or outside the sequence."""
        pos = getattr(self, "prefix_condition_position", None)
        if pos is None:
            return None
        pos = int(pos)
        return h[:, pos, :] if -h.size(1) <= pos < h.size(1) else None

    def _gate_consts(self, cond: torch.Tensor | None) -> list:
        """Every block's per-sequence gate-logit term (bias + prefix term) in
        one fp32 GEMV over the stacked prefix weights (inference); entries are
        fp32 [B, r], or None for a gate without either."""
        specs = [blk._gate_const_weights() for blk in self.blocks]
        if all(wp is None and b is None for wp, b in specs):
            return [None] * len(self.blocks)
        r = self.blocks[0].r
        params = tuple(t for wp, b in specs for t in (wp, b) if t is not None)
        D = self.embedding.embedding_dim

        def build():
            ws = [wp if wp is not None else torch.zeros(r, D, device=params[0].device) for wp, _ in specs]
            bs = [b if b is not None else torch.zeros(r, device=params[0].device) for _, b in specs]
            return torch.cat([torch.cat(ws, 0).float(), torch.cat(bs, 0).float()[:, None]], dim=1)

        with torch.autocast("cuda", enabled=False):
            Wb = _gemm_weight(self, "gate_consts", params, build)   # [n * r, D + 1] fp32
            if cond is None:
                allc = Wb[:, D].expand(1, -1)
            else:
                allc = torch.addmm(Wb[:, D], cond.float(), Wb[:, :D].t())
        B = cond.size(0) if cond is not None else 1
        return [allc[:, i * r:(i + 1) * r].expand(B, r) for i in range(len(self.blocks))]

    def _checkpointed(self, index: int) -> bool:
        if not (self.training and getattr(self, "gradient_checkpointing", False)):
            return False
        return index % max(1, int(getattr(self, "checkpoint_every_n", 1))) == 0

    def forward(self, input_ids):
        chain_fused = (self.embedding.weight.dtype == torch.float32 and len(self.blocks) > 0
                       and not self._checkpointed(0) and all(blk.fused_path_ok() for blk in self.blocks))
        pos = getattr(self, "prefix_condition_position", None)
        if (chain_fused and torch.is_grad_enabled() and pos is not None
                and -input_ids.size(1) <= int(pos) < input_ids.size(1)):
            # the prefix row looked up again alongside the tokens: its gradient
            # joins the tokens' in one table instead of flowing through a
            # full-size slice of h (or a second table)
            h, cond = ops.embedding_pair(input_ids, input_ids[:, int(pos)], self.embedding)
        else:
            h = ops.embedding(input_ids, self.embedding)
            cond = self._prefix_condition(h)
        if chain_fused:
            # each block hands its FFN term to the next block's first RMSNorm;
            # the last one is added inside norm_f
            consts = self._gate_consts(cond) if not torch.is_grad_enabled() else [None] * len(self.blocks)
            packed = self._packed_training_weights()
            pending = None
            for blk, gc, pk in zip(self.blocks, consts, packed):
                h, pending = blk.forward_fused(h, cond, pending, gc, pk)
            if not torch.is_grad_enabled():
                return ops.add_rmsnorm_final(h, pending[0], pending[1], self.norm_f.weight, self.norm_f.eps)
            return ops.add_rmsnorm(h, pending[0], pending[1], self.norm_f.weight, self.norm_f.eps,
                                   out_dtype=torch.float32)[1]
        for i, blk in enumerate(self.blocks):
            h = checkpoint(blk, h, cond, use_reentrant=False) if self._checkpointed(i) \
                else blk(h, prefix_condition=cond)
        return self.norm_f(h)


class MOGTForCausalLM(_WeightCacheOwner):
    """Backbone + weight-tied LM head (model_mogt.py:289-380)."""

    INIT_STD = 0.02            # every Linear weight and the embedding (model_mogt.py:318-324)
    CONNECTION_INIT_STD = 1e-4  # phi_conn: U starts near the identity (:308-310)

    def __init__(self, vocab_size: int, d_model: int = 768, num_layers: int = 12, r: int = 16,
                 ffn_hidden: int | None = None):
        super().__init__()
        self.mogt = MOGTModel(vocab_size=vocab_size, d_model=d_model, num_layers=num_layers, r=r,
                              ffn_hidden=ffn_hidden)
        self.lm_head = nn.Linear(d_model, vocab_size, bias=False)
        self.lm_head.weight = self.mogt.embedding.weight
        self._initialise()

    @torch.no_grad()
    def _initialise(self) -> None:
        """The reference's initialisation, draw for draw: every Linear and
        Embedding in module order gets N(0, INIT_STD) (biases zero; the tied
        head redraws the shared matrix), then each block's phi_conn
        N(0, CONNECTION_INIT_STD) and its read-outs (theta_read, ffn.w3) zero."""
        for m in self.modules():
            if isinstance(m, (nn.Linear, nn.Embedding)):
                m.weight.normal_(0.0, self.INIT_STD)
                if getattr(m, "bias", None) is not None:
                    m.bias.zero_()
        for blk in self.mogt.blocks:
            blk.phi_conn.weight.normal_(0.0, self.CONNECTION_INIT_STD)
            blk.theta_read.weight.zero_()
            blk.ffn.w3.weight.zero_()

    def forward(self, input_ids, labels=None, *, return_logits=True, loss_chunk_size=0):
        """model_mogt.py:350-380.  Without labels: logits.  With labels and
        ``loss_chunk_size <= 0``: F.cross_entropy over the full logits (mean
        over non-ignored tokens).  With ``loss_chunk_size > 0``: the summed
        cross-entropy divided by the token count -- from the kept logits
        through the HIP cross-entropy rows (``return_logits``), or without
        logits through chunked_linear_cross_entropy."""
        hidden = self.mogt(input_ids)
        chunk = int(loss_chunk_size or 0)
        with torch.autograd.profiler.record_function("mogt.lm_head_loss"):
            if labels is not None and chunk > 0 and not return_logits:
                return None, chunked_linear_cross_entropy(hidden, self.lm_head.weight, labels,
                                                          chunk_size=chunk)
            logits = self.lm_head(hidden)
            loss = None
            if labels is not None:
                flat_logits = logits.reshape(-1, logits.size(-1))
                if chunk > 0:
                    loss = logits_cross_entropy(flat_logits, labels.reshape(-1))
                else:
                    loss = F.cross_entropy(flat_logits.float(), labels.reshape(-1))
        return (logits if return_logits else None), loss


def configure_coupled_gate(model: nn.Module, *, scan_impl: str = "triton_hybrid",
                           connection_impl: str = "identity", connection_damping: float = 1.0,
                           value_gate_input: str = "current_prev_prefix",
                           value_gate_bias: float = -2.0, prefix_condition_position: int = 1,
                           zero_gate_weight: bool = True) -> None:
    """The slot-addressed, identity-coupled block wiring of the reference's
    backbone benchmark (benchmark_backbone_throughput.py:33-59)."""
    backbone = model.mogt if hasattr(model, "mogt") else model
    D = backbone.embedding.embedding_dim
    n_in = len(_gate_input_parts(value_gate_input))
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
