"""Write the golden fixtures of the MOGT layer, backbone and LM wrapper.

Run in the build container only (the GPU host has no reference checkout):

    python tests/golden/make_model_fixtures.py /path/to/reference

It imports the reference's pure-PyTorch ``model_mogt.py`` (which pulls in its
``affine_scan.py`` and ``chunked_lm_loss.py``) on the CPU, builds seeded models
in the configurations below, runs them, and stores inputs, weights and outputs
as plain arrays in ``model_fixtures.npz`` plus a manifest with a SHA-256 per
array (``model_fixtures.json``).  Only these data files are read by the tests;
no reference code is kept in this repository or run anywhere else.

Fixtures (float64 unless noted; ``scan_impl = "sequential"``, the reference's
CPU scan, which every other scan_impl evaluates to fp32 rounding):

* ``bb``   -- MOGTModel with the backbone benchmark's wiring
  (benchmark_backbone_throughput.py:33-59): identity connection, damping 1.0,
  a rank-wide value gate over ``current_prev_prefix`` with bias -2, coupled to
  the forget gate, prefix position 1; a 4x SwiGLU; non-zero seeded weights
  everywhere (theta_read, ffn.w3, the gate weight, RMSNorm weights); residual
  scales other than 1 on the second block.  Stores ids, the state dict, the
  output of every block and the backbone output.
* ``bx``, ``bc``, ``bi`` -- single MOGTBlocks: matrix_exp connection with a
  rank-wise "residual" transport gate and a scalar value gate over
  ``current_prev``; Cayley connection with a scalar "forget_relu" transport gate,
  a coupled rank gate over ``current_prev_prefix`` with a given prefix and the
  learned residual gate; identity connection (damping 0.95) with a rank-wise
  "multiply" transport gate and no value gate.
* ``lm_init`` -- (manifest only) a hash, sum and first entries of every
  parameter of a 2-layer MOGTForCausalLM built after ``torch.manual_seed(1234)``
  in float64: the reference's initialisation order and values.
* ``lm``   -- a 1-layer MOGTForCausalLM with reseeded weights and its losses on
  seeded labels: unchunked, chunked with logits, and
  chunked_linear_cross_entropy (with the gradients of the hidden states and of
  the tied weight).
* ``ga``   -- under CPU bf16 autocast, the coupled block's gate logits, the
  ``phi_val`` output and the (U, V) pair handed to the scan: the dtype flow of
  model_mogt.py:166-182 (``V_t_raw * value_gate.to(V_t_raw.dtype)`` in bf16).
* ``tt``   -- a block in ``fast_throughput_mode`` (``scan_impl =
  "transport_triton"``, model_mogt.py:71-74, 187-192): ``V_t = Y_t V_raw`` with
  ``Y_t = U_t Y_{t-1}``, ``Y_0 = I``.  The Triton kernel (triton_scan.py:13-51,
  151-175) needs a GPU and fixes R = 16 at launch, so this block has r = 16
  (d_model 64), and its recurrence is evaluated by the reference's own prefix
  product, ``affine_scan_sequential(U, 0, return_prefix=True)``
  (affine_scan.py:43-55), in place of the Triton launch.
* ``ck``   -- a 3-layer MOGTModel in training mode with
  ``gradient_checkpointing = True`` and ``checkpoint_every_n = 2``
  (model_mogt.py:278-285), the backbone wiring of ``bb``, blocks selecting
  ``parallel_reference``, ``block_reference`` (block size 7, doubling carry
  scan) and ``sequential`` (model_mogt.py:204-221); the output, the loss
  ``sum(out * w)`` for seeded ``w`` and every parameter's gradient.
* ``pr``, ``br`` -- single blocks on the dense (non-identity) transport with
  ``scan_impl = "parallel_reference"`` (matrix_exp) and ``"block_reference"``
  (Cayley, ``scan_block_size = 5``, ``block_carry_scan = "doubling"``).
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
D, R, VOCAB, B, L = 32, 4, 97, 2, 40


def _arrays_of(prefix: str, tensors: dict) -> dict:
    """Inputs and weights: every value is float32-representable by construction,
    so they are stored as float32 (checked); bf16 tensors widen exactly."""
    out = {}
    for k, v in tensors.items():
        t = v.detach().cpu()
        if t.is_floating_point():
            t32 = t.float()
            assert torch.equal(t32.to(t.dtype), t), f"{prefix}/{k} is not float32-representable"
            t = t32
        out[f"{prefix}/{k}"] = t.numpy()
    return out


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.float().to(t.dtype)


def _reseed_weights(module: torch.nn.Module, gen: torch.Generator) -> None:
    """Seeded non-zero values for every parameter (norm weights around 1)."""
    with torch.no_grad():
        for name, p in module.named_parameters():
            if name.endswith("norm_mogt.weight") or name.endswith("norm_out.weight") or \
                    name.endswith("norm_ffn.weight") or name == "norm_f.weight":
                p.copy_(_f32(1.0 + 0.2 * torch.randn(p.shape, generator=gen, dtype=p.dtype)))
            elif "phi_value_gate.bias" in name:
                p.copy_(_f32(-2.0 + 0.5 * torch.randn(p.shape, generator=gen, dtype=p.dtype)))
            elif "phi_value_gate.weight" in name or "phi_transport_gate" in name:
                p.copy_(_f32(0.3 * torch.randn(p.shape, generator=gen, dtype=p.dtype)))
            elif "mogt_residual_gate_logit" in name:
                p.copy_(_f32(torch.full(p.shape, 0.4, dtype=p.dtype)))
            else:
                fan_in = p.shape[-1] if p.ndim > 1 else 1
                p.copy_(_f32(torch.randn(p.shape, generator=gen, dtype=p.dtype) / fan_in ** 0.5))


def main(ref: Path) -> None:
    sys.path.insert(0, str(ref))
    import model_mogt as mm  # the reference's module (CPU, pure torch)
    from chunked_lm_loss import chunked_linear_cross_entropy

    torch.set_default_dtype(torch.float64)
    arrays: dict[str, np.ndarray] = {}
    meta: dict = {"D": D, "R": R, "VOCAB": VOCAB, "B": B, "L": L}
    gen = torch.Generator().manual_seed(20261202)

    # ---- bb: backbone with the benchmark's wiring -------------------------
    torch.manual_seed(1)
    model = mm.MOGTModel(vocab_size=VOCAB, d_model=D, num_layers=2, r=R)
    for i, blk in enumerate(model.blocks):
        blk.ffn = mm.SwiGLU(D, 4 * D)
        blk.scan_impl = "sequential"
        blk.connection_impl = "identity"
        blk.connection_damping = 1.0
        blk.phi_value_gate = torch.nn.Linear(3 * D, R, bias=True)
        blk.value_gate_input_mode = "current_prev_prefix"
        blk.couple_forget_to_value_gate = True
        if i == 1:
            blk.mogt_residual_scale = 0.7
            blk.mogt_ffn_residual_scale = 1.3
    model.prefix_condition_position = 1
    _reseed_weights(model, gen)
    model.eval()
    ids = torch.randint(0, VOCAB, (B, L), generator=gen)
    block_out = []
    hooks = [blk.register_forward_hook(lambda m, i, o: block_out.append(o.detach().clone()))
             for blk in model.blocks]
    with torch.no_grad():
        y = model(ids)
    for h in hooks:
        h.remove()
    arrays.update(_arrays_of("bb", model.state_dict()))
    arrays["bb/ids"] = ids.numpy()
    arrays["bb/out"] = y.numpy()
    for i, o in enumerate(block_out):
        arrays[f"bb/block{i}_out"] = o.numpy()
    meta["bb"] = {"layers": 2, "ffn_hidden": 4 * D, "prefix_condition_position": 1,
                  "blocks": [{"scan_impl": "sequential", "connection_impl": "identity",
                              "connection_damping": 1.0, "value_gate": [3 * D, R],
                              "value_gate_input_mode": "current_prev_prefix",
                              "couple_forget_to_value_gate": True,
                              "mogt_residual_scale": 0.7 if i else 1.0,
                              "mogt_ffn_residual_scale": 1.3 if i else 1.0} for i in range(2)]}

    # ---- single blocks ------------------------------------------------------
    def block_case(tag: str, cfg: dict, with_prefix: bool) -> None:
        torch.manual_seed(2)
        blk = mm.MOGTBlock(d_model=D, r=R)
        blk.ffn = mm.SwiGLU(D, 4 * D)
        blk.scan_impl = "sequential"
        blk.connection_impl = cfg["connection_impl"]
        blk.connection_damping = cfg["connection_damping"]
        if cfg.get("transport_gate"):
            blk.phi_transport_gate = torch.nn.Linear(D, cfg["transport_gate"], bias=True)
            blk.transport_gate_mode = cfg["transport_gate_mode"]
            blk.transport_gate_scale = cfg["transport_gate_scale"]
        if cfg.get("value_gate"):
            n_in = {"current": 1, "current_prev": 2, "current_prev_prefix": 3}[cfg["value_gate_input_mode"]]
            blk.phi_value_gate = torch.nn.Linear(n_in * D, cfg["value_gate"], bias=True)
            blk.value_gate_input_mode = cfg["value_gate_input_mode"]
            blk.couple_forget_to_value_gate = cfg["couple_forget_to_value_gate"]
        if cfg.get("residual_gate"):
            blk.mogt_residual_gate_enabled = True
            blk.mogt_residual_gate_logit = torch.nn.Parameter(torch.zeros(()))
        blk.mogt_residual_scale = cfg.get("mogt_residual_scale", 1.0)
        _reseed_weights(blk, gen)
        blk.eval()
        x = _f32(torch.randn(B, 24, D, generator=gen))
        prefix = _f32(torch.randn(B, D, generator=gen)) if with_prefix else None
        with torch.no_grad():
            out = blk(x, prefix_condition=prefix)
        arrays.update(_arrays_of(tag, blk.state_dict()))
        arrays[f"{tag}/x"] = x.float().numpy()
        if prefix is not None:
            arrays[f"{tag}/prefix"] = prefix.float().numpy()
        arrays[f"{tag}/out"] = out.numpy()
        meta[tag] = cfg

    block_case("bx", {"connection_impl": "matrix_exp", "connection_damping": 0.999,
                      "transport_gate": R, "transport_gate_mode": "residual", "transport_gate_scale": 0.5,
                      "value_gate": 1, "value_gate_input_mode": "current_prev",
                      "couple_forget_to_value_gate": False}, False)
    block_case("bc", {"connection_impl": "cayley", "connection_damping": 0.999,
                      "transport_gate": 1, "transport_gate_mode": "forget_relu", "transport_gate_scale": 0.8,
                      "value_gate": R, "value_gate_input_mode": "current_prev_prefix",
                      "couple_forget_to_value_gate": True, "residual_gate": True,
                      "mogt_residual_scale": 0.9}, True)
    block_case("bi", {"connection_impl": "identity", "connection_damping": 0.95,
                      "transport_gate": R, "transport_gate_mode": "multiply", "transport_gate_scale": 1.0},
               False)

    # ---- lm: init order and values, losses -----------------------------------
    torch.manual_seed(1234)
    lm = mm.MOGTForCausalLM(vocab_size=VOCAB, d_model=D, num_layers=2, r=R)
    # the initial values are only compared: a hash, the sum and the first few
    # entries per tensor
    meta["lm_init"] = {k: {"sha256": hashlib.sha256(v.detach().numpy().tobytes()).hexdigest(),
                           "sum": float(v.sum()), "head": v.detach().flatten()[:4].tolist(),
                           "shape": list(v.shape)}
                       for k, v in lm.state_dict().items()}
    torch.manual_seed(4321)
    lm = mm.MOGTForCausalLM(vocab_size=VOCAB, d_model=D, num_layers=1, r=R)
    # the zero-initialised read-outs would hide the block: reseed, then score
    _reseed_weights(lm, gen)
    for blk in lm.mogt.blocks:
        blk.scan_impl = "sequential"
    lm.eval()
    ids = torch.randint(0, VOCAB, (B, L), generator=gen)
    labels = torch.randint(0, VOCAB, (B, L), generator=gen)
    with torch.no_grad():
        logits, loss = lm(ids, labels=labels)
        logits_c, loss_c = lm(ids, labels=labels, loss_chunk_size=16)
        hid = lm.mogt(ids)
    hid_g = hid.clone().requires_grad_()
    w = lm.lm_head.weight.detach().clone().requires_grad_()
    loss_f = chunked_linear_cross_entropy(hid_g, w, labels, chunk_size=24)
    g_hid, g_w = torch.autograd.grad(loss_f, (hid_g, w))
    arrays.update(_arrays_of("lm", lm.state_dict()))
    arrays.update({"lm/ids": ids.numpy(), "lm/labels": labels.numpy(), "lm/logits": logits.numpy(),
                   "lm/loss": loss.numpy(), "lm/logits_chunked": logits_c.numpy(),
                   "lm/loss_chunked": loss_c.numpy(), "lm/hidden": hid.numpy(),
                   "lm/loss_fused": loss_f.detach().numpy(), "lm/grad_hidden": g_hid.numpy(),
                   "lm/grad_weight": g_w.numpy()})
    meta["lm"] = {"layers": 1, "init_seed": 1234, "init_layers": 2, "loss_chunk_size": 16, "ce_chunk_size": 24}

    # ---- ga: gate dtype flow under bf16 autocast ------------------------------
    torch.set_default_dtype(torch.float32)
    torch.manual_seed(3)
    blk = mm.MOGTBlock(d_model=D, r=R)
    blk.scan_impl = "sequential"
    blk.connection_impl = "identity"
    blk.connection_damping = 0.98
    blk.phi_value_gate = torch.nn.Linear(2 * D, R, bias=True)
    blk.value_gate_input_mode = "current_prev"
    blk.couple_forget_to_value_gate = True
    _reseed_weights(blk, gen)
    blk.eval()
    captured = {}
    blk.phi_val.register_forward_hook(lambda m, i, o: captured.__setitem__("v_raw", o.detach().clone()))
    blk.phi_value_gate.register_forward_hook(lambda m, i, o: captured.__setitem__("z", o.detach().float().clone()))
    original = mm.affine_scan_sequential

    def recording_scan(U, V, **kw):
        captured["U"], captured["V"] = U.detach().clone(), V.detach().clone()
        return original(U, V, **kw)

    mm.affine_scan_sequential = recording_scan
    try:
        x = torch.randn(B, L, D, generator=gen, dtype=torch.float32)
        with torch.no_grad(), torch.autocast(device_type="cpu", dtype=torch.bfloat16):
            blk(x)
    finally:
        mm.affine_scan_sequential = original
    assert captured["v_raw"].dtype == torch.bfloat16 and captured["V"].dtype == torch.bfloat16
    assert captured["U"].dtype == torch.float32
    arrays.update(_arrays_of("ga", {k: captured[k] for k in ("z", "v_raw", "U", "V")}))
    meta["ga"] = {"damping": 0.98, "dtypes": {k: str(captured[k].dtype) for k in ("z", "v_raw", "U", "V")},
                  "torch": torch.__version__}

    # ---- tt: transport-only mode (fast_throughput_mode) ----------------------
    torch.set_default_dtype(torch.float64)

    def fused_prefix(U):
        """triton_fused_scan's recurrence Y_t = U_t Y_{t-1}, Y_0 = I
        (triton_scan.py:37-48), as the reference's own prefix product."""
        Y, _ = mm.affine_scan_sequential(U, torch.zeros_like(U[..., :1]), state_dtype=U.dtype,
                                         output_dtype=U.dtype, return_prefix=True)
        return Y

    import types
    sys.modules["triton_scan"] = types.SimpleNamespace(triton_fused_scan=fused_prefix)
    torch.manual_seed(5)
    DT, RT = 64, 16
    blk = mm.MOGTBlock(d_model=DT, r=RT)
    blk.ffn = mm.SwiGLU(DT, 2 * DT)
    blk.fast_throughput_mode = True
    blk.connection_impl = "matrix_exp"
    blk.connection_damping = 0.999
    blk.phi_transport_gate = torch.nn.Linear(DT, RT, bias=True)
    blk.transport_gate_mode = "multiply"
    blk.phi_value_gate = torch.nn.Linear(DT, 1, bias=True)
    blk.value_gate_input_mode = "current"
    blk.couple_forget_to_value_gate = True
    _reseed_weights(blk, gen)
    blk.eval()
    x = _f32(torch.randn(B, 24, DT, generator=gen))
    with torch.no_grad():
        out = blk(x)
    del sys.modules["triton_scan"]
    arrays.update(_arrays_of("tt", blk.state_dict()))
    arrays["tt/x"] = x.float().numpy()
    arrays["tt/out"] = out.numpy()
    meta["tt"] = {"d_model": DT, "r": RT, "ffn_hidden": 2 * DT, "fast_throughput_mode": True,
                  "connection_impl": "matrix_exp", "connection_damping": 0.999, "transport_gate": RT,
                  "transport_gate_mode": "multiply", "value_gate": 1, "value_gate_input_mode": "current",
                  "couple_forget_to_value_gate": True}

    # ---- ck: gradient checkpointing, scan_impl per block ---------------------
    torch.manual_seed(6)
    model = mm.MOGTModel(vocab_size=VOCAB, d_model=D, num_layers=3, r=R)
    impls = ["parallel_reference", "block_reference", "sequential"]
    for i, blk in enumerate(model.blocks):
        blk.ffn = mm.SwiGLU(D, 4 * D)
        blk.scan_impl = impls[i]
        blk.scan_block_size = 7
        blk.block_carry_scan = "doubling"
        blk.connection_impl = "identity"
        blk.connection_damping = 1.0
        blk.phi_value_gate = torch.nn.Linear(3 * D, R, bias=True)
        blk.value_gate_input_mode = "current_prev_prefix"
        blk.couple_forget_to_value_gate = True
    model.prefix_condition_position = 1
    model.gradient_checkpointing = True
    model.checkpoint_every_n = 2
    _reseed_weights(model, gen)
    model.train()
    ids = torch.randint(0, VOCAB, (B, L), generator=gen)
    wts = _f32(torch.randn(B, L, D, generator=gen))
    calls = [0, 0, 0]
    hooks = [blk.register_forward_pre_hook(lambda m, a, i=i: calls.__setitem__(i, calls[i] + 1))
             for i, blk in enumerate(model.blocks)]
    y = model(ids)
    loss = (y * wts).sum()
    loss.backward()
    for h in hooks:
        h.remove()
    assert calls == [2, 1, 2], calls     # blocks 0 and 2 recomputed in backward
    arrays.update(_arrays_of("ck", model.state_dict()))
    arrays.update({"ck/ids": ids.numpy(), "ck/w": wts.float().numpy(), "ck/out": y.detach().numpy(),
                   "ck/loss": loss.detach().numpy()})
    no_grad = []
    for name, p_ in model.named_parameters():
        if p_.grad is None:          # phi_conn: the identity connection ignores A
            no_grad.append(name)
        else:
            arrays[f"ck/grad/{name}"] = p_.grad.numpy()
    meta["ck"] = {"params_without_grad": no_grad,"layers": 3, "ffn_hidden": 4 * D, "prefix_condition_position": 1,
                  "gradient_checkpointing": True, "checkpoint_every_n": 2, "scan_impl": impls,
                  "scan_block_size": 7, "block_carry_scan": "doubling", "block_calls": calls}

    # ---- pr, br: parallel / block reference scans on a dense transport -------
    def dense_case(tag: str, cfg: dict) -> None:
        torch.manual_seed(7)
        blk = mm.MOGTBlock(d_model=D, r=R)
        blk.ffn = mm.SwiGLU(D, 4 * D)
        for k_, v_ in cfg.items():
            setattr(blk, k_, v_)
        blk.phi_value_gate = torch.nn.Linear(2 * D, R, bias=True)
        blk.value_gate_input_mode = "current_prev"
        blk.couple_forget_to_value_gate = True
        _reseed_weights(blk, gen)
        blk.eval()
        x = _f32(torch.randn(B, 24, D, generator=gen))
        with torch.no_grad():
            out = blk(x)
        arrays.update(_arrays_of(tag, blk.state_dict()))
        arrays[f"{tag}/x"] = x.float().numpy()
        arrays[f"{tag}/out"] = out.numpy()
        meta[tag] = dict(cfg, value_gate=R, value_gate_input_mode="current_prev",
                         couple_forget_to_value_gate=True)

    dense_case("pr", {"scan_impl": "parallel_reference", "connection_impl": "matrix_exp",
                      "connection_damping": 0.999})
    dense_case("br", {"scan_impl": "block_reference", "connection_impl": "cayley", "connection_damping": 0.99,
                      "scan_block_size": 5, "block_carry_scan": "doubling"})

    np.savez_compressed(HERE / "model_fixtures.npz", **arrays)
    manifest = {"meta": meta,
                "sha256": {k: hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest()
                           for k, v in sorted(arrays.items())}}
    (HERE / "model_fixtures.json").write_text(json.dumps(manifest, indent=1, sort_keys=True) + "\n")
    print(f"wrote {len(arrays)} arrays")


if __name__ == "__main__":
    main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
