"""The model oracle against the reference's own classes.

tests/golden/model_fixtures.npz holds float64 outputs of the reference's
MOGTModel / MOGTBlock / MOGTForCausalLM (model_mogt.py) and chunked loss
(chunked_lm_loss.py) on seeded weights, written by
tests/golden/make_model_fixtures.py.  These tests pin the CPU restatements in
oracle/ to them; the GPU tests then compare the HIP paths with the pinned
oracle and with the same fixtures.

The reference computes some steps in float32 whatever the input dtype
(RMSNorm statistics, connection map, gates, scan state).  With
``ref_casts=True`` the oracle takes those same steps and must agree to 1e-12;
in its all-float64 mode (the one the GPU paths are checked against) it must
agree to the reference's own float32 rounding (FP32_GAP)."""
import numpy as np
import pytest
import torch

from conftest import rel_err
from golden import fixtures as fx
from oracle import lm_loss_oracle as lo
from oracle import model_oracle as mo
from oracle import scan_oracle as so

R = 4
EXACT = 1e-12
FP32_GAP = 2e-6


def _block_cfg(m: dict) -> dict:
    cfg = {"r": R, "connection_impl": m["connection_impl"], "connection_damping": m["connection_damping"]}
    for k in ("transport_gate_mode", "transport_gate_scale", "value_gate_input_mode",
              "couple_forget_to_value_gate", "mogt_residual_scale", "mogt_ffn_residual_scale"):
        if k in m:
            cfg[k] = m[k]
    cfg["residual_gate"] = bool(m.get("residual_gate"))
    return cfg


def test_fixture_checksums():
    arrays, meta = fx.load()
    assert len(arrays) > 50 and {"bb", "bx", "bc", "bi", "lm", "lm_init", "ga"} <= set(meta)


def test_backbone_oracle_matches_reference():
    g = fx.group("bb")
    m = fx.meta("bb")
    cfgs = [_block_cfg(b) for b in m["blocks"]]
    for ref_casts, tol in ((True, EXACT), (False, FP32_GAP)):
        outs = []
        y = mo.model_forward(fx.state_dict("bb"), g["ids"], m["layers"], cfgs,
                             prefix_position=m["prefix_condition_position"], block_outputs=outs,
                             ref_casts=ref_casts)
        for i, o in enumerate(outs):
            assert rel_err(o.numpy(), g[f"block{i}_out"].numpy()) < tol, f"block {i} ref_casts={ref_casts}"
        assert rel_err(y.numpy(), g["out"].numpy()) < tol


@pytest.mark.parametrize("tag", ["bx", "bc", "bi"])
def test_block_oracle_matches_reference(tag):
    g = fx.group(tag)
    cfg = _block_cfg(fx.meta(tag))
    for ref_casts, tol in ((True, EXACT), (False, FP32_GAP)):
        y = mo.block_forward(fx.state_dict(tag), g["x"], g.get("prefix"), cfg, ref_casts=ref_casts)
        assert rel_err(y.numpy(), g["out"].numpy()) < tol, f"ref_casts={ref_casts}"


def test_planted_mistakes_fail_the_backbone_pin():
    """Misreadings of model_mogt.py that the pin must catch: the previous-token
    gate input taken from the wrong position, the prefix from position 0, the
    damping dropped, the residual scales swapped."""
    g = fx.group("bb")
    m = fx.meta("bb")
    st = fx.state_dict("bb")
    good = [_block_cfg(b) for b in m["blocks"]]
    ref = g["out"].numpy()

    def err(cfgs, pos=m["prefix_condition_position"]):
        return rel_err(mo.model_forward(st, g["ids"], m["layers"], cfgs, prefix_position=pos,
                                        ref_casts=True).numpy(), ref)

    assert err(good) < EXACT
    assert err(good, pos=0) > 1e-6
    swapped = [dict(c, mogt_residual_scale=c["mogt_ffn_residual_scale"],
                    mogt_ffn_residual_scale=c["mogt_residual_scale"]) for c in good]
    assert err(swapped) > 1e-6
    undamped = [dict(c, connection_damping=0.9) for c in good]
    assert err(undamped) > 1e-6
    uncoupled = [dict(c, couple_forget_to_value_gate=False) for c in good]
    assert err(uncoupled) > 1e-6
    current_only = [dict(c, value_gate_input_mode="current") for c in good]
    with pytest.raises(RuntimeError):   # the gate weight expects the 3-part input
        err(current_only)


def test_coupled_gate_inputs_match_reference_dtype_flow():
    """Under bf16 autocast the reference multiplies the bf16 phi_val output by
    the gate cast to bf16 (model_mogt.py:180) and scales the fp32 U by (1 - g)
    (model_mogt.py:182): scan_oracle.coupled_gate_inputs reproduces both."""
    g = fx.group("ga", torch.float32)
    damping = fx.meta("ga")["damping"]
    z = g["z"].numpy()
    B, L, r, c = g["V"].shape
    v_raw = g["v_raw"].numpy().reshape(B, L, r * c)
    a, b = so.coupled_gate_inputs(z, v_raw, r, damping=damping, v_is_bf16=True)
    U = g["U"].numpy()
    diag = np.diagonal(U, axis1=-2, axis2=-1)                  # [B, L, r]
    off = U - np.einsum("blr,rs->blrs", diag, np.eye(r, dtype=U.dtype))
    assert not off.any()
    a_ref = np.repeat(diag, c, axis=-1)
    # sigmoid differs from torch's float32 one by at most an ulp
    assert np.max(np.abs(a - a_ref)) <= 2 * np.finfo(np.float32).eps
    b_ref = g["V"].numpy().reshape(B, L, r * c)
    mism = np.mean(b != b_ref)
    assert mism < 1e-3, f"{mism:.2%} of the gated values differ"
    assert rel_err(b, b_ref) < 1e-2 * 2 ** -7


def test_lm_initialisation_matches_reference():
    """MOGTForCausalLM's initialisation (model_mogt.py:295-324): same
    parameters, same order of random draws, same values at a fixed seed."""
    import hashlib

    from mogt_amd.model_mogt import MOGTForCausalLM

    init = fx.meta("lm_init")
    m = fx.meta("lm")
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    try:
        torch.manual_seed(m["init_seed"])
        lm = MOGTForCausalLM(vocab_size=fx.meta("VOCAB"), d_model=fx.meta("D"),
                             num_layers=m["init_layers"], r=R)
    finally:
        torch.set_default_dtype(old)
    sd = lm.state_dict()
    assert set(sd) == set(init)
    for k, v in sd.items():
        want = init[k]
        assert list(v.shape) == want["shape"], k
        assert v.flatten()[:4].tolist() == want["head"], k
        assert hashlib.sha256(v.detach().numpy().tobytes()).hexdigest() == want["sha256"], k


def test_lm_losses_oracle_matches_reference():
    g = fx.group("lm")
    m = fx.meta("lm")
    st = fx.state_dict("lm", strip="mogt.")
    cfg = {"r": R}   # the reference's default block: matrix_exp, damping 0.999
    hidden = mo.model_forward(st, g["ids"], m["layers"], cfg, ref_casts=True)
    assert rel_err(hidden.numpy(), g["hidden"].numpy()) < EXACT
    hidden64 = mo.model_forward(st, g["ids"], m["layers"], cfg)
    assert rel_err(hidden64.numpy(), g["hidden"].numpy()) < FP32_GAP
    # the LM head and F.cross_entropy run in the hidden states' dtype (float64)
    w = g["lm_head.weight"].numpy()
    labels = g["labels"].numpy()
    logits = g["hidden"].numpy() @ w.T
    assert rel_err(logits, g["logits"].numpy()) < EXACT
    assert rel_err(logits, g["logits_chunked"].numpy()) < EXACT
    loss, _, _ = lo.chunked_linear_ce(g["hidden"].numpy(), w, labels, 7)
    assert abs(loss - float(g["loss"])) < EXACT * abs(loss)
    assert abs(loss - float(g["loss_chunked"])) < EXACT * abs(loss)
    # chunked_linear_cross_entropy computes its logits from .float() copies
    # (chunked_lm_loss.py:29, :61): float32 logits, float64 sums
    loss, gh, gw = lo.chunked_linear_ce(g["hidden"].numpy(), w, labels, m["ce_chunk_size"])
    assert abs(loss - float(g["loss_fused"])) < FP32_GAP * abs(loss)
    assert rel_err(gh, g["grad_hidden"].numpy()) < 1e-5
    assert rel_err(gw, g["grad_weight"].numpy()) < 1e-5


def _cfg_of(m: dict, r: int = R) -> dict:
    cfg = _block_cfg(m)
    cfg["r"] = r
    for k in ("scan_impl", "fast_throughput_mode"):
        if k in m:
            cfg[k] = m[k]
    return cfg


def test_transport_only_oracle_matches_reference():
    """fast_throughput_mode / scan_impl="transport_triton" (model_mogt.py:71-74,
    187-192): V_t = (U_t ... U_1) V_raw, not the affine recurrence.  Exact with
    the reference's float32 steps; the affine scan in its place fails the pin."""
    g = fx.group("tt")
    m = fx.meta("tt")
    cfg = _cfg_of(m, r=m["r"])
    for ref_casts, tol in ((True, EXACT), (False, FP32_GAP)):
        y = mo.block_forward(fx.state_dict("tt"), g["x"], None, cfg, ref_casts=ref_casts)
        assert rel_err(y.numpy(), g["out"].numpy()) < tol, f"ref_casts={ref_casts}"
    affine = {k: v for k, v in cfg.items() if k != "fast_throughput_mode"}
    y = mo.block_forward(fx.state_dict("tt"), g["x"], None, affine, ref_casts=True)
    assert rel_err(y.numpy(), g["out"].numpy()) > 1e-3


@pytest.mark.parametrize("tag", ["pr", "br"])
def test_parallel_and_block_reference_scans_match_the_recurrence(tag):
    """scan_impl="parallel_reference" (affine_scan_doubling) and
    "block_reference" (affine_scan_block_reference, block 5, doubling carries)
    on a dense transport (model_mogt.py:204-221): the reference evaluates them
    with a float32 state, so they agree with the sequential recurrence to
    float32 rounding."""
    g = fx.group(tag)
    cfg = _cfg_of(fx.meta(tag))
    for ref_casts in (True, False):
        y = mo.block_forward(fx.state_dict(tag), g["x"], None, cfg, ref_casts=ref_casts)
        assert rel_err(y.numpy(), g["out"].numpy()) < FP32_GAP, f"ref_casts={ref_casts}"


def test_checkpointed_backbone_oracle_matches_reference():
    """A 3-layer MOGTModel trained with gradient checkpointing every 2 blocks
    (model_mogt.py:278-285; blocks 0 and 2 recomputed in the backward) and one
    scan_impl per block: output, loss and every parameter's gradient against
    float64 autograd of the oracle."""
    g = fx.group("ck")
    m = fx.meta("ck")
    assert m["block_calls"] == [2, 1, 2]
    cfg = _cfg_of(fx.meta("bb")["blocks"][0])
    st = {k: v.clone().requires_grad_() for k, v in fx.state_dict("ck").items()}
    y = mo.model_forward(st, g["ids"], m["layers"], cfg, prefix_position=m["prefix_condition_position"])
    assert rel_err(y.detach().numpy(), g["out"].numpy()) < FP32_GAP
    loss = (y * g["w"]).sum()
    assert abs(float(loss.detach()) - float(g["loss"])) < FP32_GAP * abs(float(g["loss"])) * 10
    loss.backward()
    want = fx.grads("ck")
    assert set(want) == {k for k in st if "phi_conn" not in k}
    for k, gw in want.items():
        assert rel_err(st[k].grad.numpy(), gw.numpy()) < 1e-5, k
