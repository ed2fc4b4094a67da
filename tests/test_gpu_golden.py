"""The HIP model paths against the reference's own outputs.

tests/golden/model_fixtures.npz holds float64 runs of the reference's
MOGTModel, MOGTBlock, MOGTForCausalLM and chunked loss on seeded weights
(tests/golden/make_model_fixtures.py).  Here the same weights are loaded into
this package's classes on the GPU and run in fp32 (bar 1e-4) and under bf16
autocast (bar 2e-2, normwise max relative error)."""
import pytest
import torch
import torch.nn as nn

from conftest import announce, rel_err, to_np
from golden import fixtures as fx

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
BF16_TOL = 2e-2


def _to(sd: dict, dev) -> dict:
    return {k: v.to(torch.float32).to(dev) for k, v in sd.items()}


def _backbone(dev):
    from mogt_amd.model_mogt import MOGTModel

    m = fx.meta("bb")
    D, R, V = fx.meta("D"), fx.meta("R"), fx.meta("VOCAB")
    model = MOGTModel(vocab_size=V, d_model=D, num_layers=m["layers"], r=R, ffn_hidden=m["ffn_hidden"]).to(dev)
    for blk, cfg in zip(model.blocks, m["blocks"]):
        blk.scan_impl = cfg["scan_impl"]
        blk.connection_impl = cfg["connection_impl"]
        blk.connection_damping = cfg["connection_damping"]
        blk.phi_value_gate = nn.Linear(*cfg["value_gate"], bias=True).to(dev)
        blk.value_gate_input_mode = cfg["value_gate_input_mode"]
        blk.couple_forget_to_value_gate = cfg["couple_forget_to_value_gate"]
        blk.mogt_residual_scale = cfg["mogt_residual_scale"]
        blk.mogt_ffn_residual_scale = cfg["mogt_ffn_residual_scale"]
    model.prefix_condition_position = m["prefix_condition_position"]
    model.load_state_dict(_to(fx.state_dict("bb"), dev))
    return model.eval()


@pytest.mark.parametrize("path", ["fused", "generic"])
def test_backbone_fixture_fp32(gpu, path, monkeypatch):
    announce(f"backbone fixture fp32 {path}")
    from mogt_amd.model_mogt import MOGTBlock

    model = _backbone(gpu)
    assert all(b.fused_path_ok() for b in model.blocks)
    if path == "generic":
        monkeypatch.setattr(MOGTBlock, "fused_path_ok", lambda self: False)
    g = fx.group("bb")
    with torch.no_grad():
        out = model(g["ids"].to(gpu))
    torch.cuda.synchronize()
    assert rel_err(to_np(out), g["out"].numpy()) <= FP32_TOL


def test_backbone_fixture_bf16_autocast(gpu):
    announce("backbone fixture bf16 autocast")
    model = _backbone(gpu)
    g = fx.group("bb")
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        out = model(g["ids"].to(gpu))
    torch.cuda.synchronize()
    assert rel_err(to_np(out), g["out"].numpy()) <= BF16_TOL


@pytest.mark.parametrize("tag", ["bx", "bc", "bi"])
def test_block_fixture_fp32(gpu, tag):
    """Non-identity connections (matrix_exp, Cayley) on the dense scan, every
    transport-gate mode, scalar and rank value gates, the prefix input, the
    learned residual gate; identity with a transport gate on the diagonal scan."""
    announce(f"block fixture {tag}")
    from mogt_amd.model_mogt import MOGTBlock

    m = fx.meta(tag)
    D, R = fx.meta("D"), fx.meta("R")
    blk = MOGTBlock(d_model=D, r=R, ffn_hidden=4 * D).to(gpu)
    blk.scan_impl = "sequential"
    blk.connection_impl = m["connection_impl"]
    blk.connection_damping = m["connection_damping"]
    if m.get("transport_gate"):
        blk.phi_transport_gate = nn.Linear(D, m["transport_gate"], bias=True).to(gpu)
        blk.transport_gate_mode = m["transport_gate_mode"]
        blk.transport_gate_scale = m["transport_gate_scale"]
    if m.get("value_gate"):
        n_in = {"current": 1, "current_prev": 2, "current_prev_prefix": 3}[m["value_gate_input_mode"]]
        blk.phi_value_gate = nn.Linear(n_in * D, m["value_gate"], bias=True).to(gpu)
        blk.value_gate_input_mode = m["value_gate_input_mode"]
        blk.couple_forget_to_value_gate = m["couple_forget_to_value_gate"]
    if m.get("residual_gate"):
        blk.mogt_residual_gate_enabled = True
        blk.mogt_residual_gate_logit = nn.Parameter(torch.zeros((), device=gpu))
    blk.mogt_residual_scale = m.get("mogt_residual_scale", 1.0)
    blk.load_state_dict(_to(fx.state_dict(tag), gpu))
    blk.eval()
    g = fx.group(tag, torch.float32)
    prefix = g["prefix"].to(gpu) if "prefix" in g else None
    with torch.no_grad():
        out = blk(g["x"].to(gpu), prefix_condition=prefix)
    torch.cuda.synchronize()
    assert rel_err(to_np(out), fx.group(tag)["out"].numpy()) <= FP32_TOL


def _configured_block(dev, tag: str, d_model: int, r: int, ffn_hidden: int):
    """This package's MOGTBlock with a fixture group's duck-typed attributes
    and weights."""
    from mogt_amd.model_mogt import MOGTBlock

    m = fx.meta(tag)
    blk = MOGTBlock(d_model=d_model, r=r, ffn_hidden=ffn_hidden).to(dev)
    for k in ("scan_impl", "fast_throughput_mode", "connection_impl", "connection_damping",
              "scan_block_size", "block_carry_scan", "transport_gate_mode", "value_gate_input_mode",
              "couple_forget_to_value_gate"):
        if k in m:
            setattr(blk, k, m[k])
    if m.get("transport_gate"):
        blk.phi_transport_gate = nn.Linear(d_model, m["transport_gate"], bias=True).to(dev)
    if m.get("value_gate"):
        n_in = {"current": 1, "current_prev": 2, "current_prev_prefix": 3}[m["value_gate_input_mode"]]
        blk.phi_value_gate = nn.Linear(n_in * d_model, m["value_gate"], bias=True).to(dev)
    blk.load_state_dict(_to(fx.state_dict(tag), dev))
    return blk.eval()


@pytest.mark.parametrize("autocast", [False, True])
def test_transport_only_fixture(gpu, autocast):
    """fast_throughput_mode (scan_impl = "transport_triton", model_mogt.py:71-74,
    187-192): V_t = Y_t V_raw with the HIP prefix product Y (triton_fused_scan)
    on a matrix_exp transport with rank-wise transport and coupled value gates,
    r = 16 as the reference's kernel requires."""
    announce(f"transport-only fixture autocast={autocast}")
    m = fx.meta("tt")
    blk = _configured_block(gpu, "tt", m["d_model"], m["r"], m["ffn_hidden"])
    assert blk._resolve_scan_impl() == "transport_triton"
    g = fx.group("tt", torch.float32)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        out = blk(g["x"].to(gpu))
    torch.cuda.synchronize()
    assert rel_err(to_np(out), fx.group("tt")["out"].numpy()) <= (BF16_TOL if autocast else FP32_TOL)


@pytest.mark.parametrize("tag", ["pr", "br"])
def test_parallel_and_block_reference_fixtures(gpu, tag):
    """scan_impl = "parallel_reference" (matrix_exp) and "block_reference"
    (Cayley, block 5, doubling carries) selected on the block
    (model_mogt.py:204-221), on the dense HIP scan."""
    announce(f"block fixture {tag}")
    blk = _configured_block(gpu, tag, fx.meta("D"), fx.meta("R"), 4 * fx.meta("D"))
    assert blk._resolve_scan_impl() == fx.meta(tag)["scan_impl"]
    g = fx.group(tag, torch.float32)
    with torch.no_grad():
        out = blk(g["x"].to(gpu))
    torch.cuda.synchronize()
    assert rel_err(to_np(out), fx.group(tag)["out"].numpy()) <= FP32_TOL


def test_checkpointed_backbone_fixture_training(gpu):
    """A 3-layer backbone in training mode with gradient_checkpointing and
    checkpoint_every_n = 2 (model_mogt.py:278-285) and blocks selecting
    parallel_reference / block_reference / sequential: blocks 0 and 2 run
    again in the backward, and the output, the loss and every parameter's
    gradient match the reference's float64 run."""
    announce("checkpointed backbone fixture (training)")
    from mogt_amd.model_mogt import MOGTModel

    m = fx.meta("ck")
    D, R, V = fx.meta("D"), fx.meta("R"), fx.meta("VOCAB")
    model = MOGTModel(vocab_size=V, d_model=D, num_layers=m["layers"], r=R, ffn_hidden=m["ffn_hidden"]).to(gpu)
    for blk, impl in zip(model.blocks, m["scan_impl"]):
        blk.scan_impl = impl
        blk.scan_block_size = m["scan_block_size"]
        blk.block_carry_scan = m["block_carry_scan"]
        blk.connection_impl = "identity"
        blk.connection_damping = 1.0
        blk.phi_value_gate = nn.Linear(3 * D, R, bias=True).to(gpu)
        blk.value_gate_input_mode = "current_prev_prefix"
        blk.couple_forget_to_value_gate = True
    model.prefix_condition_position = m["prefix_condition_position"]
    model.gradient_checkpointing = m["gradient_checkpointing"]
    model.checkpoint_every_n = m["checkpoint_every_n"]
    model.load_state_dict(_to(fx.state_dict("ck"), gpu))
    model.train()
    calls = [0] * len(model.blocks)
    hooks = [blk.register_forward_pre_hook(lambda mod, a, i=i: calls.__setitem__(i, calls[i] + 1))
             for i, blk in enumerate(model.blocks)]
    g = fx.group("ck", torch.float32)
    y = model(g["ids"].to(gpu))
    loss = (y * g["w"].to(gpu)).sum()
    loss.backward()
    torch.cuda.synchronize()
    for h in hooks:
        h.remove()
    assert calls == m["block_calls"]
    ref = fx.group("ck")
    assert rel_err(to_np(y.detach()), ref["out"].numpy()) <= FP32_TOL
    assert abs(float(loss.detach()) - float(ref["loss"])) <= FP32_TOL * abs(float(ref["loss"]))
    params = dict(model.named_parameters())
    want = fx.grads("ck")
    for k, gw in want.items():
        assert params[k].grad is not None, k
        assert rel_err(to_np(params[k].grad), gw.numpy()) <= FP32_TOL, k
    for k in m["params_without_grad"]:
        assert params[k].grad is None or not params[k].grad.any(), k


def _lm(dev):
    from mogt_amd.model_mogt import MOGTForCausalLM

    lm = MOGTForCausalLM(vocab_size=fx.meta("VOCAB"), d_model=fx.meta("D"), num_layers=fx.meta("lm")["layers"],
                         r=fx.meta("R")).to(dev)
    lm.load_state_dict(_to(fx.state_dict("lm"), dev))
    return lm.eval()


def test_lm_fixture_losses(gpu):
    """MOGTForCausalLM.forward's three loss paths (model_mogt.py:350-380):
    unchunked, chunked with logits, chunked without logits."""
    announce("LM fixture losses")
    lm = _lm(gpu)
    g = fx.group("lm")
    ids, labels = g["ids"].to(gpu), g["labels"].to(gpu)
    with torch.no_grad():
        logits, loss = lm(ids, labels=labels)
        logits_c, loss_c = lm(ids, labels=labels, loss_chunk_size=16)
        none, loss_f = lm(ids, labels=labels, return_logits=False, loss_chunk_size=16)
    torch.cuda.synchronize()
    assert none is None
    assert rel_err(to_np(logits), g["logits"].numpy()) <= FP32_TOL
    assert rel_err(to_np(logits_c), g["logits_chunked"].numpy()) <= FP32_TOL
    for got, want in ((loss, g["loss"]), (loss_c, g["loss_chunked"]), (loss_f, g["loss_fused"])):
        assert abs(float(got) - float(want)) <= FP32_TOL * abs(float(want))


def test_lm_fixture_chunked_ce_gradients(gpu):
    """chunked_linear_cross_entropy's loss and both gradients on the fixture's
    hidden states and tied weight."""
    announce("LM fixture chunked CE gradients")
    from mogt_amd.chunked_lm_loss import chunked_linear_cross_entropy

    g = fx.group("lm", torch.float32)
    h = g["hidden"].to(gpu).requires_grad_()
    w = g["lm_head.weight"].to(gpu).requires_grad_()
    loss = chunked_linear_cross_entropy(h, w, g["labels"].to(gpu), chunk_size=fx.meta("lm")["ce_chunk_size"])
    loss.backward()
    torch.cuda.synchronize()
    g64 = fx.group("lm")
    assert abs(float(loss.detach()) - float(g64["loss_fused"])) <= FP32_TOL * abs(float(g64["loss_fused"]))
    assert rel_err(to_np(h.grad), g64["grad_hidden"].numpy()) <= FP32_TOL
    assert rel_err(to_np(w.grad), g64["grad_weight"].numpy()) <= FP32_TOL


def test_lm_training_step_gradients_vs_float64_autograd(gpu):
    """One backward of MOGTForCausalLM (1 layer, matrix_exp connection, the
    reference's default block) against float64 autograd of the pinned oracle
    on the fixture's weights: every parameter's gradient."""
    announce("LM training step vs float64 autograd")
    from oracle import model_oracle as mo

    lm = _lm(gpu)
    lm.train()
    g = fx.group("lm")
    ids, labels = g["ids"], g["labels"]
    _, loss = lm(ids.to(gpu), labels=labels.to(gpu))
    loss.backward()
    torch.cuda.synchronize()
    st = {k: v.clone().requires_grad_() for k, v in fx.state_dict("lm").items() if k != "lm_head.weight"}
    inner = {k[len("mogt."):]: v for k, v in st.items()}
    hidden = mo.model_forward(inner, ids, 1, {"r": fx.meta("R")})
    logits = hidden @ st["mogt.embedding.weight"].t()
    ref = torch.nn.functional.cross_entropy(logits.reshape(-1, logits.size(-1)), labels.reshape(-1))
    names = list(st)
    grads = torch.autograd.grad(ref, [st[n] for n in names], allow_unused=True)
    assert abs(float(loss.detach()) - float(ref.detach())) <= FP32_TOL * abs(float(ref.detach()))
    params = dict(lm.named_parameters())
    for n, gr in zip(names, grads):
        if gr is None:
            continue
        mine = params[n].grad
        assert mine is not None, n
        assert rel_err(to_np(mine), gr.detach().numpy()) <= FP32_TOL, n


def test_chunked_ce_forward_autocast_backward_outside(gpu):
    """The forward under bf16 autocast (bf16 logits, their log-sum-exp saved)
    and the backward outside it: the backward recomputes the logits under the
    forward's autocast state, so softmax rows stay normalised; loss and both
    gradients against float64."""
    announce("chunked CE: forward under autocast, backward outside")
    from mogt_amd.chunked_lm_loss import chunked_linear_cross_entropy
    from oracle import lm_loss_oracle as lo

    gen = torch.Generator().manual_seed(21)
    B, L, D, V = 2, 300, 64, 1000
    h = torch.randn(B, L, D, generator=gen)
    w = torch.randn(V, D, generator=gen) * 0.5
    labels = torch.randint(0, V, (B, L), generator=gen)
    ht = h.to(gpu).requires_grad_()
    wt = w.to(gpu).requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss = chunked_linear_cross_entropy(ht, wt, labels.to(gpu), chunk_size=128)
    loss.backward()
    torch.cuda.synchronize()
    ref_loss, ref_gh, ref_gw = lo.chunked_linear_ce(h.double().numpy(), w.double().numpy(), labels.numpy(), 128)
    assert abs(float(loss.detach()) - ref_loss) <= BF16_TOL * abs(ref_loss)
    assert rel_err(to_np(ht.grad), ref_gh) <= BF16_TOL
    assert rel_err(to_np(wt.grad), ref_gw) <= BF16_TOL
