"""GPU parity of the MOGT block kernels, the MOGT layer and the backbone against
the float64 CPU oracle (oracle/model_oracle.py) with identical random weights.

Weights are drawn N(0, 0.02) for every projection, including theta_read, ffn.w3
and the value-gate weight (the reference zero-initialises them, which would
make every block the identity and the check vacuous).  Bars: fp32 <= 1e-4,
bf16 autocast <= 2e-2 (normwise max relative error)."""
import numpy as np
import pytest
import torch

from conftest import announce, rel_err, to_np
from oracle import model_oracle as mo

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
BF16_TOL = 2e-2


def _randomize(model, seed=0, std=0.02):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm_mogt.weight") or "norm" in name.split(".")[-2]:
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
            elif name.endswith("bias"):
                p.copy_(-2.0 + 0.5 * torch.randn(p.shape, generator=g))
            else:
                p.copy_(std * torch.randn(p.shape, generator=g))


def _state64(model):
    return {k: v.detach().double().cpu() for k, v in model.state_dict().items()}


def _coupled_cfg(block):
    return {"r": block.r, "connection_impl": block.connection_impl,
            "connection_damping": block.connection_damping,
            "value_gate_input_mode": block.value_gate_input_mode,
            "couple_forget_to_value_gate": True}


def test_rmsnorm_add_and_silu_kernels(gpu):
    announce("rmsnorm / add_rmsnorm / silu_mul")
    from mogt_amd import ops

    g = torch.Generator().manual_seed(1)
    x = torch.randn(4097, 768, generator=g)
    w = 1.0 + 0.1 * torch.randn(768, generator=g)
    z = torch.randn(4097, 768, generator=g)
    ref = mo.rmsnorm(x.double(), w.double())
    out = ops.rmsnorm(x.to(gpu), w.to(gpu))
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and rel_err(to_np(out), ref.numpy()) <= 1e-5
    xb = x.to(gpu).bfloat16()
    out_b = ops.rmsnorm(xb, w.to(gpu), out_dtype=torch.bfloat16)
    ref_b = mo.rmsnorm(xb.double().cpu(), w.double())
    assert rel_err(to_np(out_b), ref_b.numpy()) <= BF16_TOL
    zb = z.to(gpu).bfloat16()
    x_new, nrm = ops.add_rmsnorm(x.to(gpu), zb, 0.5, w.to(gpu), out_dtype=torch.float32)
    x_ref = x.double() + (0.5 * zb).float().double().cpu()
    torch.cuda.synchronize()
    assert rel_err(to_np(x_new), x_ref.numpy()) <= 1e-6
    assert rel_err(to_np(nrm), mo.rmsnorm(x_ref, w.double()).numpy()) <= 1e-5
    y = torch.randn(1000, 2 * 512, generator=g)
    s = ops.silu_mul(y.to(gpu))
    ref_s = torch.nn.functional.silu(y[:, :512].double()) * y[:, 512:].double()
    assert rel_err(to_np(s), ref_s.numpy()) <= 1e-5
    sb = ops.silu_mul(y.to(gpu).bfloat16())
    yb = y.bfloat16()
    ref_sb = (torch.nn.functional.silu(yb[:, :512]) * yb[:, 512:]).double()
    assert rel_err(to_np(sb), ref_sb.numpy()) <= BF16_TOL


@pytest.mark.parametrize("zdt,odt", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32)])
def test_add_rmsnorm_rowscale_kernel(gpu, zdt, odt):
    """x' = x + s round(r z), r = rsqrt(sum(stats) / D + eps): the residual
    update of the read-out folded around the GEMM, against float64 (z given in
    its dtype, so only the two roundings of the product differ)."""
    announce(f"add_rmsnorm_rowscale z={zdt} out={odt}")
    from mogt_amd import ops

    g = torch.Generator().manual_seed(8)
    rows, D = 3001, 768
    x = torch.randn(rows, D, generator=g)
    z = (torch.randn(rows, D, generator=g) * 30).to(zdt)
    h = torch.randn(rows, D, generator=g) * 3
    stats = (h.double() ** 2).reshape(rows, D // 64, 64).sum(-1).float()
    w = 1.0 + 0.1 * torch.randn(D, generator=g)
    x_new, out = ops.add_rmsnorm_rowscale(x.to(gpu), z.to(gpu), stats.to(gpu), 0.7, w.to(gpu), stat_eps=1e-6,
                                          eps=1e-6, out_dtype=odt)
    torch.cuda.synchronize()
    r = torch.rsqrt(h.double().pow(2).mean(-1, keepdim=True) + 1e-6)
    x_ref = x.double() + 0.7 * (r * z.double())
    tol = BF16_TOL if zdt == torch.bfloat16 else 1e-5
    assert rel_err(to_np(x_new), x_ref.numpy()) <= tol
    assert rel_err(to_np(out), mo.rmsnorm(x_ref, w.double()).numpy()) <= tol


@pytest.mark.parametrize("L", [64, 1000])
def test_fused_block_matches_oracle_fp32(gpu, L):
    announce(f"fused MOGT block fp32 L={L}")
    from mogt_amd.model_mogt import MOGTModel, configure_coupled_gate

    torch.manual_seed(0)
    model = MOGTModel(vocab_size=300, d_model=128, num_layers=2, r=16).to(gpu)
    configure_coupled_gate(model, connection_damping=0.999)
    _randomize(model, seed=L)
    model.eval()
    ids = torch.randint(0, 300, (2, L), generator=torch.Generator().manual_seed(L))
    with torch.no_grad():
        assert all(b.fused_path_ok() for b in model.blocks)
        out = model(ids.to(gpu))
    torch.cuda.synchronize()
    ref = mo.model_forward(_state64(model), ids, 2, _coupled_cfg(model.blocks[0]), prefix_position=1)
    assert rel_err(to_np(out), ref.numpy()) <= FP32_TOL


def test_fused_backbone_bf16_autocast(gpu):
    announce("fused MOGT backbone bf16 autocast L=4096")
    from mogt_amd.model_mogt import MOGTModel, configure_coupled_gate

    model = MOGTModel(vocab_size=4096, d_model=768, num_layers=2, r=16).to(gpu)
    configure_coupled_gate(model)
    _randomize(model, seed=3)
    model.eval()
    ids = torch.randint(0, 4096, (1, 4096), generator=torch.Generator().manual_seed(5))
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        out = model(ids.to(gpu))
    torch.cuda.synchronize()
    ref = mo.model_forward(_state64(model), ids, 2, _coupled_cfg(model.blocks[0]), prefix_position=1)
    assert out.dtype == torch.float32
    assert rel_err(to_np(out), ref.numpy()) <= BF16_TOL


def _configs4_model(dev, seed):
    """4 layers, d_model 768, a 4x gated MLP (hidden
    3072), vocab 32000, the benchmark's identity-coupled slot-addressed wiring;
    random weights (every projection non-zero)."""
    from mogt_amd.model_mogt import MOGTModel, configure_coupled_gate

    torch.manual_seed(seed)
    model = MOGTModel(vocab_size=32000, d_model=768, num_layers=4, r=16, ffn_hidden=3072).to(dev)
    configure_coupled_gate(model)
    _randomize(model, seed=seed)
    return model.eval()


def test_configs4_backbone_bf16_full_length(gpu):
    """configs[4] at its own shape: B = 1, L = 32768 under bf16 autocast (the
    benchmark's precision) against the float64 oracle."""
    announce("configs[4] backbone bf16 autocast L=32768")
    model = _configs4_model(gpu, seed=41)
    ids = torch.randint(0, 32000, (1, 32768), generator=torch.Generator().manual_seed(41))
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        assert all(b.fused_path_ok() for b in model.blocks)
        out = model(ids.to(gpu))
    torch.cuda.synchronize()
    out = to_np(out)
    state = _state64(model)
    del model
    torch.cuda.empty_cache()
    with torch.no_grad():
        ref = mo.model_forward(state, ids, 4, _coupled_cfg_of(state), prefix_position=1)
    assert np.isfinite(out).all()
    assert rel_err(out, ref.numpy()) <= BF16_TOL


def test_configs4_backbone_fp32(gpu):
    """configs[4]'s model in fp32 at L = 4096 against the float64 oracle."""
    announce("configs[4] backbone fp32 L=4096")
    model = _configs4_model(gpu, seed=42)
    ids = torch.randint(0, 32000, (1, 4096), generator=torch.Generator().manual_seed(42))
    with torch.no_grad():
        out = model(ids.to(gpu))
    torch.cuda.synchronize()
    with torch.no_grad():
        ref = mo.model_forward(_state64(model), ids, 4, _coupled_cfg_of(_state64(model)), prefix_position=1)
    assert rel_err(to_np(out), ref.numpy()) <= FP32_TOL


def _coupled_cfg_of(state):
    return {"r": 16, "connection_impl": "identity", "connection_damping": 1.0,
            "value_gate_input_mode": "current_prev_prefix", "couple_forget_to_value_gate": True}


@pytest.mark.parametrize("conn,tmode", [("matrix_exp", "multiply"), ("cayley", "multiply"),
                                        ("identity", "multiply"), ("matrix_exp", "residual"),
                                        ("cayley", "forget_relu")])
def test_generic_block_matches_oracle(gpu, conn, tmode):
    """The generic path (dense HIP scan) with a non-identity connection, a
    transport gate (model_mogt.py:141-163, every mode) and a scalar value gate."""
    announce(f"generic MOGT block {conn} transport gate {tmode}")
    import torch.nn as nn

    from mogt_amd.model_mogt import MOGTBlock

    torch.manual_seed(1)
    blk = MOGTBlock(d_model=64, r=16).to(gpu)
    blk.connection_impl = conn
    blk.connection_damping = 0.99
    blk.scan_impl = "triton_hybrid"
    blk.phi_transport_gate = nn.Linear(64, 16, bias=True).to(gpu)
    blk.transport_gate_mode = tmode
    blk.transport_gate_scale = 0.5
    blk.phi_value_gate = nn.Linear(128, 1, bias=True).to(gpu)
    blk.value_gate_input_mode = "current_prev"
    blk.couple_forget_to_value_gate = True
    _randomize(blk, seed=7, std=0.05)
    x = torch.randn(2, 300, 64, generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        assert not blk.fused_path_ok()
        out = blk(x.to(gpu))
    torch.cuda.synchronize()
    cfg = {"r": 16, "connection_impl": conn, "connection_damping": 0.99,
           "value_gate_input_mode": "current_prev", "couple_forget_to_value_gate": True,
           "transport_gate_mode": tmode, "transport_gate_scale": 0.5}
    p = {k: v.detach().double().cpu() for k, v in blk.state_dict().items()}
    ref = mo.block_forward(p, x.double(), None, cfg)
    assert rel_err(to_np(out), ref.numpy()) <= FP32_TOL


def test_generic_path_backward_reaches_parameters(gpu):
    """sanity_triton_gradients.py: gradients flow through the HIP scan to
    phi_val, phi_conn and the gates."""
    announce("generic MOGT block backward")
    import torch.nn as nn

    from mogt_amd.model_mogt import MOGTBlock

    blk = MOGTBlock(d_model=64, r=16).to(gpu)
    blk.connection_impl = "cayley"
    blk.scan_impl = "triton_hybrid"
    blk.phi_value_gate = nn.Linear(64, 16, bias=True).to(gpu)
    blk.couple_forget_to_value_gate = True
    _randomize(blk, seed=9, std=0.05)
    x = torch.randn(1, 128, 64, device=gpu)
    blk(x).square().mean().backward()
    for name in ("phi_val.weight", "phi_conn.weight", "phi_value_gate.weight", "theta_read.weight"):
        g = dict(blk.named_parameters())[name].grad
        assert g is not None and torch.isfinite(g).all() and g.abs().sum() > 0, name


def test_fused_path_equals_generic_path(gpu):
    """Same block, inference: fused kernels vs the generic op-by-op path."""
    announce("fused vs generic block")
    from mogt_amd.model_mogt import MOGTModel, configure_coupled_gate

    model = MOGTModel(vocab_size=100, d_model=256, num_layers=1, r=16).to(gpu)
    configure_coupled_gate(model, connection_damping=0.995)
    _randomize(model, seed=11)
    ids = torch.randint(0, 100, (1, 2000), device=gpu)
    with torch.no_grad():
        fused = model(ids)
        x = model.embedding(ids)
        generic = model.norm_f(model.blocks[0]._forward_generic(x, x[:, 1, :]))
    torch.cuda.synchronize()
    assert rel_err(to_np(fused), to_np(generic).astype(np.float64)) <= FP32_TOL


def _torch_sequential_scan(U, V, *, block_size=256, block_c=32, carry_scan="sequential", output_dtype=None,
                           return_prefix=False):
    """affine_scan_sequential (affine_scan.py:14-62) as torch ops on the GPU:
    H_t = U_t H_{t-1} + V_t with an fp32 state, outputs cast to output_dtype."""
    out_dtype = output_dtype or V.dtype
    B, L, R, C = V.shape
    H = torch.zeros(B, R, C, dtype=torch.float32, device=V.device)
    outs = []
    for t in range(L):
        H = torch.bmm(U[:, t].float().contiguous(), H) + V[:, t].float()
        outs.append(H.to(out_dtype))
    return torch.stack(outs, 1)


def test_bf16_training_regression(gpu, monkeypatch):
    """sanity_triton_training.py:17-86: a 1-layer bf16 model (vocab 257, d 64,
    r 16, seed 1234) trained one AdamW step through the HIP scan
    (scan_impl "triton_hybrid", block 16, block_c 4, doubling carry) and through
    a torch sequential scan: logits, loss, the five gradients of the reference's
    list and the parameters after the step agree to its 5e-4."""
    announce("bf16 training regression (sanity_triton_training)")
    import copy

    from mogt_amd import model_mogt, triton_scan
    from mogt_amd.model_mogt import MOGTForCausalLM

    keys = ["mogt.blocks.0.phi_conn.weight", "mogt.blocks.0.phi_val.weight", "mogt.blocks.0.theta_read.weight",
            "mogt.blocks.0.ffn.w1.weight", "mogt.embedding.weight"]
    torch.manual_seed(1234)
    base = MOGTForCausalLM(vocab_size=257, d_model=64, num_layers=1, r=16).to(gpu).to(torch.bfloat16)
    seq, hyb = copy.deepcopy(base), copy.deepcopy(base)
    seq.mogt.blocks[0].scan_impl = "sequential"
    hyb.mogt.blocks[0].scan_impl = "triton_hybrid"
    hyb.mogt.blocks[0].scan_block_size = 16
    hyb.mogt.blocks[0].scan_block_c = 4
    hyb.mogt.blocks[0].block_carry_scan = "doubling"
    ids = torch.randint(0, 257, (1, 32), device=gpu)
    labels = torch.randint(0, 257, (1, 32), device=gpu)
    opt_s = torch.optim.AdamW(seq.parameters(), lr=1e-3)
    opt_h = torch.optim.AdamW(hyb.parameters(), lr=1e-3)
    with monkeypatch.context() as m:
        m.setattr(triton_scan, "triton_affine_scan_hybrid", _torch_sequential_scan)
        assert model_mogt.triton_scan.triton_affine_scan_hybrid is _torch_sequential_scan
        logits_s, loss_s = seq(ids, labels)
        loss_s.backward()
    logits_h, loss_h = hyb(ids, labels)
    loss_h.backward()
    torch.cuda.synchronize()
    diffs = {"logits": float((logits_s.float() - logits_h.float()).abs().max().detach()),
             "loss": float((loss_s.float() - loss_h.float()).abs().detach())}
    ps, ph = dict(seq.named_parameters()), dict(hyb.named_parameters())
    for k in keys:
        diffs[k + ".grad"] = float((ps[k].grad.float() - ph[k].grad.float()).abs().max())
    opt_s.step()
    opt_h.step()
    for k in keys:
        diffs[k] = float((ps[k].float() - ph[k].float()).abs().max().detach())
    assert max(diffs.values()) <= 5e-4, diffs
    assert ph["mogt.blocks.0.theta_read.weight"].grad.abs().sum() > 0


def test_inference_weight_cache_follows_parameter_updates(gpu):
    """Inference forwards reuse the cast / concatenated GEMM weights; an in-place
    parameter update (optimizer step, load_state_dict) must invalidate them."""
    announce("inference GEMM-weight cache invalidation")
    from mogt_amd.model_mogt import MOGTModel, configure_coupled_gate

    torch.manual_seed(5)
    model = MOGTModel(vocab_size=300, d_model=64, num_layers=2, r=16).to(gpu)
    configure_coupled_gate(model, zero_gate_weight=False)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" not in name and not name.endswith("bias"):
                p.normal_(0.0, 0.05)
    ids = torch.randint(0, 300, (1, 256), device=gpu)

    def run():
        with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
            return model(ids).float().clone()

    y1 = run()
    assert torch.equal(run(), y1)                       # cached weights: same result
    with torch.no_grad():
        for p in model.parameters():
            p.mul_(0.9)
    y2 = run()
    for m in model.modules():
        m.__dict__.pop("_gemm_weight_cache", None)
    y3 = run()
    torch.cuda.synchronize()
    assert torch.equal(y2, y3) and not torch.equal(y1, y2)
    model.load_state_dict({k: v * 1.1 for k, v in model.state_dict().items()})
    y4 = run()
    for m in model.modules():
        m.__dict__.pop("_gemm_weight_cache", None)
    assert torch.equal(y4, run())
