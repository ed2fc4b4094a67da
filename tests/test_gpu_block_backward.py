"""GPU backward of the fused MOGT block's row kernels and of the fused block.

RMSNorm / residual-add + RMSNorm / SwiGLU gate backward kernels (through the
autograd of ``mogt::rmsnorm``, ``mogt::add_rmsnorm``, ``mogt::silu_mul``)
against float64 torch autograd of the reference's expressions
(model_mogt.py:15-20, 29-30, 243-256) on the same inputs; then a training step
through the fused block path against the generic op-by-op path (whose
pieces are each checked against float64 elsewhere), for every parameter.
Bars: fp32 <= 1e-4 (rows: 1e-5), bf16 <= 2e-2 (normwise)."""
import numpy as np
import pytest
import torch

from conftest import announce, rel_err, to_np

pytestmark = pytest.mark.gpu

ROW_TOL = 1e-5
FP32_TOL = 1e-4
BF16_TOL = 2e-2


def _rms64(x, w, eps=1e-6):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


@pytest.mark.parametrize("shape,dtype", [((2, 77, 768), torch.float32), ((3, 5, 8), torch.float32),
                                         ((1, 300, 4096), torch.float32), ((1, 129, 1028), torch.float32),
                                         ((2, 200, 768), torch.bfloat16)])
def test_rmsnorm_backward(gpu, shape, dtype):
    announce(f"rmsnorm backward {shape} {dtype}")
    from mogt_amd import ops

    g = torch.Generator().manual_seed(shape[1])
    x = (torch.randn(*shape, generator=g) * 2 + 0.3).to(dtype)
    w = 1 + 0.2 * torch.randn(shape[-1], generator=g)
    dy = torch.randn(*shape, generator=g)
    xt = x.to(gpu).requires_grad_()
    wt = w.to(gpu).requires_grad_()
    y = ops.rmsnorm(xt, wt, 1e-6, out_dtype=torch.float32)
    y.backward(dy.to(gpu))
    torch.cuda.synchronize()
    x64 = x.double().requires_grad_()
    w64 = w.double().requires_grad_()
    _rms64(x64, w64).backward(dy.double())
    tol = ROW_TOL if dtype == torch.float32 else BF16_TOL
    assert xt.grad.dtype == dtype and wt.grad.dtype == torch.float32
    assert rel_err(to_np(xt.grad), x64.grad.numpy()) <= tol
    assert rel_err(to_np(wt.grad), w64.grad.numpy()) <= (tol if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("zdt", [torch.float32, torch.bfloat16])
def test_add_rmsnorm_backward(gpu, zdt):
    announce(f"add_rmsnorm backward z={zdt}")
    from mogt_amd import ops

    g = torch.Generator().manual_seed(9)
    B, L, D = 2, 150, 768
    x = torch.randn(B, L, D, generator=g)
    z = torch.randn(B, L, D, generator=g).to(zdt)
    w = 1 + 0.2 * torch.randn(D, generator=g)
    c1 = torch.randn(B, L, D, generator=g)
    c2 = torch.randn(B, L, D, generator=g)
    xt, zt, wt = (t.to(gpu).requires_grad_() for t in (x, z, w))
    x_out, out = ops.add_rmsnorm(xt, zt, 0.7, wt, 1e-6, out_dtype=torch.float32)
    ((x_out * c1.to(gpu)).sum() + (out * c2.to(gpu)).sum()).backward()
    torch.cuda.synchronize()
    x64, z64, w64 = (t.double().requires_grad_() for t in (x, z, w))
    xo = x64 + 0.7 * z64
    ((xo * c1.double()).sum() + (_rms64(xo, w64) * c2.double()).sum()).backward()
    # bf16 z: the forward rounds 0.7 z to bf16, which the float64 reference does not
    tol = FP32_TOL if zdt == torch.float32 else BF16_TOL
    assert zt.grad.dtype == zdt
    errs = [rel_err(to_np(xt.grad), x64.grad.numpy()), rel_err(to_np(zt.grad), z64.grad.numpy()),
            rel_err(to_np(wt.grad), w64.grad.numpy())]
    assert max(errs) <= tol, errs


@pytest.mark.parametrize("used", ["residual_only", "norm_only"])
def test_add_rmsnorm_backward_one_output_used(gpu, used):
    """Only one of (x_out, out) reaches the loss: the other output has no
    gradient tensor at all (none is materialised), and the gradients still
    match float64 autograd."""
    announce(f"add_rmsnorm backward, {used}")
    from mogt_amd import ops

    g = torch.Generator().manual_seed(19)
    B, L, D = 1, 200, 768
    x = torch.randn(B, L, D, generator=g)
    z = torch.randn(B, L, D, generator=g)
    w = 1 + 0.2 * torch.randn(D, generator=g)
    c = torch.randn(B, L, D, generator=g)
    xt, zt, wt = (t.to(gpu).requires_grad_() for t in (x, z, w))
    x_out, out = ops.add_rmsnorm(xt, zt, 0.7, wt, 1e-6, out_dtype=torch.float32)
    ((x_out if used == "residual_only" else out) * c.to(gpu)).sum().backward()
    torch.cuda.synchronize()
    x64, z64, w64 = (t.double().requires_grad_() for t in (x, z, w))
    xo = x64 + 0.7 * z64
    ((xo if used == "residual_only" else _rms64(xo, w64)) * c.double()).sum().backward()
    assert rel_err(to_np(xt.grad), x64.grad.numpy()) <= FP32_TOL
    assert rel_err(to_np(zt.grad), z64.grad.numpy()) <= FP32_TOL
    if used == "residual_only":
        assert float(wt.grad.abs().max()) == 0.0
    else:
        assert rel_err(to_np(wt.grad), w64.grad.numpy()) <= FP32_TOL


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("H", [512, 3072])
def test_silu_mul_backward(gpu, dtype, H):
    """H = 3072: configs[4]'s 4x gated MLP (a 6144-wide fused [w1; w2] row)."""
    announce(f"silu_mul backward {dtype} H={H}")
    from mogt_amd import ops

    g = torch.Generator().manual_seed(4)
    rows = 333
    y = (torch.randn(rows, 2 * H, generator=g) * 2).to(dtype)
    d = torch.randn(rows, H, generator=g).to(dtype)
    yt = y.to(gpu).requires_grad_()
    out = ops.silu_mul(yt)
    out.backward(d.to(gpu))
    torch.cuda.synchronize()
    y64 = y.double().requires_grad_()
    (torch.nn.functional.silu(y64[:, :H]) * y64[:, H:]).backward(d.double())
    tol = ROW_TOL if dtype == torch.float32 else BF16_TOL
    assert yt.grad.dtype == dtype
    assert rel_err(to_np(yt.grad), y64.grad.numpy()) <= tol
    if dtype == torch.bfloat16:
        # bit-level: torch's own bf16 autograd of the same expression
        yb = y.to(gpu).requires_grad_()
        (torch.nn.functional.silu(yb[:, :H]) * yb[:, H:]).backward(d.to(gpu))
        assert rel_err(to_np(yt.grad), to_np(yb.grad)) <= 1e-2


def _train_grads(model, ids, labels, fused: bool):
    model.zero_grad(set_to_none=True)
    for b in model.mogt.blocks:
        b._force_generic = not fused
    _, loss = model(ids, labels=labels)
    loss.backward()
    torch.cuda.synchronize()
    return float(loss.detach()), {k: p.grad.detach().clone() for k, p in model.named_parameters()
                                   if p.grad is not None}


@pytest.mark.parametrize("autocast", [False, True])
def test_fused_block_training_step_matches_generic(gpu, autocast):
    """One training step (loss.backward) of a 2-layer coupled-gate model through
    the fused block path vs the generic path: same loss, same gradients for
    every parameter."""
    announce(f"fused vs generic training step autocast={autocast}")
    from mogt_amd.model_mogt import MOGTForCausalLM, MOGTBlock, configure_coupled_gate

    torch.manual_seed(7)
    model = MOGTForCausalLM(vocab_size=512, d_model=256, num_layers=2, r=16).to(gpu)
    configure_coupled_gate(model, connection_damping=0.995, zero_gate_weight=False)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "theta_read" in name or "ffn.w3" in name:
                p.normal_(0.0, 0.02)
    ids = torch.randint(0, 512, (1, 600), device=gpu)
    labels = torch.randint(0, 512, (1, 600), device=gpu)
    orig = MOGTBlock.fused_path_ok
    MOGTBlock.fused_path_ok = lambda self: (not getattr(self, "_force_generic", False)) and orig(self)
    try:
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            assert all(orig(b) for b in model.mogt.blocks)
            lf, gf = _train_grads(model, ids, labels, fused=True)
            lg, gg = _train_grads(model, ids, labels, fused=False)
    finally:
        MOGTBlock.fused_path_ok = orig
    tol = BF16_TOL if autocast else FP32_TOL
    assert abs(lf - lg) <= tol * abs(lg)
    assert set(gf) == set(gg)
    for k in gg:
        assert rel_err(to_np(gf[k]), to_np(gg[k])) <= tol, k


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_silu_mul_vector_widths(gpu, dtype):
    """Hidden widths and storage offsets that select every vector width of the
    SwiGLU kernels (16, 8, 4 and 2-byte accesses): forward and backward against
    float64 autograd of silu(a) * b on the same (rounded) inputs."""
    from mogt_amd import ops

    g = torch.Generator().manual_seed(11)
    rows = 37
    for H in (4, 12, 8, 64):
        for off in (0, 1, 2, 4):
            announce(f"silu_mul widths {dtype} H={H} offset={off}")
            base = (torch.randn(off + rows * 2 * H, generator=g) * 3).to(dtype).to(gpu)
            gbase = torch.randn(off + rows * H, generator=g).to(dtype).to(gpu)
            y = base[off:].view(rows, 2 * H).requires_grad_()
            d = gbase[off:].view(rows, H)
            out = ops.silu_mul(y)
            out.backward(d)
            torch.cuda.synchronize()
            y64 = y.detach().double().cpu().requires_grad_()
            ref = torch.nn.functional.silu(y64[:, :H]) * y64[:, H:]
            ref.backward(d.double().cpu())
            tol = ROW_TOL if dtype == torch.float32 else BF16_TOL
            assert rel_err(to_np(out), ref.detach().numpy()) <= tol, (H, off)
            assert rel_err(to_np(y.grad), y64.grad.numpy()) <= tol, (H, off)


@pytest.mark.parametrize("autocast", [False, True])
def test_fused_training_step_vs_float64_autograd(gpu, autocast):
    """One backward through the fused block path (2 layers, coupled gate,
    prefix condition) against float64 autograd of the pinned model oracle on
    the same weights: the loss and every parameter's gradient."""
    announce(f"fused training step vs float64 autograd autocast={autocast}")
    from mogt_amd.model_mogt import MOGTModel, configure_coupled_gate
    from oracle import model_oracle as mo

    torch.manual_seed(17)
    model = MOGTModel(vocab_size=300, d_model=128, num_layers=2, r=16, ffn_hidden=512).to(gpu)
    configure_coupled_gate(model, connection_damping=0.995, zero_gate_weight=False)
    gen = torch.Generator().manual_seed(17)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name:
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=gen))
            elif name.endswith("bias"):
                p.copy_(-1.0 + 0.5 * torch.randn(p.shape, generator=gen))
            else:
                p.copy_(0.05 * torch.randn(p.shape, generator=gen))
    model.train()
    ids = torch.randint(0, 300, (1, 256), generator=gen)
    target = torch.randn(1, 256, 128, generator=gen)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        assert all(b.fused_path_ok() for b in model.blocks)
        out = model(ids.to(gpu))
    loss = (out.float() - target.to(gpu)).square().mean()
    loss.backward()
    torch.cuda.synchronize()
    st = {k: v.detach().double().cpu().requires_grad_() for k, v in model.state_dict().items()}
    cfg = {"r": 16, "connection_impl": "identity", "connection_damping": 0.995,
           "value_gate_input_mode": "current_prev_prefix", "couple_forget_to_value_gate": True}
    ref_out = mo.model_forward(st, ids, 2, cfg, prefix_position=1)
    ref = (ref_out - target.double()).square().mean()
    names = list(st)
    grads = torch.autograd.grad(ref, [st[n] for n in names], allow_unused=True)
    tol = BF16_TOL if autocast else FP32_TOL
    assert abs(float(loss.detach()) - float(ref.detach())) <= tol * abs(float(ref.detach()))
    params = dict(model.named_parameters())
    checked = 0
    for n, gr in zip(names, grads):
        if gr is None or n not in params:
            continue
        assert params[n].grad is not None, n
        assert rel_err(to_np(params[n].grad), gr.numpy()) <= tol, n
        checked += 1
    assert checked >= 20
