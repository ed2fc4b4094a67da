"""The fused SwiGLU gate GEMM (csrc/swiglu_gemm.hip) against float64 and
against the unfused expression it replaces, silu(x w1^T) * (x w2^T) in bf16
(SwiGLU.forward, model_mogt.py:29-30).

Bar: bf16 output, normwise max relative error <= 2e-2 against float64 of the
same bf16 operands.  The kernel also rounds the two linear outputs and the
silu to bf16 as the unfused path does, so its error may not exceed the
unfused path's by more than a bf16 rounding step."""
import pytest
import torch
import torch.nn.functional as F

from conftest import announce, rel_err, to_np

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def _operands(M, K, H, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16()
    wg = (torch.randn(H, K, generator=g) / K ** 0.5).bfloat16()
    wu = (torch.randn(H, K, generator=g) / K ** 0.5).bfloat16()
    return x.to(dev), wg.to(dev), wu.to(dev)


def _f64(x, wg, wu):
    xd = x.double().cpu()
    return (F.silu(xd @ wg.double().cpu().t()) * (xd @ wu.double().cpu().t())).numpy()


@pytest.mark.parametrize("M,K,H", [(1, 32, 128), (257, 64, 128), (300, 128, 256), (1000, 768, 3072),
                                   (4096, 768, 2048), (513, 96, 384), (2048, 160, 640)])
def test_swiglu_gate_matches_float64_and_unfused(gpu, M, K, H):
    """Row tails (M not a multiple of 256), every K-stage count from 1 (K = 32)
    to the model's 24 (K = 768), odd stage counts, the reference FFN (2048)
    and the 4x FFN (3072)."""
    announce(f"swiglu_gate M={M} K={K} H={H}")
    from mogt_amd import ops

    x, wg, wu = _operands(M, K, H, seed=M + K + H, dev=gpu)
    y = ops.swiglu_gate(x, wg, wu)
    unfused = F.silu(F.linear(x, wg)) * F.linear(x, wu)
    torch.cuda.synchronize()
    ref = _f64(x, wg, wu)
    err = rel_err(to_np(y), ref)
    err_unfused = rel_err(to_np(unfused), ref)
    assert y.dtype == torch.bfloat16 and y.shape == (M, H)
    assert err <= BF16_TOL
    assert err <= err_unfused + 2 ** -8


def test_swiglu_gate_full_model_shape(gpu):
    """configs[4]'s FFN input: 32768 rows of d_model 768 into hidden 3072."""
    announce("swiglu_gate 32768 x 768 -> 3072")
    from mogt_amd import ops

    x, wg, wu = _operands(32768, 768, 3072, seed=5, dev=gpu)
    y = ops.swiglu_gate(x, wg, wu)
    unfused = F.silu(F.linear(x, wg)) * F.linear(x, wu)
    torch.cuda.synchronize()
    # float64 on a row sample (every 61st row) keeps the host check short
    rows = torch.arange(0, 32768, 61)
    ref = _f64(x[rows], wg, wu)
    assert rel_err(to_np(y[rows]), ref) <= BF16_TOL
    # and the whole output against the unfused bf16 expression
    assert rel_err(to_np(y), to_np(unfused)) <= BF16_TOL


def test_swiglu_gate_strided_rows(gpu):
    """x as a row-strided view (every row padded by 64 elements) and a leading
    batch dimension."""
    announce("swiglu_gate strided rows")
    from mogt_amd import ops

    x, wg, wu = _operands(600, 256, 384, seed=9, dev=gpu)
    padded = torch.zeros(600, 320, dtype=torch.bfloat16, device=gpu)
    padded[:, :256] = x
    view = padded[:, :256]
    assert view.stride(0) == 320
    y = ops.swiglu_gate(view.reshape(2, 300, 256), wg, wu)
    torch.cuda.synchronize()
    assert y.shape == (2, 300, 384)
    assert rel_err(to_np(y.reshape(600, 384)), _f64(x, wg, wu)) <= BF16_TOL


def test_swiglu_module_uses_the_fused_gate_without_grad(gpu):
    """SwiGLU.forward under bf16 autocast without gradients takes the fused
    gate; with gradients it keeps the differentiable path; both agree."""
    announce("SwiGLU module fused vs differentiable")
    from mogt_amd import ops
    from mogt_amd.model_mogt import SwiGLU

    torch.manual_seed(3)
    ffn = SwiGLU(256, 512).to(gpu)
    x = torch.randn(4, 200, 256, device=gpu)
    calls = []
    real = ops.swiglu_gate

    def spy(*a, **k):
        calls.append(1)
        return real(*a, **k)

    with torch.autocast("cuda", dtype=torch.bfloat16):
        with torch.no_grad():
            ops.swiglu_gate = spy
            try:
                fused = ffn(x)
            finally:
                ops.swiglu_gate = real
        grad_path = ffn(x)
    torch.cuda.synchronize()
    assert calls, "the no-grad bf16 forward did not take the fused gate"
    assert rel_err(to_np(fused), to_np(grad_path)) <= BF16_TOL


@pytest.mark.parametrize("M,K,H,ldx,ldy", [(1000, 768, 3072, 768, 3072), (32768, 768, 3072, 768, 3072),
                                           (300, 640, 256, 640, 256), (4096, 1024, 512, 1024, 512),
                                           (513, 896, 384, 960, 388), (77, 768, 128, 768, 128)])
def test_swiglu_gate_schedules_bit_identical(gpu, M, K, H, ldx, ldy):
    """The persistent schedule (each CU's work-group streams its tiles' stages
    back to back and runs a tile's gate math and stores inside the next tile's
    main loop) against one tile per work-group: same roundings in the same
    order, so the same bits.  Row tails, fewer tiles than CUs (M = 77, 300),
    every stage count the persistent schedule takes up to 32, padded row
    strides of x and y (the padding stays untouched)."""
    announce(f"swiglu_gate schedules M={M} K={K} H={H} ldx={ldx} ldy={ldy}")
    from mogt_amd import _lib

    lib = _lib.load()
    x, wg, wu = _operands(M, K, H, seed=M + 7 * K + H, dev=gpu)
    xp = torch.zeros(M, ldx, dtype=torch.bfloat16, device=gpu)
    xp[:, :K] = x
    stream = torch.cuda.current_stream(gpu).cuda_stream
    outs = []
    for path in (1, 2, 0):
        y = torch.full((M, ldy), 3.0, dtype=torch.bfloat16, device=gpu)
        rc = lib.mogt_swiglu_gate_fwd_cfg(xp.data_ptr(), wg.data_ptr(), wu.data_ptr(), y.data_ptr(), M, K, H, ldx,
                                          ldy, _lib.MOGT_BF16, path, stream)
        _lib.check(rc, "mogt_swiglu_gate_fwd_cfg")
        outs.append(y)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    assert bool((outs[1][:, H:] == 3.0).all())
    assert rel_err(to_np(outs[1][:, :H][:64].float()), _f64(x[:64], wg, wu)) <= BF16_TOL


def test_swiglu_gate_persistent_refuses_other_depths(gpu):
    """The persistent schedule needs d_in % 128 == 0 and d_in >= 640; forcing
    it elsewhere is an error, and the default path takes the one-tile kernel."""
    announce("swiglu_gate persistent schedule shape check")
    from mogt_amd import _lib, ops

    lib = _lib.load()
    x, wg, wu = _operands(256, 96, 128, seed=1, dev=gpu)
    y = torch.empty(256, 128, dtype=torch.bfloat16, device=gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    for K, xx, g_, u_ in [(96, x, wg, wu)] + [(k, *_operands(256, k, 128, seed=k, dev=gpu)) for k in (512, 704)]:
        rc = lib.mogt_swiglu_gate_fwd_cfg(xx.data_ptr(), g_.data_ptr(), u_.data_ptr(), y.data_ptr(), 256, K, 128, K,
                                          128, 1, 2, stream)
        assert rc != 0, K
    y0 = ops.swiglu_gate(x, wg, wu)
    torch.cuda.synchronize()
    assert rel_err(to_np(y0), _f64(x, wg, wu)) <= BF16_TOL
