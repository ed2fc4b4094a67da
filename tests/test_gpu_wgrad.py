"""GPU parity of the split-K weight-gradient GEMM (mogt_linear_wgrad, called
through the C-ABI): dW = dY^T X for bf16 dY [T, d_out], X [T, d_in], fp32
accumulation.

References: the float64 product of the same bf16 inputs, with the bound
|dW - ref| <= 1e-5 * (|dY|^T |X|) elementwise for fp32 output (fp32
summation error over T terms, far under the bf16 input precision the torch
bf16 path has); bf16 output must be exactly the fp32 output rounded once
(both come from the same partial sums added in the same order).  Run to run
the result is bit-identical.  At the model's shapes the result is also
compared with torch's own bf16 weight gradient of F.linear (2e-2 normwise).
"""
import ctypes

import pytest
import torch

from conftest import announce
from mogt_amd import _lib, ops

pytestmark = pytest.mark.gpu

F32_REL = 1e-5
BF16_TOL = 2e-2


def _inputs(T, O, I, seed, device, ldd=None, ldx=None):
    g = torch.Generator(device="cpu").manual_seed(seed)
    dy_full = torch.randn(T, ldd or O, generator=g).to(torch.bfloat16).to(device)
    x_full = torch.randn(T, ldx or I, generator=g).to(torch.bfloat16).to(device)
    return dy_full[:, :O], x_full[:, :I]


def _call(dy, x, out_dtype=torch.float32, splits=0, dw=None):
    """mogt_linear_wgrad through the C-ABI on the current stream."""
    lib = _lib.load()
    T, O = dy.shape
    I = x.shape[1]
    if dw is None:
        dw = torch.empty(O, I, dtype=out_dtype, device=dy.device)
    nbytes = int(lib.mogt_linear_wgrad_workspace_bytes(T, O, I, splits, 0))
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dy.device)
    code = _lib.MOGT_F32 if dw.dtype == torch.float32 else _lib.MOGT_BF16
    rc = lib.mogt_linear_wgrad(dy.data_ptr(), x.data_ptr(), dw.data_ptr(), T, O, I, dy.stride(0), x.stride(0),
                               dw.stride(0), splits, code, ws.data_ptr(), nbytes,
                               torch.cuda.current_stream(dy.device).cuda_stream)
    _lib.check(rc, "mogt_linear_wgrad")
    return dw


def _check_f32(dw, dy, x):
    ref = dy.double().t() @ x.double()
    bound = dy.double().abs().t() @ x.double().abs()
    err = (dw.double() - ref).abs()
    worst = float((err - F32_REL * bound).max()) if err.numel() else 0.0
    assert worst <= 0.0, f"max excess {worst:.3e} over the fp32 summation bound"


MODEL_SHAPES = [
    (768, 768),    # theta_read
    (800, 768),    # [phi_val; gate rows]
    (768, 3072),   # w3
    (6144, 768),   # [w1; w2]
]


@pytest.mark.parametrize("O,I", MODEL_SHAPES)
def test_model_shapes_full_length(gpu, O, I):
    """T = B * L = 32768 (the backbone's training batch) at every weight shape
    of the training path's linear layers."""
    T = 32768
    announce(f"linear_wgrad T{T} O{O} I{I}")
    dy, x = _inputs(T, O, I, seed=O + I, device=gpu)
    dw32 = _call(dy, x, torch.float32)
    dw16 = _call(dy, x, torch.bfloat16)
    again = _call(dy, x, torch.float32)
    torch.cuda.synchronize()
    _check_f32(dw32, dy, x)
    assert torch.equal(dw16, dw32.to(torch.bfloat16)), "bf16 output is not the fp32 sum rounded once"
    assert torch.equal(again, dw32), "not deterministic"
    # torch's own bf16 weight gradient of F.linear (the path this replaces)
    w = torch.zeros(O, I, dtype=torch.bfloat16, device=gpu, requires_grad=True)
    torch.nn.functional.linear(x, w).backward(dy)
    ref = dy.double().t() @ x.double()
    assert float((w.grad.double() - ref).abs().max() / ref.abs().max()) <= BF16_TOL
    assert float((dw16.double() - ref).abs().max() / ref.abs().max()) <= BF16_TOL


@pytest.mark.parametrize("T,O,I,splits", [
    (1, 8, 8, 0),          # one token
    (96, 16, 16, 1),       # 3 stages (the pipeline's short paths: 1 .. 5 stages)
    (128, 16, 16, 1),      # 4 stages
    (160, 16, 16, 1),      # 5 stages
    (33, 40, 264, 0),      # ragged everything: one token past a stage, partial tiles
    (1000, 8, 40, 0),      # auto splits with slices shorter than a stage multiple
    (4097, 264, 520, 3),   # tokens not a multiple of 32, 3 slices
    (4096, 512, 256, 1),   # one slice
    (4096, 512, 256, 64),  # many short slices (64 tokens each)
    (4096, 512, 256, 4096),  # more splits than stages: capped to one stage per slice
])
def test_ragged_shapes_and_splits(gpu, T, O, I, splits):
    announce(f"linear_wgrad ragged T{T} O{O} I{I} splits{splits}")
    dy, x = _inputs(T, O, I, seed=T + O, device=gpu)
    dw = _call(dy, x, torch.float32, splits=splits)
    dw16 = _call(dy, x, torch.bfloat16, splits=splits)
    torch.cuda.synchronize()
    _check_f32(dw, dy, x)
    assert torch.equal(dw16, dw.to(torch.bfloat16))


def test_split_counts_agree(gpu):
    """Different slice counts sum the same products in a different order:
    equal within the fp32 bound, each bit-stable."""
    announce("linear_wgrad split counts")
    dy, x = _inputs(8192, 768, 768, seed=7, device=gpu)
    outs = [_call(dy, x, torch.float32, splits=s) for s in (1, 2, 5, 28, 0)]
    torch.cuda.synchronize()
    for dw in outs:
        _check_f32(dw, dy, x)


def test_strided_rows_and_padded_output(gpu):
    """Row strides wider than the rows (column slices of wider activations) and
    an output row stride wider than d_in: the padding is left untouched."""
    announce("linear_wgrad strided")
    dy, x = _inputs(2048, 264, 768, seed=11, device=gpu, ldd=520, ldx=1024)
    assert dy.stride(0) == 520 and x.stride(0) == 1024
    dw_full = torch.full((264, 776), 7.0, dtype=torch.float32, device=gpu)
    dw = dw_full[:, :768]
    _call(dy, x, dw=dw)
    torch.cuda.synchronize()
    _check_f32(dw, dy, x)
    assert torch.all(dw_full[:, 768:] == 7.0)


def test_zero_tokens_writes_zeros(gpu):
    announce("linear_wgrad no tokens")
    dy = torch.empty(0, 16, dtype=torch.bfloat16, device=gpu)
    x = torch.empty(0, 24, dtype=torch.bfloat16, device=gpu)
    dw = torch.full((16, 24), 3.0, dtype=torch.bfloat16, device=gpu)
    _call(dy, x, dw=dw)
    torch.cuda.synchronize()
    assert torch.all(dw == 0)


def test_linear_autograd_matches_f_linear(gpu):
    """ops.linear: same forward and input gradient as F.linear (the same
    library GEMMs), weight gradient from the split-K kernel, within bf16
    rounding of torch's."""
    announce("ops.linear autograd")
    g = torch.Generator(device="cpu").manual_seed(3)
    x0 = torch.randn(2, 4096, 768, generator=g).to(torch.bfloat16).to(gpu)
    w0 = (torch.randn(800, 768, generator=g) / 28).to(torch.bfloat16).to(gpu)
    dy = torch.randn(2, 4096, 800, generator=g).to(torch.bfloat16).to(gpu)
    outs = []
    for fn in (ops.linear, torch.nn.functional.linear):
        x = x0.clone().requires_grad_(True)
        w = w0.clone().requires_grad_(True)
        y = fn(x, w)
        y.backward(dy)
        outs.append((y.detach(), x.grad, w.grad))
    torch.cuda.synchronize()
    (y1, dx1, dw1), (y2, dx2, dw2) = outs
    assert torch.equal(y1, y2)
    assert torch.equal(dx1, dx2)
    ref = dy.reshape(-1, 800).double().t() @ x0.reshape(-1, 768).double()
    assert dw1.dtype == torch.bfloat16
    assert float((dw1.double() - ref).abs().max() / ref.abs().max()) <= BF16_TOL
    assert float((dw2.double() - ref).abs().max() / ref.abs().max()) <= BF16_TOL
    # the custom op's fake (meta) shape agrees with the real one
    assert tuple(ops.linear_wgrad(dy, x0).shape) == (800, 768)
